"""Operator API of the KV movement path (the `aegaeon.ops` drop-in).

`swap` keeps the reference's positional signature, ops/ops.h:4-10
(`swap(source_block_ids, target_block_ids, is_swap_in, kv_cache, kv_swap)`),
and runs on the current stream like ops/swap.cu:21-32. `swap_segments` is the
composite-page data plane of Worker.swap_blocks (aegaeon/worker.py:2265-2329)
and `copy_blocks` the in-HBM block copy. Every call is one C-ABI call into
libaegkv.so; there is no Python or CPU fallback.
"""

from __future__ import annotations

import ctypes
import sys
import threading
import weakref
from typing import Sequence

import numpy as np
import torch

from . import _lib

MODE_AUTO = _lib.MODE_AUTO
MODE_DIRECT = _lib.MODE_DIRECT
MODE_STAGED = _lib.MODE_STAGED
FENCE_FAILED = _lib.FENCE_FAILED
MoveFailedError = _lib.MoveFailedError

_MODES = {"auto": MODE_AUTO, "direct": MODE_DIRECT, "staged": MODE_STAGED}


def _mode(mode) -> int:
    if isinstance(mode, str):
        try:
            return _MODES[mode]
        except KeyError:
            raise ValueError(f"unknown transfer mode {mode!r}") from None
    if mode not in (MODE_AUTO, MODE_DIRECT, MODE_STAGED):
        raise ValueError(f"unknown transfer mode {mode!r}")
    return int(mode)


def _ints(values) -> np.ndarray:
    """A flat integer array; floats and booleans are refused rather than
    truncated (an empty list is fine)."""
    if isinstance(values, torch.Tensor):
        values = values.detach().cpu().numpy()
    a = np.asarray(values).reshape(-1)
    if a.size and a.dtype.kind not in "iu":
        raise ValueError(f"expected integers, got {a.dtype} values")
    return a


def _i64(values) -> np.ndarray:
    return np.ascontiguousarray(_ints(values).astype(np.int64, copy=False))


def _i32(values) -> np.ndarray:
    a = _ints(values)
    if a.size and (a.min() < np.iinfo(np.int32).min or a.max() > np.iinfo(np.int32).max):
        raise ValueError("group ids must fit in 32 bits")
    return np.ascontiguousarray(a.astype(np.int32, copy=False))


def _p64(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def _p32(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def _pu64(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))


def _stream_ptr(device: torch.device, stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return s.cuda_stream


def _tensor_bytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


def _require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise ValueError(f"{what} must be a device (HIP) tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


def _require_host(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cpu":
        raise ValueError(f"{what} must be a host tensor, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


def swap(
    source_block_ids: Sequence[int],
    target_block_ids: Sequence[int],
    is_swap_in: bool,
    kv_cache: torch.Tensor,
    kv_swap: torch.Tensor,
    *,
    mode="auto",
    stream: torch.cuda.Stream | None = None,
) -> None:
    """Whole-block swap between a device cache and a pinned host pool.

    Follows ops/swap.cu:25-60: block i moves source_block_ids[i] ->
    target_block_ids[i]; is_swap_in copies host (kv_swap) -> device
    (kv_cache), otherwise device -> host. The block size is
    kv_cache.numel() * element_size / kv_cache.size(0) bytes and is used for
    both tensors; for the 2-byte dtypes the reference supports this equals
    its `numel * 2 / size(0)` (swap.cu:34). Runs on the current stream.
    Raises ValueError on bad ids (the reference checks nothing).
    """
    _require_device(kv_cache, "kv_cache")
    _require_host(kv_swap, "kv_swap")
    src = _i64(source_block_ids)
    dst = _i64(target_block_ids)
    if src.shape != dst.shape:
        raise ValueError(
            f"source ({src.size}) and target ({dst.size}) id lists differ in length"
        )
    if kv_cache.dim() == 0 or kv_cache.size(0) == 0:
        raise ValueError("kv_cache must have a non-empty block dimension")
    block_bytes = _tensor_bytes(kv_cache) // kv_cache.size(0)
    if _tensor_bytes(kv_cache) % kv_cache.size(0):
        raise ValueError("kv_cache bytes are not divisible by its block count")
    swap_blocks_total = _tensor_bytes(kv_swap) // block_bytes
    lib = _lib.load()
    with torch.cuda.device(kv_cache.device):
        rc = lib.aegkv_swap(
            _p64(src), _p64(dst), src.size, 1 if is_swap_in else 0,
            kv_cache.data_ptr(), kv_cache.size(0),
            kv_swap.data_ptr(), swap_blocks_total, block_bytes,
            _mode(mode), _stream_ptr(kv_cache.device, stream),
        )
    _lib.check(rc)


def _guard_ptr(words: torch.Tensor | None, index: int, what: str):
    """Address of a move guard word (or None): a 1-D int64 tensor in pinned
    host memory (GuardWords) or on the device."""
    if words is None:
        return None
    if words.dtype != torch.int64 or words.dim() != 1 or not words.is_contiguous():
        raise ValueError(f"{what} must be a contiguous 1-D int64 tensor")
    if not 0 <= index < words.numel():
        raise ValueError(f"{what} index {index} outside [0, {words.numel()})")
    return words.data_ptr() + 8 * index


def _call_on(device: torch.device, fn):
    """Run fn() with `device` current, switching (and restoring) only when
    another device is current. Keeps no state, so threads may share it."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if torch.cuda.current_device() == index:
        return fn()
    with torch.cuda.device(index):
        return fn()


class SegmentLayout:
    """A validated composite layout, reusable across swap calls.

    Holds the backing tensors (segments, each viewed as [device_num_blocks,
    page] bytes), their composite-page geometry (vllm_cache.py:75-101,
    worker.py:1419-1432) and the pinned host pool, checked once and kept as
    the C-ABI arrays the library takes, so a call only converts its id lists.
    The layout keeps references to the tensors it describes.
    """

    def __init__(self, segments: Sequence[torch.Tensor], segment_page_bytes: Sequence[int],
                 segment_host_offsets: Sequence[int], segment_owner_masks: Sequence[int],
                 device_num_blocks: int, group_kernel_blocks_per_page: Sequence[int],
                 host_pool: torch.Tensor, host_page_bytes: int, host_rank_offset: int):
        if not segments:
            raise ValueError("at least one segment is required")
        dev = segments[0].device
        for i, t in enumerate(segments):
            _require_device(t, f"segment {i}")
            if t.device != dev:
                raise ValueError("all segments must live on one device")
        _require_host(host_pool, "host_pool")
        n_seg = len(segments)
        self.page = _i64(segment_page_bytes)
        self.host_offsets = _i64(segment_host_offsets)
        self.owners = np.ascontiguousarray(
            np.asarray(segment_owner_masks, dtype=np.uint64).reshape(-1))
        self.kpp = _i64(group_kernel_blocks_per_page)
        if not (self.page.size == self.host_offsets.size == self.owners.size == n_seg):
            raise ValueError("segment metadata lengths must equal the number of segments")
        for i, t in enumerate(segments):
            if _tensor_bytes(t) < int(self.page[i]) * device_num_blocks:
                raise ValueError(
                    f"segment {i} holds {_tensor_bytes(t)} bytes < "
                    f"{device_num_blocks} x {int(self.page[i])}"
                )
        self.segments = list(segments)
        self.host_pool = host_pool
        self.device = dev
        self.num_segments = n_seg
        self.device_num_blocks = int(device_num_blocks)
        self.host_page_bytes = int(host_page_bytes)
        self.host_rank_offset = int(host_rank_offset)
        self.host_num_blocks = (_tensor_bytes(host_pool) // self.host_page_bytes
                                if self.host_page_bytes > 0 else 0)
        self._bases = (ctypes.c_void_p * n_seg)(*[t.data_ptr() for t in segments])
        self._args = (n_seg, self._bases, _p64(self.page), _p64(self.host_offsets),
                      _pu64(self.owners), self.device_num_blocks, self.kpp.size,
                      _p64(self.kpp), host_pool.data_ptr(), self.host_num_blocks,
                      self.host_page_bytes, self.host_rank_offset)

    def swap(self, source_block_ids, target_block_ids, group_ids, first_kernel_blocks,
             valid_kernel_blocks, is_swap_in: bool, *, mode="auto",
             stream: torch.cuda.Stream | None = None, guard: torch.Tensor | None = None,
             guard_index: int = 0) -> None:
        """One aegkv_swap_blocks call over this layout (see swap_segments).
        guard (with guard_index): a move guard word (GuardWords.tensor); when
        it is set by the time the stream reaches the swap, nothing moves."""
        src = _i64(source_block_ids)
        dst = _i64(target_block_ids)
        grp = _i32(group_ids)
        first = _i64(first_kernel_blocks)
        valid = _i64(valid_kernel_blocks)
        if not (src.size == dst.size == grp.size == first.size == valid.size):
            raise ValueError(
                f"swap lists of unequal lengths: {src.size} sources, {dst.size} targets, "
                f"{grp.size} groups, {first.size} first and {valid.size} valid kernel blocks"
            )
        gp = _guard_ptr(guard, guard_index, "guard")
        lib = _lib.load()
        rc = _call_on(self.device, lambda: lib.aegkv_swap_blocks(
            *self._args, src.size, _p64(src), _p64(dst), _p32(grp), _p64(first),
            _p64(valid), 1 if is_swap_in else 0, _mode(mode), gp,
            _stream_ptr(self.device, stream)))
        _lib.check(rc)


def swap_segments(
    segments: Sequence[torch.Tensor],
    segment_page_bytes: Sequence[int],
    segment_host_offsets: Sequence[int],
    segment_owner_masks: Sequence[int],
    device_num_blocks: int,
    group_kernel_blocks_per_page: Sequence[int],
    host_pool: torch.Tensor,
    host_page_bytes: int,
    host_rank_offset: int,
    source_block_ids,
    target_block_ids,
    group_ids,
    first_kernel_blocks,
    valid_kernel_blocks,
    is_swap_in: bool,
    *,
    mode="auto",
    stream: torch.cuda.Stream | None = None,
) -> None:
    """Composite-page swap of (segment x entry) extents in one launch.

    Byte placement of aegaeon/worker.py:2265-2329: for each segment s owned
    by the entry's group, extent (off, len) = byte_extent_for_kernel_blocks
    of (page_s, kernel blocks per page, first, valid) (cache_transfer.py:
    138-165); host bytes sit at host_id * host_page_bytes + host_rank_offset
    + host_offset_s + off; device bytes at dev_id * page_s + off of segment s.
    Callers that swap over the same layout repeatedly should build a
    SegmentLayout once and call its swap().
    """
    SegmentLayout(segments, segment_page_bytes, segment_host_offsets, segment_owner_masks,
                  device_num_blocks, group_kernel_blocks_per_page, host_pool, host_page_bytes,
                  host_rank_offset).swap(source_block_ids, target_block_ids, group_ids,
                                         first_kernel_blocks, valid_kernel_blocks, is_swap_in,
                                         mode=mode, stream=stream)


def _copy_call_args(segments, src_block_ids, dst_block_ids, segment_page_bytes,
                    device_num_blocks, stream):
    """Checked C-ABI arguments of one copy_blocks call (device first; the
    arrays are returned too so they outlive the call)."""
    if not segments:
        raise ValueError("at least one segment is required")
    dev = segments[0].device
    for i, t in enumerate(segments):
        _require_device(t, f"segment {i}")
        if t.device != dev:
            raise ValueError("all segments must live on one device")
    if device_num_blocks is None:
        device_num_blocks = segments[0].size(0)
    if segment_page_bytes is None:
        segment_page_bytes = [_tensor_bytes(t) // device_num_blocks for t in segments]
    page = _i64(segment_page_bytes)
    if page.size != len(segments):
        raise ValueError("segment_page_bytes must have one entry per segment")
    for i, t in enumerate(segments):
        if _tensor_bytes(t) < int(page[i]) * device_num_blocks:
            raise ValueError(f"segment {i} is smaller than {device_num_blocks} blocks")
    src = _i64(src_block_ids)
    dst = _i64(dst_block_ids)
    if src.shape != dst.shape:
        raise ValueError("src and dst id lists differ in length")
    bases = (ctypes.c_void_p * len(segments))(*[t.data_ptr() for t in segments])
    args = (len(segments), bases, _p64(page), int(device_num_blocks), src.size, _p64(src),
            _p64(dst), _stream_ptr(dev, stream))
    return dev, args, (page, src, dst)


def copy_blocks(
    segments: Sequence[torch.Tensor],
    src_block_ids,
    dst_block_ids,
    *,
    segment_page_bytes: Sequence[int] | None = None,
    device_num_blocks: int | None = None,
    stream: torch.cuda.Stream | None = None,
) -> None:
    """In-HBM block copy: seg[dst[i]] := seg[src[i]] for every segment.

    Each segment is viewed as [num_blocks, page] bytes; by default the page
    is the tensor's bytes / size(0). Targets must be distinct and disjoint
    from the sources. The reference has no KV copy_blocks; its in-HBM
    compaction is aegaeon/allocator.py:101-137.
    """
    dev, args, _keep = _copy_call_args(segments, src_block_ids, dst_block_ids,
                                       segment_page_bytes, device_num_blocks, stream)
    lib = _lib.load()
    _lib.check(_call_on(dev, lambda: lib.aegkv_copy_blocks(*args)))


PROBE_READ = _lib.PROBE_READ
PROBE_WRITE = _lib.PROBE_WRITE


def copy_probe(kind: int, segments: Sequence[torch.Tensor], src_block_ids, dst_block_ids,
               sink: torch.Tensor, *, magic: int = 0x9E3779B9,
               segment_page_bytes: Sequence[int] | None = None,
               device_num_blocks: int | None = None,
               stream: torch.cuda.Stream | None = None) -> None:
    """Measurement only: the read half (PROBE_READ: load every source tile)
    or the write half (PROBE_WRITE: store a fixed pattern into every target
    tile, destroying its contents) of copy_blocks with the same ids, work
    items and launch shape (aegkv_copy_probe). sink: a device int32/uint32
    tensor the read probe may write one word of."""
    if kind not in (PROBE_READ, PROBE_WRITE):
        raise ValueError(f"unknown probe kind {kind!r}")
    if sink.device.type != "cuda" or sink.element_size() != 4 or sink.numel() < 1:
        raise ValueError("sink must be a device tensor of 4-byte words")
    dev, args, _keep = _copy_call_args(segments, src_block_ids, dst_block_ids,
                                       segment_page_bytes, device_num_blocks, stream)
    lib = _lib.load()
    _lib.check(_call_on(dev, lambda: lib.aegkv_copy_probe(
        kind, *args[:-1], sink.data_ptr(), int(magic) & 0xFFFFFFFF, args[-1])))


#: limits of copy_blocks_noalloc (the fixed descriptor array of libaegkv)
NOALLOC_MAX_SEGMENTS = 1024
NOALLOC_MAX_PAIRS = 65536


def copy_blocks_noalloc(
    segments: Sequence[torch.Tensor],
    src_block_ids,
    dst_block_ids,
    *,
    segment_page_bytes: Sequence[int] | None = None,
    device_num_blocks: int | None = None,
    stream: torch.cuda.Stream | None = None,
) -> None:
    """copy_blocks through aegkv_copy_blocks_noalloc: the library allocates
    nothing for the call (its descriptor goes to a fixed device array), for
    callers that cannot allocate. At most NOALLOC_MAX_SEGMENTS segments and
    NOALLOC_MAX_PAIRS pairs (ValueError beyond). Calls that overlap on one
    device from different streams or threads race on that array; calls on
    one stream are ordered."""
    dev, args, _keep = _copy_call_args(segments, src_block_ids, dst_block_ids,
                                       segment_page_bytes, device_num_blocks, stream)
    lib = _lib.load()
    _lib.check(_call_on(dev, lambda: lib.aegkv_copy_blocks_noalloc(*args)))


def load_slices(dst: Sequence[torch.Tensor], src: Sequence[torch.Tensor], *, mode="auto",
                stream: torch.cuda.Stream | None = None) -> None:
    """dst[i] <- src[i] byte for byte for every i, pinned host -> device, in
    one aegkv_load_slices call: the weight load of a model switch, where the
    reference runs one `slice_storage.copy_(tensors_storage,
    non_blocking=True)` per tensors content
    (aegaeon/loader/quick_loader.py:325-340). mode "direct" (and "auto"):
    one kernel reads the host memory over PCIe; "staged": one runtime DMA
    copy per slice. Runs on `stream` (default: the current stream of dst's
    device)."""
    if len(dst) != len(src):
        raise ValueError(f"{len(dst)} target slices for {len(src)} source slices")
    if not dst:
        return
    dev = dst[0].device
    sizes = []
    for i, (d, h) in enumerate(zip(dst, src)):
        _require_device(d, f"target slice {i}")
        _require_host(h, f"source slice {i}")
        if d.device != dev:
            raise ValueError("all target slices must live on one device")
        if _tensor_bytes(d) != _tensor_bytes(h):
            raise ValueError(f"slice {i}: {_tensor_bytes(h)} source bytes for "
                             f"{_tensor_bytes(d)} target bytes")
        sizes.append(_tensor_bytes(d))
    n = len(dst)
    d_ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in dst])
    s_ptrs = (ctypes.c_void_p * n)(*[t.data_ptr() for t in src])
    b = np.ascontiguousarray(np.array(sizes, np.int64))
    lib = _lib.load()
    _lib.check(_call_on(dev, lambda: lib.aegkv_load_slices(
        n, d_ptrs, s_ptrs, _p64(b), _mode(mode), _stream_ptr(dev, stream))))


def migrate_blocks(
    src_segments: Sequence[torch.Tensor],
    dst_segments: Sequence[torch.Tensor],
    src_block_ids,
    dst_block_ids,
    *,
    segment_page_bytes: Sequence[int] | None = None,
    stream: torch.cuda.Stream | None = None,
    guard: torch.Tensor | None = None,
    guard_index: int = 0,
) -> None:
    """Whole-block copy from one cache to another of the same layout:
    dst_segments[s][dst[i]] := src_segments[s][src[i]] (aegkv_migrate_blocks).

    The reference plans this move (aegaeon/block_manager.py:1527-1601,
    aegaeon/worker.py:2420-2445) but leaves it unimplemented. The source
    tensors may be another engine's cache on this GPU, tensors received from
    another process (torch.multiprocessing, a HIP IPC memory handle), or a
    peer GPU's cache with peer access enabled; the work runs on the target
    cache's device. Each segment is viewed as [num_blocks, page] bytes; by
    default the page is the tensor's bytes / size(0), equal for both caches.
    guard: a move guard word, as for SegmentLayout.swap.
    """
    if not src_segments or len(src_segments) != len(dst_segments):
        raise ValueError("one source and one target tensor per segment are required")
    dev = dst_segments[0].device
    for i, (a, b) in enumerate(zip(src_segments, dst_segments)):
        _require_device(a, f"source segment {i}")
        _require_device(b, f"target segment {i}")
        if b.device != dev:
            raise ValueError("all target segments must live on one device")
    n_src = src_segments[0].size(0)
    n_dst = dst_segments[0].size(0)
    if segment_page_bytes is None:
        segment_page_bytes = [_tensor_bytes(t) // n_dst for t in dst_segments]
    page = _i64(segment_page_bytes)
    if page.size != len(dst_segments):
        raise ValueError("segment_page_bytes must have one entry per segment")
    for i, (a, b) in enumerate(zip(src_segments, dst_segments)):
        if _tensor_bytes(a) < int(page[i]) * n_src or _tensor_bytes(b) < int(page[i]) * n_dst:
            raise ValueError(f"segment {i} is smaller than its block count x page")
    src = _i64(src_block_ids)
    dst = _i64(dst_block_ids)
    if src.shape != dst.shape:
        raise ValueError("src and dst id lists differ in length")
    sb = (ctypes.c_void_p * len(src_segments))(*[t.data_ptr() for t in src_segments])
    db = (ctypes.c_void_p * len(dst_segments))(*[t.data_ptr() for t in dst_segments])
    gp = _guard_ptr(guard, guard_index, "guard")
    lib = _lib.load()
    rc = _call_on(dev, lambda: lib.aegkv_migrate_blocks(
        len(dst_segments), sb, db, _p64(page), int(n_src), int(n_dst), src.size, _p64(src),
        _p64(dst), gp, _stream_ptr(dev, stream)))
    _lib.check(rc)


class _OwnedStream(torch.cuda.ExternalStream):
    """A torch stream over a HIP stream from aegkv_stream_create that
    destroys the HIP stream when the object goes (or on _aegkv_close()).
    weakref.finalize is not used: its callback was seen not to run for
    torch stream objects. Once closed, the stream's handle and its
    synchronize / query / wait / record methods raise instead of handing
    the runtime a destroyed stream."""

    def __init__(self, stream_ptr: int, device=None):
        self._aegkv_ptr = stream_ptr

    def _aegkv_close(self) -> None:
        ptr, self._aegkv_ptr = getattr(self, "_aegkv_ptr", None), None
        if ptr:
            _lib.check(_lib.load().aegkv_stream_destroy(ctypes.c_void_p(ptr)))

    def _aegkv_require_open(self) -> None:
        if getattr(self, "_aegkv_ptr", None) is None:
            raise RuntimeError("this dedicated stream is closed")

    @property
    def closed(self) -> bool:
        return getattr(self, "_aegkv_ptr", None) is None

    @property
    def cuda_stream(self):
        self._aegkv_require_open()
        return super().cuda_stream

    def synchronize(self):
        self._aegkv_require_open()
        return super().synchronize()

    def query(self):
        self._aegkv_require_open()
        return super().query()

    def wait_event(self, event):
        self._aegkv_require_open()
        return super().wait_event(event)

    def wait_stream(self, stream):
        self._aegkv_require_open()
        return super().wait_stream(stream)

    def record_event(self, event=None):
        self._aegkv_require_open()
        return super().record_event(event)

    def __del__(self, _finalizing=sys.is_finalizing):
        # At interpreter exit the HIP runtime may already be torn down, and
        # the process is ending anyway: leave the stream to it. (The check is
        # bound at definition: module globals may be gone by then.)
        if _finalizing():
            return
        try:
            self._aegkv_close()
        except Exception:
            pass


CUS_PER_XCD = 32  # MI355X (gfx950): 8 XCDs of 32 CUs


def xcd_cu_mask(cus_per_xcd: int, first: int = 0,
                device: torch.device | None = None) -> list[int]:
    """CU mask words (for DedicatedStream(cu_mask=...)) that give a stream
    `cus_per_xcd` CUs on each of the 8 XCDs: mask bits i with
    first <= i % 32 < first + cus_per_xcd. The runtime spreads every run of
    8 consecutive mask bits over the 8 XCDs, one CU each (hardware ids read
    by workgroups of such streams show bits 0-7 on one CU per XCD, bits 0-31
    on four), so the CU count per XCD is what a mask sets; a mask cannot
    confine a stream to whole XCDs. The runtime takes runs of 8 or more bits
    starting at a multiple of 8, e.g. xcd_cu_mask(8) for the swap streams
    and xcd_cu_mask(24, first=8) for the rest."""
    if cus_per_xcd <= 0 or first < 0 or first + cus_per_xcd > CUS_PER_XCD:
        raise ValueError(f"CUs [{first}, {first + cus_per_xcd}) do not fit a "
                         f"{CUS_PER_XCD}-CU XCD")
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    n = torch.cuda.get_device_properties(dev).multi_processor_count
    words = [0] * ((n + 31) // 32)
    for i in range(n):
        if first <= i % CUS_PER_XCD < first + cus_per_xcd:
            words[i // 32] |= 1 << (i % 32)
    return words


class DedicatedStream:
    """A HIP stream on a hardware queue of its own (aegkv_stream_create),
    usable wherever torch takes a stream through `.stream`.

    Plain streams (torch.cuda.Stream included) share the process's 4
    hardware queues, and two streams on one queue run their work one after
    the other; a swap-out and a swap-in on dedicated streams always overlap.
    With cu_mask (see xcd_cu_mask) its kernels run only on those CUs.
    Unlike torch's pool streams, a dedicated stream is a blocking stream: it
    synchronizes with the legacy default (null) stream, so work on it waits
    for the default stream's earlier work and the other way round.
    The HIP stream lives exactly as long as the `.stream` object (which this
    object holds): it is destroyed by close() or as soon as the last
    reference to `.stream` goes, after its queued work, so dropped streams
    do not keep hardware queues until a garbage collection.
    """

    def __init__(self, device: torch.device | None = None, cu_mask: Sequence[int] | None = None):
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        lib = _lib.load()
        ptr = ctypes.c_void_p()
        if cu_mask is None:
            _lib.check(_call_on(dev, lambda: lib.aegkv_stream_create(ctypes.byref(ptr))))
        else:
            words = np.ascontiguousarray(np.asarray(cu_mask, dtype=np.uint32).reshape(-1))
            arg = words.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))
            _lib.check(_call_on(dev, lambda: lib.aegkv_stream_create_masked(
                ctypes.byref(ptr), arg, int(words.size))))
        self.device = dev
        self.cu_mask = None if cu_mask is None else list(cu_mask)
        self.stream = _OwnedStream(ptr.value, device=dev)

    def close(self) -> None:
        self.stream._aegkv_close()


def host_pinned_usage() -> tuple[int, int]:
    """(pinned bytes the library holds, free bytes inside its uncached
    blocks), from aegkv_host_usage: live cached pools plus every uncached
    block kept, which is what counts against the host's cap on pinned
    memory."""
    pinned, free = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(_lib.load().aegkv_host_usage(ctypes.byref(pinned), ctypes.byref(free)))
    return int(pinned.value), int(free.value)


def _free_pinned(ptr: int) -> None:
    rc = _lib.load().aegkv_host_free(ptr)
    if rc:
        raise _lib.AegkvError(rc, _lib.load().aegkv_last_error().decode(errors="replace"))


class PinnedHostPool:
    """A pinned, device-mapped host byte pool from aegkv_host_alloc.

    Counterpart of the reference's host KV pool (aegaeon/llm.py:1020-1040,
    aegaeon/worker.py:251-273), allocated pinned instead of registering an
    existing /dev/shm mapping. `tensor` is a uint8 view of the whole pool.
    The memory is released when the pool and every tensor viewing it are
    gone (views keep it alive), so a kernel can never be handed freed
    memory through a surviving view. Callers still wait for GPU work on the
    pool before dropping the last view.

    uncached=True allocates from the uncached system pool
    (AEGKV_HOST_UNCACHED): faster swaps, especially both directions at
    once, but the library keeps such memory mapped until the process ends
    and carves later uncached pools out of it. coherent=True allocates
    fine-grained coherent memory (AEGKV_HOST_COHERENT), for words the GPU and
    the host both write while kernels run (GuardWords).
    """

    def __init__(self, nbytes: int, uncached: bool = False, coherent: bool = False):
        if nbytes <= 0:
            raise ValueError("pool size must be positive")
        lib = _lib.load()
        ptr = ctypes.c_void_p()
        flags = (_lib.HOST_UNCACHED if uncached else 0) | (_lib.HOST_COHERENT if coherent else 0)
        _lib.check(lib.aegkv_host_alloc_flags(ctypes.byref(ptr), int(nbytes), flags))
        self.nbytes = int(nbytes)
        self.uncached = uncached
        self.coherent = coherent
        buf = (ctypes.c_uint8 * self.nbytes).from_address(ptr.value)
        fin = weakref.finalize(buf, _free_pinned, ptr.value)
        fin.atexit = False  # at interpreter exit the process releases it
        self.tensor = torch.frombuffer(buf, dtype=torch.uint8)

    def free(self) -> None:
        """Drop this pool's reference; the memory goes once no view remains."""
        self.tensor = None


class GuardWords:
    """Move guards: `num_words` uint64 words in coherent pinned host memory,
    zeroed, that the GPU and the host both read and write (one per stream
    that waits on fences; KVSwapper keeps one per swap stream).

    A fence wait sets its stream's guard when it gives up (1) or when the
    word it waits on carries the failure mark (2); guarded swaps and
    migrations then move nothing, and guarded signals and publishes mark
    the completion they report as failed (FENCE_FAILED), so every consumer
    sees the failure. The library never clears a guard.
    """

    def __init__(self, num_words: int = 2):
        if num_words <= 0:
            raise ValueError("num_words must be positive")
        self._pool = PinnedHostPool(8 * int(num_words), coherent=True)
        self.tensor = self._pool.tensor.view(torch.int64)
        self.tensor.zero_()
        self.num_words = int(num_words)

    def ptr(self, index: int) -> int:
        return _guard_ptr(self.tensor, index, "guard")

    def value(self, index: int) -> int:
        """The guard as the host sees it now (0: not set)."""
        if not 0 <= index < self.num_words:
            raise ValueError(f"guard index {index} outside [0, {self.num_words})")
        return int(self.tensor[index])


def _fence_word(words: torch.Tensor, index: int, what: str) -> int:
    if words.dtype != torch.int64 or words.dim() != 1:
        raise ValueError(f"{what} must be a 1-D int64 tensor")
    if not words.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if not 0 <= index < words.numel():
        raise ValueError(f"{what} index {index} outside [0, {words.numel()})")
    return words.data_ptr() + 8 * index


def _fence_value(value: int) -> int:
    if not 0 < value < FENCE_FAILED:
        raise ValueError("fence values are positive and below 2**62 (bit 62 marks a failed move)")
    return int(value)


def fence_signal(words: torch.Tensor, index: int, value: int, *,
                 guard: torch.Tensor | None = None, guard_index: int = 0,
                 stream: torch.cuda.Stream | None = None) -> None:
    """Raise words[index] to at least `value` once every operation
    enqueued earlier on `stream` (default: the current stream) has finished
    (aegkv_fence_signal). The counterpart of recording an interprocess event
    behind a swap (aegaeon/worker.py:2331,2349). With a move guard that is
    set by then, the word is raised to value | FENCE_FAILED instead.

    words: a 1-D int64 tensor on the device, e.g. one shared with other
    processes through torch.multiprocessing (a HIP IPC memory handle).
    """
    value = _fence_value(value)
    ptr = _fence_word(words, index, "fence words")
    gp = _guard_ptr(guard, guard_index, "guard")
    dev = words.device
    if dev.type != "cuda":
        raise ValueError("fence words must live on the device")
    lib = _lib.load()
    rc = _call_on(dev, lambda: lib.aegkv_fence_signal(ptr, value, gp, _stream_ptr(dev, stream)))
    _lib.check(rc)


def fence_wait(words: torch.Tensor, index: int, value: int, guard: torch.Tensor,
               guard_index: int = 0, *, timeout_s: float = 30.0,
               stream: torch.cuda.Stream | None = None) -> None:
    """Make every later operation on `stream` wait until words[index] >=
    value (aegkv_fence_wait); the counterpart of waiting on another worker's
    interprocess event (aegaeon/worker.py:2351-2394).

    A wait that has polled for `timeout_s` seconds gives up and sets the
    move guard guard[guard_index] to 1; a word that carries FENCE_FAILED
    ends the wait at once and sets it to 2. The stream then goes on, but
    guarded moves after the wait move nothing and guarded signals and
    publishes report failure. guard: GuardWords.tensor, or a device int64
    tensor on the words' device; the guard is never cleared here.
    """
    value = _fence_value(value)
    ptr = _fence_word(words, index, "fence words")
    gp = _guard_ptr(guard, guard_index, "guard")
    dev = words.device
    if dev.type != "cuda":
        raise ValueError("fence words must live on the device")
    if guard.device.type == "cuda" and guard.device != dev:
        raise ValueError("fence words and a device guard must live on one device")
    timeout_us = int(timeout_s * 1e6)
    lib = _lib.load()
    rc = _call_on(dev, lambda: lib.aegkv_fence_wait(ptr, value, timeout_us, gp,
                                                    _stream_ptr(dev, stream)))
    _lib.check(rc)


def guard_merge(guard: torch.Tensor, index: int, source: torch.Tensor, source_index: int, *,
                device: torch.device | None = None,
                stream: torch.cuda.Stream | None = None) -> None:
    """Once `stream` (default: the current stream of `device`) reaches it, set
    guard[index] to 2 (a source failed) when source[source_index] is set
    (aegkv_guard_merge): a consumer that waits on a producer's completion
    event inherits the producer's failure."""
    gp = _guard_ptr(guard, index, "guard")
    sp = _guard_ptr(source, source_index, "source guard")
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    lib = _lib.load()
    _lib.check(_call_on(dev, lambda: lib.aegkv_guard_merge(gp, sp, _stream_ptr(dev, stream))))


class HostFenceWords:
    """Host fence words shared by processes: a file in /dev/shm of
    `num_words` uint64 counters, mapped shared. Workers raise them behind
    their swaps (fence_publish) and a controller in any process reads them
    (fence_host_wait), where the reference's controller polls the workers'
    interprocess events (aegaeon/block_manager.py:804-851).

    HostFenceWords(n) creates a new zeroed file (its `name` is the path) and
    removes it on close(); HostFenceWords.attach(name) maps an existing one.
    close() first waits for every stream that a publish into these words was
    enqueued on, so no host function writes into an unmapped page.
    """

    def __init__(self, num_words: int | None = None, *, _name: str | None = None):
        import mmap
        import os
        import uuid

        if _name is None:
            if num_words is None or num_words <= 0:
                raise ValueError("num_words must be positive")
            name = f"/dev/shm/aegkv-fence-{os.getpid()}-{uuid.uuid4().hex[:12]}"
            fd = os.open(name, os.O_RDWR | os.O_CREAT | os.O_EXCL, 0o600)
            try:
                os.ftruncate(fd, 8 * int(num_words))
            except BaseException:
                os.close(fd)
                os.unlink(name)
                raise
            self.owner = True
        else:
            name = _name
            # a publish writes through the mapping: only this library's own files
            if (os.path.dirname(os.path.abspath(name)) != "/dev/shm"
                    or not os.path.basename(name).startswith("aegkv-fence-")):
                raise ValueError(f"{name} is not a host fence file (/dev/shm/aegkv-fence-*)")
            fd = os.open(name, os.O_RDWR)
            self.owner = False
        try:
            size = os.fstat(fd).st_size
            if size < 8 or size % 8:
                raise ValueError(f"{name} is not a file of fence words ({size} bytes)")
            self._mm = mmap.mmap(fd, size, mmap.MAP_SHARED, mmap.PROT_READ | mmap.PROT_WRITE)
        finally:
            os.close(fd)
        self.name = name
        self.num_words = size // 8
        self._anchor = ctypes.c_char.from_buffer(self._mm)
        self._base = ctypes.addressof(self._anchor)
        self.words = np.frombuffer(self._mm, dtype=np.uint64)
        # streams holding publishes into these words: stream handle -> stream
        self._publishers: dict = {}
        self._publishers_lock = threading.Lock()

    @classmethod
    def attach(cls, name: str) -> "HostFenceWords":
        return cls(_name=name)

    def ptr(self, index: int) -> int:
        if self._mm is None:
            raise ValueError("these host fence words are closed")
        if not 0 <= index < self.num_words:
            raise ValueError(f"host fence index {index} outside [0, {self.num_words})")
        return self._base + 8 * index

    def _note_publisher(self, stream: torch.cuda.Stream) -> None:
        with self._publishers_lock:
            self._publishers[stream.cuda_stream] = stream

    def close(self) -> None:
        """Wait for the streams that publishes into these words were enqueued
        on (a closed dedicated stream was synchronized when it closed), then
        unmap, and remove the file for the creator."""
        import os

        if self._mm is None:
            return
        with self._publishers_lock:
            streams, self._publishers = list(self._publishers.values()), {}
        for st in streams:
            if not getattr(st, "closed", False):
                st.synchronize()
        self.words = None
        self._anchor = None
        self._mm.close()
        self._mm = None
        if self.owner:
            try:
                os.unlink(self.name)
            except FileNotFoundError:
                pass


_attached_lock = threading.Lock()
_attached: dict = {}


def attached_host_fence_words(name: str) -> HostFenceWords:
    """This process's mapping of the host fence words at `name` (mapped once,
    kept until the process ends)."""
    with _attached_lock:
        hw = _attached.get(name)
        if hw is None or hw._mm is None:
            hw = HostFenceWords.attach(name)
            _attached[name] = hw
        return hw


def fence_publish(host_words: HostFenceWords, index: int, value: int, *,
                  guard: torch.Tensor | None = None, guard_index: int = 0,
                  device: torch.device | None = None,
                  stream: torch.cuda.Stream | None = None) -> None:
    """Raise host_words[index] to at least `value` once every operation
    enqueued earlier on `stream` (default: the current stream of `device`)
    has finished (aegkv_fence_publish, a host function on the stream). With
    a move guard (GuardWords.tensor: the host function reads it) that is set
    by then, the word is raised to value | FENCE_FAILED instead."""
    value = _fence_value(value)
    ptr = host_words.ptr(index)
    gp = _guard_ptr(guard, guard_index, "guard")
    if guard is not None and guard.device.type != "cpu":
        raise ValueError("a published fence's guard must be pinned host memory (GuardWords)")
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    lib = _lib.load()
    rc = _call_on(dev, lambda: lib.aegkv_fence_publish(ptr, value, gp, st.cuda_stream))
    _lib.check(rc)
    host_words._note_publisher(st)


def fence_host_wait(host_words: HostFenceWords, index: int, value: int,
                    timeout_s: float = 0.0) -> bool:
    """True once host_words[index] >= value; waits on this thread for at most
    timeout_s seconds (0: look once). No GPU call; the GIL is released.
    Raises MoveFailedError when the word carries the failure mark."""
    value = _fence_value(value)
    if timeout_s < 0:
        raise ValueError("timeout_s must be >= 0")
    rc = _lib.load().aegkv_fence_host_wait(host_words.ptr(index), value,
                                           int(timeout_s * 1e6))
    if rc < 0:
        _lib.check(rc)
    if rc == 2:
        raise MoveFailedError(f"host fence {host_words.name}[{index}] carries the failure mark: "
                              f"the move it counts (value {value}) or one before it on its "
                              "stream moved nothing")
    return rc == 1
