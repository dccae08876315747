"""Worker-side swap execution: the data plane of Worker.swap_blocks.

Mirrors aegaeon/worker.py: the segment -> owning-group map (:1397-1417),
the host page view (:1419-1432), the swap streams (:278-280),
swap_blocks (:2204-2349), the source-event waits (:2351-2394) and
wait_for_all_move_in/out (:2406-2418). The reference issues one
torch copy_ per (segment, entry) extent from a Python double loop; here the
whole list is one call into libaegkv.so, one kernel launch per call.

A source event may be a local torch.cuda.Event, the IPC handle bytes
another process exported (utils.py:263-288 reduce/rebuild_cuda_event), or a
FenceToken. With interprocess_events=True the completion events are created
interprocess-capable like the reference's (worker.py:2249) and
event_ipc_handle() exports them; the default is local events, because the
HIP runtime used here rejects recording interprocess events
(hipErrorInvalidValue). Ordering across processes therefore uses fences: a
device int64 tensor of counters shared by the workers (fence_words), in
which each swapper owns one word per swap stream (fence_slots). After each
swap the swapper raises its word to the next count on that stream and
publishes FenceToken(word, count) as last_fence; a swap in another process
that lists the token among its source events waits on the device until the
word has reached the count. With fence_host (host fence words in a shared
/dev/shm file) the swapper also publishes each count to the host behind the
swap, so a controller in any process can poll the token on the CPU
(FenceToken.query / synchronize) before it frees the move's source blocks.
Ray object refs are not part of this module.

Failed waits. The reference waits on source events without a limit
(worker.py:2387) and stops the worker when it cannot get them
(:2364-2368), so a swap never reads a block before its producer wrote it.
Here a fence wait is bounded, and a wait that gives up sets the swap
stream's move guard (ops.GuardWords, one word per swap stream). Every swap
on that stream then moves nothing, its fence signal and host publish carry
the failure mark (ops.FENCE_FAILED), consumers of its MoveEvent or
FenceToken get MoveFailedError instead of completion, and a consumer's own
guard inherits the failure (through the fence word, or ops.guard_merge
behind a producer's event). A failure is sticky, like the reference's
stopped worker: the stream's later swaps fail too.
"""

from __future__ import annotations

import logging
import weakref
from collections import defaultdict, deque
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import ops
from .cache_groups import CacheGroupRuntimeConfig
from .layout import CompositeCache, host_page_geometry

logger = logging.getLogger("aegaeon_amd.swap")


@dataclass(frozen=True)
class FenceToken:
    """Completion of a swap as a fence: the swap has finished once
    fence_words[slot] >= value. Plain ints (and a file name), so it crosses
    process boundaries like the reference's event handle bytes.

    With `host` (the name of the swapper's HostFenceWords) the token also
    answers on the CPU, in any process: query() and synchronize() read the
    host word the swapper publishes behind the swap, which is how a
    controller polls a worker's move before it frees the source blocks
    (the reference polls the rebuilt IPC events, block_manager.py:804-851).
    That makes a token a move event for BlockPools.record_move.
    """

    slot: int
    value: int
    host: Optional[str] = None

    def _host_words(self) -> "ops.HostFenceWords":
        if self.host is None:
            raise ValueError("this FenceToken has no host fence words; give the swapper "
                             "fence_host=HostFenceWords(...) to poll moves on the CPU")
        return ops.attached_host_fence_words(self.host)

    def query(self) -> bool:
        """True once the swap behind this token has finished; MoveFailedError
        if it (or an earlier swap on its stream) failed and moved nothing."""
        return ops.fence_host_wait(self._host_words(), self.slot, self.value, 0.0)

    def synchronize(self, timeout_s: float = 600.0) -> None:
        """Block this thread until the swap has finished; TimeoutError after
        timeout_s seconds, MoveFailedError if it failed."""
        if not ops.fence_host_wait(self._host_words(), self.slot, self.value, timeout_s):
            raise TimeoutError(f"fence {self.slot} did not reach {self.value} within "
                               f"{timeout_s} s")


class MoveEvent(torch.cuda.Event):
    """Completion event of one swap or migration (what KVSwapper.swap_blocks
    and migrate_blocks return): a torch.cuda.Event recorded behind the move
    that also knows the move guard of the stream it ran on. query() and
    synchronize() raise MoveFailedError once the move has completed with
    that guard set (a fence wait before it gave up, or a move it waited for
    had failed: it moved nothing), so a ledger never frees the sources of a
    move that did not happen. The guard is the stream's, so a failure there
    also fails the stream's earlier events that are looked at afterwards.
    Swappers that list it as a source event inherit the failure through
    ops.guard_merge."""

    def __new__(cls, guards: "ops.GuardWords", side: int, interprocess: bool = False):
        return super().__new__(cls, interprocess=interprocess)

    def __init__(self, guards: "ops.GuardWords", side: int, interprocess: bool = False):
        self.guards = guards
        self.side = side

    @property
    def failed(self) -> bool:
        """True when the stream's guard is set (meaningful once complete)."""
        return self.guards.value(self.side) != 0

    def _raise_if_failed(self) -> None:
        why = self.guards.value(self.side)
        if why:
            direction = "in" if self.side else "out"
            cause = "a fence wait timed out" if why == 1 else "a source move failed"
            raise ops.MoveFailedError(
                f"the move behind this event ran on a swap-{direction} stream whose guard is "
                f"set ({cause}): it moved nothing")

    def query(self) -> bool:
        done = super().query()
        if done:
            self._raise_if_failed()
        return done

    def synchronize(self) -> None:
        super().synchronize()
        self._raise_if_failed()


_ipc_event_refusal: Dict[int, Optional[str]] = {}

# Fences raised by swappers of this process: (address of the fence words,
# slot) -> (the raising swapper, its recent (count, completion event) pairs
# in count order). A waiting fence kernel holds its stream's hardware queue,
# and a stream of this process may share that queue with the producing
# stream, so a token produced here is waited on through the producer's
# event instead: the event of the smallest recorded count that reaches the
# token's value, so a consumer waits for the move it names and not for later
# ones queued behind it. An entry holds only while its swapper lives: the
# swapper keeps its fence words alive, and once both are gone the address
# may belong to other words.
_LOCAL_FENCE_HISTORY = 64
_local_fences: Dict[Tuple[int, int], Tuple["weakref.ref", deque]] = {}


def _note_local_fence(words_ptr: int, slot: int, count: int, event, owner) -> None:
    entry = _local_fences.get((words_ptr, slot))
    if entry is None or entry[0]() is not owner:
        entry = (weakref.ref(owner), deque(maxlen=_LOCAL_FENCE_HISTORY))
        _local_fences[(words_ptr, slot)] = entry
    entry[1].append((count, event))


def _local_fence_event(words_ptr: int, slot: int, value: int):
    """The completion event of this process's swap that raised (words, slot)
    to `value` (the first recorded count >= value; once the history no
    longer holds that count, the oldest one kept, which completes after it),
    or None (not raised here, not that far yet, or raised by a swapper that
    no longer exists)."""
    entry = _local_fences.get((words_ptr, slot))
    if entry is None:
        return None
    owner, history = entry
    if owner() is None:
        del _local_fences[(words_ptr, slot)]
        return None
    for count, event in history:
        if count >= value:
            return event
    return None


def interprocess_event_refusal(device: torch.device) -> Optional[str]:
    """None if this process's HIP runtime records interprocess events on
    `device`, else the error it gave (tried once per device)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _ipc_event_refusal:
        try:
            with torch.cuda.device(index):
                ev = torch.cuda.Event(interprocess=True)
                ev.record(torch.cuda.current_stream(index))
                ev.synchronize()
            _ipc_event_refusal[index] = None
        except RuntimeError as exc:
            _ipc_event_refusal[index] = str(exc).strip().splitlines()[0]
    return _ipc_event_refusal[index]


class KVSwapper:
    """Executes swap lists between a CompositeCache and a pinned host pool."""

    def __init__(self, cache: CompositeCache, group_layer_names: Sequence[set],
                 group_descriptors: Sequence[CacheGroupRuntimeConfig],
                 host_pool: torch.Tensor, tp_rank: int = 0, tp_size: int = 1,
                 host_element_size: int = 2, interprocess_events: bool = False,
                 fence_words: Optional[torch.Tensor] = None,
                 fence_slots: Optional[Tuple[int, int]] = None,
                 fence_timeout_s: float = 30.0,
                 fence_host: Optional[Union["ops.HostFenceWords", str]] = None,
                 dedicated_streams: bool = False,
                 swap_cu_mask: Optional[Sequence[int]] = None, mode: str = "auto"):
        if len(group_layer_names) != len(group_descriptors):
            raise ValueError("one layer-name set per cache group is required")
        if len(group_descriptors) > 64:
            raise ValueError("at most 64 cache groups are supported")
        if not 0 <= tp_rank < tp_size:
            raise ValueError(f"tp_rank {tp_rank} outside [0, {tp_size})")
        self.cache = cache
        # transfer design for swaps that do not name one: "auto" (the
        # library's choice, DIRECT), "direct", or "staged" (link traffic on
        # DMA engines; the mode to use while a model computes beside swaps)
        ops._mode(mode)
        self.mode = mode
        self.interprocess_events = interprocess_events
        self.group_descriptors = list(group_descriptors)
        self.tp_rank = tp_rank
        self.tp_size = tp_size
        # segment -> owning groups (worker.py:1403-1417)
        self.segment_group_ids: List[frozenset] = []
        for seg in cache.segments:
            owners = frozenset(g for g, names in enumerate(group_layer_names)
                               if set(seg.shared_by) & set(names))
            if not owners:
                raise ValueError(f"no cache group names a layer of segment {seg.layer_name}")
            self.segment_group_ids.append(owners)
        # host view (worker.py:1419-1432)
        self.host_page_bytes = host_page_geometry(cache.page_size_bytes, tp_size,
                                                  host_element_size)
        if host_pool.dtype != torch.uint8:
            host_pool = host_pool.view(torch.uint8)
        self.num_host_blocks = host_pool.numel() // self.host_page_bytes
        self.kv_swap_view = host_pool.narrow(
            0, 0, self.num_host_blocks * self.host_page_bytes
        ).view(self.num_host_blocks, self.host_page_bytes)
        # flattened C-ABI layout
        self._segments = [cache.segment_tensor(i) for i in range(len(cache.segments))]
        self._page = np.array([s.page_size_bytes for s in cache.segments], np.int64)
        self._cpu_off = np.array([s.cpu_offset for s in cache.segments], np.int64)
        self._owner_mask = np.array(
            [sum(1 << g for g in owners) for owners in self.segment_group_ids], np.uint64)
        self._kpp = np.array([d.blocks_per_kv_block for d in self.group_descriptors], np.int64)
        for s, owners in enumerate(self.segment_group_ids):
            for g in owners:
                if self._page[s] % self._kpp[g]:
                    raise ValueError(
                        f"segment {s}'s {int(self._page[s])}-byte page does not split into "
                        f"{int(self._kpp[g])} equal kernel blocks"
                    )
        # bytes and extents one entry of group g moves per kernel block
        n_groups = len(self.group_descriptors)
        self._bytes_per_kb = np.zeros(n_groups, np.int64)
        self._extents_per_entry = np.zeros(n_groups, np.int64)
        for s, owners in enumerate(self.segment_group_ids):
            for g in owners:
                self._bytes_per_kb[g] += self._page[s] // self._kpp[g]
                self._extents_per_entry[g] += 1
        device = self._segments[0].device
        self.device = device
        if interprocess_events:
            refusal = interprocess_event_refusal(device)
            if refusal is not None:
                raise ValueError(
                    f"this HIP runtime refuses to record interprocess events ({refusal}); "
                    "order moves across processes with fences instead (fence_words, "
                    "fence_slots and, for CPU-side completion, fence_host)")
        self._layout = ops.SegmentLayout(
            self._segments, self._page, self._cpu_off, self._owner_mask, cache.num_blocks,
            self._kpp, self.kv_swap_view.view(-1), self.host_page_bytes,
            self.tp_rank * cache.page_size_bytes)
        # swap streams (worker.py:278-280). Plain torch streams share the
        # process's 4 hardware queues (two swaps on one queue run back to
        # back). dedicated_streams=True gives each its own queue, but such
        # streams also synchronize with the legacy default (null) stream, so
        # they suit processes whose other GPU work runs on non-default
        # streams.
        # swap_cu_mask (ops.xcd_cu_mask) confines the swap kernels to those
        # CUs, leaving the others to HBM-bound work on other streams.
        if swap_cu_mask is not None and not dedicated_streams:
            raise ValueError("swap_cu_mask needs dedicated_streams=True")
        if dedicated_streams:
            self._streams = [ops.DedicatedStream(device, swap_cu_mask),
                             ops.DedicatedStream(device, swap_cu_mask)]
            self.swap_in_stream = self._streams[0].stream
            self.swap_out_stream = self._streams[1].stream
        else:
            self._streams = []
            self.swap_in_stream = torch.cuda.Stream(device)
            self.swap_out_stream = torch.cuda.Stream(device)
        self.move_event_table: Dict[int, List[torch.cuda.Event]] = defaultdict(list)
        # fences: (swap-out word, swap-in word) this swapper raises; flags
        # its waits set on timeout, [swap-out stream, swap-in stream]
        if fence_slots is not None and fence_words is None:
            raise ValueError("fence_slots need fence_words")
        if fence_words is not None:
            if fence_words.device != device:
                raise ValueError("fence words must live on the cache's device")
            if fence_slots is not None:
                for w in fence_slots:
                    if not 0 <= w < fence_words.numel():
                        raise ValueError(f"fence slot {w} outside the fence words")
                if fence_slots[0] == fence_slots[1]:
                    raise ValueError("each swap stream needs its own fence word")
        if fence_host is not None:
            if fence_slots is None:
                raise ValueError("fence_host needs fence_slots")
            if isinstance(fence_host, str):
                fence_host = ops.attached_host_fence_words(fence_host)
            for w in fence_slots:
                if not 0 <= w < fence_host.num_words:
                    raise ValueError(f"fence slot {w} outside the host fence words")
        self.fence_host = fence_host
        self.fence_words = fence_words
        self.fence_slots = tuple(fence_slots) if fence_slots is not None else None
        self.fence_timeout_s = fence_timeout_s
        self._fence_count = [0, 0]
        # move guards of the swap-out (0) and swap-in (1) streams, set by a
        # failed fence wait or inherited from a failed source move
        self.guards = ops.GuardWords(2)
        self.last_fence: Optional[FenceToken] = None
        # other engines' caches this worker can migrate blocks from
        self._own_pages = [cache.segment_pages(i) for i in range(len(cache.segments))]
        self.peer_caches: Dict[int, List[torch.Tensor]] = {}

    def swap_blocks(self, request_ids: Sequence[int], source_block_ids: Sequence[int],
                    target_block_ids: Sequence[int], group_ids: Sequence[int],
                    first_kernel_blocks: Sequence[int], valid_kernel_blocks: Sequence[int],
                    source_events: Sequence[Optional[Union[torch.cuda.Event, bytes,
                                                           "FenceToken"]]],
                    is_swap_in: bool, mode=None) -> torch.cuda.Event:
        """Move the live extents of some blocks between host and device.

        is_swap_in: host block source_block_ids[i] -> device block
        target_block_ids[i]; otherwise device -> host. Waits on the source
        events of requests that still have a move in flight, then enqueues
        the whole list on the swap stream and returns an event recorded
        behind it (worker.py:2204-2349).
        """
        lengths = {len(source_block_ids), len(target_block_ids), len(group_ids),
                   len(first_kernel_blocks), len(valid_kernel_blocks)}
        if len(lengths) != 1:
            raise ValueError(
                f"swap lists of unequal lengths: {len(source_block_ids)} sources, "
                f"{len(target_block_ids)} targets, {len(group_ids)} groups, "
                f"{len(first_kernel_blocks)} first and {len(valid_kernel_blocks)} valid "
                "kernel blocks"
            )
        self._require_open()
        groups = np.asarray(group_ids, dtype=np.int64).reshape(-1)
        if groups.size and (groups.min() < 0 or groups.max() >= len(self.group_descriptors)):
            bad = groups[(groups < 0) | (groups >= len(self.group_descriptors))][0]
            raise ValueError(f"cache-group id {int(bad)} of a swap entry is not one of the "
                             f"{len(self.group_descriptors)} groups")
        side = 1 if is_swap_in else 0
        self._require_not_failed(side)
        stream = self.swap_in_stream if is_swap_in else self.swap_out_stream
        new_event = MoveEvent(self.guards, side, interprocess=self.interprocess_events)
        # wait for in-flight moves of the same requests (worker.py:2351-2394);
        # bytes are IPC handles exported by another process
        self._wait_sources(request_ids, source_events, stream, side)
        self._layout.swap(source_block_ids, target_block_ids, groups.astype(np.int32),
                          first_kernel_blocks, valid_kernel_blocks, is_swap_in,
                          mode=self.mode if mode is None else mode, stream=stream,
                          guard=self.guards.tensor, guard_index=side)
        self._finish(request_ids, side, stream, new_event)
        if logger.isEnabledFor(logging.INFO):
            valid = np.asarray(valid_kernel_blocks, dtype=np.int64).reshape(-1)
            copied = int((valid * self._bytes_per_kb[groups]).sum()) if groups.size else 0
            extents = int(((valid > 0) * self._extents_per_entry[groups]).sum()) if groups.size else 0
            full = len(source_block_ids) * self.cache.page_size_bytes
            saved = 0.0 if full == 0 else 1.0 - copied / full
            logger.info("requests %s moved %s: %d of %d page bytes (%.2f%% skipped), "
                        "%d extents, one launch", list(request_ids),
                        "host->device" if is_swap_in else "device->host",
                        copied, full, saved * 100, extents)
        return new_event

    def _wait_sources(self, request_ids, source_events, stream, side: int) -> None:
        """Order `stream` after the requests' previous moves
        (worker.py:2351-2394): local events, IPC event handles or fences.
        A source move's failure reaches this stream's guard: through the
        fence word for a FenceToken from another process, through
        ops.guard_merge for a MoveEvent or a token raised in this process.
        Each distinct source is waited on once."""
        if len(source_events) != len(request_ids):
            raise ValueError("one source event slot per request is required")
        seen_events, seen_tokens, merged = set(), set(), set()

        def merge_from(ev) -> None:
            if isinstance(ev, MoveEvent) and (id(ev.guards), ev.side) not in merged:
                merged.add((id(ev.guards), ev.side))
                ops.guard_merge(self.guards.tensor, side, ev.guards.tensor, ev.side,
                                device=self.device, stream=stream)

        for ev in source_events:
            if ev is None:
                continue
            if isinstance(ev, FenceToken):
                if (ev.slot, ev.value) in seen_tokens:
                    continue
                seen_tokens.add((ev.slot, ev.value))
                if self.fence_words is None:
                    raise ValueError("a FenceToken source needs fence_words")
                local = _local_fence_event(self.fence_words.data_ptr(), ev.slot, ev.value)
                if local is not None:
                    # raised in this process: wait on the producer's event
                    # and take over its stream's failure, if any
                    stream.wait_event(local)
                    merge_from(local)
                    continue
                ops.fence_wait(self.fence_words, ev.slot, ev.value, self.guards.tensor, side,
                               timeout_s=self.fence_timeout_s, stream=stream)
            else:
                if id(ev) in seen_events:
                    continue
                seen_events.add(id(ev))
                if isinstance(ev, (bytes, bytearray)):
                    ev = torch.cuda.Event.from_ipc_handle(self.device, bytes(ev))
                stream.wait_event(ev)
                merge_from(ev)

    def _finish(self, request_ids, side: int, stream, new_event: torch.cuda.Event) -> None:
        """Record the move's completion event behind the enqueued work, list
        it for the requests (worker.py:2252-2257) and raise the stream's
        fence word when fences are configured."""
        new_event.record(stream)
        for rid in request_ids:
            self.move_event_table[rid].append(new_event)
        self._signal(side, stream, new_event)

    def _signal(self, side: int, stream, event: torch.cuda.Event) -> None:
        if self.fence_slots is not None:
            self._fence_count[side] += 1
            slot, count = self.fence_slots[side], self._fence_count[side]
            ops.fence_signal(self.fence_words, slot, count, guard=self.guards.tensor,
                             guard_index=side, stream=stream)
            _note_local_fence(self.fence_words.data_ptr(), slot, count, event, self)
            host = None
            if self.fence_host is not None:
                ops.fence_publish(self.fence_host, slot, count, guard=self.guards.tensor,
                                  guard_index=side, device=self.device, stream=stream)
                host = self.fence_host.name
            self.last_fence = FenceToken(slot, count, host)

    def register_peer_cache(self, engine_id: int, segment_pages: Sequence[torch.Tensor]) -> None:
        """Make another engine's cache a migration source
        (Worker.register_kvcache_mem_handles, worker.py:2439-2445).

        segment_pages: that cache's segments as [num_blocks, page] uint8
        tensors in segment order, e.g. received from its process through
        torch.multiprocessing (HIP IPC memory) or CompositeCache.segment_pages
        of a cache in this process. Pages must match this cache's.
        """
        pages = list(segment_pages)
        if len(pages) != len(self._own_pages):
            raise ValueError(f"peer cache has {len(pages)} segments, expected "
                             f"{len(self._own_pages)}")
        for i, (p, own) in enumerate(zip(pages, self._own_pages)):
            if p.dim() != 2 or p.size(1) != own.size(1) or p.dtype != torch.uint8:
                raise ValueError(f"peer segment {i} must be uint8 [blocks, {own.size(1)}]")
            if p.size(0) != pages[0].size(0):
                raise ValueError("peer segments disagree on the block count")
        self.peer_caches[engine_id] = pages

    def unregister_peer_cache(self, engine_id: int) -> None:
        """Worker.unregister_kvcache_mem_handles (worker.py:2447-2451)."""
        self.peer_caches.pop(engine_id, None)

    def migrate_blocks(self, request_ids: Sequence[int], source_engine_id: int,
                       source_block_ids: Sequence[int], target_block_ids: Sequence[int],
                       source_events: Sequence[Optional[Union[torch.cuda.Event, bytes,
                                                              "FenceToken"]]]
                       ) -> torch.cuda.Event:
        """Copy whole blocks from a registered peer cache into this cache
        (Worker.migrate_blocks, worker.py:2420-2430, unimplemented upstream).

        Runs on the swap-in stream after the requests' previous moves, one
        aegkv_migrate_blocks launch; returns the completion event and, with
        fences configured, publishes last_fence for the swap-in word.
        """
        self._require_open()
        if source_engine_id not in self.peer_caches:
            raise KeyError(f"engine {source_engine_id}'s cache is not registered")
        if len(source_block_ids) != len(target_block_ids):
            raise ValueError("source and target block lists differ in length")
        self._require_not_failed(1)
        stream = self.swap_in_stream
        new_event = MoveEvent(self.guards, 1, interprocess=self.interprocess_events)
        self._wait_sources(request_ids, source_events, stream, 1)
        ops.migrate_blocks(self.peer_caches[source_engine_id], self._own_pages,
                           source_block_ids, target_block_ids, stream=stream,
                           guard=self.guards.tensor, guard_index=1)
        self._finish(request_ids, 1, stream, new_event)
        return new_event

    @staticmethod
    def event_ipc_handle(event: torch.cuda.Event) -> bytes:
        """IPC handle of a swap's completion event, for another process to
        open with torch.cuda.Event.from_ipc_handle (worker.py:2349)."""
        return event.ipc_handle()

    def clear_request_resource(self, request_id: int) -> None:
        self.move_event_table.pop(request_id, None)

    def clear_request_resource_batched(self, request_ids: Sequence[int]) -> None:
        for rid in request_ids:
            self.clear_request_resource(rid)

    def _require_not_failed(self, side: int) -> None:
        """MoveFailedError once this side's guard is set (as the host sees it
        now; the device also stops every later guarded swap on the stream)."""
        why = self.guards.value(side)
        if why:
            direction = "in" if side else "out"
            cause = (f"a fence wait gave up after {self.fence_timeout_s} s" if why == 1
                     else "a move it waited for had failed")
            raise ops.MoveFailedError(
                f"this swapper's swap-{direction} stream has failed ({cause}): its swaps from "
                "then on moved nothing and their completion reports failure; the failure is "
                "sticky, as the reference stops the worker")

    def _require_open(self) -> None:
        if self.swap_in_stream is None:
            raise RuntimeError("this KVSwapper is closed")

    def close(self) -> None:
        """Wait for this swapper's swaps and release its dedicated streams,
        if it has any (their hardware queues are returned at once). The
        swapper is not usable afterwards."""
        for st in (self.swap_in_stream, self.swap_out_stream):
            if st is not None:
                st.synchronize()
        for owner in self._streams:
            owner.close()
        self._streams = []
        self.swap_in_stream = self.swap_out_stream = None

    def wait_for_all_move_in(self) -> None:
        """Wait for every swap-in (worker.py:2406-2412); MoveFailedError if the
        swap-in stream's guard is set."""
        self._require_open()
        self.swap_in_stream.synchronize()
        self._require_not_failed(1)

    def wait_for_all_move_out(self) -> None:
        """Wait for every swap-out (worker.py:2414-2418); MoveFailedError if the
        swap-out stream's guard is set."""
        self._require_open()
        self.swap_out_stream.synchronize()
        self._require_not_failed(0)
