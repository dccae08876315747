"""Host-side logic and the C-ABI library, without a GPU."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from aegaeon_amd import cache_transfer as ct
from aegaeon_amd.cache_groups import (
    LOGICAL_NULL_BLOCK_ID,
    BlockTable,
    CacheGroupConfig,
    CacheGroupRuntimeConfig,
)
from aegaeon_amd.layout import KVCacheTensorSpec, kv_tensor_specs, make_composite_layout

REPO = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------ cache_transfer --

def test_product_extent_matches_oracle(oracle, golden):
    rows = golden("kernel_block_extent.npz")["rows"]
    for t, b, phys, kern, w, f, c in rows.tolist():
        w = None if w < 0 else w
        assert ct.kernel_block_extent_for_attention_page(t, b, phys, kern, w) == (f, c)
    for page, kpp in ((2162688, 33), (384, 4), (65536, 1)):
        for first in range(kpp + 1):
            for num in range(kpp - first + 1):
                assert ct.byte_extent_for_kernel_blocks(page, kpp, first, num) == \
                    oracle.byte_extent(page, kpp, first, num)


@pytest.mark.parametrize("args", [
    (-1, 0, 16, 16, None), (0, -1, 16, 16, None), (0, 0, 0, 16, None), (0, 0, 16, 0, None),
    (0, 0, 48, 32, None), (5, 0, 16, 16, 0),
])
def test_product_extent_rejects_like_oracle(oracle, args):
    with pytest.raises(ValueError):
        oracle.kernel_block_extent(*args)
    with pytest.raises(ValueError):
        ct.kernel_block_extent_for_attention_page(*args)


def test_product_window_helpers_match_oracle(oracle):
    for bs in (1, 4, 16):
        for w in (1, 2, 5, 16, 33):
            for t in range(0, 80):
                assert ct.logical_blocks_for_tokens(t, bs) == oracle.logical_blocks_for_tokens(t, bs)
                assert ct.num_skipped_sliding_window_blocks(t, bs, w) == \
                    oracle.num_skipped_sliding_window_blocks(t, bs, w)
                assert ct.sliding_window_resident_block_bound(t, bs, w) == \
                    oracle.sliding_window_resident_block_bound(t, bs, w)
                assert ct.valid_kernel_blocks_for_attention_page(t, 1, 32, bs) == \
                    oracle.kernel_block_extent(t, 1, 32, bs)[1] if 32 % bs == 0 else True
    for bad in ((-1, 16), (3, 0)):
        with pytest.raises(ValueError):
            ct.logical_blocks_for_tokens(*bad)
    with pytest.raises(ValueError):
        ct.prefix_bytes_for_kernel_blocks(384, 4, 5)
    with pytest.raises(ValueError):
        ct.byte_extent_for_kernel_blocks(384, 4, 3, 2)


# ------------------------------------------------------------ cache groups --

def test_to_kernel_block_ids_known_answer():
    """block_manager.py:342-344: 272-token physical / 16-token kernel blocks,
    physical id 3 -> kernel ids 51..67; a released column -> the null block."""
    g = CacheGroupRuntimeConfig("attention", 272, 16)
    assert g.to_kernel_block_ids([3]) == list(range(51, 68))
    assert g.to_kernel_block_ids([-1]) == [0] * 17
    assert CacheGroupRuntimeConfig("mamba_none", 4, 4).to_kernel_block_ids([5, 9]) == [5, 9]


def test_slot_for_position():
    g = CacheGroupRuntimeConfig("attention", 64, 16)
    ids = [7, -1, 2]
    # position 130 -> column 2 (id 2), inside 2 -> kernel id 2*4 + 0 -> slot 8*16 + 2
    assert g.slot_for_position(ids, 130) == 130 - 128 + 2 * 64
    assert g.slot_for_position(ids, 17) == 7 * 64 + 17
    with pytest.raises(RuntimeError):
        g.slot_for_position(ids, 70)
    with pytest.raises(IndexError):
        g.slot_for_position(ids, 200)


def test_group_validation():
    with pytest.raises(ValueError):
        CacheGroupConfig("attention", 48, 32)
    with pytest.raises(ValueError):
        CacheGroupConfig("mamba_none", 16, 8)
    with pytest.raises(ValueError):
        CacheGroupConfig("mamba_none", 16, 16, sliding_window=4)
    with pytest.raises(ValueError):
        CacheGroupConfig("attention", 16, 16, sliding_window=0)
    with pytest.raises(NotImplementedError):
        CacheGroupConfig("linear", 16, 16)


def _table():
    groups = (CacheGroupConfig("attention", 32, 16),
              CacheGroupConfig("attention", 32, 16, sliding_window=20),
              CacheGroupConfig("mamba_none", 1, 1))
    return BlockTable(location=0, block_shape=(8,), cache_groups=groups,
                      group_blocks=[[5, 6, 7, 8], [9, 10, 11, 12], [13]])


def transfer_rows_by_enumeration(groups, group_blocks, t):
    """Rows transfer_entries must give, from token visibility alone
    (block_manager.py:446-478 over :205-266 and cache_transfer.py:31-94):
    the next query sits at position t and sees every committed position
    (p < t) under full attention, the w-1 most recent ones under a window w.
    A column is dropped when it was released (-1) or when all of its
    positions are committed and invisible; a kept attention column's extent
    is the span of kernel blocks holding visible positions ((0, 0) when it
    holds none); a state page moves whole as (0, 1)."""
    rows = []
    for g, (grp, cols) in enumerate(zip(groups, group_blocks)):
        for c, block in enumerate(cols):
            if block == -1:
                continue
            if grp.kind == "mamba_none":
                rows.append((g, c, block, 0, 1))
                continue
            w = grp.sliding_window
            page = range(c * grp.block_size, (c + 1) * grp.block_size)
            visible = [p for p in page if p < t and (w is None or t - p < w)]
            if not visible and all(p < t for p in page):
                continue   # wholly committed and invisible: released by the window
            kbs = {(p - page.start) // grp.kernel_block_size for p in visible}
            rows.append((g, c, block, min(kbs), max(kbs) - min(kbs) + 1) if kbs
                        else (g, c, block, 0, 0))
    return rows


def test_transfer_entries_brute_force():
    """Every retained page, with its live kernel-block extent; pages wholly
    before the window are skipped; the mamba page moves whole."""
    t = 100
    tab = _table()
    rows = tab.transfer_entries(t)
    assert rows == transfer_rows_by_enumeration(tab.cache_groups, tab.group_blocks, t)
    # window 20 at position 100 sees 81..100: columns 0 and 1 of group 1 go
    assert [r[1] for r in rows if r[0] == 1] == [2, 3]


def test_transfer_entries_random_tables_by_enumeration(aegkv_lib):
    """Random groups (page sizes, kernel blocks per page, windows 1..70),
    random released columns and token counts: the Python BlockTable and the
    native planner both give the enumerated rows."""
    import numpy as np

    from aegaeon_amd.planner import native_transfer_entries

    rng = np.random.default_rng(123)
    for _ in range(60):
        groups = []
        for _g in range(int(rng.integers(1, 4))):
            kbs = int(rng.choice([1, 2, 4, 8]))
            bs = kbs * int(rng.choice([1, 2, 3, 4]))
            w = None if rng.random() < 0.3 else int(rng.integers(1, 71))
            groups.append(CacheGroupConfig("attention", bs, kbs, sliding_window=w))
        if rng.random() < 0.3:
            groups.append(CacheGroupConfig("mamba_none", 1, 1))
        tables = []
        for _t in range(4):
            t = int(rng.integers(0, 120))
            cols = []
            for grp in groups:
                n = 1 if grp.kind == "mamba_none" else -(-(t + 1) // grp.block_size)
                ids = rng.integers(1, 1000, n)
                ids[rng.random(n) < 0.15] = -1
                cols.append([int(x) for x in ids])
            tables.append((BlockTable(location=0, block_shape=(8,), cache_groups=tuple(groups),
                                      group_blocks=cols), t))
        native = native_transfer_entries(groups, tables)
        for (tab, t), nat in zip(tables, native):
            want = transfer_rows_by_enumeration(groups, tab.group_blocks, t)
            assert tab.transfer_entries(t) == want, (groups, tab.group_blocks, t)
            assert nat == want, (groups, tab.group_blocks, t)


def test_moved_tables_and_metadata():
    tab = _table()
    t = 100
    rows = tab.transfer_entries(t)
    targets = list(range(100, 100 + len(rows)))
    moved = tab.moved_group_blocks(t, targets)
    assert moved[1][:2] == [LOGICAL_NULL_BLOCK_ID] * 2
    flat = [b for col in moved for b in col if b != LOGICAL_NULL_BLOCK_ID]
    assert flat == targets
    with pytest.raises(ValueError):
        tab.moved_group_blocks(t, targets[:-1])
    groups, firsts, counts = tab.swap_metadata(t)
    assert all(c > 0 for c in counts)
    assert len(groups) == sum(1 for r in rows if r[4] > 0)


def test_release_and_replace():
    tab = _table()
    released = tab.release_skipped_blocks(100)
    assert released == [9, 10]
    assert tab.group_blocks[1][:2] == [LOGICAL_NULL_BLOCK_ID] * 2
    assert tab.blocks == [5, 6, 7, 8, 11, 12, 13]
    tab.replace_flat_blocks([1, 2, 3, 4, 5, 6, 7])
    assert tab.group_blocks == [[1, 2, 3, 4], [-1, -1, 5, 6], [7]]
    with pytest.raises(ValueError):
        tab.replace_flat_blocks([1])


def test_sliding_window_one_keeps_destination_without_bytes():
    """A W=1 window retains its current page with nothing to copy
    (block_manager.py:1440-1446): count 0, still a transfer entry."""
    groups = (CacheGroupConfig("attention", 16, 16, sliding_window=1),)
    tab = BlockTable(0, (8,), groups, [[4, 5]])
    rows = tab.transfer_entries(20)
    assert rows == [(0, 1, 5, 0, 0)]
    assert tab.swap_metadata(20) == ([], [], [])


# ------------------------------------------------------------------ layout --

def test_composite_layout():
    specs = kv_tensor_specs(36, 8, 16, 8, 128, 2)
    segs, page = make_composite_layout(specs, 8)
    assert len(segs) == 72
    assert page == 72 * 32768 == 2_359_296
    assert [s.cpu_offset for s in segs[:3]] == [0, 32768, 65536]
    assert segs[1].layer_name == "layers.0.v"
    with pytest.raises(ValueError):
        make_composite_layout([KVCacheTensorSpec(10, ("a",))], 3)
    with pytest.raises(NotImplementedError):
        make_composite_layout([KVCacheTensorSpec(12, ("a",), block_stride=4)], 3)
    with pytest.raises(ValueError):
        make_composite_layout([KVCacheTensorSpec(12, ())], 3)


# ------------------------------------------------------------------ C ABI --

def _declared_symbols():
    hdr = (REPO / "include" / "aegkv.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(aegkv_\w+)\(", hdr, re.M)))


def test_library_exports_every_declared_symbol(aegkv_lib):
    from aegaeon_amd import _lib

    declared = _declared_symbols()
    assert declared == sorted(_lib.EXPORTED_SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (aegkv_\w+)", out))
    for name in declared:
        assert name in exported, name
        assert hasattr(aegkv_lib, name)
    assert aegkv_lib.aegkv_abi_version() == _lib.ABI_VERSION


def test_library_binds_to_torch_hip_runtime():
    """Every HIP symbol libaegkv imports must be exported by the HIP runtime
    torch ships, so that in a torch process both share one runtime."""
    import torch
    from aegaeon_amd import _lib

    torch_hip = Path(torch.__file__).parent / "lib" / "libamdhip64.so"
    if not torch_hip.exists():
        pytest.skip("torch without a bundled HIP runtime")
    need = subprocess.run(["nm", "-D", "--undefined-only", str(_lib.LIB_PATH)],
                          capture_output=True, text=True, check=True).stdout
    have = subprocess.run(["nm", "-D", "--defined-only", str(torch_hip)],
                          capture_output=True, text=True, check=True).stdout
    have_syms = set(re.findall(r" [TW] (\S+)", have))
    for sym in re.findall(r" U (\S*hip\S*)", need):
        assert sym.replace("@", "@@", 1) in have_syms or sym.split("@")[0] in have_syms, sym


def test_early_validation_without_gpu(aegkv_lib):
    from aegaeon_amd import _lib

    lib = aegkv_lib
    rc = lib.aegkv_swap(None, None, 0, 0, None, 1, None, 1, 0, 0, None)
    assert rc == _lib.EINVAL
    assert b"block_bytes" in lib.aegkv_last_error()
    rc = lib.aegkv_copy_blocks(0, None, None, 1, 0, None, None, None)
    assert rc == _lib.EINVAL
    rc = lib.aegkv_swap_blocks(1, None, None, None, None, 1, 1, None, None, 1, 1, 0, 1, None,
                               None, None, None, None, 0, 0, None, None)
    assert rc == _lib.EINVAL
    assert b"metadata" in lib.aegkv_last_error()
    with pytest.raises(ValueError):
        _lib.check(rc)
    assert lib.aegkv_host_alloc(None, 16) == _lib.EINVAL
    assert lib.aegkv_host_free(None) == 0


def test_prepared_layout_rejects_host_segments():
    """SegmentLayout checks its tensors before it touches the library."""
    from aegaeon_amd import ops

    seg = torch.zeros(4, 64, dtype=torch.uint8)
    pool = torch.zeros(4 * 64, dtype=torch.uint8)
    with pytest.raises(ValueError, match="device"):
        ops.SegmentLayout([seg], [64], [0], [1], 4, [1], pool, 64, 0)
    with pytest.raises(ValueError, match="at least one"):
        ops.SegmentLayout([], [], [], [], 4, [1], pool, 64, 0)


def test_id_arrays_refuse_floats_and_wide_group_ids():
    """Ids, extents and layout sizes are converted without truncation:
    float or boolean arrays and group ids beyond 32 bits raise ValueError
    (an empty list is an empty id array)."""
    from aegaeon_amd import ops

    assert ops._i64([]).dtype == np.int64 and ops._i64([]).size == 0
    assert ops._i64(torch.tensor([3, 4])).tolist() == [3, 4]
    assert ops._i32(np.array([2], np.uint8)).dtype == np.int32
    for bad in ([1.5], np.array([True]), torch.tensor([2.0])):
        with pytest.raises(ValueError, match="integers"):
            ops._i64(bad)
    with pytest.raises(ValueError, match="32 bits"):
        ops._i32([1 << 32])


def test_masked_stream_rejections_before_any_hip_call(aegkv_lib):
    """aegkv_stream_create_masked refuses a missing stream pointer or an
    empty mask before touching the device; xcd_cu_mask refuses CU ranges
    that do not fit a 32-CU XCD."""
    from aegaeon_amd import _lib, ops

    lib = aegkv_lib
    st = ctypes.c_void_p()
    words = (ctypes.c_uint32 * 1)(0xFF)
    assert lib.aegkv_stream_create_masked(None, words, 1) == _lib.EINVAL
    assert lib.aegkv_stream_create_masked(ctypes.byref(st), None, 1) == _lib.EINVAL
    assert lib.aegkv_stream_create_masked(ctypes.byref(st), words, 0) == _lib.EINVAL
    assert b"empty" in lib.aegkv_last_error()
    for cus, first in ((0, 0), (8, 28), (33, 0), (8, -1)):
        with pytest.raises(ValueError, match="XCD"):
            ops.xcd_cu_mask(cus, first)


def test_fence_rejections_before_any_hip_call(aegkv_lib):
    from aegaeon_amd import _lib

    lib = aegkv_lib
    assert lib.aegkv_fence_signal(None, 1, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_signal(0x1004, 1, None, None) == _lib.EINVAL   # not 8-byte aligned
    assert b"aligned" in lib.aegkv_last_error()
    # bit 62 is the failure mark: values stay below it
    assert lib.aegkv_fence_signal(0x1000, 1 << 62, None, None) == _lib.EINVAL
    assert b"2^62" in lib.aegkv_last_error()
    assert lib.aegkv_fence_signal(0x1000, 0, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_wait(0x1000, 1, 0, 0x2000, None) == _lib.ERANGE
    assert lib.aegkv_fence_wait(0x1000, 1, 601 * 10**6, 0x2000, None) == _lib.ERANGE
    assert lib.aegkv_fence_wait(None, 1, 1000, 0x2000, None) == _lib.EINVAL
    assert lib.aegkv_fence_wait(0x1000, 1 << 62, 1000, 0x2000, None) == _lib.EINVAL
    assert lib.aegkv_guard_merge(None, 0x2000, None) == _lib.EINVAL
    assert lib.aegkv_guard_merge(0x1000, 0x2004, None) == _lib.EINVAL    # not 8-byte aligned
    from aegaeon_amd import ops

    with pytest.raises(ValueError, match="int64"):
        ops.fence_signal(torch.zeros(4, dtype=torch.int32), 0, 1)
    with pytest.raises(ValueError, match="device"):
        ops.fence_signal(torch.zeros(4, dtype=torch.int64), 0, 1)
    with pytest.raises(ValueError, match="positive"):
        ops.fence_signal(torch.zeros(4, dtype=torch.int64), 0, 0)
    with pytest.raises(ValueError, match="2\\*\\*62"):
        ops.fence_signal(torch.zeros(4, dtype=torch.int64), 0, ops.FENCE_FAILED)
    with pytest.raises(ValueError, match="guard index"):
        ops.fence_signal(torch.zeros(4, dtype=torch.int64), 0, 1,
                         guard=torch.zeros(2, dtype=torch.int64), guard_index=2)


def test_host_fence_words_across_processes(aegkv_lib):
    """Host fence words live in a shared file: a value written by another
    process is seen by fence_host_wait here, with a bounded wait; the
    creator removes the file on close."""
    import os
    import sys
    import time

    from aegaeon_amd import ops

    hw = ops.HostFenceWords(3)
    assert hw.name.startswith("/dev/shm/") and hw.num_words == 3
    assert not ops.fence_host_wait(hw, 1, 1)
    code = ("import sys, time; sys.path.insert(0, '.'); from aegaeon_amd import ops; "
            f"h = ops.HostFenceWords.attach({hw.name!r}); time.sleep(0.3); h.words[1] = 7; "
            "h.close()")
    proc = subprocess.Popen([sys.executable, "-c", code], cwd=str(REPO))
    t0 = time.perf_counter()
    assert ops.fence_host_wait(hw, 1, 7, timeout_s=60)
    assert time.perf_counter() - t0 >= 0.2
    assert proc.wait(60) == 0
    assert ops.fence_host_wait(hw, 1, 6) and not ops.fence_host_wait(hw, 1, 8, 0.02)
    with pytest.raises(ValueError):
        hw.ptr(3)
    with pytest.raises(ValueError, match="not a host fence file"):
        ops.HostFenceWords.attach(str(REPO / "README.md"))
    name = hw.name
    hw.close()
    assert not os.path.exists(name)


def test_host_fence_rejections_before_any_hip_call(aegkv_lib):
    from aegaeon_amd import _lib

    lib = aegkv_lib
    word = (ctypes.c_uint64 * 2)()
    base = ctypes.addressof(word)
    assert lib.aegkv_fence_publish(None, 1, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_publish(base + 4, 1, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_publish(base, 0, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_publish(base, 1 << 62, None, None) == _lib.EINVAL
    assert lib.aegkv_fence_publish(base, 1, base + 12, None) == _lib.EINVAL   # guard unaligned
    assert lib.aegkv_fence_host_wait(None, 1, 0) == _lib.EINVAL
    assert lib.aegkv_fence_host_wait(base + 1, 1, 0) == _lib.EINVAL
    assert lib.aegkv_fence_host_wait(base, 1, -1) == _lib.ERANGE
    assert lib.aegkv_fence_host_wait(base, 1, 601_000_000) == _lib.ERANGE
    word[0] = 5
    assert lib.aegkv_fence_host_wait(base, 5, 0) == 1
    assert lib.aegkv_fence_host_wait(base, 6, 1000) == 0
    # a word with the failure mark answers "failed" (2) whatever the count
    word[0] = 3 | (1 << 62)
    assert lib.aegkv_fence_host_wait(base, 2, 0) == 2
    assert lib.aegkv_fence_host_wait(base, 9, 1000) == 2


def test_local_fence_entries_end_with_their_swapper():
    """A fence token raised in this process is waited on through the
    raising swap's event only while the raising swapper exists: once it is
    gone, its fence words may have been freed and the address reused by
    other words, so the entry must not answer for them."""
    import gc

    from aegaeon_amd import swapper as swm

    class Raiser:
        pass

    raiser, ev = Raiser(), object()
    addr = 0x7F00_0000_1000
    swm._note_local_fence(addr, 3, 5, ev, raiser)
    assert swm._local_fence_event(addr, 3, 5) is ev
    assert swm._local_fence_event(addr, 3, 2) is ev      # later raise covers earlier counts
    assert swm._local_fence_event(addr, 3, 6) is None    # not raised that far yet
    assert swm._local_fence_event(addr, 4, 1) is None    # another slot
    assert swm._local_fence_event(addr + 8, 3, 1) is None
    del raiser
    gc.collect()
    assert swm._local_fence_event(addr, 3, 1) is None
    assert (addr, 3) not in swm._local_fences


def test_local_fence_waits_on_the_move_the_token_names():
    """A token for count k is waited on through the event of count k (the
    first recorded count >= k), not through the latest swap's, so a consumer
    does not wait for later swaps queued on the producer's stream; once the
    history has dropped count k, the oldest kept event (later than k) stands
    in, which still orders the consumer after move k."""
    from aegaeon_amd import swapper as swm

    class Raiser:
        pass

    raiser = Raiser()
    addr = 0x7F00_0000_2000
    events = {c: object() for c in range(1, 200)}
    for c in (1, 2, 3):
        swm._note_local_fence(addr, 0, c, events[c], raiser)
    assert swm._local_fence_event(addr, 0, 1) is events[1]
    assert swm._local_fence_event(addr, 0, 2) is events[2]
    assert swm._local_fence_event(addr, 0, 3) is events[3]
    for c in range(4, 200):
        swm._note_local_fence(addr, 0, c, events[c], raiser)
    oldest = 200 - swm._LOCAL_FENCE_HISTORY
    assert swm._local_fence_event(addr, 0, 1) is events[oldest]      # trimmed: a later one
    assert swm._local_fence_event(addr, 0, 150) is events[150]
    assert swm._local_fence_event(addr, 0, 200) is None
    # another swapper raising the same words (the old one gone) starts afresh
    other = Raiser()
    swm._note_local_fence(addr, 0, 1, events[1], other)
    assert swm._local_fence_event(addr, 0, 150) is None
    del swm._local_fences[(addr, 0)]


def test_tuning_knobs(aegkv_lib):
    from aegaeon_amd import _lib

    prev = _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS)
    assert prev >= 1
    assert _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS, 4) == prev
    assert _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS, prev) == 4
    assert _lib.tune(_lib.TUNE_AUTO_D2H) in (_lib.MODE_DIRECT, _lib.MODE_STAGED)
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_AUTO_D2H, 7)
    with pytest.raises(ValueError):
        _lib.tune(99, 1)
    assert _lib.tune(_lib.TUNE_COPY_LDS_BYTES) == 96 * 1024
    assert _lib.tune(_lib.TUNE_SWAP_UNROLL) == 2
    assert _lib.tune(_lib.TUNE_STAGED_WORKGROUPS) == 0
    assert _lib.tune(_lib.TUNE_STAGED_OVERLAP) == 3
    assert _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED) == 112
    assert _lib.tune(_lib.TUNE_COPY_LANES) == 0
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_COPY_LANES, 512)
    assert _lib.tune(_lib.TUNE_COPY_UNROLL, 10) == 0
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_COPY_LANES, 256)           # 256 lanes have no unroll of 10
    assert _lib.tune(_lib.TUNE_COPY_UNROLL, 0) == 10
    assert _lib.tune(_lib.TUNE_COPY_LANES, 256) == 0
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_COPY_UNROLL, 5)
    assert _lib.tune(_lib.TUNE_COPY_UNROLL, 8) == 0
    assert _lib.tune(_lib.TUNE_COPY_UNROLL, 0) == 8
    assert _lib.tune(_lib.TUNE_COPY_LANES, 0) == 256
    with pytest.raises(ValueError, match="unknown tuning key 16"):
        _lib.tune(16)          # the retired library-driven DMA key
    assert _lib.tune(_lib.TUNE_COPY_ORDER) == 1              # by target id
    with pytest.raises(ValueError, match="copy order"):
        _lib.tune(_lib.TUNE_COPY_ORDER, 3)
    assert _lib.tune(_lib.TUNE_COPY_ORDER, 2) == 1
    assert _lib.tune(_lib.TUNE_COPY_ORDER, 1) == 2
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, 0)
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_STAGED_OVERLAP, 4)
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_STAGED_WORKGROUPS, 1 << 25)
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_SWAP_UNROLL, 3)
    with pytest.raises(ValueError):
        _lib.tune(_lib.TUNE_COPY_LDS_BYTES, 161 * 1024)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; asking for more exits with a message."""
    import sys

    res = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def _swap_blocks_call(lib, *, n_seg=2, page=(4096, 4096), hoff=(0, 4096), owners=(1, 1),
                      dev_blocks=8, kpp=(4,), host_blocks=6, host_page=8192, rank_off=0,
                      src=(1,), dst=(2,), grp=(0,), first=(0,), valid=(4,), is_in=0, mode=1):
    """Call aegkv_swap_blocks with placeholder (never dereferenced) pointers:
    every case here must be rejected before any HIP call."""
    import numpy as np

    P64 = ctypes.POINTER(ctypes.c_int64)
    arr = lambda x, t=np.int64: np.ascontiguousarray(np.array(x, dtype=t))  # noqa: E731
    keep = [arr(page), arr(hoff), arr(owners, np.uint64), arr(kpp), arr(src), arr(dst),
            arr(grp, np.int32), arr(first), arr(valid)]
    bases = (ctypes.c_void_p * n_seg)(*[0x10000 + 0x100000 * i for i in range(n_seg)])
    p = lambda a, t=P64: a.ctypes.data_as(t)  # noqa: E731
    return lib.aegkv_swap_blocks(
        n_seg, bases, p(keep[0]), p(keep[1]), p(keep[2], ctypes.POINTER(ctypes.c_uint64)),
        dev_blocks, len(kpp), p(keep[3]), ctypes.c_void_p(0x7000000), host_blocks, host_page,
        rank_off, len(src), p(keep[4]), p(keep[5]), p(keep[6], ctypes.POINTER(ctypes.c_int32)),
        p(keep[7]), p(keep[8]), is_in, mode, None, None)


@pytest.mark.parametrize("kwargs,code,word", [
    (dict(src=(8,)), -2, "source block id"),
    (dict(dst=(6,)), -2, "target block id"),
    (dict(src=(1, 2), dst=(3, 3), grp=(0, 0), first=(0, 0), valid=(4, 4)), -3, "twice"),
    (dict(grp=(1,)), -2, "group id"),
    (dict(first=(1,), valid=(4,)), -4, "run past a page"),
    (dict(first=(-1,), valid=(1,)), -4, "run past a page"),
    (dict(kpp=(3,)), -4, "equal kernel blocks"),
    (dict(hoff=(0, 4097)), -2, "overruns"),
    (dict(rank_off=8192), -1, "host_rank_offset"),
    (dict(dev_blocks=1 << 62), -2, "overflows"),
    (dict(host_blocks=1 << 62), -2, "overflows"),
    (dict(owners=(1, 2)), -2, "owner mask"),
    (dict(owners=(1, 0)), -1, "no owning group"),
    (dict(mode=7), -1, "transfer mode"),
])
def test_swap_blocks_rejections_before_any_hip_call(aegkv_lib, kwargs, code, word):
    rc = _swap_blocks_call(aegkv_lib, **kwargs)
    assert rc == code
    assert word.encode() in aegkv_lib.aegkv_last_error()


@pytest.mark.parametrize("entry", ["aegkv_copy_blocks", "aegkv_copy_blocks_noalloc"])
def test_copy_blocks_rejections_before_any_hip_call(aegkv_lib, entry):
    import numpy as np

    P64 = ctypes.POINTER(ctypes.c_int64)
    bases = (ctypes.c_void_p * 1)(0x10000)
    page = np.array([4096], np.int64)
    fn = getattr(aegkv_lib, entry)

    def call(src, dst, blocks=8):
        s, d = np.array(src, np.int64), np.array(dst, np.int64)
        return fn(1, bases, page.ctypes.data_as(P64), blocks, s.size, s.ctypes.data_as(P64),
                  d.ctypes.data_as(P64), None)

    assert call([1, 2], [2, 3]) == -5
    assert call([1, 2], [3, 3]) == -3
    assert call([1], [8]) == -2
    assert call([1], [2], blocks=1 << 62) == -2
    assert call([], []) == 0  # nothing to do, nothing touched


def _expected_copy_status(src, dst, blocks):
    """Status the copy checks give: ranges (pair order), then duplicate
    targets, then sources that are targets (brute force over the lists)."""
    for s_, d_ in zip(src, dst):
        if not (0 <= s_ < blocks and 0 <= d_ < blocks):
            return -2
    if len(set(dst)) != len(dst):
        return -3
    if set(src) & set(dst):
        return -5
    return 0


def test_copy_blocks_noalloc_checks_agree_with_copy_blocks(aegkv_lib):
    """The allocation-free entry checks ids by sorting where aegkv_copy_blocks
    uses a block map: on random invalid lists both give the status the
    brute-force rule gives (valid lists would reach the device checks)."""
    import numpy as np

    P64 = ctypes.POINTER(ctypes.c_int64)
    bases = (ctypes.c_void_p * 1)(0x10000)
    page = np.array([4096], np.int64)
    rng = np.random.default_rng(77)
    seen = set()
    for _ in range(600):
        blocks = int(rng.integers(2, 40))
        n = int(rng.integers(1, 30))
        src = rng.integers(-1, blocks + 1, n).astype(np.int64)
        dst = rng.integers(-1, blocks + 1, n).astype(np.int64)
        if rng.random() < 0.5:   # mostly in range, to reach the id checks
            src, dst = np.clip(src, 0, blocks - 1), np.clip(dst, 0, blocks - 1)
        want = _expected_copy_status(src.tolist(), dst.tolist(), blocks)
        if want == 0:
            continue
        seen.add(want)
        for entry in ("aegkv_copy_blocks", "aegkv_copy_blocks_noalloc"):
            rc = getattr(aegkv_lib, entry)(1, bases, page.ctypes.data_as(P64), blocks, n,
                                           src.ctypes.data_as(P64), dst.ctypes.data_as(P64),
                                           None)
            assert rc == want, (entry, src.tolist(), dst.tolist(), blocks)
    assert seen == {-2, -3, -5}


def test_copy_probe_rejections_before_any_hip_call(aegkv_lib):
    import numpy as np

    from aegaeon_amd import _lib

    P64 = ctypes.POINTER(ctypes.c_int64)
    bases = (ctypes.c_void_p * 1)(0x10000)
    page = np.array([4096], np.int64)
    s, d = np.array([1], np.int64), np.array([2], np.int64)

    def call(kind, sink=0x20000, pg=page, src=s, dst=d):
        return aegkv_lib.aegkv_copy_probe(kind, 1, bases, pg.ctypes.data_as(P64), 8, src.size,
                                          src.ctypes.data_as(P64), dst.ctypes.data_as(P64),
                                          sink, 7, None)

    assert call(0) == _lib.EINVAL
    assert call(3) == _lib.EINVAL
    assert call(_lib.PROBE_READ, sink=None) == _lib.EINVAL
    assert call(_lib.PROBE_WRITE, sink=0x20002) == _lib.EINVAL
    assert call(_lib.PROBE_READ, pg=np.array([4000 + 8], np.int64)) == _lib.EINVAL  # not 16 B
    assert b"16 B" in aegkv_lib.aegkv_last_error()
    assert call(_lib.PROBE_WRITE, dst=np.array([1], np.int64)) == _lib.EOVERLAP
    assert call(_lib.PROBE_READ, src=np.array([], np.int64), dst=np.array([], np.int64)) == 0


def test_load_slices_rejections_before_any_hip_call(aegkv_lib):
    import numpy as np

    from aegaeon_amd import _lib

    P64 = ctypes.POINTER(ctypes.c_int64)

    def call(dst, src, sizes, mode=1):
        n = len(sizes)
        d = (ctypes.c_void_p * max(n, 1))(*dst)
        s_ = (ctypes.c_void_p * max(n, 1))(*src)
        b = np.array(sizes, np.int64)
        return aegkv_lib.aegkv_load_slices(n, d, s_, b.ctypes.data_as(P64), mode, None)

    assert call([], [], []) == 0
    assert call([0x10000], [0x20000], [0]) == 0                       # empty slices skipped
    assert call([0x10000], [0x20000], [-1]) == _lib.EINVAL
    assert call([0x10000], [0x20000], [16], mode=7) == _lib.EINVAL
    assert call([0x10000, 0x10100], [0x20000, 0x30000], [512, 16]) == _lib.EOVERLAP
    assert b"overlap" in aegkv_lib.aegkv_last_error()
    assert call([0, 0x10000], [0x20000, 0x30000], [16, 16]) == _lib.EINVAL  # null target
    assert aegkv_lib.aegkv_load_slices(2, None, None, None, 1, None) == _lib.EINVAL


def test_qwen2_weight_contents():
    """Qwen2.5-7B's contents add up to its 7.6 B bf16 parameters: the
    embedding, 28 layers and the output head."""
    from aegaeon_amd import weights

    sizes = weights.qwen2_content_bytes()
    assert len(sizes) == 30
    params = sum(sizes) // 2
    assert 7.60e9 < params < 7.63e9
    assert sizes[1] == sizes[28] and sizes[0] == 152064 * 3584 * 2


def test_copy_blocks_noalloc_limits(aegkv_lib):
    """Calls beyond the fixed descriptor array are refused with a clear
    error before anything else happens."""
    import numpy as np

    from aegaeon_amd import _lib, ops

    P64 = ctypes.POINTER(ctypes.c_int64)
    n = ops.NOALLOC_MAX_PAIRS + 1
    ids = np.arange(n, dtype=np.int64)
    page = np.full(ops.NOALLOC_MAX_SEGMENTS + 1, 4096, np.int64)
    bases = (ctypes.c_void_p * page.size)(*([0x10000] * page.size))
    fn = aegkv_lib.aegkv_copy_blocks_noalloc
    rc = fn(1, bases, page.ctypes.data_as(P64), 2 * n, n, ids.ctypes.data_as(P64),
            (ids + n).ctypes.data_as(P64), None)
    assert rc == _lib.ENOMEM
    assert b"65537 pairs exceed" in aegkv_lib.aegkv_last_error()
    rc = fn(page.size, bases, page.ctypes.data_as(P64), 8, 1, ids.ctypes.data_as(P64),
            (ids + 1).ctypes.data_as(P64), None)
    assert rc == _lib.ENOMEM
    assert b"1025 segments exceed" in aegkv_lib.aegkv_last_error()
    # at the limits the size checks pass and the id checks run
    m = ops.NOALLOC_MAX_PAIRS
    dup = np.zeros(m, np.int64)
    rc = fn(ops.NOALLOC_MAX_SEGMENTS, bases, page.ctypes.data_as(P64), 2 * m, m,
            (ids[:m] + m).ctypes.data_as(P64), dup.ctypes.data_as(P64), None)
    assert rc == _lib.EDUP


def _run_with_env(env_extra, code):
    import os
    import sys

    env = dict(os.environ, **env_extra)
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         timeout=300, env=env, cwd=str(REPO))
    assert res.returncode == 0, res.stderr
    return res.stdout.strip()


def test_environment_picks_auto_modes_and_staging(aegkv_lib):
    code = ("from aegaeon_amd import _lib; "
            "print(_lib.tune(_lib.TUNE_AUTO_D2H), _lib.tune(_lib.TUNE_AUTO_H2D), "
            "_lib.tune(_lib.TUNE_STAGING_BYTES))")
    out = _run_with_env({"AEGKV_AUTO_D2H": "staged", "AEGKV_STAGING_BYTES": str(64 << 20)}, code)
    assert out.split() == ["2", "1", str(64 << 20)]


def test_invalid_environment_fails_every_transfer_call(aegkv_lib):
    code = ("from aegaeon_amd import _lib; lib = _lib.load(); "
            "rc = lib.aegkv_copy_blocks(1, None, None, 1, 0, None, None, None); "
            "print(rc, lib.aegkv_last_error().decode())")
    out = _run_with_env({"AEGKV_AUTO_H2D": "fast"}, code)
    assert out.startswith("-1 ") and "AEGKV_AUTO_H2D=fast" in out


def test_host_alloc_flags_rejections(aegkv_lib):
    import ctypes

    from aegaeon_amd import _lib

    p = ctypes.c_void_p()
    assert aegkv_lib.aegkv_host_alloc_flags(ctypes.byref(p), 4096, 4) == _lib.EINVAL
    assert b"flags" in aegkv_lib.aegkv_last_error()
    assert aegkv_lib.aegkv_host_alloc_flags(ctypes.byref(p), 0, 1) == _lib.EINVAL
    assert aegkv_lib.aegkv_host_alloc_flags(None, 16, 1) == _lib.EINVAL
    both = _lib.HOST_UNCACHED | _lib.HOST_COHERENT      # hipHostMalloc refuses the pair
    assert aegkv_lib.aegkv_host_alloc_flags(ctypes.byref(p), 4096, both) == _lib.EINVAL
    assert b"do not combine" in aegkv_lib.aegkv_last_error()
    assert aegkv_lib.aegkv_host_free(ctypes.c_void_p(0x1000)) == _lib.EINVAL   # not a pool
    assert b"live pool" in aegkv_lib.aegkv_last_error()


def test_migrate_blocks_rejections_before_any_hip_call(aegkv_lib):
    import ctypes

    from aegaeon_amd import _lib

    lib = aegkv_lib
    A = (ctypes.c_void_p * 2)(0x10000000, 0x20000000)
    B = (ctypes.c_void_p * 2)(0x30000000, 0x40000000)
    page = np.array([4096, 4096], np.int64)
    p64 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))  # noqa: E731

    def call(src_b, dst_b, src, dst, n_src=8, n_dst=8, n_seg=2):
        s, d = np.array(src, np.int64), np.array(dst, np.int64)
        return lib.aegkv_migrate_blocks(n_seg, src_b, dst_b, p64(page), n_src, n_dst, s.size,
                                        p64(s), p64(d), None, None)

    assert call(A, B, [1], [2], n_seg=0) == _lib.EINVAL
    assert call(None, B, [1], [2]) == _lib.EINVAL
    assert call(A, A, [1], [2]) == _lib.EOVERLAP          # one cache: use copy_blocks
    assert b"overlap" in lib.aegkv_last_error()
    assert call(A, B, [8], [2]) == _lib.ERANGE            # source id past the source cache
    assert call(A, B, [1], [3], n_dst=3) == _lib.ERANGE   # target id past the target cache
    assert call(A, B, [1, 2], [5, 5]) == _lib.EDUP
    assert call(A, B, [], []) == _lib.OK                   # nothing to move, no GPU needed


def test_launch_item_bound_before_any_hip_call(aegkv_lib):
    """The kernels walk their work items with a 32-bit grid-stride loop, so a
    launch may hold at most 2^32 - 1 - (2^32 - 1) // 256 items (the item
    index plus the largest grid then stays below 2^32 and the loop cannot
    wrap). Calls over that bound are refused before any HIP call; a call at
    exactly the bound passes it and only then meets the device checks (which
    fail here, with no GPU: the fake bases are not device memory). The sizes
    come from huge page sizes over placeholder pointers that nothing
    dereferences."""
    from aegaeon_amd import _lib

    lib = aegkv_lib
    limit = (2**32 - 1) - (2**32 - 1) // 256
    assert limit == 4_278_190_080 == 255 << 24
    p64 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))  # noqa: E731
    src, dst = np.array([0], np.int64), np.array([1], np.int64)

    def copy(entry, n_seg, page):
        bases = (ctypes.c_void_p * n_seg)(*[0x10000 * (i + 1) for i in range(n_seg)])
        pages = np.full(n_seg, page, np.int64)
        if entry == "migrate":
            other = (ctypes.c_void_p * n_seg)(*[(1 << 60) + 0x10000 * i
                                                for i in range(n_seg)])
            return lib.aegkv_migrate_blocks(n_seg, bases, other, p64(pages), 2, 2, 1, p64(src),
                                            p64(dst), None, None)
        return getattr(lib, entry)(n_seg, bases, p64(pages), 2, 1, p64(src), p64(dst), None)

    # copy shapes: a page of 2^24 x 10 rows of 16 KiB moves 10 rows per item
    # (2^24 items per tile); a page of (limit + 1) rows of 16 KiB (not a
    # multiple of 2, 3 or 5) moves one row per item
    at_limit = ((limit // 10) * 10 * 16384, 10)      # 10 segments x limit/10 items
    over = ((limit + 1) * 16384, 1)                  # 1 segment x (limit + 1) items
    for entry in ("aegkv_copy_blocks", "aegkv_copy_blocks_noalloc", "migrate"):
        page, n_seg = over
        assert copy(entry, n_seg, page) == _lib.EINVAL, entry
        assert b"work items of one launch" in lib.aegkv_last_error(), entry
        page, n_seg = at_limit
        rc = copy(entry, n_seg, page)
        assert rc == _lib.EINVAL and b"device memory" in lib.aegkv_last_error(), (entry, rc)

    # swap kernels move 8 KiB per item (256 lanes x 2 loads of 16 B)
    for items, refused in ((limit + 1, True), (limit, False)):
        page = items * 8192
        rc = _swap_blocks_call(lib, n_seg=1, page=(page,), hoff=(0,), owners=(1,), kpp=(1,),
                               host_page=page, dev_blocks=2, host_blocks=1, src=(0,), dst=(0,),
                               valid=(1,))
        assert rc == _lib.EINVAL
        msg = lib.aegkv_last_error()
        assert (b"work items of one launch" in msg) == refused, msg

    # weight slices: 8 KiB per item as well
    for items, refused in ((limit + 1, True), (limit, False)):
        d = (ctypes.c_void_p * 1)(0x10000)
        h = (ctypes.c_void_p * 1)(0x20000)
        b = np.array([items * 8192], np.int64)
        rc = lib.aegkv_load_slices(1, d, h, p64(b), 1, None)
        assert rc == _lib.EINVAL
        msg = lib.aegkv_last_error()
        assert (b"work items of one launch" in msg) == refused, msg
