"""GPU tests of failed fence waits: a swap behind a wait that gives up moves
nothing, and every consumer of its completion sees the failure.

The reference never runs a swap before its source is ready: it waits on the
source events without a limit (aegaeon/worker.py:2387) and stops the worker
when it cannot get them (:2364-2368). Here fence waits are bounded, so the
give-up is forced from the host with a tiny budget on a word nobody
signals: every kernel still ends normally.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from aegaeon_amd import ops

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _cache(gpu, n_blocks, page, seed):
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache

    cache = allocate_composite_cache([KVCacheTensorSpec(n_blocks * page, ("l0",))], n_blocks, gpu)
    g = torch.Generator(device=gpu).manual_seed(seed)
    cache.backing[0].view(torch.int32).random_(generator=g)
    return cache


def test_timed_out_source_fails_the_swap_and_everything_downstream(gpu):
    """Swapper A swaps two blocks out behind a FenceToken that is never
    signalled, with a 2 ms budget. Then:
      - A's swap moved nothing (its host pages keep their zeros);
      - A's fence word and host word carry FENCE_FAILED;
      - A's MoveEvent, its FenceToken (query and synchronize), the ledger's
        reclaim and wait_for_all_move_out raise MoveFailedError, and stay
        failed; a new swap on that stream is refused;
      - consumer B in this process, swapping A's host pages back in behind
        A's token (through A's event and a guard merge), moves nothing and
        reports failure too;
      - a consumer waiting on A's fence word on the device ends its wait at
        once (no 30 s budget spent), its guard reads 2 and its guarded swap
        moves nothing;
      - A's swap-in stream, which waited on nothing, still works."""
    from aegaeon_amd.cache_groups import CacheGroupConfig, CacheGroupRuntimeConfig
    from aegaeon_amd.planner import BlockPools
    from aegaeon_amd.swapper import FenceToken, KVSwapper, MoveEvent

    _say("failed fence wait: swap, tokens, events, ledger, consumers")
    n_blocks, page = 16, 64 * 1024
    caches = [_cache(gpu, n_blocks, page, s) for s in (7, 8)]
    pool = ops.PinnedHostPool(8 * page)
    pool.tensor.zero_()
    words = torch.zeros(8, dtype=torch.int64, device=gpu)
    hw = ops.HostFenceWords(8)
    descr = [CacheGroupRuntimeConfig("attention", 16, 16)]
    a = KVSwapper(caches[0], [{"l0"}], descr, pool.tensor, fence_words=words, fence_slots=(0, 1),
                  fence_host=hw, fence_timeout_s=0.002, dedicated_streams=True)
    b = KVSwapper(caches[1], [{"l0"}], descr, pool.tensor, fence_words=words, fence_slots=(2, 3),
                  fence_host=hw, fence_timeout_s=30, dedicated_streams=True)
    before = [c.segment_pages(0).clone() for c in caches]
    torch.cuda.synchronize()
    try:
        ev = a.swap_blocks([1], [2, 3], [0, 1], [0, 0], [0, 0], [1, 1], [FenceToken(7, 9)],
                           False)
        assert isinstance(ev, MoveEvent)
        with pytest.raises(ops.MoveFailedError, match="fence wait timed out"):
            ev.synchronize()
        assert ev.failed
        assert a.guards.value(0) == 1 and a.guards.value(1) == 0
        assert bool((pool.tensor == 0).all()), "the swap behind the failed wait moved bytes"
        assert int(words[0]) == 1 | ops.FENCE_FAILED
        token = a.last_fence
        assert token == FenceToken(0, 1, hw.name)
        with pytest.raises(ops.MoveFailedError):
            token.query()
        with pytest.raises(ops.MoveFailedError):
            token.synchronize(timeout_s=1)
        assert int(hw.words[0]) == 1 | ops.FENCE_FAILED
        # the controller's ledger keeps the move and its sources
        shape = (page // 2,)
        pools = BlockPools(1, 8 * page)
        pools.register_gpu_space(0, n_blocks, shape, (CacheGroupConfig("attention", 16, 16),))
        free_before = list(pools.gpu_free_blocks[0])
        plan = SimpleNamespace(release_source_block_ids=[2, 3], source_location=0,
                               block_shape=shape)
        pools.record_move(plan, [ev])
        with pytest.raises(ops.MoveFailedError):
            pools.reclaim_gpu_moves(0, wait=False)
        with pytest.raises(ops.MoveFailedError):
            pools.reclaim_gpu_moves(0, wait=True)
        assert pools.gpu_free_blocks[0] == free_before
        assert len(pools.move_events_gpu[0]) == 1
        # the swapper itself: sticky, and no new swap on that stream
        for _ in range(2):
            with pytest.raises(ops.MoveFailedError, match="fence wait gave up"):
                a.wait_for_all_move_out()
        with pytest.raises(ops.MoveFailedError):
            a.swap_blocks([2], [4], [2], [0], [0], [1], [None], False)

        # consumer B in this process: A's token is waited on through A's
        # event, and A's guard is merged into B's swap-in guard
        ev_b = b.swap_blocks([1], [0, 1], [5, 6], [0, 0], [0, 0], [1, 1], [token], True)
        with pytest.raises(ops.MoveFailedError, match="source move failed"):
            ev_b.synchronize()
        assert b.guards.value(1) == 2 and b.guards.value(0) == 0
        assert torch.equal(caches[1].segment_pages(0), before[1]), "B's swap-in moved bytes"
        assert int(words[3]) == 1 | ops.FENCE_FAILED
        with pytest.raises(ops.MoveFailedError):
            b.wait_for_all_move_in()

        # a consumer on the device: the marked word ends its wait at once
        import time

        guard = torch.zeros(1, dtype=torch.int64, device=gpu)
        st = ops.DedicatedStream(gpu)
        lay = ops.SegmentLayout([caches[1].segment_pages(0)], [page], [0], [1], n_blocks, [1],
                                pool.tensor, page, 0)
        t0 = time.perf_counter()
        ops.fence_wait(words, 0, 1, guard, 0, timeout_s=30, stream=st.stream)
        lay.swap([0, 1], [9, 10], np.zeros(2, np.int32), np.zeros(2, np.int64),
                 np.ones(2, np.int64), True, stream=st.stream, guard=guard)
        st.stream.synchronize()
        assert time.perf_counter() - t0 < 10, "the wait did not see the failure mark"
        assert int(guard[0]) == 2
        assert torch.equal(caches[1].segment_pages(0), before[1]), "the guarded swap moved bytes"
        st.close()

        # A's other stream waited on nothing and still moves blocks
        ev_in = a.swap_blocks([3], [4, 5], [8, 9], [0, 0], [0, 0], [1, 1], [None], True)
        ev_in.synchronize()
        a.wait_for_all_move_in()
        pages = caches[0].segment_pages(0)
        for h, d in ((4, 8), (5, 9)):
            assert torch.equal(pages[d].cpu(), pool.tensor.view(8, page)[h]), (h, d)
        assert int(words[1]) == 1                     # no mark on the swap-in word
    finally:
        torch.cuda.synchronize()
        a.close()
        b.close()
        hw.close()
    pool.free()


def test_guard_merge_and_guarded_signal(gpu):
    """aegkv_guard_merge marks a guard (2) behind the stream's work when the
    source guard is set, and leaves it alone when the source is clear;
    aegkv_fence_signal with a clear guard raises the word to the value, with
    a set guard to value | FENCE_FAILED; a publish with a set guard marks
    the host word; guarded migrations move nothing."""
    src = ops.GuardWords(2)
    dst = ops.GuardWords(2)
    words = torch.zeros(2, dtype=torch.int64, device=gpu)
    hw = ops.HostFenceWords(2)
    st = ops.DedicatedStream(gpu)
    try:
        src.tensor[1] = 1
        ops.guard_merge(dst.tensor, 0, src.tensor, 0, device=gpu, stream=st.stream)  # clear
        ops.guard_merge(dst.tensor, 1, src.tensor, 1, device=gpu, stream=st.stream)  # set
        ops.fence_signal(words, 0, 5, guard=dst.tensor, guard_index=0, stream=st.stream)
        ops.fence_signal(words, 1, 5, guard=dst.tensor, guard_index=1, stream=st.stream)
        ops.fence_publish(hw, 0, 5, guard=dst.tensor, guard_index=0, device=gpu, stream=st.stream)
        ops.fence_publish(hw, 1, 5, guard=dst.tensor, guard_index=1, device=gpu, stream=st.stream)
        n, page = 8, 4096
        a = [torch.randint(0, 256, (n, page), dtype=torch.uint8, device=gpu) for _ in range(2)]
        b = [torch.zeros(n, page, dtype=torch.uint8, device=gpu) for _ in range(2)]
        ops.migrate_blocks(a, b, [1, 2], [3, 4], stream=st.stream, guard=dst.tensor,
                           guard_index=1)
        st.stream.synchronize()
        assert dst.value(0) == 0 and dst.value(1) == 2
        assert int(words[0]) == 5 and int(words[1]) == 5 | ops.FENCE_FAILED
        assert ops.fence_host_wait(hw, 0, 5)
        with pytest.raises(ops.MoveFailedError):
            ops.fence_host_wait(hw, 1, 5)
        assert all(int(t.sum()) == 0 for t in b), "the guarded migration moved bytes"
        ops.migrate_blocks(a, b, [1, 2], [3, 4], stream=st.stream, guard=dst.tensor,
                           guard_index=0)
        st.stream.synchronize()
        assert all(torch.equal(t[[3, 4]], s[[1, 2]]) for s, t in zip(a, b))
    finally:
        torch.cuda.synchronize()
        st.close()
        hw.close()


@pytest.mark.parametrize("mode", ["direct", "staged"])
def test_guarded_swaps_in_both_modes(gpu, mode):
    """A set guard stops a swap in either transfer mode: a swap-in moves
    nothing into the cache (STAGED: the scatter kernel reads the guard; the
    runtime's copies into staging still run); a swap-out leaves the cache
    alone (DIRECT: the host pages too). With the guard clear, the same
    calls move the blocks."""
    _say(f"guarded swaps, {mode}")
    n_seg, n_blocks, tile = 4, 32, 16 * 1024
    g = torch.Generator(device=gpu).manual_seed(41)
    segs = [torch.empty(n_blocks, tile, dtype=torch.uint8, device=gpu) for _ in range(n_seg)]
    for t in segs:
        t.view(torch.int32).random_(generator=g)
    page = n_seg * tile
    pool = ops.PinnedHostPool(8 * page)
    host = pool.tensor.view(8, n_seg, tile)
    host.view(torch.int32).random_()
    lay = ops.SegmentLayout(segs, [tile] * n_seg, [s * tile for s in range(n_seg)], [1] * n_seg,
                            n_blocks, [1], pool.tensor, page, 0)
    guards = ops.GuardWords(1)
    st = ops.DedicatedStream(gpu)
    z, f, o = np.zeros(3, np.int32), np.zeros(3, np.int64), np.ones(3, np.int64)
    try:
        before_dev = [t.clone() for t in segs]
        before_host = host.clone()
        guards.tensor[0] = 1
        lay.swap([0, 1, 2], [5, 6, 7], z, f, o, True, mode=mode, stream=st.stream,
                 guard=guards.tensor)
        lay.swap([8, 9, 10], [3, 4, 5], z, f, o, False, mode=mode, stream=st.stream,
                 guard=guards.tensor)
        st.stream.synchronize()
        for a, b in zip(segs, before_dev):
            assert torch.equal(a, b), "a guarded swap changed the cache"
        if mode == "direct":
            assert torch.equal(host, before_host), "a guarded swap-out wrote host pages"
        else:   # STAGED swap-out pages are undefined; only the untouched ones are checked
            for h in (0, 1, 2, 6, 7):
                assert torch.equal(host[h], before_host[h]), h
        guards.tensor[0] = 0
        lay.swap([0, 1, 2], [5, 6, 7], z, f, o, True, mode=mode, stream=st.stream,
                 guard=guards.tensor)
        lay.swap([8, 9, 10], [3, 4, 5], z, f, o, False, mode=mode, stream=st.stream,
                 guard=guards.tensor)
        st.stream.synchronize()
        for s in range(n_seg):
            for h, d in ((0, 5), (1, 6), (2, 7)):
                assert torch.equal(segs[s][d].cpu(), host[h, s]), (s, h, d)
            for d, h in ((8, 3), (9, 4), (10, 5)):
                assert torch.equal(host[h, s], segs[s][d].cpu()), (s, d, h)
    finally:
        torch.cuda.synchronize()
        st.close()
    del lay, host
    pool.free()
