"""GPU tests of resource lifetimes inside one process: streams the library
recorded events on and that are then destroyed, pinned host pools carved out
of uncached memory the library keeps, closed dedicated streams, and the
allocation-free copy's first call under graph capture in a fresh process."""

import numpy as np
import pytest
import torch

from aegaeon_amd import ops

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _segments(gpu, n_seg, n_blocks, tile, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    segs = []
    for _ in range(n_seg):
        t = torch.empty(n_blocks, tile, dtype=torch.uint8, device=gpu)
        t.view(torch.int32).random_(generator=g)
        segs.append(t)
    return segs


def _layout(segs, pool, tile):
    n_seg = len(segs)
    return ops.SegmentLayout(segs, [tile] * n_seg, [s * tile for s in range(n_seg)],
                             [1] * n_seg, segs[0].size(0), [1], pool.tensor, n_seg * tile, 0)


def _entries(n):
    return np.zeros(n, np.int32), np.zeros(n, np.int64), np.ones(n, np.int64)


def test_streams_destroyed_after_library_calls_then_new_streams_and_pools(gpu):
    """The sequence that once ended a benchmark process, in one process at a
    moderate size: swaps and a block copy on three CU-masked streams at once
    (their descriptor regions and events recorded there), the streams
    destroyed; the uncached pool freed and two smaller uncached pools carved
    out of its memory; a ring call on another stream (which retires the
    regions the destroyed streams read); four new dedicated streams; a swap-out
    and a swap-in on them. Every step is checked byte for byte."""
    _say("streams destroyed after library calls, pools carved, new streams")
    n_seg, n_blocks, tile = 24, 512, 64 * 1024        # 24 x 32 MiB segments
    segs = _segments(gpu, n_seg, n_blocks, tile, 31)
    page = n_seg * tile
    rng = np.random.default_rng(31)
    perm = rng.permutation(n_blocks)
    n_out, n_in, n_cp = 96, 64, 48
    out_ids, in_ids = perm[:n_out], perm[n_out:n_out + n_in]
    csrc = perm[n_out + n_in:n_out + n_in + n_cp]
    cdst = perm[n_out + n_in + n_cp:n_out + n_in + 2 * n_cp]
    pool = ops.PinnedHostPool((n_out + n_in) * page, uncached=True)
    base_a = pool.tensor.data_ptr()
    lay = _layout(segs, pool, tile)
    hp = rng.permutation(n_out + n_in)
    hx, hy = hp[:n_out], hp[n_out:]
    zi, fi, oi = _entries(n_in)
    zo, fo, oo = _entries(n_out)
    lay.swap(in_ids, hy, zi, fi, oi, False)           # the incoming blocks' host pages
    di = torch.from_numpy(in_ids).to(gpu)
    want_in = [t[di].clone() for t in segs]
    for t in segs:
        t.index_fill_(0, di, 0)
    before = [t.clone() for t in segs]
    masks = [ops.xcd_cu_mask(8), ops.xcd_cu_mask(8), ops.xcd_cu_mask(24, first=8)]
    owners = [ops.DedicatedStream(gpu, m) for m in masks]
    torch.cuda.synchronize()
    lay.swap(out_ids, hx, zo, fo, oo, False, stream=owners[0].stream)
    lay.swap(hy, in_ids, zi, fi, oi, True, stream=owners[1].stream)
    ops.copy_blocks(segs, csrc, cdst, stream=owners[2].stream)
    torch.cuda.synchronize()
    host = pool.tensor.view(n_out + n_in, n_seg, tile)[torch.from_numpy(hx)].to(gpu)
    dcs, dcd = torch.from_numpy(csrc).to(gpu), torch.from_numpy(cdst).to(gpu)
    do = torch.from_numpy(out_ids).to(gpu)
    for s in range(n_seg):
        assert torch.equal(host[:, s], before[s][do]), s
        assert torch.equal(segs[s][di], want_in[s]), s
        assert torch.equal(segs[s][dcd], before[s][dcs]), s
    for o in owners:
        o.close()
        with pytest.raises(RuntimeError, match="closed"):
            o.stream.synchronize()
    del lay, host
    pinned_before, free_before = ops.host_pinned_usage()
    pool.free()
    pinned_freed, free_freed = ops.host_pinned_usage()
    assert pinned_freed == pinned_before                 # uncached memory stays pinned
    assert free_freed >= free_before + (n_out + n_in) * page

    # two smaller uncached pools come out of memory the library already
    # holds (the freed pool's or another free range): nothing new is pinned
    p1 = ops.PinnedHostPool(40 * page, uncached=True)
    p2 = ops.PinnedHostPool(40 * page, uncached=True)
    pinned_now, free_now = ops.host_pinned_usage()
    assert pinned_now == pinned_freed, "a new pinned block was allocated"
    assert free_now == free_freed - 80 * page
    assert abs(p1.tensor.data_ptr() - p2.tensor.data_ptr()) >= 40 * page
    del base_a

    # a ring call on the current stream retires the destroyed streams' regions
    ops.copy_blocks(segs, cdst[:8], csrc[:8])
    torch.cuda.synchronize()
    for s in range(n_seg):
        assert torch.equal(segs[s][dcs[:8]], before[s][dcs[:8]]), s

    # four new dedicated streams; swaps through the carved pools
    fresh = [ops.DedicatedStream(gpu) for _ in range(4)]
    lay1, lay2 = _layout(segs, p1, tile), _layout(segs, p2, tile)
    z, f, o = _entries(40)
    ids_a, ids_b = perm[:40], perm[40:80]
    lay1.swap(ids_a, np.arange(40), z, f, o, False, stream=fresh[0].stream)
    lay2.swap(ids_b, np.arange(40), z, f, o, False, stream=fresh[3].stream)
    torch.cuda.synchronize()
    back = perm[n_blocks - 40:]
    lay1.swap(np.arange(40), back, z, f, o, True, stream=fresh[1].stream)
    torch.cuda.synchronize()
    da, db, dback = (torch.from_numpy(x).to(gpu) for x in (ids_a, ids_b, back))
    h2 = p2.tensor.view(40, n_seg, tile).to(gpu)
    for s in range(n_seg):
        assert torch.equal(segs[s][dback], segs[s][da]), s
        assert torch.equal(h2[:, s], segs[s][db]), s
    for st in fresh:
        st.close()
    del lay1, lay2, h2
    p1.free()
    p2.free()


def _carve_child(q):
    """Fresh process (an empty free list): the carving addresses."""
    try:
        import torch

        from aegaeon_amd import ops as cops

        torch.cuda.set_device(0)
        kib = 1024
        size = 8 * 1024 * kib + 12 * kib
        a = cops.PinnedHostPool(size, uncached=True)
        base = a.tensor.data_ptr()
        a.free()
        b = cops.PinnedHostPool(3 * 1024 * kib, uncached=True)
        c = cops.PinnedHostPool(3 * 1024 * kib + 1, uncached=True)   # rounded up to 4 KiB
        d = cops.PinnedHostPool(2 * 1024 * kib, uncached=True)
        got = [x.tensor.data_ptr() - base for x in (b, c, d)]
        pinned, free = cops.host_pinned_usage()
        c.free()
        b.free()                                        # merges with c's range
        e = cops.PinnedHostPool(6 * 1024 * kib + 4 * kib, uncached=True)
        got.append(e.tensor.data_ptr() - base)
        q.put(("ok", (got, pinned, free, size)))
    except Exception as exc:
        q.put(("error", repr(exc)))


def test_uncached_pools_are_carved_and_merged(gpu):
    """Uncached pools: in a fresh process, a freed pool's memory serves the
    next pools in address order (smallest free range that fits, from its
    start), with nothing new pinned; two freed neighbours merge into one
    range that a pool of their joint size reuses. Here, a carved pool at an
    offset works for swaps in both directions, and a pool of a freed pool's
    exact (unusual) size gets the same memory back."""
    mp = torch.multiprocessing.get_context("spawn")
    q = mp.Queue()
    child = mp.Process(target=_carve_child, args=(q,), daemon=True)
    child.start()
    try:
        kind, value = q.get(timeout=240)
    finally:
        child.join(60)
        if child.is_alive():
            child.kill()
    assert kind == "ok", value
    got, pinned, free, size = value
    kib = 1024
    assert got == [0, 3 * 1024 * kib, 6 * 1024 * kib + 4 * kib, 0], got
    assert pinned == size and free == size - 8 * 1024 * kib - 4 * kib

    size = 8 * 1024 * kib + 12 * kib                   # an unusual size: no other range fits
    a = ops.PinnedHostPool(size, uncached=True)
    base = a.tensor.data_ptr()
    a.free()
    c = ops.PinnedHostPool(size, uncached=True)
    assert c.tensor.data_ptr() == base
    # swaps through the reused pool, both directions
    tile = 64 * kib
    segs = _segments(gpu, 4, 64, tile, 5)
    lay = _layout(segs, c, tile)
    n = (3 * 1024 * kib) // (4 * tile)
    z, f, o = _entries(n)
    src = np.arange(1, 1 + n)
    lay.swap(src, np.arange(n), z, f, o, False)
    lay.swap(np.arange(n), src + 20, z, f, o, True)
    torch.cuda.synchronize()
    for t in segs:
        assert torch.equal(t[20 + 1:20 + 1 + n], t[1:1 + n])
    del lay
    c.free()


def test_closed_dedicated_stream_refuses_use(gpu):
    """After close(), a DedicatedStream's torch stream raises instead of
    handing the runtime a destroyed HIP stream (library calls too), and
    KVSwapper.close() leaves a swapper that refuses further swaps."""
    owner = ops.DedicatedStream(gpu)
    assert not owner.stream.closed
    owner.close()
    assert owner.stream.closed
    for fn in (owner.stream.synchronize, owner.stream.query,
               lambda: owner.stream.wait_event(torch.cuda.Event()),
               lambda: owner.stream.cuda_stream):
        with pytest.raises(RuntimeError, match="closed"):
            fn()
    segs = _segments(gpu, 2, 8, 4096, 1)
    with pytest.raises(RuntimeError, match="closed"):
        ops.copy_blocks(segs, [1], [2], stream=owner.stream)


def _noalloc_capture_child(q):
    """Fresh process: the first libaegkv call is copy_blocks_noalloc inside
    a graph capture (the library is loaded there too); three replays, each
    checked against the pairs it captured."""
    try:
        import torch

        from aegaeon_amd import ops as child_ops

        dev = torch.device("cuda:0")
        torch.cuda.set_device(dev)
        segs = [torch.randint(0, 256, (64, 8192), dtype=torch.uint8, device=dev)
                for _ in range(3)]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        st = torch.cuda.Stream(dev)
        with torch.cuda.graph(g, stream=st):
            child_ops.copy_blocks_noalloc(segs, [1, 2, 3], [10, 11, 12])
        torch.cuda.synchronize()
        ok = []
        for r in range(3):
            for t in segs:
                t[[10, 11, 12]] = 0
                t[[1, 2, 3]] = r + 7
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            ok.append(all(bool((t[[10, 11, 12]] == r + 7).all()) for t in segs))
        q.put(("ok", ok))
    except Exception as exc:       # reported to the parent, which fails the test
        q.put(("error", repr(exc)))


def test_noalloc_first_call_under_capture_in_a_fresh_process(gpu):
    """A process whose very first library call is the allocation-free copy
    under graph capture: the library's per-device set-up runs when it is
    loaded, outside any stream operation, and the captured copy replays
    correctly."""
    _say("allocation-free copy, first call under capture, fresh process")
    mp = torch.multiprocessing.get_context("spawn")
    q = mp.Queue()
    child = mp.Process(target=_noalloc_capture_child, args=(q,), daemon=True)
    child.start()
    try:
        kind, value = q.get(timeout=240)
    finally:
        child.join(60)
        if child.is_alive():
            child.kill()
    assert kind == "ok", value
    assert value == [True, True, True]
