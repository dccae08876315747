"""GPU parity: libaegkv kernels against the oracle and the golden fixtures.

Every comparison is byte equality. Small cases compare with the oracle run
on host copies of the same seeded inputs; full-size cases (the benchmark
shapes) check size-independent properties: swap-out/swap-in round trips,
host pages equal to the device tiles they came from, untouched blocks
unchanged.
"""

import ctypes
import itertools

import numpy as np
import pytest
import torch

from aegaeon_amd import _lib, ops

pytestmark = pytest.mark.gpu


MODES = ("direct", "staged")


def _say(*a):
    print(*a, flush=True)


def _pool_from(arr: np.ndarray) -> ops.PinnedHostPool:
    pool = ops.PinnedHostPool(arr.size)
    pool.tensor.copy_(torch.from_numpy(arr.reshape(-1)))
    return pool


# ------------------------------------------------------------ golden cases --

@pytest.mark.parametrize("mode", MODES)
def test_legacy_swap_golden(gpu, golden, mode):
    z = golden("legacy_swap.npz")
    shape = tuple(int(x) for x in z["cache_shape"])
    cache = torch.from_numpy(z["cache"].copy()).view(torch.bfloat16).view(shape).to(gpu)
    pool = torch.from_numpy(z["pool"].copy()).view(torch.bfloat16).view(
        (z["pool"].shape[0],) + shape[1:]).pin_memory()
    ops.swap(z["out_src"].tolist(), z["out_dst"].tolist(), False, cache, pool, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(pool.view(torch.uint8).reshape(pool.shape[0], -1).numpy(),
                          z["pool_after_out"])
    ops.swap(z["in_src"].tolist(), z["in_dst"].tolist(), True, cache, pool, mode=mode)
    torch.cuda.synchronize()
    got = cache.cpu().view(torch.uint8).reshape(shape[0], -1).numpy()
    assert np.array_equal(got, z["cache_after_in"])


@pytest.mark.parametrize("dtype", [torch.uint8, torch.float32])
def test_legacy_swap_block_size_for_other_dtypes(gpu, oracle, dtype):
    """The one deliberate difference of ops.swap from swap.cu: the block is
    kv_cache.numel() * element_size / size(0) bytes, where swap.cu:34 uses
    numel * 2 / size(0) whatever the dtype. For bf16/fp16 the two agree
    (test_legacy_swap_golden); for a 1-byte cache the reference's formula
    gives twice the block (it would copy the next block too, and read past
    the cache for the last one), for a 4-byte cache half of it. The product
    moves exactly one block; the oracle, which keeps the reference's
    formula, moves the other amount."""
    n_dev, n_host, per_block = 8, 6, 64
    elem = torch.tensor([], dtype=dtype).element_size()
    rng = np.random.default_rng(elem)
    cache_np = rng.integers(0, 256, n_dev * per_block * elem, dtype=np.uint8)
    cache = torch.from_numpy(cache_np.copy()).view(dtype).view(n_dev, per_block).to(gpu)
    pool = torch.zeros(n_host, per_block, dtype=dtype).pin_memory()
    ops.swap([3], [1], False, cache, pool)
    torch.cuda.synchronize()
    block = per_block * elem
    got = pool.view(torch.uint8).reshape(-1).numpy()
    want = np.zeros(n_host * block, np.uint8)
    want[block:2 * block] = cache_np[3 * block:4 * block]      # exactly one block
    assert np.array_equal(got, want)
    ref = np.zeros(n_host * block, np.uint8)
    oracle.swap_legacy([3], [1], False, cache_np.copy(), cache_np.size // elem, n_dev, ref)
    ref_block = (cache_np.size // elem) * 2 // n_dev            # swap.cu:34
    assert ref_block == 2 * block // elem and ref_block != block
    assert not np.array_equal(ref, want)                        # the documented difference


@pytest.mark.parametrize("mode", MODES)
def test_composite_swap_golden(gpu, golden, mode):
    z = golden("composite_swap.npz")
    segs = [torch.from_numpy(z[f"seg{s}"].copy()).to(gpu) for s in range(5)]
    pool = _pool_from(z["host"])
    common = (z["page"], z["cpu_off"], z["owners"], int(z["n_gpu"]), z["kpp"], pool.tensor,
              int(z["host_page"]), int(z["tp_rank"]) * int(z["composite"]))
    ops.swap_segments(segs, *common, z["src"], z["dst"], z["grp"], z["first"], z["valid"],
                      False, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(pool.tensor.numpy().reshape(z["host"].shape), z["host_after_out"])
    ops.swap_segments(segs, *common, z["in_src"], z["in_dst"], z["grp"], z["first"],
                      z["valid"], True, mode=mode)
    torch.cuda.synchronize()
    for s in range(5):
        assert np.array_equal(segs[s].cpu().numpy(), z[f"seg{s}_after_in"]), s
    pool.free()


def test_copy_blocks_golden(gpu, golden):
    z = golden("copy_blocks.npz")
    segs = [torch.from_numpy(z[f"seg{i}"].copy()).to(gpu) for i in range(3)]
    ops.copy_blocks(segs, z["src"], z["dst"])
    torch.cuda.synchronize()
    for i in range(3):
        assert np.array_equal(segs[i].cpu().numpy(), z[f"seg{i}_after"])


# ------------------------------------------------------- seeded vs oracle --

def _random_layout(rng):
    """Mixed page sizes (16 B multiples up to 80 KiB), 3 groups, TP 2."""
    n_groups = 3
    kpp = np.array([1, 4, 2], np.int64)
    n_seg = 11
    page = (rng.integers(1, 5, n_seg) * 4 * 16 * rng.choice([1, 16, 80, 320], n_seg)).astype(np.int64)
    owners = rng.integers(1, 1 << n_groups, n_seg).astype(np.uint64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    return kpp, page, owners, cpu_off


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("mode", MODES)
def test_seeded_swap_vs_oracle(gpu, oracle, seed, mode):
    rng = np.random.default_rng(100 + seed)
    kpp, page, owners, cpu_off = _random_layout(rng)
    composite = int(page.sum())
    tp_size, tp_rank = 2, seed % 2
    host_page = composite * tp_size
    n_gpu, n_host, n = 48, 40, 30
    _say("seeded swap", seed, mode, "segments", len(page), "composite", composite)
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    host_np = rng.integers(0, 256, (n_host, host_page), dtype=np.uint8)
    grp = rng.integers(0, 3, n).astype(np.int32)
    first = np.array([rng.integers(0, kpp[g] + 1) for g in grp], np.int64)
    valid = np.array([rng.integers(0, kpp[g] - f + 1) for g, f in zip(grp, first)], np.int64)
    src = rng.permutation(n_gpu)[:n]
    dst = rng.permutation(n_host)[:n]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    pool = _pool_from(host_np)
    common = (page, cpu_off, owners, n_gpu, kpp, pool.tensor, host_page, tp_rank * composite)
    ops.swap_segments(segs, *common, src, dst, grp, first, valid, False, mode=mode)
    want_host = host_np.copy()
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       want_host.reshape(-1), host_page, tp_rank, composite, src, dst, grp,
                       first, valid, False)
    torch.cuda.synchronize()
    assert np.array_equal(pool.tensor.numpy().reshape(want_host.shape), want_host)
    # swap back in to other device ids
    back = rng.permutation(n_gpu)[:n]
    ops.swap_segments(segs, *common, dst, back, grp, first, valid, True, mode=mode)
    want_segs = [x.copy() for x in segs_np]
    oracle.swap_blocks([x.reshape(-1) for x in want_segs], page, cpu_off, owners, n_gpu, kpp,
                       want_host.reshape(-1), host_page, tp_rank, composite, dst, back, grp,
                       first, valid, True)
    torch.cuda.synchronize()
    for s in range(len(page)):
        assert np.array_equal(segs[s].cpu().numpy(), want_segs[s]), s
    pool.free()


def test_prepared_layout_reused_across_calls_vs_oracle(gpu, oracle):
    """One SegmentLayout serves a sequence of calls of varying size, both
    directions and both modes (including an empty call); after each call the
    device and host bytes equal the oracle's state."""
    rng = np.random.default_rng(21)
    kpp, page, owners, cpu_off = _random_layout(rng)
    composite = int(page.sum())
    n_gpu, n_host = 40, 36
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    host_np = rng.integers(0, 256, (n_host, composite), dtype=np.uint8)
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    pool = _pool_from(host_np)
    lay = ops.SegmentLayout(segs, page, cpu_off, owners, n_gpu, kpp, pool.tensor, composite, 0)
    for step, (n, is_in, mode) in enumerate([(30, False, "direct"), (0, True, "staged"),
                                              (7, True, "staged"), (1, False, "staged"),
                                              (25, True, "direct"), (3, False, "auto")]):
        _say("prepared layout step", step, "n", n, "swap_in", is_in, mode)
        grp = rng.integers(0, 3, n).astype(np.int32)
        first = np.array([rng.integers(0, kpp[g] + 1) for g in grp], np.int64)
        valid = np.array([rng.integers(0, kpp[g] - f + 1) for g, f in zip(grp, first)],
                         np.int64)
        dev_ids = rng.permutation(n_gpu)[:n]
        host_ids = rng.permutation(n_host)[:n]
        src, dst = (host_ids, dev_ids) if is_in else (dev_ids, host_ids)
        lay.swap(src, dst, grp, first, valid, is_in, mode=mode)
        oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu,
                           kpp, host_np.reshape(-1), composite, 0, composite, src, dst, grp,
                           first, valid, is_in)
        torch.cuda.synchronize()
        assert np.array_equal(pool.tensor.numpy().reshape(host_np.shape), host_np), step
        for s in range(len(page)):
            assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), (step, s)
    del lay
    pool.free()


def test_prepared_layout_rejects_bad_geometry(gpu):
    seg = torch.zeros(8, 256, dtype=torch.uint8, device=gpu)
    pool = ops.PinnedHostPool(4 * 256)
    with pytest.raises(ValueError, match="holds"):
        ops.SegmentLayout([seg], [256], [0], [1], 9, [1], pool.tensor, 256, 0)
    with pytest.raises(ValueError, match="lengths"):
        ops.SegmentLayout([seg], [256, 256], [0], [1], 8, [1], pool.tensor, 256, 0)
    with pytest.raises(ValueError, match="host tensor"):
        ops.SegmentLayout([seg], [256], [0], [1], 8, [1], seg.view(-1), 256, 0)
    lay = ops.SegmentLayout([seg], [256], [0], [1], 8, [1], pool.tensor, 256, 0)
    with pytest.raises(ValueError, match="unequal lengths"):
        lay.swap([1], [0], [0, 0], [0], [1], False)
    pool.free()


def test_threads_swap_concurrently_on_their_own_streams(gpu):
    """Four host threads share one layout (and the library's descriptor ring
    and DMA streams) and swap out, each on its own stream, alternating
    DIRECT and STAGED; every call lands its own blocks in its own host pages."""
    import threading

    n_gpu, page, n, n_thr, iters = 64, 8192, 16, 4, 40
    segs = [torch.randint(0, 256, (n_gpu, page), dtype=torch.uint8, device=gpu)
            for _ in range(3)]
    segs_cpu = [x.cpu() for x in segs]
    pool = ops.PinnedHostPool(n_thr * n * 3 * page)
    lay = ops.SegmentLayout(segs, [page] * 3, [0, page, 2 * page], [1, 1, 1], n_gpu, [1],
                            pool.tensor, 3 * page, 0)
    host = pool.tensor.view(n_thr * n, 3, page)
    errors = []

    def worker(t):
        try:
            st = torch.cuda.Stream(gpu)
            rng = np.random.default_rng(t)
            dst = t * n + np.arange(n)
            for it in range(iters):
                src = rng.permutation(n_gpu)[:n]
                lay.swap(src, dst, np.zeros(n, np.int32), np.zeros(n, np.int64), np.ones(n, np.int64), False,
                         mode=MODES[it % 2], stream=st)
                st.synchronize()
                mine = host[t * n:(t + 1) * n]
                idx = torch.from_numpy(src)
                for s in range(3):
                    if not torch.equal(mine[:, s], segs_cpu[s][idx]):
                        errors.append((t, it, s))
        except Exception as e:  # surfaced below
            errors.append(e)

    _say("threads", n_thr, "iterations", iters)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(n_thr)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads)
    assert errors == []
    del lay
    pool.free()


@pytest.mark.parametrize("mode", MODES)
def test_unaligned_host_pool_vs_oracle(gpu, oracle, mode):
    """A host pool starting 1 byte into its allocation forces the
    byte-granular kernel path (and unaligned DMA in staged mode)."""
    rng = np.random.default_rng(7)
    page = np.array([256, 512, 64], np.int64)
    cpu_off = np.array([0, 256, 768], np.int64)
    owners = np.ones(3, np.uint64)
    kpp = np.array([4], np.int64)
    composite = 832
    n_gpu, n_host, n = 16, 12, 9
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    raw = ops.PinnedHostPool(n_host * composite + 1)
    raw.tensor.zero_()
    host = raw.tensor.narrow(0, 1, n_host * composite)
    src, dst = rng.permutation(n_gpu)[:n], rng.permutation(n_host)[:n]
    first = rng.integers(0, 3, n)
    valid = np.array([rng.integers(0, 4 - f + 1) for f in first])
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    ops.swap_segments(segs, page, cpu_off, owners, n_gpu, kpp, host, composite, 0, src, dst,
                      np.zeros(n, np.int32), first, valid, False, mode=mode)
    want = np.zeros((n_host, composite), np.uint8)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       want.reshape(-1), composite, 0, composite, src, dst,
                       np.zeros(n, np.int32), first, valid, False)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy().reshape(want.shape), want)
    assert raw.tensor[0].item() == 0
    raw.free()


def test_copy_blocks_seeded_vs_oracle(gpu, oracle):
    rng = np.random.default_rng(3)
    n = 64
    page = np.array([16, 4096, 160 * 1024, 48 * 1024 + 16, 100], np.int64)  # last: byte path
    segs_np = [rng.integers(0, 256, (n, int(p)), dtype=np.uint8) for p in page]
    perm = rng.permutation(n)
    src, dst = perm[:25], perm[25:50]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np[:4]]
    ops.copy_blocks(segs, src, dst)
    oracle.copy_blocks([x.reshape(-1) for x in segs_np[:4]], page[:4], n, src, dst)
    torch.cuda.synchronize()
    for s in range(4):
        assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), s
    # unaligned page size takes the byte path
    seg = torch.from_numpy(segs_np[4].copy()).to(gpu)
    ops.copy_blocks([seg], src, dst)
    oracle.copy_blocks([segs_np[4].reshape(-1)], page[4:], n, src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(seg.cpu().numpy(), segs_np[4])


@pytest.mark.parametrize("case", range(96))
def test_randomized_block_copies_vs_oracle(gpu, oracle, restore_tuning, case):
    """Random copy_blocks within one cache (1-20 segments of 16 B-multiple
    or odd pages, repeated sources, random kernel shapes, grids, LDS
    reservations and store kinds) against the oracle; every third case a
    migrate_blocks between two caches of different block counts against
    the closed form dst[d] = src[s]."""
    rng = np.random.default_rng(7000 + case)
    _lib.tune(_lib.TUNE_COPY_UNROLL, int(rng.choice([0, 0, 1, 2, 3, 4, 5, 6, 8, 10])))
    _lib.tune(_lib.TUNE_COPY_WGS_PER_CU, int(rng.choice([0, 0, 1, 4])))
    _lib.tune(_lib.TUNE_COPY_LDS_BYTES, int(rng.choice([0, 96 << 10])))
    _lib.tune(_lib.TUNE_NT_STORES, int(rng.integers(0, 2)))
    n_seg = int(rng.integers(1, 21))
    if rng.random() < 0.2:
        page = rng.choice([5, 48, 100, 4096 + 3], n_seg)           # byte path
    else:
        page = rng.choice([16, 256, 4096, 16384, 32768, 48 * 1024 + 16, 160 * 1024], n_seg)
    page = page.astype(np.int64)
    n_src = int(rng.integers(2, 81))
    migrate = case % 3 == 2
    n_dst = int(rng.integers(2, 81)) if migrate else n_src
    _say("randomized block copies", case, "migrate" if migrate else "copy_blocks", "segments",
         n_seg, "blocks", n_src, n_dst)
    src_np = [rng.integers(0, 256, (n_src, int(p)), dtype=np.uint8) for p in page]
    if migrate:
        n = int(rng.integers(0, n_dst + 1))
        dst_ids = rng.permutation(n_dst)[:n]
        src_ids = rng.integers(0, n_src, n)
        dst_np = [rng.integers(0, 256, (n_dst, int(p)), dtype=np.uint8) for p in page]
        src_t = [torch.from_numpy(x.copy()).to(gpu) for x in src_np]
        dst_t = [torch.from_numpy(x.copy()).to(gpu) for x in dst_np]
        ops.migrate_blocks(src_t, dst_t, src_ids, dst_ids)
        for x, y in zip(src_np, dst_np):
            y[dst_ids] = x[src_ids]
        torch.cuda.synchronize()
        for i in range(n_seg):
            assert np.array_equal(dst_t[i].cpu().numpy(), dst_np[i]), i
            assert np.array_equal(src_t[i].cpu().numpy(), src_np[i]), i
        return
    perm = rng.permutation(n_src)
    n = int(rng.integers(0, n_src // 2 + 1))
    dst_ids = perm[:n]
    pool = perm[n:]
    src_ids = pool[rng.integers(0, pool.size, n)] if n else perm[:0]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in src_np]
    ops.copy_blocks(segs, src_ids, dst_ids)
    oracle.copy_blocks([x.reshape(-1) for x in src_np], page, n_src, src_ids, dst_ids)
    torch.cuda.synchronize()
    for i in range(n_seg):
        assert np.array_equal(segs[i].cpu().numpy(), src_np[i]), i


@pytest.fixture
def restore_tuning():
    keys = (_lib.TUNE_COPY_UNROLL, _lib.TUNE_COPY_WGS_PER_CU, _lib.TUNE_SWAP_SHAPE_AUTO,
            _lib.TUNE_SWAP_OUT_WORKGROUPS, _lib.TUNE_SWAP_IN_WORKGROUPS, _lib.TUNE_NT_STORES,
            _lib.TUNE_STAGED_DMA_STREAMS, _lib.TUNE_STAGING_BYTES, _lib.TUNE_COPY_LDS_BYTES,
            _lib.TUNE_SWAP_UNROLL, _lib.TUNE_STAGED_WORKGROUPS, _lib.TUNE_STAGED_OVERLAP,
            _lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, _lib.TUNE_COPY_LANES, _lib.TUNE_COPY_ORDER)
    saved = {k: _lib.tune(k) for k in keys}
    yield
    for k, v in saved.items():
        _lib.tune(k, v)


@pytest.mark.parametrize("page", [16 * 1024, 64 * 1024, 160 * 1024, 4096, 4000 + 16 * 3])
def test_copy_probes_touch_only_their_tiles(gpu, page):
    """The read probe changes nothing; the write probe fills exactly the
    target tiles with its pattern (third word 0x5a5a5a5a, fourth the magic
    value) and leaves every other byte alone."""
    n_seg, n_blocks, n = 6, 96, 30
    g = torch.Generator(device=gpu).manual_seed(page)
    segs = [torch.randint(0, 256, (n_blocks, page), dtype=torch.uint8, device=gpu, generator=g)
            for _ in range(n_seg)]
    before = [t.clone() for t in segs]
    rng = np.random.default_rng(page)
    perm = rng.permutation(n_blocks)
    src, dst = perm[:n], perm[n:2 * n]
    sink = torch.zeros(4, dtype=torch.int32, device=gpu)
    ops.copy_probe(ops.PROBE_READ, segs, src, dst, sink)
    torch.cuda.synchronize()
    for a, b in zip(segs, before):
        assert torch.equal(a, b)
    magic = 0x12345677
    ops.copy_probe(ops.PROBE_WRITE, segs, src, dst, sink, magic=magic)
    torch.cuda.synchronize()
    di = torch.from_numpy(dst).to(gpu)
    keep = torch.ones(n_blocks, dtype=torch.bool, device=gpu)
    keep[di] = False
    for a, b in zip(segs, before):
        assert torch.equal(a[keep], b[keep])
        words = a[di].view(torch.int32).view(n, page // 16, 4)
        assert bool((words[:, :, 2] == 0x5a5a5a5a).all())
        assert bool((words[:, :, 3] == magic).all())


def test_copy_blocks_every_shape_vs_oracle(gpu, oracle, restore_tuning):
    """Every instantiated copy shape, both grid policies and three LDS
    reservations (none, one workgroup per CU, the whole LDS), on tiles that
    divide evenly, leave tails, or are smaller than one row."""
    rng = np.random.default_rng(21)
    n = 24
    page = np.array([160 * 1024, 48 * 1024 + 16, 4096, 32 * 1024, 112], np.int64)
    shapes = [(1024, u) for u in (0, 1, 2, 3, 4, 5, 6, 8, 10)] + [(256, u) for u in (1, 2, 4, 8)]
    for (lanes, unroll), wpc, lds in itertools.product(shapes, (0, 3),
                                                       (0, 96 * 1024, 160 * 1024)):
        _lib.tune(_lib.TUNE_COPY_UNROLL, 0)
        _lib.tune(_lib.TUNE_COPY_LANES, lanes)
        _lib.tune(_lib.TUNE_COPY_UNROLL, unroll)
        _lib.tune(_lib.TUNE_COPY_WGS_PER_CU, wpc)
        _lib.tune(_lib.TUNE_COPY_LDS_BYTES, lds)
        segs_np = [rng.integers(0, 256, (n, int(p)), dtype=np.uint8) for p in page[:4]]
        perm = rng.permutation(n)
        src, dst = perm[:9], perm[9:18]
        segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
        ops.copy_blocks(segs, src, dst)
        oracle.copy_blocks([x.reshape(-1) for x in segs_np], page[:4], n, src, dst)
        torch.cuda.synchronize()
        for s in range(4):
            assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), (lanes, unroll, wpc, lds, s)


@pytest.mark.parametrize("order", [0, 1, 2])
def test_copy_blocks_pair_orders_vs_oracle(gpu, oracle, restore_tuning, order):
    """The library may hand the kernel the pairs in the caller's order, by
    target id or by source id (a counting sort, one pass per byte of the
    largest id): every order gives the oracle's bytes, for ids of one, two
    and three bytes, pairs already in order, one pair, and the
    allocation-free copy."""
    _lib.tune(_lib.TUNE_COPY_ORDER, order)
    rng = np.random.default_rng(70 + order)
    page = 4096
    for n_blocks, n in ((200, 60), (5000, 1500), (70000, 300), (70000, 1), (3000, 1000)):
        segs_np = [rng.integers(0, 256, (n_blocks, page // 2), dtype=np.uint8) for _ in range(2)]
        perm = rng.permutation(n_blocks)
        src, dst = perm[:n], perm[n:2 * n]
        if n_blocks == 3000:                      # already in order of both ids
            src, dst = np.sort(src), np.sort(dst)
        segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
        ops.copy_blocks(segs, src, dst)
        oracle.copy_blocks([x.reshape(-1) for x in segs_np], np.array([page // 2] * 2, np.int64),
                           n_blocks, src, dst)
        torch.cuda.synchronize()
        for s in range(2):
            assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), (order, n_blocks, n, s)
    segs_np = [rng.integers(0, 256, (900, 1024), dtype=np.uint8) for _ in range(3)]
    perm = rng.permutation(900)
    src, dst = perm[:400], perm[400:800]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    ops.copy_blocks_noalloc(segs, src, dst)
    oracle.copy_blocks([x.reshape(-1) for x in segs_np], np.array([1024] * 3, np.int64), 900,
                       src, dst)
    torch.cuda.synchronize()
    for s in range(3):
        assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), (order, "noalloc", s)


@pytest.mark.parametrize("shape_auto,unroll", [(0, 4), (0, 2), (0, 1), (1, 4)])
@pytest.mark.parametrize("wpc", [1, 37, 4096])
def test_swap_kernel_shapes_vs_oracle(gpu, oracle, restore_tuning, shape_auto, unroll, wpc):
    _lib.tune(_lib.TUNE_SWAP_SHAPE_AUTO, shape_auto)
    _lib.tune(_lib.TUNE_SWAP_UNROLL, unroll)
    _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS, wpc)
    _lib.tune(_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, wpc)
    _lib.tune(_lib.TUNE_SWAP_IN_WORKGROUPS, wpc)
    rng = np.random.default_rng(31 + wpc)
    page = np.array([160 * 1024, 32 * 1024, 4096, 48 * 1024 + 16 * 4], np.int64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    owners = np.array([1, 3, 2, 1], np.uint64)
    kpp = np.array([1, 4], np.int64)
    composite = int(page.sum())
    n_gpu, n_host, n = 20, 16, 10
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    grp = rng.integers(0, 2, n).astype(np.int32)
    first = np.array([0 if g == 0 else rng.integers(0, 4) for g in grp], np.int64)
    valid = np.array([1 if g == 0 else rng.integers(0, 4 - f + 1) for g, f in zip(grp, first)],
                     np.int64)
    src, dst = rng.permutation(n_gpu)[:n], rng.permutation(n_host)[:n]
    for mode in MODES:
        segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
        pool = ops.PinnedHostPool(n_host * composite)
        pool.tensor.zero_()
        ops.swap_segments(segs, page, cpu_off, owners, n_gpu, kpp, pool.tensor, composite, 0,
                          src, dst, grp, first, valid, False, mode=mode)
        want = np.zeros((n_host, composite), np.uint8)
        oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                           want.reshape(-1), composite, 0, composite, src, dst, grp, first,
                           valid, False)
        torch.cuda.synchronize()
        assert np.array_equal(pool.tensor.numpy().reshape(want.shape), want), mode
        back = rng.permutation(n_gpu)[:n]
        ops.swap_segments(segs, page, cpu_off, owners, n_gpu, kpp, pool.tensor, composite, 0,
                          dst, back, grp, first, valid, True, mode=mode)
        want_segs = [x.copy() for x in segs_np]
        oracle.swap_blocks([x.reshape(-1) for x in want_segs], page, cpu_off, owners, n_gpu,
                           kpp, want.reshape(-1), composite, 0, composite, dst, back, grp, first,
                           valid, True)
        torch.cuda.synchronize()
        for s in range(len(page)):
            assert np.array_equal(segs[s].cpu().numpy(), want_segs[s]), (mode, s)
        pool.free()


@pytest.mark.parametrize("dma_streams", [0, 1, 2, 3, 4])
def test_staged_dma_fanout_vs_oracle(gpu, oracle, restore_tuning, dma_streams):
    """STAGED copies forked over 0-4 library streams (and split into small
    staging chunks) land exactly where the oracle puts them, both ways."""
    _lib.tune(_lib.TUNE_STAGED_DMA_STREAMS, dma_streams)
    _lib.tune(_lib.TUNE_STAGING_BYTES, 1 << 20)
    _lib.tune(_lib.TUNE_STAGED_WORKGROUPS, (0, 3, 64, 1)[dma_streams % 4])
    rng = np.random.default_rng(50 + dma_streams)
    page = np.array([64 * 1024, 16 * 1024, 48 * 1024], np.int64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    owners = np.ones(3, np.uint64)
    kpp = np.array([4], np.int64)
    composite = int(page.sum())
    n_gpu, n_host, n = 40, 48, 33
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    src = rng.permutation(n_gpu)[:n]
    dst = np.sort(rng.permutation(n_host)[:n])  # partly contiguous host runs
    first = rng.integers(0, 2, n)
    valid = np.array([rng.integers(0, 4 - f + 1) for f in first])
    grp = np.zeros(n, np.int32)
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    pool = ops.PinnedHostPool(n_host * composite)
    pool.tensor.zero_()
    common = (page, cpu_off, owners, n_gpu, kpp, pool.tensor, composite, 0)
    ops.swap_segments(segs, *common, src, dst, grp, first, valid, False, mode="staged")
    want = np.zeros((n_host, composite), np.uint8)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       want.reshape(-1), composite, 0, composite, src, dst, grp, first, valid,
                       False)
    torch.cuda.synchronize()
    assert np.array_equal(pool.tensor.numpy().reshape(want.shape), want)
    back = rng.permutation(n_gpu)[:n]
    ops.swap_segments(segs, *common, dst, back, grp, first, valid, True, mode="staged")
    want_segs = [x.copy() for x in segs_np]
    oracle.swap_blocks([x.reshape(-1) for x in want_segs], page, cpu_off, owners, n_gpu, kpp,
                       want.reshape(-1), composite, 0, composite, dst, back, grp, first, valid,
                       True)
    torch.cuda.synchronize()
    for s in range(3):
        assert np.array_equal(segs[s].cpu().numpy(), want_segs[s]), s
    pool.free()


@pytest.mark.parametrize("dma_streams,contiguous,overlap",
                         [(2, True, 3), (2, False, 3), (4, False, 3), (2, False, 0),
                          (1, True, 3), (3, True, 1), (3, False, 2)])
def test_staged_chunked_round_trip(gpu, restore_tuning, dma_streams, contiguous, overlap):
    """STAGED over library streams with two staging buffers in flight (the
    gather or scatter of one chunk beside the copies of another), one chunk
    at a time, and on the caller's stream; with 8 MiB chunks of 3 Qwen3-4B
    pages, 200 blocks pass through 67 chunks each way, so each buffer is
    reused many times. Host pages must equal the device tiles they came
    from and the round trip must be exact."""
    _lib.tune(_lib.TUNE_STAGED_DMA_STREAMS, dma_streams)
    _lib.tune(_lib.TUNE_STAGING_BYTES, 8 << 20)
    _lib.tune(_lib.TUNE_STAGED_OVERLAP, overlap)
    _say("STAGED chunks", dma_streams, "contiguous" if contiguous else "scattered", overlap)
    segs = _kv_segments(36, 512, 8, 128, torch.bfloat16, gpu, 11)
    tile = 16 * 8 * 128 * 2
    S, n = len(segs), 200
    pool = ops.PinnedHostPool(512 * S * tile)
    g = torch.Generator().manual_seed(12 + dma_streams)
    perm = torch.randperm(512, generator=g).numpy()
    out_ids, in_ids = perm[:n], perm[n:2 * n]
    host_ids = (np.arange(100, 100 + n) if contiguous
                else torch.randperm(512, generator=g)[:n].numpy())
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, 512, [1], pool.tensor,
              S * tile, 0)
    z = np.zeros(n, np.int32)
    ops.swap_segments(segs, *common, out_ids, host_ids, z, z, z + 1, False, mode="staged")
    torch.cuda.synchronize()
    dev_out = torch.from_numpy(out_ids).to(gpu)
    want = torch.stack([s_.view(512, -1).view(torch.uint8)[dev_out] for s_ in segs], dim=1)
    pages = pool.tensor.view(512, S, tile)[torch.from_numpy(host_ids)].to(gpu)
    assert torch.equal(pages, want)
    del pages, want
    ops.swap_segments(segs, *common, host_ids, in_ids, z, z, z + 1, True, mode="staged")
    torch.cuda.synchronize()
    dev_in = torch.from_numpy(in_ids).to(gpu)
    for s in range(S):
        assert torch.equal(segs[s][dev_in], segs[s][dev_out]), s
    pool.free()


def _random_case(rng):
    """A random composite layout, host pool geometry and swap list: 1-4
    cache groups with 1-17 kernel blocks per page, 1-24 segments owned by
    random group sets, 16 B-multiple or odd tile units, TP 1-3."""
    n_groups = int(rng.integers(1, 5))
    kpp = rng.choice([1, 2, 4, 8, 17], n_groups).astype(np.int64)
    n_seg = int(rng.integers(1, 25))
    owners = rng.integers(1, 1 << n_groups, n_seg).astype(np.uint64)
    byte_path = rng.random() < 0.25
    page = []
    for o in owners:
        lcm = 1
        for g in range(n_groups):
            if (int(o) >> g) & 1:
                lcm = int(np.lcm(lcm, int(kpp[g])))
        unit = int(rng.choice([3, 7, 5])) if byte_path else int(rng.choice([16, 32, 64, 1024, 4096]))
        page.append(lcm * unit)
    page = np.array(page, np.int64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    tp_size = int(rng.integers(1, 4))
    n_gpu, n_host = int(rng.integers(1, 41)), int(rng.integers(1, 41))
    n = int(rng.integers(0, min(n_gpu, n_host) + 1))
    grp = rng.integers(0, n_groups, n).astype(np.int32)
    first = np.array([rng.integers(0, kpp[g] + 1) for g in grp], np.int64)
    valid = np.array([rng.integers(0, kpp[g] - f + 1) for g, f in zip(grp, first)], np.int64)
    return dict(kpp=kpp, page=page, owners=owners, cpu_off=cpu_off, tp_size=tp_size,
                tp_rank=int(rng.integers(0, tp_size)), n_gpu=n_gpu, n_host=n_host, n=n,
                grp=grp, first=first, valid=valid)


@pytest.mark.parametrize("case", range(160))
def test_randomized_swaps_vs_oracle(gpu, oracle, restore_tuning, case):
    """Random layouts (groups, extents, TP ranks, byte and 16 B paths),
    both modes, random staging chunk sizes, DMA stream counts, overlap
    settings and host-pool alignments: swap-out then swap-in to other ids,
    each byte-equal to the oracle."""
    rng = np.random.default_rng(9000 + case)
    c = _random_case(rng)
    mode = MODES[case % 2]
    _lib.tune(_lib.TUNE_STAGING_BYTES, int(rng.choice([1 << 20, 3 << 20, 512 << 20])))
    _lib.tune(_lib.TUNE_STAGED_DMA_STREAMS, int(rng.choice([0, 1, 2, 4])))
    _lib.tune(_lib.TUNE_STAGED_OVERLAP, int(rng.integers(0, 4)))
    rng.integers(0, 2)  # draw kept so that every seed still yields the same case
    shift = int(rng.choice([0, 0, 16, 1]))
    page, kpp, n = c["page"], c["kpp"], c["n"]
    composite = int(page.sum())
    host_page = composite * c["tp_size"]
    _say("randomized swap", case, mode, "segments", len(page), "groups", len(kpp), "entries", n,
         "tp", c["tp_size"], "host shift", shift)
    segs_np = [rng.integers(0, 256, (c["n_gpu"], int(p)), dtype=np.uint8) for p in page]
    host_np = rng.integers(0, 256, (c["n_host"], host_page), dtype=np.uint8)
    raw = ops.PinnedHostPool(host_np.size + shift)
    host = raw.tensor.narrow(0, shift, host_np.size)
    host.copy_(torch.from_numpy(host_np.reshape(-1)))
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    src = rng.permutation(c["n_gpu"])[:n]
    dst = rng.permutation(c["n_host"])[:n]
    common = (page, c["cpu_off"], c["owners"], c["n_gpu"], kpp, host, host_page,
              c["tp_rank"] * composite)
    ops.swap_segments(segs, *common, src, dst, c["grp"], c["first"], c["valid"], False,
                      mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, c["cpu_off"], c["owners"],
                       c["n_gpu"], kpp, host_np.reshape(-1), host_page, c["tp_rank"], composite,
                       src, dst, c["grp"], c["first"], c["valid"], False)
    back = rng.permutation(c["n_gpu"])[:n]
    ops.swap_segments(segs, *common, dst, back, c["grp"], c["first"], c["valid"], True,
                      mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, c["cpu_off"], c["owners"],
                       c["n_gpu"], kpp, host_np.reshape(-1), host_page, c["tp_rank"], composite,
                       dst, back, c["grp"], c["first"], c["valid"], True)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy().reshape(host_np.shape), host_np)
    for i in range(len(page)):
        assert np.array_equal(segs[i].cpu().numpy(), segs_np[i]), i
    raw.free()


@pytest.mark.parametrize("dma_streams", [1, 2, 4])
def test_staged_swap_out_and_in_at_once(gpu, restore_tuning, dma_streams):
    """A STAGED swap-out and a STAGED swap-in enqueued together on two
    streams, each double-buffered over its own DMA streams with 8 MiB
    chunks (67 chunks each way): the host pages and device tiles land as
    the closed form says and nothing else changes."""
    _lib.tune(_lib.TUNE_STAGING_BYTES, 8 << 20)
    _lib.tune(_lib.TUNE_STAGED_OVERLAP, 3)
    _lib.tune(_lib.TUNE_STAGED_DMA_STREAMS, dma_streams)
    segs = _kv_segments(36, 512, 8, 128, torch.bfloat16, gpu, 21)
    tile = 16 * 8 * 128 * 2
    S, n = len(segs), 200
    pool = ops.PinnedHostPool(512 * S * tile)
    host = pool.tensor.view(512, S, tile)
    g = torch.Generator().manual_seed(22)
    host.copy_(torch.randint(0, 256, host.shape, dtype=torch.uint8, generator=g))
    perm = torch.randperm(512, generator=g).numpy()
    out_ids, in_ids = perm[:n], perm[n:2 * n]
    out_host, in_host = np.arange(n), np.arange(256, 256 + n)
    want_in = host[torch.from_numpy(in_host)].to(gpu)            # what the swap-in brings
    before = [x.clone() for x in segs]
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, 512, [1], pool.tensor, S * tile, 0)
    lay = ops.SegmentLayout(segs, *common)
    a, b = torch.cuda.Stream(gpu), torch.cuda.Stream(gpu)
    z, one = np.zeros(n, np.int32), np.ones(n, np.int64)
    torch.cuda.synchronize()
    lay.swap(out_ids, out_host, z, z, one, False, mode="staged", stream=a)
    lay.swap(in_host, in_ids, z, z, one, True, mode="staged", stream=b)
    torch.cuda.synchronize()
    do, di = torch.from_numpy(out_ids).to(gpu), torch.from_numpy(in_ids).to(gpu)
    got_out = host[torch.from_numpy(out_host)].to(gpu)
    keep = torch.ones(512, dtype=torch.bool, device=gpu)
    keep[di] = False
    for s in range(S):
        assert torch.equal(got_out[:, s], before[s][do].view(torch.uint8).reshape(n, -1)), s
        assert torch.equal(segs[s][di].view(torch.uint8).reshape(n, -1), want_in[:, s]), s
        assert torch.equal(segs[s][keep], before[s][keep]), s
    del lay
    pool.free()


# ------------------------------------------------------------ weight loads --

@pytest.mark.parametrize("mode,aligned", [("direct", True), ("direct", False),
                                          ("staged", True), ("staged", False)])
def test_load_slices_vs_expectation(gpu, mode, aligned):
    """Weight slices of random sizes (empty, small, a few MiB) at random
    offsets of one pinned pool and one device arena land byte for byte;
    arena bytes outside the slices keep their guard value. Aligned: every
    size and offset a 16 B multiple (the kernel's 16 B path); otherwise odd
    sizes and offsets (its byte path)."""
    rng = np.random.default_rng(31 + 2 * (mode == "staged") + aligned)
    sizes = [0, 1, 15, 16, 4096, 8192 + 48, 3 << 20, 65537, 16 * 1000] + \
        [int(x) for x in rng.integers(1, 200_000, 24)]
    if aligned:
        sizes = [-(-n // 16) * 16 for n in sizes]
    host = ops.PinnedHostPool(64 << 20)
    host.tensor.copy_(torch.from_numpy(rng.integers(0, 256, 64 << 20, dtype=np.uint8)))
    arena = torch.full((64 << 20,), 0xA5, dtype=torch.uint8, device=gpu)
    src, dst, hoff, doff = [], [], 0, 0
    for n in sizes:
        if not aligned:
            hoff += int(rng.integers(0, 7))
            doff += int(rng.integers(0, 7))
        src.append(host.tensor.narrow(0, hoff, n))
        dst.append(arena.narrow(0, doff, n))
        hoff += -(-max(n, 1) // 256) * 256
        doff += -(-max(n, 1) // 256) * 256
    ops.load_slices(dst, src, mode=mode)
    torch.cuda.synchronize()
    covered = torch.zeros(64 << 20, dtype=torch.bool, device=gpu)
    for d, h in zip(dst, src):
        assert torch.equal(d, h.to(gpu))
        if d.numel():
            covered[d.data_ptr() - arena.data_ptr():][:d.numel()] = True
    assert bool((arena[~covered] == 0xA5).all())
    with pytest.raises(ValueError, match="overlap"):
        ops.load_slices([arena.narrow(0, 0, 512), arena.narrow(0, 256, 512)],
                        [host.tensor.narrow(0, 0, 512)] * 2, mode=mode)
    with pytest.raises(ValueError, match="pinned"):
        ops.load_slices([arena.narrow(0, 0, 64)], [torch.zeros(64, dtype=torch.uint8)], mode=mode)
    host.free()


@pytest.mark.parametrize("mode", MODES)
def test_qwen25_7b_weight_load_full_size(gpu, mode):
    """A whole Qwen2.5-7B bf16 model (30 contents, 15.2 GB) from pinned
    host memory into a device arena in one call: every content equals the
    bytes it came from."""
    from aegaeon_amd import weights

    sizes = weights.qwen2_content_bytes()
    host = weights.HostWeights(sizes)
    dev_w = weights.DeviceWeights(sizes, gpu)
    g = torch.Generator(device=gpu).manual_seed(7)
    origin = []
    for h in host.slices:      # random contents, written to the host through the DMA
        o = torch.randint(0, 256, (h.numel(),), dtype=torch.uint8, device=gpu, generator=g)
        h.copy_(o)
        origin.append(o)
    torch.cuda.synchronize()
    weights.load_model(dev_w, host, mode=mode)
    torch.cuda.synchronize()
    for i, (d, o) in enumerate(zip(dev_w.slices, origin)):
        assert torch.equal(d, o), i
    del origin
    host.free()


# ------------------------------------------------------- uncached host pool --

@pytest.mark.parametrize("mode", MODES)
def test_uncached_host_pool_vs_oracle(gpu, oracle, mode):
    """Swaps through an uncached (MTYPE UC) pool land where the oracle puts
    them; a released uncached pool is parked and reused by the next
    uncached pool of a fitting size."""
    rng = np.random.default_rng(90)
    kpp, page, owners, cpu_off = _random_layout(rng)
    composite = int(page.sum())
    n_gpu, n_host, n = 24, 20, 16
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    first_pool = ops.PinnedHostPool(n_host * composite, uncached=True)
    first_ptr = first_pool.tensor.data_ptr()
    first_pool.free()
    pool = ops.PinnedHostPool(n_host * composite, uncached=True)
    assert pool.tensor.data_ptr() == first_ptr          # parked memory reused
    small = ops.PinnedHostPool(1 << 16, uncached=True)
    small_ptr = small.tensor.data_ptr()
    small.free()
    big = ops.PinnedHostPool(8 << 20, uncached=True)
    big_ptr = big.tensor.data_ptr()
    big.free()
    again = ops.PinnedHostPool(4 << 20, uncached=True)   # the smallest parked pool that fits
    assert again.tensor.data_ptr() == big_ptr != small_ptr
    again.free()
    lib = _lib.load()
    assert lib.aegkv_host_free(ctypes.c_void_p(first_ptr + 4096)) == _lib.EINVAL
    host_np = rng.integers(0, 256, (n_host, composite), dtype=np.uint8)
    pool.tensor.copy_(torch.from_numpy(host_np.reshape(-1)))
    grp = rng.integers(0, 3, n).astype(np.int32)
    first = np.array([rng.integers(0, kpp[g] + 1) for g in grp], np.int64)
    valid = np.array([rng.integers(0, kpp[g] - f + 1) for g, f in zip(grp, first)], np.int64)
    lay = ops.SegmentLayout(segs, page, cpu_off, owners, n_gpu, kpp, pool.tensor, composite, 0)
    src, dst = rng.permutation(n_gpu)[:n], rng.permutation(n_host)[:n]
    lay.swap(src, dst, grp, first, valid, False, mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       host_np.reshape(-1), composite, 0, composite, src, dst, grp, first,
                       valid, False)
    back = rng.permutation(n_gpu)[:n]
    lay.swap(dst, back, grp, first, valid, True, mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       host_np.reshape(-1), composite, 0, composite, dst, back, grp, first,
                       valid, True)
    torch.cuda.synchronize()
    assert np.array_equal(pool.tensor.numpy().reshape(host_np.shape), host_np)
    for s in range(len(page)):
        assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), s
    del lay
    pool.free()


# ------------------------------------------------------------- edge cases --

@pytest.mark.parametrize("mode", MODES)
def test_edge_cases_vs_oracle(gpu, oracle, restore_tuning, mode):
    """Empty calls on every entry point; ids at both ends of each pool;
    6-byte blocks (byte path) through the legacy swap; composite pages larger
    than the staging chunk (one entry per chunk)."""
    rng = np.random.default_rng(77)
    # legacy swap, 6-byte blocks, ids 0 and N-1 on both sides
    n_dev, n_host = 9, 5
    cache_np = rng.integers(0, 256, (n_dev, 6), dtype=np.uint8)
    pool_np = rng.integers(0, 256, (n_host, 6), dtype=np.uint8)
    cache = torch.from_numpy(cache_np.copy()).view(torch.bfloat16).to(gpu)   # [9, 3] bf16
    pool = torch.from_numpy(pool_np.copy()).view(torch.bfloat16).pin_memory()
    ops.swap([], [], False, cache, pool, mode=mode)
    ops.swap([], [], True, cache, pool, mode=mode)
    ops.swap([0, n_dev - 1], [n_host - 1, 0], False, cache, pool, mode=mode)
    oracle.swap_legacy([0, n_dev - 1], [n_host - 1, 0], False, cache_np, cache_np.size // 2,
                       n_dev, pool_np)
    ops.swap([n_host - 1, 0], [n_dev - 1, 0], True, cache, pool, mode=mode)
    oracle.swap_legacy([n_host - 1, 0], [n_dev - 1, 0], True, cache_np, cache_np.size // 2,
                       n_dev, pool_np)
    torch.cuda.synchronize()
    assert np.array_equal(pool.view(torch.uint8).numpy(), pool_np)
    assert np.array_equal(cache.cpu().view(torch.uint8).numpy(), cache_np)

    # composite page (1.5 MiB) above the 1 MiB staging chunk
    _lib.tune(_lib.TUNE_STAGING_BYTES, 1 << 20)
    page = np.array([512 * 1024, 1024 * 1024], np.int64)
    cpu_off = np.array([0, 512 * 1024], np.int64)
    owners = np.array([1, 1], np.uint64)
    kpp = np.array([2], np.int64)
    composite = int(page.sum())
    n_gpu, n_hp = 6, 4
    segs_np = [rng.integers(0, 256, (n_gpu, int(p)), dtype=np.uint8) for p in page]
    host_np = rng.integers(0, 256, (n_hp, composite), dtype=np.uint8)
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    hp = _pool_from(host_np)
    lay = ops.SegmentLayout(segs, page, cpu_off, owners, n_gpu, kpp, hp.tensor, composite, 0)
    e = np.zeros(0, np.int64)
    lay.swap(e, e, e.astype(np.int32), e, e, False, mode=mode)
    src, dst = np.array([0, n_gpu - 1, 2]), np.array([n_hp - 1, 0, 1])
    grp, first, valid = np.zeros(3, np.int32), np.array([0, 1, 2]), np.array([2, 1, 0])
    lay.swap(src, dst, grp, first, valid, False, mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       host_np.reshape(-1), composite, 0, composite, src, dst, grp, first,
                       valid, False)
    lay.swap(dst[::-1].copy(), src, grp, first, valid, True, mode=mode)
    oracle.swap_blocks([x.reshape(-1) for x in segs_np], page, cpu_off, owners, n_gpu, kpp,
                       host_np.reshape(-1), composite, 0, composite, dst[::-1].copy(), src,
                       grp, first, valid, True)
    torch.cuda.synchronize()
    assert np.array_equal(hp.tensor.numpy().reshape(host_np.shape), host_np)
    for s in range(2):
        assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), s

    # copy_blocks: empty, then the two ends of the pool
    ops.copy_blocks(segs, [], [])
    ops.copy_blocks(segs, [n_gpu - 1], [0])
    oracle.copy_blocks([x.reshape(-1) for x in segs_np], page, n_gpu, [n_gpu - 1], [0])
    torch.cuda.synchronize()
    for s in range(2):
        assert np.array_equal(segs[s].cpu().numpy(), segs_np[s]), s
    del lay
    hp.free()


# --------------------------------------------------------- error behaviour --

def test_rejections_enqueue_nothing(gpu):
    seg = torch.arange(8 * 64, dtype=torch.int32, device=gpu).view(torch.uint8).view(8, 256)
    before = seg.clone()
    pool = ops.PinnedHostPool(4 * 256)
    pool.tensor.fill_(7)
    args = ([256], [0], [1], 8, [1], pool.tensor, 256, 0)
    cases = [
        ([1, 2], [0, 4], "target"),     # host id 4 outside [0, 4)
        ([9], [0], "source"),           # device id 9 outside [0, 8)
        ([1, 2], [3, 3], "twice"),      # duplicate target
    ]
    for src, dst, word in cases:
        with pytest.raises(ValueError, match=word):
            ops.swap_segments([seg], *args, src, dst, [0] * len(src), [0] * len(src),
                              [1] * len(src), False)
    with pytest.raises(ValueError, match="run past a page"):
        ops.swap_segments([seg], *args, [1], [0], [0], [0], [2], False)
    with pytest.raises(ValueError, match="unequal lengths"):
        ops.swap_segments([seg], *args, [1], [0], [0, 0], [0], [1], False)
    with pytest.raises(ValueError, match="both a source and a target"):
        ops.copy_blocks([seg], [1, 2], [2, 3])
    with pytest.raises(ValueError, match="twice"):
        ops.copy_blocks([seg], [1, 2], [3, 3])
    pageable = torch.zeros(4 * 256, dtype=torch.uint8)
    for mode in ("direct", "staged"):
        with pytest.raises(ValueError, match="pinned"):
            ops.swap_segments([seg], [256], [0], [1], 8, [1], pageable, 256, 0, [1], [0], [0],
                              [0], [1], False, mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(seg, before)
    assert bool((pool.tensor == 7).all())
    pool.free()


def test_rejected_swap_leaves_no_event_behind(gpu):
    """A swap the library rejects raises before anything is recorded: the
    request gets no completion event and the fence count does not move."""
    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import KVSwapper

    cache = allocate_composite_cache([KVCacheTensorSpec(8 * 4096, ("l0",))], 8, gpu)
    pool = ops.PinnedHostPool(4 * 4096)
    words = torch.zeros(2, dtype=torch.int64, device=gpu)
    sw = KVSwapper(cache, [{"l0"}], [CacheGroupRuntimeConfig("attention", 16, 16)], pool.tensor,
                   fence_words=words, fence_slots=(0, 1))
    with pytest.raises(ValueError, match="outside"):
        sw.swap_blocks([3], [9], [0], [0], [0], [1], [None], False)   # device id 9 of 8
    assert 3 not in sw.move_event_table and sw.last_fence is None
    torch.cuda.synchronize()
    assert int(words[0]) == 0
    pool.free()


def test_runs_on_current_stream_and_orders_by_events(gpu):
    """Work goes on the caller's current stream (ops/swap.cu:21-32): a
    consumer on another stream sees the data only after waiting on an event
    recorded behind the swap."""
    n, page = 64, 65536
    seg = torch.randint(0, 256, (n, page), dtype=torch.uint8, device=gpu)
    pool = ops.PinnedHostPool(n * page)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        ops.swap_segments([seg], [page], [0], [1], n, [1], pool.tensor, page, 0,
                          np.arange(n), np.arange(n)[::-1].copy(), np.zeros(n, np.int32),
                          np.zeros(n, np.int64), np.ones(n, np.int64), False)
        done = torch.cuda.Event()
        done.record(side)
    fresh = torch.zeros_like(seg)
    torch.cuda.current_stream().wait_event(done)
    ops.swap_segments([fresh], [page], [0], [1], n, [1], pool.tensor, page, 0,
                      np.arange(n)[::-1].copy(), np.arange(n), np.zeros(n, np.int32),
                      np.zeros(n, np.int64), np.ones(n, np.int64), True)
    torch.cuda.synchronize()
    assert torch.equal(fresh, seg)
    pool.free()


# ------------------------------------------------------------ swapper --

@pytest.mark.parametrize("streams", ["pool", "dedicated", "partitioned", "staged"])
def test_swapper_block_table_round_trip(gpu, oracle, streams):
    """BlockTable.transfer_entries -> KVSwapper.swap_blocks out and back in,
    partial extents included, checked against the oracle; on torch pool
    streams, dedicated streams, dedicated streams on 8 CUs of every XCD,
    and with the swapper's default mode set to STAGED."""
    from aegaeon_amd.cache_groups import BlockTable, CacheGroupConfig, CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import KVSwapper

    n_blocks, n_host = 40, 32
    specs = [KVCacheTensorSpec(n_blocks * 4096, ("full.0",)),
             KVCacheTensorSpec(n_blocks * 4096, ("win.0",)),
             KVCacheTensorSpec(n_blocks * 8192, ("full.1", "win.1"))]
    cache = allocate_composite_cache(specs, n_blocks, gpu)
    for t in cache.backing:
        t.random_(-128, 127)
    groups = (CacheGroupConfig("attention", 64, 16), CacheGroupConfig("attention", 64, 16, 40))
    descr = [CacheGroupRuntimeConfig("attention", 64, 16),
             CacheGroupRuntimeConfig("attention", 64, 16, 40)]
    pool = ops.PinnedHostPool(n_host * cache.page_size_bytes)
    pool.tensor.zero_()
    sw = KVSwapper(cache, [{"full.0", "full.1"}, {"win.0", "win.1"}], descr, pool.tensor,
                   dedicated_streams=streams not in ("pool", "staged"),
                   swap_cu_mask=ops.xcd_cu_mask(8) if streams == "partitioned" else None,
                   mode="staged" if streams == "staged" else "auto")
    table = BlockTable(0, (cache.page_size_bytes // 2,), groups,
                       [[3, 4, 5, 6], [7, 8, 9, 10]])
    tokens = 230
    rows = table.transfer_entries(tokens)
    copy = [r for r in rows if r[4] > 0]
    host_ids = list(range(len(copy)))
    dev_src = [r[2] for r in copy]
    before = [t.cpu().numpy().view(np.uint8).copy() for t in cache.backing]
    ev = sw.swap_blocks([1], dev_src, host_ids, [r[0] for r in copy], [r[3] for r in copy],
                        [r[4] for r in copy], [None], False)
    ev.synchronize()
    owners = np.array([1, 2, 3], np.uint64)
    page = np.array([4096, 4096, 8192], np.int64)
    want_host = np.zeros((n_host, cache.page_size_bytes), np.uint8)
    oracle.swap_blocks([x.reshape(-1) for x in before], page, [0, 4096, 8192], owners,
                       n_blocks, [4, 4], want_host.reshape(-1), cache.page_size_bytes, 0,
                       cache.page_size_bytes, dev_src, host_ids, [r[0] for r in copy],
                       [r[3] for r in copy], [r[4] for r in copy], False)
    assert np.array_equal(pool.tensor.numpy().reshape(want_host.shape), want_host)
    new_ids = [20 + i for i in range(len(copy))]
    ev2 = sw.swap_blocks([1], host_ids, new_ids, [r[0] for r in copy], [r[3] for r in copy],
                         [r[4] for r in copy], [ev], True)
    sw.wait_for_all_move_in()
    oracle.swap_blocks([x.reshape(-1) for x in before], page, [0, 4096, 8192], owners,
                       n_blocks, [4, 4], want_host.reshape(-1), cache.page_size_bytes, 0,
                       cache.page_size_bytes, host_ids, new_ids, [r[0] for r in copy],
                       [r[3] for r in copy], [r[4] for r in copy], True)
    for t, w in zip(cache.backing, before):
        assert np.array_equal(t.cpu().numpy().view(np.uint8), w)
    assert ev2.query()
    sw.close()
    with pytest.raises(RuntimeError, match="closed"):
        sw.wait_for_all_move_in()
    pool.free()


def test_planner_swap_out_and_back_in(gpu):
    """plan_move -> KVSwapper out to the host pool, reclaim, plan_move ->
    KVSwapper back in: every live extent of every retained page arrives at
    its new device id unchanged."""
    import random

    from aegaeon_amd.cache_groups import CacheGroupConfig, CacheGroupRuntimeConfig, BlockTable
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.planner import BLOCK_LOCATION_CPU, BlockPools, plan_move
    from aegaeon_amd.swapper import KVSwapper

    rng = random.Random(4)
    n_blocks = 256
    groups = (CacheGroupConfig("attention", 32, 16), CacheGroupConfig("attention", 32, 16, 24))
    descr = [CacheGroupRuntimeConfig("attention", 32, 16),
             CacheGroupRuntimeConfig("attention", 32, 16, 24)]
    specs = [KVCacheTensorSpec(n_blocks * 2048, ("full.0",)),
             KVCacheTensorSpec(n_blocks * 2048, ("win.0",)),
             KVCacheTensorSpec(n_blocks * 4096, ("full.1", "win.1"))]
    cache = allocate_composite_cache(specs, n_blocks, gpu)
    for t in cache.backing:
        t.random_(-128, 127)
    shape = (cache.page_size_bytes // 2,)
    slab = 4 * cache.page_size_bytes + 100
    pools = BlockPools(cpu_num_slabs=40, cpu_slab_size_bytes=slab)
    pools.register_gpu_space(0, n_blocks, shape, groups)
    host = ops.PinnedHostPool(40 * slab)
    sw = KVSwapper(cache, [{"full.0", "full.1"}, {"win.0", "win.1"}], descr, host.tensor)
    tables, reqs = {}, []
    for rid in range(5):
        tokens = rng.randint(1, 150)
        cols = [groups[0].table_blocks_for_tokens(tokens), groups[1].table_blocks_for_tokens(tokens)]
        ids = pools.allocate(sum(cols), 0, shape)
        tables[rid] = BlockTable(0, shape, groups, [ids[:cols[0]], ids[cols[0]:]])
        tables[rid].release_skipped_blocks(tokens)
        reqs.append((rid, tokens))
    before = [t.clone() for t in cache.backing]
    orig = {rid: [list(c) for c in tables[rid].group_blocks] for rid, _ in reqs}
    out = plan_move(reqs, tables, BLOCK_LOCATION_CPU, pools)
    ev = sw.swap_blocks(out.request_ids, out.source_block_ids, out.target_block_ids,
                        out.group_ids, out.first_kernel_blocks, out.valid_kernel_blocks,
                        [None] * len(out.request_ids), False)
    pools.record_move(out, [ev])          # device sources stay taken until ev completes
    back = plan_move(reqs, tables, 0, pools)
    ev2 = sw.swap_blocks(back.request_ids, back.source_block_ids, back.target_block_ids,
                         back.group_ids, back.first_kernel_blocks, back.valid_kernel_blocks,
                         [ev] * len(back.request_ids), True)
    pools.record_move(back, [ev2])
    assert not set(back.target_block_ids) & set(out.release_source_block_ids)
    assert pools.reclaim_cpu_moves(shape) == (1, len(back.release_source_block_ids))
    assert ev2.query() and ev.query()
    assert pools.reclaim_gpu_moves(0, wait=False) == (1, len(out.release_source_block_ids))
    assert sum(pools.cpu_slab_usage) == 0 and len(pools.cpu_free_slabs) == 40
    owners = [(0, 0), (1, 1), (2, 0), (2, 1)]  # (backing tensor, group)
    pages = [2048, 2048, 4096]
    checked = 0
    for rid, tokens in reqs:
        for g in range(2):
            for col, (old, new) in enumerate(zip(orig[rid][g], tables[rid].group_blocks[g])):
                if old < 0:
                    continue
                first, count = groups[g].kernel_block_extent(tokens, col)
                for seg, og in owners:
                    if og != g:
                        continue
                    unit = pages[seg] // 2
                    lo, hi = unit * first, unit * (first + count)
                    a = before[seg].view(n_blocks, pages[seg])[old, lo:hi]
                    b = cache.backing[seg].view(n_blocks, pages[seg])[new, lo:hi]
                    assert torch.equal(a, b), (rid, g, col, seg)
                    checked += 1
    assert checked > 20
    host.free()


# ---------------------------------------------------- full benchmark shapes --

def _kv_segments(n_layers, n_blocks, heads, dim, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    segs = []
    for _ in range(2 * n_layers):
        t = torch.empty(n_blocks, 16, heads, dim, dtype=dtype, device=dev)
        t.normal_(generator=g)
        segs.append(t)
    return segs


def test_qwen3_4b_swap_full_size_round_trip(gpu):
    """72 x [8192,16,8,128] bf16; 1024 non-contiguous blocks out to a 4096
    block pinned pool and back in to fresh ids; host pages must equal the
    device tiles they came from and the round trip must be exact."""
    _say("Qwen3-4B full-size round trip")
    segs = _kv_segments(36, 8192, 8, 128, torch.bfloat16, gpu, 1)
    tile = 16 * 8 * 128 * 2
    S = len(segs)
    pool = ops.PinnedHostPool(4096 * S * tile)
    g = torch.Generator().manual_seed(1)
    out_ids = (torch.randperm(8191, generator=g)[:1024] + 1).numpy()
    host_ids = torch.randperm(4096, generator=g)[:1024].numpy()
    rest = np.setdiff1d(np.arange(1, 8192), out_ids)
    in_ids = rest[torch.randperm(rest.size, generator=g)[:1024].numpy()]
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, 8192, [1], pool.tensor,
              S * tile, 0)
    z = np.zeros(1024, np.int32)
    for mode in MODES:
        ops.swap_segments(segs, *common, out_ids, host_ids, z, z, z + 1, False, mode=mode)
        ops.swap_segments(segs, *common, host_ids, in_ids, z, z, z + 1, True, mode=mode)
        torch.cuda.synchronize()
        dev_in = torch.from_numpy(in_ids).to(gpu)
        dev_out = torch.from_numpy(out_ids).to(gpu)
        for s in range(S):
            assert torch.equal(segs[s][dev_in], segs[s][dev_out]), (mode, s)
        pages = pool.tensor.view(4096, S, tile)
        for k in (0, 511, 1023):
            for s in (0, 37, 71):
                assert torch.equal(pages[int(host_ids[k]), s].to(gpu),
                                   segs[s][int(out_ids[k])].view(torch.uint8).reshape(-1))
    pool.free()


def test_llama2_13b_copy_blocks_full_size(gpu):
    """80 x [8192,16,40,128] fp16 (100 GiB); 4096 pairs, distinct targets
    disjoint from the sources: every target equals its source afterwards and
    every other block keeps its checksum."""
    _say("Llama-2-13B full-size copy_blocks")
    segs = _kv_segments(40, 8192, 40, 128, torch.float16, gpu, 2)
    g = torch.Generator().manual_seed(2)
    perm = torch.randperm(8192, generator=g)
    src, dst = perm[:4096], perm[4096:]
    keep = torch.ones(8192, dtype=torch.bool)
    keep[dst] = False
    keep = keep.to(gpu)
    sums = [s.view(8192, -1).view(torch.int16).sum(dim=1, dtype=torch.int64) for s in segs]
    ops.copy_blocks(segs, src.numpy(), dst.numpy())
    torch.cuda.synchronize()
    ds, dd = src.to(gpu), dst.to(gpu)
    for i, s in enumerate(segs):
        assert torch.equal(s[dd], s[ds]), i
        after = s.view(8192, -1).view(torch.int16).sum(dim=1, dtype=torch.int64)
        assert torch.equal(after[keep], sums[i][keep]), i


def test_qwen25_7b_varlen_batched_round_trip(gpu):
    """56 x [16384,16,4,128] bf16; 64 requests with log-normal lengths,
    blocks at seeded random device ids, host ids from the slab allocator;
    one batched call per direction in each mode, bit-exact round trip."""
    from aegaeon_amd.planner import BLOCK_LOCATION_CPU, BlockPools

    _say("Qwen2.5-7B variable-length batched round trip")
    segs = _kv_segments(28, 16384, 4, 128, torch.bfloat16, gpu, 3)
    S, tile = len(segs), 16 * 4 * 128 * 2
    page = S * tile
    rng = np.random.default_rng(30)
    tokens = np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, 64))), 16, 32768)
    total = int(np.ceil(tokens / 16).sum())
    perm = rng.permutation(np.arange(1, 16384))
    assert 2 * total <= perm.size
    out_ids, in_ids = perm[:total], perm[total:2 * total]
    slab = 1 << 30
    n_slabs = -(-total * page // slab) + 1
    pools = BlockPools(n_slabs, slab)
    host_ids = np.array(pools.allocate(total, BLOCK_LOCATION_CPU, (page // 2,)), np.int64)
    pool = ops.PinnedHostPool(n_slabs * slab)
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, 16384, [1], pool.tensor, page, 0)
    z, one = np.zeros(total, np.int32), np.ones(total, np.int64)
    di, do = torch.from_numpy(in_ids).to(gpu), torch.from_numpy(out_ids).to(gpu)
    for mode in MODES:
        for t in segs:
            t.index_fill_(0, di, 0)
        ops.swap_segments(segs, *common, out_ids, host_ids, z, z, one, False, mode=mode)
        ops.swap_segments(segs, *common, host_ids, in_ids, z, z, one, True, mode=mode)
        torch.cuda.synchronize()
        for s in range(S):
            assert torch.equal(segs[s][di], segs[s][do]), (mode, s)
    pool.free()


def test_three_stream_overlap_correctness(gpu):
    """Qwen1.5-MoE tile shape (48 x 64 KiB), scaled to 4096 blocks: swap-out,
    swap-in and copy_blocks enqueued together on three streams must each be
    exact."""
    _say("three-stream overlap")
    NB, NOUT, NIN, NP = 4096, 1024, 768, 512
    segs = _kv_segments(24, NB, 16, 128, torch.bfloat16, gpu, 4)
    S, tile = len(segs), 16 * 16 * 128 * 2
    page = S * tile
    rng = np.random.default_rng(40)
    perm = rng.permutation(NB)
    out_ids, in_ids = perm[:NOUT], perm[NOUT:NOUT + NIN]
    csrc = perm[NOUT + NIN:NOUT + NIN + NP]
    cdst = perm[NOUT + NIN + NP:NOUT + NIN + 2 * NP]
    pool = ops.PinnedHostPool((NOUT + NIN) * page)
    hp = rng.permutation(NOUT + NIN)
    hx, hy = hp[:NOUT], hp[NOUT:]
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, NB, [1], pool.tensor, page, 0)
    zo, oo = np.zeros(NOUT, np.int32), np.ones(NOUT, np.int64)
    zi, oi = np.zeros(NIN, np.int32), np.ones(NIN, np.int64)
    ops.swap_segments(segs, *common, in_ids, hy, zi, zi, oi, False)
    di = torch.from_numpy(in_ids).to(gpu)
    want_in = [t[di].clone() for t in segs]
    for t in segs:
        t.index_fill_(0, di, 0)
    want_cp = [t[torch.from_numpy(csrc).to(gpu)].clone() for t in segs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(3)]
    begin = torch.cuda.Event()
    begin.record()
    for st in streams:
        st.wait_event(begin)
    with torch.cuda.stream(streams[0]):
        ops.swap_segments(segs, *common, out_ids, hx, zo, zo, oo, False)
    with torch.cuda.stream(streams[1]):
        ops.swap_segments(segs, *common, hy, in_ids, zi, zi, oi, True)
    with torch.cuda.stream(streams[2]):
        ops.copy_blocks(segs, csrc, cdst)
    torch.cuda.synchronize()
    dcd = torch.from_numpy(cdst).to(gpu)
    pages = pool.tensor.view(NOUT + NIN, S, tile)
    for s in range(S):
        assert torch.equal(segs[s][di], want_in[s]), s
        assert torch.equal(segs[s][dcd], want_cp[s]), s
    hxt = torch.from_numpy(hx)
    for s in (0, S // 2, S - 1):
        got = pages[hxt, s].to(gpu)
        want = segs[s][torch.from_numpy(out_ids).to(gpu)].view(NOUT, -1).view(torch.uint8)
        assert torch.equal(got, want), s
    pool.free()


def _ipc_producer(q_in, q_out):
    """Child process: write a pattern into a block of the parent's cache
    after a long kernel, record an interprocess event behind it and hand out
    its IPC handle without waiting."""
    import torch

    seg = q_in.get()
    torch.cuda.set_device(0)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        busy = torch.zeros(1 << 28, dtype=torch.float32, device="cuda")
        for _ in range(400):
            busy.add_(1.0)
        seg[5].fill_(0x2B)
        ev = torch.cuda.Event(interprocess=True)
        ev.record(st)
    q_out.put(ev.ipc_handle())
    q_in.get()  # keep the event and tensor alive until the parent is done


def _hip_interprocess_event_status():
    """(create, export, record) statuses of an interprocess event, straight
    from the HIP runtime torch loaded (hipEventInterprocess 0x4 |
    hipEventDisableTiming 0x2), recorded on the null stream."""
    hip = ctypes.CDLL("libamdhip64.so.7")   # the runtime already loaded by torch
    ev = ctypes.c_void_p()
    create = hip.hipEventCreateWithFlags(ctypes.byref(ev), ctypes.c_uint(0x6))
    if create != 0:
        return create, None, None
    handle = (ctypes.c_char * 64)()
    export = hip.hipIpcGetEventHandle(handle, ev)
    record = hip.hipEventRecord(ev, ctypes.c_void_p(0))
    hip.hipDeviceSynchronize()
    hip.hipGetLastError()
    hip.hipEventDestroy(ev)
    return create, export, record


def test_interprocess_event_contract(gpu):
    """The reference chains moves across processes with interprocess events
    (worker.py:2249,2331,2349 record and export; :2351-2394 open and wait).
    This runtime creates them but refuses to export or record them
    (hipErrorInvalidValue = 1): then a swapper asked for interprocess
    events refuses up front, naming the fence path instead. If the runtime
    exports and records them, the reference's handle path must work end to
    end."""
    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import KVSwapper

    create, export, record = _hip_interprocess_event_status()
    _say("interprocess event statuses (create, export, record):", create, export, record)
    assert create == 0
    if export != 0 or record != 0:
        assert 1 in (export, record), (export, record)   # hipErrorInvalidValue
        cache = allocate_composite_cache([KVCacheTensorSpec(16 * 4096, ("l0",))], 16, gpu)
        pool = ops.PinnedHostPool(4 * 4096)
        with pytest.raises(ValueError, match="fence"):
            KVSwapper(cache, [{"l0"}], [CacheGroupRuntimeConfig("attention", 16, 16)],
                      pool.tensor, interprocess_events=True)
        pool.free()
        return
    _swap_waits_on_ipc_event_from_another_process(gpu)


def _swap_waits_on_ipc_event_from_another_process(gpu):
    """A source event exported by another process orders the swap after that
    process's write (worker.py:2351-2394)."""
    import time

    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import KVSwapper

    _say("IPC event ordering across processes")
    n_blocks, page = 16, 65536
    cache = allocate_composite_cache([KVCacheTensorSpec(n_blocks * page, ("l0",))], n_blocks, gpu)
    pool = ops.PinnedHostPool(4 * page)
    pool.tensor.zero_()
    sw = KVSwapper(cache, [{"l0"}], [CacheGroupRuntimeConfig("attention", 16, 16)], pool.tensor,
                   interprocess_events=True)
    mp = torch.multiprocessing.get_context("spawn")
    q_in, q_out = mp.Queue(), mp.Queue()
    child = mp.Process(target=_ipc_producer, args=(q_in, q_out), daemon=True)
    child.start()
    try:
        q_in.put(cache.segment_pages(0))
        handle = q_out.get(timeout=240)
        ev = sw.swap_blocks([7], [5], [2], [0], [0], [1], [handle], False)
        deadline = time.time() + 120
        while not ev.query():
            assert time.time() < deadline, "swap event never completed"
            time.sleep(0.01)
        got = pool.tensor.view(4, page)[2]
        assert bool((got == 0x2B).all()), "swap ran before the other process's write"
        handle2 = KVSwapper.event_ipc_handle(ev)
        assert isinstance(handle2, (bytes, bytearray)) and len(handle2) > 0
    finally:
        q_in.put(None)
        child.join(60)
        if child.is_alive():
            child.kill()
    pool.free()


# --------------------------------------------------------------- migration --

def test_migrate_blocks_between_caches_vs_expectation(gpu):
    """aegkv_migrate_blocks copies whole blocks between two caches with the
    same pages (one tile shape per segment, unaligned pages included);
    everything else in both caches stays as it was."""
    rng = np.random.default_rng(61)
    pages = [160 * 1024, 32 * 1024, 4100, 100]
    n_src, n_dst, n = 24, 20, 12
    src_np = [rng.integers(0, 256, (n_src, p), dtype=np.uint8) for p in pages]
    dst_np = [rng.integers(0, 256, (n_dst, p), dtype=np.uint8) for p in pages]
    src = [torch.from_numpy(x.copy()).to(gpu) for x in src_np]
    dst = [torch.from_numpy(x.copy()).to(gpu) for x in dst_np]
    s_ids = rng.integers(0, n_src, n)                     # a source may repeat
    d_ids = rng.permutation(n_dst)[:n]
    _say("migrate blocks, pages", pages)
    ops.migrate_blocks(src[:2], dst[:2], s_ids, d_ids)    # vector path
    ops.migrate_blocks(src[2:], dst[2:], s_ids, d_ids)    # byte path (unaligned pages)
    ops.migrate_blocks(src, dst, [], [])
    torch.cuda.synchronize()
    for k in range(len(pages)):
        want = dst_np[k].copy()
        want[d_ids] = src_np[k][s_ids]
        assert np.array_equal(dst[k].cpu().numpy(), want), k
        assert np.array_equal(src[k].cpu().numpy(), src_np[k]), k
    with pytest.raises(ValueError, match="overlap"):
        ops.migrate_blocks(src, src, [0], [1])


def test_engine_to_engine_migration_through_planner(gpu):
    """plan_migrate -> KVSwapper.migrate_blocks from a registered peer cache
    -> record_move: the requests' blocks arrive whole at their new ids."""
    from aegaeon_amd.cache_groups import CacheGroupConfig, CacheGroupRuntimeConfig, BlockTable
    from aegaeon_amd.layout import allocate_composite_cache, kv_tensor_specs
    from aegaeon_amd.planner import BlockPools, plan_migrate
    from aegaeon_amd.swapper import KVSwapper

    n_blocks = 96
    specs = kv_tensor_specs(2, n_blocks, 16, 2, 64, 2)
    caches = [allocate_composite_cache(specs, n_blocks, gpu) for _ in range(2)]
    for t in caches[0].backing:
        t.random_(-128, 127)
    names = [{f"layers.{l}.{kv}" for l in range(2) for kv in ("k", "v")}]
    descr = [CacheGroupRuntimeConfig("attention", 16, 16)]
    groups = (CacheGroupConfig("attention", 16, 16),)
    shape = (caches[0].page_size_bytes // 2,)
    pools = BlockPools(2, 1 << 20)
    for e in range(2):
        pools.register_gpu_space(e, n_blocks, shape, groups)
    pools.gpu_free_blocks[1].reverse()                    # scatter the target ids
    host = ops.PinnedHostPool(4 * caches[0].page_size_bytes)
    sw = [KVSwapper(c, names, descr, host.tensor) for c in caches]
    sw[1].register_peer_cache(0, [caches[0].segment_pages(i) for i in range(4)])
    tables = {r: BlockTable(0, shape, groups, [pools.allocate(5 + r, 0, shape)]) for r in range(6)}
    before = {r: [caches[0].segment_pages(i)[tables[r].blocks].clone() for i in range(4)]
              for r in tables}
    plan = plan_migrate(list(tables), tables, 1, pools)
    ev = sw[1].migrate_blocks(plan.request_ids, 0, plan.source_block_ids, plan.target_block_ids,
                              [None] * len(plan.request_ids))
    pools.record_move(plan, [ev])
    ev.synchronize()
    for r, table in tables.items():
        assert table.location == 1
        for i in range(4):
            assert torch.equal(caches[1].segment_pages(i)[table.blocks], before[r][i]), (r, i)
    assert pools.reclaim_gpu_moves(0, wait=False) == (1, len(plan.source_block_ids))
    with pytest.raises(KeyError):
        sw[0].migrate_blocks([0], 7, [1], [2], [None])
    sw[1].unregister_peer_cache(0)
    host.free()


def _cache_owner(q_in, q_out):
    """Child process: own a cache, fill it, hand its segments out through
    torch IPC and keep them open until told to stop."""
    import torch

    torch.cuda.set_device(0)
    pages = [torch.randint(0, 256, (32, p), dtype=torch.uint8, device="cuda")
             for p in (65536, 16384)]
    torch.cuda.synchronize()
    q_out.put(pages)
    q_in.get()


def test_migrate_from_another_process_cache(gpu):
    """A cache owned by another process, opened through IPC memory handles,
    is a migration source (the reference's register_kvcache_mem_handles +
    migrate_blocks plan, worker.py:2420-2445)."""
    _say("migration from another process's cache")
    mp = torch.multiprocessing.get_context("spawn")
    q_in, q_out = mp.Queue(), mp.Queue()
    child = mp.Process(target=_cache_owner, args=(q_in, q_out), daemon=True)
    child.start()
    try:
        peer = q_out.get(timeout=100)
        own = [torch.zeros(40, p.size(1), dtype=torch.uint8, device=gpu) for p in peer]
        s_ids, d_ids = np.arange(3, 19), np.arange(39, 23, -1)
        ops.migrate_blocks(peer, own, s_ids, d_ids)
        torch.cuda.synchronize()
        for p, o in zip(peer, own):
            assert torch.equal(o[torch.from_numpy(d_ids).to(gpu)], p[torch.from_numpy(s_ids).to(gpu)])
            assert int(o[:23].count_nonzero()) == 0
        del peer
    finally:
        q_in.put(None)
        child.join(60)
        if child.is_alive():
            child.kill()


def test_dedicated_stream_lives_with_its_torch_stream(gpu):
    """A DedicatedStream's `.stream` keeps the HIP stream alive after the
    owner object is dropped; work on it completes and orders normally; the
    HIP stream is destroyed as soon as the last reference to `.stream` goes
    (no garbage collection needed), and close() releases it explicitly."""
    import gc

    st = ops.DedicatedStream(gpu).stream
    gc.collect()
    x = torch.arange(1 << 20, device=gpu, dtype=torch.int32)
    with torch.cuda.stream(st):
        y = x * 3
        done = torch.cuda.Event()
        done.record(st)
    torch.cuda.current_stream().wait_event(done)
    assert int((y - 3 * x).abs().sum()) == 0
    import weakref

    ref = weakref.ref(st)
    assert st._aegkv_ptr
    torch.cuda.synchronize()
    del st
    assert ref() is None                            # destroyed with its last reference
    owner = ops.DedicatedStream(gpu)
    owner.close()                                   # explicit release, once
    assert owner.stream._aegkv_ptr is None
    owner.close()


def test_swaps_and_copy_on_cu_partitioned_streams(gpu):
    """Swap streams on 8 CUs of every XCD and a copy_blocks stream on the
    other 24, running at once: every block lands where the closed form says."""
    swap_mask = ops.xcd_cu_mask(8)
    copy_mask = ops.xcd_cu_mask(24, first=8)
    assert all(a & b == 0 for a, b in zip(swap_mask, copy_mask))
    n_gpu, page, n, S = 256, 32768, 96, 6
    segs = [torch.randint(0, 256, (n_gpu, page), dtype=torch.uint8, device=gpu) for _ in range(S)]
    before = [x.clone() for x in segs]
    pool = ops.PinnedHostPool(n * S * page)
    lay = ops.SegmentLayout(segs, [page] * S, [i * page for i in range(S)], [1] * S, n_gpu, [1],
                            pool.tensor, S * page, 0)
    perm = np.random.default_rng(61).permutation(n_gpu)
    out_ids, csrc, cdst = perm[:n], perm[n:n + 64], perm[n + 64:n + 128]
    a, b = ops.DedicatedStream(gpu, swap_mask), ops.DedicatedStream(gpu, copy_mask)
    z, one = np.zeros(n, np.int32), np.ones(n, np.int64)
    torch.cuda.synchronize()
    lay.swap(out_ids, np.arange(n), z, z, one, False, stream=a.stream)
    ops.copy_blocks(segs, csrc, cdst, stream=b.stream)
    torch.cuda.synchronize()
    host = pool.tensor.view(n, S, page)
    for s in range(S):
        assert torch.equal(host[:, s].to(gpu), before[s][torch.from_numpy(out_ids).to(gpu)]), s
        assert torch.equal(segs[s][torch.from_numpy(cdst).to(gpu)],
                           before[s][torch.from_numpy(csrc).to(gpu)]), s
    a.close()
    b.close()
    del lay
    pool.free()


# ------------------------------------------------------------------ fences --

def _busy(n_iter=200):
    """Keep the current stream busy for a while (bounded elementwise work)."""
    busy = torch.zeros(1 << 26, dtype=torch.float32, device="cuda")
    for _ in range(n_iter):
        busy.add_(1.0)


def test_fence_orders_a_swap_after_another_streams_write(gpu):
    """Stream A writes the blocks late and signals; stream B waits on the
    fence, then swaps the blocks out: B sees A's bytes, not the zeros that
    were there when B's work was enqueued."""
    n, page = 16, 65536
    words = torch.zeros(4, dtype=torch.int64, device=gpu)
    flags = torch.zeros(2, dtype=torch.int64, device=gpu)
    seg = torch.zeros(n, page, dtype=torch.uint8, device=gpu)
    pool = ops.PinnedHostPool(n * page)
    pool.tensor.fill_(1)
    lay = ops.SegmentLayout([seg], [page], [0], [1], n, [1], pool.tensor, page, 0)
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(a):
        _busy()
        seg.fill_(0x5A)
        ops.fence_signal(words, 1, 7)
    ops.fence_wait(words, 1, 7, flags, 0, timeout_s=30, stream=b)
    lay.swap(np.arange(n), np.arange(n)[::-1].copy(), np.zeros(n, np.int32), np.zeros(n, np.int64),
             np.ones(n, np.int64), False, stream=b)
    b.synchronize()
    assert int(flags[0]) == 0
    assert bool((pool.tensor == 0x5A).all()), "the swap ran before the fence was signalled"
    assert int(words[1]) == 7
    ops.fence_signal(words, 1, 3)          # atomic max: a smaller value leaves it
    torch.cuda.synchronize()
    assert int(words[1]) == 7
    del lay
    pool.free()


def test_fence_wait_gives_up_after_its_budget(gpu):
    """An unsignalled fence ends the wait after its budget and sets the move
    guard to 1, in device memory or in pinned host memory (GuardWords); the
    guard is never cleared. What the swaps behind such a wait do is in
    test_gpu_guards.py."""
    words = torch.zeros(4, dtype=torch.int64, device=gpu)
    flags = torch.zeros(2, dtype=torch.int64, device=gpu)
    host_guard = ops.GuardWords(2)
    st = ops.DedicatedStream(gpu)
    ops.fence_wait(words, 0, 5, flags, 1, timeout_s=0.002, stream=st.stream)
    ops.fence_wait(words, 0, 5, host_guard.tensor, 0, timeout_s=0.002, stream=st.stream)
    ops.fence_wait(words, 0, 5, flags, 1, timeout_s=0.002, stream=st.stream)
    st.stream.synchronize()
    assert flags.tolist() == [0, 1]
    assert host_guard.value(0) == 1 and host_guard.value(1) == 0
    with pytest.raises(ValueError, match="timeout"):
        ops.fence_wait(words, 0, 5, flags, 1, timeout_s=0, stream=st.stream)
    with pytest.raises(ValueError, match="index"):
        ops.fence_signal(words, 4, 1)
    st.close()


def test_same_process_fence_token_waits_on_the_producers_event(gpu):
    """A FenceToken raised by a swapper of this process, handed to another
    swapper of this process as a source event, orders the consumer through
    the producer's completion event: the consumer's swap-in reads the host
    pages the producer's swap-out wrote, with no fence wait to time out
    (a waiting fence would hold its queue, which plain streams of one
    process may share with the producer's)."""
    import time

    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import FenceToken, KVSwapper, _local_fences

    n_blocks, page = 64, 256 * 1024
    caches = [allocate_composite_cache([KVCacheTensorSpec(n_blocks * page, ("l0",))], n_blocks,
                                       gpu) for _ in range(2)]
    caches[0].backing[0].random_(-128, 127)
    words = torch.zeros(8, dtype=torch.int64, device=gpu)
    pool = ops.PinnedHostPool(32 * page)
    descr = [CacheGroupRuntimeConfig("attention", 16, 16)]
    a = KVSwapper(caches[0], [{"l0"}], descr, pool.tensor, fence_words=words, fence_slots=(0, 1),
                  fence_timeout_s=30)
    b = KVSwapper(caches[1], [{"l0"}], descr, pool.tensor, fence_words=words, fence_slots=(2, 3),
                  fence_timeout_s=30)
    torch.cuda.synchronize()
    src, host, dst = list(range(1, 31)), list(range(30)), list(range(33, 63))
    t0 = time.perf_counter()
    a.swap_blocks([1], src, host, [0] * 30, [0] * 30, [1] * 30, [None], False)
    token = a.last_fence
    assert token == FenceToken(0, 1)
    assert _local_fences[(words.data_ptr(), 0)][1][-1][0] == 1     # (count, event) history
    b.swap_blocks([1], host, dst, [0] * 30, [0] * 30, [1] * 30, [token], True)
    b.wait_for_all_move_in()               # raises if a fence wait had timed out
    assert time.perf_counter() - t0 < 10
    si, di = torch.tensor(src, device=gpu), torch.tensor(dst, device=gpu)
    assert torch.equal(caches[1].segment_pages(0)[di], caches[0].segment_pages(0)[si])
    a.close()
    b.close()
    pool.free()


def _fence_producer(q_in, q_out):
    """Child process: open the parent's fence words and cache blocks, then,
    when told, write a pattern late and signal the fence behind it."""
    import torch

    from aegaeon_amd import ops as child_ops

    words, pages = q_in.get()
    torch.cuda.set_device(0)
    q_out.put("ready")
    assert q_in.get() == "go"
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        _busy(400)
        pages[3:7].fill_(0x2B)
        child_ops.fence_signal(words, 4, 1)
    st.synchronize()
    q_out.put("done")
    q_in.get()  # keep the shared tensors open until the parent is done


def test_swap_waits_on_fence_from_another_process(gpu):
    """A FenceToken from another process orders the swap after that
    process's write (the reference's cross-worker event wait,
    worker.py:2351-2394): the swap is enqueued before the child writes."""
    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import KVCacheTensorSpec, allocate_composite_cache
    from aegaeon_amd.swapper import FenceToken, KVSwapper

    _say("fence ordering across processes")
    n_blocks, page = 16, 65536
    cache = allocate_composite_cache([KVCacheTensorSpec(n_blocks * page, ("l0",))], n_blocks, gpu)
    words = torch.zeros(8, dtype=torch.int64, device=gpu)
    pool = ops.PinnedHostPool(4 * page)
    pool.tensor.zero_()
    sw = KVSwapper(cache, [{"l0"}], [CacheGroupRuntimeConfig("attention", 16, 16)], pool.tensor,
                   fence_words=words, fence_slots=(0, 1), fence_timeout_s=60)
    torch.cuda.synchronize()
    mp = torch.multiprocessing.get_context("spawn")
    q_in, q_out = mp.Queue(), mp.Queue()
    child = mp.Process(target=_fence_producer, args=(q_in, q_out), daemon=True)
    child.start()
    try:
        q_in.put((words, cache.segment_pages(0)))
        assert q_out.get(timeout=100) == "ready"
        sw.swap_blocks([7], [3, 4, 5, 6], [0, 1, 2, 3], [0] * 4, [0] * 4, [1] * 4,
                       [FenceToken(4, 1)], False)
        q_in.put("go")
        sw.wait_for_all_move_out()
        assert q_out.get(timeout=100) == "done"
        got = pool.tensor.view(4, page)
        assert bool((got == 0x2B).all()), "the swap ran before the other process's write"
        assert sw.last_fence == FenceToken(0, 1) and int(words[0]) == 1
    finally:
        q_in.put(None)
        child.join(60)
        if child.is_alive():
            child.kill()
    pool.free()


def test_fence_publish_follows_stream_work(gpu):
    """A host fence word is raised only after the work enqueued before the
    publish: here a device fence wait that the test releases from another
    stream, so the host word stays low until then (no timing involved)."""
    words = torch.zeros(2, dtype=torch.int64, device=gpu)
    flags = torch.zeros(1, dtype=torch.int64, device=gpu)
    hw = ops.HostFenceWords(2)
    # hardware queues of their own: a waiting fence holds its queue, so a
    # signal on a stream that shares it would run only after the time-out
    owners = [ops.DedicatedStream(gpu), ops.DedicatedStream(gpu)]
    try:
        a, b = (o.stream for o in owners)
        torch.cuda.synchronize()
        ops.fence_wait(words, 0, 1, flags, timeout_s=60, stream=a)
        ops.fence_publish(hw, 1, 9, device=gpu, stream=a)
        assert not ops.fence_host_wait(hw, 1, 9, timeout_s=0.2)
        ops.fence_signal(words, 0, 1, stream=b)
        assert ops.fence_host_wait(hw, 1, 9, timeout_s=60)
        a.synchronize()
        assert int(flags[0]) == 0 and int(hw.words[1]) == 9
        ops.fence_publish(hw, 1, 4, device=gpu, stream=a)   # a smaller count never lowers it
        a.synchronize()
        assert int(hw.words[1]) == 9
    finally:
        torch.cuda.synchronize()
        hw.close()
        for o in owners:
            o.close()


def _reclaim_worker(q_in, q_out):
    """Child process (a worker): open the controller's cache, device fence
    words and host fence words, swap the planned blocks out behind the
    controller's "go" fence, hand back the swap's FenceToken without
    waiting, and on request report whether the host pages hold the bytes
    the source blocks had before the swap."""
    import torch

    from aegaeon_amd import ops as cops
    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import kv_tensor_specs, wrap_composite_cache
    from aegaeon_amd.swapper import FenceToken, KVSwapper

    torch.cuda.set_device(0)
    backing, words, host_name, geometry, lists = q_in.get()
    n_layers, n_blocks, heads, dim, n_host = geometry
    rids, src, dst, grp, first, valid = lists
    cache = wrap_composite_cache(kv_tensor_specs(n_layers, n_blocks, 16, heads, dim, 2),
                                 n_blocks, backing)
    S = len(cache.segments)
    pool = cops.PinnedHostPool(n_host * cache.page_size_bytes)
    names = [{s.layer_name for s in cache.segments}]
    sw = KVSwapper(cache, names, [CacheGroupRuntimeConfig("attention", 16, 16)], pool.tensor,
                   fence_words=words, fence_slots=(0, 1), fence_host=host_name,
                   fence_timeout_s=60)
    si = torch.tensor(src, device="cuda")
    expect = [cache.segment_pages(i)[si].clone() for i in range(S)]
    torch.cuda.synchronize()
    sw.swap_blocks(rids, src, dst, grp, first, valid,
                   [FenceToken(4, 1)] + [None] * (len(rids) - 1), False)
    q_out.put(sw.last_fence)
    assert q_in.get() == "check"
    sw.wait_for_all_move_out()
    pages = pool.tensor.view(n_host, S, -1)[torch.tensor(dst)].to("cuda")
    q_out.put(all(torch.equal(pages[:, i], expect[i]) for i in range(S)))
    q_in.get()   # keep the shared memory open until the controller is done
    sw.close()


def test_controller_reclaims_after_worker_fence_across_processes(gpu):
    """The controller half of the reference's move chaining
    (block_manager.py:804-851): a worker process swaps a plan's blocks out
    and hands back a FenceToken; the controller's BlockPools keeps the
    source ids until the token completes on the host, frees them then, and
    at once overwrites the freed blocks. The worker's host pages must hold
    the old bytes: the sources were freed only after the swap read them."""
    from aegaeon_amd.cache_groups import BLOCK_LOCATION_CPU, BlockTable, CacheGroupConfig
    from aegaeon_amd.layout import allocate_composite_cache, kv_tensor_specs
    from aegaeon_amd.planner import BlockPools, plan_move

    _say("controller reclaim after a worker's fence across processes")
    n_layers, n_blocks, heads, dim = 8, 256, 16, 128       # 16 x 64 KiB tiles, 1 MiB pages
    cache = allocate_composite_cache(kv_tensor_specs(n_layers, n_blocks, 16, heads, dim, 2),
                                     n_blocks, gpu)
    for t in cache.backing:
        t.random_(-128, 127)
    page = cache.page_size_bytes
    n_host = 256
    groups = (CacheGroupConfig("attention", 16, 16),)
    shape = (page // 2,)
    pools = BlockPools(cpu_num_slabs=1, cpu_slab_size_bytes=n_host * page)
    pools.register_gpu_space(0, n_blocks, shape, groups)
    tables = {r: BlockTable(0, shape, groups, [pools.allocate(60, 0, shape)]) for r in range(4)}
    plan = plan_move([(r, 60 * 16) for r in range(4)], tables, BLOCK_LOCATION_CPU, pools)
    free_before = list(pools.gpu_free_blocks[0])
    words = torch.zeros(8, dtype=torch.int64, device=gpu)
    hw = ops.HostFenceWords(8)
    torch.cuda.synchronize()
    mp = torch.multiprocessing.get_context("spawn")
    q_in, q_out = mp.Queue(), mp.Queue()
    child = mp.Process(target=_reclaim_worker, args=(q_in, q_out), daemon=True)
    child.start()
    try:
        lists = (plan.request_ids, plan.source_block_ids, plan.target_block_ids, plan.group_ids,
                 plan.first_kernel_blocks, plan.valid_kernel_blocks)
        q_in.put((cache.backing, words, hw.name, (n_layers, n_blocks, heads, dim, n_host),
                  lists))
        token = q_out.get(timeout=200)
        assert token.host == hw.name and token.slot == 0 and token.value == 1
        pools.record_move(plan, [token])
        assert pools.reclaim_gpu_moves(0, wait=False) == (0, 0)   # waiting for "go"
        assert not token.query()
        assert pools.gpu_free_blocks[0] == free_before
        ops.fence_signal(words, 4, 1)                            # go
        n = len(plan.release_source_block_ids)
        assert pools.reclaim_gpu_moves(0, wait=True) == (1, n)
        assert token.query()
        freed = torch.tensor(plan.release_source_block_ids, device=gpu)
        for i in range(len(cache.segments)):
            cache.segment_pages(i).index_fill_(0, freed, 0x5A)   # reuse at once
        torch.cuda.synchronize()
        assert sorted(pools.gpu_free_blocks[0]) == sorted(free_before +
                                                           plan.release_source_block_ids)
        q_in.put("check")
        assert q_out.get(timeout=100) is True, "the worker's swap read blocks after their reuse"
    finally:
        q_in.put(None)
        child.join(60)
        if child.is_alive():
            child.kill()
        hw.close()


def test_tensor_parallel_ranks_share_host_pages(gpu):
    """Two TP ranks' swappers write disjoint halves of the same host
    composite pages (host offset tp_rank * composite, worker.py:2304-2309);
    each rank's bytes survive the other's swap and come back exactly."""
    from aegaeon_amd.cache_groups import CacheGroupRuntimeConfig
    from aegaeon_amd.layout import allocate_composite_cache, kv_tensor_specs
    from aegaeon_amd.swapper import KVSwapper

    n_blocks, n_host = 32, 12
    specs = kv_tensor_specs(3, n_blocks, 16, 2, 64, 2)
    caches = [allocate_composite_cache(specs, n_blocks, gpu) for _ in range(2)]
    for c in caches:
        for t in c.backing:
            t.random_(-128, 127)
    composite = caches[0].page_size_bytes
    pool = ops.PinnedHostPool(n_host * composite * 2)
    pool.tensor.zero_()
    names = [{f"layers.{l}.{kv}" for l in range(3) for kv in ("k", "v")}]
    descr = [CacheGroupRuntimeConfig("attention", 16, 16)]
    sw = [KVSwapper(c, names, descr, pool.tensor, tp_rank=r, tp_size=2)
          for r, c in enumerate(caches)]
    src, host = [3, 9, 17, 30], [0, 5, 6, 11]
    z = [0] * 4
    before = [[t.clone() for t in c.backing] for c in caches]
    evs = [s.swap_blocks([1], src, host, z, z, [1] * 4, [None], False) for s in sw]
    for e in evs:
        e.synchronize()
    view = pool.tensor.view(n_host, 2, composite)
    for r, c in enumerate(caches):
        for k, (b, h) in enumerate(zip(src, host)):
            want = torch.cat([t.view(n_blocks, -1)[b].view(torch.uint8) for t in before[r]])
            assert torch.equal(view[h, r].to(gpu), want), (r, k)
    back = [20, 21, 22, 23]
    evs = [s.swap_blocks([1], host, back, z, z, [1] * 4, [None], True) for s in sw]
    for e in evs:
        e.synchronize()
    for r, c in enumerate(caches):
        for t, t0 in zip(c.backing, before[r]):
            tv, t0v = t.view(n_blocks, -1), t0.view(n_blocks, -1)
            assert torch.equal(tv[back], t0v[src]), r
    pool.free()


# ------------------------------------------- randomized weight-load cases --

@pytest.mark.parametrize("case", range(24))
def test_randomized_weight_loads(gpu, case):
    """Random weight-load calls: 1-40 slices of 0 B-2 MiB at random 1 B or
    16 B aligned offsets, random modes and stream kinds; every slice lands
    byte for byte and the arena outside the slices keeps its guard value."""
    rng = np.random.default_rng(7000 + case)
    aligned = bool(rng.integers(0, 2))
    mode = ("direct", "staged", "auto")[case % 3]
    n = int(rng.integers(1, 41))
    sizes = [int(rng.choice([0, 1, 16, 4096, int(rng.integers(1, 1 << 21))])) for _ in range(n)]
    if aligned:
        sizes = [-(-x // 16) * 16 for x in sizes]
    total = sum(-(-max(x, 1) // 256) * 256 + 256 for x in sizes)
    host = ops.PinnedHostPool(total)
    host.tensor.copy_(torch.from_numpy(rng.integers(0, 256, total, dtype=np.uint8)))
    arena = torch.full((total,), 0x3C, dtype=torch.uint8, device=gpu)
    order = rng.permutation(n)                  # targets in another order than sources
    src, dst, hoff = [], [None] * n, 0
    doffs = np.zeros(n, np.int64)
    off = 0
    for k in order:
        off += 0 if aligned else int(rng.integers(0, 16))
        doffs[k] = off
        off += -(-max(sizes[k], 1) // 256) * 256
    for k in range(n):
        hoff += 0 if aligned else int(rng.integers(0, 16))
        src.append(host.tensor.narrow(0, hoff, sizes[k]))
        dst[k] = arena.narrow(0, int(doffs[k]), sizes[k])
        hoff += -(-max(sizes[k], 1) // 256) * 256
    stream = torch.cuda.Stream(gpu) if case % 2 else None
    _say("randomized weight load", case, mode, "aligned" if aligned else "bytes", n, "slices")
    ops.load_slices(dst, src, mode=mode, stream=stream)
    torch.cuda.synchronize()
    covered = torch.zeros(total, dtype=torch.bool, device=gpu)
    for d, h in zip(dst, src):
        assert torch.equal(d, h.to(gpu))
        if d.numel():
            covered[d.data_ptr() - arena.data_ptr():][:d.numel()] = True
    assert bool((arena[~covered] == 0x3C).all())
    host.free()


@pytest.mark.parametrize("case", range(16))
def test_randomized_noalloc_copies_vs_oracle(gpu, oracle, case):
    """The allocation-free copy on random layouts (1-30 segments of random
    16 B-multiple or odd pages, 2-3 calls in a row with shrinking and
    growing pair lists) against the oracle's in-order copy."""
    rng = np.random.default_rng(8000 + case)
    n_seg = int(rng.integers(1, 31))
    n_blocks = int(rng.integers(4, 97))
    odd = rng.random() < 0.3
    page = [int(rng.choice([16, 64, 4096, 16384, 48 * 1024])) + (int(rng.integers(1, 16)) if odd else 0)
            for _ in range(n_seg)]
    segs_np = [rng.integers(0, 256, (n_blocks, p), dtype=np.uint8) for p in page]
    segs = [torch.from_numpy(x.copy()).to(gpu) for x in segs_np]
    calls = int(rng.integers(2, 4))
    for _ in range(calls):
        k = int(rng.integers(0, n_blocks // 2 + 1))
        perm = rng.permutation(n_blocks)
        src, dst = perm[:k], perm[k:2 * k]
        ops.copy_blocks_noalloc(segs, src, dst)
        oracle.copy_blocks([x.reshape(-1) for x in segs_np], np.array(page, np.int64), n_blocks,
                           src, dst)
    torch.cuda.synchronize()
    for i in range(n_seg):
        assert np.array_equal(segs[i].cpu().numpy(), segs_np[i]), i


def test_fence_publish_from_several_streams_keeps_the_largest(gpu):
    """Publishes of increasing counts from several streams into one host
    word, each stream gated by its own device fence that the test releases
    in reverse order: the word ends at the largest count, never goes down,
    and each stream's count shows up only after its gate opened. Every
    stream has a hardware queue of its own: a waiting fence holds its queue,
    so a signal queued behind it on a shared queue would wait for the
    wait's time-out."""
    words = torch.zeros(4, dtype=torch.int64, device=gpu)
    flags = torch.zeros(4, dtype=torch.int64, device=gpu)
    hw = ops.HostFenceWords(1)
    owners = [ops.DedicatedStream(gpu) for _ in range(5)]
    try:
        streams = [o.stream for o in owners[:4]]
        torch.cuda.synchronize()
        for i, st in enumerate(streams):
            ops.fence_wait(words, i, 1, flags, i, timeout_s=60, stream=st)
            ops.fence_publish(hw, 0, 10 * (i + 1), device=gpu, stream=st)
        assert not ops.fence_host_wait(hw, 0, 1, timeout_s=0.1)
        releaser = owners[4].stream
        seen = []
        for i in reversed(range(4)):
            ops.fence_signal(words, i, 1, stream=releaser)
            streams[i].synchronize()
            seen.append(int(hw.words[0]))
        assert seen == [40, 40, 40, 40]          # the largest count came first and stays
        assert int(flags.sum()) == 0
    finally:
        torch.cuda.synchronize()
        for o in owners:
            o.close()
        hw.close()


def _capture(gpu, fn):
    """Run fn() under torch.cuda.graph capture on a side stream; returns
    the graph (the caller replays it)."""
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream(gpu)
    with torch.cuda.graph(g, stream=st):
        fn()
    return g


def test_ring_entry_points_refuse_graph_capture(gpu):
    """Calls that upload their descriptors through the library's host ring
    (and the fence publish, whose host callback frees its record) return
    AEGKV_EINVAL on a capturing stream with nothing enqueued, so a graph
    can never replay a reused ring slot; the library works normally after."""
    _say("ring entry points under graph capture")
    a = [torch.randint(0, 256, (64, 4096), dtype=torch.uint8, device=gpu) for _ in range(3)]
    kv = torch.randint(0, 256, (64, 4096), dtype=torch.uint8, device=gpu)
    host = ops.PinnedHostPool(64 * 4096)
    hw = ops.HostFenceWords(1)
    dev_w = torch.zeros(1 << 16, dtype=torch.uint8, device=gpu)
    host_w = ops.PinnedHostPool(1 << 16)
    torch.cuda.synchronize()
    calls = [
        ("copy_blocks", lambda: ops.copy_blocks(a, [1, 2], [3, 4])),
        ("swap", lambda: ops.swap([1, 5], [2, 6], False, kv, host.tensor)),
        ("load_slices direct", lambda: ops.load_slices([dev_w], [host_w.tensor], mode="direct")),
        ("fence_publish", lambda: ops.fence_publish(hw, 0, 1, device=gpu,
                                                    stream=torch.cuda.current_stream(gpu))),
    ]
    for name, fn in calls:
        with pytest.raises(ValueError, match="captured"):
            _capture(gpu, fn)
        torch.cuda.synchronize()
    assert int(hw.words[0]) == 0
    before = [t.clone() for t in a]
    ops.copy_blocks(a, [1, 2], [3, 4])
    torch.cuda.synchronize()
    for t, b in zip(a, before):
        assert torch.equal(t[[3, 4]], b[[1, 2]])
    hw.close()
    host.free()
    host_w.free()


def test_fence_signal_and_wait_replay_from_a_graph(gpu):
    """The fence kernels take their arguments by value, so a captured signal
    and wait replay as captured: three replays, the word reset eagerly
    before each, each ending with the word at the captured value and no
    time-out flagged."""
    words = torch.zeros(2, dtype=torch.int64, device=gpu)
    flags = torch.zeros(2, dtype=torch.int64, device=gpu)
    torch.cuda.synchronize()

    def body():
        st = torch.cuda.current_stream(gpu)
        ops.fence_signal(words, 1, 5, stream=st)
        ops.fence_wait(words, 1, 5, flags, 1, timeout_s=10, stream=st)

    g = _capture(gpu, body)
    torch.cuda.synchronize()
    assert int(words[1]) == 0          # capturing ran nothing
    for r in range(3):
        words.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert int(words[1]) == 5, r
        assert int(flags.sum()) == 0, r
    del g
