"""Pins the oracle before anything is compared against it (CPU only).

The reference holds no tests or vectors for this path, so the oracle is
pinned by: golden fixtures whose expected outputs come from torch/numpy
index operations (tests/golden/make_golden.py), brute force over token
positions, the reference's own docstring and benchmark known answers, a
byte-provenance check that traces every moved byte back through the
inverse of the layout, and planted mistakes that these checks must catch.
"""

import math
import subprocess

import numpy as np
import pytest
import torch


# ------------------------------------------------------------- extent math --

def _brute(t, b, phys, kern, window):
    lo = 0 if window is None else max(0, t - window + 1)
    kbs = sorted({(p - b * phys) // kern for p in range(b * phys, (b + 1) * phys)
                  if lo <= p < t})
    return (kbs[0], len(kbs)) if kbs else (0, 0)


def test_extent_matches_golden_brute_force(oracle, golden):
    rows = golden("kernel_block_extent.npz")["rows"]
    assert len(rows) > 6000
    for t, b, phys, kern, w, f, c in rows.tolist():
        got = oracle.kernel_block_extent(t, b, phys, kern, None if w < 0 else w)
        assert got == (f, c), (t, b, phys, kern, w)


def test_extent_brute_force_dense_small(oracle):
    for phys, kern in ((16, 16), (32, 8), (48, 16), (12, 4)):
        for window in (None, 1, 3, 7, 16, 25):
            for t in range(0, 70):
                for b in range(0, 6):
                    assert oracle.kernel_block_extent(t, b, phys, kern, window) == \
                        _brute(t, b, phys, kern, window)


def test_extent_rejections(oracle):
    bad = [(-1, 0, 16, 16, None), (0, -1, 16, 16, None), (0, 0, 0, 16, None),
           (0, 0, 16, 0, None), (0, 0, 48, 32, None), (5, 0, 16, 16, 0)]
    for args in bad:
        with pytest.raises(ValueError):
            oracle.kernel_block_extent(*args)


def test_byte_extent_and_prefix(oracle):
    # every kernel block of a page maps to an equal, disjoint byte slice
    for page, kpp in ((65536, 1), (2162688, 33), (1114112, 17), (384, 4)):
        unit = page // kpp
        for first in range(kpp + 1):
            for num in range(kpp - first + 1):
                assert oracle.byte_extent(page, kpp, first, num) == (unit * first, unit * num)
    with pytest.raises(ValueError):
        oracle.byte_extent(384, 4, 3, 2)        # extent past the page
    with pytest.raises(ValueError):
        oracle.byte_extent(384, 4, -1, 1)
    with pytest.raises(ValueError):
        oracle.byte_extent(385, 4, 0, 1)        # page not divisible
    with pytest.raises(ValueError):
        oracle.prefix_bytes_for_kernel_blocks(384, 4, 5)


def visible_to_next_query(p: int, t: int, w) -> bool:
    """Whether committed token position p (< t) is visible to the next query,
    which sits at absolute position t: every earlier position for full
    attention (w None), the w-1 most recent ones under a sliding window of w
    (the window counts the query itself; block_manager.py:205-213)."""
    return p < t and (w is None or t - p < w)


def skipped_pages_by_enumeration(t: int, bs: int, w: int) -> int:
    """Leading pages of bs positions none of whose positions the next query
    can see and all of whose positions are committed: the pages a sliding
    window of w lets the cache release (cache_transfer.py:31-45,
    'leading complete pages invisible to the next SW query')."""
    n = 0
    while all(p < t and not visible_to_next_query(p, t, w)
              for p in range(n * bs, (n + 1) * bs)):
        n += 1
    return n


def check_window_helpers(oracle):
    for bs in (1, 4, 16):
        for w in (1, 2, 5, 16, 33):
            for t in range(0, 120):
                assert oracle.logical_blocks_for_tokens(t, bs) == math.ceil(t / bs)
                assert oracle.num_skipped_sliding_window_blocks(t, bs, w) == \
                    skipped_pages_by_enumeration(t, bs, w), (t, bs, w)
                # worst case over a query landing anywhere: pages a W-1 token
                # history plus the current page can touch
                worst = 0
                for start in range(bs):
                    span = set(range(start, start + w))
                    worst = max(worst, len({p // bs for p in span}))
                want = min(math.ceil(t / bs), worst) if t else 0
                assert oracle.sliding_window_resident_block_bound(t, bs, w) == want


def test_window_helpers_brute_force(oracle):
    check_window_helpers(oracle)


def test_skip_rule_known_answers(oracle):
    """Hand-worked cases of the release rule. 100 committed tokens, 32-token
    pages, window 20: the next query (position 100) sees 81..100, so pages
    0 (0-31) and 1 (32-63) are invisible and page 2 (64-95) is not. A
    window of 1 sees only the query: every complete committed page goes.
    A window one token short of reaching a page keeps it."""
    assert oracle.num_skipped_sliding_window_blocks(100, 32, 20) == 2
    assert oracle.num_skipped_sliding_window_blocks(96, 32, 1) == 3
    assert oracle.num_skipped_sliding_window_blocks(95, 32, 1) == 2    # page 2 holds 64-94
    assert oracle.num_skipped_sliding_window_blocks(64, 32, 1) == 2
    assert oracle.num_skipped_sliding_window_blocks(64, 32, 2) == 1    # sees 63
    assert oracle.num_skipped_sliding_window_blocks(0, 16, 5) == 0
    assert oracle.num_skipped_sliding_window_blocks(10, 16, 100) == 0


def test_reference_benchmark_extent_plan(oracle):
    """benchmark/benchmark_composite_swap.py:35-64,119-133 defaults: 8
    segments of a 17,301,504-byte page, 528-token pages, 16-token kernel
    blocks, 3 fixed pages. Bytes moved = sum over attention pages of
    ceil(tokens in page / 16) kernel blocks of 65,536 bytes, plus the fixed
    pages whole."""
    seg_page = 17_301_504 // 8
    kpp = 528 // 16
    assert seg_page // kpp == 65_536
    for length in (1, 128, 256, 512, 528, 529, 1057):
        pages = math.ceil(length / 528)
        new = 3 * seg_page
        for b in range(pages):
            f, c = oracle.kernel_block_extent(length, b, 528, 16)
            off, ln = oracle.byte_extent(seg_page, kpp, f, c)
            assert off == 0  # full attention: always a prefix
            new += ln
        tokens_per_page = [min(528, length - 528 * b) for b in range(pages)]
        want = 3 * seg_page + sum(math.ceil(t / 16) for t in tokens_per_page) * 65_536
        assert new == want, length


# ---------------------------------------------------------- whole-block moves --

def test_legacy_swap_golden(oracle, golden):
    z = golden("legacy_swap.npz")
    shape = tuple(z["cache_shape"])
    numel = int(np.prod(shape))
    cache = z["cache"].copy()
    pool = z["pool"].copy()
    oracle.swap_legacy(z["out_src"], z["out_dst"], False, cache.reshape(-1), numel,
                       shape[0], pool.reshape(-1))
    assert np.array_equal(pool, z["pool_after_out"])
    assert np.array_equal(cache, z["cache"])  # source untouched
    oracle.swap_legacy(z["in_src"], z["in_dst"], True, cache.reshape(-1), numel, shape[0],
                       pool.reshape(-1))
    assert np.array_equal(cache, z["cache_after_in"])


def test_legacy_swap_two_byte_block_size_quirk(oracle):
    """swap.cu:34 derives B = numel * 2 / size(0): for a 1-byte dtype that is
    twice the real block. The oracle keeps the quirk (it restates the
    reference); the product takes B explicitly."""
    cache = np.arange(4 * 8, dtype=np.uint8)  # 4 blocks of 8 one-byte elements
    pool = np.zeros(64, dtype=np.uint8)
    oracle.swap_legacy([1], [0], False, cache, 32, 4, pool)
    assert np.array_equal(pool[:16], cache[16:32])  # moved 16 bytes, not 8


def test_copy_blocks_golden(oracle, golden):
    z = golden("copy_blocks.npz")
    segs = [z[f"seg{i}"].copy() for i in range(3)]
    oracle.copy_blocks([s.reshape(-1) for s in segs], z["page"], 16, z["src"], z["dst"])
    for i in range(3):
        assert np.array_equal(segs[i], z[f"seg{i}_after"])


def test_copy_blocks_in_order_semantics(oracle):
    """Chained pairs apply in order (allocator.py:101-137 copies one tensor
    after another): 1->2 then 2->3 leaves block 1's bytes in block 3."""
    seg = np.repeat(np.arange(4, dtype=np.uint8), 4)
    oracle.copy_blocks([seg], [4], 4, [1, 2], [2, 3])
    assert seg.tolist() == [0] * 4 + [1] * 4 + [1] * 4 + [1] * 4


# --------------------------------------------------------- composite swaps --

def _composite(z):
    return dict(
        page=z["page"], cpu_off=z["cpu_off"], owners=z["owners"], kpp=z["kpp"],
        composite=int(z["composite"]), tp_rank=int(z["tp_rank"]),
        host_page=int(z["host_page"]), n_gpu=int(z["n_gpu"]),
    )


def _run_swap(oracle, z, segs, host, is_in, src, dst, lib=None):
    c = _composite(z)
    fn = oracle.swap_blocks if lib is None else lib
    return fn([s.reshape(-1) for s in segs], c["page"], c["cpu_off"], c["owners"], c["n_gpu"],
              c["kpp"], host.reshape(-1), c["host_page"], c["tp_rank"], c["composite"],
              src, dst, z["grp"], z["first"], z["valid"], is_in)


def test_swap_blocks_golden(oracle, golden):
    z = golden("composite_swap.npz")
    segs = [z[f"seg{s}"].copy() for s in range(5)]
    host = z["host"].copy()
    copied, ops = _run_swap(oracle, z, segs, host, False, z["src"], z["dst"])
    assert np.array_equal(host, z["host_after_out"])
    assert (copied, ops) == (int(z["copied_bytes"]), int(z["copy_operations"]))
    _run_swap(oracle, z, segs, host, True, z["in_src"], z["in_dst"])
    for s in range(5):
        assert np.array_equal(segs[s], z[f"seg{s}_after_in"])


def _provenance_check(oracle, swap_fn=None):
    """Label every device byte with its (segment, block, offset), swap out,
    then trace each host byte back through the inverse layout map: find the
    segment whose [cpu_off, cpu_off + page) holds the byte, the entry whose
    host id owns the page, and the kernel block the byte falls in."""
    rng = np.random.default_rng(5)
    page = np.array([64, 128, 96, 64], np.int64)
    owners = np.array([0b01, 0b11, 0b10, 0b01], np.uint64)
    kpp = np.array([4, 2], np.int64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    composite = int(page.sum())
    tp_size, tp_rank = 3, 2
    host_page = composite * tp_size
    n_gpu, n_host = 9, 7
    # 32-bit labels: segment * 2^24 + block * 2^12 + word offset (4-byte words)
    segs = []
    for s, p in enumerate(page):
        lab = (s << 24) + (np.arange(n_gpu)[:, None] << 12) + np.arange(p // 4)[None, :]
        segs.append(lab.astype(np.uint32).view(np.uint8).reshape(n_gpu, int(p)).copy())
    host = np.full((n_host, host_page), 0xEE, np.uint8)
    src = np.array([1, 4, 7, 2, 8], np.int64)
    dst = np.array([6, 0, 3, 5, 1], np.int64)
    grp = np.array([0, 1, 0, 1, 0], np.int32)
    first = np.array([0, 1, 2, 0, 1], np.int64)
    valid = np.array([4, 1, 2, 0, 2], np.int64)
    fn = swap_fn or oracle.swap_blocks
    fn([s.reshape(-1) for s in segs], page, cpu_off, owners, n_gpu, kpp, host.reshape(-1),
       host_page, tp_rank, composite, src, dst, grp, first, valid, False)
    words = host.view(np.uint32)
    for h in range(n_host):
        hits = np.nonzero(dst == h)[0]
        for wpos in range(host_page // 4):
            byte = wpos * 4
            rank, inside = divmod(byte, composite)
            expect = None
            if hits.size and rank == tp_rank:
                e = int(hits[0])
                s = int(np.searchsorted(cpu_off, inside, side="right") - 1)
                o = inside - int(cpu_off[s])
                g = int(grp[e])
                unit = int(page[s]) // int(kpp[g])
                kb = o // unit
                if (int(owners[s]) >> g) & 1 and first[e] <= kb < first[e] + valid[e]:
                    expect = (s << 24) + (int(src[e]) << 12) + o // 4
            got = int(words[h, wpos])
            if expect is None:
                assert got == 0xEEEEEEEE, (h, byte)
            else:
                assert got == expect, (h, byte, hex(got), hex(expect))


def test_swap_blocks_byte_provenance(oracle):
    _provenance_check(oracle)


def test_swap_blocks_round_trip_property(oracle):
    rng = np.random.default_rng(9)
    page = np.array([48, 48, 96], np.int64)
    owners = np.array([1, 1, 1], np.uint64)
    kpp = np.array([1], np.int64)
    composite = int(page.sum())
    n = 30
    segs = [rng.integers(0, 256, (n, int(p)), dtype=np.uint8) for p in page]
    host = np.zeros((n, composite), np.uint8)
    src = rng.permutation(n)[:12]
    hdst = rng.permutation(n)[:12]
    back = np.setdiff1d(np.arange(n), src)[:12]
    args = (page, np.concatenate([[0], np.cumsum(page)[:-1]]), owners, n, kpp)
    oracle.swap_blocks([s.reshape(-1) for s in segs], *args, host.reshape(-1), composite, 0,
                       composite, src, hdst, np.zeros(12, np.int32), np.zeros(12), np.ones(12),
                       False)
    oracle.swap_blocks([s.reshape(-1) for s in segs], *args, host.reshape(-1), composite, 0,
                       composite, hdst, back, np.zeros(12, np.int32), np.zeros(12), np.ones(12),
                       True)
    for s in segs:
        assert np.array_equal(s[back], s[src])


def test_swap_blocks_rejects_bad_extent(oracle, golden):
    z = golden("composite_swap.npz")
    segs = [z[f"seg{s}"].copy() for s in range(5)]
    c = _composite(z)
    with pytest.raises(ValueError):
        oracle.swap_blocks([s.reshape(-1) for s in segs], c["page"], c["cpu_off"], c["owners"],
                           c["n_gpu"], c["kpp"], z["host"].copy().reshape(-1), c["host_page"],
                           c["tp_rank"], c["composite"], [1], [1], [0], [3], [2], False)


def test_torch_path_port_matches_oracle(oracle, golden):
    """The CPU baseline's torch restatement (worker.py:2272-2328) agrees with
    the C oracle and the golden output, counters included."""
    z = golden("composite_swap.npz")
    c = _composite(z)
    segs = [torch.from_numpy(z[f"seg{s}"].copy()) for s in range(5)]
    host = torch.from_numpy(z["host"].copy())
    owners = [{g for g in range(3) if (int(m) >> g) & 1} for m in c["owners"]]
    copied, ops = oracle.swap_blocks_torch(
        segs, host, c["cpu_off"].tolist(), owners, c["kpp"].tolist(), c["tp_rank"],
        c["composite"], z["src"].tolist(), z["dst"].tolist(), z["grp"].tolist(),
        z["first"].tolist(), z["valid"].tolist(), False)
    assert np.array_equal(host.numpy(), z["host_after_out"])
    assert (copied, ops) == (int(z["copied_bytes"]), int(z["copy_operations"]))


# ------------------------------------------------------- planted mistakes --

MUTANTS = {
    # drop the segment's offset inside the composite page
    "no_cpu_offset": ("hoff = tp_rank * composite_page_bytes + segment_cpu_offsets[s] + off;",
                      "hoff = tp_rank * composite_page_bytes + off;"),
    # ignore the tensor-parallel rank's page
    "no_tp_rank": ("hoff = tp_rank * composite_page_bytes + segment_cpu_offsets[s] + off;",
                   "hoff = segment_cpu_offsets[s] + off;"),
    # start every extent at kernel block 0
    "first_ignored": ("oracle_prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,\n"
                      "                                            first_kernel_block, offset)",
                      "oracle_prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,\n"
                      "                                            0, offset)"),
    # copy segments the entry's group does not own
    "owner_ignored": ("if (!((segment_owner_masks[s] >> g) & 1u)) continue;", ""),
    # off-by-one at the window's first live token
    "window_off_by_one": ("live_start = cached_tokens - sliding_window + 1;",
                          "live_start = cached_tokens - sliding_window;"),
    # count a partly visible page as released (ceil instead of floor)
    "skip_rounds_up": ("*out = skipped / block_size;",
                       "*out = (skipped + block_size - 1) / block_size;"),
    # drop the query's own slot from the window in the release rule
    "skip_window_off_by_one": ("skipped = processed_computed_tokens - sliding_window + 1;",
                               "skipped = processed_computed_tokens - sliding_window;"),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistake_is_caught(oracle, tmp_path, name, golden):
    """Each mutant of the oracle source must fail the provenance check, the
    golden fixture or the brute-force extent check."""
    import importlib

    src = oracle.SRC.read_text()
    old, new = MUTANTS[name]
    assert old in src, name
    mutant_src = tmp_path / "mutant.c"
    mutant_src.write_text(src.replace(old, new))
    so = tmp_path / "libmutant.so"
    subprocess.run(["gcc", "-O1", "-std=c99", "-fPIC", "-shared", str(mutant_src), "-o",
                    str(so)], check=True, capture_output=True)
    mod = importlib.import_module("oracle.oracle")
    saved = mod._lib
    try:
        mod._lib = None
        orig_path = mod.LIB
        mod.LIB = so
        caught = False
        try:
            _provenance_check(mod)
        except AssertionError:
            caught = True
        if not caught:
            try:
                test_swap_blocks_golden(mod, golden)
            except AssertionError:
                caught = True
        if not caught:
            try:
                test_extent_matches_golden_brute_force(mod, golden)
            except AssertionError:
                caught = True
        if not caught:
            try:
                check_window_helpers(mod)
            except AssertionError:
                caught = True
        assert caught, f"mutant {name} survived"
    finally:
        mod._lib = saved
        mod.LIB = orig_path
