"""aegkv_copy_blocks_noalloc against aegkv_copy_blocks on the GPU.

Both entry points run the same copies on two identical caches, two calls in
a row on one stream (the second with fewer pairs) with no synchronization in
between, so a descriptor that was not taken from the fixed host area before
the next call overwrote it would show up as a difference. Byte equality
between the two caches, and the closed form seg[dst] == old seg[src].
"""

import ctypes
import sys

import numpy as np
import pytest
import torch

from aegaeon_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, file=sys.stderr, flush=True)


def _caches(n_seg, n_blocks, page, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    a = [torch.randint(0, 256, (n_blocks, page), dtype=torch.uint8, device=dev, generator=g)
         for _ in range(n_seg)]
    return a, [t.clone() for t in a]


def _pairs(rng, n_blocks, n):
    perm = rng.permutation(n_blocks)
    return perm[:n], perm[n:2 * n]


@pytest.mark.parametrize("n_seg,n_blocks,page,n1,n2", [
    (24, 512, 64 * 1024, 200, 37),        # 64 KiB tiles, one workgroup per tile
    (40, 256, 160 * 1024, 100, 1),        # 160 KiB tiles (10 loads per lane)
    (8, 1024, 16 * 1024, 500, 499),       # 16 KiB tiles
    (5, 64, 4000, 30, 7),                 # 16 B path with a tail chunk
    (3, 64, 1001, 20, 3),                 # byte path (odd page)
    (1, 2 * 65536 + 5, 256, 65536, 1000),  # the largest pair table
    (1024, 16, 64, 8, 5),                 # the largest segment table
])
def test_copy_blocks_noalloc_matches_copy_blocks(gpu, n_seg, n_blocks, page, n1, n2):
    _say("copy_blocks_noalloc vs copy_blocks", n_seg, n_blocks, page, n1, n2)
    rng = np.random.default_rng(n_seg * 1000 + n1)
    a, b = _caches(n_seg, n_blocks, page, n_seg + n1, gpu)
    before = [t.clone() for t in a]
    s1, d1 = _pairs(rng, n_blocks, n1)
    s2, d2 = _pairs(rng, n_blocks, n2)
    torch.cuda.synchronize()
    ops.copy_blocks(a, s1, d1)
    ops.copy_blocks(a, s2, d2)
    ops.copy_blocks_noalloc(b, s1, d1)
    ops.copy_blocks_noalloc(b, s2, d2)
    torch.cuda.synchronize()
    want = [t.clone() for t in before]
    for s_, d_ in ((s1, d1), (s2, d2)):
        si, di = torch.from_numpy(s_).to(gpu), torch.from_numpy(d_).to(gpu)
        for w in want:
            w[di] = w[si]
    for i in range(n_seg):
        assert torch.equal(a[i], b[i]), i
        assert torch.equal(b[i], want[i]), i


def test_copy_blocks_noalloc_after_rejection_and_on_a_second_stream(gpu):
    """A rejected call enqueues nothing and leaves the next call intact; the
    entry point runs on the stream it is given."""
    rng = np.random.default_rng(5)
    a, b = _caches(6, 128, 32 * 1024, 6, gpu)
    s1, d1 = _pairs(rng, 128, 40)
    with pytest.raises(ValueError, match="twice"):
        ops.copy_blocks_noalloc(b, s1[:2], [d1[0], d1[0]])
    with pytest.raises(ValueError, match="exceed"):
        ops.copy_blocks_noalloc(b, np.arange(ops.NOALLOC_MAX_PAIRS + 1),
                                np.arange(ops.NOALLOC_MAX_PAIRS + 1))
    st = torch.cuda.Stream(gpu)
    st.wait_stream(torch.cuda.current_stream(gpu))
    ops.copy_blocks(a, s1, d1)
    ops.copy_blocks_noalloc(b, s1, d1, stream=st)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert ctypes.sizeof(ctypes.c_int64) == 8 and _lib.load().aegkv_copy_blocks_noalloc


def test_copy_blocks_noalloc_under_graph_capture(gpu):
    """A graph that captures the call replays its own descriptor. Between
    replays the test rewrites the captured targets and makes other
    allocation-free calls (which rewrite the library's packing area and the
    device array), then synchronizes; each of three replays must copy the
    captured pairs, and only those. The captured descriptor (250 pairs over
    12 segments, 4512 bytes) spans three fill launches."""
    _say("copy_blocks_noalloc under graph capture")
    rng = np.random.default_rng(11)
    n_seg, n_blocks, page = 12, 1024, 32 * 1024
    a, _ = _caches(n_seg, n_blocks, page, 11, gpu)
    perm = rng.permutation(n_blocks)
    sa, da = perm[:250], perm[250:500]          # captured pairs
    sb, db = perm[500:600], perm[600:700]       # eager pairs between replays
    ops.copy_blocks_noalloc(a, sb[:1], db[:1])  # first call on the device outside the capture
    torch.cuda.synchronize()
    before = [t.clone() for t in a]
    graph = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream(gpu)
    with torch.cuda.graph(graph, stream=st):
        ops.copy_blocks_noalloc(a, sa, da)
    torch.cuda.synchronize()
    for x, y in zip(a, before):
        assert torch.equal(x, y)  # capturing ran nothing
    ia, ja = torch.from_numpy(sa).to(gpu), torch.from_numpy(da).to(gpu)
    for r in range(3):
        for t in a:
            t[ja] = r + 1
        k = 30 * r
        ops.copy_blocks_noalloc(a, sb[k:k + 30], db[k:k + 30])
        torch.cuda.synchronize()
        want = [t.clone() for t in a]
        for w in want:
            w[ja] = w[ia]
        graph.replay()
        torch.cuda.synchronize()
        for i in range(n_seg):
            assert torch.equal(a[i], want[i]), (r, i)
    del graph
