"""Write the small seeded golden fixtures under tests/golden/.

The expected outputs are produced WITHOUT the oracle's loops:
  * whole-block moves (legacy swap, copy_blocks) with torch index_select /
    index_copy_ on uint8 [blocks, bytes] views, the textbook closed form of
    ops/swap.cu:36-58;
  * composite-page swaps with numpy fancy indexing built from per-byte
    liveness masks (token positions -> kernel blocks -> bytes), not from
    byte_extent arithmetic;
  * kernel-block extents by brute force over token positions.
No reference code is imported or run. Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def brute_extent(cached_tokens, block_index, phys, kern, window):
    """(first kernel block, count) of live tokens in one physical page, by
    enumerating positions: live = [max(0, t - W + 1) or 0, t)."""
    lo = 0 if window is None else max(0, cached_tokens - window + 1)
    live = [p for p in range(block_index * phys, (block_index + 1) * phys)
            if lo <= p < cached_tokens]
    if not live:
        return 0, 0
    kbs = sorted({(p - block_index * phys) // kern for p in live})
    assert kbs == list(range(kbs[0], kbs[-1] + 1))
    return kbs[0], len(kbs)


def legacy_swap_fixture():
    g = torch.Generator().manual_seed(11)
    n_cache, n_pool = 10, 8
    cache = torch.randn(n_cache, 16, 2, 8, generator=g).to(torch.bfloat16)
    pool = torch.randn(n_pool, 16, 2, 8, generator=g).to(torch.bfloat16)
    out_src = torch.tensor([3, 7, 1, 9, 4], dtype=torch.int64)
    out_dst = torch.tensor([6, 0, 2, 5, 7], dtype=torch.int64)
    in_src = torch.tensor([6, 2, 0, 5], dtype=torch.int64)
    in_dst = torch.tensor([2, 8, 5, 0], dtype=torch.int64)
    cb = cache.view(n_cache, -1).view(torch.uint8)
    pb = pool.view(n_pool, -1).view(torch.uint8)
    # swap-out: pool[dst] <- cache[src]
    pool_after = pb.clone().index_copy_(0, out_dst, cb.index_select(0, out_src))
    # swap-in (applied to the swapped-out pool): cache[dst] <- pool[src]
    cache_after = cb.clone().index_copy_(0, in_dst, pool_after.index_select(0, in_src))
    np.savez_compressed(
        OUT / "legacy_swap.npz",
        cache=cb.numpy(), pool=pb.numpy(), cache_shape=np.array(cache.shape),
        out_src=out_src.numpy(), out_dst=out_dst.numpy(),
        in_src=in_src.numpy(), in_dst=in_dst.numpy(),
        pool_after_out=pool_after.numpy(), cache_after_in=cache_after.numpy(),
    )


def composite_fixture():
    """Hybrid layout: 3 cache groups, 5 backing tensors, tp_size 2 (rank 1)."""
    rng = np.random.default_rng(12)
    # group: (kind, physical block tokens, kernel block tokens, window)
    groups = [("attention", 64, 16, None), ("mamba_none", 1, 1, None),
              ("attention", 32, 16, 20)]
    kpp = np.array([4, 1, 2], dtype=np.int64)
    page = np.array([256, 512, 128, 192, 384], dtype=np.int64)
    owners = np.array([0b001, 0b011, 0b010, 0b100, 0b101], dtype=np.uint64)
    cpu_off = np.concatenate([[0], np.cumsum(page)[:-1]]).astype(np.int64)
    composite = int(page.sum())
    tp_size, tp_rank = 2, 1
    host_page = composite * tp_size
    n_gpu, n_host = 12, 9
    segs = [rng.integers(0, 256, size=(n_gpu, int(p)), dtype=np.uint8) for p in page]
    host = rng.integers(0, 256, size=(n_host, host_page), dtype=np.uint8)
    # entries: (src, dst, group, cached_tokens, block_index) -> extent by brute force
    spec = [(3, 4, 0, 150, 0), (5, 1, 0, 150, 2), (7, 6, 0, 150, 1), (2, 0, 1, 0, 0),
            (9, 8, 2, 70, 1), (10, 2, 2, 70, 2), (11, 3, 2, 70, 0), (1, 7, 0, 64, 1)]
    src, dst, grp, first, valid = [], [], [], [], []
    for s_id, d_id, g, t, b in spec:
        kind, phys, kern, win = groups[g]
        if kind == "mamba_none":
            f, c = 0, 1
        else:
            f, c = brute_extent(t, b, phys, kern, win)
        src.append(s_id); dst.append(d_id); grp.append(g); first.append(f); valid.append(c)
    src, dst = np.array(src, np.int64), np.array(dst, np.int64)
    grp = np.array(grp, np.int32)
    first, valid = np.array(first, np.int64), np.array(valid, np.int64)

    def live_mask(s, e):
        """Byte mask of segment s's page that entry e moves, from the
        kernel-block liveness of each byte (byte b is in kernel block
        b // (page / kpp))."""
        g = grp[e]
        if not (int(owners[s]) >> int(g)) & 1:
            return np.zeros(int(page[s]), bool)
        kb = np.arange(int(page[s])) // (int(page[s]) // int(kpp[g]))
        return (kb >= first[e]) & (kb < first[e] + valid[e])

    # swap-out: device (src) -> host (dst)
    host_out = host.copy()
    for s in range(len(page)):
        for e in range(len(src)):
            m = live_mask(s, e)
            cols = tp_rank * composite + cpu_off[s] + np.nonzero(m)[0]
            host_out[dst[e], cols] = segs[s][src[e], np.nonzero(m)[0]]
    # swap-in: host (dst of the swap-out) -> device ids `in_dst`
    in_src = dst.copy()
    in_dst = np.array([0, 2, 5, 8, 11, 9, 6, 10], np.int64)
    segs_in = [x.copy() for x in segs]
    for s in range(len(page)):
        for e in range(len(in_src)):
            m = live_mask(s, e)
            idx = np.nonzero(m)[0]
            segs_in[s][in_dst[e], idx] = host_out[in_src[e], tp_rank * composite + cpu_off[s] + idx]
    copied = sum(int(live_mask(s, e).sum()) for s in range(len(page)) for e in range(len(src)))
    ops = sum(int(live_mask(s, e).any()) for s in range(len(page)) for e in range(len(src)))
    np.savez_compressed(
        OUT / "composite_swap.npz",
        kpp=kpp, page=page, owners=owners, cpu_off=cpu_off,
        composite=np.int64(composite), tp_rank=np.int64(tp_rank), host_page=np.int64(host_page),
        n_gpu=np.int64(n_gpu), host=host, src=src, dst=dst, grp=grp, first=first, valid=valid,
        host_after_out=host_out, in_src=in_src, in_dst=in_dst,
        copied_bytes=np.int64(copied), copy_operations=np.int64(ops),
        **{f"seg{s}": segs[s] for s in range(len(page))},
        **{f"seg{s}_after_in": segs_in[s] for s in range(len(page))},
    )


def copy_blocks_fixture():
    g = torch.Generator().manual_seed(13)
    n = 16
    pages = [64, 160, 48]
    segs = [torch.randint(0, 256, (n, p), dtype=torch.uint8, generator=g) for p in pages]
    src = torch.tensor([1, 4, 9, 12, 0], dtype=torch.int64)
    dst = torch.tensor([15, 3, 7, 2, 10], dtype=torch.int64)
    after = [t.clone().index_copy_(0, dst, t.index_select(0, src)) for t in segs]
    np.savez_compressed(
        OUT / "copy_blocks.npz", page=np.array(pages, np.int64), src=src.numpy(),
        dst=dst.numpy(), **{f"seg{i}": t.numpy() for i, t in enumerate(segs)},
        **{f"seg{i}_after": t.numpy() for i, t in enumerate(after)},
    )


def extent_fixture():
    rows = []
    for phys, kern in ((16, 16), (32, 16), (48, 16), (64, 16), (272, 16), (48, 8)):
        for window in (None, 1, 2, 15, 16, 17, 33, 40):
            for t in range(0, 100, 3):
                for b in range(0, 4):
                    f, c = brute_extent(t, b, phys, kern, window)
                    rows.append((t, b, phys, kern, -1 if window is None else window, f, c))
    np.savez_compressed(OUT / "kernel_block_extent.npz", rows=np.array(rows, np.int32))


if __name__ == "__main__":
    legacy_swap_fixture()
    composite_fixture()
    copy_blocks_fixture()
    extent_fixture()
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)
