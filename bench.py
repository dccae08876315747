#!/usr/bin/env python
"""Benchmark of the KV-cache movement path on one MI355X.

Metric: KV swap GB/s (D2H/H2D, % of the measured host link) + HBM
block-copy GB/s (% of HBM peak). GB = 1e9 bytes.

One step = one pass of the path over one batch:
  * Qwen3-4B KV shape (72 x [8192,16,8,128] bf16): swap-out of 1024 seeded
    non-contiguous device blocks to a 4096-block pinned host pool, then
    swap-in of those 1024 host blocks to 1024 fresh device ids;
  * Llama-2-13B KV shape (80 x [8192,16,40,128] fp16): copy_blocks of 4096
    (src, dst) pairs, distinct targets disjoint from the sources.
Every operation is one libaegkv call on the current stream, timed with HIP
events recorded on that stream. Other configs (--config): varlen, overlap,
refplan, switch (see --help). `value` is the swap throughput (both
directions' bytes over their summed time); the copy_blocks kernel carries
the HBM roofline, the swaps the measured-host-link roofline. The line also
reports the two host-transfer designs (DIRECT, STAGED) side by side on the
same blocks, one call at a time, the reference's per-extent copy loop on the
same GPU, a model switch (both link directions at once) and the swaps
beside a GEMM loop (serving).

The CPU baseline times the reference's torch path (one narrow().copy_() per
(segment, block) extent, aegaeon/worker.py:2272-2328) on host tensors of the
Qwen3-4B shape with 2048 blocks: gather 256 blocks into contiguous staging,
scatter them to 256 other ids.
"""

from __future__ import annotations

import argparse
import faulthandler
import json
import os
import statistics
import subprocess
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = ("KV swap GB/s (D2H/H2D, % host link) + HBM block-copy GB/s (% HBM peak)")
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
# PCIe 5.0 x16, one direction: 16 lanes x 32 GT/s x 128/130 encoding; packet
# headers take a further share, which the measured link rate includes
PCIE_GEN5_X16_GBPS = round(16 * 32e9 * 128 / 130 / 8 / 1e9, 3)
TRAFFIC_FILE = REPO / "profiles" / "copy_blocks_traffic.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--mode", default="auto", choices=["auto", "direct", "staged"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-overlap", action="store_true",
                   help="skip the three-stream overlap config (run first, in a child process)")
    p.add_argument("--no-switch", action="store_true",
                   help="skip the model-switch line (both link directions at once)")
    p.add_argument("--cpu-runs", type=int, default=5)
    p.add_argument("--no-serving", action="store_true",
                   help="skip the serving line (swaps beside a GEMM loop)")
    p.add_argument("--weight-mode", default="auto", choices=["auto", "direct", "staged"],
                   help="switch config: how the incoming model's weights are loaded "
                        "(kernel over PCIe or the runtime's DMA per content)")
    p.add_argument("--no-weights", dest="weights", action="store_false",
                   help="switch config: KV swaps only, no weight loads")
    p.add_argument("--no-cu-partition", action="store_true",
                   help="overlap config: run the three streams on every CU")
    p.add_argument("--no-copy-partition", action="store_true",
                   help="skip the copy_blocks run on a 24-CU-per-XCD stream (keeps the "
                        "copy kernel's launches to the roofline ones)")
    p.add_argument("--no-side-by-side", action="store_true",
                   help="skip the DIRECT vs STAGED side-by-side measurement")
    p.add_argument("--no-reference-loop", action="store_true",
                   help="skip timing the reference per-extent copy loop on the GPU "
                        "(about 147k copy_ calls; very slow under a memory-copy trace)")
    p.add_argument("--swap-workgroups", default=None,
                   help="OUT,IN: swap-out (cached and uncached pools) and swap-in "
                        "workgroups for this process's swaps instead of the library's "
                        "defaults (the overlap child keeps --overlap-workgroups)")
    p.add_argument("--overlap-workgroups", default="16,16",
                   help="overlap config: swap-out,swap-in workgroups of its first run "
                        "(the second always uses the library's defaults)")
    p.add_argument("--config", default="headline",
                   choices=["headline", "varlen", "overlap", "refplan", "switch", "serving",
                            "tiles", "copy-beside-swaps"],
                   help="headline: Qwen3-4B swaps + Llama-2-13B copy_blocks (the metric line); "
                        "varlen: Qwen2.5-7B variable-length batched swap; overlap: "
                        "Qwen1.5-MoE swap-out + swap-in + copy_blocks on three streams; "
                        "refplan: the reference benchmark's extent plans, libaegkv beside "
                        "the reference's per-extent copy_ loop on the same GPU; switch: "
                        "two models' KV swapped out and in at once through the planner, "
                        "swapper and move ledger; serving: a bf16 GEMM loop beside both "
                        "swaps, for the default and a smaller swap grid; tiles: copy_blocks "
                        "by tile size (16-160 KiB) beside its read-only and write-only probes; "
                        "copy-beside-swaps: an HBM copy beside the swap kernels by swap grid")
    return p.parse_args()


def log_pinned(ops, where):
    """Pinned host memory the library holds (what counts against the host's
    per-process cap), on stderr."""
    pinned, free = ops.host_pinned_usage()
    log(f"pinned host memory {where}: {pinned / 2**30:.2f} GiB held, "
        f"{free / 2**30:.2f} GiB of it free for uncached pools")


def kv_segments(torch, n_layers, n_blocks, heads, dim, dtype, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    segs = []
    for _ in range(2 * n_layers):
        t = torch.empty(n_blocks, 16, heads, dim, dtype=dtype, device=dev)
        t.normal_(generator=g)
        segs.append(t)
    return segs


def measure_link(torch, ops, dev, nbytes=1 << 30, reps=3):
    """Host-link ceilings: contiguous pinned hipMemcpyAsync each way, best of reps."""
    pool = ops.PinnedHostPool(nbytes)
    d = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = {}
    for name, fn in (("d2h", lambda: pool.tensor.copy_(d, non_blocking=True)),
                     ("h2d", lambda: d.copy_(pool.tensor, non_blocking=True))):
        best = 0.0
        for _ in range(reps + 1):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            best = max(best, nbytes / (a.elapsed_time(b) / 1e3) / 1e9)
        out[name] = best
    del d
    pool.free()
    return out


def measure_link_bidir(torch, ops, dev, nbytes=4 << 30, retries=6):
    """Both directions at once, aggregate GB/s: a D2H and an H2D runtime
    copy started together on two streams with hardware queues of their own
    (on streams that share a queue the copies run one after the other);
    best of three runs. Returns (ceiling, attempts).

    Right after another GPU process has exited (a test run, say), the two
    copies were seen running one after the other for some seconds (60 GB/s
    instead of 97) while its queues were still being released; a result
    below 1.25x one direction is measured again after 5 s, up to `retries`
    times. Every attempt is returned, so the record shows when that
    happened."""
    attempts = [_bidir_once(torch, ops, dev, nbytes)]
    for _ in range(retries):
        if max(attempts) > 1.25 * 57.0:
            break
        log(f"bidirectional copies ran one after the other ({attempts[-1]:.1f} GB/s); "
            "measuring again in 5 s")
        time.sleep(5)
        attempts.append(_bidir_once(torch, ops, dev, nbytes))
    return max(attempts), [round(x, 3) for x in attempts]


def _bidir_once(torch, ops, dev, nbytes):
    hp = [ops.PinnedHostPool(nbytes) for _ in range(2)]
    dv = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(2)]
    owners = [ops.DedicatedStream(dev) for _ in range(2)]
    st = [o.stream for o in owners]
    best = 0.0
    for _ in range(3):
        begin = torch.cuda.Event(enable_timing=True)
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        begin.record()
        for s_ in st:
            s_.wait_event(begin)
        with torch.cuda.stream(st[0]):
            hp[0].tensor.copy_(dv[0], non_blocking=True)
            ends[0].record()
        with torch.cuda.stream(st[1]):
            dv[1].copy_(hp[1].tensor, non_blocking=True)
            ends[1].record()
        torch.cuda.synchronize()
        span = max(begin.elapsed_time(e) for e in ends) / 1e3
        best = max(best, 2 * nbytes / span / 1e9)
    del dv
    for h in hp:
        h.free()
    for o in owners:
        o.close()
    return best


def measure_stream_copy(torch, dev, nbytes=4 << 30, reps=3):
    """Plain device-to-device copy of known size (torch's copy kernel)."""
    a_ = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b_ = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    best = 0.0
    for _ in range(reps + 1):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        b_.copy_(a_)
        e1.record()
        e1.synchronize()
        best = max(best, 2 * nbytes / (e0.elapsed_time(e1) / 1e3) / 1e9)
    del a_, b_
    return best


def copy_probes(torch, ops, segs, src, dst, nbytes, reps=5):
    """The copy's two halves on the same tiles with the same launch shape
    (aegkv_copy_probe): reading every source tile, then writing every target
    tile (their contents are lost). nbytes = bytes each half moves. Returns
    the rates and the read+write bound they imply for a copy (2 nbytes in
    nbytes/read + nbytes/write seconds); average over `reps` launches after
    one warm-up, timed with HIP events on the launching stream."""
    sink = torch.zeros(4, dtype=torch.int32, device=segs[0].device)
    out = {}
    for name, kind in (("read", ops.PROBE_READ), ("write", ops.PROBE_WRITE)):
        ops.copy_probe(kind, segs, src, dst, sink)
        a, b = ev_pair(torch)
        a.record()
        for _ in range(reps):
            ops.copy_probe(kind, segs, src, dst, sink)
        b.record()
        b.synchronize()
        out[name] = nbytes / (a.elapsed_time(b) / 1e3 / reps) / 1e9
    out["rw_bound"] = 2.0 / (1.0 / out["read"] + 1.0 / out["write"])
    return out


def copy_on_cu_partition(torch, ops, segs, src, dst, nbytes, cus_per_xcd, reps=5):
    """copy_blocks of the same pairs on a dedicated stream whose kernels run
    only on CUs [0, cus_per_xcd) of every XCD: fewer tiles in flight at once
    (one per CU), which eases the DRAM write contention a copy on every CU
    meets. nbytes = read + write bytes per copy. Average over `reps` launches
    after one warm-up, HIP events on that stream; the targets are checked
    against the sources afterwards on a sample of segments."""
    st = ops.DedicatedStream(segs[0].device, cu_mask=ops.xcd_cu_mask(cus_per_xcd))
    try:
        torch.cuda.synchronize()
        ops.copy_blocks(segs, src, dst, stream=st.stream)
        a, b = ev_pair(torch)
        a.record(st.stream)
        for _ in range(reps):
            ops.copy_blocks(segs, src, dst, stream=st.stream)
        b.record(st.stream)
        b.synchronize()
        gbps = nbytes / (a.elapsed_time(b) / 1e3 / reps) / 1e9
    finally:
        st.close()
    cs = torch.from_numpy(src).to(segs[0].device)
    cd = torch.from_numpy(dst).to(segs[0].device)
    if not all(torch.equal(s[cd], s[cs]) for s in segs[::10]):
        raise AssertionError("copy_blocks on the CU partition is not bit-exact")
    return {"cus_per_xcd": cus_per_xcd, "GBps_rw": round(gbps, 1),
            "frac_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}


def cpu_baseline(runs: int):
    """The reference's torch path on host tensors (oracle restatement), timed
    with one torch thread (the stated baseline) and with torch's default
    thread count."""
    import torch

    from oracle import oracle

    layers, blocks, heads, dim = 36, 2048, 8, 128
    g = torch.Generator().manual_seed(0)
    tensors = [torch.randn(blocks, 16, heads, dim, generator=g).to(torch.bfloat16)
               for _ in range(2 * layers)]
    pages = [t.view(torch.uint8).view(blocks, -1) for t in tensors]
    tile = pages[0].shape[1]
    S = len(pages)
    composite = S * tile
    n = 256
    perm = torch.randperm(blocks - 1, generator=g) + 1
    src, dst = perm[:n].tolist(), perm[n:2 * n].tolist()
    staging = torch.empty(n, composite, dtype=torch.uint8)
    owners = [{0}] * S
    cpu_off = [s * tile for s in range(S)]
    z, one = [0] * n, [1] * n
    default_threads = torch.get_num_threads()
    moved = 2 * n * composite
    rates = {}
    for threads in (1, default_threads):
        torch.set_num_threads(threads)
        times = []
        for r in range(runs + 1):
            t0 = time.perf_counter()
            oracle.swap_blocks_torch(pages, staging, cpu_off, owners, [1], 0, composite, src,
                                     list(range(n)), z, z, one, False)
            oracle.swap_blocks_torch(pages, staging, cpu_off, owners, [1], 0, composite,
                                     list(range(n)), dst, z, z, one, True)
            dt = time.perf_counter() - t0
            if r:
                times.append(dt)
        rates[threads] = moved / statistics.median(times) / 1e9
    torch.set_num_threads(default_threads)
    idx_s, idx_d = torch.tensor(src), torch.tensor(dst)
    ok = all(torch.equal(p[idx_d], p[idx_s]) for p in pages)
    if not ok:
        raise AssertionError("CPU baseline round trip is not bit-exact")
    return {
        "value": round(rates[1], 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "default_threads": default_threads,
        "value_default_threads": round(rates[default_threads], 3),
        "os_cpu_count": os.cpu_count(),
        "sample": (f"reference torch path (per-extent narrow().copy_(), worker.py:2272-2328) on "
                   f"host tensors: 72 x [2048,16,8,128] bf16 N(0,1); gather 256 blocks to "
                   f"staging + scatter to 256 other ids = {moved} bytes; median of {runs} runs "
                   f"each with torch threads 1 (value) and {default_threads} "
                   f"(value_default_threads), os.cpu_count()={os.cpu_count()}; bit-exact "
                   f"round trip"),
    }


def ev_pair(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def bench_varlen(args):
    """Qwen2.5-7B KV shape (56 x [16384,16,4,128] bf16): 64 requests with
    log-normal token lengths (median 1024, sigma 1.0, clipped to [16, 32768],
    rounded up to 16-token blocks) whose blocks sit at seeded random device
    ids; all of them swapped out in one batched call to host ids from the
    slab allocator, then back in to fresh seeded device ids in one call."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops
    from aegaeon_amd.planner import BLOCK_LOCATION_CPU, BlockPools

    dev = torch.device("cuda:0")
    _lib.load()
    L, NB, H, D = 28, 16384, 4, 128
    segs = kv_segments(torch, L, NB, H, D, torch.bfloat16, dev, 3)
    S = len(segs)
    tile = 16 * H * D * 2
    page = S * tile
    rng = np.random.default_rng(3)
    tokens = np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, 64))), 16, 32768)
    blocks = (np.ceil(tokens / 16)).astype(np.int64)
    total = int(blocks.sum())
    perm = rng.permutation(np.arange(1, NB))
    out_ids = perm[:total]
    in_ids = perm[total:2 * total]
    if in_ids.size < total:
        raise RuntimeError(f"{total} blocks per direction do not fit twice in {NB - 1} ids")
    slab = 1 << 30
    n_slabs = -(-total * page // slab) + 2
    pools = BlockPools(n_slabs, slab)
    host_ids = np.array(pools.allocate(total, BLOCK_LOCATION_CPU, (page // 2,)), np.int64)
    pool = ops.PinnedHostPool(n_slabs * slab, uncached=True)
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, NB, [1], pool.tensor, page, 0)
    lay = ops.SegmentLayout(segs, *common)
    z = np.zeros(total, np.int32)
    one = np.ones(total, np.int64)
    res = {}
    for mode in ("direct", "staged"):
        for _ in range(args.warmup):
            lay.swap(out_ids, host_ids, z, z, one, False, mode=mode)
            lay.swap(host_ids, in_ids, z, z, one, True, mode=mode)
        outs, ins = [], []
        for _ in range(args.steps):
            a, b = ev_pair(torch)
            c, d = ev_pair(torch)
            a.record()
            lay.swap(out_ids, host_ids, z, z, one, False, mode=mode)
            b.record()
            c.record()
            lay.swap(host_ids, in_ids, z, z, one, True, mode=mode)
            d.record()
            outs.append((a, b))
            ins.append((c, d))
        torch.cuda.synchronize()
        t_out = statistics.median(x.elapsed_time(y) / 1e3 for x, y in outs)
        t_in = statistics.median(x.elapsed_time(y) / 1e3 for x, y in ins)
        di, do = torch.from_numpy(in_ids).to(dev), torch.from_numpy(out_ids).to(dev)
        ok = all(torch.equal(t[di], t[do]) for t in segs)
        if not ok:
            raise AssertionError(f"varlen round trip not bit-exact ({mode})")
        res[mode] = {"d2h_GBps": round(total * page / t_out / 1e9, 3),
                     "h2d_GBps": round(total * page / t_in / 1e9, 3),
                     "d2h_ms": round(t_out * 1e3, 3), "h2d_ms": round(t_in * 1e3, 3)}
    link = measure_link(torch, ops, dev)
    pool.free()
    return {
        "metric": "KV swap GB/s, variable-length batched swap",
        "unit": "GB/s",
        "config": {"workload": "Qwen2.5-7B KV 56 x [16384,16,4,128] bf16, 64 requests, "
                               "log-normal lengths (median 1024, sigma 1.0), one call per direction",
                   "blocks_per_direction": total, "bytes_per_direction": total * page,
                   "host_ids": "slab allocator (contiguous runs)"},
        "modes": res,
        "link_GBps": {"d2h": round(link["d2h"], 3), "h2d": round(link["h2d"], 3)},
        "bit_exact_round_trip": True,
    }


TILE_SHAPES = (   # (name, layers, blocks, kv_heads): tiles of 16 x heads x 128 x 2 bytes
    ("Qwen2.5-7B 16 KiB tiles", 28, 16384, 4),
    ("Qwen3-4B 32 KiB tiles", 36, 8192, 8),
    ("Qwen1.5-MoE 64 KiB tiles", 24, 32768, 16),
    ("Llama-2-13B 160 KiB tiles", 40, 8192, 40),
)


def bench_tiles(args):
    """copy_blocks by tile size, beside its read-only and write-only probes
    on the same tiles: each workload's KV shape (Qwen2.5-7B, Qwen3-4B,
    Qwen1.5-MoE, Llama-2-13B), pairs = two disjoint seeded
    halves of the blocks (every block is a source or a target)."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    rows = []
    for name, layers, blocks, heads in TILE_SHAPES:
        log(f"tiles: {name}")
        segs = kv_segments(torch, layers, blocks, heads, 128, torch.bfloat16, dev, 7)
        tile = 16 * heads * 128 * 2
        perm = torch.randperm(blocks, generator=torch.Generator().manual_seed(7)).numpy()
        n = blocks // 2
        src, dst = perm[:n], perm[n:2 * n]
        nbytes = n * len(segs) * tile

        def timed():
            ops.copy_blocks(segs, src, dst)
            a, b = ev_pair(torch)
            a.record()
            for _ in range(args.steps):
                ops.copy_blocks(segs, src, dst)
            b.record()
            b.synchronize()
            return a.elapsed_time(b) / 1e3 / args.steps

        # the library's pair orders side by side (3 interleaved rounds,
        # medians): as given, by target id (the default), by source id
        default_order = _lib.tune(_lib.TUNE_COPY_ORDER)
        by_order = {o: [] for o in (0, 1, 2)}
        try:
            for _ in range(3):
                for o in by_order:
                    _lib.tune(_lib.TUNE_COPY_ORDER, o)
                    by_order[o].append(timed())
        finally:
            _lib.tune(_lib.TUNE_COPY_ORDER, default_order)
        t = statistics.median(by_order[default_order])
        si, di = torch.from_numpy(src).to(dev), torch.from_numpy(dst).to(dev)
        if not all(torch.equal(x[di], x[si]) for x in segs):
            raise AssertionError(f"{name}: copy_blocks is not bit-exact")
        pr = copy_probes(torch, ops, segs, src, dst, nbytes, reps=args.steps)
        copy = 2 * nbytes / t / 1e9
        rows.append({"shape": name, "tile_bytes": tile, "segments": len(segs), "pairs": n,
                     "bytes_rw": 2 * nbytes, "copy_ms": round(t * 1e3, 3),
                     "copy_GBps": round(copy, 1), "copy_frac_hbm_peak": round(copy / HBM_PEAK_GBPS, 4),
                     "copy_GBps_by_pair_order": {
                         k: round(2 * nbytes / statistics.median(by_order[o]) / 1e9, 1)
                         for k, o in (("as_given", 0), ("by_target", 1), ("by_source", 2))},
                     "read_GBps": round(pr["read"], 1), "write_GBps": round(pr["write"], 1),
                     "rw_bound_GBps": round(pr["rw_bound"], 1),
                     "copy_frac_of_rw_bound": round(copy / pr["rw_bound"], 4)})
        del segs
        torch.cuda.empty_cache()
    # a plain device copy of known size (4 GiB each way), the calibration
    # that HBM traffic counters of the kernels above are scaled by
    a_ = torch.empty(1 << 32, dtype=torch.uint8, device=dev)
    b_ = torch.empty_like(a_)
    b_.copy_(a_)
    torch.cuda.synchronize()
    del a_, b_
    return {"metric": "copy_blocks GB/s by tile size (read+write) with read/write probes",
            "unit": "GB/s", "steps": args.steps, "rows": rows,
            "calibration": "one torch copy_ of 4294967296 bytes each way at the end"}


def bench_overlap(args):
    """Qwen1.5-MoE KV shape (48 x [32768,16,16,128] bf16, 96 GiB): swap-out
    of 16384 blocks, swap-in of 12288 blocks and copy_blocks of 2048 pairs,
    each on its own stream, all enqueued together."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops

    dev = torch.device("cuda:0")
    _lib.load()
    # CU partition: the link-bound swap kernels on 8 CUs of every XCD, the
    # HBM-bound copy on the other 24, so the copy does not share CUs with waves
    # that wait on PCIe (without it the copy ran 150-200 ms instead of 11)
    partition = not getattr(args, "no_cu_partition", False)
    masks = ([ops.xcd_cu_mask(8, device=dev)] * 2 + [ops.xcd_cu_mask(24, 8, device=dev)]
             if partition else [None] * 3)
    owners = [ops.DedicatedStream(dev, m) for m in masks]
    bidir = getattr(args, "bidir", None) or measure_link_bidir(torch, ops, dev)[0]
    L, NB, H, D = 24, 32768, 16, 128
    NOUT, NIN, NP = 16384, 12288, 2048
    segs = kv_segments(torch, L, NB, H, D, torch.bfloat16, dev, 4)
    S = len(segs)
    tile = 16 * H * D * 2
    page = S * tile
    # 28,672 host pages need 84 GiB of pinned memory; hosts that cap pinned
    # memory lower (these pin 63 GiB but not 84) run the same shape with 7/8
    # or 3/4 of the swapped blocks.
    pool = None
    for scale in (1.0, 0.875, 0.75):
        try:
            pool = ops.PinnedHostPool((int(NOUT * scale) + int(NIN * scale)) * page,
                                      uncached=True)
            break
        except _lib.AegkvError as exc:
            log(f"pinned pool at swap scale {scale} refused: {exc}")
    if pool is None:
        raise RuntimeError("no pinned pool for the overlap config, even at 3/4 scale")
    NOUT, NIN = int(NOUT * scale), int(NIN * scale)
    log(f"overlap: swap-out {NOUT}, swap-in {NIN} blocks (scale {scale})")
    rng = np.random.default_rng(4)
    perm = rng.permutation(NB)
    out_ids, in_ids = perm[:NOUT], perm[NOUT:NOUT + NIN]
    csrc = perm[NOUT + NIN:NOUT + NIN + NP]
    cdst = perm[NOUT + NIN + NP:NOUT + NIN + 2 * NP]
    host_out = rng.permutation(NOUT + NIN)
    host_x, host_y = host_out[:NOUT], host_out[NOUT:]
    common = ([tile] * S, [i * tile for i in range(S)], [1] * S, NB, [1], pool.tensor, page, 0)
    lay = ops.SegmentLayout(segs, *common)
    zo, oo = np.zeros(NOUT, np.int32), np.ones(NOUT, np.int64)
    zi, oi = np.zeros(NIN, np.int32), np.ones(NIN, np.int64)
    # the incoming model's blocks were swapped out earlier: put them on the
    # host, remember their checksums, and clear them on the device
    lay.swap(in_ids, host_y, zi, zi, oi, False)
    di = torch.from_numpy(in_ids).to(dev)
    want_in = [t[di].view(NIN, -1).view(torch.int16).sum(dim=1, dtype=torch.int64) for t in segs]
    for t in segs:
        t.index_fill_(0, di, 0)
    torch.cuda.synchronize()
    # Three streams with hardware queues of their own; three runs, the
    # medians reported, for two swap grids: the library's defaults (sized
    # for the link alone) and 16 workgroups per swap kernel (128 KiB in
    # flight per direction), which leaves the L2 channels' memory request
    # queues to the copy: beyond about 16-24 workgroups the swap kernels'
    # host-bound requests, which take microseconds to complete, fill those
    # queues and the copy's HBM requests wait behind them.
    streams = [o.stream for o in owners]
    grid_keys = (_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, _lib.TUNE_SWAP_IN_WORKGROUPS)
    default_grid = tuple(_lib.tune(k) for k in grid_keys)
    shared_grid = tuple(int(x) for x in
                        getattr(args, "overlap_workgroups", "16,16").split(","))
    if len(shared_grid) != 2 or min(shared_grid) <= 0:
        raise ValueError(f"--overlap-workgroups takes two counts above zero, "
                         f"not {args.overlap_workgroups!r}")

    def three_streams(grid):
        for k, v in zip(grid_keys, grid):
            _lib.tune(k, v)
        runs = []
        for _ in range(3):
            evs = [ev_pair(torch) for _ in range(3)]
            begin = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            begin.record()
            for st in streams:
                st.wait_event(begin)
            with torch.cuda.stream(streams[0]):
                evs[0][0].record()
                lay.swap(out_ids, host_x, zo, zo, oo, False)
                evs[0][1].record()
            with torch.cuda.stream(streams[1]):
                evs[1][0].record()
                lay.swap(host_y, in_ids, zi, zi, oi, True)
                evs[1][1].record()
            with torch.cuda.stream(streams[2]):
                evs[2][0].record()
                ops.copy_blocks(segs, csrc, cdst)
                evs[2][1].record()
            torch.cuda.synchronize()
            runs.append((evs[0][0].elapsed_time(evs[0][1]) / 1e3,
                         evs[1][0].elapsed_time(evs[1][1]) / 1e3,
                         evs[2][0].elapsed_time(evs[2][1]) / 1e3,
                         max(begin.elapsed_time(e[1]) for e in evs) / 1e3))
        return tuple(statistics.median(r[i] for r in runs) for i in range(4))

    try:
        t_out, t_in, t_cp, span = three_streams(shared_grid)
        d_out, d_in, d_cp, d_span = three_streams(default_grid)
    finally:
        for k, v in zip(grid_keys, default_grid):
            _lib.tune(k, v)
    # the same copy alone on its stream (same CUs), for comparison
    alone = []
    for _ in range(3):
        a, b = ev_pair(torch)
        torch.cuda.synchronize()
        a.record(streams[2])
        ops.copy_blocks(segs, csrc, cdst, stream=streams[2])
        b.record(streams[2])
        b.synchronize()
        alone.append(a.elapsed_time(b) / 1e3)
    t_cp_alone = statistics.median(alone)
    # correctness of everything that ran concurrently
    ok_in = all(torch.equal(t[di].view(NIN, -1).view(torch.int16).sum(dim=1, dtype=torch.int64), w)
                for t, w in zip(segs, want_in))
    cs, cd = torch.from_numpy(csrc).to(dev), torch.from_numpy(cdst).to(dev)
    ok_cp = all(torch.equal(t[cd], t[cs]) for t in segs)
    pages = pool.tensor.view(NOUT + NIN, S, tile)
    ok_out = all(torch.equal(pages[int(host_x[k]), s].to(dev),
                             segs[s][int(out_ids[k])].view(torch.uint8).reshape(-1))
                 for k in (0, NOUT // 2, NOUT - 1) for s in (0, S // 2, S - 1))
    if not (ok_in and ok_cp and ok_out):
        raise AssertionError(f"overlap check failed: in {ok_in} copy {ok_cp} out {ok_out}")
    b_out, b_in, b_cp = NOUT * page, NIN * page, 2 * NP * page
    del lay, pages
    pool.free()
    del segs
    for o in owners:
        o.close()
    torch.cuda.empty_cache()
    return {
        "metric": "KV swap + copy_blocks GB/s, three streams at once",
        "unit": "GB/s",
        "config": {"workload": f"Qwen1.5-MoE KV 48 x [32768,16,16,128] bf16; swap-out {NOUT}, "
                               f"swap-in {NIN}, copy_blocks {NP} pairs, one stream each",
                   "bytes": {"d2h": b_out, "h2d": b_in, "copy_rw": b_cp},
                   "swap_block_scale": scale, "blocks": {"d2h": NOUT, "h2d": NIN, "pairs": NP},
                   "cu_partition": ("swap streams on 8 CUs of each XCD, copy stream on the other 24 of each XCD"
                                    if partition else None)},
        "swap_workgroups": {"d2h": shared_grid[0], "h2d": shared_grid[1],
                            "loads_per_lane": 2, "lanes": 256},
        "d2h_GBps": round(b_out / t_out / 1e9, 3),
        "h2d_GBps": round(b_in / t_in / 1e9, 3),
        "copy_blocks_GBps": round(b_cp / t_cp / 1e9, 1),
        "copy_blocks_alone_GBps": round(b_cp / t_cp_alone / 1e9, 1),
        "link_aggregate_GBps": round((b_out + b_in) / span / 1e9, 3),
        "link_bidirectional_ceiling_GBps": round(bidir, 3),
        "frac_bidirectional_ceiling": round((b_out + b_in) / span / 1e9 / bidir, 4),
        "wall_ms": round(span * 1e3, 3),
        "per_stream_ms": {"d2h": round(t_out * 1e3, 3), "h2d": round(t_in * 1e3, 3),
                          "copy": round(t_cp * 1e3, 3), "copy_alone": round(t_cp_alone * 1e3, 3)},
        "default_grid": {
            "swap_workgroups": {"d2h": default_grid[0], "h2d": default_grid[1]},
            "d2h_GBps": round(b_out / d_out / 1e9, 3),
            "h2d_GBps": round(b_in / d_in / 1e9, 3),
            "copy_blocks_GBps": round(b_cp / d_cp / 1e9, 1),
            "link_aggregate_GBps": round((b_out + b_in) / d_span / 1e9, 3),
            "frac_bidirectional_ceiling": round((b_out + b_in) / d_span / 1e9 / bidir, 4),
            "per_stream_ms": {"d2h": round(d_out * 1e3, 3), "h2d": round(d_in * 1e3, 3),
                              "copy": round(d_cp * 1e3, 3)}},
        "runs": 3, "statistic": "median",
        "bit_exact": True,
    }


def bench_copy_beside_swaps(args):
    """An HBM-bound copy beside the swap kernels, by swap grid: copy_blocks of
    2048 pairs of Qwen1.5-MoE tiles (48 x 64 KiB, 12.9 GB R+W) on 24 CUs of
    every XCD, started 25 ms into a DIRECT swap-out and/or swap-in of
    2048 blocks (6.4 GB each, uncached pool) on the other 8, for several
    workgroup counts per swap kernel (2 loads of 16 B per lane, 8 KiB per
    workgroup in flight). Reports each swap's rate, the copy's time and rate,
    and with both swaps the link aggregate over their span. Medians of 2."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    L, NB, H, D, NP, NS = 24, 8192, 16, 128, 2048, 2048
    segs = kv_segments(torch, L, NB, H, D, torch.bfloat16, dev, 4)
    S, tile = len(segs), 16 * H * D * 2
    page = S * tile
    pool = ops.PinnedHostPool(2 * NS * page, uncached=True)
    lay = ops.SegmentLayout(segs, [tile] * S, [i * tile for i in range(S)], [1] * S, NB, [1],
                            pool.tensor, page, 0)
    rng = np.random.default_rng(4)
    perm = rng.permutation(NB)
    out_ids, in_ids = perm[:NS], perm[NS:2 * NS]
    csrc, cdst = perm[2 * NS:2 * NS + NP], perm[2 * NS + NP:2 * NS + 2 * NP]
    hx, hy = np.arange(NS), np.arange(NS, 2 * NS)
    z, o = np.zeros(NS, np.int32), np.ones(NS, np.int64)
    lay.swap(in_ids, hy, z, z, o, False)
    torch.cuda.synchronize()
    s_out = ops.DedicatedStream(dev, ops.xcd_cu_mask(8))
    s_in = ops.DedicatedStream(dev, ops.xcd_cu_mask(8))
    s_cp = ops.DedicatedStream(dev, ops.xcd_cu_mask(24, 8))
    sbytes, cbytes = NS * page, 2 * NP * S * tile
    keys = (_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, _lib.TUNE_SWAP_IN_WORKGROUPS)
    saved = [_lib.tune(k) for k in keys]

    def once(out_wg, in_wg, with_copy):
        if out_wg:
            _lib.tune(keys[0], out_wg)
        if in_wg:
            _lib.tune(keys[1], in_wg)
        torch.cuda.synchronize()
        begin = torch.cuda.Event(enable_timing=True)
        begin.record()
        ev = {}
        for name, wg, st in (("out", out_wg, s_out.stream), ("in", in_wg, s_in.stream)):
            if not wg:
                continue
            st.wait_event(begin)
            a, b = ev_pair(torch)
            a.record(st)
            if name == "out":
                lay.swap(out_ids, hx, z, z, o, False, stream=st)
            else:
                lay.swap(hy, in_ids, z, z, o, True, stream=st)
            b.record(st)
            ev[name] = (a, b)
        if with_copy:
            c = s_cp.stream
            c.wait_event(begin)
            a, b = ev_pair(torch)
            with torch.cuda.stream(c):
                torch.cuda._sleep(50_000_000)     # about 25 ms of shader clock
                a.record(c)
                ops.copy_blocks(segs, csrc, cdst, stream=c)
                b.record(c)
            ev["copy"] = (a, b)
        torch.cuda.synchronize()
        r = {k: a.elapsed_time(b) / 1e3 for k, (a, b) in ev.items()}
        if out_wg and in_wg:
            r["span"] = max(begin.elapsed_time(ev[k][1]) for k in ("out", "in")) / 1e3
        return r

    rows = []

    def record(case, out_wg, in_wg, with_copy, reps=2):
        rs = [once(out_wg, in_wg, with_copy) for _ in range(reps)]
        m = {k: statistics.median(r[k] for r in rs) for k in rs[0]}
        row = {"case": case, "swap_out_workgroups": out_wg or None,
               "swap_in_workgroups": in_wg or None}
        if "out" in m:
            row["d2h_GBps"] = round(sbytes / m["out"] / 1e9, 2)
        if "in" in m:
            row["h2d_GBps"] = round(sbytes / m["in"] / 1e9, 2)
        if "copy" in m:
            row["copy_ms"] = round(m["copy"] * 1e3, 3)
            row["copy_GBps"] = round(cbytes / m["copy"] / 1e9, 1)
        if "span" in m:
            row["link_aggregate_GBps"] = round(2 * sbytes / m["span"] / 1e9, 2)
        log(json.dumps(row))
        rows.append(row)

    try:
        record("copy alone", 0, 0, True, reps=3)
        for w in (8, 16, 24, 32, 64, 112):
            record("swap-out alone", w, 0, False)
            record("copy beside swap-out", w, 0, True)
        for w in (16, 32, 48, 64, 128):
            record("swap-in alone", 0, w, False)
            record("copy beside swap-in", 0, w, True)
        for wo, wi in ((8, 16), (16, 16), (16, 32), (24, 24), (24, 32), (32, 32), (32, 64),
                       (48, 64), (112, 128)):
            record("both swaps", wo, wi, False)
            record("copy beside both swaps", wo, wi, True)
    finally:
        for k, v in zip(keys, saved):
            _lib.tune(k, v)
        for st in (s_out, s_in, s_cp):
            st.close()
    cs, cd = torch.from_numpy(csrc).to(dev), torch.from_numpy(cdst).to(dev)
    if not all(torch.equal(t[cd], t[cs]) for t in segs):
        raise AssertionError("copy_blocks beside the swaps is not bit-exact")
    del lay
    pool.free()
    return {"metric": "copy_blocks GB/s beside the swap kernels, by swap grid",
            "unit": "GB/s",
            "config": {"workload": "Qwen1.5-MoE tiles (48 x [8192,16,16,128] bf16): copy_blocks "
                                   "of 2048 pairs on 24 CUs of every XCD, 25 ms into a swap-out "
                                   "and/or swap-in of 2048 blocks on the other 8",
                       "copy_bytes_rw": cbytes, "swap_bytes_per_direction": sbytes},
            "rows": rows, "statistic": "median of 2 (3 for the copy alone)", "bit_exact": True}


def bench_switch(args):
    """Token-level model switch through the whole host stack: two engines
    (models A and B, Qwen2.5-7B KV shape 56 x [16384,16,4,128] bf16 each) on
    one GPU and one pinned host pool. A switch moves every request of the
    active model out (plan_move -> KVSwapper.swap_blocks on its swap-out
    stream -> BlockPools.record_move) and every request of the other model in
    (same, swap-in stream, waiting on the requests' previous move events), so
    both link directions run at once. 64 requests per model, log-normal
    lengths as in the variable-length config; device free lists start
    shuffled so ids are scattered."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops
    from aegaeon_amd.cache_groups import BlockTable, CacheGroupConfig, CacheGroupRuntimeConfig
    from aegaeon_amd.layout import allocate_composite_cache, kv_tensor_specs
    from aegaeon_amd.planner import BLOCK_LOCATION_CPU, BlockPools, plan_move
    from aegaeon_amd.swapper import KVSwapper

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    bidir = getattr(args, "bidir", None)
    if bidir is None:   # measured before the swappers create their streams
        bidir = measure_link_bidir(torch, ops, dev)[0]
    L, NB, H, D, NREQ = 28, 16384, 4, 128, 64
    specs = kv_tensor_specs(L, NB, 16, H, D, 2)
    names = [{f"layers.{l}.{kv}" for l in range(L) for kv in ("k", "v")}]
    groups = (CacheGroupConfig("attention", 16, 16),)
    descr = [CacheGroupRuntimeConfig("attention", 16, 16)]
    caches = [allocate_composite_cache(specs, NB, dev) for _ in range(2)]
    g = torch.Generator(device=dev).manual_seed(5)
    for c in caches:
        for t in c.backing:
            t.view(torch.int32).random_(generator=g)
    page = caches[0].page_size_bytes
    shape = (page // 2,)
    rng = np.random.default_rng(5)
    lengths = [np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, NREQ))), 16, 32768)
               .astype(np.int64) for _ in range(2)]
    blocks = [int(np.ceil(x / 16).sum()) for x in lengths]
    slab = 1 << 30
    n_slabs = -(-sum(blocks) * page // slab) + 4
    pools = BlockPools(n_slabs, slab)
    host = ops.PinnedHostPool(n_slabs * slab, uncached=True)
    log_pinned(ops, "with the model-switch pool")
    sw = []
    for e in range(2):
        pools.register_gpu_space(e, NB, shape, groups)
        free = pools.gpu_free_blocks[e]
        free[:] = list(rng.permutation(free))
        # dedicated streams: nothing else runs on the GPU here, and the
        # swap-out and swap-in never land on one hardware queue
        sw.append(KVSwapper(caches[e], names, descr, host.tensor, dedicated_streams=True,
                            mode=getattr(args, "mode", "auto")))
    tables, reqs = {}, [[], []]
    for e in range(2):
        for i, tok in enumerate(lengths[e]):
            rid = e * 1000 + i
            n = groups[0].table_blocks_for_tokens(int(tok))
            tables[rid] = BlockTable(e, shape, groups, [pools.allocate(n, e, shape)])
            reqs[e].append((rid, int(tok)))
    # reference copies of every request's blocks, to check the final state
    want = {}
    for e in range(2):
        for rid, _ in reqs[e]:
            ids = torch.tensor(tables[rid].group_blocks[0], device=dev)
            want[rid] = [t.view(torch.uint8).view(NB, -1)[ids].clone() for t in caches[e].backing]
    latest = {}

    def move(e, target):
        plan = plan_move(reqs[e], tables, target, pools)
        s = sw[e]
        ev = s.swap_blocks(plan.request_ids, plan.source_block_ids, plan.target_block_ids,
                           plan.group_ids, plan.first_kernel_blocks, plan.valid_kernel_blocks,
                           [latest.get(r) for r in plan.request_ids], plan.is_swap_in)
        pools.record_move(plan, [ev])
        for r in plan.request_ids:
            latest[r] = ev
        return ev, len(plan.source_block_ids) * page

    log("parking model B on the host")
    move(1, BLOCK_LOCATION_CPU)[0].synchronize()
    active = 0
    runs = []
    for it in range(args.warmup + args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev_out, b_out = move(active, BLOCK_LOCATION_CPU)
        ev_in, b_in = move(1 - active, 1 - active)
        t1 = time.perf_counter()
        ev_out.synchronize()
        ev_in.synchronize()
        t2 = time.perf_counter()
        pools.reclaim_gpu_moves(active, wait=False)
        pools.reclaim_cpu_moves(shape, wait=False)
        if it >= args.warmup:
            runs.append((t2 - t0, t1 - t0, b_out, b_in))
        active = 1 - active
    # The same switches with the incoming model's weights loaded too (one
    # Qwen2.5-7B bf16 model, 30 contents, 15.2 GB, pinned on the host): on
    # the incoming swap-in stream before its KV swap-in, as Worker.switch
    # loads the model before the KV cache (worker.py:455-551). The weights
    # share the host-to-device direction with the KV swap-in.
    wruns = []
    w_bytes = 0
    link = getattr(args, "link", None)
    if getattr(args, "weights", True):
        from aegaeon_amd import weights as wmod

        sizes = wmod.qwen2_content_bytes()
        host_w = wmod.HostWeights(sizes, uncached=True)
        g8 = torch.Generator(device=dev).manual_seed(8)
        for h in host_w.slices:
            h.copy_(torch.randint(0, 256, (h.numel(),), dtype=torch.uint8, device=dev,
                                  generator=g8))
        dev_w = wmod.DeviceWeights(sizes, dev)
        w_bytes = host_w.total_bytes
        torch.cuda.synchronize()
        if link is None:
            link = measure_link(torch, ops, dev)
        wmode = getattr(args, "weight_mode", "auto")
        for it in range(1 + args.steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ev_out, b_out = move(active, BLOCK_LOCATION_CPU)
            wmod.load_model(dev_w, host_w, mode=wmode, stream=sw[1 - active].swap_in_stream)
            ev_in, b_in = move(1 - active, 1 - active)
            ev_out.synchronize()
            ev_in.synchronize()
            t2 = time.perf_counter()
            pools.reclaim_gpu_moves(active, wait=False)
            pools.reclaim_cpu_moves(shape, wait=False)
            if it >= 1:
                wruns.append((t2 - t0, b_out, b_in))
            active = 1 - active
        w_ok = all(torch.equal(d, h.to(dev)) for d, h in zip(dev_w.slices, host_w.slices))
        if not w_ok:
            raise AssertionError("weights loaded during the switch differ from the host copy")
        del dev_w
        host_w.free()
    # bring everything back to its own engine and compare with the copies
    for e in range(2):
        if tables[reqs[e][0][0]].location != e:
            move(e, e)[0].synchronize()
    ok = True
    for e in range(2):
        for rid, _ in reqs[e]:
            ids = torch.tensor(tables[rid].group_blocks[0], device=dev)
            got = [t.view(torch.uint8).view(NB, -1)[ids] for t in caches[e].backing]
            ok = ok and all(torch.equal(a, b) for a, b in zip(got, want[rid]))
    if not ok:
        raise AssertionError("model-switch round trips are not bit-exact")
    wall = statistics.median(r[0] for r in runs)
    host_ms = statistics.median(r[1] for r in runs) * 1e3
    moved = statistics.median(r[2] + r[3] for r in runs)
    with_weights = None
    if wruns:
        w_wall = statistics.median(r[0] for r in wruns)
        w_out = statistics.median(r[1] for r in wruns)
        w_in = statistics.median(r[2] for r in wruns)
        bound = max(w_out / (link["d2h"] * 1e9), (w_in + w_bytes) / (link["h2d"] * 1e9))
        with_weights = {
            "what": ("the same switches plus the incoming model's weights (Qwen2.5-7B bf16, 30 "
                     "contents) loaded with aegkv_load_slices on the incoming swap-in stream "
                     "before its KV swap-in"),
            "weight_bytes": w_bytes, "weight_mode": getattr(args, "weight_mode", "auto"),
            "switch_wall_ms": round(w_wall * 1e3, 3),
            "bytes_per_switch": {"kv_d2h": int(w_out), "kv_h2d": int(w_in), "weights_h2d": w_bytes},
            "h2d_GBps": round((w_in + w_bytes) / w_wall / 1e9, 3),
            "d2h_GBps": round(w_out / w_wall / 1e9, 3),
            "link_bound_ms": round(bound * 1e3, 3),
            "frac_link_bound": round(bound / w_wall, 4),
            "link_bound": "max(KV out / measured D2H link, (KV in + weights) / measured H2D link)",
            "bit_exact": True,
        }
    for s in sw:
        s.close()
    host.free()
    return {
        "with_weights": with_weights,
        "metric": "model-switch wall time and link rate through planner + swapper + ledger",
        "unit": "GB/s",
        "config": {"workload": "two Qwen2.5-7B KV caches (56 x [16384,16,4,128] bf16 each), "
                               f"{NREQ} requests per model, log-normal lengths (median 1024, "
                               "sigma 1.0); each switch swaps the active model out and the other "
                               "in at once",
                   "blocks": {"A": blocks[0], "B": blocks[1]}, "page_bytes": page,
                   "switches": args.steps, "warmup": args.warmup},
        "switch_wall_ms": round(wall * 1e3, 3),
        "host_plan_and_enqueue_ms": round(host_ms, 3),
        "bytes_per_switch": int(moved),
        "link_aggregate_GBps": round(moved / wall / 1e9, 3),
        "link_bidirectional_ceiling_GBps": round(bidir, 3),
        "frac_bidirectional_ceiling": round(moved / wall / 1e9 / bidir, 4),
        "statistic": "median over switches",
        "bit_exact": True,
    }


def bench_serving(args):
    """Swaps beside model compute: a bf16 8192 x 8192 x 8192 GEMM loop
    (torch.mm, 40 products) on its own stream while the Qwen3-4B swap-out
    and swap-in of 1024 blocks run on two more streams, all started
    together on streams with hardware queues of their own. Host ids are
    contiguous runs, as the slab allocator hands them out. Reported: the
    GEMM's TFLOP/s alone and beside the swaps, and the swap rates, for
    DIRECT with the default swap grid, DIRECT with a smaller grid (24
    workgroups per direction, 4 loads per lane) and STAGED (gather/scatter
    kernels in HBM, the link crossed by runtime copies)."""
    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()
    L, NB, H, D, HOST, N = 36, 8192, 8, 128, 4096, 1024
    segs = kv_segments(torch, L, NB, H, D, torch.bfloat16, dev, 1)
    S = len(segs)
    tile = 16 * H * D * 2
    page = S * tile
    g = torch.Generator().manual_seed(1)
    out_ids = (torch.randperm(NB - 1, generator=g)[:N] + 1).numpy()
    rest = np.setdiff1d(np.arange(1, NB), out_ids)
    in_ids = rest[torch.randperm(rest.size, generator=g)[:N].numpy()]
    host_ids, host_in = np.arange(N), np.arange(2 * N, 3 * N)
    z, one = np.zeros(N, np.int32), np.ones(N, np.int64)
    pool = ops.PinnedHostPool(HOST * page, uncached=True)
    lay = ops.SegmentLayout(segs, [tile] * S, [i * tile for i in range(S)], [1] * S, NB, [1],
                            pool.tensor, page, 0)
    lay.swap(in_ids, host_in, z, z, one, False)      # the incoming blocks, parked on the host
    M, iters = 8192, 40
    a = torch.randn(M, M, device=dev, dtype=torch.bfloat16)
    b = torch.randn(M, M, device=dev, dtype=torch.bfloat16)
    c = torch.empty(M, M, device=dev, dtype=torch.bfloat16)
    flops = iters * 2 * M ** 3
    streams = [ops.DedicatedStream(dev) for _ in range(3)]
    gemm_st, out_st, in_st = (x.stream for x in streams)
    with torch.cuda.stream(gemm_st):
        for _ in range(3):
            torch.mm(a, b, out=c)
    torch.cuda.synchronize()

    def once(with_swaps, mode="direct"):
        begin = torch.cuda.Event(enable_timing=True)
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda.synchronize()
        begin.record()
        for st in (gemm_st, out_st, in_st):
            st.wait_event(begin)
        with torch.cuda.stream(gemm_st):
            for _ in range(iters):
                torch.mm(a, b, out=c)
            ends[0].record()
        if with_swaps:
            lay.swap(out_ids, host_ids, z, z, one, False, mode=mode, stream=out_st)
            ends[1].record(out_st)
            lay.swap(host_in, in_ids, z, z, one, True, mode=mode, stream=in_st)
            ends[2].record(in_st)
        torch.cuda.synchronize()
        t = [begin.elapsed_time(e) / 1e3 for e in ends[:3 if with_swaps else 1]]
        return [flops / t[0] / 1e12] + [N * page / x / 1e9 for x in t[1:]]

    def median3(with_swaps, mode="direct"):
        runs = [once(with_swaps, mode) for _ in range(3)]
        return [round(statistics.median(r[i] for r in runs), 2) for i in range(len(runs[0]))]

    keys = (_lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED, _lib.TUNE_SWAP_IN_WORKGROUPS,
            _lib.TUNE_SWAP_UNROLL)
    saved = [_lib.tune(k) for k in keys]
    out = {"gemm_alone_TFLOPs": median3(False)[0]}
    for name, grid in (("default_grid", saved), ("grid_24x4", (24, 24, 4))):
        for k, v in zip(keys, grid):
            _lib.tune(k, int(v))
        gemm, d2h, h2d = median3(True)
        out[name] = {"workgroups_out_in_unroll": [int(v) for v in grid], "gemm_TFLOPs": gemm,
                     "swap_out_GBps": d2h, "swap_in_GBps": h2d}
    for k, v in zip(keys, saved):
        _lib.tune(k, v)
    gemm, d2h, h2d = median3(True, "staged")
    out["staged"] = {"gemm_TFLOPs": gemm, "swap_out_GBps": d2h, "swap_in_GBps": h2d}
    di, do = torch.from_numpy(in_ids).to(dev), torch.from_numpy(out_ids).to(dev)
    pages = pool.tensor.view(HOST, S, tile)
    ok = all(torch.equal(pages[int(host_ids[k]), s].to(dev),
                         segs[s][int(out_ids[k])].view(torch.uint8).reshape(-1))
             for k in (0, N // 2, N - 1) for s in (0, S - 1))
    if not ok:
        raise AssertionError("serving config: swapped pages are not bit-exact")
    for x in streams:
        x.close()
    del lay
    pool.free()
    return {"metric": "model GEMM TFLOP/s and swap GB/s when both run at once",
            "config": {"workload": "bf16 8192^3 torch.mm x 40 beside the Qwen3-4B swap-out and "
                                   "swap-in of 1024 blocks (72 x [8192,16,8,128] bf16, uncached "
                                   "4096-block pool, contiguous host ids)", "runs": 3,
                       "statistic": "median"},
            **out, "bit_exact": True}


def reference_submit_copies(cpu_pages, gpu_segments, extents, is_swap_in):
    """The reference benchmark's copy loop (benchmark_composite_swap.py:67-87):
    one narrow().copy_(non_blocking=True) per (segment, page) extent."""
    seg_page = gpu_segments[0].shape[1]
    for s, gpu_pages in enumerate(gpu_segments):
        for page_id, (off, ln) in enumerate(extents):
            if ln == 0:
                continue
            cpu_ext = cpu_pages[page_id].narrow(0, s * seg_page + off, ln)
            gpu_ext = gpu_pages[page_id].narrow(0, off, ln)
            if is_swap_in:
                gpu_ext.copy_(cpu_ext, non_blocking=True)
            else:
                cpu_ext.copy_(gpu_ext, non_blocking=True)


def reference_worker_loop(gpu_pages, host_view, tile, src_ids, dst_ids, is_swap_in):
    """Worker.swap_blocks' copy loop (aegaeon/worker.py:2272-2328) for whole
    tiles: segment-outer, entry-inner, one copy_(non_blocking=True) each."""
    for s, pages in enumerate(gpu_pages):
        hoff = s * tile
        for src, dst in zip(src_ids, dst_ids):
            if is_swap_in:
                pages[dst].copy_(host_view[src].narrow(0, hoff, tile), non_blocking=True)
            else:
                host_view[dst].narrow(0, hoff, tile).copy_(pages[src], non_blocking=True)


def bench_refplan(args):
    """The extent plans of benchmark/benchmark_composite_swap.py:35-64 with
    its defaults (:119-133): 8 segments of a 17,301,504-byte physical page,
    528-token physical pages, 16-token kernel blocks, 3 fixed pages, lengths
    1..1057. Each plan moves page i of the host pool to/from page i of every
    segment, either whole ("full") or only the live kernel blocks
    ("optimized"). Timed: libaegkv (one launch per call) and the reference's
    own per-extent copy_(non_blocking=True) loop (submit_copies,
    benchmark_composite_swap.py:67-87, restated below) on the same GPU and
    stream; p50 and p95 of `--steps` iterations after `--warmup`."""
    import math

    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops
    from aegaeon_amd.cache_transfer import (byte_extent_for_kernel_blocks,
                                            kernel_block_extent_for_attention_page)

    dev = torch.device("cuda:0")
    _lib.load()
    seg_n, phys_bytes, phys_tok, kern_tok, fixed = 8, 17_301_504, 528, 16, 3
    seg_page = phys_bytes // seg_n
    kpp = phys_tok // kern_tok
    stream = torch.cuda.Stream()
    out = []

    def timed(fn):
        """(p50, p95) ms per call; p95 is the nearest-rank percentile the
        reference benchmark reports (benchmark_composite_swap.py:30-32)."""
        for _ in range(args.warmup):
            with torch.cuda.stream(stream):
                fn()
        samples = []
        for _ in range(args.steps):
            a, b = ev_pair(torch)
            with torch.cuda.stream(stream):
                a.record(stream)
                fn()
                b.record(stream)
            b.synchronize()
            samples.append(a.elapsed_time(b))
        ordered = sorted(samples)
        return statistics.median(samples), ordered[math.ceil(0.95 * len(ordered)) - 1]

    def p50(fn):
        return timed(fn)[0]

    for length in (1, 128, 256, 512, 528, 529, 1057):
        pages = fixed + math.ceil(length / phys_tok)
        plans = {"full": [(0, kpp)] * pages,
                 "optimized": [(0, kpp)] * fixed + [
                     kernel_block_extent_for_attention_page(length, b, phys_tok, kern_tok)
                     for b in range(pages - fixed)]}
        host = ops.PinnedHostPool(pages * phys_bytes, uncached=True)
        segs = [torch.empty(pages, seg_page, dtype=torch.uint8, device=dev) for _ in range(seg_n)]
        for t in segs:
            t.random_(0, 256)
        ids = np.arange(pages)
        host_view = host.tensor.view(pages, phys_bytes)
        plan_lay = ops.SegmentLayout(segs, [seg_page] * seg_n,
                                     [s * seg_page for s in range(seg_n)], [1] * seg_n, pages,
                                     [kpp], host.tensor, phys_bytes, 0)
        row = {"length": length, "pages": pages}
        for name, plan in plans.items():
            first = np.array([f for f, _ in plan], np.int64)
            valid = np.array([c for _, c in plan], np.int64)
            grp = np.zeros(pages, np.int32)
            moved = int(valid.sum()) * (seg_page // kpp) * seg_n
            row[f"{name}_bytes"] = moved
            for direction, is_in in (("H2D", True), ("D2H", False)):
                t_aeg = timed(lambda: plan_lay.swap(ids, ids, grp, first, valid, is_in))
                extents = [byte_extent_for_kernel_blocks(seg_page, kpp, f, c) for f, c in plan]
                t_ref = timed(lambda: reference_submit_copies(host_view, segs, extents, is_in))
                row[f"{name}_{direction}_ms"] = {
                    "aegkv": round(t_aeg[0], 4), "reference_loop": round(t_ref[0], 4),
                    "aegkv_p95": round(t_aeg[1], 4), "reference_loop_p95": round(t_ref[1], 4)}
        # the last plan run both ways: check it landed where the plan says
        torch.cuda.synchronize()
        for s in range(seg_n):
            for pg, (f, c) in enumerate(plans["optimized"]):
                lo, hi = f * (seg_page // kpp), (f + c) * (seg_page // kpp)
                if hi > lo and not torch.equal(
                        segs[s][pg, lo:hi].cpu(),
                        host_view[pg, s * seg_page + lo:s * seg_page + hi]):
                    raise AssertionError(f"refplan mismatch at length {length}")
        out.append(row)
        del segs, plan_lay
        host.free()

    # Qwen3-4B: 1024 scattered blocks each way, whole tiles.
    S1, NB1, tile1, HOST1, n = 72, 8192, 32768, 4096, 1024
    segs1 = kv_segments(torch, 36, NB1, 8, 128, torch.bfloat16, dev, 1)
    pages1 = [t.view(torch.uint8).view(NB1, tile1) for t in segs1]
    pool = ops.PinnedHostPool(HOST1 * S1 * tile1, uncached=True)
    hv = pool.tensor.view(HOST1, S1 * tile1)
    g = torch.Generator().manual_seed(1)
    out_ids = (torch.randperm(NB1 - 1, generator=g)[:n] + 1).numpy()
    host_ids = torch.randperm(HOST1, generator=g)[:n].numpy()
    rest = np.setdiff1d(np.arange(1, NB1), out_ids)
    in_ids = rest[torch.randperm(rest.size, generator=g)[:n].numpy()]
    common = ([tile1] * S1, [i * tile1 for i in range(S1)], [1] * S1, NB1, [1], pool.tensor,
              S1 * tile1, 0)
    lay = ops.SegmentLayout(segs1, *common)
    z, one = np.zeros(n, np.int32), np.ones(n, np.int64)
    t_out = p50(lambda: lay.swap(out_ids, host_ids, z, z, one, False))
    t_in = p50(lambda: lay.swap(host_ids, in_ids, z, z, one, True))
    pl_out, pl_h, pl_in = out_ids.tolist(), host_ids.tolist(), in_ids.tolist()
    r_out = p50(lambda: reference_worker_loop(pages1, hv, tile1, pl_out, pl_h, False))
    r_in = p50(lambda: reference_worker_loop(pages1, hv, tile1, pl_h, pl_in, True))
    torch.cuda.synchronize()
    di, do = torch.from_numpy(in_ids).to(dev), torch.from_numpy(out_ids).to(dev)
    if not all(torch.equal(t[di], t[do]) for t in segs1):
        raise AssertionError("Qwen3-4B reference-loop round trip not bit-exact")
    # wall-clock latency of one swap-out call (host work + transfer), small to
    # large, as a model switch sees it
    latency = []
    for nb in (1, 4, 16, 64, 256, 1024):
        o_ids, h_ids = out_ids[:nb], host_ids[:nb]
        zz, oo = np.zeros(nb, np.int32), np.ones(nb, np.int64)
        pl_o, pl_h = o_ids.tolist(), h_ids.tolist()

        def wall(fn, reps=max(3, min(20, 2048 // nb))):
            fn()
            torch.cuda.synchronize()
            samples = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                torch.cuda.synchronize()
                samples.append((time.perf_counter() - t0) * 1e3)
            return statistics.median(samples)

        latency.append({
            "blocks": nb, "bytes": nb * S1 * tile1,
            "aegkv_ms": round(wall(lambda: lay.swap(o_ids, h_ids, zz, zz, oo, False)), 4),
            "reference_loop_ms": round(wall(lambda: reference_worker_loop(
                pages1, hv, tile1, pl_o, pl_h, False)), 4),
        })
    b1 = n * S1 * tile1
    qwen = {"blocks": n, "extents_per_direction": n * S1, "bytes_per_direction": b1,
            "swap_out_latency_wall": latency,
            "aegkv_ms": {"D2H": round(t_out, 3), "H2D": round(t_in, 3)},
            "reference_loop_ms": {"D2H": round(r_out, 3), "H2D": round(r_in, 3)},
            "aegkv_GBps": {"D2H": round(b1 / t_out / 1e6, 2), "H2D": round(b1 / t_in / 1e6, 2)},
            "reference_loop_GBps": {"D2H": round(b1 / r_out / 1e6, 2),
                                    "H2D": round(b1 / r_in / 1e6, 2)}}
    pool.free()
    return {
        "metric": "reference benchmark extent plans: p50 (and p95) ms per call",
        "config": {"workload": "benchmark_composite_swap defaults: 8 segments, 17,301,504-byte "
                               "physical page, 528-token pages, 16-token kernel blocks, 3 fixed "
                               "pages", "warmup": args.warmup, "iters": args.steps},
        "rows": out,
        "qwen3_4b_1024_blocks": qwen,
    }


def apply_swap_workgroups(args):
    """--swap-workgroups OUT,IN: this process's swap grids (loads the
    library, so it runs after any child process has been started)."""
    if not args.swap_workgroups:
        return
    from aegaeon_amd import _lib

    out_wg, in_wg = (int(x) for x in args.swap_workgroups.split(","))
    for key in (_lib.TUNE_SWAP_OUT_WORKGROUPS, _lib.TUNE_SWAP_OUT_WORKGROUPS_UNCACHED):
        _lib.tune(key, out_wg)
    _lib.tune(_lib.TUNE_SWAP_IN_WORKGROUPS, in_wg)
    log(f"swap workgroups set to {out_wg} out, {in_wg} in")


def main():
    # a crash in native code prints the Python stack of every thread
    faulthandler.enable()
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              "(swaps shard per GPU with no exchange step; run one process per GPU).",
              file=sys.stderr)
        sys.exit(2)
    if args.config != "headline":
        apply_swap_workgroups(args)
        fn = {"varlen": bench_varlen, "overlap": bench_overlap, "refplan": bench_refplan,
              "copy-beside-swaps": bench_copy_beside_swaps,
              "switch": bench_switch, "serving": bench_serving,
              "tiles": bench_tiles}[args.config]
        print(json.dumps(fn(args)), flush=True)
        return
    # Config c4 (Qwen1.5-MoE: swap-out, swap-in and copy_blocks on three
    # streams at once) runs first, in a process of its own, before this one
    # touches the GPU: its 96 GiB cache and 63 GiB pinned pool are gone when
    # the legs below start. Reported beside the metric.
    overlap = None
    if not args.no_overlap:
        log("overlap (Qwen1.5-MoE, three streams at once) in a process of its own")
        res = subprocess.run([sys.executable, str(REPO / "bench.py"), "--config", "overlap"],
                             stdout=subprocess.PIPE, text=True, timeout=900)
        if res.returncode == 0 and res.stdout.strip():
            ov = json.loads(res.stdout.strip().splitlines()[-1])
            overlap = {k: ov[k] for k in ("swap_workgroups", "d2h_GBps", "h2d_GBps",
                                          "copy_blocks_GBps", "copy_blocks_alone_GBps",
                                          "link_aggregate_GBps", "default_grid",
                                          "link_bidirectional_ceiling_GBps",
                                          "frac_bidirectional_ceiling", "wall_ms",
                                          "per_stream_ms", "bit_exact")}
            overlap["workload"] = ov["config"]["workload"]
            overlap["swap_block_scale"] = ov["config"]["swap_block_scale"]
            overlap["cu_partition"] = ov["config"]["cu_partition"]
            overlap["process"] = "bench.py --config overlap, a child process run first"
        else:
            overlap = {"error": f"bench.py --config overlap exited with {res.returncode}"}
    apply_swap_workgroups(args)   # after the child: this process touches the GPU from here

    import numpy as np
    import torch

    from aegaeon_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load()

    log("measuring host-link and stream-copy ceilings")
    log_pinned(ops, "before the link ceilings")
    bidir, bidir_attempts = measure_link_bidir(torch, ops, dev)
    link = measure_link(torch, ops, dev)
    stream_copy = measure_stream_copy(torch, dev)


    # ---- Qwen3-4B swap workload
    log("allocating Qwen3-4B KV cache and pinned pool")
    L1, NB1, H1, D1, HOST1, NSW = 36, 8192, 8, 128, 4096, 1024
    segs1 = kv_segments(torch, L1, NB1, H1, D1, torch.bfloat16, dev, 1)
    S1 = len(segs1)
    tile1 = 16 * H1 * D1 * 2
    pool = ops.PinnedHostPool(HOST1 * S1 * tile1, uncached=True)
    log_pinned(ops, "with the Qwen3-4B pool")
    g = torch.Generator().manual_seed(1)
    out_ids = (torch.randperm(NB1 - 1, generator=g)[:NSW] + 1).numpy()
    host_ids = torch.randperm(HOST1, generator=g)[:NSW].numpy()
    rest = np.setdiff1d(np.arange(1, NB1), out_ids)
    in_ids = rest[torch.randperm(rest.size, generator=g)[:NSW].numpy()]
    common1 = ([tile1] * S1, [s * tile1 for s in range(S1)], [1] * S1, NB1, [1], pool.tensor,
               S1 * tile1, 0)
    lay = ops.SegmentLayout(segs1, *common1)
    zero = np.zeros(NSW, np.int32)
    ones = np.ones(NSW, np.int64)
    swap_bytes = NSW * S1 * tile1

    # ---- Llama-2-13B copy_blocks workload
    log("allocating Llama-2-13B KV cache")
    L2, NB2, H2, D2, NP = 40, 8192, 40, 128, 4096
    segs2 = kv_segments(torch, L2, NB2, H2, D2, torch.float16, dev, 2)
    S2 = len(segs2)
    tile2 = 16 * H2 * D2 * 2
    g2 = torch.Generator().manual_seed(2)
    perm = torch.randperm(NB2, generator=g2)
    csrc, cdst = perm[:NP].numpy(), perm[NP:2 * NP].numpy()
    copy_bytes = 2 * NP * S2 * tile2

    def step(evs):
        evs[0].record()
        lay.swap(out_ids, host_ids, zero, zero, ones, False, mode=args.mode)
        evs[1].record()
        lay.swap(host_ids, in_ids, zero, zero, ones, True, mode=args.mode)
        evs[2].record()
        ops.copy_blocks(segs2, csrc, cdst)
        evs[3].record()

    def events():
        return [torch.cuda.Event(enable_timing=True) for _ in range(4)]

    log(f"warmup {args.warmup} steps")
    for _ in range(args.warmup):
        step(events())
    torch.cuda.synchronize()

    log(f"timing {args.steps} steps")
    all_evs = [events() for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for evs in all_evs:
        step(evs)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    d2h = [e[0].elapsed_time(e[1]) / 1e3 for e in all_evs]
    h2d = [e[1].elapsed_time(e[2]) / 1e3 for e in all_evs]
    cpy = [e[2].elapsed_time(e[3]) / 1e3 for e in all_evs]

    # ---- correctness of what was timed (size-independent properties)
    di, do = torch.from_numpy(in_ids).to(dev), torch.from_numpy(out_ids).to(dev)
    swap_ok = all(torch.equal(s[di], s[do]) for s in segs1)
    cs, cd = torch.from_numpy(csrc).to(dev), torch.from_numpy(cdst).to(dev)
    copy_ok = all(torch.equal(s[cd], s[cs]) for s in segs2)
    if not (swap_ok and copy_ok):
        raise AssertionError(f"bit-exact check failed: swap {swap_ok}, copy_blocks {copy_ok}")

    log("read-only and write-only probes over the copy's tiles")
    probes = copy_probes(torch, ops, segs2, csrc, cdst, copy_bytes // 2)

    part = None
    if not args.no_copy_partition:
        log("the same copy on a stream confined to 24 CUs of every XCD")
        part = copy_on_cu_partition(torch, ops, segs2, csrc, cdst, copy_bytes, 24)

    t_d2h, t_h2d, t_cpy = sum(d2h) / len(d2h), sum(h2d) / len(h2d), sum(cpy) / len(cpy)
    d2h_gbps = swap_bytes / t_d2h / 1e9
    h2d_gbps = swap_bytes / t_h2d / 1e9
    swap_gbps = 2 * swap_bytes / (t_d2h + t_h2d) / 1e9
    copy_gbps = copy_bytes / t_cpy / 1e9
    resolved = {0: "direct", 1: "direct", 2: "staged"}
    mode_d2h = args.mode if args.mode != "auto" else resolved[_lib.tune(_lib.TUNE_AUTO_D2H)]
    mode_h2d = args.mode if args.mode != "auto" else resolved[_lib.tune(_lib.TUNE_AUTO_H2D)]

    traffic = None
    if TRAFFIC_FILE.exists():
        tr = json.loads(TRAFFIC_FILE.read_text())
        if tr.get("workload") == "llama2-13b copy_blocks 4096 pairs":
            traffic = tr.get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(swap_gbps, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic: seeded N(0,1) bf16/fp16 KV caches, seeded block ids",
        "config": {
            "workload": ("Qwen3-4B KV swap-out + swap-in of 1024 blocks (72 x [8192,16,8,128] "
                         "bf16, 4096-block pinned pool) + Llama-2-13B copy_blocks of 4096 pairs "
                         "(80 x [8192,16,40,128] fp16)"),
            "swap_bytes_per_direction": swap_bytes,
            "copy_blocks_bytes_rw": copy_bytes,
            "transfer_mode": {"d2h": mode_d2h, "h2d": mode_h2d},
            "host_pool": "pinned, uncached (aegkv_host_alloc_flags AEGKV_HOST_UNCACHED)",
        },
        "swap": {
            "d2h_GBps": round(d2h_gbps, 3),
            "h2d_GBps": round(h2d_gbps, 3),
            "d2h_blocks_per_s": round(NSW / t_d2h, 1),
            "h2d_blocks_per_s": round(NSW / t_h2d, 1),
            "link_d2h_GBps": round(link["d2h"], 3),
            "link_h2d_GBps": round(link["h2d"], 3),
            "d2h_frac_link": round(d2h_gbps / link["d2h"], 4),
            "h2d_frac_link": round(h2d_gbps / link["h2d"], 4),
        },
        "copy_blocks": {
            "GBps_rw": round(copy_gbps, 1),
            "pairs_per_s": round(NP / t_cpy, 1),
            "frac_hbm_peak": round(copy_gbps / HBM_PEAK_GBPS, 4),
            "stream_copy_ceiling_GBps": round(stream_copy, 1),
            "pair_order": ("as_given", "by_target", "by_source")[_lib.tune(_lib.TUNE_COPY_ORDER)],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "copy_blocks_kernel",
            "achieved": round(copy_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(copy_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": (None if traffic is None else
                               "profiles/copy_blocks_traffic.json: rocprofv3 FETCH_SIZE and "
                               "WRITE_SIZE passes over this workload, scaled by a plain 4 GiB "
                               "copy's counts (not measured in this run)"),
            "avg_launch_ms": round(t_cpy * 1e3, 3),
        },
        "hbm_probes": {
            "what": ("the copy's halves alone on the same tiles, ids and launch shape "
                     "(aegkv_copy_probe): read every source tile / write every target tile; "
                     "a copy of B bytes each way needs at least B/read + B/write seconds"),
            "hbm_read_GBps": round(probes["read"], 1),
            "hbm_write_GBps": round(probes["write"], 1),
            "rw_bound_GBps": round(probes["rw_bound"], 1),
            "rw_bound_frac_hbm_peak": round(probes["rw_bound"] / HBM_PEAK_GBPS, 4),
            "copy_frac_of_rw_bound": round(copy_gbps / probes["rw_bound"], 4),
        },
        "copy_blocks_cu_partition": None if part is None else dict(part, what=(
            "the same copy on a dedicated stream masked to CUs 0-23 of every XCD "
            "(DedicatedStream(cu_mask=xcd_cu_mask(24))), a caller's choice, not the roofline "
            "value: one tile in flight per CU on 192 CUs instead of 256")),
        "link_roofline": {
            "bound": "host-link (measured)",
            "kernel": "swap_tiles_kernel",
            "achieved_d2h": round(d2h_gbps, 3),
            "achieved_h2d": round(h2d_gbps, 3),
            "peak_d2h": round(link["d2h"], 3),
            "peak_h2d": round(link["h2d"], 3),
            "unit": "GB/s",
            "frac_d2h": round(d2h_gbps / link["d2h"], 4),
            "frac_h2d": round(h2d_gbps / link["h2d"], 4),
            "avg_launch_ms_d2h": round(t_d2h * 1e3, 3),
            "avg_launch_ms_h2d": round(t_h2d * 1e3, 3),
            "pcie_gen5_x16_GBps": PCIE_GEN5_X16_GBPS,
            "frac_d2h_of_pcie": round(d2h_gbps / PCIE_GEN5_X16_GBPS, 4),
            "frac_h2d_of_pcie": round(h2d_gbps / PCIE_GEN5_X16_GBPS, 4),
        },
    }
    line["overlap"] = overlap
    line["link_bidirectional"] = {
        "ceiling_GBps": round(bidir, 3), "attempts_GBps": bidir_attempts,
        "what": "a D2H and an H2D 4 GiB runtime copy at once on two dedicated streams, best "
                "of 3 per attempt; an attempt below 1.25x one direction is repeated after 5 s"}
    # The reference's own data path on this GPU: Worker.swap_blocks' loop of
    # one copy_(non_blocking=True) per (segment, block) tile, same blocks.
    line["reference_path_same_gpu"] = None
    if not args.no_reference_loop:
        pages1 = [t.view(torch.uint8).view(NB1, tile1) for t in segs1]
        hv = pool.tensor.view(HOST1, S1 * tile1)
        ref = {}
        for name, src_l, dst_l, is_in in (("d2h", out_ids.tolist(), host_ids.tolist(), False),
                                          ("h2d", host_ids.tolist(), in_ids.tolist(), True)):
            log(f"timing the reference per-extent copy loop on the same GPU ({name})")
            reference_worker_loop(pages1, hv, tile1, src_l, dst_l, is_in)  # warm-up
            a, b = ev_pair(torch)
            a.record()
            reference_worker_loop(pages1, hv, tile1, src_l, dst_l, is_in)
            b.record()
            b.synchronize()
            ref[name] = swap_bytes / (a.elapsed_time(b) / 1e3) / 1e9
        if not all(torch.equal(s[di], s[do]) for s in segs1):
            raise AssertionError("reference-loop round trip is not bit-exact")
        line["reference_path_same_gpu"] = {
            "what": "reference per-extent copy_ loop (aegaeon/worker.py:2272-2328), 73,728 "
                    "copies per direction, same blocks and pool",
            "d2h_GBps": round(ref["d2h"], 3), "h2d_GBps": round(ref["h2d"], 3),
            "speedup_d2h": round(d2h_gbps / ref["d2h"], 2),
            "speedup_h2d": round(h2d_gbps / ref["h2d"], 2),
        }
    # The two host-transfer designs side by side on the same blocks, one
    # call at a time (each call timed alone, GPU idle when it is enqueued).
    line["designs_side_by_side"] = None
    if not args.no_side_by_side:
        log("DIRECT and STAGED side by side, one call at a time")
        side = {}
        for mode in ("direct", "staged"):
            rates = {"d2h": [], "h2d": []}
            for rep in range(4):
                for name, sargs in (("d2h", (out_ids, host_ids, zero, zero, ones, False)),
                                    ("h2d", (host_ids, in_ids, zero, zero, ones, True))):
                    torch.cuda.synchronize()
                    a, b = ev_pair(torch)
                    a.record()
                    lay.swap(*sargs, mode=mode)
                    b.record()
                    b.synchronize()
                    if rep:
                        rates[name].append(swap_bytes / (a.elapsed_time(b) / 1e3) / 1e9)
            if not all(torch.equal(s[di], s[do]) for s in segs1):
                raise AssertionError(f"{mode} side-by-side round trip is not bit-exact")
            side[mode] = {k: round(float(np.median(v)), 3) for k, v in rates.items()}
        line["designs_side_by_side"] = {
            "what": "same 1024 blocks and pool; median of 3 calls per direction after one "
                    "warm-up, each call timed alone",
            "direct_GBps": side["direct"], "staged_GBps": side["staged"]}
    pool.free()
    del segs1, segs2
    torch.cuda.empty_cache()
    # Both link directions at once, as a token-level model switch drives
    # them: planner + swapper + move ledger on two engines (see --config
    # switch). Reported beside the metric, not part of `value`.
    line["model_switch"] = None
    if not args.no_switch:
        log("model switch: two engines, swap-out and swap-in at once")
        sw = bench_switch(argparse.Namespace(steps=5, warmup=1, bidir=bidir, link=link,
                                             weights=True, weight_mode="auto"))
        line["model_switch"] = {k: sw[k] for k in (
            "switch_wall_ms", "host_plan_and_enqueue_ms", "bytes_per_switch",
            "link_aggregate_GBps", "link_bidirectional_ceiling_GBps",
            "frac_bidirectional_ceiling", "bit_exact", "with_weights")}
        line["model_switch"]["workload"] = sw["config"]["workload"]
        torch.cuda.empty_cache()
    # Swaps beside model compute (see --config serving): DIRECT or STAGED
    # against a concurrent GEMM. Reported beside the metric.
    line["serving"] = None
    if not args.no_serving:
        log("serving: swaps beside a bf16 GEMM loop")
        sv = bench_serving(args)
        line["serving"] = {k: sv[k] for k in ("gemm_alone_TFLOPs", "default_grid", "grid_24x4",
                                              "staged", "bit_exact")}
        line["serving"]["workload"] = sv["config"]["workload"]
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (reference torch path on host tensors)")
        line["cpu_baseline"] = cpu_baseline(args.cpu_runs)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
