"""Oracle for the KV movement path: TEST INFRASTRUCTURE, never product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only to check results / time the CPU baseline. It wraps the plain-C
restatement in aegkv_oracle.c (built by oracle/build.py into
oracle/liboracle_aegkv.so) and adds `swap_blocks_torch`, a torch-on-host
restatement of the reference's per-extent copy_ loop that the CPU baseline
times.

Parity status per function (the checks live in tests/test_oracle.py):
  swap_legacy, swap_blocks, copy_blocks, swap_blocks_torch: pinned by the
    golden fixtures (torch index ops, a different route than the loops) and
    by byte-provenance labels traced back through the inverse layout map.
  kernel_block_extent, byte_extent and the cache_transfer helpers: pinned by
    brute force over token positions, the reference's docstring known
    answers and its benchmark's extent plans.
  slab_range, plan_lists (tests/test_planner.py): pinned by invariants the
    reference's allocator and planner guarantee - a host page never
    straddles a slab, targets are distinct, every retained page appears
    once, pages with nothing to copy get a destination but no copy entry.
No function is "parity unpinned".
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Sequence

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
SRC = ORACLE_DIR / "aegkv_oracle.c"
LIB = ORACLE_DIR / "liboracle_aegkv.so"

OK, EVALUE, ERANGE = 0, -1, -2

_lib = None

_I64 = ctypes.c_int64
_I64P = ctypes.POINTER(ctypes.c_int64)
_I32P = ctypes.POINTER(ctypes.c_int32)
_U64P = ctypes.POINTER(ctypes.c_uint64)
_U8P = ctypes.POINTER(ctypes.c_uint8)
_U8PP = ctypes.POINTER(ctypes.POINTER(ctypes.c_uint8))


def build() -> Path:
    """Compile aegkv_oracle.c with gcc (always rebuilds)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c99", "-Wall", "-fPIC", "-shared", str(SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{res.stderr}")
    tmp.replace(LIB)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.oracle_logical_blocks_for_tokens.argtypes = [_I64, _I64, _I64P]
        L.oracle_sliding_window_resident_block_bound.argtypes = [_I64, _I64, _I64, _I64P]
        L.oracle_num_skipped_sliding_window_blocks.argtypes = [_I64, _I64, _I64, _I64P]
        L.oracle_kernel_block_extent.argtypes = [_I64, _I64, _I64, _I64, ctypes.c_int, _I64,
                                                 _I64P, _I64P]
        L.oracle_prefix_bytes_for_kernel_blocks.argtypes = [_I64, _I64, _I64, _I64P]
        L.oracle_byte_extent.argtypes = [_I64, _I64, _I64, _I64, _I64P, _I64P]
        L.oracle_swap_legacy.argtypes = [_I64P, _I64P, _I64, ctypes.c_int, _U8P, _I64, _I64,
                                         _I64, _U8P, _I64]
        L.oracle_swap_blocks.argtypes = [
            ctypes.c_int32, _U8PP, _I64P, _I64P, _U64P, _I64, _I64P, ctypes.c_int32, _U8P,
            _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I32P, _I64P, _I64P, ctypes.c_int,
            _I64P, _I64P,
        ]
        L.oracle_copy_blocks.argtypes = [ctypes.c_int32, _U8PP, _I64P, _I64, _I64, _I64P, _I64P]
        for name in ("oracle_logical_blocks_for_tokens",
                     "oracle_sliding_window_resident_block_bound",
                     "oracle_num_skipped_sliding_window_blocks", "oracle_kernel_block_extent",
                     "oracle_prefix_bytes_for_kernel_blocks", "oracle_byte_extent",
                     "oracle_swap_legacy", "oracle_swap_blocks", "oracle_copy_blocks"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


class OracleValueError(ValueError):
    pass


def _chk(rc: int) -> None:
    if rc == EVALUE:
        raise OracleValueError("rejected by the reference's validation")
    if rc == ERANGE:
        raise IndexError("byte range outside a buffer")
    if rc != OK:
        raise RuntimeError(f"oracle status {rc}")


def _a64(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.int64).reshape(-1))


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _u8(buf: np.ndarray) -> np.ndarray:
    if buf.dtype != np.uint8 or not buf.flags.c_contiguous:
        raise TypeError("oracle buffers must be C-contiguous uint8 arrays")
    return buf


# ------------------------------------------------------------ cache_transfer --

def logical_blocks_for_tokens(num_tokens: int, block_size: int) -> int:
    out = _I64()
    _chk(lib().oracle_logical_blocks_for_tokens(num_tokens, block_size, ctypes.byref(out)))
    return out.value


def sliding_window_resident_block_bound(num_tokens: int, block_size: int, window: int) -> int:
    out = _I64()
    _chk(lib().oracle_sliding_window_resident_block_bound(num_tokens, block_size, window,
                                                          ctypes.byref(out)))
    return out.value


def num_skipped_sliding_window_blocks(tokens: int, block_size: int, window: int) -> int:
    out = _I64()
    _chk(lib().oracle_num_skipped_sliding_window_blocks(tokens, block_size, window,
                                                        ctypes.byref(out)))
    return out.value


def kernel_block_extent(cached_tokens: int, physical_block_index: int,
                        physical_block_size: int, kernel_block_size: int,
                        sliding_window: int | None = None) -> tuple[int, int]:
    first, count = _I64(), _I64()
    has = 0 if sliding_window is None else 1
    _chk(lib().oracle_kernel_block_extent(cached_tokens, physical_block_index,
                                          physical_block_size, kernel_block_size, has,
                                          0 if sliding_window is None else sliding_window,
                                          ctypes.byref(first), ctypes.byref(count)))
    return first.value, count.value


def prefix_bytes_for_kernel_blocks(page: int, kpp: int, valid: int) -> int:
    out = _I64()
    _chk(lib().oracle_prefix_bytes_for_kernel_blocks(page, kpp, valid, ctypes.byref(out)))
    return out.value


def byte_extent(page: int, kpp: int, first: int, num: int) -> tuple[int, int]:
    off, ln = _I64(), _I64()
    _chk(lib().oracle_byte_extent(page, kpp, first, num, ctypes.byref(off), ctypes.byref(ln)))
    return off.value, ln.value


# ---------------------------------------------------------------- movement --

def swap_legacy(src_ids, dst_ids, is_swap_in: bool, kv_cache: np.ndarray,
                cache_numel: int, cache_size0: int, kv_swap: np.ndarray) -> None:
    """ops/swap.cu:25-60 on host byte buffers (modified in place)."""
    s, d = _a64(src_ids), _a64(dst_ids)
    kv_cache, kv_swap = _u8(kv_cache), _u8(kv_swap)
    _chk(lib().oracle_swap_legacy(_p(s, _I64P), _p(d, _I64P), s.size, int(is_swap_in),
                                  _p(kv_cache, _U8P), cache_numel, cache_size0,
                                  kv_cache.size, _p(kv_swap, _U8P), kv_swap.size))


def swap_blocks(segments: Sequence[np.ndarray], segment_page_bytes, segment_cpu_offsets,
                segment_owner_masks, num_gpu_blocks: int, group_kernel_blocks_per_page,
                host: np.ndarray, host_page_bytes: int, tp_rank: int,
                composite_page_bytes: int, src_ids, dst_ids, group_ids, first, valid,
                is_swap_in: bool) -> tuple[int, int]:
    """aegaeon/worker.py:2265-2329 on host byte buffers; returns the
    (copied_bytes, copy_operations) counters the reference logs."""
    segs = [_u8(x) for x in segments]
    arr = (ctypes.POINTER(ctypes.c_uint8) * len(segs))(*[_p(x, _U8P) for x in segs])
    page, coff = _a64(segment_page_bytes), _a64(segment_cpu_offsets)
    owners = np.ascontiguousarray(np.asarray(segment_owner_masks, dtype=np.uint64))
    kpp = _a64(group_kernel_blocks_per_page)
    s, d, f, v = _a64(src_ids), _a64(dst_ids), _a64(first), _a64(valid)
    g = np.ascontiguousarray(np.asarray(group_ids, dtype=np.int32).reshape(-1))
    host = _u8(host)
    cb, co = _I64(), _I64()
    _chk(lib().oracle_swap_blocks(
        len(segs), arr, _p(page, _I64P), _p(coff, _I64P), _p(owners, _U64P), num_gpu_blocks,
        _p(kpp, _I64P), kpp.size, _p(host, _U8P), host.size // host_page_bytes,
        host_page_bytes, tp_rank, composite_page_bytes, s.size, _p(s, _I64P), _p(d, _I64P),
        _p(g, _I32P), _p(f, _I64P), _p(v, _I64P), int(is_swap_in), ctypes.byref(cb),
        ctypes.byref(co)))
    return cb.value, co.value


def copy_blocks(segments: Sequence[np.ndarray], segment_page_bytes, num_blocks: int,
                src_ids, dst_ids) -> None:
    """In-order seg[dst] := seg[src] for every pair and segment (in place)."""
    segs = [_u8(x) for x in segments]
    arr = (ctypes.POINTER(ctypes.c_uint8) * len(segs))(*[_p(x, _U8P) for x in segs])
    page = _a64(segment_page_bytes)
    s, d = _a64(src_ids), _a64(dst_ids)
    _chk(lib().oracle_copy_blocks(len(segs), arr, _p(page, _I64P), num_blocks, s.size,
                                  _p(s, _I64P), _p(d, _I64P)))


# ------------------------------------------------- torch-on-host restatement --

def swap_blocks_torch(gpu_pages, host_view, segment_cpu_offsets, segment_owners,
                      group_kernel_blocks_per_page, tp_rank: int, composite_page_bytes: int,
                      src_ids, dst_ids, group_ids, first, valid, is_swap_in: bool,
                      non_blocking: bool = False):
    """The reference's torch path, aegaeon/worker.py:2272-2328, on host tensors.

    gpu_pages[s] is backing tensor s viewed as uint8 [num_blocks, page_s]
    (worker.py:2273-2277); host_view is uint8 [num_host_blocks, host_page]
    (worker.py:1428-1432). One narrow(...).copy_() per (segment, entry)
    extent, segment-outer, exactly as the reference issues them (without
    non_blocking, which has no effect between host tensors; pass
    non_blocking=True for device tensors, as the reference does).
    """
    copied = 0
    ops = 0
    for s, pages in enumerate(gpu_pages):
        page = pages.shape[1]
        owners = segment_owners[s]
        for src, dst, g, f, v in zip(src_ids, dst_ids, group_ids, first, valid):
            if g not in owners:
                continue
            kpp = group_kernel_blocks_per_page[g]
            off, ln = byte_extent(page, kpp, f, v)
            if ln == 0:
                continue
            copied += ln
            ops += 1
            hoff = tp_rank * composite_page_bytes + segment_cpu_offsets[s] + off
            if is_swap_in:
                pages[dst].narrow(0, off, ln).copy_(host_view[src].narrow(0, hoff, ln),
                                                    non_blocking=non_blocking)
            else:
                host_view[dst].narrow(0, hoff, ln).copy_(pages[src].narrow(0, off, ln),
                                                         non_blocking=non_blocking)
    return copied, ops


# ----------------------------------------------------------- move planning --

def slab_range(slab: int, slab_size_bytes: int, block_size_bytes: int) -> tuple[int, int]:
    """aegaeon/block_manager.py:656-659, with its float division."""
    import math

    return (math.ceil(slab * slab_size_bytes / block_size_bytes),
            math.floor((slab + 1) * slab_size_bytes / block_size_bytes))


def plan_lists(per_table_entries, targets):
    """aegaeon/block_manager.py:1439-1470: split the reserved `targets`
    across the tables in order; copy lists keep only entries with count > 0;
    each table's destination columns get their target ids (released columns
    stay -1). per_table_entries[i] = (entries, columns_per_group) with
    entries as BlockTable.transfer_entries rows."""
    src, dst, grp, first, valid, tables = [], [], [], [], [], []
    cursor = 0
    for entries, cols in per_table_entries:
        new_ids = targets[cursor:cursor + len(entries)]
        cursor += len(entries)
        for entry, t in zip(entries, new_ids):
            if entry[4] > 0:
                src.append(entry[2])
                dst.append(t)
                grp.append(entry[0])
                first.append(entry[3])
                valid.append(entry[4])
        moved = [[-1] * n for n in cols]
        for entry, t in zip(entries, new_ids):
            moved[entry[0]][entry[1]] = t
        tables.append(moved)
    return src, dst, grp, first, valid, tables
