"""Swap planning: destination allocation and the per-move copy lists.

Synchronous mirror of the planning half of the reference's BlockManager:
the GPU free lists (aegaeon/block_manager.py:718-793, 956-974), the CPU slab
allocator (:653-659, 976-1029), the move planner of move_requests
(:1355-1478), the move-event ledger (:518-563, 1498-1518) and the
reclamation of finished moves' source blocks (:661-690, 804-939). Ray RPC is
not part of it: a caller runs the returned SwapPlan through
KVSwapper.swap_blocks (or the C ABI) and either records the move with the
event that call returns (BlockPools.record_move; the ids come back when the
event has completed, in move order) or calls BlockPools.reclaim(plan) itself
once the move is known to be done. Where the reference awaits an event in an
asyncio task, this code polls it (query) or blocks on it (synchronize).
"""

from __future__ import annotations

import ctypes
import itertools
import math
from collections import defaultdict, deque
from dataclasses import dataclass, field
from typing import Callable, Deque, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _lib
from .cache_groups import (
    BLOCK_LOCATION_CPU,
    VLLM_NULL_BLOCK_ID,
    BlockTable,
    CacheGroupConfig,
    is_gpu,
)


def slab_range(slab: int, slab_size_bytes: int, block_size_bytes: int) -> Tuple[int, int]:
    """Host block ids wholly inside slab `slab` (block_manager.py:656-659):
    [ceil(slab * S / B), floor((slab + 1) * S / B))."""
    start = -(-(slab * slab_size_bytes) // block_size_bytes)
    end = ((slab + 1) * slab_size_bytes) // block_size_bytes
    return start, end


class BlockPools:
    """Free block ids per location: GPU engines and the CPU slab pool."""

    def __init__(self, cpu_num_slabs: int, cpu_slab_size_bytes: int, dtype_size: int = 2):
        if cpu_num_slabs < 0 or cpu_slab_size_bytes <= 0:
            raise ValueError("slab geometry must be positive")
        self.dtype_size = dtype_size
        self.cpu_num_slabs = cpu_num_slabs
        self.cpu_slab_size_bytes = cpu_slab_size_bytes
        self.cpu_free_blocks: Dict[Tuple[int, ...], Deque[int]] = defaultdict(deque)
        self.cpu_free_slabs: List[int] = list(range(cpu_num_slabs))
        self.cpu_slab_usage = np.zeros(cpu_num_slabs, np.int64)  # used blocks per slab
        self.cpu_block_shape: List[Optional[Tuple[int, ...]]] = [None] * cpu_num_slabs
        self.gpu_free_blocks: Dict[int, List[int]] = {}
        self.gpu_block_shape: Dict[int, Tuple[int, ...]] = {}
        self.gpu_cache_groups: Dict[int, Tuple[CacheGroupConfig, ...]] = {}
        # moves whose source ids are not free yet: swap-outs by source engine,
        # swap-ins by host block shape (block_manager.py:619-636)
        self._serial = itertools.count()
        self.move_events_gpu: Dict[int, Deque["MoveRecord"]] = defaultdict(deque)
        self.move_gpu_num_blocks: Dict[int, int] = defaultdict(int)
        self.move_events_cpu: Dict[Tuple[int, ...], Deque["MoveRecord"]] = defaultdict(deque)
        self.move_cpu_num_blocks: Dict[Tuple[int, ...], int] = defaultdict(int)

    def block_size_bytes(self, block_shape: Tuple[int, ...]) -> int:
        return math.prod(block_shape) * self.dtype_size

    def register_gpu_space(self, engine_id: int, num_max_blocks: int,
                           block_shape: Tuple[int, ...],
                           cache_groups: Sequence[CacheGroupConfig],
                           block_tables: Optional[Dict[int, BlockTable]] = None) -> None:
        """Expose device ids 1..num_max_blocks-1 (block 0 is vLLM's null
        block), as block_manager.py:775-792 does.

        Registering an engine again replaces its cache space
        (block_manager.py:718-761): no request in `block_tables` may still
        reside there, the engine's pending swap-outs are dropped (its free
        list is rebuilt whole) and the host ids of swap-ins into the old
        space are freed at once, since a model switch has already waited for
        every move into it. The arguments are checked before any state
        changes.
        """
        if num_max_blocks <= 1:
            raise ValueError(
                f"a GPU cache of {num_max_blocks} blocks has no block besides the null "
                "block 0"
            )
        if not cache_groups:
            raise ValueError("a GPU cache space needs at least one cache group")
        if engine_id in self.gpu_free_blocks and block_tables is not None:
            for rid, table in block_tables.items():
                if table.location == engine_id:
                    raise ValueError(
                        f"engine {engine_id}'s cache space cannot be replaced while "
                        f"request {rid} has blocks in it"
                    )
        self.move_events_gpu.pop(engine_id, None)
        self.move_gpu_num_blocks[engine_id] = 0
        old_shape = self.gpu_block_shape.get(engine_id)
        if old_shape is not None:
            pending = self.move_events_cpu[old_shape]
            keep = deque()
            for rec in pending:
                if rec.plan.target_location == engine_id:
                    self._reclaim_record(rec)
                else:
                    keep.append(rec)
            pending.clear()
            pending.extend(keep)
        self.gpu_block_shape[engine_id] = tuple(block_shape)
        self.gpu_cache_groups[engine_id] = tuple(cache_groups)
        self.gpu_free_blocks[engine_id] = list(range(VLLM_NULL_BLOCK_ID + 1, num_max_blocks))

    def _cpu_blocks_available(self, block_bytes: int, needed: int) -> bool:
        if needed <= 0:
            return True
        for slab in self.cpu_free_slabs:
            lo, hi = slab_range(slab, self.cpu_slab_size_bytes, block_bytes)
            needed -= hi - lo
            if needed <= 0:
                return True
        return False

    def allocate(self, num_blocks: int, location: int,
                 block_shape: Tuple[int, ...]) -> List[int]:
        """Reserve `num_blocks` ids at `location` (block_manager.py:942-1031).

        GPU: the FIFO prefix of the engine's free list. CPU: the shape's free
        deque, refilled from free slabs taken from the end of the slab list;
        each id lies wholly inside one slab. Raises ResourceWarning when the
        location cannot supply the ids (nothing is reserved then).
        """
        if num_blocks < 0:
            raise ValueError("num_blocks must be >= 0")
        block_shape = tuple(block_shape)
        if is_gpu(location):
            if location not in self.gpu_free_blocks:
                raise KeyError(f"no GPU cache space registered for engine {location}")
            free = self.gpu_free_blocks[location]
            if len(free) < num_blocks:
                # wait for this engine's swap-outs and take back their sources
                self.reclaim_gpu_moves(location, wait=True)
            if len(free) < num_blocks:
                raise ResourceWarning(
                    f"engine {location} has {len(free)} free blocks, {num_blocks} "
                    "asked for"
                )
            out = free[:num_blocks]
            del free[:num_blocks]
            return out
        block_bytes = self.block_size_bytes(block_shape)
        free = self.cpu_free_blocks[block_shape]
        if not self._cpu_blocks_available(block_bytes, num_blocks - len(free)):
            # wait for swap-ins of this shape, free their host ids and any
            # slab left empty (which may shrink `free`)
            self.reclaim_cpu_moves(block_shape, wait=True)
        if not self._cpu_blocks_available(block_bytes, num_blocks - len(free)):
            raise ResourceWarning(
                f"the host pool has {len(free)} free blocks and "
                f"{len(self.cpu_free_slabs)} free slabs, {num_blocks} blocks asked for"
            )
        while len(free) < num_blocks:
            slab = self.cpu_free_slabs.pop()
            lo, hi = slab_range(slab, self.cpu_slab_size_bytes, block_bytes)
            self.cpu_block_shape[slab] = block_shape
            free.extend(range(lo, hi))
        # the first num_blocks ids of the deque, in order
        out = list(itertools.islice(free, num_blocks))
        rest = list(itertools.islice(free, num_blocks, None))
        free.clear()
        free.extend(rest)
        if out:
            slabs = np.asarray(out, np.int64) * block_bytes // self.cpu_slab_size_bytes
            np.add.at(self.cpu_slab_usage, slabs, 1)
        return out

    def release(self, blocks: Sequence[int], location: int,
                block_shape: Tuple[int, ...]) -> None:
        """Return ids to their free list (block_manager.py:663-690)."""
        if is_gpu(location):
            self.gpu_free_blocks[location].extend(blocks)
            return
        block_shape = tuple(block_shape)
        block_bytes = self.block_size_bytes(block_shape)
        self.cpu_free_blocks[block_shape].extend(blocks)
        if len(blocks):
            slabs = np.asarray(blocks, np.int64) * block_bytes // self.cpu_slab_size_bytes
            np.subtract.at(self.cpu_slab_usage, slabs, 1)

    def reclaim(self, plan: "SwapPlan") -> None:
        """Free a completed move's source ids (all of them, including pages
        that were not copied)."""
        self.release(plan.release_source_block_ids, plan.source_location, plan.block_shape)

    # ------------------------------------------------------ move ledger --

    def record_move(self, plan: "SwapPlan", events: Sequence,
                    finished: Optional[Callable[[], bool]] = None) -> "MoveRecord":
        """Remember a submitted move until its events complete
        (block_manager.py:1498-1518).

        events: one completion event per worker that runs the move (objects
        with query() -> bool and synchronize(), e.g. the MoveEvent
        KVSwapper.swap_blocks returns or a FenceToken). finished: optional
        predicate that is true once every request of the move has finished,
        after which the move counts as done without looking at its events.

        An event whose move failed (a fence wait before it gave up, or a move
        it waited for failed) raises MoveFailedError from query() and
        synchronize(): the reclaim calls let it through and leave the move in
        the ledger, so its source ids are never freed for a move that did not
        happen (the reference stops the worker, worker.py:2364-2368).
        """
        rec = MoveRecord(next(self._serial), plan, list(events), finished)
        n = len(plan.release_source_block_ids)
        if is_gpu(plan.source_location):
            self.move_gpu_num_blocks[plan.source_location] += n
            self.move_events_gpu[plan.source_location].append(rec)
        else:
            self.move_cpu_num_blocks[plan.block_shape] += n
            self.move_events_cpu[plan.block_shape].append(rec)
        return rec

    def _reclaim_record(self, rec: "MoveRecord") -> int:
        """Return one finished move's source ids (block_manager.py:661-690)."""
        plan = rec.plan
        n = len(plan.release_source_block_ids)
        if is_gpu(plan.source_location):
            self.move_gpu_num_blocks[plan.source_location] -= n
        else:
            self.move_cpu_num_blocks[plan.block_shape] -= n
        self.release(plan.release_source_block_ids, plan.source_location, plan.block_shape)
        return n

    def _reclaim_queue(self, queue: Deque["MoveRecord"], wait: bool) -> Tuple[int, int]:
        """Reclaim moves in the order they were recorded, up to the newest
        one present at the call (block_manager.py:804-851). With wait, block
        on each move's events; without, stop at the first move still
        running. Returns (moves, blocks) reclaimed."""
        if not queue:
            return 0, 0
        target = queue[-1].serial
        moves = blocks = 0
        while queue and queue[0].serial <= target:
            rec = queue[0]
            if wait:
                rec.wait()
            elif not rec.done():
                break
            queue.popleft()
            moves += 1
            blocks += self._reclaim_record(rec)
        return moves, blocks

    def reclaim_gpu_moves(self, location: int, wait: bool = True) -> Tuple[int, int]:
        """Free the source ids of engine `location`'s swap-outs
        (block_manager.py:853-880)."""
        return self._reclaim_queue(self.move_events_gpu[location], wait)

    def reclaim_cpu_moves(self, block_shape: Tuple[int, ...],
                          wait: bool = True) -> Tuple[int, int]:
        """Free the host ids of swap-ins of `block_shape`, then every slab
        left empty (block_manager.py:882-916)."""
        got = self._reclaim_queue(self.move_events_cpu[tuple(block_shape)], wait)
        self.reclaim_cpu_slabs()
        return got

    def reclaim_cpu_slabs(self) -> int:
        """Give slabs with no used block back to the free slab list and drop
        their ids from the shape's free deque (block_manager.py:918-939)."""
        reclaimed = 0
        for slab, usage in enumerate(self.cpu_slab_usage):
            shape = self.cpu_block_shape[slab]
            if usage != 0 or shape is None:
                continue
            lo, hi = slab_range(slab, self.cpu_slab_size_bytes, self.block_size_bytes(shape))
            free = self.cpu_free_blocks[shape]
            kept = [b for b in free if not lo <= b < hi]
            free.clear()
            free.extend(kept)
            self.cpu_free_slabs.append(slab)
            self.cpu_block_shape[slab] = None
            reclaimed += 1
        return reclaimed


@dataclass
class MoveRecord:
    """One submitted move whose source ids are not free yet
    (MoveEvent, block_manager.py:518-563)."""

    serial: int
    plan: "SwapPlan"
    events: List
    finished: Optional[Callable[[], bool]] = None

    def done(self) -> bool:
        if self.finished is not None and self.finished():
            return True
        return all(ev.query() for ev in self.events)

    def wait(self) -> None:
        if self.finished is not None and self.finished():
            return
        for ev in self.events:
            ev.synchronize()


_KIND = {"attention": 0, "mamba_none": 1}


_Rows = Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray, np.ndarray, np.ndarray]


def _native_rows(groups: Sequence[CacheGroupConfig],
                 tables: Sequence[Tuple[BlockTable, int]]) -> _Rows:
    """aegkv_transfer_entries over many tables sharing `groups`: row arrays
    (table index, group, column, block id, first, count), rows in table,
    group, column order."""
    n_groups = len(groups)
    kind = np.array([_KIND[g.kind] for g in groups], np.int32)
    bs = np.array([g.block_size for g in groups], np.int64)
    kbs = np.array([g.kernel_block_size for g in groups], np.int64)
    win = np.array([0 if g.sliding_window is None else g.sliding_window for g in groups],
                   np.int64)
    tokens = np.array([tok for _, tok in tables], np.int64)
    lengths = [len(col) for table, _ in tables for col in table.group_blocks]
    if any(len(table.group_blocks) != n_groups for table, _ in tables):
        raise ValueError("every table must have one column list per cache group")
    offsets = np.zeros(len(lengths) + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    ids = np.fromiter(itertools.chain.from_iterable(
        col for table, _ in tables for col in table.group_blocks),
        dtype=np.int64, count=int(offsets[-1]))
    cap = max(1, int(offsets[-1]))
    out = {name: np.empty(cap, np.int64) for name in ("table", "column", "block", "first",
                                                       "count")}
    out_group = np.empty(cap, np.int32)
    n = ctypes.c_int64()
    p64 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))  # noqa: E731
    rc = _lib.load().aegkv_transfer_entries(
        n_groups, kind.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), p64(bs), p64(kbs),
        p64(win), len(tables), p64(tokens), p64(offsets), p64(ids), cap, p64(out["table"]),
        out_group.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), p64(out["column"]),
        p64(out["block"]), p64(out["first"]), p64(out["count"]), ctypes.byref(n))
    _lib.check(rc)
    m = n.value
    return (out["table"][:m], out_group[:m].astype(np.int64), out["column"][:m],
            out["block"][:m], out["first"][:m], out["count"][:m])


def _rows_from_lists(per_table: Sequence[Sequence[Tuple[int, int, int, int, int]]]) -> _Rows:
    """Row arrays from BlockTable.transfer_entries lists, one per table."""
    flat = [(t,) + row for t, rows in enumerate(per_table) for row in rows]
    a = np.array(flat, np.int64).reshape(-1, 6)
    return a[:, 0], a[:, 1], a[:, 2], a[:, 3], a[:, 4], a[:, 5]


def native_transfer_entries(groups: Sequence[CacheGroupConfig],
                            tables: Sequence[Tuple[BlockTable, int]]
                            ) -> List[List[Tuple[int, int, int, int, int]]]:
    """BlockTable.transfer_entries for many tables sharing `groups`, in one
    call into libaegkv (aegkv_transfer_entries). Returns one row list per
    table, each row (group, column, block id, first, count)."""
    tbl, grp, col, blk, first, count = _native_rows(groups, tables)
    rows: List[List[Tuple[int, int, int, int, int]]] = [[] for _ in tables]
    for t, g, c, b, f, k in zip(tbl.tolist(), grp.tolist(), col.tolist(), blk.tolist(),
                                first.tolist(), count.tolist()):
        rows[t].append((g, c, b, f, k))
    return rows


@dataclass
class SwapPlan:
    """One swap_blocks call's lists plus the bookkeeping of the move."""

    request_ids: List[int]
    source_location: int
    target_location: int
    block_shape: Tuple[int, ...]
    source_block_ids: List[int] = field(default_factory=list)
    target_block_ids: List[int] = field(default_factory=list)
    group_ids: List[int] = field(default_factory=list)
    first_kernel_blocks: List[int] = field(default_factory=list)
    valid_kernel_blocks: List[int] = field(default_factory=list)
    release_source_block_ids: List[int] = field(default_factory=list)

    @property
    def is_swap_in(self) -> bool:
        return is_gpu(self.target_location) and not is_gpu(self.source_location)

    @property
    def is_migration(self) -> bool:
        """GPU engine -> GPU engine (whole blocks, no host pages)."""
        return is_gpu(self.target_location) and is_gpu(self.source_location)

    @property
    def engine_id(self) -> int:
        """The GPU side of the swap, whose worker runs it."""
        return self.target_location if is_gpu(self.target_location) else self.source_location


def plan_move(requests: Sequence[Tuple[int, int]], block_tables: Dict[int, BlockTable],
              target_location: int, pools: BlockPools) -> Optional[SwapPlan]:
    """Plan moving requests' blocks to `target_location`
    (block_manager.py:1355-1478).

    requests: (request_id, processed_computed_tokens) pairs; duplicates are
    ignored, requests already at the target are skipped. All moved requests
    must share one source location and block shape. Destinations for every
    retained page are reserved in one allocation before any table changes;
    pages with nothing to copy get a destination but stay out of the copy
    lists; the tables are rewritten to the destination. Returns None when
    nothing moves.
    """
    seen = set()
    plans = []
    src_loc: Optional[int] = None
    shape: Optional[Tuple[int, ...]] = None
    moved_ids: List[int] = []
    release: List[int] = []
    for rid, tokens in requests:
        if rid in seen:
            continue
        seen.add(rid)
        table = block_tables.get(rid)
        if table is None:
            raise KeyError(f"request {rid} not allocated")
        if table.location == target_location:
            continue
        if is_gpu(table.location) and is_gpu(target_location):
            raise NotImplementedError("GPU to GPU moves go through plan_migrate")
        if src_loc is not None and table.location != src_loc:
            raise ValueError(f"request {rid} is on {table.location}; expected {src_loc}")
        if shape is not None and tuple(table.block_shape) != shape:
            raise ValueError(f"request {rid}'s shape is not {shape}")
        src_loc = table.location
        shape = tuple(table.block_shape)
        if is_gpu(target_location):
            groups = pools.gpu_cache_groups.get(target_location)
            if tuple(table.cache_groups) != groups:
                raise ValueError(
                    f"request {rid}'s cache groups differ from engine {target_location}'s"
                )
        plans.append((table, tokens, None))
        moved_ids.append(rid)
        release += table.blocks
    if not plans:
        return None
    # every moved table shares the source's cache groups; plan them in one call
    groups = plans[0][0].cache_groups
    if all(tuple(t.cache_groups) == tuple(groups) for t, _, _ in plans):
        rows = _native_rows(groups, [(t, tok) for t, tok, _ in plans])
    else:
        rows = _rows_from_lists([t.transfer_entries(tok) for t, tok, _ in plans])
    tbl, grp, col, blk, first, count = rows
    targets = np.asarray(pools.allocate(int(tbl.size), target_location, shape), np.int64)
    # copy lists: retained pages with live bytes, in table, group, column order
    live = count > 0
    plan = SwapPlan(moved_ids, src_loc, target_location, shape,
                    source_block_ids=blk[live].tolist(),
                    target_block_ids=targets[live].tolist(),
                    group_ids=grp[live].tolist(),
                    first_kernel_blocks=first[live].tolist(),
                    valid_kernel_blocks=count[live].tolist(),
                    release_source_block_ids=release)
    # destination tables: retained columns get their new ids, everything
    # else stays released (BlockTable.moved_group_blocks, same rows)
    bounds = np.searchsorted(tbl, np.arange(len(plans) + 1))
    for i, (table, _, _) in enumerate(plans):
        lo, hi = int(bounds[i]), int(bounds[i + 1])
        g_i, c_i, t_i = grp[lo:hi], col[lo:hi], targets[lo:hi]
        moved = []
        for g, cols in enumerate(table.group_blocks):
            new = np.full(len(cols), -1, np.int64)
            sel = g_i == g
            new[c_i[sel]] = t_i[sel]
            moved.append(new.tolist())
        table.group_blocks = moved
        table.location = target_location
    return plan


def plan_migrate(requests: Sequence[int], block_tables: Dict[int, BlockTable],
                 target_location: int, pools: BlockPools) -> Optional[SwapPlan]:
    """Plan moving requests' blocks from one GPU engine to another
    (BlockManager._migrate_requests, block_manager.py:1527-1601, which the
    reference declares but leaves unimplemented).

    Every moved request must sit on one source engine with one block shape,
    and the target engine must use the tables' cache groups. Each request's
    flat (non-released) blocks get fresh target ids in one allocation; the
    table keeps its released columns (replace_flat_blocks) and moves to the
    target. The returned plan lists whole blocks: source_block_ids on the
    source engine, target_block_ids on the target engine, and all source ids
    to free once the copy has finished (BlockPools.record_move). Returns
    None when nothing moves.
    """
    if not is_gpu(target_location):
        raise ValueError("migration targets a GPU engine; use plan_move for the host")
    seen = set()
    tables: List[Tuple[int, BlockTable]] = []
    src_loc: Optional[int] = None
    shape: Optional[Tuple[int, ...]] = None
    for rid in requests:
        if rid in seen:
            continue
        seen.add(rid)
        table = block_tables.get(rid)
        if table is None:
            raise KeyError(f"request {rid} not allocated")
        if table.location == target_location:
            continue
        if not is_gpu(table.location):
            raise ValueError(f"request {rid} is on the host; migration moves GPU blocks")
        if src_loc is not None and table.location != src_loc:
            raise ValueError(f"request {rid} is on {table.location}; expected {src_loc}")
        if shape is not None and tuple(table.block_shape) != shape:
            raise ValueError(f"request {rid}'s shape is not {shape}")
        if tuple(table.cache_groups) != pools.gpu_cache_groups.get(target_location):
            raise ValueError(
                f"request {rid}'s cache groups differ from engine {target_location}'s")
        src_loc = table.location
        shape = tuple(table.block_shape)
        tables.append((rid, table))
    if not tables:
        return None
    old = [table.blocks for _, table in tables]
    targets = pools.allocate(sum(len(b) for b in old), target_location, shape)
    plan = SwapPlan([rid for rid, _ in tables], src_loc, target_location, shape)
    cursor = 0
    for (_, table), blocks in zip(tables, old):
        new = targets[cursor:cursor + len(blocks)]
        cursor += len(blocks)
        table.replace_flat_blocks(new)
        table.location = target_location
        plan.source_block_ids += blocks
        plan.target_block_ids += new
    plan.release_source_block_ids = list(plan.source_block_ids)
    return plan


__all__ = ["BLOCK_LOCATION_CPU", "BlockPools", "MoveRecord", "SwapPlan", "plan_migrate",
           "plan_move", "slab_range"]
