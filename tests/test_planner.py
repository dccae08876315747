"""Swap planning: allocation and copy lists (CPU only)."""

import copy
import random

import pytest

from aegaeon_amd.cache_groups import LOGICAL_NULL_BLOCK_ID, BlockTable, CacheGroupConfig
from aegaeon_amd.planner import BLOCK_LOCATION_CPU, BlockPools, plan_move, slab_range

GROUPS = (CacheGroupConfig("attention", 32, 16),
          CacheGroupConfig("attention", 32, 16, sliding_window=40),
          CacheGroupConfig("mamba_none", 1, 1))
SHAPE = (1000,)  # 2000-byte host blocks


def test_slab_range_matches_reference_formula(oracle):
    for slab_bytes in (4096, 1 << 20, 3 * 7 * 1000):
        for block in (2000, 2048, 4096, 2_359_296, 3_145_728):
            for slab in range(0, 40):
                assert slab_range(slab, slab_bytes, block) == oracle.slab_range(slab, slab_bytes, block)


def test_cpu_blocks_never_straddle_slabs():
    pools = BlockPools(cpu_num_slabs=6, cpu_slab_size_bytes=7000)
    got = pools.allocate(12, BLOCK_LOCATION_CPU, SHAPE)
    assert len(set(got)) == 12
    for b in got:
        # bytes [b*2000, (b+1)*2000) inside one 7000-byte slab
        assert b * 2000 // 7000 == ((b + 1) * 2000 - 1) // 7000
    # slabs are taken from the end of the slab list, ids ascend inside a slab
    assert got[:3] == list(range(*slab_range(5, 7000, 2000)))
    assert sum(pools.cpu_slab_usage) == 12
    with pytest.raises(ResourceWarning):
        pools.allocate(100, BLOCK_LOCATION_CPU, SHAPE)
    pools.release(got[:5], BLOCK_LOCATION_CPU, SHAPE)
    assert sum(pools.cpu_slab_usage) == 7


def test_gpu_free_list_fifo_and_null_block():
    pools = BlockPools(1, 1 << 20)
    pools.register_gpu_space(0, 10, SHAPE, GROUPS)
    assert pools.allocate(3, 0, SHAPE) == [1, 2, 3]
    assert pools.allocate(2, 0, SHAPE) == [4, 5]
    with pytest.raises(ResourceWarning):
        pools.allocate(5, 0, SHAPE)
    pools.release([2, 4], 0, SHAPE)
    assert pools.allocate(6, 0, SHAPE) == [6, 7, 8, 9, 2, 4]
    with pytest.raises(ValueError):
        pools.register_gpu_space(1, 1, SHAPE, GROUPS)


def _tables(rng, n_req, pools):
    tables = {}
    reqs = []
    for rid in range(n_req):
        tokens = rng.randint(1, 200)
        cols = [GROUPS[0].table_blocks_for_tokens(tokens), GROUPS[1].table_blocks_for_tokens(tokens), 1]
        ids = pools.allocate(sum(cols), 0, SHAPE)
        it = iter(ids)
        groups = [[next(it) for _ in range(c)] for c in cols]
        t = BlockTable(0, SHAPE, GROUPS, groups)
        t.release_skipped_blocks(tokens)
        tables[rid] = t
        reqs.append((rid, tokens))
    return tables, reqs


@pytest.mark.parametrize("seed", range(5))
def test_plan_move_matches_reference_list_building(oracle, seed):
    rng = random.Random(seed)
    pools = BlockPools(cpu_num_slabs=64, cpu_slab_size_bytes=1 << 16)
    pools.register_gpu_space(0, 4096, SHAPE, GROUPS)
    tables, reqs = _tables(rng, 6, pools)
    before = copy.deepcopy(tables)
    reqs = reqs + [reqs[0]]  # duplicate request id is ignored
    plan = plan_move(reqs, tables, BLOCK_LOCATION_CPU, pools)
    per_table = []
    for rid, tokens in reqs[:-1]:
        t = before[rid]
        per_table.append((t.transfer_entries(tokens), [len(c) for c in t.group_blocks]))
    n_targets = sum(len(e) for e, _ in per_table)
    # the reserved targets are exactly what a fresh pool hands out in order
    fresh = BlockPools(cpu_num_slabs=64, cpu_slab_size_bytes=1 << 16)
    targets = fresh.allocate(n_targets, BLOCK_LOCATION_CPU, SHAPE)
    src, dst, grp, first, valid, new_tables = oracle.plan_lists(per_table, targets)
    assert plan.source_block_ids == src and plan.target_block_ids == dst
    assert plan.group_ids == grp and plan.first_kernel_blocks == first
    assert plan.valid_kernel_blocks == valid
    for (rid, _), want in zip(reqs[:-1], new_tables):
        assert tables[rid].group_blocks == want
        assert tables[rid].location == BLOCK_LOCATION_CPU
    assert sorted(plan.release_source_block_ids) == sorted(
        b for rid, _ in reqs[:-1] for b in before[rid].blocks)
    assert not plan.is_swap_in and plan.engine_id == 0
    # every source page copied once, every target distinct
    assert len(set(plan.target_block_ids)) == len(plan.target_block_ids)
    # moving back plans a swap-in with the same extents
    back = plan_move(reqs, tables, 0, pools)
    assert back.is_swap_in and back.valid_kernel_blocks == plan.valid_kernel_blocks
    assert back.source_block_ids == plan.target_block_ids
    pools.reclaim(plan)


def test_plan_move_rejections():
    pools = BlockPools(cpu_num_slabs=8, cpu_slab_size_bytes=1 << 16)
    pools.register_gpu_space(0, 64, SHAPE, GROUPS)
    pools.register_gpu_space(1, 64, SHAPE, GROUPS[:1])
    t0 = BlockTable(0, SHAPE, GROUPS, [[1], [2], [3]])
    t1 = BlockTable(BLOCK_LOCATION_CPU, SHAPE, GROUPS, [[4], [5], [6]])
    tables = {0: t0, 1: t1}
    with pytest.raises(NotImplementedError):
        plan_move([(0, 10)], tables, 1, pools)
    tables[2] = BlockTable(1, SHAPE, GROUPS[:1], [[9]])
    with pytest.raises(ValueError):
        plan_move([(0, 10), (2, 10)], tables, BLOCK_LOCATION_CPU, pools)  # mixed sources
    tables[3] = BlockTable(0, (999,), GROUPS, [[10], [11], [12]])
    with pytest.raises(ValueError):
        plan_move([(0, 10), (3, 10)], tables, BLOCK_LOCATION_CPU, pools)  # mixed shapes
    with pytest.raises(ValueError):
        plan_move([(1, 10)], tables, 1, pools)            # cache groups differ
    with pytest.raises(KeyError):
        plan_move([(7, 10)], tables, 0, pools)
    assert plan_move([(0, 10)], tables, 0, pools) is None  # already there
    small = BlockPools(cpu_num_slabs=1, cpu_slab_size_bytes=4000)
    small.register_gpu_space(0, 64, SHAPE, GROUPS)
    with pytest.raises(ResourceWarning):
        plan_move([(0, 10)], {0: BlockTable(0, SHAPE, GROUPS, [[1, 2], [3], [4]])},
                  BLOCK_LOCATION_CPU, small)


def test_zero_count_pages_get_destinations_only():
    """W = 1: the current page keeps a destination and no bytes move."""
    groups = (CacheGroupConfig("attention", 16, 16, sliding_window=1),)
    pools = BlockPools(cpu_num_slabs=4, cpu_slab_size_bytes=1 << 16)
    pools.register_gpu_space(0, 64, SHAPE, groups)
    tables = {0: BlockTable(0, SHAPE, groups, [[7, 8]])}
    plan = plan_move([(0, 20)], tables, BLOCK_LOCATION_CPU, pools)
    assert plan.source_block_ids == []
    assert tables[0].group_blocks[0][0] == LOGICAL_NULL_BLOCK_ID
    assert tables[0].group_blocks[0][1] >= 0
    assert sorted(plan.release_source_block_ids) == [7, 8]


@pytest.mark.parametrize("seed", range(6))
def test_native_transfer_entries_match_block_table(aegkv_lib, seed):
    """aegkv_transfer_entries (libaegkv, host-only) equals
    BlockTable.transfer_entries on random tables with windows, released
    columns and state pages."""
    from aegaeon_amd.planner import native_transfer_entries

    rng = random.Random(100 + seed)
    groups = (CacheGroupConfig("attention", rng.choice([16, 32, 64]), 16),
              CacheGroupConfig("attention", 48, 16, sliding_window=rng.randint(1, 90)),
              CacheGroupConfig("mamba_none", 4, 4),
              CacheGroupConfig("attention", 32, 8, sliding_window=rng.randint(1, 40)))
    tables = []
    next_id = 1
    for _ in range(rng.randint(1, 12)):
        tokens = rng.randint(0, 400)
        cols = []
        for g in groups:
            n = g.table_blocks_for_tokens(tokens)
            cols.append(list(range(next_id, next_id + n)))
            next_id += n
        t = BlockTable(0, SHAPE, groups, cols)
        if rng.random() < 0.5:
            t.release_skipped_blocks(tokens)
        tables.append((t, tokens))
    native = native_transfer_entries(groups, tables)
    for (t, tokens), rows in zip(tables, native):
        assert rows == t.transfer_entries(tokens)


def test_native_transfer_entries_rejections(aegkv_lib):
    from aegaeon_amd.planner import native_transfer_entries

    t = BlockTable(0, SHAPE, GROUPS, [[5, -7], [], [3]])
    with pytest.raises(ValueError):
        native_transfer_entries(GROUPS, [(t, 40)])     # id below the released marker
    t2 = BlockTable(0, SHAPE, GROUPS, [[5], [6]])
    with pytest.raises(ValueError):
        native_transfer_entries(GROUPS, [(t2, 10)])    # column lists per group missing
    assert native_transfer_entries(GROUPS, []) == []


# ------------------------------------------------------------ move ledger --

G1 = (CacheGroupConfig("attention", 16, 16),)


class FakeEvent:
    """A completion event the test finishes by hand."""

    def __init__(self):
        self.complete = False
        self.waited = 0

    def query(self):
        return self.complete

    def synchronize(self):
        self.waited += 1
        self.complete = True


def _engine_with_requests(n_req, per_req, num_max_blocks=12, **pool_kw):
    pools = BlockPools(**(pool_kw or dict(cpu_num_slabs=8, cpu_slab_size_bytes=1 << 16)))
    pools.register_gpu_space(0, num_max_blocks, SHAPE, G1)
    tables = {rid: BlockTable(0, SHAPE, G1, [pools.allocate(per_req, 0, SHAPE)])
              for rid in range(n_req)}
    return pools, tables


def test_move_ledger_reclaims_in_record_order():
    """Source ids return only when the move's event has completed, and in
    the order moves were recorded (block_manager.py:804-851)."""
    pools, tables = _engine_with_requests(2, 4)
    assert pools.gpu_free_blocks[0] == [9, 10, 11]
    p0 = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
    p1 = plan_move([(1, 64)], tables, BLOCK_LOCATION_CPU, pools)
    e0, e1 = FakeEvent(), FakeEvent()
    r0 = pools.record_move(p0, [e0])
    r1 = pools.record_move(p1, [e1])
    assert r0.serial < r1.serial
    assert pools.move_gpu_num_blocks[0] == 8
    e1.complete = True
    assert pools.reclaim_gpu_moves(0, wait=False) == (0, 0)   # e0 still running
    assert pools.gpu_free_blocks[0] == [9, 10, 11]
    e0.complete = True
    assert pools.reclaim_gpu_moves(0, wait=False) == (2, 8)
    assert pools.gpu_free_blocks[0] == [9, 10, 11, 1, 2, 3, 4, 5, 6, 7, 8]
    assert pools.move_gpu_num_blocks[0] == 0
    assert e0.waited == e1.waited == 0
    assert pools.reclaim_gpu_moves(0) == (0, 0)


def test_move_ledger_takes_fence_tokens():
    """A FenceToken with host fence words is a move event: the ledger frees
    the sources once the host word reaches the token's count, and a
    waiting reclaim returns once another thread publishes it (the
    controller's poll of block_manager.py:804-851, with host words in place
    of rebuilt IPC events)."""
    import threading
    import time

    from aegaeon_amd import ops
    from aegaeon_amd.swapper import FenceToken

    hw = ops.HostFenceWords(4)
    try:
        pools, tables = _engine_with_requests(2, 4)
        p0 = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
        p1 = plan_move([(1, 64)], tables, BLOCK_LOCATION_CPU, pools)
        pools.record_move(p0, [FenceToken(2, 3, hw.name)])
        pools.record_move(p1, [FenceToken(2, 4, hw.name), FenceToken(3, 1, hw.name)])
        hw.words[2] = 2
        assert pools.reclaim_gpu_moves(0, wait=False) == (0, 0)
        hw.words[2] = 4
        assert pools.reclaim_gpu_moves(0, wait=False) == (1, 4)   # p1 needs word 3 too
        threading.Timer(0.2, lambda: hw.words.__setitem__(3, 1)).start()
        t0 = time.perf_counter()
        assert pools.reclaim_gpu_moves(0, wait=True) == (1, 4)
        assert time.perf_counter() - t0 >= 0.15
        assert sorted(pools.gpu_free_blocks[0]) == list(range(1, 12))
        with pytest.raises(TimeoutError):
            FenceToken(0, 1, hw.name).synchronize(timeout_s=0.05)
        with pytest.raises(ValueError, match="no host fence words"):
            FenceToken(0, 1).query()
    finally:
        hw.close()


def test_gpu_allocation_waits_for_swap_outs():
    """A GPU allocation the free list cannot serve waits for the engine's
    swap-outs and takes back their sources (block_manager.py:956-970)."""
    pools, tables = _engine_with_requests(2, 4)
    p0 = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
    e0 = FakeEvent()
    pools.record_move(p0, [e0])
    assert pools.allocate(3, 0, SHAPE) == [9, 10, 11]       # no wait needed
    assert e0.waited == 0
    assert pools.allocate(2, 0, SHAPE) == [1, 2]            # waits on the swap-out
    assert e0.waited == 1
    with pytest.raises(ResourceWarning):
        pools.allocate(3, 0, SHAPE)


def test_finished_requests_end_their_move():
    pools, tables = _engine_with_requests(1, 4)
    p0 = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
    never = FakeEvent()
    pools.record_move(p0, [never], finished=lambda: True)
    assert pools.reclaim_gpu_moves(0, wait=False) == (1, 4)
    assert never.waited == 0


def test_swap_in_reclaim_frees_host_ids_and_empty_slabs():
    pools, tables = _engine_with_requests(1, 4)
    out = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
    pools.record_move(out, [FakeEvent()])
    used = [s for s, u in enumerate(pools.cpu_slab_usage) if u]
    assert len(used) == 1 and pools.cpu_slab_usage[used[0]] == 4
    back = plan_move([(0, 64)], tables, 0, pools)             # allocates 4 GPU ids
    e = FakeEvent()
    pools.record_move(back, [e])
    assert pools.move_cpu_num_blocks[SHAPE] == 4
    assert pools.reclaim_cpu_moves(SHAPE, wait=False) == (0, 0)
    e.complete = True
    assert pools.reclaim_cpu_moves(SHAPE, wait=False) == (1, 4)
    assert sum(pools.cpu_slab_usage) == 0
    assert sorted(pools.cpu_free_slabs) == list(range(8))
    assert len(pools.cpu_free_blocks[SHAPE]) == 0
    assert all(s is None for s in pools.cpu_block_shape)


def test_cpu_allocation_waits_for_swap_ins():
    """One slab of exactly four host blocks: a second swap-out must wait for
    the swap-in that still reads the first request's host pages."""
    pools, tables = _engine_with_requests(2, 4, num_max_blocks=16, cpu_num_slabs=1,
                                          cpu_slab_size_bytes=8000)
    out = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)
    pools.reclaim(out)
    back = plan_move([(0, 64)], tables, 0, pools)
    e = FakeEvent()
    pools.record_move(back, [e])
    out1 = plan_move([(1, 64)], tables, BLOCK_LOCATION_CPU, pools)
    assert e.waited == 1
    assert sorted(out1.target_block_ids) == [0, 1, 2, 3]


def test_reregistering_an_engine_settles_its_moves():
    pools, tables = _engine_with_requests(2, 4)
    with pytest.raises(ValueError, match="has blocks in it"):
        pools.register_gpu_space(0, 12, SHAPE, G1, block_tables=tables)
    out = plan_move([(0, 64), (1, 64)], tables, BLOCK_LOCATION_CPU, pools)
    pools.record_move(out, [FakeEvent()])
    back = plan_move([(0, 64)], tables, 0, pools)
    e = FakeEvent()
    pools.record_move(back, [e])
    with pytest.raises(ValueError):
        pools.register_gpu_space(0, 1, SHAPE, G1)     # rejected before any change
    assert pools.move_cpu_num_blocks[SHAPE] == 4
    again = plan_move([(0, 64)], tables, BLOCK_LOCATION_CPU, pools)   # switch away
    pools.record_move(again, [FakeEvent()])
    assert sum(pools.cpu_slab_usage) == 12
    pools.register_gpu_space(0, 20, SHAPE, G1, block_tables=tables)
    assert e.waited == 0                               # freed without waiting
    assert pools.move_cpu_num_blocks[SHAPE] == 0
    assert len(pools.move_events_gpu[0]) == 0 and pools.move_gpu_num_blocks[0] == 0
    assert pools.gpu_free_blocks[0] == list(range(1, 20))
    assert sum(pools.cpu_slab_usage) == 8              # both requests on the host


# ---------------------------------------------------------------- migration --

def test_plan_migrate_moves_flat_blocks_and_keeps_released_columns():
    from aegaeon_amd.planner import plan_migrate

    pools = BlockPools(cpu_num_slabs=4, cpu_slab_size_bytes=1 << 16)
    pools.register_gpu_space(0, 64, SHAPE, GROUPS)
    pools.register_gpu_space(1, 64, SHAPE, GROUPS)
    t0 = BlockTable(0, SHAPE, GROUPS, [pools.allocate(3, 0, SHAPE), pools.allocate(2, 0, SHAPE),
                                       pools.allocate(1, 0, SHAPE)])
    t0.group_blocks[1][0] = LOGICAL_NULL_BLOCK_ID          # a released window column
    t1 = BlockTable(0, SHAPE, GROUPS, [pools.allocate(2, 0, SHAPE), [], pools.allocate(1, 0, SHAPE)])
    tables = {0: t0, 1: t1}
    old = [list(t0.blocks), list(t1.blocks)]
    plan = plan_migrate([0, 1, 0], tables, 1, pools)
    assert plan.is_migration and not plan.is_swap_in and plan.engine_id == 1
    assert plan.source_block_ids == old[0] + old[1]
    assert len(plan.target_block_ids) == len(plan.source_block_ids) == 8
    assert plan.release_source_block_ids == plan.source_block_ids
    assert t0.location == t1.location == 1
    assert t0.group_blocks[1][0] == LOGICAL_NULL_BLOCK_ID
    assert t0.blocks + t1.blocks == plan.target_block_ids
    assert plan_migrate([0], tables, 1, pools) is None        # already there
    pools.record_move(plan, [])
    assert pools.move_gpu_num_blocks[0] == 8
    assert pools.reclaim_gpu_moves(0, wait=False) == (1, 8)


def test_plan_migrate_rejections():
    from aegaeon_amd.planner import plan_migrate

    pools = BlockPools(cpu_num_slabs=4, cpu_slab_size_bytes=1 << 16)
    pools.register_gpu_space(0, 64, SHAPE, GROUPS)
    pools.register_gpu_space(1, 64, SHAPE, GROUPS)
    pools.register_gpu_space(2, 64, SHAPE, GROUPS[:1])
    tables = {0: BlockTable(0, SHAPE, GROUPS, [[1], [2], [3]]),
              1: BlockTable(BLOCK_LOCATION_CPU, SHAPE, GROUPS, [[4], [5], [6]]),
              2: BlockTable(2, SHAPE, GROUPS[:1], [[7]])}
    with pytest.raises(ValueError, match="GPU engine"):
        plan_migrate([0], tables, BLOCK_LOCATION_CPU, pools)
    with pytest.raises(ValueError, match="host"):
        plan_migrate([1], tables, 1, pools)
    with pytest.raises(ValueError, match="cache groups"):
        plan_migrate([0], tables, 2, pools)
    with pytest.raises(ValueError, match="expected"):
        plan_migrate([0, 2], tables, 1, pools)
    with pytest.raises(KeyError):
        plan_migrate([9], tables, 1, pools)
