"""Cache-group contracts and per-request block tables (swap planning).

Host-side mirror of the reference's block_manager types on the swap path:
CacheGroupConfig (aegaeon/block_manager.py:133-267), CacheGroupRuntimeConfig
(:269-383) and BlockTable (:385-516), re-exported by the reference as
aegaeon/cache_groups.py:9-23. Names, argument meaning and ValueError
behaviour follow the reference; the implementation is this package's own.

A request's table holds, per cache group, one physical block id per logical
column; released sliding-window columns hold LOGICAL_NULL_BLOCK_ID.
`transfer_entries` turns a table into the (group, column, id, first, count)
rows a swap moves.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

from .cache_transfer import (
    byte_extent_for_kernel_blocks,
    kernel_block_extent_for_attention_page,
    logical_blocks_for_tokens,
    num_skipped_sliding_window_blocks,
    sliding_window_resident_block_bound,
)

#: vLLM reserves device block 0 as its null block (block_manager.py:117-120)
VLLM_NULL_BLOCK_ID = 0
#: control-plane sentinel for a released logical column (block_manager.py:122-126)
LOGICAL_NULL_BLOCK_ID = -1
#: location of host-resident blocks (block_manager.py:112-115)
BLOCK_LOCATION_CPU = -1

_KINDS = ("attention", "mamba_none")


def is_gpu(location: int) -> bool:
    return location >= 0


def _check_group(kind: str, block: int, kernel: int, window: Optional[int],
                 block_name: str) -> None:
    if block <= 0 or kernel <= 0:
        raise ValueError(
            f"{block_name} block of {block} tokens and kernel block of {kernel}: both "
            "need to be above zero"
        )
    if kind == "attention":
        if block % kernel:
            raise ValueError(
                f"an attention {block_name} block of {block} tokens does not hold whole "
                f"{kernel}-token kernel blocks"
            )
    elif kind == "mamba_none":
        if block != kernel:
            raise ValueError("a state-page (mamba_none) group keeps one kernel block per page")
        if window is not None:
            raise ValueError("a state-page (mamba_none) group takes no sliding window")
    else:
        raise NotImplementedError(f"cache group kind {kind!r} is not one this planner knows")
    if window is not None and window <= 0:
        raise ValueError(f"a sliding window of {window} tokens is not above zero")


@dataclass
class CacheGroupConfig:
    """Scheduler-side policy of one cache group (block_manager.py:133-267).

    block_size is the physical (KV-manager) page in tokens; kernel_block_size
    the attention kernel's page; a "mamba_none" group keeps one state page.
    """

    kind: str
    block_size: int
    kernel_block_size: int
    sliding_window: Optional[int] = None

    def __post_init__(self) -> None:
        _check_group(self.kind, self.block_size, self.kernel_block_size,
                     self.sliding_window, "physical")

    def table_blocks_for_tokens(self, num_tokens: int) -> int:
        if num_tokens < 0:
            raise ValueError(f"{num_tokens} tokens is negative")
        if self.kind == "attention":
            return logical_blocks_for_tokens(num_tokens, self.block_size)
        return 1

    def blocks_for_tokens(self, num_tokens: int) -> int:
        """Resident-page bound used for admission (block_manager.py:173-194)."""
        if num_tokens < 0:
            raise ValueError(f"{num_tokens} tokens is negative")
        if self.kind == "mamba_none":
            return 1
        if self.sliding_window is None:
            return self.table_blocks_for_tokens(num_tokens)
        return sliding_window_resident_block_bound(num_tokens, self.block_size,
                                                   self.sliding_window)

    def num_skipped_blocks(self, processed_computed_tokens: int) -> int:
        if processed_computed_tokens < 0:
            raise ValueError(f"{processed_computed_tokens} processed tokens is negative")
        if self.kind != "attention" or self.sliding_window is None:
            return 0
        return num_skipped_sliding_window_blocks(processed_computed_tokens, self.block_size,
                                                 self.sliding_window)

    def block_is_skipped(self, processed_computed_tokens: int, logical_block_index: int) -> bool:
        if logical_block_index < 0:
            raise ValueError(f"logical block {logical_block_index} is negative")
        return logical_block_index < self.num_skipped_blocks(processed_computed_tokens)

    @property
    def kernel_blocks_per_physical_block(self) -> int:
        return self.block_size // self.kernel_block_size

    def kernel_block_extent(self, cached_tokens: int, block_index: int) -> Tuple[int, int]:
        """(first kernel block, live count) of one page (block_manager.py:254-266)."""
        if self.kind == "mamba_none":
            return (0, 1)
        return kernel_block_extent_for_attention_page(
            cached_tokens, block_index, self.block_size, self.kernel_block_size,
            self.sliding_window,
        )

    def valid_kernel_blocks(self, cached_tokens: int, block_index: int) -> int:
        if cached_tokens < 0:
            raise ValueError(f"{cached_tokens} cached tokens is negative")
        if block_index < 0:
            raise ValueError(f"block {block_index} is negative")
        if self.kind == "mamba_none":
            return 1
        return self.kernel_block_extent(cached_tokens, block_index)[1]


@dataclass(frozen=True)
class CacheGroupRuntimeConfig:
    """Worker-side block-size contract of one group (block_manager.py:269-383)."""

    kind: str
    kv_block_size: int
    kernel_block_size: int
    sliding_window: Optional[int] = None

    def __post_init__(self) -> None:
        _check_group(self.kind, self.kv_block_size, self.kernel_block_size,
                     self.sliding_window, "KV-manager")

    @property
    def blocks_per_kv_block(self) -> int:
        return self.kv_block_size // self.kernel_block_size

    def byte_extent_for_kernel_blocks(self, page_size_bytes: int, first_kernel_block: int,
                                      num_kernel_blocks: int) -> Tuple[int, int]:
        return byte_extent_for_kernel_blocks(page_size_bytes, self.blocks_per_kv_block,
                                             first_kernel_block, num_kernel_blocks)

    def bytes_for_kernel_blocks(self, page_size_bytes: int, valid_kernel_blocks: int) -> int:
        return self.byte_extent_for_kernel_blocks(page_size_bytes, 0, valid_kernel_blocks)[1]

    def to_kernel_block_ids(self, kv_block_ids: Sequence[int]) -> List[int]:
        """Physical ids -> attention-kernel ids; released columns map to the
        null block (block_manager.py:339-355). With 272-token physical and
        16-token kernel blocks, physical id 3 -> kernel ids 51..67."""
        if self.kind != "attention":
            return list(kv_block_ids)
        r = self.blocks_per_kv_block
        out: List[int] = []
        for pid in kv_block_ids:
            out.extend([VLLM_NULL_BLOCK_ID] * r if pid < 0 else range(pid * r, pid * r + r))
        return out

    def slot_for_position(self, kv_block_ids: Sequence[int], position: int) -> int:
        """Token position -> slot in the kernel-shaped cache (block_manager.py:357-382)."""
        if self.kind != "attention":
            raise ValueError(f"a {self.kind} group maps no token positions to slots")
        if position < 0:
            raise ValueError(f"token position {position} is negative")
        column, inside = divmod(position, self.kv_block_size)
        if column >= len(kv_block_ids):
            raise IndexError(
                f"token {position} falls in column {column} of a "
                f"{len(kv_block_ids)}-column table"
            )
        pid = kv_block_ids[column]
        if pid < 0:
            raise RuntimeError(
                f"token {position} falls in column {column}, which was released"
            )
        kernel_id = pid * self.blocks_per_kv_block + inside // self.kernel_block_size
        return kernel_id * self.kernel_block_size + inside % self.kernel_block_size


@dataclass
class BlockTable:
    """Per-request block ids by cache group (block_manager.py:385-516)."""

    location: int
    block_shape: Tuple[int, ...]
    cache_groups: Tuple[CacheGroupConfig, ...]
    group_blocks: List[List[int]]

    @property
    def blocks(self) -> List[int]:
        """All live physical ids, group-major (released columns dropped)."""
        return [b for col in self.group_blocks for b in col if b != LOGICAL_NULL_BLOCK_ID]

    def replace_flat_blocks(self, blocks: List[int]) -> None:
        live = sum(b != LOGICAL_NULL_BLOCK_ID for col in self.group_blocks for b in col)
        if len(blocks) != live:
            raise ValueError(f"{len(blocks)} ids for a table with {live} live columns")
        it = iter(blocks)
        self.group_blocks = [
            [b if b == LOGICAL_NULL_BLOCK_ID else next(it) for b in col]
            for col in self.group_blocks
        ]

    def release_skipped_blocks(self, processed_computed_tokens: int) -> List[int]:
        """Null out and return pages wholly before each group's window."""
        released: List[int] = []
        for group, col in zip(self.cache_groups, self.group_blocks):
            n = min(group.num_skipped_blocks(processed_computed_tokens), len(col))
            for i in range(n):
                if col[i] != LOGICAL_NULL_BLOCK_ID:
                    released.append(col[i])
                    col[i] = LOGICAL_NULL_BLOCK_ID
        return released

    def transfer_entries(self, processed_computed_tokens: int
                         ) -> List[Tuple[int, int, int, int, int]]:
        """Retained pages as (group, column, id, first, count)
        (block_manager.py:446-478). count may be 0 for a retained page with no
        cached bytes; such a page still needs a destination id."""
        rows: List[Tuple[int, int, int, int, int]] = []
        for g, (group, col) in enumerate(zip(self.cache_groups, self.group_blocks)):
            skipped = group.num_skipped_blocks(processed_computed_tokens)
            for i, pid in enumerate(col):
                if pid == LOGICAL_NULL_BLOCK_ID or i < skipped:
                    continue
                first, count = group.kernel_block_extent(processed_computed_tokens, i)
                rows.append((g, i, pid, first, count))
        return rows

    def moved_group_blocks(self, processed_computed_tokens: int,
                           target_block_ids: Sequence[int]) -> List[List[int]]:
        """Destination table for a compact list of new ids (block_manager.py:480-495)."""
        rows = self.transfer_entries(processed_computed_tokens)
        if len(rows) != len(target_block_ids):
            raise ValueError(
                f"{len(target_block_ids)} target ids for {len(rows)} retained pages"
            )
        moved = [[LOGICAL_NULL_BLOCK_ID] * len(col) for col in self.group_blocks]
        for (g, i, _, _, _), tid in zip(rows, target_block_ids):
            moved[g][i] = tid
        return moved

    def swap_metadata(self, cached_tokens: int) -> Tuple[List[int], List[int], List[int]]:
        """(groups, firsts, counts) of the non-empty extents (block_manager.py:497-515)."""
        rows = [r for r in self.transfer_entries(cached_tokens) if r[4] > 0]
        return [r[0] for r in rows], [r[3] for r in rows], [r[4] for r in rows]
