"""Extent math for partial KV-page transfers (host-side planning).

Same functions, argument meaning and ValueError behaviour as the
reference's aegaeon/cache_transfer.py:4-165. A physical page of
`physical_block_size` tokens is split into kernel blocks of
`kernel_block_size` tokens; a transfer moves the kernel blocks that hold
live tokens, which is always one contiguous run, expressed as a
(first kernel block, count) pair and then as a (byte offset, byte length)
pair inside one backing tensor's page.
"""

from __future__ import annotations


def _need_nonneg(name: str, value: int) -> None:
    if value < 0:
        raise ValueError(f"{name} = {value} is negative")


def _need_pos(name: str, value: int) -> None:
    if value <= 0:
        raise ValueError(f"{name} = {value} is not above zero")


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def logical_blocks_for_tokens(num_tokens: int, block_size: int) -> int:
    """Block-table columns that address positions [0, num_tokens)
    (cache_transfer.py:4-10)."""
    _need_nonneg("num_tokens", num_tokens)
    _need_pos("block_size", block_size)
    return _ceil_div(num_tokens, block_size)


def sliding_window_resident_block_bound(num_tokens: int, block_size: int,
                                        sliding_window: int) -> int:
    """Upper bound on pages a W-token window keeps resident
    (cache_transfer.py:13-28): the current page plus the pages holding the
    W-1 tokens before it, never more than the table has."""
    _need_pos("sliding_window", sliding_window)
    columns = logical_blocks_for_tokens(num_tokens, block_size)
    if columns == 0:
        return 0
    return min(columns, _ceil_div(sliding_window - 1, block_size) + 1)


def num_skipped_sliding_window_blocks(processed_computed_tokens: int, block_size: int,
                                      sliding_window: int) -> int:
    """Leading whole pages the next query's window cannot see
    (cache_transfer.py:31-45)."""
    _need_nonneg("processed_computed_tokens", processed_computed_tokens)
    _need_pos("block_size", block_size)
    _need_pos("sliding_window", sliding_window)
    invisible = max(0, processed_computed_tokens - (sliding_window - 1))
    return invisible // block_size


def kernel_block_extent_for_attention_page(
    cached_tokens: int,
    physical_block_index: int,
    physical_block_size: int,
    kernel_block_size: int,
    sliding_window: int | None = None,
) -> tuple[int, int]:
    """(first kernel block, count) of the live tokens inside one physical
    page (cache_transfer.py:48-94).

    Live tokens are [0, cached_tokens) for full attention and the last W-1
    of them, [cached_tokens - W + 1, cached_tokens), for a window W (the next
    query brings its own K/V). The page covers
    [index * physical, (index + 1) * physical). (0, 0) when they miss.
    """
    _need_nonneg("cached_tokens", cached_tokens)
    _need_nonneg("physical_block_index", physical_block_index)
    if physical_block_size <= 0 or kernel_block_size <= 0:
        raise ValueError(f"block sizes need to be > 0 (physical {physical_block_size}, "
                         f"kernel {kernel_block_size})")
    if physical_block_size % kernel_block_size:
        raise ValueError(
            f"a {physical_block_size}-token physical block does not hold a whole number of "
            f"{kernel_block_size}-token kernel blocks"
        )
    if sliding_window is not None:
        _need_pos("sliding_window", sliding_window)
    page_lo = physical_block_index * physical_block_size
    page_hi = page_lo + physical_block_size
    live_lo = 0 if sliding_window is None else max(0, cached_tokens - sliding_window + 1)
    lo = max(page_lo, live_lo) - page_lo
    hi = min(page_hi, cached_tokens) - page_lo
    if lo >= hi:
        return (0, 0)
    first = lo // kernel_block_size
    return first, _ceil_div(hi, kernel_block_size) - first


def valid_kernel_blocks_for_attention_page(cached_tokens: int, physical_block_index: int,
                                           physical_block_size: int,
                                           kernel_block_size: int) -> int:
    """Kernel blocks in a full-attention page's live prefix
    (cache_transfer.py:97-110)."""
    return kernel_block_extent_for_attention_page(
        cached_tokens, physical_block_index, physical_block_size, kernel_block_size
    )[1]


def prefix_bytes_for_kernel_blocks(page_size_bytes: int, kernel_blocks_per_page: int,
                                   valid_kernel_blocks: int) -> int:
    """Bytes of the first `valid_kernel_blocks` kernel blocks of a page
    (cache_transfer.py:113-135)."""
    _need_pos("page_size_bytes", page_size_bytes)
    _need_pos("kernel_blocks_per_page", kernel_blocks_per_page)
    if not 0 <= valid_kernel_blocks <= kernel_blocks_per_page:
        raise ValueError(
            f"{valid_kernel_blocks} live kernel blocks for a page of {kernel_blocks_per_page}"
        )
    if page_size_bytes % kernel_blocks_per_page:
        raise ValueError(
            f"a {page_size_bytes}-byte page does not split into {kernel_blocks_per_page} "
            f"equal kernel blocks"
        )
    return (page_size_bytes // kernel_blocks_per_page) * valid_kernel_blocks


def byte_extent_for_kernel_blocks(page_size_bytes: int, kernel_blocks_per_page: int,
                                  first_kernel_block: int,
                                  num_kernel_blocks: int) -> tuple[int, int]:
    """(byte offset, byte length) of kernel blocks
    [first, first + num) in one backing page (cache_transfer.py:138-165)."""
    _need_nonneg("first_kernel_block", first_kernel_block)
    last = first_kernel_block + num_kernel_blocks
    if last > kernel_blocks_per_page:
        raise ValueError(
            f"kernel blocks [{first_kernel_block}, {last}) run past a page of "
            f"{kernel_blocks_per_page}"
        )
    return (
        prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,
                                       first_kernel_block),
        prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,
                                       num_kernel_blocks),
    )
