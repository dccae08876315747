/*
 * aegkv_oracle.c - CPU restatement of the reference's KV movement path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the reference restatement the tests,
 * the smoke run and the benchmark's CPU-baseline leg compare libaegkv against. The
 * product (aegaeon_amd/, libaegkv.so) never links, loads or calls it.
 *
 * Every function restates one piece of pkusys/Aegaeon, cited by file:line,
 * as a plain sequential loop over host memory in the reference's own
 * iteration order. Return values: 0 ok, -1 for the inputs the reference
 * rejects with ValueError (cache_transfer.py), -2 for a byte range outside
 * a buffer (the reference would read/write out of bounds there).
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   oracle_swap_legacy      golden vectors from torch index_select/index_copy
 *                           + byte-provenance labels
 *   oracle_swap_blocks      golden vectors + inverse-map provenance check
 *                           (every host byte traced back to (segment, block,
 *                           offset) by searching the layout, not by the loop)
 *   oracle_copy_blocks      golden vectors from torch index ops + provenance
 *   oracle_kernel_block_extent / oracle_byte_extent / helpers
 *                           brute force over token positions, the reference's
 *                           docstring known answers, and the reference
 *                           benchmark's extent plans
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_OK 0
#define ORACLE_EVALUE (-1)
#define ORACLE_ERANGE (-2)

/* ---------------------------------------------------- cache_transfer.py -- */

/* aegaeon/cache_transfer.py:4-10 */
int oracle_logical_blocks_for_tokens(int64_t num_tokens, int64_t block_size, int64_t* out) {
  if (num_tokens < 0 || block_size <= 0) return ORACLE_EVALUE;
  *out = (num_tokens + block_size - 1) / block_size;
  return ORACLE_OK;
}

/* aegaeon/cache_transfer.py:13-28 */
int oracle_sliding_window_resident_block_bound(int64_t num_tokens, int64_t block_size,
                                               int64_t sliding_window, int64_t* out) {
  int64_t logical, max_resident;
  if (sliding_window <= 0) return ORACLE_EVALUE;
  if (oracle_logical_blocks_for_tokens(num_tokens, block_size, &logical)) return ORACLE_EVALUE;
  if (logical == 0) {
    *out = 0;
    return ORACLE_OK;
  }
  max_resident = (sliding_window - 1 + block_size - 1) / block_size + 1;
  *out = logical < max_resident ? logical : max_resident;
  return ORACLE_OK;
}

/* aegaeon/cache_transfer.py:31-45 */
int oracle_num_skipped_sliding_window_blocks(int64_t processed_computed_tokens,
                                             int64_t block_size, int64_t sliding_window,
                                             int64_t* out) {
  int64_t skipped;
  if (processed_computed_tokens < 0 || block_size <= 0 || sliding_window <= 0)
    return ORACLE_EVALUE;
  skipped = processed_computed_tokens - sliding_window + 1;
  if (skipped < 0) skipped = 0;
  *out = skipped / block_size;
  return ORACLE_OK;
}

/* aegaeon/cache_transfer.py:48-94. sliding_window <= 0 encodes None; the
 * reference rejects an explicit non-positive window, which callers of this
 * function express by passing has_window = 1 with sliding_window <= 0. */
int oracle_kernel_block_extent(int64_t cached_tokens, int64_t physical_block_index,
                               int64_t physical_block_size, int64_t kernel_block_size,
                               int has_window, int64_t sliding_window, int64_t* first,
                               int64_t* count) {
  int64_t block_start, block_end, live_start, ext_start, ext_end, rel_start, rel_end, end_kb;
  if (cached_tokens < 0 || physical_block_index < 0) return ORACLE_EVALUE;
  if (physical_block_size <= 0 || kernel_block_size <= 0) return ORACLE_EVALUE;
  if (physical_block_size % kernel_block_size) return ORACLE_EVALUE;
  if (has_window && sliding_window <= 0) return ORACLE_EVALUE;
  block_start = physical_block_index * physical_block_size;
  block_end = block_start + physical_block_size;
  live_start = 0;
  if (has_window) {
    live_start = cached_tokens - sliding_window + 1;
    if (live_start < 0) live_start = 0;
  }
  ext_start = block_start > live_start ? block_start : live_start;
  ext_end = block_end < cached_tokens ? block_end : cached_tokens;
  if (ext_start >= ext_end) {
    *first = 0;
    *count = 0;
    return ORACLE_OK;
  }
  rel_start = ext_start - block_start;
  rel_end = ext_end - block_start;
  *first = rel_start / kernel_block_size;
  end_kb = (rel_end + kernel_block_size - 1) / kernel_block_size;
  *count = end_kb - *first;
  return ORACLE_OK;
}

/* aegaeon/cache_transfer.py:113-135 */
int oracle_prefix_bytes_for_kernel_blocks(int64_t page_size_bytes, int64_t kernel_blocks_per_page,
                                          int64_t valid_kernel_blocks, int64_t* out) {
  if (page_size_bytes <= 0 || kernel_blocks_per_page <= 0) return ORACLE_EVALUE;
  if (valid_kernel_blocks < 0 || valid_kernel_blocks > kernel_blocks_per_page)
    return ORACLE_EVALUE;
  if (page_size_bytes % kernel_blocks_per_page) return ORACLE_EVALUE;
  *out = page_size_bytes / kernel_blocks_per_page * valid_kernel_blocks;
  return ORACLE_OK;
}

/* aegaeon/cache_transfer.py:138-165 */
int oracle_byte_extent(int64_t page_size_bytes, int64_t kernel_blocks_per_page,
                       int64_t first_kernel_block, int64_t num_kernel_blocks, int64_t* offset,
                       int64_t* length) {
  if (first_kernel_block < 0) return ORACLE_EVALUE;
  if (first_kernel_block + num_kernel_blocks > kernel_blocks_per_page) return ORACLE_EVALUE;
  if (oracle_prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,
                                            first_kernel_block, offset))
    return ORACLE_EVALUE;
  if (oracle_prefix_bytes_for_kernel_blocks(page_size_bytes, kernel_blocks_per_page,
                                            num_kernel_blocks, length))
    return ORACLE_EVALUE;
  return ORACLE_OK;
}

/* ------------------------------------------------------------ ops/swap.cu -- */

/* ops/swap.cu:25-60. The block size is derived exactly as swap.cu:34 does,
 * numel * 2 / size(0) (the reference assumes 2-byte elements), and the same
 * stride is used for both buffers. Ids are not checked by the reference;
 * here an out-of-range id returns ORACLE_ERANGE before anything is copied. */
int oracle_swap_legacy(const int64_t* source_block_ids, const int64_t* target_block_ids,
                       int64_t num_ids, int is_swap_in, uint8_t* kv_cache,
                       int64_t cache_numel, int64_t cache_size0, int64_t cache_bytes,
                       uint8_t* kv_swap, int64_t swap_bytes) {
  int64_t i, b;
  if (cache_size0 <= 0) return ORACLE_EVALUE;
  b = cache_numel * 2 / cache_size0;
  for (i = 0; i < num_ids; ++i) {
    const int64_t s = source_block_ids[i], t = target_block_ids[i];
    const int64_t dev_id = is_swap_in ? t : s, host_id = is_swap_in ? s : t;
    if (dev_id < 0 || (dev_id + 1) * b > cache_bytes) return ORACLE_ERANGE;
    if (host_id < 0 || (host_id + 1) * b > swap_bytes) return ORACLE_ERANGE;
  }
  for (i = 0; i < num_ids; ++i) {
    const int64_t s = source_block_ids[i], t = target_block_ids[i];
    if (is_swap_in)
      memcpy(kv_cache + t * b, kv_swap + s * b, (size_t)b); /* swap.cu:40-48 */
    else
      memcpy(kv_swap + t * b, kv_cache + s * b, (size_t)b); /* swap.cu:49-57 */
  }
  return ORACLE_OK;
}

/* ---------------------------------------------- Worker.swap_blocks loop -- */

/* aegaeon/worker.py:2265-2329 (hot loop of Worker.swap_blocks).
 *   segments in composite order (worker.py:2272), entries inner (:2279-2291);
 *   skip when the entry's group does not own the segment (:2292-2293);
 *   (off, len) = byte_extent_for_kernel_blocks (:2294-2299, via
 *     block_manager.py:326-337 -> cache_transfer.py:138-165);
 *   skip len == 0 (:2300-2301);
 *   host offset = tp_rank * composite_page + cpu_offset + off (:2304-2309);
 *   swap-in  gpu[target][off:+len] <- host[source][hoff:+len] (:2310-2318);
 *   swap-out host[target][hoff:+len] <- gpu[source][off:+len] (:2319-2328).
 * segments[s] points at backing tensor s, viewed as [num_gpu_blocks, page]
 * (worker.py:2273-2277); host is [host_num_blocks, host_page_bytes] with
 * host_page_bytes = composite_page * tp_size (worker.py:1419-1432).
 * copied_bytes / copy_operations are the two counters the reference logs
 * (worker.py:2302-2303, 2338-2348). */
int oracle_swap_blocks(int32_t num_segments, uint8_t* const* segments,
                       const int64_t* segment_page_bytes, const int64_t* segment_cpu_offsets,
                       const uint64_t* segment_owner_masks, int64_t num_gpu_blocks,
                       const int64_t* group_kernel_blocks_per_page, int32_t num_groups,
                       uint8_t* host, int64_t host_num_blocks, int64_t host_page_bytes,
                       int64_t tp_rank, int64_t composite_page_bytes, int64_t num_entries,
                       const int64_t* source_block_ids, const int64_t* target_block_ids,
                       const int32_t* group_ids, const int64_t* first_kernel_blocks,
                       const int64_t* valid_kernel_blocks, int is_swap_in,
                       int64_t* copied_bytes, int64_t* copy_operations) {
  int32_t s;
  int64_t i;
  *copied_bytes = 0;
  *copy_operations = 0;
  for (i = 0; i < num_entries; ++i) /* worker.py:2241-2246 */
    if (group_ids[i] < 0 || group_ids[i] >= num_groups) return ORACLE_EVALUE;
  for (s = 0; s < num_segments; ++s) {
    const int64_t page = segment_page_bytes[s];
    for (i = 0; i < num_entries; ++i) {
      const int32_t g = group_ids[i];
      int64_t off, len, hoff, dev_id, host_id;
      if (!((segment_owner_masks[s] >> g) & 1u)) continue;
      if (oracle_byte_extent(page, group_kernel_blocks_per_page[g], first_kernel_blocks[i],
                             valid_kernel_blocks[i], &off, &len))
        return ORACLE_EVALUE;
      if (len == 0) continue;
      *copied_bytes += len;
      *copy_operations += 1;
      hoff = tp_rank * composite_page_bytes + segment_cpu_offsets[s] + off;
      dev_id = is_swap_in ? target_block_ids[i] : source_block_ids[i];
      host_id = is_swap_in ? source_block_ids[i] : target_block_ids[i];
      if (dev_id < 0 || dev_id >= num_gpu_blocks) return ORACLE_ERANGE;
      if (host_id < 0 || host_id >= host_num_blocks) return ORACLE_ERANGE;
      if (hoff < 0 || hoff + len > host_page_bytes) return ORACLE_ERANGE;
      if (is_swap_in)
        memcpy(segments[s] + dev_id * page + off, host + host_id * host_page_bytes + hoff,
               (size_t)len);
      else
        memcpy(host + host_id * host_page_bytes + hoff, segments[s] + dev_id * page + off,
               (size_t)len);
    }
  }
  return ORACLE_OK;
}

/* -------------------------------------------------------------- copy_blocks -- */

/* In-HBM block copy. The reference has no KV copy_blocks
 * (aegaeon/block_manager.py:1392-1393 raises for GPU->GPU moves); its
 * in-HBM compactions copy tensor by tensor with copy_ in a fixed order
 * (aegaeon/allocator.py:101-137). This restates the closed form the build
 * defines: for each pair in order, for each segment, seg[dst] := seg[src],
 * one whole block of page bytes. Applied sequentially, so with overlapping
 * pairs the result is the in-order one; the product rejects overlaps. */
int oracle_copy_blocks(int32_t num_segments, uint8_t* const* segments,
                       const int64_t* segment_page_bytes, int64_t num_blocks, int64_t num_pairs,
                       const int64_t* src_block_ids, const int64_t* dst_block_ids) {
  int64_t i;
  int32_t s;
  for (i = 0; i < num_pairs; ++i)
    if (src_block_ids[i] < 0 || src_block_ids[i] >= num_blocks || dst_block_ids[i] < 0 ||
        dst_block_ids[i] >= num_blocks)
      return ORACLE_ERANGE;
  for (i = 0; i < num_pairs; ++i)
    for (s = 0; s < num_segments; ++s) {
      const int64_t page = segment_page_bytes[s];
      memmove(segments[s] + dst_block_ids[i] * page, segments[s] + src_block_ids[i] * page,
              (size_t)page);
    }
  return ORACLE_OK;
}
