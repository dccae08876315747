// Native swap planning: the transfer entries of many block tables at once.
//
// Host-only C++ (no device code). Follows, per column, the rules of
// BlockTable.transfer_entries (aegaeon/block_manager.py:446-478) over
// CacheGroupConfig.num_skipped_blocks / kernel_block_extent (:196-266) and
// cache_transfer.kernel_block_extent_for_attention_page (cache_transfer.py:
// 48-94). Contract in include/aegkv.h.

#include "aegkv.h"
#include "errors.h"

#define plan_fail aegkv_set_error

namespace {

constexpr int kAttention = 0;
constexpr int kMambaNone = 1;
constexpr int64_t kReleased = -1;  // LOGICAL_NULL_BLOCK_ID

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

extern "C" {

int aegkv_transfer_entries(int32_t num_groups, const int32_t* group_kind,
                           const int64_t* group_block_size,
                           const int64_t* group_kernel_block_size,
                           const int64_t* group_sliding_window, int64_t num_tables,
                           const int64_t* processed_tokens, const int64_t* column_offsets,
                           const int64_t* column_ids, int64_t max_rows, int64_t* out_table,
                           int32_t* out_group, int64_t* out_column, int64_t* out_block,
                           int64_t* out_first, int64_t* out_count, int64_t* num_rows) {
  aegkv_clear_error();
  if (!num_rows) return plan_fail(AEGKV_EINVAL, "num_rows must not be null");
  *num_rows = 0;
  if (num_groups <= 0 || num_tables < 0)
    return plan_fail(AEGKV_EINVAL, "need at least one group and a non-negative table count");
  if (!group_kind || !group_block_size || !group_kernel_block_size || !group_sliding_window)
    return plan_fail(AEGKV_EINVAL, "group arrays must not be null");
  if (num_tables > 0 && (!processed_tokens || !column_offsets || !column_ids))
    return plan_fail(AEGKV_EINVAL, "table arrays must not be null");
  // CacheGroupConfig.__post_init__ (block_manager.py:147-171)
  for (int32_t g = 0; g < num_groups; ++g) {
    const int64_t bs = group_block_size[g], kbs = group_kernel_block_size[g];
    const int64_t w = group_sliding_window[g];
    if (bs <= 0 || kbs <= 0)
      return plan_fail(AEGKV_EINVAL, "group %d: cache block sizes must both be positive", g);
    if (group_kind[g] == kAttention) {
      if (bs % kbs)
        return plan_fail(AEGKV_EINVAL, "group %d: kernel block size %lld must divide %lld", g,
                         static_cast<long long>(kbs), static_cast<long long>(bs));
    } else if (group_kind[g] == kMambaNone) {
      if (bs != kbs)
        return plan_fail(AEGKV_EINVAL, "group %d: state pages cannot be split", g);
      if (w > 0) return plan_fail(AEGKV_EINVAL, "group %d: state pages have no window", g);
    } else {
      return plan_fail(AEGKV_EINVAL, "group %d: unsupported kind %d", g, group_kind[g]);
    }
  }
  int64_t rows = 0;
  for (int64_t t = 0; t < num_tables; ++t) {
    const int64_t tokens = processed_tokens[t];
    if (tokens < 0) return plan_fail(AEGKV_EINVAL, "table %lld: negative token count",
                                     static_cast<long long>(t));
    for (int32_t g = 0; g < num_groups; ++g) {
      const int64_t lo = column_offsets[t * num_groups + g];
      const int64_t hi = column_offsets[t * num_groups + g + 1];
      if (lo < 0 || hi < lo)
        return plan_fail(AEGKV_EINVAL, "table %lld group %d: bad column offsets",
                         static_cast<long long>(t), g);
      const bool attention = group_kind[g] == kAttention;
      const int64_t bs = group_block_size[g], kbs = group_kernel_block_size[g];
      const int64_t w = group_sliding_window[g];
      const bool windowed = attention && w > 0;
      // num_skipped_sliding_window_blocks (cache_transfer.py:31-45)
      int64_t skipped = 0;
      int64_t live_lo = 0;
      if (windowed) {
        live_lo = tokens - w + 1 > 0 ? tokens - w + 1 : 0;
        skipped = live_lo / bs;
      }
      for (int64_t c = lo; c < hi; ++c) {
        const int64_t col = c - lo;
        const int64_t id = column_ids[c];
        if (id == kReleased || col < skipped) continue;
        if (id < 0)
          return plan_fail(AEGKV_EINVAL, "table %lld group %d column %lld: block id %lld",
                           static_cast<long long>(t), g, static_cast<long long>(col),
                           static_cast<long long>(id));
        int64_t first = 0, count = 1;
        if (attention) {
          // kernel_block_extent_for_attention_page (cache_transfer.py:77-94)
          const int64_t page_lo = col * bs, page_hi = page_lo + bs;
          const int64_t ext_lo = page_lo > live_lo ? page_lo : live_lo;
          const int64_t ext_hi = page_hi < tokens ? page_hi : tokens;
          if (ext_lo >= ext_hi) {
            first = 0;
            count = 0;
          } else {
            first = (ext_lo - page_lo) / kbs;
            count = ceil_div(ext_hi - page_lo, kbs) - first;
          }
        }
        if (rows >= max_rows)
          return plan_fail(AEGKV_ENOMEM, "more than %lld transfer entries",
                           static_cast<long long>(max_rows));
        if (out_table) out_table[rows] = t;
        if (out_group) out_group[rows] = g;
        if (out_column) out_column[rows] = col;
        if (out_block) out_block[rows] = id;
        if (out_first) out_first[rows] = first;
        if (out_count) out_count[rows] = count;
        ++rows;
      }
    }
  }
  *num_rows = rows;
  return 0;
}

}  // extern "C"
