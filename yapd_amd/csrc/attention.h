// Internal interface of the paged block attention (attention.hip): the
// argument checks and the launcher shared by the C entry points that differ
// only in where the split-KV partials live.
#pragma once

#include <cstdint>

namespace yapd {

// Checks shared by every attention entry point; YAPD_OK or YAPD_EINVAL (with the message set).
int attn_checks(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work, int n_work,
                void* out);

// Enqueues the attention kernel (and the split-KV merge when n_merge > 0) on `stream`.
// part_o [n_slots, bl, H, 64] and part_ml [n_slots, bl, H, 2] are fp32 device memory
// (NULL with n_slots = 0 when no item is split).
int attn_launch(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work, int n_work,
                const int32_t* merge, int n_merge, const int32_t* counts, float* part_o, float* part_ml, int n_slots,
                float scale, int causal, void* out, void* stream);

}  // namespace yapd
