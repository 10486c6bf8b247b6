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
// (NULL with n_slots = 0 when no item is split).  With q_start (device int32
// [rows + 1]) the queries are packed: row r's are rows [q_start[r], q_start[r+1])
// of q and out (n_q rows in all, at most bl per row; causal masking counts
// from the row's own query count); NULL means rows r*bl .. r*bl + bl - 1.
int attn_launch(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work, int n_work,
                const int32_t* merge, int n_merge, const int32_t* counts, float* part_o, float* part_ml, int n_slots,
                float scale, int causal, void* out, void* stream, const int32_t* q_start = nullptr, int n_q = 0);

}  // namespace yapd
