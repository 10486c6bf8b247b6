// Internal interface of the packed prefill chunk (step.cpp): the QKV GEMM
// whose rows are several sequences' tokens back to back (gemm.hip).  The
// attention half is attn_launch with q_start (attention.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace yapd {

// yapd_gemm_qkv_rope_kv over n_tokens packed rows: token m belongs to row
// tok_row[m] (of `rows`; device int32 [n_tokens]) at position
// pos0[row] + m - row_start[row] (row_start device int32 [rows + 1]).  q_out
// [n_tokens, H*64] keeps the packed order.
int gemm_qkv_rope_kv_packed(const void* A, int64_t lda, const void* W_qkv, int n_tokens, int K, int n_heads,
                            const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int rows,
                            const int32_t* row_start, const int32_t* tok_row, void* q_out, void* kv_pool,
                            int64_t n_pages, const int32_t* page_table, int table_stride, int table_cols,
                            hipStream_t stream);

}  // namespace yapd
