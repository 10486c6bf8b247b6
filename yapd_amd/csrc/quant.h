// Internal interface of the affine-quantised layer projections (gemm.hip)
// used by the step driver (step.cpp): the fused QKV + RoPE + KV write, the
// o / down projection with the residual add and gate/up + SiLU, on weights in
// the MLX layout (chatterbox_flash/engines/mlx.py:221-255, nn.quantize with
// group 64).  Each dequantises W into bf16 once on its way into LDS and then
// runs the bf16 kernel's MFMA loop and epilogue, so its output equals the bf16
// kernel's on the dequantised weights bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace yapd {

// Codes LSB-first in uint32 [N, K * bits / 32], fp16 scale and bias per 64
// inputs [N, K / 64]; bits 4 or 8.
struct QWeight {
  const uint32_t* packed;
  const uint16_t* scales;
  const uint16_t* biases;
  int bits;
};

// Argument checks of a quantised weight of N rows and K inputs (nothing launched).
int qweight_checks(const QWeight& w, int N, int K, const char* what);

// residual[M, N] = bf16(residual + bf16(A W^T)) (o_proj / down_proj).
int qgemm_residual(const void* A, int64_t lda, const QWeight& w, int M, int N, int K, void* residual, int64_t ld_res,
                   hipStream_t stream);

// act[M, F] = silu(A Wg^T) * (A Wu^T), W rows gate/up interleaved per 32.
int qgemm_swiglu(const void* A, int64_t lda, const QWeight& w_gate_up, int M, int F, int K, void* act,
                 int64_t ld_act, hipStream_t stream);

// yapd_gemm_qkv_rope_kv on a quantised W_qkv; with row_start and tok_row the
// rows are packed as in gemm_qkv_rope_kv_packed (rows = their count, bl unused).
int qgemm_qkv_rope_kv(const void* A, int64_t lda, const QWeight& w_qkv, int M, int K, int n_heads, const float* cos_t,
                      const float* sin_t, int max_pos, const int32_t* pos0, int bl, int rows, const int32_t* row_start,
                      const int32_t* tok_row, void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table,
                      int table_stride, int table_cols, hipStream_t stream);

// bf16(scale * q + bias) of n <= kMaxDqJobs weights (one bit width) into
// out[i] [N[i], K[i]] (row pitch K[i], 16-byte aligned), in one launch: the
// weights the fused kernels dequantise on their way into LDS, bit for bit.
constexpr int kMaxDqJobs = 4;
int dequant_affine(const QWeight* w, const int* N, const int* K, uint16_t* const* out, int n, hipStream_t stream);

}  // namespace yapd
