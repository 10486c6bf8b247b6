// (b) bf16 MFMA GEMMs of the T3 layer with fused epilogues, plus the
// (residual-add +) RMSNorm row kernels.
//
// C[M, N] = A[M, K] * W[N, K]^T (nn.Linear layout), fp32 accumulation on
// v_mfma_f32_32x32x16_bf16.  A 256-thread workgroup owns a 128 x 128 tile as
// 2 x 2 waves of 64 x 64 (2 x 2 MFMA tiles each); K advances in steps of 64
// through double-buffered LDS (rows padded by 16 bytes so the 16-byte
// fragment reads of 8 consecutive lanes hit distinct banks); the next K step
// is fetched into registers while the current one is multiplied.
//
// Epilogues (once per output element, so their VALU cost is small):
//   * store   -- plain bf16 store (o_proj / down / speech head);
//   * qkv     -- NeoX RoPE on q and k from a cos/sin table at each row's
//                absolute position, q to its buffer, k and v straight into
//                the paged KV pool (engines/flashinfer.py:998-1035);
//   * swiglu  -- silu(gate) * up from interleaved gate/up weight rows
//                (engines/flashinfer.py:433-455).
// The bf16 roundings of the reference's separate ops are reproduced (HF
// computes q*cos, rotate_half(q)*sin and their sum in bf16; silu(g) and the
// product in bf16), so the fused results differ from it only through the
// fp32 accumulation order.
//
// A prologue mode "shift" reads A row (r, j) from hidden row (r, j-1) and
// row (r, 0) from shift_ctx[r]: the token-shifted speech head
// (engines/flashinfer.py:1452-1461).
#include "common.h"
#include "kv_layout.h"

namespace yapd {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kLdsPitch = BK + 8;  // bf16 elements per LDS row
constexpr int kThreadsG = 256;

enum EpiMode { kEpiStore = 0, kEpiQkv = 1, kEpiSwiglu = 2 };
enum AMode { kAPlain = 0, kAShift = 1 };

struct GemmParams {
  const uint16_t* A;
  int64_t lda;
  const uint16_t* shift_ctx;  // [M / bl, K] (kAShift)
  int shift_bl;
  const uint16_t* W;
  int64_t ldw;
  int M, N, K;
  uint16_t* C;
  int64_t ldc;
  // qkv epilogue
  const float* cos_t;  // [max_pos, 64] fp32 (values of the model-dtype table)
  const float* sin_t;
  int max_pos;
  const int32_t* pos0;  // [M / bl] first position of each row's block
  int bl;
  int n_heads;
  uint16_t* q_out;  // [M, n_heads * 64]
  uint16_t* pool;   // [n_pages, 2, n_heads, 1024]
  int64_t n_pages;
  const int32_t* table;
  int table_stride, table_cols;
};

__device__ __forceinline__ u32x4_t ldg16(const uint16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }

template <int AM>
__device__ __forceinline__ const uint16_t* a_row_ptr(const GemmParams& p, int m) {
  if (AM == kAShift) {
    const int r = m / p.shift_bl;
    const int j = m - r * p.shift_bl;
    return j == 0 ? p.shift_ctx + static_cast<int64_t>(r) * p.K : p.A + static_cast<int64_t>(m - 1) * p.lda;
  }
  return p.A + static_cast<int64_t>(m) * p.lda;
}

__device__ __forceinline__ float bf16r(float x) { return round_bf16(x); }

template <int EPI>
__device__ __forceinline__ void epilogue(const GemmParams& p, const f32x16_t (&acc)[2][2], int m_base, int n_base,
                                         int lane) {
  const int col = lane & 31;
  const int rgrp = 4 * (lane >> 5);
  if (EPI == kEpiStore) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n_base + 32 * j + col;
        if (n >= p.N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
          if (m < p.M) p.C[static_cast<int64_t>(m) * p.ldc + n] = static_cast<uint16_t>(f32_to_bf16(acc[i][j][e]));
        }
      }
  } else if (EPI == kEpiSwiglu) {
    // Wave tile columns [n_base, n_base+32) are gate rows and [n_base+32, n_base+64)
    // the matching up rows of features f = n_base/2 + col.
    const int f = (n_base >> 1) + col;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
        if (m >= p.M) continue;
        const float g = bf16r(acc[i][0][e]);
        const float u = bf16r(acc[i][1][e]);
        const float s = bf16r(g / (1.f + __expf(-g)));
        p.C[static_cast<int64_t>(m) * p.ldc + f] = static_cast<uint16_t>(f32_to_bf16(s * u));
      }
  } else {  // kEpiQkv: the wave tile is one head of q, k or v (64 columns)
    const int HD = p.n_heads * kHeadDim;
    const int section = n_base / HD;  // 0 q, 1 k, 2 v
    const int head = (n_base - section * HD) / kHeadDim;
    const int d = col;  // this lane's columns are d and d + 32 of the head
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
        if (m >= p.M) continue;
        const int r = m / p.bl;
        const int pos = p.pos0[r] + (m - r * p.bl);
        float x0 = bf16r(acc[i][0][e]);  // element d
        float x1 = bf16r(acc[i][1][e]);  // element d + 32
        if (section < 2) {
          const int pc = min(max(pos, 0), p.max_pos - 1);
          const float c0 = p.cos_t[pc * kHeadDim + d], c1 = p.cos_t[pc * kHeadDim + d + 32];
          const float s0 = p.sin_t[pc * kHeadDim + d], s1 = p.sin_t[pc * kHeadDim + d + 32];
          // x*cos + rotate_half(x)*sin, rotate_half = [-x2, x1], each op rounded to bf16
          const float y0 = bf16r(bf16r(x0 * c0) + bf16r(-x1 * s0));
          const float y1 = bf16r(bf16r(x1 * c1) + bf16r(x0 * s1));
          x0 = y0;
          x1 = y1;
        }
        if (section == 0) {
          uint16_t* qp = p.q_out + static_cast<int64_t>(m) * HD + head * kHeadDim;
          qp[d] = static_cast<uint16_t>(f32_to_bf16(x0));
          qp[d + 32] = static_cast<uint16_t>(f32_to_bf16(x1));
        } else {
          const int pi = min(max(pos, 0) / kPageSize, p.table_cols - 1);
          int64_t page = p.table[static_cast<int64_t>(r) * p.table_stride + pi];
          page = min(max(page, int64_t{0}), p.n_pages - 1);
          const int slot = pos & (kPageSize - 1);
          if (section == 1) {
            p.pool[k_offset(page, head, p.n_heads, slot, d)] = static_cast<uint16_t>(f32_to_bf16(x0));
            p.pool[k_offset(page, head, p.n_heads, slot, d + 32)] = static_cast<uint16_t>(f32_to_bf16(x1));
          } else {
            p.pool[v_offset(page, head, p.n_heads, slot, d)] = static_cast<uint16_t>(f32_to_bf16(x0));
            p.pool[v_offset(page, head, p.n_heads, slot, d + 32)] = static_cast<uint16_t>(f32_to_bf16(x1));
          }
        }
      }
  }
}

template <int EPI, int AM>
__global__ __launch_bounds__(kThreadsG) void gemm_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * kLdsPitch];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * kLdsPitch];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;

  // Global -> register staging: 4 A and 4 B chunks of 16 bytes per thread.
  const uint16_t* a_src[4];
  const uint16_t* b_src[4];
  bool a_ok[4], b_ok[4];
  int lds_off[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int chunk = tid + c * kThreadsG;
    const int row = chunk >> 3, kc = (chunk & 7) * 8;
    lds_off[c] = row * kLdsPitch + kc;
    const int m = m0 + row, n = n0 + row;
    a_ok[c] = m < p.M;
    b_ok[c] = n < p.N;
    a_src[c] = (a_ok[c] ? a_row_ptr<AM>(p, m) : p.A) + kc;
    b_src[c] = p.W + static_cast<int64_t>(b_ok[c] ? n : 0) * p.ldw + kc;
  }
  u32x4_t ra[4], rb[4];
  auto fetch = [&](int k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ra[c] = a_ok[c] ? ldg16(a_src[c] + k) : u32x4_t{0u, 0u, 0u, 0u};
      rb[c] = b_ok[c] ? ldg16(b_src[c] + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      *reinterpret_cast<u32x4_t*>(&sA[buf][lds_off[c]]) = ra[c];
      *reinterpret_cast<u32x4_t*>(&sB[buf][lds_off[c]]) = rb[c];
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int kt_n = p.K / BK;
  fetch(0);
  stash(0);
  __syncthreads();
  const int frag_row = lane & 31;
  const int frag_k = 8 * (lane >> 5);
  for (int kt = 0; kt < kt_n; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < kt_n) fetch((kt + 1) * BK);
    const uint16_t* a_l = sA[buf] + (wm * 64 + frag_row) * kLdsPitch + frag_k;
    const uint16_t* b_l = sB[buf] + (wn * 64 + frag_row) * kLdsPitch + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      bf16x8_t af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l + 32 * i * kLdsPitch + ks));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bfr[j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(b_l + 32 * j * kLdsPitch + ks));
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < kt_n) stash(buf ^ 1);
    __syncthreads();
  }
  epilogue<EPI>(p, acc, m0 + wm * 64, n0 + wn * 64, lane);
}

// ---------------------------------------------------------------------------
// RMSNorm rows (HF LlamaRMSNorm): y = w * bf16(x * rsqrt(mean(x^2) + eps)).
// With delta != nullptr: residual = bf16(residual + delta) first (the
// residual add of the decoder layer), written back in place.
struct NormParams {
  const uint16_t* delta;
  uint16_t* residual;
  const uint16_t* x;  // input when delta == nullptr
  const uint16_t* w;
  float eps;
  int M, D;
  uint16_t* out;
};

// One wave per row; D = 1024 -> 16 bf16 per lane (two 16-byte chunks).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const NormParams p) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= p.M) return;
  const int64_t base = static_cast<int64_t>(row) * p.D;
  constexpr int kMaxChunks = 4;  // D <= 2048
  u32x4_t xv[kMaxChunks];
  const int nch = p.D / (64 * 8);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (c >= nch) break;
    const int64_t off = base + (c * 64 + lane) * 8;
    u32x4_t x;
    if (p.delta) {
      const u32x4_t r = ldg16(p.residual + off);
      const u32x4_t dl = ldg16(p.delta + off);
#pragma unroll
      for (int w = 0; w < 4; ++w) x[w] = pack_bf16x2(bf16lo(r[w]) + bf16lo(dl[w]), bf16hi(r[w]) + bf16hi(dl[w]));
      *reinterpret_cast<u32x4_t*>(p.residual + off) = x;
    } else {
      x = ldg16(p.x + off);
      if (p.residual) *reinterpret_cast<u32x4_t*>(p.residual + off) = x;  // residual = clone(x)
    }
    xv[c] = x;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = bf16lo(x[w]), b = bf16hi(x[w]);
      ss += a * a + b * b;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float rs = rsqrtf(ss / static_cast<float>(p.D) + p.eps);
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (c >= nch) break;
    const int64_t off = base + (c * 64 + lane) * 8;
    const u32x4_t wv = ldg16(p.w + (c * 64 + lane) * 8);
    u32x4_t y;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = bf16lo(wv[w]) * round_bf16(bf16lo(xv[c][w]) * rs);
      const float b = bf16hi(wv[w]) * round_bf16(bf16hi(xv[c][w]) * rs);
      y[w] = pack_bf16x2(a, b);
    }
    *reinterpret_cast<u32x4_t*>(p.out + off) = y;
  }
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

template <int EPI, int AM>
int launch_gemm(const GemmParams& p, hipStream_t st) {
  const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM), block(kThreadsG);
  hipLaunchKernelGGL((gemm_kernel<EPI, AM>), grid, block, 0, st, p);
  YAPD_LAUNCH_CHECK("gemm_kernel launch");
  return YAPD_OK;
}

int check_common(const GemmParams& p) {
  YAPD_REQUIRE(p.A && p.W, "gemm: NULL operand");
  YAPD_REQUIRE(p.M >= 1 && p.N >= 1 && p.K >= BK && p.K % BK == 0, "gemm: need M, N >= 1 and K %% %d == 0 (K=%d)", BK,
               p.K);
  YAPD_REQUIRE(al16(p.A) && al16(p.W) && p.lda % 8 == 0 && p.ldw % 8 == 0 && p.lda >= p.K && p.ldw >= p.K,
               "gemm: A/W must be 16-byte aligned with leading dims >= K and multiples of 8");
  return YAPD_OK;
}

}  // namespace
}  // namespace yapd

using yapd::GemmParams;

extern "C" int yapd_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, int M, int N, int K, void* C,
                              int64_t ldc, void* stream) {
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.W = static_cast<const uint16_t*>(W);
  p.ldw = ldw;
  p.M = M;
  p.N = N;
  p.K = K;
  p.C = static_cast<uint16_t*>(C);
  p.ldc = ldc;
  if (int rc = yapd::check_common(p)) return rc;
  YAPD_REQUIRE(C != nullptr && ldc >= N, "gemm: bad C");
  return yapd::launch_gemm<yapd::kEpiStore, yapd::kAPlain>(p, static_cast<hipStream_t>(stream));
}

extern "C" int yapd_gemm_head_shift(const void* hidden, const void* shift_ctx, int rows, int bl, int K,
                                    const void* W, int64_t ldw, int N, void* logits, int64_t ldc, void* stream) {
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(hidden);
  p.lda = K;
  p.shift_ctx = static_cast<const uint16_t*>(shift_ctx);
  p.shift_bl = bl;
  p.W = static_cast<const uint16_t*>(W);
  p.ldw = ldw;
  p.M = rows * bl;
  p.N = N;
  p.K = K;
  p.C = static_cast<uint16_t*>(logits);
  p.ldc = ldc;
  if (int rc = yapd::check_common(p)) return rc;
  YAPD_REQUIRE(shift_ctx && yapd::al16(shift_ctx) && logits && ldc >= N && rows >= 1 && bl >= 1,
               "gemm_head_shift: bad shift_ctx / logits");
  return yapd::launch_gemm<yapd::kEpiStore, yapd::kAShift>(p, static_cast<hipStream_t>(stream));
}

extern "C" int yapd_gemm_swiglu(const void* A, int64_t lda, const void* W_gu_interleaved, int M, int F, int K,
                                void* act, int64_t ld_act, void* stream) {
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.W = static_cast<const uint16_t*>(W_gu_interleaved);
  p.ldw = K;
  p.M = M;
  p.N = 2 * F;
  p.K = K;
  p.C = static_cast<uint16_t*>(act);
  p.ldc = ld_act;
  if (int rc = yapd::check_common(p)) return rc;
  YAPD_REQUIRE(act && F % 64 == 0 && ld_act >= F, "gemm_swiglu: F must be a multiple of 64");
  return yapd::launch_gemm<yapd::kEpiSwiglu, yapd::kAPlain>(p, static_cast<hipStream_t>(stream));
}

extern "C" int yapd_gemm_qkv_rope_kv(const void* A, int64_t lda, const void* W_qkv, int M, int K, int n_heads,
                                     const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int bl,
                                     void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table,
                                     int table_stride, int table_cols, void* stream) {
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.W = static_cast<const uint16_t*>(W_qkv);
  p.ldw = K;
  p.M = M;
  p.N = 3 * n_heads * yapd::kHeadDim;
  p.K = K;
  p.cos_t = cos_t;
  p.sin_t = sin_t;
  p.max_pos = max_pos;
  p.pos0 = pos0;
  p.bl = bl;
  p.n_heads = n_heads;
  p.q_out = static_cast<uint16_t*>(q_out);
  p.pool = static_cast<uint16_t*>(kv_pool);
  p.n_pages = n_pages;
  p.table = page_table;
  p.table_stride = table_stride;
  p.table_cols = table_cols;
  if (int rc = yapd::check_common(p)) return rc;
  YAPD_REQUIRE(cos_t && sin_t && pos0 && q_out && kv_pool && page_table, "gemm_qkv: NULL pointer");
  YAPD_REQUIRE(max_pos >= 1 && bl >= 1 && M % bl == 0 && n_heads >= 1 && n_pages >= 1 && table_cols >= 1 &&
                   table_stride >= table_cols,
               "gemm_qkv: bad positions / table shape");
  return yapd::launch_gemm<yapd::kEpiQkv, yapd::kAPlain>(p, static_cast<hipStream_t>(stream));
}

extern "C" int yapd_rmsnorm(const void* delta, void* residual, const void* x, const void* w, float eps, int M, int D,
                            void* out, void* stream) {
  YAPD_REQUIRE(w && out && M >= 1, "rmsnorm: NULL pointer or empty");
  YAPD_REQUIRE(D % 512 == 0 && D <= 2048, "rmsnorm: D must be a multiple of 512 and <= 2048 (got %d)", D);
  YAPD_REQUIRE(delta ? (residual != nullptr) : (x != nullptr), "rmsnorm: need (delta, residual) or x");
  YAPD_REQUIRE(!(delta && x), "rmsnorm: pass either delta (residual add) or x, not both");
  yapd::NormParams p{static_cast<const uint16_t*>(delta), static_cast<uint16_t*>(residual),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), eps, M, D,
                     static_cast<uint16_t*>(out)};
  hipLaunchKernelGGL(yapd::rmsnorm_kernel, dim3((M + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream), p);
  YAPD_LAUNCH_CHECK("rmsnorm_kernel launch");
  return YAPD_OK;
}
