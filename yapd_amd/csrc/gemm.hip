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

// Macro tile BM x BN x BK, WM x WN waves; each wave owns (BM/WM) x (BN/WN)
// as TM x TN MFMA tiles of 32 x 32.
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int PITCH = BK + 8;  // bf16 per LDS row: +16 bytes keeps 16-byte fragment reads conflict-free
  static constexpr int KCH = BK / 8;    // 16-byte chunks per tile row
  static constexpr int CA = BM * KCH / THREADS;
  static constexpr int CB = BN * KCH / THREADS;
  static_assert(TM >= 1 && TN >= 2 && TN % 2 == 0, "wave tile must be >= 32 x 64");
  static_assert(CA * THREADS == BM * KCH && CB * THREADS == BN * KCH, "tile loads must divide evenly");
};
constexpr int BK = 64;  // K granularity every config shares

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
  // affine-quantised W (MLX layout): uint32-packed codes [N, K*bits/32],
  // fp16 scale and bias per (row, 64-column group) [N, K/64]
  const uint32_t* Wq;
  int64_t ldq;  // uint32 words per row
  const uint16_t* qscale;
  const uint16_t* qbias;
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

template <int EPI, int TM, int TN>
__device__ __forceinline__ void epilogue(const GemmParams& p, const f32x16_t (&acc)[TM][TN], int m_base, int n_base,
                                         int lane) {
  const int col = lane & 31;
  const int rgrp = 4 * (lane >> 5);
  if (EPI == kEpiStore) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n_base + 32 * j + col;
        if (n >= p.N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
          if (m < p.M) p.C[static_cast<int64_t>(m) * p.ldc + n] = static_cast<uint16_t>(f32_to_bf16(acc[i][j][e]));
        }
      }
  } else if (EPI == kEpiSwiglu) {
    // Each 64-column group of W holds gate rows of 32 features, then their up rows:
    // tile 2q is gate and tile 2q+1 is up of features f = (n_base + 64q)/2 + col.
#pragma unroll
    for (int q2 = 0; q2 < TN / 2; ++q2) {
      const int f = ((n_base + 64 * q2) >> 1) + col;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
          if (m >= p.M) continue;
          const float g = bf16r(acc[i][2 * q2][e]);
          const float u = bf16r(acc[i][2 * q2 + 1][e]);
          const float s = bf16r(g / (1.f + __expf(-g)));
          p.C[static_cast<int64_t>(m) * p.ldc + f] = static_cast<uint16_t>(f32_to_bf16(s * u));
        }
    }
  } else {  // kEpiQkv: tiles 2q, 2q+1 are head dims d and d + 32 of one head of q, k or v
    const int HD = p.n_heads * kHeadDim;
    const int d = col;
#pragma unroll
    for (int q2 = 0; q2 < TN / 2; ++q2) {
      const int nb = n_base + 64 * q2;
      const int section = nb / HD;  // 0 q, 1 k, 2 v
      const int head = (nb - section * HD) / kHeadDim;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m_base + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
          if (m >= p.M) continue;
          const int r = m / p.bl;
          const int pos = p.pos0[r] + (m - r * p.bl);
          float x0 = bf16r(acc[i][2 * q2][e]);      // element d
          float x1 = bf16r(acc[i][2 * q2 + 1][e]);  // element d + 32
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
}

// Plain-store epilogue through LDS: the waves park their bf16 tile in the
// (now idle) LDS staging area, then every thread writes whole 16-byte row
// chunks, instead of one 2-byte store per accumulator.
template <class T>
__device__ __forceinline__ void store_tile_via_lds(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN],
                                                   uint16_t* lds, int m0, int n0, int wm, int wn, int lane, int tid) {
  constexpr int CP = T::BN + 8;  // staging row pitch (bf16)
  static_assert(T::BM * CP <= 2 * (T::BM + T::BN) * T::PITCH, "C tile must fit in the LDS staging area");
  const int col = lane & 31;
  const int rgrp = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = wm * T::WTM + 32 * i + 8 * (e >> 2) + rgrp + (e & 3);
        const int c = wn * T::WTN + 32 * j + col;
        lds[r * CP + c] = static_cast<uint16_t>(f32_to_bf16(acc[i][j][e]));
      }
  __syncthreads();
  const bool vec_ok = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0);
  constexpr int CPR = T::BN / 8;  // 16-byte chunks per tile row
  for (int idx = tid; idx < T::BM * CPR; idx += T::THREADS) {
    const int r = idx / CPR, cc = (idx % CPR) * 8;
    const int m = m0 + r, n = n0 + cc;
    if (m >= p.M || n >= p.N) continue;
    const uint16_t* src = lds + r * CP + cc;
    uint16_t* dst = p.C + static_cast<int64_t>(m) * p.ldc + n;
    if (vec_ok && n + 8 <= p.N) {
      *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(src);
    } else {
      for (int t = 0; t < 8 && n + t < p.N; ++t) dst[t] = src[t];
    }
  }
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

// Dequantise 8 codes of `bits` each starting at bit `shift0` of packed words:
// w = scale * q + bias, rounded once to bf16 (the MFMA operand).
template <int BITS>
__device__ __forceinline__ uint32_t dq_pair(uint32_t word, int shift, float sc, float bi) {
  constexpr uint32_t mask = (1u << BITS) - 1u;
  const float q0 = static_cast<float>((word >> shift) & mask);
  const float q1 = static_cast<float>((word >> (shift + BITS)) & mask);
  return pack_bf16x2(__builtin_fmaf(sc, q0, bi), __builtin_fmaf(sc, q1, bi));
}

template <class T, int EPI, int AM, int BQ = 0>
__global__ __launch_bounds__(T::THREADS) void gemm_kernel(const GemmParams p) {
  // One LDS block: two A stages, then two B stages; the store epilogue reuses all of it.
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (T::BM + T::BN) * T::PITCH];
  uint16_t(*sA)[T::BM * T::PITCH] = reinterpret_cast<uint16_t(*)[T::BM * T::PITCH]>(smem);
  uint16_t(*sB)[T::BN * T::PITCH] = reinterpret_cast<uint16_t(*)[T::BN * T::PITCH]>(smem + 2 * T::BM * T::PITCH);
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int m0 = blockIdx.y * T::BM, n0 = blockIdx.x * T::BN;

  // Global -> register staging: CA (CB) chunks of 16 bytes per thread.  Rows
  // past M (N) re-read the last valid row: they only feed accumulator rows
  // (columns) the epilogue never stores, and the loads stay unpredicated.
  const uint16_t* a_src[T::CA];
  const uint16_t* b_src[T::CB];
  int a_lds[T::CA], b_lds[T::CB];
#pragma unroll
  for (int c = 0; c < T::CA; ++c) {
    const int chunk = tid + c * T::THREADS;
    const int row = chunk / T::KCH, kc = (chunk % T::KCH) * 8;
    a_lds[c] = row * T::PITCH + kc;
    a_src[c] = a_row_ptr<AM>(p, min(m0 + row, p.M - 1)) + kc;
  }
#pragma unroll
  for (int c = 0; c < T::CB; ++c) {
    const int chunk = tid + c * T::THREADS;
    const int row = chunk / T::KCH, kc = (chunk % T::KCH) * 8;
    b_lds[c] = row * T::PITCH + kc;
    b_src[c] = BQ ? p.W : p.W + static_cast<int64_t>(min(n0 + row, p.N - 1)) * p.ldw + kc;
  }
  // Quantised W: one 16-byte chunk holds 128/BQ codes of one row; a 64-wide K
  // tile is exactly one quantisation group, so a chunk needs one scale/bias.
  constexpr int QVALS = BQ ? 128 / BQ : 8;          // codes per 16-byte chunk
  constexpr int QCH = BQ ? T::BK / QVALS : 1;       // chunks per tile row
  constexpr int CQ = BQ ? T::BN * QCH / T::THREADS : 1;
  static_assert(!BQ || CQ * T::THREADS == T::BN * QCH, "quantised tile loads must divide evenly");
  const uint32_t* q_src[CQ];
  const uint16_t* s_src[CQ];
  const uint16_t* z_src[CQ];
  int q_lds[CQ];
  if constexpr (BQ != 0) {
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      const int chunk = tid + c * T::THREADS;
      const int row = chunk / QCH, part = chunk % QCH;
      const int64_t n = min(n0 + row, p.N - 1);
      q_lds[c] = row * T::PITCH + part * QVALS;
      q_src[c] = p.Wq + n * p.ldq + part * (QVALS * BQ / 32);
      s_src[c] = p.qscale + n * (p.K / 64);
      z_src[c] = p.qbias + n * (p.K / 64);
    }
  }
  u32x4_t rq[CQ];
  uint16_t rs[CQ], rz[CQ];
  // Register staging: tile k+1 is fetched while tile k is multiplied and
  // stashed into the other LDS buffer after the MFMAs.
  u32x4_t ra[T::CA], rb[T::CB];
  auto fetch = [&](int k) {
#pragma unroll
    for (int c = 0; c < T::CA; ++c) ra[c] = ldg16(a_src[c] + k);
    if constexpr (BQ == 0) {
#pragma unroll
      for (int c = 0; c < T::CB; ++c) rb[c] = ldg16(b_src[c] + k);
    } else {
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        rq[c] = *reinterpret_cast<const u32x4_t*>(q_src[c] + k * BQ / 32);
        rs[c] = s_src[c][k / 64];
        rz[c] = z_src[c][k / 64];
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int c = 0; c < T::CA; ++c) *reinterpret_cast<u32x4_t*>(&sA[buf][a_lds[c]]) = ra[c];
    if constexpr (BQ == 0) {
#pragma unroll
      for (int c = 0; c < T::CB; ++c) *reinterpret_cast<u32x4_t*>(&sB[buf][b_lds[c]]) = rb[c];
    } else {
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        const float sc = f16_to_f32(rs[c]), bi = f16_to_f32(rz[c]);
        uint16_t* dst = &sB[buf][q_lds[c]];
        // QVALS codes -> QVALS bf16, written 8 at a time (16 bytes)
#pragma unroll
        for (int o = 0; o < QVALS / 8; ++o) {
          u32x4_t v;
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const int first = o * 8 + 2 * h;  // code index inside the chunk
            const int word = first * BQ / 32, shift = (first * BQ) % 32;
            v[h] = dq_pair<BQ>(rq[c][word], shift, sc, bi);
          }
          *reinterpret_cast<u32x4_t*>(dst + 8 * o) = v;
        }
      }
    }
  };

  f32x16_t acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int kt_n = p.K / T::BK;
  const int frag_row = lane & 31;
  const int frag_k = 8 * (lane >> 5);
  constexpr int KS = T::BK / 16;
  // Fragment registers double-buffered across k-steps: the LDS reads of step
  // s+1 are in flight while the MFMAs of step s run.
  bf16x8_t af[2][T::TM], bfr[2][T::TN];
  auto read_frags = [&](int buf, int ks, int slot) {
    const uint16_t* a_l = sA[buf] + (wm * T::WTM + frag_row) * T::PITCH + frag_k + 16 * ks;
    const uint16_t* b_l = sB[buf] + (wn * T::WTN + frag_row) * T::PITCH + frag_k + 16 * ks;
#pragma unroll
    for (int i = 0; i < T::TM; ++i) af[slot][i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l + 32 * i * T::PITCH));
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      bfr[slot][j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(b_l + 32 * j * T::PITCH));
  };

  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
  };
  // MFMAs of one k-step interleaved with the TM + TN fragment reads of the next.
  auto interleave = [&]() {
#pragma unroll
    for (int r = 0; r < T::TM + T::TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
      __builtin_amdgcn_sched_group_barrier(0x008, (T::TM * T::TN) / (T::TM + T::TN), 0);  // MFMAs
    }
  };

  // Pipeline: the last k-step of tile kt is multiplied after the barrier, so
  // its MFMAs (register operands only) cover the first LDS reads of tile kt+1.
  fetch(0);
  stash(0);
  __syncthreads();
  read_frags(0, 0, 0);
  for (int kt = 0; kt < kt_n; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < kt_n;
    if (more) fetch((kt + 1) * T::BK);
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      read_frags(buf, ks + 1, (ks + 1) & 1);
      mfma_step(ks & 1);
      interleave();
    }
    if (more) stash(buf ^ 1);
    __syncthreads();
    if (more) read_frags(buf ^ 1, 0, 0);
    mfma_step((KS - 1) & 1);
    if (more) interleave();
  }
  if (EPI == kEpiStore) {
    store_tile_via_lds<T>(p, acc, smem, m0, n0, wm, wn, lane, tid);
  } else {
    epilogue<EPI, T::TM, T::TN>(p, acc, m0 + wm * T::WTM, n0 + wn * T::WTN, lane);
  }
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

using TileS = Tile<128, 128, BK, 2, 2>;  // small M: more workgroups
using TileL = Tile<256, 256, BK, 2, 4>;  // large M: 8 waves of 128 x 64

template <class T, int EPI, int AM, int BQ>
int launch_tile(const GemmParams& p, hipStream_t st) {
  const dim3 grid((p.N + T::BN - 1) / T::BN, (p.M + T::BM - 1) / T::BM), block(T::THREADS);
  hipLaunchKernelGGL((gemm_kernel<T, EPI, AM, BQ>), grid, block, 0, st, p);
  YAPD_LAUNCH_CHECK("gemm_kernel launch");
  return YAPD_OK;
}

template <int EPI, int AM, int BQ = 0>
int launch_gemm(const GemmParams& p, hipStream_t st) {
  // Large tiles once they still give at least one workgroup per CU.
  const int64_t big_tiles = static_cast<int64_t>((p.M + 255) / 256) * ((p.N + 255) / 256);
  if (big_tiles >= 256) return launch_tile<TileL, EPI, AM, BQ>(p, st);
  return launch_tile<TileS, EPI, AM, BQ>(p, st);
}

int check_common(const GemmParams& p) {
  YAPD_REQUIRE(p.A && (p.W || p.Wq), "gemm: NULL operand");
  YAPD_REQUIRE(p.M >= 1 && p.N >= 1 && p.K >= BK && p.K % BK == 0, "gemm: need M, N >= 1 and K %% %d == 0 (K=%d)", BK,
               p.K);
  YAPD_REQUIRE(al16(p.A) && p.lda % 8 == 0 && p.lda >= p.K, "gemm: A must be 16-byte aligned, lda >= K, lda %% 8 == 0");
  YAPD_REQUIRE(p.Wq || (al16(p.W) && p.ldw % 8 == 0 && p.ldw >= p.K),
               "gemm: W must be 16-byte aligned with ldw >= K and a multiple of 8");
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

extern "C" int yapd_qgemm_affine(const void* A, int64_t lda, const uint32_t* w_packed, const void* scales,
                                 const void* biases, int bits, int group_size, int M, int N, int K, void* C,
                                 int64_t ldc, void* stream) {
  YAPD_REQUIRE(bits == 4 || bits == 8, "qgemm: bits must be 4 or 8 (got %d)", bits);
  YAPD_REQUIRE(group_size == 64, "qgemm: group_size must be 64 (got %d)", group_size);
  YAPD_REQUIRE(w_packed && scales && biases && C && ldc >= N, "qgemm: NULL pointer or bad ldc");
  YAPD_REQUIRE((reinterpret_cast<uintptr_t>(w_packed) & 15u) == 0, "qgemm: packed weights must be 16-byte aligned");
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.M = M;
  p.N = N;
  p.K = K;
  p.C = static_cast<uint16_t*>(C);
  p.ldc = ldc;
  p.Wq = w_packed;
  p.ldq = static_cast<int64_t>(K) * bits / 32;
  p.qscale = static_cast<const uint16_t*>(scales);
  p.qbias = static_cast<const uint16_t*>(biases);
  if (int rc = yapd::check_common(p)) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return bits == 4 ? yapd::launch_gemm<yapd::kEpiStore, yapd::kAPlain, 4>(p, st)
                   : yapd::launch_gemm<yapd::kEpiStore, yapd::kAPlain, 8>(p, st);
}
