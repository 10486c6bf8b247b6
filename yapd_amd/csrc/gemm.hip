// (b) bf16 MFMA GEMMs of the T3 layer with fused epilogues, plus the RMSNorm
// row kernel.
//
// C[M, N] = A[M, K] * W[N, K]^T (nn.Linear layout), fp32 accumulation on
// v_mfma_f32_32x32x16_bf16.  Grids of at least two 256 x 256 tiles per CU
// (gate/up, QKV, the speech head), or one with the plain or residual epilogue
// (o, down): `gemm_pt_kernel`, one persistent 4-wave workgroup per CU.  Other
// large M: `gemm_dl_kernel`, a 256 x 256 tile of
// 8 waves (128 x 64 each) whose A and W k-slices go global -> LDS by direct
// loads into two 64 KB stages.  Small M: the same kernel on one-wave 64 x 64
// tiles with three stages.  Mid M: the same kernel on 128 x 128 tiles of 8
// waves (32 x 64 each).  `gemm_kernel` (register-staged tiles with padded LDS
// rows) serves the quantised path below large M.  Every kernel runs the same MFMA over the same K
// order, so a row's result does not depend on which kernel the batch size
// selects.  Affine-quantised W: `gemm_dlq_kernel` (the direct-load layout with
// W dequantised from registers into LDS) at large M, `gemm_kernel` below.  K
// advances in steps of 64.
//
// Epilogues (once per output element):
//   * store    -- plain bf16 store (speech head, small projections);
//   * residual -- C = bf16(C + bf16(acc)): o_proj / down_proj with the
//                 decoder layer's residual add (engines/flashinfer.py:1040-1060);
//   * qkv      -- NeoX RoPE on q and k from a cos/sin table at each row's
//                 absolute position, q to its buffer, k and v straight into
//                 the paged KV pool (engines/flashinfer.py:998-1035);
//   * swiglu   -- silu(gate) * up from interleaved gate/up weight rows
//                 (engines/flashinfer.py:433-455).
// The bf16 roundings of the reference's separate ops are reproduced (HF
// computes q*cos, rotate_half(q)*sin and their sum in bf16; silu(g) and the
// product in bf16; the residual add of two bf16 values), so the fused results
// differ from it only through the fp32 accumulation order.
//
// A prologue mode "shift" reads A row (r, j) from hidden row (r, j-1) and
// row (r, 0) from shift_ctx[r]: the token-shifted speech head
// (engines/flashinfer.py:1452-1461).
#include "common.h"
#include "kv_layout.h"
#include "packed.h"
#include "quant.h"

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

enum EpiMode { kEpiStore = 0, kEpiQkv = 1, kEpiSwiglu = 2, kEpiResidual = 3 };
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
  const float* cos_t;  // [max_pos, 64] fp32 (values of the model-dtype table; columns 0..31 are read)
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
  // packed rows (NULL: row m / bl, slot m % bl): token m belongs to row
  // tok_row[m] of n_rows and sits at slot m - row_start[row] of it
  const int32_t* tok_row;
  const int32_t* row_start;
  int n_rows;
  // affine-quantised W (MLX layout): uint32-packed codes [N, K*bits/32],
  // fp16 scale and bias per (row, 64-column group) [N, K/64]
  const uint32_t* Wq;
  int64_t ldq;  // uint32 words per row
  const uint16_t* qscale;
  const uint16_t* qbias;
  int xcd_band;  // 1, 2: XCD-banded tile orders (set by the launcher)
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

// Position and KV page of one tile row for the qkv epilogue.  Computed at
// kernel start by thread `row` (< BM), so the loads of pos0 and of the page
// table overlap the main loop; parked in LDS for the epilogue.
struct RowMeta {
  int pos, page;
};

template <class T>
__device__ __forceinline__ RowMeta qkv_row_meta(const GemmParams& p, int m0, int row) {
  RowMeta rm{0, 0};
  if (row < T::BM) {
    const int m = min(m0 + row, p.M - 1);
    int r, slot;
    if (p.tok_row != nullptr) {
      r = min(max(p.tok_row[m], 0), p.n_rows - 1);
      slot = m - p.row_start[r];
    } else {
      r = m / p.bl;
      slot = m - r * p.bl;
    }
    const int pos = p.pos0[r] + slot;
    const int pi = min(max(pos, 0) / kPageSize, p.table_cols - 1);
    int64_t page = p.table[static_cast<int64_t>(r) * p.table_stride + pi];
    page = min(max(page, int64_t{0}), p.n_pages - 1);
    rm.pos = pos;
    rm.page = static_cast<int>(page);
  }
  return rm;
}

// Columns 0..31 of the cos and sin rows at every tile row's position, copied
// to LDS by the whole workgroup with one round trip to memory: the epilogue
// then reads LDS, whose waits (lgkmcnt) do not cover its own global stores,
// instead of a load and a store acknowledgement per 4-dim run.  Layout: a
// [BM][kRopePitch] cos block, then the sin block; the 36-float pitch puts the
// 16-byte reads of 8 consecutive rows in distinct banks.
constexpr int kRopePitch = 36;

template <class T>
constexpr int qkv_lds_bytes() {
  return T::BM * static_cast<int>(sizeof(RowMeta)) + 2 * T::BM * kRopePitch * 4;
}

template <class T>
__device__ __forceinline__ void stage_rope_rows(const GemmParams& p, const RowMeta* meta, float* rope, int tid) {
  constexpr int kChunks = T::BM * 16;  // per row: 8 x 16 bytes of cos, 8 of sin
  static_assert(kChunks % T::THREADS == 0, "whole chunks per thread");
  constexpr int kPer = kChunks / T::THREADS;
  f32x4_t v[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int c = tid + j * T::THREADS;
    const int row = c >> 4, part = c & 15;
    const int pc = min(max(meta[row].pos, 0), p.max_pos - 1);
    v[j] = *reinterpret_cast<const f32x4_t*>((part < 8 ? p.cos_t : p.sin_t) + pc * kHeadDim + 4 * (part & 7));
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int c = tid + j * T::THREADS;
    const int row = c >> 4, part = c & 15;
    *reinterpret_cast<f32x4_t*>(rope + ((part >> 3) * T::BM + row) * kRopePitch + 4 * (part & 7)) = v[j];
  }
}

// qkv epilogue: NeoX RoPE on q and k from the cos/sin tables at each row's
// position; the tables are HF's cat(freqs, freqs) layout, so column d + 32
// equals column d and only columns 0..31 are read (staged in `rope`).  The qkv GEMM multiplies
// W x A^T (MFMA operands swapped), so lane l holds token (l & 31) of each
// 32-row block and, in each 32-column block, head dims
// 8 * (e / 4) + 4 * (l / 32) + e % 4 for accumulator element e: four runs of
// 4 consecutive dims.  Tiles 2q, 2q+1 of a wave are dims d and d + 32 of one
// head of q, k or v (the section is uniform per wave: n_base is a multiple of
// 64 and 64 divides n_heads * 64).  So a lane does RoPE on whole runs
// (16-byte cos/sin loads), stores q and k as 8-byte runs, and a V column
// (layout d * 16 + slot) is written by 32 lanes with consecutive slots.
// `meta` holds the RowMeta of the tile rows, `rope` their cos/sin columns.
template <class T, int SECTION>
__device__ __forceinline__ void epilogue_qkv_section(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN],
                                                     const RowMeta* meta, const float* rope, int m0, int nb, int q2,
                                                     int wm, int lane) {
  const int tok = lane & 31;
  const int dgrp = 4 * (lane >> 5);
  const int HD = p.n_heads * kHeadDim;
  const int head = (nb - SECTION * HD) / kHeadDim;
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    const int rl = wm * T::WTM + 32 * i + tok;
    const int m = m0 + rl;
    if (m >= p.M) continue;
    const RowMeta mt = meta[rl];
    const int slot = mt.pos & (kPageSize - 1);
    uint16_t* const kv = p.pool + kv_plane_offset(mt.page, SECTION == 2 ? 1 : 0, head, p.n_heads);
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = 8 * r4 + dgrp;
      // Dims d0 + t (x0) and d0 + 32 + t (x1), rounded to bf16 two at a time:
      // a packed pair holds dims (t, t + 1), which is also the store layout.
      uint32_t X0[2], X1[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        X0[h] = pack_bf16x2(acc[i][2 * q2][4 * r4 + 2 * h], acc[i][2 * q2][4 * r4 + 2 * h + 1]);
        X1[h] = pack_bf16x2(acc[i][2 * q2 + 1][4 * r4 + 2 * h], acc[i][2 * q2 + 1][4 * r4 + 2 * h + 1]);
      }
      if constexpr (SECTION < 2) {
        const f32x4_t c = *reinterpret_cast<const f32x4_t*>(rope + rl * kRopePitch + d0);
        const f32x4_t sn = *reinterpret_cast<const f32x4_t*>(rope + (T::BM + rl) * kRopePitch + d0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // x*cos + rotate_half(x)*sin, rotate_half = [-x2, x1], each op rounded
          // to bf16; bf16(-x2*s) = -bf16(x2*s) (round-to-nearest-even is symmetric)
          const float a0 = bf16lo(X0[h]), a1 = bf16hi(X0[h]);
          const float b0 = bf16lo(X1[h]), b1 = bf16hi(X1[h]);
          const float c0 = c[2 * h], c1 = c[2 * h + 1], s0 = sn[2 * h], s1 = sn[2 * h + 1];
          const uint32_t ac = pack_bf16x2(a0 * c0, a1 * c1), bs = pack_bf16x2(b0 * s0, b1 * s1);
          const uint32_t bc = pack_bf16x2(b0 * c0, b1 * c1), as = pack_bf16x2(a0 * s0, a1 * s1);
          X0[h] = pack_bf16x2(bf16lo(ac) - bf16lo(bs), bf16hi(ac) - bf16hi(bs));
          X1[h] = pack_bf16x2(bf16lo(bc) + bf16lo(as), bf16hi(bc) + bf16hi(as));
        }
      }
      const u32x2_t lo = {X0[0], X0[1]};
      const u32x2_t hi = {X1[0], X1[1]};
      if constexpr (SECTION == 0) {
        uint16_t* qp = p.q_out + static_cast<int64_t>(m) * HD + head * kHeadDim + d0;
        *reinterpret_cast<u32x2_t*>(qp) = lo;
        *reinterpret_cast<u32x2_t*>(qp + 32) = hi;
      } else if constexpr (SECTION == 1) {
        *reinterpret_cast<u32x2_t*>(kv + slot * kHeadDim + d0) = lo;
        *reinterpret_cast<u32x2_t*>(kv + slot * kHeadDim + d0 + 32) = hi;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          kv[(d0 + t) * kPageSize + slot] = static_cast<uint16_t>(X0[t >> 1] >> (16 * (t & 1)));
          kv[(d0 + 32 + t) * kPageSize + slot] = static_cast<uint16_t>(X1[t >> 1] >> (16 * (t & 1)));
        }
      }
    }
  }
}

template <class T>
__device__ __forceinline__ void epilogue_qkv(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN],
                                             const RowMeta* meta, const float* rope, int m0, int n_base, int wm,
                                             int lane) {
  const int HD = p.n_heads * kHeadDim;
#pragma unroll
  for (int q2 = 0; q2 < T::TN / 2; ++q2) {
    const int nb = n_base + 64 * q2;
    // Columns past N (a last tile wider than what is left of 3 * HD) belong to
    // no head: skip them (N is a multiple of 64, so a group is all in or out).
    if (nb >= p.N) continue;
    const int section = nb / HD;  // 0 q, 1 k, 2 v
    if (section == 0) {
      epilogue_qkv_section<T, 0>(p, acc, meta, rope, m0, nb, q2, wm, lane);
    } else if (section == 1) {
      epilogue_qkv_section<T, 1>(p, acc, meta, rope, m0, nb, q2, wm, lane);
    } else {
      epilogue_qkv_section<T, 2>(p, acc, meta, rope, m0, nb, q2, wm, lane);
    }
  }
}

// swiglu epilogue.  Each 64-column group of W holds the gate rows of 32
// features, then their up rows, so tiles 2q and 2q+1 of a wave are gate and
// up of the same 32 features.  The swiglu GEMM multiplies W x A^T (MFMA
// operands swapped, as for qkv): lane l holds token (l & 31) of each 32-row
// block and features 8 * (e / 4) + 4 * (l / 32) + e % 4 of the group for
// accumulator element e -- four runs of 4 consecutive features.  silu(g) and
// the product are rounded to bf16 as the reference's separate ops are; silu
// uses the hardware reciprocal (<= 1 ulp in fp32 before the bf16 rounding).
// Neighbouring features share each bf16 conversion, and every run leaves as
// one 8-byte store straight from registers.
template <class T>
__device__ __forceinline__ void epilogue_swiglu(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN], int m0,
                                                int n0, int wm, int wn, int lane) {
  const int F = p.N / 2;
  const int tok = lane & 31;
  const int fsub = 4 * (lane >> 5);
  const bool vec_ok = (p.ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 7u) == 0);
  auto silu_mul = [](float g0, float g1, float u0, float u1) {
    const uint32_t gp = pack_bf16x2(g0, g1), up = pack_bf16x2(u0, u1);
    const float gb0 = bf16lo(gp), gb1 = bf16hi(gp);
    const uint32_t sp = pack_bf16x2(gb0 * __builtin_amdgcn_rcpf(1.f + __expf(-gb0)),
                                    gb1 * __builtin_amdgcn_rcpf(1.f + __expf(-gb1)));
    return pack_bf16x2(bf16lo(sp) * bf16lo(up), bf16hi(sp) * bf16hi(up));
  };
#pragma unroll
  for (int i = 0; i < T::TM; ++i) {
    const int m = m0 + wm * T::WTM + 32 * i + tok;
    if (m >= p.M) continue;
    uint16_t* const row = p.C + static_cast<int64_t>(m) * p.ldc;
#pragma unroll
    for (int q2 = 0; q2 < T::TN / 2; ++q2) {
      const int fb = (n0 + wn * T::WTN + 64 * q2) / 2;
      if (fb >= F) continue;  // F % 64 == 0: a group is all in or all out
      const f32x16_t& g = acc[i][2 * q2];
      const f32x16_t& u = acc[i][2 * q2 + 1];
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int e = 4 * r4;
        const u32x2_t y = {silu_mul(g[e], g[e + 1], u[e], u[e + 1]), silu_mul(g[e + 2], g[e + 3], u[e + 2], u[e + 3])};
        uint16_t* dst = row + fb + 8 * r4 + fsub;
        if (vec_ok) {
          *reinterpret_cast<u32x2_t*>(dst) = y;
        } else {
          dst[0] = static_cast<uint16_t>(y[0] & 0xffffu);
          dst[1] = static_cast<uint16_t>(y[0] >> 16);
          dst[2] = static_cast<uint16_t>(y[1] & 0xffffu);
          dst[3] = static_cast<uint16_t>(y[1] >> 16);
        }
      }
    }
  }
}

// Plain-store epilogue through LDS: the waves park their bf16 tile in the
// (now idle) LDS staging area, then every thread writes whole 16-byte row
// chunks, instead of one 2-byte store per accumulator.  With ADD the tile is
// the residual branch's delta: C = bf16(C + bf16(acc)), the decoder layer's
// residual add (HF LlamaDecoderLayer; engines/flashinfer.py:1040-1060) with
// the reference's two roundings (the fp32 sum of two bf16 values is exact).
template <class T, bool ADD = false>
__device__ __forceinline__ void store_tile_via_lds(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN],
                                                   uint16_t* lds, int m0, int n0, int wm, int wn, int lane, int tid) {
  constexpr int CP = T::BN + 8;  // staging row pitch (bf16)
  static_assert(T::BM * CP <= 2 * (T::BM + T::BN) * T::PITCH, "C tile must fit in the LDS staging area");
  constexpr int CPR = T::BN / 8;                       // 16-byte chunks per tile row
  constexpr int ITER = T::BM * CPR / T::THREADS;        // chunks per thread
  static_assert(ITER * T::THREADS == T::BM * CPR, "tile chunks must split evenly over the threads");
  const bool vec_ok = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0);
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
  // With ADD, all of this thread's residual chunks are requested at once
  // (the accumulators are dead now), so they cost one round trip, which the
  // barrier waits for; loads placed after stores to the same array would
  // otherwise run one round trip per chunk.  Addresses: the tile's uniform
  // base plus a 32-bit byte offset per chunk (a tile spans far less than
  // 4 GiB), half the registers of 64-bit pointers.
  const char* const c_base = reinterpret_cast<const char*>(p.C + static_cast<int64_t>(m0) * p.ldc + n0);
  auto c_ofs = [&](int r, int cc) { return static_cast<uint32_t>((r * p.ldc + cc) * 2); };
  u32x4_t res[ADD ? ITER : 1];
  if constexpr (ADD) {
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int idx = tid + it * T::THREADS;
      const int r = idx / CPR, cc = (idx % CPR) * 8;
      const int m = m0 + r, n = n0 + cc;
      if (vec_ok && m < p.M && n + 8 <= p.N) res[it] = *reinterpret_cast<const u32x4_t*>(c_base + c_ofs(r, cc));
    }
  }
  __syncthreads();
  // the stores' indices from an opaque copy of tid: recomputed here, so the
  // loads' offsets need not stay live beside the residual chunks
  int tid_s = tid;
  if constexpr (ADD) asm volatile("" : "+v"(tid_s));
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int idx = tid_s + it * T::THREADS;
    const int r = idx / CPR, cc = (idx % CPR) * 8;
    const int m = m0 + r, n = n0 + cc;
    if (m >= p.M || n >= p.N) continue;
    const uint16_t* src = lds + r * CP + cc;
    uint16_t* dst = reinterpret_cast<uint16_t*>(const_cast<char*>(c_base) + c_ofs(r, cc));
    if (vec_ok && n + 8 <= p.N) {
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(src);
      if constexpr (ADD) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          v[w] = pack_bf16x2(bf16lo(res[it][w]) + bf16lo(v[w]), bf16hi(res[it][w]) + bf16hi(v[w]));
      }
      *reinterpret_cast<u32x4_t*>(dst) = v;
    } else {
      for (int t = 0; t < 8 && n + t < p.N; ++t) {
        if constexpr (ADD) {
          dst[t] = static_cast<uint16_t>(f32_to_bf16(bf16_to_f32(dst[t]) + bf16_to_f32(src[t])));
        } else {
          dst[t] = src[t];
        }
      }
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

// XCD-aware tile order for single-round grids (at most one workgroup per
// CU).  Workgroups are dispatched round-robin over the 8 XCDs (linear id L
// runs on XCD L % 8), each with its own L2.  In row-major order the column
// tiles of one A row block land on different XCDs, so every one of them
// fetches that block; with `band` set, XCD j instead takes the band of row
// tiles [j R/8, (j+1) R/8) across all column tiles, and each A row block is
// fetched into one L2.  Mode 2 is for multi-round grids with few column tiles
// and large A row blocks (down at M > 16384) and for QKV: the same bands,
// columns fastest, so the workgroups an XCD runs at once cover whole row
// blocks (8 row blocks x 4 columns for N = 1024) and each A row block is
// fetched once, by one XCD, while in row-major order 4 XCDs fetch it.
// (gate/up, 32 column tiles, keeps the row-major order, in which each XCD
// keeps the same 4 column tiles of W in its L2 for every round; the banded
// order measured slower there.)
__device__ __forceinline__ int2 tile_coords(int xcd_band) {
  const int C = gridDim.x, R = gridDim.y;
  const int L = blockIdx.x + C * blockIdx.y;
  if (!xcd_band || R % 8 != 0) return make_int2(blockIdx.x, blockIdx.y);
  const int band = R / 8;
  const int j = L % 8, i = L / 8;
  if (xcd_band == 2) return make_int2(i % C, j * band + i / C);
  return make_int2(i / band, j * band + i % band);  // (column tile, row tile)
}

// Epilogue dispatch.  Every wave has finished reading the LDS stages (the
// main loop ends with a barrier and no LDS reads after it), so the epilogues
// may reuse all of LDS (at least qkv_lds_bytes<T>() of it for kEpiQkv).
template <class T, int EPI>
__device__ __forceinline__ void finish_tile(const GemmParams& p, const f32x16_t (&acc)[T::TM][T::TN], uint16_t* lds,
                                            const RowMeta& rm, int m0, int n0, int wm, int wn, int lane, int tid) {
  if constexpr (EPI == kEpiStore) {
    store_tile_via_lds<T>(p, acc, lds, m0, n0, wm, wn, lane, tid);
  } else if constexpr (EPI == kEpiResidual) {
    store_tile_via_lds<T, true>(p, acc, lds, m0, n0, wm, wn, lane, tid);
  } else if constexpr (EPI == kEpiSwiglu) {
    epilogue_swiglu<T>(p, acc, m0, n0, wm, wn, lane);
  } else {
    RowMeta* meta = reinterpret_cast<RowMeta*>(lds);
    float* rope = reinterpret_cast<float*>(meta + T::BM);
    if (tid < T::BM) meta[tid] = rm;
    __syncthreads();
    if (n0 < 2 * p.n_heads * kHeadDim) {  // q or k columns in this tile (uniform per workgroup)
      stage_rope_rows<T>(p, meta, rope, tid);
      __syncthreads();
    }
    epilogue_qkv<T>(p, acc, meta, rope, m0, n0 + wn * T::WTN, wm, lane);
  }
}

template <class T, int EPI, int AM, int BQ = 0>
__global__ __launch_bounds__(T::THREADS) void gemm_kernel(const GemmParams p) {
  // One LDS block: two A stages, then two B stages; the store epilogue reuses all of it.
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (T::BM + T::BN) * T::PITCH];
  uint16_t(*sA)[T::BM * T::PITCH] = reinterpret_cast<uint16_t(*)[T::BM * T::PITCH]>(smem);
  uint16_t(*sB)[T::BN * T::PITCH] = reinterpret_cast<uint16_t(*)[T::BN * T::PITCH]>(smem + 2 * T::BM * T::PITCH);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // wave index: uniform
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int2 tc = tile_coords(p.xcd_band);
  const int m0 = tc.y * T::BM, n0 = tc.x * T::BN;

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
        acc[i][j] = EPI == kEpiQkv || EPI == kEpiSwiglu  // transposed product for these epilogues
                        ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
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
  const RowMeta rm = EPI == kEpiQkv ? qkv_row_meta<T>(p, m0, tid) : RowMeta{0, 0};
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
  static_assert(EPI != kEpiQkv || qkv_lds_bytes<T>() <= static_cast<int>(sizeof(smem)), "qkv epilogue LDS");
  finish_tile<T, EPI>(p, acc, smem, rm, m0, n0, wm, wn, lane, tid);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS variant for bf16 W.  A and W tiles travel global -> LDS with
// global_load_lds_dwordx4 (64 lanes x 16 bytes land as one contiguous 1 KB
// run at the wave-uniform LDS address in M0), so there is no register
// staging and no ds_write: LDS writes through ds_write_b128 sustain about a
// third of the ds_read_b128 rate on gfx950 and were the bound of the staged
// kernel.
//
// LDS rows hold BK = 64 bf16 (128 bytes) unpadded.  The 16-byte chunk c of
// row r sits in slot c ^ ((r >> 1) & 7): the 16 consecutive rows one
// 16-lane group of a fragment read touches then cover 16 distinct 16-byte
// bank groups (two 128-byte rows share one 256-byte bank line).  A load
// instruction covers 8 rows; lane i writes slot i % 8 of row i / 8, so it
// fetches the chunk that belongs there.
template <class T, int NS>
struct DlLayout {
  static_assert(T::BK == 64, "direct-load tiles use 128-byte LDS rows");
  static constexpr int WAVES = T::THREADS / 64;
  static_assert(NS >= 2 && NS <= 4, "two to four LDS stages");
  static constexpr int ROWB = 128;
  static constexpr int CPR = 8;  // 16-byte chunks per row
  static constexpr int RPI = 8;  // rows per 1 KB load instruction
  static constexpr int A_BYTES = T::BM * ROWB, B_BYTES = T::BN * ROWB;
  __device__ static __forceinline__ int swz(int r) { return (r >> 1) & 7; }  // slot of chunk c is c ^ swz(r)
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LA = T::BM / 8 / WAVES;  // 1 KB loads per wave and k-tile
  static constexpr int LB = T::BN / 8 / WAVES;
  static_assert(LA * 8 * WAVES == T::BM && LB * 8 * WAVES == T::BN, "rows must split evenly over the waves");
  static constexpr int LPT = LA + LB;  // loads per wave and k-tile
  static_assert((NS - 2) * LPT <= 63, "the vmcnt counter holds at most 63 loads");
  static constexpr int C_BYTES = T::BM * (T::BN + 8) * 2;  // store-epilogue staging
  static constexpr int LDS = NS * STAGE > C_BYTES ? NS * STAGE : C_BYTES;
};

// Wait until at most N of this wave's vector-memory loads are outstanding
// (they complete in issue order).  The memory clobber keeps the LDS reads
// that follow below the wait.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Hand-off of an LDS stage across the workgroup: this wave's loads up to the
// stage have landed (at most N later loads still in flight), its LDS reads
// have completed (so the stage it read last may be overwritten), then the
// workgroup barrier.  __syncthreads would also drain the later tiles' loads.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// 16 bytes per lane from src into LDS at lds_run + 16 * lane (lds_run must be
// the same for the whole wave: it is the M0 base of global_load_lds_dwordx4).
__device__ __forceinline__ void load_lds16(const uint16_t* src, char* lds_run) {
  __builtin_amdgcn_global_load_lds(
      src, reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(lds_run)), 16, 0, 0);
}

template <class T, int EPI, int AM, int NS>
__global__ __launch_bounds__(T::THREADS) void gemm_dl_kernel(const GemmParams p) {
  using L = DlLayout<T, NS>;
  // Dynamic LDS: the compiler cannot see the DMA writes into a static
  // __shared__ array and would treat its contents as undefined.
  extern __shared__ __attribute__((aligned(16))) uint16_t dyn_lds[];
  char* lds = reinterpret_cast<char*>(dyn_lds);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;  // wave index: uniform
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int2 tc = tile_coords(p.xcd_band);
  const int m0 = tc.y * T::BM, n0 = tc.x * T::BN;

  // Per-lane sources of this wave's LA + LB loads (k offset added per tile).
  // Rows past M (N) re-read the last valid row, as in the staged kernel.
  const uint16_t* a_src[L::LA];
  const uint16_t* b_src[L::LB];
#pragma unroll
  for (int j = 0; j < L::LA; ++j) {
    const int r = (wave * L::LA + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    a_src[j] = a_row_ptr<AM>(p, min(m0 + r, p.M - 1)) + 8 * c;
  }
#pragma unroll
  for (int j = 0; j < L::LB; ++j) {
    const int r = (wave * L::LB + j) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    b_src[j] = p.W + static_cast<int64_t>(min(n0 + r, p.N - 1)) * p.ldw + 8 * c;
  }
  auto issue = [&](int kt, int stage) {
    const int k = kt * T::BK;
    char* a_dst = lds + stage * L::STAGE + wave * L::LA * 1024;
    char* b_dst = lds + stage * L::STAGE + L::A_BYTES + wave * L::LB * 1024;
#pragma unroll
    for (int j = 0; j < L::LA; ++j) load_lds16(a_src[j] + k, a_dst + j * 1024);
#pragma unroll
    for (int j = 0; j < L::LB; ++j) load_lds16(b_src[j] + k, b_dst + j * 1024);
  };

  f32x16_t acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment addressing: lane l reads row (l & 31) of a 32-row MFMA tile,
  // logical chunk 2 * ks + (l >> 5); the swizzle term depends on the lane
  // only because every tile starts at a multiple of 16 rows.
  const int frag_row = lane & 31;
  const int ysw = (lane >> 5) ^ ((frag_row >> 1) & 7);
  const int a_off = (wm * T::WTM + frag_row) * L::ROWB;
  const int b_off = L::A_BYTES + (wn * T::WTN + frag_row) * L::ROWB;
  constexpr int KS = T::BK / 16;
  bf16x8_t af[2][T::TM], bfr[2][T::TN];
  auto read_frags = [&](int stage, int ks, int slot) {
    const int cofs = ((2 * ks) ^ ysw) * 16;
    const char* a_l = lds + stage * L::STAGE + a_off + cofs;
    const char* b_l = lds + stage * L::STAGE + b_off + cofs;
    // Issue order = first use by mfma_step (i-major): A0, B0..B(TN-1), A1, ...
    // LDS reads complete in order, so the wait before each MFMA only covers
    // the reads it needs.
    af[slot][0] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l));
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      bfr[slot][j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(b_l + 32 * j * L::ROWB));
#pragma unroll
    for (int i = 1; i < T::TM; ++i)
      af[slot][i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l + 32 * i * L::ROWB));
  };
  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
        acc[i][j] = EPI == kEpiQkv || EPI == kEpiSwiglu  // transposed product for these epilogues
                        ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
  };
  // One MFMA, then one fragment read of the next k-step: the step's first
  // MFMAs never wait on a read issued in the same step.
  auto interleave = [&]() {
#pragma unroll
    for (int r = 0; r < T::TM + T::TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, T::TM * T::TN - (T::TM + T::TN), 0);
  };

  // NS LDS stages, NS - 1 tiles in flight.  Tile kt+NS-1 is requested at the
  // top of tile kt into the stage tile kt-1 used: its last fragments were
  // consumed by the MFMAs that ended tile kt-1.  Before the first fragments
  // of tile kt+1 are read, the wave waits for its loads of that tile and
  // keeps the later tiles in flight; with several waves a barrier then covers
  // the other waves' loads of it (with two stages nothing later is in flight
  // and __syncthreads does both).
  const int kt_n = p.K / T::BK;
#pragma unroll
  for (int s = 0; s + 1 < NS; ++s)
    if (s < kt_n) issue(s, s);
  const RowMeta rm = EPI == kEpiQkv ? qkv_row_meta<T>(p, m0, tid) : RowMeta{0, 0};
  // Tiles issued after tile t, when the fragments of tile t are first read.
  auto wait_tile = [&](int t) {
    if constexpr (NS == 2) {
      if constexpr (L::WAVES > 1) {
        __syncthreads();
      } else {
        wait_vmcnt<0>();
      }
    } else {
      // the same condition in every wave: all of them take the same barriers
      const bool full = min(t + NS - 2, kt_n - 1) - t == NS - 2;
      if constexpr (L::WAVES > 1) {
        if (full) {
          stage_barrier<(NS - 2) * L::LPT>();
        } else {
          stage_barrier<0>();
        }
      } else {
        if (full) {
          wait_vmcnt<(NS - 2) * L::LPT>();
        } else {
          wait_vmcnt<0>();
        }
      }
    }
  };
  wait_tile(0);
  read_frags(0, 0, 0);
  int stage = 0;
  for (int kt = 0; kt < kt_n; ++kt) {
    const bool more = kt + 1 < kt_n;
    const int next = stage + 1 == NS ? 0 : stage + 1;
    if (kt + NS - 1 < kt_n) issue(kt + NS - 1, stage == 0 ? NS - 1 : stage - 1);
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      read_frags(stage, ks + 1, (ks + 1) & 1);
      mfma_step(ks & 1);
      interleave();
    }
    if (more) {
      wait_tile(kt + 1);
      read_frags(next, 0, 0);
    } else if constexpr (L::WAVES > 1) {
      __syncthreads();  // every wave is done with the stages before the epilogue reuses LDS
    }
    mfma_step((KS - 1) & 1);
    if (more) interleave();
    stage = next;
  }
  static_assert(EPI != kEpiQkv || qkv_lds_bytes<T>() <= L::LDS, "qkv epilogue LDS");
  finish_tile<T, EPI>(p, acc, dyn_lds, rm, m0, n0, wm, wn, lane, tid);
}

// Affine-quantised W on the direct-load layout: A moves global -> LDS by
// direct loads as in gemm_dl_kernel; W's codes (one 16-byte chunk per code
// row and k-half or quarter -- 8-byte chunks where 16-byte ones would not
// give every thread one: 4-bit codes on 128-column tiles), scales and biases
// come into registers one k-tile ahead, and after the k-tile's MFMAs each thread dequantises its
// chunk (w = scale * q + bias, rounded once to bf16, as in gemm_kernel) and
// writes it into the next stage's B tile in the same swizzled layout, so the
// fragment reads and the MFMA loop are gemm_dl_kernel's.  Only W passes
// through ds_write (half of the register-staged kernel's LDS writes).  The
// epilogues are gemm_dl_kernel's: a row's result equals the bf16 kernel's on
// the dequantised weights bit for bit (same W values, MFMA and K order).
template <class T, int EPI, int AM, int BQ>
__global__ __launch_bounds__(T::THREADS) void gemm_dlq_kernel(const GemmParams p) {
  using L = DlLayout<T, 2>;
  static_assert(BQ == 4 || BQ == 8, "4- or 8-bit codes");
  extern __shared__ __attribute__((aligned(16))) uint16_t dyn_lds[];
  char* lds = reinterpret_cast<char*>(dyn_lds);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave / T::WN, wn = wave % T::WN;
  const int2 tc = tile_coords(p.xcd_band);
  const int m0 = tc.y * T::BM, n0 = tc.x * T::BN;

  const uint16_t* a_src[L::LA];
#pragma unroll
  for (int j = 0; j < L::LA; ++j) {
    const int r = (wave * L::LA + j) * L::RPI + lane / L::CPR;
    const int c = (lane % L::CPR) ^ L::swz(r);
    a_src[j] = a_row_ptr<AM>(p, min(m0 + r, p.M - 1)) + 8 * c;
  }
  auto issue_a = [&](int kt, int stage) {
    char* a_dst = lds + stage * L::STAGE + wave * L::LA * 1024;
#pragma unroll
    for (int j = 0; j < L::LA; ++j) load_lds16(a_src[j] + kt * T::BK, a_dst + j * 1024);
  };

  // W codes: a chunk of QB bytes holds QVALS codes of one row; a row's k-tile
  // (one quantisation group of 64) is QCH chunks; each thread owns CQ chunks.
  constexpr int QB = (T::BN * (T::BK * BQ / 128)) % T::THREADS == 0 ? 16 : 8;
  constexpr int QW = QB / 4;  // 32-bit words per chunk
  constexpr int QVALS = QB * 8 / BQ;
  constexpr int QCH = T::BK / QVALS;
  constexpr int CQ = T::BN * QCH / T::THREADS;
  static_assert(CQ >= 1 && CQ * T::THREADS == T::BN * QCH, "quantised tile loads must divide evenly");
  const uint32_t* q_src[CQ];
  const uint16_t* s_src[CQ];
  const uint16_t* z_src[CQ];
  int q_row[CQ], q_part[CQ];
#pragma unroll
  for (int c = 0; c < CQ; ++c) {
    const int chunk = tid + c * T::THREADS;
    const int row = chunk / QCH, part = chunk % QCH;
    const int64_t n = min(n0 + row, p.N - 1);
    q_row[c] = row;
    q_part[c] = part;
    q_src[c] = p.Wq + n * p.ldq + part * (QVALS * BQ / 32);
    s_src[c] = p.qscale + n * (p.K / 64);
    z_src[c] = p.qbias + n * (p.K / 64);
  }
  uint32_t rq[CQ][QW];
  uint16_t rs[CQ], rz[CQ];
  auto fetch_w = [&](int kt) {
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      const uint32_t* src = q_src[c] + kt * T::BK * BQ / 32;
      if constexpr (QW == 4) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src);
#pragma unroll
        for (int w = 0; w < 4; ++w) rq[c][w] = v[w];
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        rq[c][0] = v.x;
        rq[c][1] = v.y;
      }
      rs[c] = s_src[c][kt];
      rz[c] = z_src[c][kt];
    }
  };
  auto stash_w = [&](int stage) {
    char* b_base = lds + stage * L::STAGE + L::A_BYTES;
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      const float sc = f16_to_f32(rs[c]), bi = f16_to_f32(rz[c]);
      const int r = q_row[c];
#pragma unroll
      for (int o = 0; o < QVALS / 8; ++o) {  // 8 codes -> one 16-byte bf16 chunk
        u32x4_t v;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int first = o * 8 + 2 * h;  // code index inside the chunk
          const int word = first * BQ / 32, shift = (first * BQ) % 32;
          v[h] = dq_pair<BQ>(rq[c][word], shift, sc, bi);
        }
        const int lc = q_part[c] * (QVALS / 8) + o;  // logical 16-byte chunk of the row
        *reinterpret_cast<u32x4_t*>(b_base + r * L::ROWB + ((lc ^ L::swz(r)) * 16)) = v;
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

  const int frag_row = lane & 31;
  const int ysw = (lane >> 5) ^ L::swz(frag_row);
  const int a_off = (wm * T::WTM + frag_row) * L::ROWB;
  const int b_off = L::A_BYTES + (wn * T::WTN + frag_row) * L::ROWB;
  constexpr int KS = T::BK / 16;
  bf16x8_t af[2][T::TM], bfr[2][T::TN];
  auto read_frags = [&](int stage, int ks, int slot) {
    const int cofs = ((2 * ks) ^ ysw) * 16;
    const char* a_l = lds + stage * L::STAGE + a_off + cofs;
    const char* b_l = lds + stage * L::STAGE + b_off + cofs;
    af[slot][0] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l));
#pragma unroll
    for (int j = 0; j < T::TN; ++j)
      bfr[slot][j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(b_l + 32 * j * L::ROWB));
#pragma unroll
    for (int i = 1; i < T::TM; ++i)
      af[slot][i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(a_l + 32 * i * L::ROWB));
  };
  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
        acc[i][j] = EPI == kEpiQkv || EPI == kEpiSwiglu  // transposed product for these epilogues
                        ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0)
                        : __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int r = 0; r < T::TM + T::TN; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, T::TM * T::TN - (T::TM + T::TN), 0);
  };
  const RowMeta rm = EPI == kEpiQkv ? qkv_row_meta<T>(p, m0, tid) : RowMeta{0, 0};

  // Two stages.  Tile kt+1's A is requested and its W codes fetched at the
  // top of tile kt; W is dequantised into the other stage after the k-tile's
  // reads of it are done (the previous barrier), before the barrier that ends
  // tile kt, whose fence covers both the direct loads and the LDS writes.
  const int kt_n = p.K / T::BK;
  issue_a(0, 0);
  fetch_w(0);
  stash_w(0);
  __syncthreads();
  read_frags(0, 0, 0);
  int stage = 0;
  for (int kt = 0; kt < kt_n; ++kt) {
    const bool more = kt + 1 < kt_n;
    if (more) {
      issue_a(kt + 1, stage ^ 1);
      fetch_w(kt + 1);
    }
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      read_frags(stage, ks + 1, (ks + 1) & 1);
      mfma_step(ks & 1);
      interleave();
    }
    if (more) stash_w(stage ^ 1);
    __syncthreads();
    if (more) read_frags(stage ^ 1, 0, 0);
    mfma_step((KS - 1) & 1);
    if (more) interleave();
    stage ^= 1;
  }
  static_assert(EPI != kEpiQkv || qkv_lds_bytes<T>() <= L::LDS, "qkv epilogue LDS");
  finish_tile<T, EPI>(p, acc, dyn_lds, rm, m0, n0, wm, wn, lane, tid);
}

// ---------------------------------------------------------------------------
// Persistent kernel for grids of at least two 256 x 256 tiles per CU (the
// gate/up, QKV and speech-head GEMMs): one workgroup per CU walks the tiles
// T = blockIdx.x, blockIdx.x + gridDim.x, ... (row-major, so a workgroup
// keeps its XCD's column tiles of W; QKV in XCD row bands, columns fastest,
// so each A row block is fetched by one XCD), and the first two k-tiles of
// the next tile are requested before the current tile's epilogue, which then
// runs while they are in flight (QKV: after it, as its epilogue stages the
// rows' positions, pages and RoPE columns in LDS).
//
// Four waves, one per SIMD, each 128 x 128 of the tile (accumulators in the
// AGPRs); BK 64 with two LDS stages.  A k-tile is four k-steps of 16 MFMAs;
// each k-step reads the next k-step's fragments into the other register slot.
// Stage s of k-tile kt may be refilled once every wave has read k-step 3's
// fragments of kt (the barrier before k-step 3), so the loads of k-tile kt + 2
// go out half in k-step 3 of kt and half early in k-step 0 of kt + 1, two
// k-steps before the barrier that waits for them.  Against BK 32 with four
// stages (three k-tiles in flight) this halves the barriers and requests each
// operand row as whole 128-byte lines (the L2 requests of a 64-byte half-line
// layout were twice the vendor library's for the same bytes): gate/up 265 ->
// 242 us plain, QKV plain 105 -> 98 us, bit-identical.  Per-wave cycle
// counters showed a burst of direct-to-LDS loads stalling the in-order wave
// that issues it while the same loads spread over MFMAs cost little, and the
// compiler keeps neither such a spread nor loads ahead of a long epilogue on
// its own; so each k-step is written as 16 groups of one MFMA, at most one
// fragment read and at most one load, each fenced with sched_barrier.  The
// MFMA and the K order are those of the other kernels, so a row's result does
// not depend on which kernel runs it.
//
// LDS rows hold BK = 64 bf16 (128 bytes); chunk c of row r sits in slot
// c ^ ((r >> 1) & 7), so the 16 rows one 16-lane group of a fragment read
// touches fill the 16 slots of a 256-byte bank line.  A 1 KB load
// instruction covers 8 rows; lane i fills slot i % 8 of row i / 8.
namespace pt {
constexpr int BM = 256, BN = 256, BK = 64, NS = 2, WAVES = 4, THREADS = 64 * WAVES;
constexpr int TM = 4, TN = 4;  // 32 x 32 MFMA tiles per wave
constexpr int ROWB = BK * 2, CPR = BK / 8, RPI = 64 / CPR;
constexpr int A_BYTES = BM * ROWB, B_BYTES = BN * ROWB, STAGE = A_BYTES + B_BYTES;
constexpr int LA = BM / RPI / WAVES, LB = BN / RPI / WAVES, LPT = LA + LB, HL = LPT / 2;
constexpr int LDS = NS * STAGE;
// The residual epilogue stages the C tile in LDS (rows padded by 16 bytes).
template <int EPI>
constexpr int lds_bytes() {
  return EPI == kEpiResidual && BM * (BN + 8) * 2 > LDS ? BM * (BN + 8) * 2 : LDS;
}
constexpr int NM = TM * TN, NR = TM + TN;
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }
// Stores per lane of one full tile's epilogue (16-byte runs): swiglu 16, plain 32.
template <int EPI>
constexpr int tile_stores() {
  return EPI == kEpiSwiglu ? TM * (TN / 2) * 2 : TM * TN * 2;
}
constexpr int kStoresCap(int n) { return n < 63 ? n : 63; }

// The transposed product leaves lane l and lane l + 32 with the 4-column runs
// 8 r + 0..3 and 8 r + 4..7 of the same token.  Given a lane's runs of r = 2 h
// (even) and 2 h + 1 (odd), v_permlane32_swap returns columns 16 h + 0..7 in
// lanes 0-31 and 16 h + 8..15 in lanes 32-63: one 16-byte store per lane.
__device__ __forceinline__ u32x4_t pair_runs(u32x2_t even, u32x2_t odd) {
  const auto a = __builtin_amdgcn_permlane32_swap(even[0], odd[0], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(even[1], odd[1], false, false);
  return u32x4_t{a[0], b[0], a[1], b[1]};
}

// s_waitcnt vmcnt(N) lgkmcnt(0) + s_barrier, with nothing moved across.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
  __builtin_amdgcn_sched_barrier(0);
}
}  // namespace pt

template <int EPI, int AM>
__global__ __launch_bounds__(pt::THREADS) void gemm_pt_kernel(const GemmParams p) {
  constexpr int BM = pt::BM, BN = pt::BN, BK = pt::BK;
  constexpr int TM = pt::TM, TN = pt::TN, ROWB = pt::ROWB, CPR = pt::CPR, RPI = pt::RPI;
  constexpr int A_BYTES = pt::A_BYTES, STAGE = pt::STAGE, LA = pt::LA, LB = pt::LB, LPT = pt::LPT, HL = pt::HL;
  constexpr int NM = pt::NM, NR = pt::NR;
  using pt::pair_runs;
  using pt::swz;
  static_assert(EPI == kEpiSwiglu || EPI == kEpiStore || EPI == kEpiQkv || EPI == kEpiResidual,
                "persistent kernel epilogues: swiglu, plain store, qkv, residual");
  using TT = Tile<BM, BN, BK, 2, 2>;  // the wave layout, for the shared qkv epilogue
  static_assert(EPI != kEpiQkv || qkv_lds_bytes<TT>() <= pt::LDS, "qkv epilogue LDS");
  extern __shared__ __attribute__((aligned(16))) uint16_t dyn_lds[];
  char* lds = reinterpret_cast<char*>(dyn_lds);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int kt_n = p.K / BK;
  const int ntx = (p.N + BN - 1) / BN, nty = (p.M + BM - 1) / BM;
  const int ntiles = ntx * nty;
  // Tile k of this workgroup.  Row-major: T = blockIdx.x + k * gridDim.x.
  // Bands (QKV, and grids the launcher marks: single-round ones and narrow
  // long-K ones; workgroups go round-robin to the 8 XCDs): XCD x takes row
  // tiles [x R, (x + 1) R), R = nty / 8, walked columns fastest by its
  // workgroups, so each A row block is fetched by one XCD.
  const bool band = (EPI == kEpiQkv || p.xcd_band != 0) && nty % 8 == 0 && gridDim.x % 8 == 0;
  auto tile_at = [&](int k, int& m0, int& n0) {
    if (band) {
      const int g8 = gridDim.x / 8, t = blockIdx.x / 8 + k * g8, rows = nty / 8;
      if (t >= rows * ntx) return false;
      m0 = ((blockIdx.x % 8) * rows + t / ntx) * BM;
      n0 = (t % ntx) * BN;
      return true;
    }
    const int T = blockIdx.x + k * gridDim.x;
    if (T >= ntiles) return false;
    m0 = (T / ntx) * BM;
    n0 = (T % ntx) * BN;
    return true;
  };

  // Load sources: a uniform tile base (SGPRs) plus a 32-bit byte offset per
  // load, which halves the address registers of 64-bit row pointers.  With
  // the token shift, a row reads either the hidden row before it or its
  // block's shift_ctx row: bit 0 of the offset (offsets are multiples of 16)
  // selects the shift_ctx base.
  uint32_t a_ofs[LA], b_ofs[LB];
  const char* a_base = nullptr;
  const char* s_base = nullptr;
  const char* w_base = nullptr;
  auto set_tile = [&](int m0, int n0) {
    if constexpr (AM == kAShift) {
      // relative to hidden row m0 - 1 and to shift_ctx row m0 / bl
      a_base = reinterpret_cast<const char*>(p.A + (static_cast<int64_t>(m0) - 1) * p.lda);
      s_base = reinterpret_cast<const char*>(p.shift_ctx + static_cast<int64_t>(m0 / p.shift_bl) * p.K);
    } else {
      a_base = reinterpret_cast<const char*>(p.A + static_cast<int64_t>(m0) * p.lda);
    }
    w_base = reinterpret_cast<const char*>(p.W + static_cast<int64_t>(n0) * p.ldw);
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int r = (wave * LA + j) * RPI + lane / CPR;
      const int c = (lane % CPR) ^ swz(r);
      const int m = min(m0 + r, p.M - 1);
      if constexpr (AM == kAShift) {
        const int blk = m / p.shift_bl;
        a_ofs[j] = m - blk * p.shift_bl == 0
                       ? static_cast<uint32_t>(((static_cast<int64_t>(blk - m0 / p.shift_bl) * p.K + 8 * c) * 2) | 1)
                       : static_cast<uint32_t>((static_cast<int64_t>(m - m0) * p.lda + 8 * c) * 2);
      } else {
        a_ofs[j] = static_cast<uint32_t>((static_cast<int64_t>(m - m0) * p.lda + 8 * c) * 2);
      }
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int r = (wave * LB + j) * RPI + lane / CPR;
      const int c = (lane % CPR) ^ swz(r);
      b_ofs[j] = static_cast<uint32_t>((static_cast<int64_t>(min(n0 + r, p.N - 1) - n0) * p.ldw + 8 * c) * 2);
    }
  };
  // load j of this wave's LPT for k-tile kt into stage (A loads first)
  auto issue1 = [&](int kt, int stage, int j) {
    const int k = kt * BK;
    if (j < LA) {
      const char* src;
      if constexpr (AM == kAShift) {
        src = ((a_ofs[j] & 1u) ? s_base : a_base) + 2 * k + (a_ofs[j] & ~1u);
      } else {
        src = a_base + 2 * k + a_ofs[j];
      }
      load_lds16(reinterpret_cast<const uint16_t*>(src), lds + stage * STAGE + (wave * LA + j) * 1024);
    } else {
      load_lds16(reinterpret_cast<const uint16_t*>(w_base + 2 * k + b_ofs[j - LA]),
                 lds + stage * STAGE + A_BYTES + (wave * LB + j - LA) * 1024);
    }
  };
  auto prologue = [&]() {
#pragma unroll
    for (int s = 0; s < pt::NS; ++s)
#pragma unroll
      for (int j = 0; j < LPT; ++j) issue1(s, s, j);
  };

  f32x16_t acc[TM][TN];
  const int frag_row = lane & 31;
  const int a_off = (wm * 128 + frag_row) * ROWB;
  const int b_off = A_BYTES + (wn * 128 + frag_row) * ROWB;
  const int fsw = swz(frag_row);  // fragment tiles start at multiples of 32 rows
  bf16x8_t af[2][TM], bfr[2][TN];
  auto frag_rd = [&](int stage, int ks, int slot, int idx) {
    const int cofs = ((2 * ks + (lane >> 5)) ^ fsw) * 16;
    if (idx < TM) {
      af[slot][idx] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(lds + stage * STAGE + a_off + cofs + 32 * idx * ROWB));
    } else {
      bfr[slot][idx - TM] =
          as_bf16x8(*reinterpret_cast<const u32x4_t*>(lds + stage * STAGE + b_off + cofs + 32 * (idx - TM) * ROWB));
    }
  };
  // One k-step: the MFMAs on fragment slot `slot`; with rd the fragments of
  // k-step rks of stage rstage into the other slot; with nl > 0 the loads
  // lj0 .. lj0 + nl - 1 of k-tile lkt into stage lstage, one after every
  // NM / nl MFMAs.  The register epilogues (swiglu, plain, qkv) use the
  // transposed product (W x A^T: a lane holds one token and 4-column runs);
  // the residual epilogue, staged through LDS, the direct one.
  auto kstep = [&](int slot, bool rd, int rstage, int rks, int nl, int lkt, int lstage, int lj0) {
#pragma unroll
    for (int r = 0; r < NM; ++r) {
      const int i = r % TM, j = r / TM;
      acc[i][j] = EPI == kEpiResidual
                      ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[slot][i], bfr[slot][j], acc[i][j], 0, 0, 0)
                      : __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[slot][j], af[slot][i], acc[i][j], 0, 0, 0);
      if (rd && r < NR) frag_rd(rstage, rks, slot ^ 1, r);
      if (nl > 0 && r % (NM / nl) == NM / nl - 1) issue1(lkt, lstage, lj0 + r / (NM / nl));
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  const int tok = lane & 31;
  const bool vec_ok = (p.ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15u) == 0);
  int m0 = 0, n0 = 0;
  if (tile_at(0, m0, n0)) {
    set_tile(m0, n0);
    prologue();
  }
  // Stores the previous tile's epilogue surely issued after this tile's
  // prologue (0 for the first tile, after a partial tile, and for QKV).
  bool after_full = false;
  for (int kti = 0; tile_at(kti, m0, n0); ++kti) {
    // qkv: this tile's row positions and pages, loaded while the k-loop runs
    const RowMeta rm = EPI == kEpiQkv ? qkv_row_meta<TT>(p, m0, tid) : RowMeta{0, 0};
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    // k-tile 0 has landed: k-tile 1 (and the stores of a full previous
    // epilogue, issued after it) may stay in flight
    if (after_full) {
      pt::stage_barrier<pt::kStoresCap(LPT + pt::tile_stores<EPI>())>();
    } else {
      pt::stage_barrier<LPT>();
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) frag_rd(0, 0, 0, r);
    // k-tile 0 (k-tile 1 came with the prologue)
    kstep(0, true, 0, 1, 0, 0, 0, 0);
    kstep(1, true, 0, 2, 0, 0, 0, 0);
    kstep(0, true, 0, 3, 0, 0, 0, 0);
    // k-tile 1 has landed (the stores may stay in flight); stage 0 is free
    if (after_full) {
      pt::stage_barrier<pt::kStoresCap(pt::tile_stores<EPI>())>();
    } else {
      pt::stage_barrier<0>();
    }
    kstep(1, true, 1, 0, kt_n > 2 ? HL : 0, 2, 0, 0);
    int kt = 1;
    for (; kt + 1 < kt_n; ++kt) {
      const int s = kt & 1;
      // the other half of k-tile kt + 1's loads, two k-steps ahead of the barrier
      kstep(0, true, s, 1, LPT - HL, kt + 1, s ^ 1, HL);
      kstep(1, true, s, 2, 0, 0, 0, 0);
      kstep(0, true, s, 3, 0, 0, 0, 0);
      // k-tile kt + 1 has landed and every wave has read stage s
      pt::stage_barrier<0>();
      kstep(1, true, s ^ 1, 0, kt + 2 < kt_n ? HL : 0, kt + 2, s, 0);
    }
    // the last k-tile
    kstep(0, true, kt & 1, 1, 0, 0, 0, 0);
    kstep(1, true, kt & 1, 2, 0, 0, 0, 0);
    kstep(0, true, kt & 1, 3, 0, 0, 0, 0);
    pt::stage_barrier<0>();
    // No LDS read is left in this tile: request the next tile's first
    // k-tiles, kept ahead of the epilogue so they land while it runs.
    int m1 = 0, n1 = 0;
    const bool next = tile_at(kti + 1, m1, n1);
    if constexpr (EPI == kEpiQkv || EPI == kEpiResidual) {
      // epilogues that use LDS: the next tile's loads follow them
      kstep(1, false, 0, 0, 0, 0, 0, 0);
      // The epilogue's addresses depend only on the thread; computed from
      // these opaque copies they stay here instead of being hoisted out of
      // the tile loop and held (spilled) across the k-loop.
      int tid_e = tid, lane_e = lane;
      asm volatile("" : "+v"(tid_e), "+v"(lane_e));
      finish_tile<TT, EPI>(p, acc, dyn_lds, rm, m0, n0, wm, wn, lane_e, tid_e);
      __syncthreads();  // the epilogue's LDS reads are done before the next tile's loads land there
      if (next) {
        set_tile(m1, n1);
        prologue();
      }
      continue;
    }
    if (next) {
      set_tile(m1, n1);
      prologue();
    }
    __builtin_amdgcn_sched_barrier(0);
    kstep(1, false, 0, 0, 0, 0, 0, 0);

    const bool full = m0 + BM <= p.M && n0 + BN <= p.N && vec_ok;
    after_full = full;
    // 8 bf16 (columns c .. c + 7 after pair_runs) of a row, bounded by n_end
    auto put8 = [&](uint16_t* row, int c, int n_end, const u32x4_t& v) {
      if (vec_ok && c + 8 <= n_end) {
        *reinterpret_cast<u32x4_t*>(row + c) = v;
      } else {
        for (int t = 0; t < 8 && c + t < n_end; ++t) row[c + t] = static_cast<uint16_t>(v[t >> 1] >> (16 * (t & 1)));
      }
    };
    if constexpr (EPI == kEpiSwiglu) {
      // Lane: token (lane & 31) of each 32-row block; tiles j = 2 q2, 2 q2 + 1
      // are gate and up of 32 features (interleaved W rows).  Roundings as
      // the reference's separate ops: g and u to bf16, silu(g) to bf16, the
      // product to bf16; silu with the hardware reciprocal.
      const int F = p.N / 2;
      auto silu_mul = [](float g0, float g1, float u0, float u1) {
        const uint32_t gp = pack_bf16x2(g0, g1), up = pack_bf16x2(u0, u1);
        const float gb0 = bf16lo(gp), gb1 = bf16hi(gp);
        const uint32_t sp = pack_bf16x2(gb0 * __builtin_amdgcn_rcpf(1.f + __expf(-gb0)),
                                        gb1 * __builtin_amdgcn_rcpf(1.f + __expf(-gb1)));
        return pack_bf16x2(bf16lo(sp) * bf16lo(up), bf16hi(sp) * bf16hi(up));
      };
      auto run = [&](const f32x16_t& g, const f32x16_t& u, int e) {
        return u32x2_t{silu_mul(g[e], g[e + 1], u[e], u[e + 1]), silu_mul(g[e + 2], g[e + 3], u[e + 2], u[e + 3])};
      };
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * 128 + 32 * i + tok;  // lanes l and l + 32: the same token
        if (m >= p.M) continue;
        uint16_t* const row = p.C + static_cast<int64_t>(m) * p.ldc;
#pragma unroll
        for (int q2 = 0; q2 < TN / 2; ++q2) {
          const int fb = (n0 + wn * 128 + 64 * q2) / 2;
          if (fb >= F) continue;  // F % 64 == 0: a group is all in or all out
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4_t v = pair_runs(run(acc[i][2 * q2], acc[i][2 * q2 + 1], 8 * h),
                                        run(acc[i][2 * q2], acc[i][2 * q2 + 1], 8 * h + 4));
            put8(row, fb + 16 * h + 8 * (lane >> 5), F, v);
          }
        }
      }
    } else {
      // Plain bf16 store of the wave's 128 x 128: token (lane & 31), columns 32 j + 16 h + 8 (lane >> 5) ..
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * 128 + 32 * i + tok;
        if (m >= p.M) continue;
        uint16_t* const row = p.C + static_cast<int64_t>(m) * p.ldc;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int e = 8 * h;
            const u32x2_t lo = {pack_bf16x2(acc[i][j][e], acc[i][j][e + 1]), pack_bf16x2(acc[i][j][e + 2], acc[i][j][e + 3])};
            const u32x2_t hi = {pack_bf16x2(acc[i][j][e + 4], acc[i][j][e + 5]),
                                pack_bf16x2(acc[i][j][e + 6], acc[i][j][e + 7])};
            put8(row, n0 + wn * 128 + 32 * j + 16 * h + 8 * (lane >> 5), p.N, pair_runs(lo, hi));
          }
        }
      }
    }
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

// Two rows per wave; D = 1024 -> 16 bf16 per lane and row (two 16-byte chunks).  All of a
// wave's loads (both rows and the gain) are requested before the first reduction: one row per
// wave with the gain read after the reduction took 12.1 us at 16384 x 1024 against 11.3 us
// (four rows per wave: 12.35 us), bit-identical.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const NormParams p) {
  constexpr int kRows = 2;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows;
  const int lane = threadIdx.x & 63;
  if (row0 >= p.M) return;
  constexpr int kMaxChunks = 4;  // D <= 2048
  const int nch = p.D / (64 * 8);
  u32x4_t wv[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c)
    if (c < nch) wv[c] = ldg16(p.w + (c * 64 + lane) * 8);
  u32x4_t xv[kRows][kMaxChunks];
  float ss[kRows];
#pragma unroll
  for (int rr = 0; rr < kRows; ++rr) {
    ss[rr] = 0.f;
    const int row = min(row0 + rr, p.M - 1);
    const int64_t base = static_cast<int64_t>(row) * p.D;
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
        if (row0 + rr < p.M) *reinterpret_cast<u32x4_t*>(p.residual + off) = x;
      } else {
        x = ldg16(p.x + off);
        if (p.residual && row0 + rr < p.M) *reinterpret_cast<u32x4_t*>(p.residual + off) = x;
      }
      xv[rr][c] = x;
    }
  }
#pragma unroll
  for (int rr = 0; rr < kRows; ++rr) {
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (c >= nch) break;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = bf16lo(xv[rr][c][w]), b = bf16hi(xv[rr][c][w]);
        ss[rr] += a * a + b * b;
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < kRows; ++rr) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss[rr] += __shfl_xor(ss[rr], o, 64);
  }
#pragma unroll
  for (int rr = 0; rr < kRows; ++rr) {
    if (row0 + rr >= p.M) break;
    const float rs = rsqrtf(ss[rr] / static_cast<float>(p.D) + p.eps);
    const int64_t base = static_cast<int64_t>(row0 + rr) * p.D;
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      if (c >= nch) break;
      const int64_t off = base + (c * 64 + lane) * 8;
      u32x4_t y;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = bf16lo(wv[c][w]) * round_bf16(bf16lo(xv[rr][c][w]) * rs);
        const float b = bf16hi(wv[c][w]) * round_bf16(bf16hi(xv[rr][c][w]) * rs);
        y[w] = pack_bf16x2(a, b);
      }
      *reinterpret_cast<u32x4_t*>(p.out + off) = y;
    }
  }
}

bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

using TileS = Tile<128, 128, BK, 2, 2>;  // small M: more workgroups

template <class T, int EPI, int AM, int BQ>
int launch_tile(const GemmParams& p, hipStream_t st) {
  const dim3 grid((p.N + T::BN - 1) / T::BN, (p.M + T::BM - 1) / T::BM), block(T::THREADS);
  hipLaunchKernelGGL((gemm_kernel<T, EPI, AM, BQ>), grid, block, 0, st, p);
  YAPD_LAUNCH_CHECK("gemm_kernel launch");
  return YAPD_OK;
}

template <class T, int EPI, int AM, int NS = 2>
int launch_dl(const GemmParams& p, hipStream_t st) {
  using L = DlLayout<T, NS>;
  // The dynamic-LDS limit is raised once per kernel and device (setting it
  // twice, e.g. from two threads, is harmless).
  static bool lds_set[64] = {false};
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= 64 || !lds_set[dev]) {
    if (int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dl_kernel<T, EPI, AM, NS>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, L::LDS),
                           "gemm_dl_kernel LDS attribute"))
      return rc;
    if (dev >= 0 && dev < 64) lds_set[dev] = true;
  }
  const dim3 grid((p.N + T::BN - 1) / T::BN, (p.M + T::BM - 1) / T::BM), block(T::THREADS);
  hipLaunchKernelGGL((gemm_dl_kernel<T, EPI, AM, NS>), grid, block, L::LDS, st, p);
  YAPD_LAUNCH_CHECK("gemm_dl_kernel launch");
  return YAPD_OK;
}

using TileD = Tile<256, 256, BK, 2, 4>;  // direct-load large tile
using TileM = Tile<128, 128, BK, 4, 2>;  // direct-load mid tile: 8 waves of 32 x 64

template <class T, int EPI, int AM, int BQ>
int launch_dlq(const GemmParams& p, hipStream_t st) {
  using L = DlLayout<T, 2>;
  static bool lds_set[64] = {false};
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= 64 || !lds_set[dev]) {
    if (int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dlq_kernel<T, EPI, AM, BQ>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, L::LDS),
                           "gemm_dlq_kernel LDS attribute"))
      return rc;
    if (dev >= 0 && dev < 64) lds_set[dev] = true;
  }
  const dim3 grid((p.N + T::BN - 1) / T::BN, (p.M + T::BM - 1) / T::BM), block(T::THREADS);
  hipLaunchKernelGGL((gemm_dlq_kernel<T, EPI, AM, BQ>), grid, block, L::LDS, st, p);
  YAPD_LAUNCH_CHECK("gemm_dlq_kernel launch");
  return YAPD_OK;
}

using TileW = Tile<64, 64, BK, 1, 1>;     // direct-load one-wave tile (small batches)

// The persistent kernel: one workgroup per CU (fewer when there are fewer tiles).
template <int EPI, int AM>
int launch_pt(const GemmParams& p, hipStream_t st, int cus) {
  static bool lds_set[64] = {false};
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= 64 || !lds_set[dev]) {
    if (int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_pt_kernel<EPI, AM>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, pt::lds_bytes<EPI>()),
                           "gemm_pt_kernel LDS attribute"))
      return rc;
    if (dev >= 0 && dev < 64) lds_set[dev] = true;
  }
  const int64_t tiles = static_cast<int64_t>((p.M + pt::BM - 1) / pt::BM) * ((p.N + pt::BN - 1) / pt::BN);
  const int grid = static_cast<int>(tiles < cus ? tiles : cus);
  hipLaunchKernelGGL((gemm_pt_kernel<EPI, AM>), dim3(grid), dim3(pt::THREADS), pt::lds_bytes<EPI>(), st, p);
  YAPD_LAUNCH_CHECK("gemm_pt_kernel launch");
  return YAPD_OK;
}

// Compute units of the current device (cached per device id).
int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int EPI, int AM, int BQ = 0>
int launch_gemm(GemmParams p, hipStream_t st) {
  // Large tiles once they fill three quarters of the CUs (direct-load kernel;
  // measured at M = 4096: QKV 37.6 -> 33.4 us with 192 tiles, while at 128
  // tiles the 128 x 128 kernel is still faster) or, for the quantised path,
  // once they give one workgroup per CU.
  const int64_t big_tiles = static_cast<int64_t>((p.M + 255) / 256) * ((p.N + 255) / 256);
  // bf16 W and at least two tiles per CU, or for the plain and residual
  // epilogues at least one: the persistent kernel, which overlaps each tile's
  // epilogue with the next tile's first loads where the epilogue works from
  // registers (gate/up + SiLU at M = 16384: 318 -> 266 us on one box,
  // bit-identical; the speech head likewise).  On single-round grids its XCD
  // bands beat the 8-wave kernel's (plain down at M = 16384: 124.2 -> 112.8 us,
  // o 36.3 -> 34.9 us, bit-identical).  Banded: single-round grids and, for
  // the residual epilogue, narrow long-K ones (down at M > 16384, as below).
  if constexpr (BQ == 0 && (EPI == kEpiSwiglu || EPI == kEpiStore || EPI == kEpiQkv || EPI == kEpiResidual)) {
    const int64_t min_tiles = EPI == kEpiStore || EPI == kEpiResidual ? cu_count() : 2 * cu_count();
    if (big_tiles >= min_tiles && p.K >= pt::BK * pt::NS && p.K % pt::BK == 0) {
      const bool narrow_long = (p.N + 255) / 256 <= 8 && p.K >= 2048;
      p.xcd_band = big_tiles <= cu_count() || (EPI == kEpiResidual && narrow_long) ? 1 : 0;
      if constexpr (EPI == kEpiStore) {
        // the head's last 2 columns (N = 8194) as below: their own one-wave launch
        const int tail = p.N % 256;
        if (tail != 0 && tail <= 64) {
          GemmParams rest = p;
          p.N -= tail;
          rest.W = p.W + static_cast<int64_t>(p.N) * p.ldw;
          rest.C = p.C + p.N;
          rest.N = tail;
          rest.xcd_band = (p.M + 63) / 64 <= cu_count() ? 1 : 0;
          if (int rc = launch_pt<EPI, AM>(p, st, cu_count())) return rc;
          return launch_dl<TileW, EPI, AM, 3>(rest, st);
        }
      }
      return launch_pt<EPI, AM>(p, st, cu_count());
    }
  }
  if (big_tiles >= (BQ == 0 ? cu_count() * 3 / 4 : cu_count())) {
    // banded orders: single-round grids; multi-round grids with few column
    // tiles and a long K (down at M > 16384: 336 -> 276 us at M = 32768,
    // 263 -> 244 us at M = 24576; o with K = 1024 measured 90 -> 96 us at
    // M = 32768 and keeps the row-major order), and QKV's 12 column tiles
    // (step 22.71 -> 22.64 ms in three alternating pairs on one box; the
    // rows-fastest band order measured 23.17 ms there)
    const bool band2 = ((p.N + 255) / 256 <= 8 && p.K >= 2048) || EPI == kEpiQkv;
    p.xcd_band = big_tiles <= cu_count() ? 1 : band2 ? 2 : 0;
    if constexpr (BQ == 0) {
      if constexpr (EPI == kEpiStore) {
        // A last column tile of at most 64 columns that would add a round of
        // 256 x 256 tiles (the speech head: N = 8194 = 32 x 256 + 2, 2112
        // tiles) goes to a second launch on one-wave 64 x 64 tiles.  Every
        // element keeps the same MFMA and K order, so the output is the same.
        const int64_t row_tiles = (p.M + 255) / 256, cols = p.N / 256, cus = cu_count();
        const int tail = p.N % 256;
        if (cols >= 1 && tail != 0 && tail <= 64 &&
            (row_tiles * (cols + 1) + cus - 1) / cus > (row_tiles * cols + cus - 1) / cus) {
          GemmParams rest = p;
          p.N = static_cast<int>(cols * 256);
          p.xcd_band = row_tiles * cols <= cus ? 1 : 0;
          rest.W = p.W + static_cast<int64_t>(p.N) * p.ldw;
          rest.C = p.C + p.N;
          rest.N = tail;
          rest.xcd_band = (p.M + 63) / 64 <= cus ? 1 : 0;
          if (int rc = launch_dl<TileD, EPI, AM>(p, st)) return rc;
          return launch_dl<TileW, EPI, AM, 3>(rest, st);
        }
      }
      return launch_dl<TileD, EPI, AM>(p, st);
    } else {
      return launch_dlq<TileD, EPI, AM, BQ>(p, st);
    }
  }
  // Few tiles (small batches): one-wave 64 x 64 direct-load tiles with two
  // k-tiles in flight, while they give at most two workgroups per CU
  // (measured down at M = 256..2048: 46-51 -> 36-41 us; beyond that the
  // 128 x 128 kernel is faster).
  if constexpr (BQ == 0) {
    const int64_t wave_tiles = static_cast<int64_t>((p.M + 63) / 64) * ((p.N + 63) / 64);
    if (wave_tiles <= 2 * cu_count()) {
      p.xcd_band = wave_tiles <= cu_count() ? 1 : 0;
      return launch_dl<TileW, EPI, AM, 3>(p, st);
    }
  }
  // In between, 128 x 128 tiles: the direct-load kernel with 8 waves of 32 x 64
  // (measured against the register-staged 128 x 128 kernel, same session,
  // bit-identical: o 18.5 -> 16.9 us and down 53.4 -> 50.4 us at M = 4096,
  // down 72.9 -> 62.5 us at M = 6144); the quantised path keeps the
  // register-staged kernel, which dequantises W on its way into LDS.  With at
  // most one tile per CU a k-tile is too short to cover the load latency, so
  // three stages keep two tiles in flight (o 16.8 -> 14.3-14.9 us, down
  // 50.3-51.1 -> 41.0-42.9 us at M = 2304-4096, bit-identical); with more
  // tiles two stages let two workgroups share a CU, which measured faster
  // (down 61 vs 83 us at M = 6144).
  const int64_t small_tiles = static_cast<int64_t>((p.M + 127) / 128) * ((p.N + 127) / 128);
  p.xcd_band = small_tiles <= cu_count() ? 1 : 0;
  if constexpr (BQ == 0) {
    if (small_tiles <= cu_count()) return launch_dl<TileM, EPI, AM, 3>(p, st);
    return launch_dl<TileM, EPI, AM>(p, st);
  } else {
    // Quantised W: the direct-load kernel on 128 x 128 tiles while the grid
    // has at most one tile per CU (M = 256-4096, bit-identical: down 4-bit
    // 58.1 -> 44.7 us at M = 256, 78.0 -> 72.5 us at M = 4096); larger grids
    // keep the register-staged kernel (o at M = 8192: 29.3 vs 32.5 us).
    if (small_tiles <= cu_count()) return launch_dlq<TileM, EPI, AM, BQ>(p, st);
    return launch_tile<TileS, EPI, AM, BQ>(p, st);
  }
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

extern "C" int yapd_gemm_bf16_residual(const void* A, int64_t lda, const void* W, int64_t ldw, int M, int N, int K,
                                       void* residual, int64_t ld_res, void* stream) {
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.W = static_cast<const uint16_t*>(W);
  p.ldw = ldw;
  p.M = M;
  p.N = N;
  p.K = K;
  p.C = static_cast<uint16_t*>(residual);
  p.ldc = ld_res;
  if (int rc = yapd::check_common(p)) return rc;
  YAPD_REQUIRE(residual != nullptr && ld_res >= N, "gemm_residual: bad residual");
  return yapd::launch_gemm<yapd::kEpiResidual, yapd::kAPlain>(p, static_cast<hipStream_t>(stream));
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

namespace yapd {
namespace {
// Parameters and argument checks of the QKV + RoPE + KV-write GEMM (nothing launched).
// With q != nullptr the weight is quantised (W_qkv unused).
int qkv_params(GemmParams& p, const void* A, int64_t lda, const void* W_qkv, int M, int K, int n_heads,
               const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int bl, void* q_out,
               void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride, int table_cols,
               const QWeight* q = nullptr) {
  p = GemmParams{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  if (q != nullptr) {
    p.Wq = q->packed;
    p.ldq = static_cast<int64_t>(K) * q->bits / 32;
    p.qscale = q->scales;
    p.qbias = q->biases;
  } else {
    p.W = static_cast<const uint16_t*>(W_qkv);
  }
  p.ldw = K;
  p.M = M;
  p.N = 3 * n_heads * kHeadDim;
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
  if (int rc = check_common(p)) return rc;
  YAPD_REQUIRE(cos_t && sin_t && pos0 && q_out && kv_pool && page_table, "gemm_qkv: NULL pointer");
  YAPD_REQUIRE(al16(cos_t) && al16(sin_t) && (reinterpret_cast<uintptr_t>(q_out) & 7u) == 0 &&
                   (reinterpret_cast<uintptr_t>(kv_pool) & 7u) == 0,
               "gemm_qkv: cos/sin must be 16-byte aligned, q_out and kv_pool 8-byte aligned");
  YAPD_REQUIRE(max_pos >= 1 && bl >= 1 && M % bl == 0 && n_heads >= 1 && n_pages >= 1 && n_pages <= INT32_MAX &&
                   table_cols >= 1 && table_stride >= table_cols,
               "gemm_qkv: bad positions / table shape");
  return YAPD_OK;
}

int rmsnorm_checks(const void* delta, const void* residual, const void* x, const void* w, int M, int D,
                   const void* out) {
  YAPD_REQUIRE(w && out && M >= 1, "rmsnorm: NULL pointer or empty");
  YAPD_REQUIRE(D % 512 == 0 && D <= 2048, "rmsnorm: D must be a multiple of 512 and <= 2048 (got %d)", D);
  YAPD_REQUIRE(delta ? (residual != nullptr) : (x != nullptr), "rmsnorm: need (delta, residual) or x");
  YAPD_REQUIRE(!(delta && x), "rmsnorm: pass either delta (residual add) or x, not both");
  return YAPD_OK;
}

int rmsnorm_launch(const void* delta, void* residual, const void* x, const void* w, float eps, int M, int D,
                   void* out, hipStream_t st) {
  NormParams p{static_cast<const uint16_t*>(delta), static_cast<uint16_t*>(residual), static_cast<const uint16_t*>(x),
               static_cast<const uint16_t*>(w), eps, M, D, static_cast<uint16_t*>(out)};
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((M + 7) / 8), dim3(256), 0, st, p);
  YAPD_LAUNCH_CHECK("rmsnorm_kernel launch");
  return YAPD_OK;
}
}  // namespace

// The QKV + RoPE + KV-write GEMM over packed rows (declared in packed.h).
int gemm_qkv_rope_kv_packed(const void* A, int64_t lda, const void* W_qkv, int n_tokens, int K, int n_heads,
                            const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int rows,
                            const int32_t* row_start, const int32_t* tok_row, void* q_out, void* kv_pool,
                            int64_t n_pages, const int32_t* page_table, int table_stride, int table_cols,
                            hipStream_t stream) {
  YAPD_REQUIRE(row_start && tok_row && rows >= 1, "gemm_qkv packed: NULL row map or no rows");
  GemmParams p;
  if (int rc = qkv_params(p, A, lda, W_qkv, n_tokens, K, n_heads, cos_t, sin_t, max_pos, pos0, 1, q_out, kv_pool,
                          n_pages, page_table, table_stride, table_cols))
    return rc;
  p.tok_row = tok_row;
  p.row_start = row_start;
  p.n_rows = rows;
  return launch_gemm<kEpiQkv, kAPlain>(p, stream);
}

int qweight_checks(const QWeight& w, int N, int K, const char* what) {
  YAPD_REQUIRE(w.bits == 4 || w.bits == 8, "%s: bits must be 4 or 8 (got %d)", what, w.bits);
  YAPD_REQUIRE(w.packed && w.scales && w.biases, "%s: NULL quantised weight", what);
  YAPD_REQUIRE(al16(w.packed), "%s: packed weights must be 16-byte aligned", what);
  YAPD_REQUIRE(N >= 1 && K >= BK && K % BK == 0, "%s: need N >= 1 and K %% %d == 0", what, BK);
  return YAPD_OK;
}

namespace {
// GemmParams of a quantised projection (A, M, N, K, C set by the caller).
void set_q(GemmParams& p, const QWeight& w, int K) {
  p.Wq = w.packed;
  p.ldq = static_cast<int64_t>(K) * w.bits / 32;
  p.qscale = w.scales;
  p.qbias = w.biases;
}

template <int EPI>
int launch_q(const GemmParams& p, int bits, hipStream_t st) {
  return bits == 4 ? launch_gemm<EPI, kAPlain, 4>(p, st) : launch_gemm<EPI, kAPlain, 8>(p, st);
}
}  // namespace

int qgemm_residual(const void* A, int64_t lda, const QWeight& w, int M, int N, int K, void* residual, int64_t ld_res,
                   hipStream_t stream) {
  if (int rc = qweight_checks(w, N, K, "qgemm_residual")) return rc;
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.M = M;
  p.N = N;
  p.K = K;
  p.C = static_cast<uint16_t*>(residual);
  p.ldc = ld_res;
  set_q(p, w, K);
  if (int rc = check_common(p)) return rc;
  YAPD_REQUIRE(residual != nullptr && ld_res >= N, "qgemm_residual: bad residual");
  return launch_q<kEpiResidual>(p, w.bits, stream);
}

int qgemm_swiglu(const void* A, int64_t lda, const QWeight& w, int M, int F, int K, void* act, int64_t ld_act,
                 hipStream_t stream) {
  if (int rc = qweight_checks(w, 2 * F, K, "qgemm_swiglu")) return rc;
  GemmParams p{};
  p.A = static_cast<const uint16_t*>(A);
  p.lda = lda;
  p.M = M;
  p.N = 2 * F;
  p.K = K;
  p.C = static_cast<uint16_t*>(act);
  p.ldc = ld_act;
  set_q(p, w, K);
  if (int rc = check_common(p)) return rc;
  YAPD_REQUIRE(act && F % 64 == 0 && ld_act >= F, "qgemm_swiglu: F must be a multiple of 64");
  return launch_q<kEpiSwiglu>(p, w.bits, stream);
}

int qgemm_qkv_rope_kv(const void* A, int64_t lda, const QWeight& w, int M, int K, int n_heads, const float* cos_t,
                      const float* sin_t, int max_pos, const int32_t* pos0, int bl, int rows, const int32_t* row_start,
                      const int32_t* tok_row, void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table,
                      int table_stride, int table_cols, hipStream_t stream) {
  if (int rc = qweight_checks(w, 3 * n_heads * kHeadDim, K, "qgemm_qkv")) return rc;
  const bool packed = row_start != nullptr;
  YAPD_REQUIRE(!packed || (tok_row && rows >= 1), "qgemm_qkv packed: NULL row map or no rows");
  GemmParams p;
  if (int rc = qkv_params(p, A, lda, nullptr, M, K, n_heads, cos_t, sin_t, max_pos, pos0, packed ? 1 : bl, q_out,
                          kv_pool, n_pages, page_table, table_stride, table_cols, &w))
    return rc;
  if (packed) {
    p.tok_row = tok_row;
    p.row_start = row_start;
    p.n_rows = rows;
  }
  return launch_q<kEpiQkv>(p, w.bits, stream);
}

namespace {
// Dequantisation of up to four weights in one launch: each thread turns the
// 8 codes of one 16-byte output chunk into bf16(scale * q + bias) with the
// arithmetic of the fused kernels' W loader (dq_pair), so a GEMM on the
// result equals the fused quantised GEMM bit for bit.
struct DqJob {
  const uint32_t* packed;
  const uint16_t* scales;
  const uint16_t* biases;
  uint16_t* out;       // bf16 [N, K], row pitch K
  int N, K;
  int64_t chunk0;      // first 16-byte output chunk of this job in the launch
};
struct DqParams {
  DqJob job[kMaxDqJobs];
  int n_jobs;
  int64_t chunks;      // all jobs' chunks
};

template <int BITS>
__global__ __launch_bounds__(256) void dequant_affine_kernel(const DqParams p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= p.chunks) return;
  int j = 0;
#pragma unroll
  for (int i = 1; i < kMaxDqJobs; ++i)
    if (i < p.n_jobs && t >= p.job[i].chunk0) j = i;
  const DqJob& q = p.job[j];
  const int64_t c = t - q.chunk0;
  const int cpr = q.K / 8;  // chunks per row
  const int n = static_cast<int>(c / cpr), k0 = static_cast<int>(c % cpr) * 8;
  const float sc = f16_to_f32(q.scales[static_cast<int64_t>(n) * (q.K / 64) + k0 / 64]);
  const float bi = f16_to_f32(q.biases[static_cast<int64_t>(n) * (q.K / 64) + k0 / 64]);
  const uint32_t* row = q.packed + static_cast<int64_t>(n) * (q.K * BITS / 32);
  u32x4_t v;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int first = k0 + 2 * h;  // code index in the row
    v[h] = dq_pair<BITS>(row[first * BITS / 32], (first * BITS) % 32, sc, bi);
  }
  *reinterpret_cast<u32x4_t*>(q.out + static_cast<int64_t>(n) * q.K + k0) = v;
}
}  // namespace

int dequant_affine(const QWeight* w, const int* N, const int* K, uint16_t* const* out, int n, hipStream_t stream) {
  YAPD_REQUIRE(n >= 1 && n <= kMaxDqJobs, "dequant_affine: 1 to %d weights per launch (got %d)", kMaxDqJobs, n);
  DqParams p{};
  int64_t chunks = 0;
  for (int i = 0; i < n; ++i) {
    if (int rc = qweight_checks(w[i], N[i], K[i], "dequant_affine")) return rc;
    YAPD_REQUIRE(w[i].bits == w[0].bits, "dequant_affine: one bit width per launch");
    YAPD_REQUIRE(out[i] && (reinterpret_cast<uintptr_t>(out[i]) & 15u) == 0,
                 "dequant_affine: outputs must be non-NULL and 16-byte aligned");
    p.job[i] = DqJob{w[i].packed, w[i].scales, w[i].biases, out[i], N[i], K[i], chunks};
    chunks += static_cast<int64_t>(N[i]) * K[i] / 8;
  }
  p.n_jobs = n;
  p.chunks = chunks;
  const int64_t blocks = (chunks + 255) / 256;
  YAPD_REQUIRE(blocks <= INT32_MAX, "dequant_affine: weights too large");
  if (w[0].bits == 4) {
    hipLaunchKernelGGL(dequant_affine_kernel<4>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  } else {
    hipLaunchKernelGGL(dequant_affine_kernel<8>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p);
  }
  YAPD_LAUNCH_CHECK("dequant_affine_kernel launch");
  return YAPD_OK;
}

}  // namespace yapd

extern "C" int yapd_gemm_qkv_rope_kv(const void* A, int64_t lda, const void* W_qkv, int M, int K, int n_heads,
                                     const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int bl,
                                     void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table,
                                     int table_stride, int table_cols, void* stream) {
  yapd::GemmParams p;
  if (int rc = yapd::qkv_params(p, A, lda, W_qkv, M, K, n_heads, cos_t, sin_t, max_pos, pos0, bl, q_out, kv_pool,
                                n_pages, page_table, table_stride, table_cols))
    return rc;
  return yapd::launch_gemm<yapd::kEpiQkv, yapd::kAPlain>(p, static_cast<hipStream_t>(stream));
}

extern "C" int yapd_gemm_rmsnorm_qkv_rope_kv(const void* x, const void* ln_w, float eps, void* normed,
                                             const void* W_qkv, int M, int K, int n_heads, const float* cos_t,
                                             const float* sin_t, int max_pos, const int32_t* pos0, int bl,
                                             void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table,
                                             int table_stride, int table_cols, void* stream) {
  // Every argument of both launches is checked before the first one starts.
  if (int rc = yapd::rmsnorm_checks(nullptr, nullptr, x, ln_w, M, K, normed)) return rc;
  yapd::GemmParams p;
  if (int rc = yapd::qkv_params(p, normed, K, W_qkv, M, K, n_heads, cos_t, sin_t, max_pos, pos0, bl, q_out, kv_pool,
                                n_pages, page_table, table_stride, table_cols))
    return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (int rc = yapd::rmsnorm_launch(nullptr, nullptr, x, ln_w, eps, M, K, normed, st)) return rc;
  return yapd::launch_gemm<yapd::kEpiQkv, yapd::kAPlain>(p, st);
}

extern "C" int yapd_rmsnorm(const void* delta, void* residual, const void* x, const void* w, float eps, int M, int D,
                            void* out, void* stream) {
  if (int rc = yapd::rmsnorm_checks(delta, residual, x, w, M, D, out)) return rc;
  return yapd::rmsnorm_launch(delta, residual, x, w, eps, M, D, out, static_cast<hipStream_t>(stream));
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

extern "C" int yapd_dequant_affine(const uint32_t* w_packed, const void* scales, const void* biases, int bits,
                                   int group_size, int N, int K, void* W_out, void* stream) {
  YAPD_REQUIRE(group_size == 64, "dequant_affine: group_size must be 64 (got %d)", group_size);
  const yapd::QWeight w{w_packed, static_cast<const uint16_t*>(scales), static_cast<const uint16_t*>(biases), bits};
  uint16_t* out = static_cast<uint16_t*>(W_out);
  return yapd::dequant_affine(&w, &N, &K, &out, 1, static_cast<hipStream_t>(stream));
}
