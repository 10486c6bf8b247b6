// (a) Paged-KV block attention for the block-diffusion step.
//
// Every query of a row's current block attends to all kv_len = cache_start +
// bl keys of that row: the committed prefix plus the whole block,
// bidirectionally (engines/flashinfer.py:884-886 plans causal=False;
// engines/torch_sdpa.py:299-307 uses a zero mask).  The block's own K/V are
// already in the pool (written by the QKV epilogue or yapd_kv_write).
//
// Work decomposition: a workgroup of four waves serves one (row, key range)
// work item for four heads, one head per wave, so a workgroup streams
// 4 heads x (2 KiB K + 2 KiB V) contiguous bytes per page.  The H / 4
// workgroups of one item are consecutive in the 1-D grid: they are dispatched
// together and read the neighbouring 8 KiB runs of the same pages at about
// the same time (measured 170 -> 164 us per layer at 512 rows x 32 against a
// 2-D grid whose head groups of one item were a whole grid row apart).  Per 32-key chunk a
// wave computes S^T = K Q^T (v_mfma_f32_16x16x32_bf16, M = keys, N = 16
// queries) and O^T += V^T P^T (M = head dim, N = queries): with the
// transposed products every lane owns one query, so the online-softmax
// statistics and the O^T accumulator need no lane shuffles except the
// 4-lane-group row max/sum.  Key rows inside the S^T tiles are permuted so
// that a lane's P^T operand covers 8 consecutive keys, which are 8 consecutive
// bf16 of one V^T row in the pool (kv_layout.h).
//
// Long rows may be split over several work items (split-KV); their partial
// (O, max, sum) go to a workspace and a merge kernel combines them.  The host
// planner orders work items longest first.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <vector>

#include "attention.h"
#include "common.h"
#include "kv_layout.h"

namespace yapd {
namespace {

constexpr int kWaves = 4;
constexpr int kChunk = 32;  // keys per inner step (two pages)

struct AttnParams {
  const uint16_t* q;     // [rows, bl, H, 64]
  const uint16_t* pool;  // [n_pages, 2, H, 1024]
  int64_t n_pages;
  const int32_t* table;
  int table_stride, table_cols;
  const int32_t* kv_len;
  int rows, bl, H;
  const int32_t* work;  // [n_work][4]: row, key_begin, key_end, slot (-1: final output)
  const int32_t* counts;  // optional device {n_work, n_merge}: grids sized by upper bounds (graph replay)
  float* part_o;        // [slots, bl, H, 64]
  float* part_ml;       // [slots, bl, H, 2]
  int n_slots;          // partials exist for slots [0, n_slots); an item naming another slot writes nothing
  float scale_log2;     // softmax scale * log2(e)
  int causal;           // 1: query i of the block sees keys < kv_len - n_q(row) + i + 1 (prefix prefill)
  uint16_t* out;        // [rows, bl, H, 64] (packed: [n_q, H, 64])
  // Packed queries (NULL: row r's bl queries are rows r*bl ..): row r's queries
  // are q / out rows [q_start[r], q_start[r+1]) of n_q, at most bl of them.
  const int32_t* q_start;
  int n_q;
};

// First query row of row r in q / out and its query count.
__device__ __forceinline__ int2 row_queries(const int32_t* q_start, int n_q, int r, int bl) {
  if (q_start == nullptr) return make_int2(r * bl, bl);
  const int qs = min(max(q_start[r], 0), n_q);
  return make_int2(qs, min(max(q_start[r + 1] - qs, 0), min(bl, n_q - qs)));
}

__device__ __forceinline__ u32x4_t load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// K/V pages are streamed once per step: non-temporal loads keep them from
// evicting the q / K / V lines the QKV GEMM has just written, whose
// write-back would otherwise land in the middle of this stream (measured
// 195 -> 179 us per layer right after the QKV GEMM).
__device__ __forceinline__ u32x4_t load16_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// Lane l combined with lane l ^ 16 (l ^ 32): v_permlane16_swap (32_swap) of a
// value with itself returns the two halves of every exchanged pair, so the
// max or sum of its two results is the pair's in both lanes -- a VALU
// exchange instead of an LDS permute.
__device__ __forceinline__ float2 swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor16_32(float v) {
  const float2 a = swap16(v);
  const float2 b = swap32(fmaxf(a.x, a.y));
  return fmaxf(b.x, b.y);
}
__device__ __forceinline__ float sum_xor16_32(float v) {
  const float2 a = swap16(v);
  const float2 b = swap32(a.x + a.y);
  return b.x + b.y;
}

// Occupancy by query tiles, measured (no spills at any of them): three and
// four tiles (blocks of 33-64 queries, the 64-token prefill chunks) are held
// to two waves per SIMD -- without the bound the compiler takes 222 VGPRs +
// 64 AGPRs for four tiles, one wave per SIMD (prefill 294 -> 280 ms).  One and
// two tiles keep the compiler's three and two: one more wave per SIMD made
// two tiles 3.7 % slower, and one tile 2 % faster on 256 rows of <= 540 keys
// but 4.5 % slower on the 30-layer stress shape (prefixes up to 2048 keys):
// more resident waves are more scattered page streams at once.
template <int NQT>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(NQT >= 3 ? 2 : 1))) void
attn_paged_kernel(const AttnParams P) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int hgroups = P.H / kWaves;
  const int item = static_cast<int>(blockIdx.x) / hgroups;
  const int h = (static_cast<int>(blockIdx.x) - item * hgroups) * kWaves + wave;
  if (P.counts != nullptr && item >= P.counts[0]) return;
  const int4 it = reinterpret_cast<const int4*>(P.work)[item];
  const int r = it.x, kb = it.y, ke = it.z, slot = it.w;
  const int kvl = P.kv_len[r];
  const int g = lane >> 4;   // lane group: key group / head-dim group
  const int n = lane & 15;   // query within a 16-query tile / row within an M tile
  const int H = P.H, bl = P.bl;
  const int2 rq = row_queries(P.q_start, P.n_q, r, bl);
  const int qs = rq.x, qc = rq.y;  // the row's first query row and query count

  // Q^T fragments (B operand): lane holds Q[q = qt*16 + n][hd = ks*32 + 8g .. +7].
  bf16x8_t qf[NQT][2];
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    const int q = qt * 16 + n;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (q < qc) v = load16(P.q + ((static_cast<int64_t>(qs) + q) * H + h) * kHeadDim + ks * 32 + 8 * g);
      qf[qt][ks] = as_bf16x8(v);
    }
  }

  f32x4_t o[NQT][4];
  float m[NQT], l[NQT];
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[qt][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int32_t* tab = P.table + static_cast<int64_t>(r) * P.table_stride;
  // Page-table reads stay inside the row even if kv_len exceeds what the table maps.
  const int last_page = min((kvl + kPageSize - 1) / kPageSize, P.table_cols) - 1;
  // Key served by row n of S^T tile t: 8*(n/4) + 4t + n%4, so that lane group g
  // ends up holding keys 8g .. 8g+7 of the chunk.
  const int key_t0 = 8 * (n >> 2) + (n & 3);

  // The row's page ids, 64 at a time: lane i holds the page of table column
  // tab_base + i (clamped), and a chunk picks its two with readlane, so the
  // K/V loads never wait on a page-table load inside the loop.
  int tab_base = -1;
  int tabv = 0;
  auto page_of = [&](int pi) -> int64_t {
    pi = min(pi, last_page);
    if (pi - tab_base >= 64 || tab_base < 0) {  // uniform: pi is the same for the wave
      tab_base = pi;
      tabv = tab[min(tab_base + lane, last_page)];
    }
    const int64_t pg = __builtin_amdgcn_readlane(tabv, pi - tab_base);
    return min(max(pg, int64_t{0}), P.n_pages - 1);  // a bad table entry cannot fault
  };
  // K fragments (A operand of S^T): tile t row n -> key key_t0 + 4t.
  // V^T fragments (A operand of O^T): row hd = 16mt + n, keys 8g .. 8g+7.
  auto load_chunk = [&](int k0, u32x4_t (&kf)[2][2], u32x4_t (&vf)[4]) {
    const int pi0 = k0 / kPageSize;
    const int64_t p0 = page_of(pi0);
    const int64_t p1 = page_of(pi0 + 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = key_t0 + 4 * t;
      const int64_t pg = key < kPageSize ? p0 : p1;
      const uint16_t* kp = P.pool + k_offset(pg, h, H, key & (kPageSize - 1), 8 * g);
      kf[t][0] = load16_stream(kp);
      kf[t][1] = load16_stream(kp + 32);
    }
    const int64_t pg = g < 2 ? p0 : p1;
    const uint16_t* vp = P.pool + v_offset(pg, h, H, 8 * (g & 1), n);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) vf[mt] = load16_stream(vp + 16 * mt * kPageSize);
  };

  // Chunk k0 + 32 is loaded while chunk k0 is multiplied.
  u32x4_t kf[2][2], vf[4], kn[2][2], vn[4];
  if (kb < ke) load_chunk(kb, kf, vf);
  // The first chunk (and q) complete here, before the loop: with a load still
  // pending on entry the compiler's wait at the loop's first MFMA is vmcnt(0),
  // which would also wait for the next chunk's loads issued just before it.
#pragma unroll
  for (int t = 0; t < 2; ++t) asm volatile("" ::"v"(kf[t][0]), "v"(kf[t][1]));
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) asm volatile("" ::"v"(vf[mt]));
  for (int k0 = kb; k0 < ke; k0 += kChunk) {
    if (k0 + kChunk < ke) load_chunk(k0 + kChunk, kn, vn);
    const bool tail = k0 + kChunk > kvl;
    const int diag0 = kvl - qc;  // causal: query q may see keys <= diag0 + q
    const bool mask_chunk = tail || (P.causal && k0 + kChunk > diag0 + 1);
    if (tail) {
      // Keys past kv_len contribute P = 0; clear their V too so stale or
      // uninitialised pool memory can never turn 0 * V into NaN.
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int key = k0 + 8 * g + 2 * w;
          uint32_t x = vf[mt][w];
          if (key >= kvl) x &= 0xffff0000u;
          if (key + 1 >= kvl) x &= 0x0000ffffu;
          vf[mt][w] = x;
        }
      }
    }

#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      f32x4_t s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[t][0]), qf[qt][0], f32x4_t{0.f, 0.f, 0.f, 0.f},
                                                       0, 0, 0);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[t][1]), qf[qt][1], s[t], 0, 0, 0);
      }
      // s[t][j] = S[q = n][key 8g + 4t + j]
      float sv[8];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float x = s[t][j] * P.scale_log2;
          if (mask_chunk) {
            const int key = k0 + 8 * g + 4 * t + j;
            if (key >= kvl || (P.causal && key > diag0 + qt * 16 + n)) x = -INFINITY;
          }
          sv[4 * t + j] = x;
        }
      }
      float cm = sv[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) cm = fmaxf(cm, sv[i]);
      cm = max_xor16_32(cm);
      const float mn = fmaxf(m[qt], cm);
      // A query that has seen no key yet (every score so far -inf: a split
      // item past the query's causal limit, or a plan longer than the device
      // kv_len) keeps m = -inf; exponents taken against 0 then give alpha = 0
      // and p = 0 instead of exp2(-inf - -inf) = NaN, so its l and O stay 0.
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m[qt] - mref);
      float ps = 0.f;
      float p[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        p[i] = __builtin_amdgcn_exp2f(sv[i] - mref);
        ps += p[i];
      }
      l[qt] = l[qt] * alpha + ps;
      m[qt] = mn;
      u32x4_t pw;
#pragma unroll
      for (int w = 0; w < 4; ++w) pw[w] = pack_bf16x2(p[2 * w], p[2 * w + 1]);
      const bf16x8_t pf = as_bf16x8(pw);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        o[qt][mt] *= alpha;
        o[qt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vf[mt]), pf, o[qt][mt], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      kf[t][0] = kn[t][0];
      kf[t][1] = kn[t][1];
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) vf[mt] = vn[mt];
  }

  // o[qt][mt][j] = O^T[hd = 16mt + 4g + j][q = qt*16 + n]
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    const float L = sum_xor16_32(l[qt]);
    const int q = qt * 16 + n;
    if (q >= qc) continue;
    const int64_t row_q = (static_cast<int64_t>(qs) + q) * H + h;
    if (slot < 0) {
      // L = 0 only for a query that sees no key at all (an empty row): zeros, not NaN
      const float inv = L > 0.f ? 1.f / L : 0.f;
      uint16_t* op = P.out + row_q * kHeadDim + 4 * g;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        u32x2_t w2;
        w2[0] = pack_bf16x2(o[qt][mt][0] * inv, o[qt][mt][1] * inv);
        w2[1] = pack_bf16x2(o[qt][mt][2] * inv, o[qt][mt][3] * inv);
        *reinterpret_cast<u32x2_t*>(op + 16 * mt) = w2;
      }
    } else if (slot < P.n_slots) {
      const int64_t prow = (static_cast<int64_t>(slot) * bl + q) * H + h;
      float* pp = P.part_o + prow * kHeadDim + 4 * g;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4_t*>(pp + 16 * mt) = o[qt][mt];
      if (g == 0) {
        P.part_ml[prow * 2] = m[qt];
        P.part_ml[prow * 2 + 1] = L;
      }
    }
  }
}

struct MergeParams {
  const int32_t* merge;  // [n_merge][3]: row, first slot, n slots
  const int32_t* counts;
  const float* part_o;
  const float* part_ml;
  int bl, H;
  int n_slots;  // parts outside [0, n_slots) are skipped
  uint16_t* out;
  const int32_t* q_start;  // packed queries, as in AttnParams
  int n_q;
};

__device__ __forceinline__ void merge_one(const MergeParams& P, int3 mi, int q) {
  const int2 rq = row_queries(P.q_start, P.n_q, mi.x, P.bl);
  if (q >= rq.y) return;
  mi.y = max(mi.y, 0);
  mi.z = max(min(mi.z, P.n_slots - mi.y), 0);  // a merge record past the partials reads nothing
  for (int t = threadIdx.x; t < P.H * 16; t += blockDim.x) {
    const int h = t >> 4;
    const int d0 = (t & 15) * 4;
    float M = -INFINITY;
    for (int s = 0; s < mi.z; ++s) {
      const int64_t prow = (static_cast<int64_t>(mi.y + s) * P.bl + q) * P.H + h;
      M = fmaxf(M, P.part_ml[prow * 2]);
    }
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
    for (int s = 0; s < mi.z; ++s) {
      const int64_t prow = (static_cast<int64_t>(mi.y + s) * P.bl + q) * P.H + h;
      const float ls = P.part_ml[prow * 2 + 1];
      if (!(ls > 0.f)) continue;  // a part in which this query saw no key
      const float w = __builtin_amdgcn_exp2f(P.part_ml[prow * 2] - M);
      L += w * ls;
      acc += w * *reinterpret_cast<const f32x4_t*>(P.part_o + prow * kHeadDim + d0);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    u32x2_t w2;
    w2[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
    w2[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
    *reinterpret_cast<u32x2_t*>(P.out + ((static_cast<int64_t>(rq.x) + q) * P.H + h) * kHeadDim + d0) = w2;
  }
}

// A grid-stride loop over (split row, query) pairs, at most kMergeGrid
// workgroups: with no live split row (the device count of a graph-replayed
// plan is often 0) the launch is a handful of empty workgroups rather than
// one per planned slot.  A thread owns 4 head-dim values of one head.
constexpr int kMergeGrid = 1024;

__global__ __launch_bounds__(256) void attn_merge_kernel(const MergeParams P, int n_merge) {
  const int live = P.counts != nullptr ? min(P.counts[1], n_merge) : n_merge;
  for (int it = blockIdx.x; it < live * P.bl; it += gridDim.x) {
    const int mrow = it / P.bl, q = it - mrow * P.bl;
    const int3 mi = make_int3(P.merge[mrow * 3], P.merge[mrow * 3 + 1], P.merge[mrow * 3 + 2]);
    merge_one(P, mi, q);
  }
}

struct KvWriteParams {
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_tok_stride, v_tok_stride;  // elements between consecutive tokens
  uint16_t* pool;
  int64_t n_pages;
  const int32_t* table;
  int table_stride, table_cols;
  const int32_t* pos0;  // [rows] first position of the block
  int rows, bl, H;
};

// Thread per (token, head, 8 head-dim values).
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteParams P) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(P.rows) * P.bl * P.H * 8;
  if (idx >= total) return;
  const int d0 = static_cast<int>(idx & 7) * 8;
  const int h = static_cast<int>((idx >> 3) % P.H);
  const int64_t tok = (idx >> 3) / P.H;
  const int r = static_cast<int>(tok / P.bl);
  const int pos = P.pos0[r] + static_cast<int>(tok - static_cast<int64_t>(r) * P.bl);
  const int pi = min(max(pos, 0) / kPageSize, P.table_cols - 1);
  int64_t page = P.table[static_cast<int64_t>(r) * P.table_stride + pi];
  page = min(max(page, int64_t{0}), P.n_pages - 1);
  const int s = pos & (kPageSize - 1);
  const u32x4_t kx = load16(P.k + tok * P.k_tok_stride + h * kHeadDim + d0);
  *reinterpret_cast<u32x4_t*>(P.pool + k_offset(page, h, P.H, s, d0)) = kx;
  const u32x4_t vx = load16(P.v + tok * P.v_tok_stride + h * kHeadDim + d0);
  uint16_t* vp = P.pool + v_offset(page, h, P.H, s, d0);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    vp[(2 * w) * kPageSize] = static_cast<uint16_t>(vx[w] & 0xffffu);
    vp[(2 * w + 1) * kPageSize] = static_cast<uint16_t>(vx[w] >> 16);
  }
}

struct KvGatherParams {
  const uint16_t* pool;
  int64_t n_pages;
  const int32_t* table_row;
  int table_len, kv_len, H;
  uint16_t* k_out;  // [kv_len, H, 64]
  uint16_t* v_out;
};

__global__ __launch_bounds__(256) void kv_gather_kernel(const KvGatherParams P) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = static_cast<int64_t>(P.kv_len) * P.H * kHeadDim;
  if (idx >= total) return;
  const int d = static_cast<int>(idx % kHeadDim);
  const int h = static_cast<int>((idx / kHeadDim) % P.H);
  const int pos = static_cast<int>(idx / (kHeadDim * P.H));
  int64_t page = P.table_row[min(pos / kPageSize, P.table_len - 1)];
  page = min(max(page, int64_t{0}), P.n_pages - 1);
  const int s = pos & (kPageSize - 1);
  P.k_out[idx] = P.pool[k_offset(page, h, P.H, s, d)];
  P.v_out[idx] = P.pool[v_offset(page, h, P.H, s, d)];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace yapd

extern "C" int yapd_attn_plan(const int32_t* kv_len, int rows, int target_items, int min_split_keys,
                              int32_t* work, int work_cap, int32_t* merge, int merge_cap, int* n_work, int* n_merge,
                              int* n_slots) {
  YAPD_REQUIRE(kv_len && work && merge && n_work && n_merge && n_slots, "attn_plan: NULL pointer");
  YAPD_REQUIRE(rows >= 1 && target_items >= 1 && min_split_keys >= yapd::kChunk,
               "attn_plan: need rows >= 1, target_items >= 1, min_split_keys >= 32");
  const int unit = yapd::kChunk;
  int64_t total_units = 0;
  for (int r = 0; r < rows; ++r) {
    YAPD_REQUIRE(kv_len[r] >= 1, "attn_plan: kv_len[%d] = %d < 1", r, kv_len[r]);
    total_units += (kv_len[r] + unit - 1) / unit;
  }
  const int64_t min_units = min_split_keys / unit;
  const int64_t per_item = std::max<int64_t>(min_units, (total_units + target_items - 1) / target_items);
  struct Item {
    int row, kb, ke, slot;
  };
  std::vector<Item> items;
  std::vector<int32_t> mrg;
  int slots = 0;
  for (int r = 0; r < rows; ++r) {
    const int units = (kv_len[r] + unit - 1) / unit;
    const int splits = static_cast<int>(std::min<int64_t>(units, (units + per_item - 1) / per_item));
    if (splits <= 1) {
      items.push_back({r, 0, kv_len[r], -1});
      continue;
    }
    const int base = units / splits, extra = units % splits;
    int u = 0;
    for (int s = 0; s < splits; ++s) {
      const int take = base + (s < extra ? 1 : 0);
      items.push_back({r, u * unit, std::min(kv_len[r], (u + take) * unit), slots + s});
      u += take;
    }
    mrg.insert(mrg.end(), {r, slots, splits});
    slots += splits;
  }
  // Longest first, so short items fill the tail of the launch.
  std::stable_sort(items.begin(), items.end(),
                   [](const Item& a, const Item& b) { return (a.ke - a.kb) > (b.ke - b.kb); });
  YAPD_REQUIRE(static_cast<int>(items.size()) <= work_cap, "attn_plan: work_cap %d < %zu", work_cap, items.size());
  YAPD_REQUIRE(static_cast<int>(mrg.size() / 3) <= merge_cap, "attn_plan: merge_cap %d < %zu", merge_cap,
               mrg.size() / 3);
  for (size_t i = 0; i < items.size(); ++i) {
    work[4 * i] = items[i].row;
    work[4 * i + 1] = items[i].kb;
    work[4 * i + 2] = items[i].ke;
    work[4 * i + 3] = items[i].slot;
  }
  std::copy(mrg.begin(), mrg.end(), merge);
  *n_work = static_cast<int>(items.size());
  *n_merge = static_cast<int>(mrg.size() / 3);
  *n_slots = slots;
  return YAPD_OK;
}

namespace yapd {

int attn_checks(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work, int n_work,
                void* out) {
  YAPD_REQUIRE(q && kv_pool && page_table && kv_len && work && out, "attn: NULL pointer");
  YAPD_REQUIRE(yapd::aligned16(q) && yapd::aligned16(kv_pool) && yapd::aligned16(out) && yapd::aligned16(work),
               "attn: q, kv_pool, out and work must be 16-byte aligned");
  YAPD_REQUIRE(rows >= 1 && bl >= 1 && bl <= 64, "attn: need rows >= 1 and 1 <= bl <= 64 (got %d, %d)", rows, bl);
  YAPD_REQUIRE(n_heads >= yapd::kWaves && n_heads % yapd::kWaves == 0, "attn: n_heads must be a multiple of %d",
               yapd::kWaves);
  YAPD_REQUIRE(n_pages >= 1 && table_cols >= 1 && table_stride >= table_cols, "attn: empty pool or table");
  YAPD_REQUIRE(n_work >= 1 && n_work < (1 << 30), "attn: n_work = %d", n_work);
  return YAPD_OK;
}

int attn_launch(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work, int n_work,
                const int32_t* merge, int n_merge, const int32_t* counts, float* part_o, float* part_ml, int n_slots,
                float scale, int causal, void* out, void* stream, const int32_t* q_start, int n_q) {
  yapd::AttnParams P;
  P.q = static_cast<const uint16_t*>(q);
  P.pool = static_cast<const uint16_t*>(kv_pool);
  P.n_pages = n_pages;
  P.table = page_table;
  P.table_stride = table_stride;
  P.table_cols = table_cols;
  P.kv_len = kv_len;
  P.rows = rows;
  P.bl = bl;
  P.H = n_heads;
  P.work = work;
  P.counts = counts;
  P.part_o = part_o;
  P.part_ml = part_ml;
  P.n_slots = (part_o != nullptr && part_ml != nullptr) ? n_slots : 0;
  P.scale_log2 = scale * 1.4426950408889634f;
  P.causal = causal != 0;
  P.out = static_cast<uint16_t*>(out);
  P.q_start = q_start;
  P.n_q = n_q;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(n_work * (n_heads / yapd::kWaves)), block(64 * yapd::kWaves);
  switch ((bl + 15) / 16) {
    case 1: hipLaunchKernelGGL(yapd::attn_paged_kernel<1>, grid, block, 0, st, P); break;
    case 2: hipLaunchKernelGGL(yapd::attn_paged_kernel<2>, grid, block, 0, st, P); break;
    case 3: hipLaunchKernelGGL(yapd::attn_paged_kernel<3>, grid, block, 0, st, P); break;
    default: hipLaunchKernelGGL(yapd::attn_paged_kernel<4>, grid, block, 0, st, P); break;
  }
  YAPD_LAUNCH_CHECK("attn_paged_kernel launch");
  if (n_merge > 0) {
    yapd::MergeParams M{merge, counts, part_o, part_ml, bl, n_heads, P.n_slots, static_cast<uint16_t*>(out), q_start,
                        n_q};
    const int64_t pairs = static_cast<int64_t>(n_merge) * bl;
    const dim3 mgrid(static_cast<unsigned>(pairs < yapd::kMergeGrid ? pairs : yapd::kMergeGrid));
    hipLaunchKernelGGL(yapd::attn_merge_kernel, mgrid, dim3(256), 0, st, M, n_merge);
    YAPD_LAUNCH_CHECK("attn_merge_kernel launch");
  }
  return YAPD_OK;
}

}  // namespace yapd

extern "C" int yapd_attn_paged_block(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table,
                                     int table_stride, int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads,
                                     const int32_t* work, int n_work, const int32_t* merge, int n_merge,
                                     const int32_t* counts, float* part_o, float* part_ml, int n_slots,
                                     float scale, int causal, void* out, void* stream) {
  const int rc = yapd::attn_checks(q, kv_pool, n_pages, page_table, table_stride, table_cols, kv_len, rows, bl, n_heads,
                             work, n_work, out);
  if (rc != YAPD_OK) return rc;
  YAPD_REQUIRE(n_merge == 0 || (merge && part_o && part_ml && n_slots >= 1), "attn: split items need a workspace");
  YAPD_REQUIRE(n_merge == 0 || (yapd::aligned16(part_o)), "attn: part_o must be 16-byte aligned");
  return yapd::attn_launch(q, kv_pool, n_pages, page_table, table_stride, table_cols, kv_len, rows, bl, n_heads, work,
                           n_work, merge, n_merge, counts, part_o, part_ml, n_slots, scale, causal, out, stream);
}

extern "C" int yapd_kv_write(const void* k, const void* v, int64_t k_tok_stride, int64_t v_tok_stride, void* kv_pool,
                             int64_t n_pages, const int32_t* page_table, int table_stride, int table_cols,
                             const int32_t* pos0, int rows, int bl, int n_heads, void* stream) {
  YAPD_REQUIRE(k && v && kv_pool && page_table && pos0, "kv_write: NULL pointer");
  YAPD_REQUIRE(yapd::aligned16(k) && yapd::aligned16(v) && yapd::aligned16(kv_pool),
               "kv_write: k, v, kv_pool must be 16-byte aligned");
  YAPD_REQUIRE(k_tok_stride % 8 == 0 && v_tok_stride % 8 == 0, "kv_write: token strides must be multiples of 8");
  YAPD_REQUIRE(rows >= 1 && bl >= 1 && n_heads >= 1 && n_pages >= 1, "kv_write: empty shape");
  YAPD_REQUIRE(table_cols >= 1 && table_stride >= table_cols, "kv_write: bad table shape");
  const int64_t total = static_cast<int64_t>(rows) * bl * n_heads * 8;
  yapd::KvWriteParams P{static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), k_tok_stride, v_tok_stride,
                        static_cast<uint16_t*>(kv_pool), n_pages, page_table, table_stride, table_cols, pos0, rows, bl,
                        n_heads};
  hipLaunchKernelGGL(yapd::kv_write_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), P);
  YAPD_LAUNCH_CHECK("kv_write_kernel launch");
  return YAPD_OK;
}

extern "C" int yapd_kv_gather(const void* kv_pool, int64_t n_pages, const int32_t* table_row, int table_len,
                              int kv_len, int n_heads, void* k_out, void* v_out, void* stream) {
  YAPD_REQUIRE(kv_pool && table_row && k_out && v_out, "kv_gather: NULL pointer");
  YAPD_REQUIRE(kv_len >= 1 && n_heads >= 1 && n_pages >= 1 && table_len >= 1, "kv_gather: empty shape");
  const int64_t total = static_cast<int64_t>(kv_len) * n_heads * yapd::kHeadDim;
  yapd::KvGatherParams P{static_cast<const uint16_t*>(kv_pool), n_pages, table_row, table_len, kv_len, n_heads,
                         static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out)};
  hipLaunchKernelGGL(yapd::kv_gather_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), P);
  YAPD_LAUNCH_CHECK("kv_gather_kernel launch");
  return YAPD_OK;
}
