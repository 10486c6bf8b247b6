// (c) CFG combine + prior-calibrated PMI + time-shifted-quantile unmask.
//
// One workgroup of 16 waves per CFG pair.  Each wave scores whole positions:
// it streams the position's cond and null logit rows once from HBM (dword
// loads; rows are only 4-byte aligned since V = 8194), each lane keeping a
// running (max, sum-exp) per branch and its best guided score, then reduces
// across the wave on DPP.  The guided argmax uses (1+w)*lc - w*lu, which
// differs from the reference's lsc + w*(lsc - lsu) (server/engine.py:536-539)
// only by a per-row constant; the index of the maximum is found once per
// position from LDS copies of the passes that raised a lane's best.  The
// position's statistics go to LDS, and after one barrier wave 0 finishes the
// pair lane-parallel (lane = position): the pmi of each sampled token, then
// the decision rule of server/engine.py:563-593 -- ranks by pairwise
// comparison, the linear quantile with the reference's fp32 op order, top-n
// unmask.  Keeping the pair in one workgroup makes the handoff an LDS barrier:
// across workgroups it would need agent-scope release/acquire fences, which
// on a multi-XCD part write back / invalidate the XCD's L2, or a second
// launch.
#include <cmath>

#include "common.h"

namespace yapd {
namespace {

constexpr int kPairWaves = 16;  // waves per workgroup; one workgroup per CFG pair
constexpr int kUnroll = 16;    // dwords per row per lane per pass (V = 8194: four passes + 1 dword)

struct ScoreParams {
  const uint16_t* logits;
  int64_t seq_stride, pos_stride;
  int n_pairs, bl, vocab, cond_row0, pair_row_step, has_uncond, null_row_offset;
  const float* log_prior;
  const int64_t* xt_in;
  const int64_t* k_step;
  const uint8_t* active;
  const int32_t* sched;
  const float* q_tab;
  int K;
  float cfg_w, cfg_w1;  // w and (float)(1 + w)
  float rank_c;         // (float)((1 + w) / w): argmax rank c*lc - lu (w > 0, no sampling)
  int quantile_on;
  int64_t mask_id, stop_id;
  float temperature;
  int pos_gumbel;
  uint64_t seed, rng_offset;
  int64_t* sampled;
  float* pmi;
  uint8_t* unmask;
  int64_t* xt_out;
  int32_t* n_mask_after;
  uint8_t* hit_eos;
};

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ u32x4_t philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                 uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
    const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
    const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
    c1 = static_cast<uint32_t>(p1);
    c3 = static_cast<uint32_t>(p0);
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return u32x4_t{c0, c1, c2, c3};
}

__device__ __forceinline__ float gumbel_from_u32(uint32_t x) {
  const float u = (static_cast<float>(x >> 9) + 0.5f) * 0x1p-23f;  // in (0, 1), exact
  return -logf(-logf(u));
}

struct RowStats {
  float m, s;
};

__device__ __forceinline__ RowStats merge_stats(RowStats a, RowStats b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.f};
  constexpr float kLog2e = 1.4426950408889634f;
  const float sa = a.m == -INFINITY ? 0.f : a.s * __builtin_amdgcn_exp2f((a.m - m) * kLog2e);
  const float sb = b.m == -INFINITY ? 0.f : b.s * __builtin_amdgcn_exp2f((b.m - m) * kLog2e);
  return {m, sa + sb};
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave reductions on DPP: within each 16-lane row the two quad permutes, the
// half-row mirror and the row mirror leave the row's result in all of its
// lanes; v_permlane16_swap and v_permlane32_swap then combine the four row
// results, so every lane ends with the wave's result and no LDS permute is
// issued.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp_f<kDppQuadXor1>(v));
  v = op(v, dpp_f<kDppQuadXor2>(v));
  v = op(v, dpp_f<kDppHalfMirror>(v));
  v = op(v, dpp_f<kDppMirror>(v));
  // rows: v_permlane16_swap pairs row 0 with 1 and 2 with 3, v_permlane32_swap
  // the halves -- op(op(r0, r1), op(r2, r3)) in every lane
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

// The minimum of a wave, in every lane.
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, dpp_i<kDppQuadXor1>(v));
  v = min(v, dpp_i<kDppQuadXor2>(v));
  v = min(v, dpp_i<kDppHalfMirror>(v));
  v = min(v, dpp_i<kDppMirror>(v));
  const auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = min(static_cast<int>(s16[0]), static_cast<int>(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return min(static_cast<int>(s32[0]), static_cast<int>(s32[1]));
}

typedef __attribute__((ext_vector_type(2))) uint64_t u64x2_t;

// A scored position: the sampled token and each branch's maximum and sum of
// exponentials, the same in every lane.
struct ItemStats {
  int x;
  float Mc, Sc, Mu, Su;
};

// One (pair, position) scored by one wave: a streaming pass over the cond
// and null rows (dword loads; rows are only 4-byte aligned at V = 8194), each
// lane keeping running softmax statistics and its best guided score, then
// wave reductions on DPP.  Per element the VALU work is what the math needs
// (bf16 unpack, max, one FMA + v_exp and an add per branch, the guided score
// and its maximum).  A pass's 32 loads per lane are issued back to back; the
// other waves of the workgroup (4 per SIMD) cover their latency.  The argmax
// index is not searched per pass: a pass that raises a lane's best stores its
// guided values to the lane's part of the wave's LDS slot (``sav``, 8 KB),
// and once per position the lowest index at the wave's maximum is read back
// from the slots of the lanes that hold it.
template <bool kHasU, bool kSample, bool kRank>
__device__ __forceinline__ ItemStats score_item(const ScoreParams& P, int item, int pair, int pos, int lane,
                                                float4* __restrict__ sav) {
  const int64_t crow = static_cast<int64_t>(P.cond_row0) + static_cast<int64_t>(pair) * P.pair_row_step;
  const uint16_t* rc = P.logits + crow * P.seq_stride + static_cast<int64_t>(pos) * P.pos_stride;
  const uint16_t* ru = rc + static_cast<int64_t>(P.null_row_offset) * P.seq_stride;
  const uint32_t* wc = reinterpret_cast<const uint32_t*>(rc);
  const uint32_t* wu = reinterpret_cast<const uint32_t*>(ru);
  const int V = P.vocab;
  const int nw = V >> 1;
  const float w = P.cfg_w, w1 = P.cfg_w1;
  const uint32_t key0 = static_cast<uint32_t>(P.seed), key1 = static_cast<uint32_t>(P.seed >> 32);
  const uint32_t off0 = static_cast<uint32_t>(P.rng_offset), off1 = static_cast<uint32_t>(P.rng_offset >> 32);
  constexpr float kLog2e = 1.4426950408889634f;
  constexpr int kPass = 64 * kUnroll;  // dwords per row per pass

  RowStats sc{-INFINITY, 0.f}, su{-INFINITY, 0.f};
  float best_g = -INFINITY;
  int best_v = 0x7fffffff;  // the lane's best element when it came from the tail
  int best_pass = -1;       // else the pass whose guided values sit in the lane's slot

  // Guided score of element v (+ T * Gumbel noise when sampling).  Without
  // sampling only its order matters, and for w > 0 the argmax ranks by
  // c*lc - lu, c = (1+w)/w: the same order as (1+w)*lc - w*lu (one FMA per
  // element; exact for bf16 logits at w = 0.5, where c = 3).
  auto guided = [&](float lc, float lu, int v) {
    if constexpr (kRank) return __builtin_fmaf(P.rank_c, lc, -lu);
    // one rounding less than (1+w)*lc - w*lu; only ulp-level near-ties can tell
    float g = kHasU ? __builtin_fmaf(w1, lc, -w * lu) : lc;
    if (kSample) {
      const u32x4_t r = philox4x32_10(static_cast<uint32_t>(v >> 2), static_cast<uint32_t>(item), off0, off1,
                                      key0, key1);
      const uint32_t word = (v & 3) == 0 ? r.x : (v & 3) == 1 ? r.y : (v & 3) == 2 ? r.z : r.w;
      g = __fadd_rn(g, __fmul_rn(P.temperature, gumbel_from_u32(word)));
    }
    return g;
  };
  // Running statistics of one branch after a pass with maximum mp and values
  // f: one rescale exp, then the pass's exps against the new maximum (a
  // maximum of -inf keeps the sum at 0).
  auto update = [&](RowStats& st, float mp, const float* f) {
    const float mn = fmaxf(st.m, mp);
    const float mns = mn == -INFINITY ? 0.f : mn * kLog2e;
    float acc = st.m == -INFINITY ? 0.f : st.s * __builtin_amdgcn_exp2f(st.m * kLog2e - mns);
#pragma unroll
    for (int e = 0; e < 2 * kUnroll; ++e) acc += __builtin_amdgcn_exp2f(__builtin_fmaf(f[e], kLog2e, -mns));
    st = RowStats{mn, acc};
  };

  const int n_pass = nw / kPass;
  uint32_t xc[kUnroll], xu[kUnroll];
  // Cached loads: in the step the head GEMM has just written the logits and
  // much of them is still in the MALL (non-temporal loads measured ~1 % faster
  // on cold inputs but 7 us slower inside the step graph).
  auto load_pass = [&](int base) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      xc[u] = wc[base + u * 64 + lane];
      if (kHasU) xu[u] = wu[base + u * 64 + lane];
    }
  };
  // the first tail word, requested with the first pass rather than after the
  // last one
  const int jt = n_pass * kPass + lane;
  uint32_t tc0 = 0u, tu0 = 0u;
  if (jt < nw) {
    tc0 = wc[jt];
    if (kHasU) tu0 = wu[jt];
  }
  for (int pi = 0; pi < n_pass; ++pi) {
    const int base = pi * kPass;
    load_pass(base);
    float fc[2 * kUnroll], fu[2 * kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      fc[2 * u] = bf16lo(xc[u]);
      fc[2 * u + 1] = bf16hi(xc[u]);
      if (kHasU) {
        fu[2 * u] = bf16lo(xu[u]);
        fu[2 * u + 1] = bf16hi(xu[u]);
      }
    }
    float mc = fc[0], mu = kHasU ? fu[0] : 0.f;
#pragma unroll
    for (int e = 1; e < 2 * kUnroll; ++e) {
      mc = fmaxf(mc, fc[e]);
      if (kHasU) mu = fmaxf(mu, fu[e]);
    }
    update(sc, mc, fc);
    if (kHasU) update(su, mu, fu);
    // argmax; the first maximum in index order wins, as torch.argmax does:
    // the maximum by a max3 tree, then the lowest element equal to it (the
    // guided values reuse the registers of fc, which are dead by now).
    float gv[2 * kUnroll];
#pragma unroll
    for (int e = 0; e < 2 * kUnroll; ++e)
      gv[e] = guided(fc[e], kHasU ? fu[e] : 0.f, 2 * (base + (e >> 1) * 64 + lane) + (e & 1));
    float pg = gv[0];
#pragma unroll
    for (int e = 1; e < 2 * kUnroll; ++e) pg = fmaxf(pg, gv[e]);
    if (pg > best_g) {
      best_g = pg;
      best_pass = pi;
#pragma unroll
      for (int q = 0; q < kUnroll / 2; ++q)
        sav[q * 64 + lane] = make_float4(gv[4 * q], gv[4 * q + 1], gv[4 * q + 2], gv[4 * q + 3]);
    }
  }
  // Tail: the remaining dwords, one per lane at a time.
  for (int j = jt; j < nw; j += 64) {
    const uint32_t tc = j == jt ? tc0 : wc[j];
    const uint32_t tu = j == jt ? tu0 : kHasU ? wu[j] : 0u;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float lc = h ? bf16hi(tc) : bf16lo(tc);
      const float lu = h ? bf16hi(tu) : bf16lo(tu);
      sc = merge_stats(sc, RowStats{lc, 1.f});
      if (kHasU) su = merge_stats(su, RowStats{lu, 1.f});
      const float g = guided(lc, lu, 2 * j + h);
      if (g > best_g) {
        best_g = g;
        best_v = 2 * j + h;
        best_pass = -1;
      }
    }
  }
  if ((V & 1) && lane == 0) {  // odd vocab: the last element sits alone
    const float lc = bf16_to_f32(rc[V - 1]);
    const float lu = kHasU ? bf16_to_f32(ru[V - 1]) : 0.f;
    sc = merge_stats(sc, RowStats{lc, 1.f});
    if (kHasU) su = merge_stats(su, RowStats{lu, 1.f});
    const float g = guided(lc, lu, V - 1);
    if (g > best_g) {
      best_g = g;
      best_v = V - 1;
      best_pass = -1;
    }
  }

  // Wave reductions: the maximum of each branch (with the argmax), then each
  // lane rescales its sum once to it and the sums are added.
  auto fmax_op = [](float a, float b) { return fmaxf(a, b); };
  auto add_op = [](float a, float b) { return a + b; };
  const float Mc = wave_reduce(sc.m, fmax_op);
  const float Mu = kHasU ? wave_reduce(su.m, fmax_op) : 0.f;
  // argmax: the lowest element index whose guided value is the wave's maximum,
  // as torch.argmax.  Each lane's best is its first occurrence in index order
  // (strict > above); a lane whose best lies in a pass finds it in its slot:
  // lane e < 2 * kUnroll checks element e of that pass.  One lane holds the
  // maximum unless values tie exactly.
  const float Gm = wave_reduce(best_g, fmax_op);
  // the slots were written by other lanes of this wave: LDS runs a wave's
  // accesses in order, the fences keep the compiler from moving them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int best_idx = best_g == Gm && best_pass < 0 ? best_v : 0x7fffffff;
  uint64_t cand = __ballot(best_g == Gm && best_pass >= 0);
  const float* savf = reinterpret_cast<const float*>(sav);
  while (cand) {
    const int L = __ffsll(static_cast<unsigned long long>(cand)) - 1;
    cand &= cand - 1;
    const int pL = __builtin_amdgcn_readlane(best_pass, L);
    if (lane < 2 * kUnroll && savf[((lane >> 2) * 64 + L) * 4 + (lane & 3)] == Gm)
      best_idx = min(best_idx, 2 * (pL * kPass + (lane >> 1) * 64 + L) + (lane & 1));
  }
  best_idx = wave_min_i(best_idx);
  // the next position's slot writes stay after these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // a lane with no finite value (m = -inf) contributes nothing; so does a row
  // whose maximum is -inf, whose sum stays 0
  const float Sc = wave_reduce(sc.m == -INFINITY ? 0.f : sc.s * __builtin_amdgcn_exp2f((sc.m - Mc) * kLog2e), add_op);
  const float Su = kHasU ? wave_reduce(su.m == -INFINITY ? 0.f : su.s * __builtin_amdgcn_exp2f((su.m - Mu) * kLog2e),
                                       add_op)
                         : 0.f;
  const int x = best_idx < V ? best_idx : 0;  // a row of only -inf / NaN scores: token 0, as torch.argmax
  return ItemStats{x, Mc, Sc, Mu, Su};
}

// The pmi of one scored item from its row statistics (lane-parallel: one
// item per lane).
template <bool kHasU>
__device__ __forceinline__ float item_pmi(const ScoreParams& P, int item, int pair, int pos, const ItemStats& st,
                                          int64_t xt) {
  const int64_t crow = static_cast<int64_t>(P.cond_row0) + static_cast<int64_t>(pair) * P.pair_row_step;
  const uint16_t* rc = P.logits + crow * P.seq_stride + static_cast<int64_t>(pos) * P.pos_stride;
  const uint16_t* ru = rc + static_cast<int64_t>(P.null_row_offset) * P.seq_stride;
  const int x = st.x;
  const float w = P.cfg_w, w1 = P.cfg_w1;
  const float lpr = P.log_prior[x];
  // probs.gather(sampled).clamp_min(1e-8).log() - log_prior[sampled]
  const float lcx = bf16_to_f32(rc[x]);
  float pmi = __fsub_rn(logf(fmaxf(__fdiv_rn(expf(lcx - st.Mc), st.Sc), 1e-8f)), lpr);
  if (kHasU) {
    const float lux = bf16_to_f32(ru[x]);
    const float pmi_u = __fsub_rn(logf(fmaxf(__fdiv_rn(expf(lux - st.Mu), st.Su), 1e-8f)), lpr);
    pmi = __fsub_rn(__fmul_rn(w1, pmi), __fmul_rn(w, pmi_u));
  }
  if (P.pos_gumbel && xt == P.mask_id) {
    const uint32_t key0 = static_cast<uint32_t>(P.seed), key1 = static_cast<uint32_t>(P.seed >> 32);
    const uint32_t off0 = static_cast<uint32_t>(P.rng_offset), off1 = static_cast<uint32_t>(P.rng_offset >> 32);
    const u32x4_t r = philox4x32_10(0xffffffffu, static_cast<uint32_t>(item), off0, off1, key0, key1);
    pmi = __fadd_rn(pmi, gumbel_from_u32(r.x));
  }
  return pmi;
}

// The per-pair inputs of the decision rule, one entry per lane: every load is
// independent, and the step tables are picked by readlane once k is known.
struct PairInputs {
  int64_t k;
  float q_lane;
  int sched_lane;
  bool act;
  int64_t xt;
};

__device__ __forceinline__ PairInputs load_pair_inputs(const ScoreParams& P, int pair, int lane) {
  const int64_t ib = static_cast<int64_t>(pair) * P.bl;
  PairInputs in;
  in.k = P.k_step[pair];
  in.q_lane = lane < P.K ? P.q_tab[lane] : 0.f;
  in.sched_lane = lane < P.K ? P.sched[lane] : 0;
  in.act = P.active == nullptr || P.active[pair] != 0;
  in.xt = lane < P.bl ? P.xt_in[ib + lane] : 0;
  return in;
}

// The decision rule of server/engine.py:563-593 for one pair, one wave, lane
// = position: rank by pairwise compare (ties -> lowest position), p =
// q_k (m-1), linear quantile, n = min(max(min(sched, m), n_quant), m), top-n
// unmask, n_mask_after and hit_eos.
__device__ __forceinline__ void decide_pair(const ScoreParams& P, int pair, int lane, const PairInputs& in, float key,
                                            int64_t smp, uint64_t* s_ka, uint64_t* s_kd) {
  const int bl = P.bl;
  const int64_t ib = static_cast<int64_t>(pair) * bl;
  const bool valid = lane < bl;
  const int64_t k = in.k;
  const int64_t xt = in.xt;
  const bool msk = valid && xt == P.mask_id;
  const uint64_t bal = __ballot(msk);
  const int m = __popcll(bal);

  // Ranks among the masked positions.  asc counts masked j with p_j < key, or
  // p_j == key and j < lane; desc the same with p_j > key.  Each position's
  // key becomes two 64-bit words -- its float order as an unsigned number
  // (-0 taken as +0), or that number's complement, above the position index
  // -- so one unsigned compare decides both the order and the tie.  Positions
  // that are not masked and NaN keys hold all ones, which no compare counts, as
  // no float compare counts a NaN.  With at most 32 positions the two halves
  // of the wave each compare with half of the keys.
  const bool num = msk && key == key;
  const uint32_t ku = __float_as_uint(key + 0.f);
  const uint32_t ord = ku ^ (static_cast<uint32_t>(static_cast<int32_t>(ku) >> 31) | 0x80000000u);
  s_ka[lane] = num ? (static_cast<uint64_t>(ord) << 32 | static_cast<uint32_t>(lane)) : ~0ull;
  s_kd[lane] = num ? (static_cast<uint64_t>(~ord) << 32 | static_cast<uint32_t>(lane)) : ~0ull;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool split = bl <= 32;
  const int own = split ? (lane & 31) : lane;
  const int j0 = split ? (lane >> 5) * 16 : 0;
  const int nj = split ? 16 : bl;  // entries past bl hold all ones
  const uint64_t a_own = s_ka[own], d_own = s_kd[own];
  int asc = 0, desc = 0;
  if (split) {  // all 16 words of the half requested at once: one LDS round trip
    u64x2_t a2[8], d2[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      a2[t] = *reinterpret_cast<const u64x2_t*>(s_ka + j0 + 2 * t);
      d2[t] = *reinterpret_cast<const u64x2_t*>(s_kd + j0 + 2 * t);
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      asc += (a2[t][0] < a_own) + (a2[t][1] < a_own);
      desc += (d2[t][0] < d_own) + (d2[t][1] < d_own);
    }
  } else {
    for (int t = 0; t < nj; t += 2) {
      const u64x2_t a2 = *reinterpret_cast<const u64x2_t*>(s_ka + j0 + t);
      const u64x2_t d2 = *reinterpret_cast<const u64x2_t*>(s_kd + j0 + t);
      asc += (a2[0] < a_own) + (a2[1] < a_own);
      desc += (d2[0] < d_own) + (d2[1] < d_own);
    }
  }
  if (split) {
    const auto sa = __builtin_amdgcn_permlane32_swap(asc, asc, false, false);
    const auto sd = __builtin_amdgcn_permlane32_swap(desc, desc, false, false);
    asc = static_cast<int>(sa[0]) + static_cast<int>(sa[1]);
    desc = static_cast<int>(sd[0]) + static_cast<int>(sd[1]);
  }
  if (!num) asc = desc = 0;  // a NaN key compares false with every key
  int kc = k < P.K - 1 ? static_cast<int>(k) : P.K - 1;
  kc = kc < 0 ? 0 : kc;
  // p = q_t[k] * (m-1).clamp_min(0).float(); lo/hi = floor/ceil; linear interpolation.
  const float p = __fmul_rn(readlane_f(in.q_lane, kc), static_cast<float>(m > 1 ? m - 1 : 0));
  int lo = static_cast<int>(floorf(p));
  int hi = static_cast<int>(ceilf(p));
  lo = lo < 0 ? 0 : lo;
  hi = hi < 0 ? 0 : hi;
  const uint64_t blo = __ballot(msk && asc == lo);
  const uint64_t bhi = __ballot(msk && asc == hi);
  const float v_lo = blo ? readlane_f(key, __ffsll(static_cast<unsigned long long>(blo)) - 1) : INFINITY;
  const float v_hi = bhi ? readlane_f(key, __ffsll(static_cast<unsigned long long>(bhi)) - 1) : INFINITY;
  const float tau = __fadd_rn(v_lo, __fmul_rn(__fsub_rn(p, static_cast<float>(lo)), __fsub_rn(v_hi, v_lo)));
  const int n_quant = P.quantile_on ? __popcll(__ballot(msk && key >= tau)) : 0;
  const int n_sched = min(__builtin_amdgcn_readlane(in.sched_lane, kc), m);
  int n = min(max(n_sched, n_quant), m);
  if (k >= P.K - 1) n = m;
  if (m == 0) n = 0;
  const bool unm = in.act && msk && desc < n;
  const int64_t xo = unm ? smp : xt;
  if (valid) {
    P.unmask[ib + lane] = unm ? 1 : 0;
    P.xt_out[ib + lane] = xo;
  }
  const int n_after = __popcll(__ballot(valid && xo == P.mask_id));
  const bool eos = __ballot(valid && xo == P.stop_id) != 0ull;
  if (lane == 0) {
    P.n_mask_after[pair] = n_after;
    P.hit_eos[pair] = eos ? 1 : 0;
  }
}

// One workgroup per pair: wave w scores positions w, w + kPairWaves, ...
// into LDS; after the barrier wave 0 computes the pair's pmi lane-parallel --
// the gathers of log_prior and the logits at the sampled tokens are one round
// trip for the whole pair, and the per-pair inputs ride along -- and applies
// the decision rule.  One launch, no handoff through global memory between
// workgroups.
template <bool kHasU, bool kSample, bool kRank = false>
__global__ __launch_bounds__(64 * kPairWaves) void score_pair_kernel(const ScoreParams P) {
  const int pair = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __shared__ ItemStats s_st[64];
  __shared__ __align__(16) uint64_t s_ka[64];
  __shared__ __align__(16) uint64_t s_kd[64];
  __shared__ float4 s_sav[kPairWaves * (kUnroll / 2) * 64];  // 8 KB per wave: guided values of a lane's best pass
  for (int pos = wave; pos < P.bl; pos += kPairWaves) {
    const ItemStats st = score_item<kHasU, kSample, kRank>(P, pair * P.bl + pos, pair, pos, lane,
                                                           s_sav + wave * (kUnroll / 2) * 64);
    if (lane == 0) s_st[pos] = st;
  }
  __syncthreads();
  if (wave == 0) {
    const PairInputs in = load_pair_inputs(P, pair, lane);
    const bool valid = lane < P.bl;
    float pmi = 0.f;
    int64_t x = 0;
    if (valid) {
      const int item = pair * P.bl + lane;
      const ItemStats st = s_st[lane];
      pmi = item_pmi<kHasU>(P, item, pair, lane, st, in.xt);
      x = st.x;
      P.sampled[item] = x;
      P.pmi[item] = pmi;
    }
    decide_pair(P, pair, lane, in, pmi, x, s_ka, s_kd);
  }
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_score_cfg_pmi_unmask(
    const void* logits, int64_t seq_stride, int64_t pos_stride, int n_pairs, int bl, int vocab, int cond_row0,
    int pair_row_step, int has_uncond, int null_row_offset, const float* log_prior, const int64_t* xt_in,
    const int64_t* k_step, const uint8_t* active, const int32_t* sched, const float* q_tab, int K, float cfg_w,
    int quantile_on, int64_t mask_id, int64_t stop_id, float temperature, int pos_gumbel, uint64_t seed,
    uint64_t rng_offset, int64_t* sampled_out, float* pmi_out, uint8_t* unmask_out, int64_t* xt_out,
    int32_t* n_mask_after_out, uint8_t* hit_eos_out, void* stream) {
  YAPD_REQUIRE(logits != nullptr, "score: logits is NULL");
  YAPD_REQUIRE((reinterpret_cast<uintptr_t>(logits) & 3u) == 0, "score: logits must be 4-byte aligned");
  YAPD_REQUIRE(n_pairs >= 1 && bl >= 1 && bl <= 64, "score: need n_pairs >= 1 and 1 <= bl <= 64 (got %d, %d)",
               n_pairs, bl);
  YAPD_REQUIRE(vocab >= 1, "score: vocab must be >= 1 (got %d)", vocab);
  YAPD_REQUIRE(static_cast<int64_t>(n_pairs) * bl < (int64_t{1} << 31), "score: too many items");
  YAPD_REQUIRE(seq_stride % 2 == 0 && pos_stride % 2 == 0, "score: strides must be even (got %lld, %lld)",
               static_cast<long long>(seq_stride), static_cast<long long>(pos_stride));
  YAPD_REQUIRE(pos_stride >= vocab, "score: pos_stride %lld < vocab %d", static_cast<long long>(pos_stride), vocab);
  YAPD_REQUIRE(cond_row0 >= 0 && pair_row_step >= 0, "score: negative row layout");
  YAPD_REQUIRE(K >= 1 && K <= 64, "score: need 1 <= K <= 64 (got %d)", K);
  YAPD_REQUIRE(temperature >= 0.f, "score: temperature must be >= 0");
  YAPD_REQUIRE(log_prior && xt_in && k_step && sched && q_tab, "score: NULL input pointer");
  YAPD_REQUIRE(sampled_out && pmi_out && unmask_out && xt_out && n_mask_after_out && hit_eos_out,
               "score: NULL output pointer");
  yapd::ScoreParams P;
  P.logits = static_cast<const uint16_t*>(logits);
  P.seq_stride = seq_stride;
  P.pos_stride = pos_stride;
  P.n_pairs = n_pairs;
  P.bl = bl;
  P.vocab = vocab;
  P.cond_row0 = cond_row0;
  P.pair_row_step = pair_row_step;
  P.has_uncond = has_uncond;
  P.null_row_offset = has_uncond ? null_row_offset : 0;
  P.log_prior = log_prior;
  P.xt_in = xt_in;
  P.k_step = k_step;
  P.active = active;
  P.sched = sched;
  P.q_tab = q_tab;
  P.K = K;
  P.cfg_w = cfg_w;
  P.cfg_w1 = static_cast<float>(1.0 + static_cast<double>(cfg_w));
  P.rank_c = cfg_w > 0.f ? static_cast<float>((1.0 + static_cast<double>(cfg_w)) / static_cast<double>(cfg_w)) : 0.f;
  P.quantile_on = quantile_on;
  P.mask_id = mask_id;
  P.stop_id = stop_id;
  P.temperature = temperature;
  P.pos_gumbel = pos_gumbel;
  P.seed = seed;
  P.rng_offset = rng_offset;
  P.sampled = sampled_out;
  P.pmi = pmi_out;
  P.unmask = unmask_out;
  P.xt_out = xt_out;
  P.n_mask_after = n_mask_after_out;
  P.hit_eos = hit_eos_out;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(n_pairs), block(64 * yapd::kPairWaves);
  if (has_uncond && temperature > 0.f)
    hipLaunchKernelGGL((yapd::score_pair_kernel<true, true>), grid, block, 0, st, P);
  else if (has_uncond && cfg_w > 0.f)
    hipLaunchKernelGGL((yapd::score_pair_kernel<true, false, true>), grid, block, 0, st, P);
  else if (has_uncond)
    hipLaunchKernelGGL((yapd::score_pair_kernel<true, false>), grid, block, 0, st, P);
  else if (temperature > 0.f)
    hipLaunchKernelGGL((yapd::score_pair_kernel<false, true>), grid, block, 0, st, P);
  else
    hipLaunchKernelGGL((yapd::score_pair_kernel<false, false>), grid, block, 0, st, P);
  YAPD_LAUNCH_CHECK("score_pair_kernel launch");
  return YAPD_OK;
}
