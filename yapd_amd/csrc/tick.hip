// Continuous-batching tick bookkeeping: the per-slot state machine of
// server/engine.py FlashEngine._step_gpu (:522-612) after the scorer, as one
// small kernel so the step needs no host round trip.  One 256-thread
// workgroup per slot: thread j < bl handles block position j, thread 0 the
// slot scalars, and all threads copy the shift-context rows of a committing
// slot.
#include "common.h"

namespace yapd {
namespace {

struct TickParams {
  int n_slots, bl, n_branch, D, K;
  int64_t mask_id, stop_id, max_len, n_max;
  int64_t* xt;
  int64_t xt_stride;
  const int64_t* xt_blk;
  const int64_t* xt_new;
  int64_t* k_step;
  int64_t* cache_len;
  int64_t* blk_start;
  uint8_t* is_commit;
  const int64_t* n_speech;
  const uint16_t* hidden;
  uint16_t* shift_ctx;
  int64_t* flags;
  int64_t* xt_final;
};

constexpr int kTickThreads = 256;
constexpr int kMaxBlock = 64;

__global__ __launch_bounds__(kTickThreads) void tick_update_kernel(const TickParams p) {
  const int s = blockIdx.x;
  const int t = threadIdx.x;
  __shared__ int n_mask, eos;
  if (t == 0) {
    n_mask = 0;
    eos = 0;
  }
  __syncthreads();
  const bool commit = p.is_commit[s] != 0;
  const int64_t bs = p.blk_start[s];
  const int64_t bs_in = min(max(bs, int64_t{0}), p.n_max - p.bl);  // a bad state cannot write out of the row
  if (t < p.bl) {
    const int64_t v = commit ? p.xt_blk[static_cast<int64_t>(s) * p.bl + t] : p.xt_new[static_cast<int64_t>(s) * p.bl + t];
    p.xt_final[static_cast<int64_t>(s) * p.bl + t] = v;
    p.xt[static_cast<int64_t>(s) * p.xt_stride + bs_in + t] = v;
    if (v == p.mask_id) atomicAdd(&n_mask, 1);
    if (v == p.stop_id) atomicOr(&eos, 1);
  }
  if (commit) {
    // shift_ctx rows of this slot <- hidden row (slot row, bl - 1)
    const int n_words = p.n_branch * p.D / 2;
    for (int w = t; w < n_words; w += kTickThreads) {
      const int b = w / (p.D / 2), c = w % (p.D / 2);
      const int64_t row = static_cast<int64_t>(s) * p.n_branch + b;
      const uint32_t* src = reinterpret_cast<const uint32_t*>(p.hidden + (row * p.bl + p.bl - 1) * p.D);
      reinterpret_cast<uint32_t*>(p.shift_ctx + row * p.D)[c] = src[c];
    }
  }
  __syncthreads();
  if (t == 0) {
    const int64_t nm = n_mask;
    const bool hit = eos != 0;
    int64_t ks = commit ? 0 : p.k_step[s] + 1;
    int64_t cl = p.cache_len[s], b0 = bs;
    if (commit) {
      cl = min(cl + p.bl, p.max_len - p.bl);
      b0 = min(b0 + p.bl, p.n_max - p.bl);
    }
    const bool to_commit = !commit && !hit && (nm == 0 || ks >= p.K);
    p.k_step[s] = ks;
    p.cache_len[s] = cl;
    p.blk_start[s] = b0;
    p.is_commit[s] = to_commit ? 1 : 0;
    int64_t* f = p.flags + static_cast<int64_t>(s) * 6;
    f[0] = commit ? 1 : 0;
    f[1] = nm;
    f[2] = hit ? 1 : 0;
    f[3] = ks;
    f[4] = b0;
    f[5] = p.n_speech[s];
  }
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_tick_update(int n_slots, int bl, int n_branch, int D, int K, int64_t mask_id, int64_t stop_id,
                                int64_t max_len, int64_t n_max, int64_t* xt, int64_t xt_stride,
                                const int64_t* xt_blk, const int64_t* xt_new, int64_t* k_step, int64_t* cache_len,
                                int64_t* blk_start, uint8_t* is_commit, const int64_t* n_speech, const void* hidden,
                                void* shift_ctx, int64_t* flags, int64_t* xt_final, void* stream) {
  YAPD_REQUIRE(n_slots >= 0 && bl >= 1 && bl <= yapd::kMaxBlock && (n_branch == 1 || n_branch == 2) && D >= 2 &&
                   D % 2 == 0 && K >= 1,
               "tick_update: bad sizes (bl in [1, %d], n_branch 1 or 2, even D)", yapd::kMaxBlock);
  YAPD_REQUIRE(max_len >= 2 * bl && n_max >= bl && xt_stride >= n_max, "tick_update: bad max_len / n_max / xt_stride");
  if (n_slots == 0) return YAPD_OK;
  YAPD_REQUIRE(xt && xt_blk && xt_new && k_step && cache_len && blk_start && is_commit && n_speech && hidden &&
                   shift_ctx && flags && xt_final,
               "tick_update: NULL pointer");
  YAPD_REQUIRE((reinterpret_cast<uintptr_t>(hidden) & 3u) == 0 && (reinterpret_cast<uintptr_t>(shift_ctx) & 3u) == 0,
               "tick_update: hidden / shift_ctx must be 4-byte aligned");
  yapd::TickParams p{n_slots, bl, n_branch, D, K, mask_id, stop_id, max_len, n_max, xt, xt_stride, xt_blk, xt_new,
                     k_step, cache_len, blk_start, is_commit, n_speech, static_cast<const uint16_t*>(hidden),
                     static_cast<uint16_t*>(shift_ctx), flags, xt_final};
  hipLaunchKernelGGL(yapd::tick_update_kernel, dim3(n_slots), dim3(yapd::kTickThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  YAPD_LAUNCH_CHECK("tick_update_kernel launch");
  return YAPD_OK;
}
