// yapd_attn_paged_block_noalloc: the paged block attention of attention.hip
// with its split-KV partials in a file-scope device array instead of a
// caller-provided workspace, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops).  The array is 16 MiB
// per GPU, held until the process ends; every call on one GPU shares it, so
// calls that overlap on one GPU race (one stream per GPU, or ordered streams).
// Nothing has to start at zero: every partial the merge reads is written by
// the attention kernel of the same call first.
#include <mutex>

#include "attention.h"
#include "common.h"
#include "kv_layout.h"

namespace yapd {
namespace {

// part_o [slots, bl, H, 64] followed by part_ml [slots, bl, H, 2], fp32.
constexpr int64_t kScratchBytes = int64_t{16} << 20;
__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// The device address of `scratch` on each GPU, looked up once per device with
// that device current.  In host code the name `scratch` is a host-side
// stand-in, not a device address: only these pointers go to kernels.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The lookup is not a stream operation.  When the first call on a device comes
// while `stream` is being captured into a graph, it runs with this thread's
// capture mode switched to relaxed (the documented way for a library to make
// such a call during a capture) and the mode is restored afterwards.
int scratch_for_current_device(float** out, hipStream_t stream) {
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "attn_noalloc: hipGetDevice");
  if (rc != YAPD_OK) return rc;
  YAPD_REQUIRE(dev >= 0 && dev < kMaxDevices, "attn_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    rc = check_hip(hipStreamIsCapturing(stream, &cap), "attn_noalloc: hipStreamIsCapturing");
    if (rc != YAPD_OK) return rc;
    const bool capturing = cap == hipStreamCaptureStatusActive;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (capturing) {
      rc = check_hip(hipThreadExchangeStreamCaptureMode(&mode), "attn_noalloc: hipThreadExchangeStreamCaptureMode");
      if (rc != YAPD_OK) return rc;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (capturing) {
      rc = check_hip(hipThreadExchangeStreamCaptureMode(&mode), "attn_noalloc: restoring the capture mode");
      if (rc != YAPD_OK) return rc;
    }
    rc = check_hip(e, "attn_noalloc: hipGetSymbolAddress(scratch)");
    if (rc != YAPD_OK) return rc;
    YAPD_REQUIRE(p != nullptr && (reinterpret_cast<uintptr_t>(p) & 255u) == 0,
                 "attn_noalloc: scratch address is not 256-byte aligned");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return YAPD_OK;
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_attn_paged_block_noalloc(const void* q, const void* kv_pool, int64_t n_pages,
                                             const int32_t* page_table, int table_stride, int table_cols,
                                             const int32_t* kv_len, int rows, int bl, int n_heads, const int32_t* work,
                                             int n_work, const int32_t* merge, int n_merge, const int32_t* counts,
                                             int n_slots, float scale, int causal, void* out, void* stream) {
  int rc = yapd::attn_checks(q, kv_pool, n_pages, page_table, table_stride, table_cols, kv_len, rows, bl, n_heads,
                             work, n_work, out);
  if (rc != YAPD_OK) return rc;
  YAPD_REQUIRE(n_slots >= 0, "attn_noalloc: n_slots = %d", n_slots);
  YAPD_REQUIRE(n_merge == 0 || (merge && n_slots >= 1), "attn_noalloc: split items need n_slots >= 1 and a merge list");
  float* part_o = nullptr;
  float* part_ml = nullptr;
  if (n_slots > 0) {
    const int64_t o_floats = static_cast<int64_t>(n_slots) * bl * n_heads * yapd::kHeadDim;
    const int64_t ml_floats = static_cast<int64_t>(n_slots) * bl * n_heads * 2;
    const int64_t need = (o_floats + ml_floats) * static_cast<int64_t>(sizeof(float));
    YAPD_REQUIRE(need <= yapd::kScratchBytes,
                 "attn_noalloc: split-KV partials need %lld bytes (n_slots %d x bl %d x heads %d x 66 floats); "
                 "the static scratch holds %lld",
                 static_cast<long long>(need), n_slots, bl, n_heads, static_cast<long long>(yapd::kScratchBytes));
    float* base = nullptr;
    rc = yapd::scratch_for_current_device(&base, static_cast<hipStream_t>(stream));
    if (rc != YAPD_OK) return rc;
    part_o = base;
    part_ml = base + o_floats;  // o_floats is a multiple of 64 floats: 16-byte aligned
  }
  return yapd::attn_launch(q, kv_pool, n_pages, page_table, table_stride, table_cols, kv_len, rows, bl, n_heads, work,
                           n_work, merge, n_merge, counts, part_o, part_ml, n_slots, scale, causal, out, stream);
}
