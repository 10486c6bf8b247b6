// Calibration kernels for the measured denominators the harness reports next
// to the published peaks: the sustained bf16 MFMA rate on register operands
// (it depends on the operand values: random operands draw more power than
// few-bit constants and the part sustains ~20 % less with them), and the
// streaming HBM read rate (the bound of read-dominated kernels, which a
// read + write copy understates).
#include "common.h"
#include "../../include/yapd_probe.h"

namespace yapd {
namespace {

constexpr int kProbeAcc = 8;

__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Eight independent accumulators, each with its own operand pair.  RANDOM:
// the pairs hold random bf16 spread like the step's operands (activations of
// unit scale, weights of scale 0.02), so consecutive MFMAs switch between
// unrelated values; otherwise all eight pairs are the same few-bit constants.
template <bool RANDOM>
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* out, int iters) {
  bf16x8_t a[kProbeAcc], b[kProbeAcc];
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (RANDOM) {
        const uint32_t h = probe_hash(threadIdx.x * 131u + j * 17u + i * 7919u + blockIdx.x * 104729u);
        a[j][i] = static_cast<__bf16>((static_cast<float>(h & 0xffffu) * 0x1p-16f - 0.5f) * 3.4f);
        b[j][i] = static_cast<__bf16>((static_cast<float>(h >> 16) * 0x1p-16f - 0.5f) * 0.07f);
      } else {
        a[j][i] = static_cast<__bf16>(static_cast<float>(threadIdx.x & 7) * 0.125f + static_cast<float>(i));
        b[j][i] = static_cast<__bf16>(static_cast<float>(i) * 0.5f - 1.f);
      }
    }
  f32x16_t acc[kProbeAcc];
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], b[j], acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

// Streaming read: workgroup b reads the contiguous words [b P, (b + 1) P) (P
// = ceil(n16 / blocks) rounded up to a multiple of 256), thread t the words
// b P + t, b P + t + 256, ..., eight non-temporal 16-byte loads in flight per
// round (measured: ~6.7 TB/s against ~5.3 TB/s for a grid-stride walk with
// cached loads), folded by XOR so no load can be dropped; one word per thread
// is stored.
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ out) {
  const int64_t per = ((n16 + gridDim.x - 1) / gridDim.x + 255) / 256 * 256;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per, b1 = min(n16, b0 + per);
  u32x4_t acc = {0u, 0u, 0u, 0u};
  int64_t i = b0 + threadIdx.x;
  for (; i + 7 * 256 < b1; i += 8 * 256) {
    u32x4_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __builtin_nontemporal_load(src + i + k * 256);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k];
  }
  for (; i < b1; i += 256) acc ^= __builtin_nontemporal_load(src + i);
  out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_hbm_read_probe(const void* src, int64_t bytes, int blocks, uint32_t* out, void* stream) {
  YAPD_REQUIRE(src && out && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 && bytes >= 16 && bytes % 16 == 0 &&
                   blocks >= 1 && blocks <= (1 << 20),
               "hbm_read_probe: need a 16-byte aligned src, bytes a positive multiple of 16, 1 <= blocks <= 2^20");
  hipLaunchKernelGGL(yapd::hbm_read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const yapd::u32x4_t*>(src), bytes / 16, out);
  YAPD_LAUNCH_CHECK("hbm_read_kernel launch");
  return YAPD_OK;
}

extern "C" int yapd_mfma_peak_probe(int blocks, int iters, int random_operands, float* out, void* stream) {
  YAPD_REQUIRE(out != nullptr && blocks >= 1 && blocks <= (1 << 20) && iters >= 1,
               "mfma_peak_probe: need out and 1 <= blocks <= 2^20, iters >= 1");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (random_operands)
    hipLaunchKernelGGL(yapd::mfma_peak_kernel<true>, dim3(blocks), dim3(256), 0, st, out, iters);
  else
    hipLaunchKernelGGL(yapd::mfma_peak_kernel<false>, dim3(blocks), dim3(256), 0, st, out, iters);
  YAPD_LAUNCH_CHECK("mfma_peak_kernel launch");
  return YAPD_OK;
}
