// Sustained bf16 MFMA rate on register operands (the measured denominator the
// harness reports next to the published 2.5 PFLOP/s).
#include "common.h"
#include "../../include/yapd_probe.h"

namespace yapd {
namespace {

constexpr int kProbeAcc = 8;

__global__ __launch_bounds__(256) void mfma_peak_kernel(float* out, int iters) {
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(static_cast<float>(threadIdx.x & 7) * 0.125f + static_cast<float>(i));
    b[i] = static_cast<__bf16>(static_cast<float>(i) * 0.5f - 1.f);
  }
  f32x16_t acc[kProbeAcc];
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kProbeAcc; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[j][e];
  out[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

}  // namespace
}  // namespace yapd

extern "C" int yapd_mfma_peak_probe(int blocks, int iters, float* out, void* stream) {
  YAPD_REQUIRE(out != nullptr && blocks >= 1 && blocks <= (1 << 20) && iters >= 1,
               "mfma_peak_probe: need out and 1 <= blocks <= 2^20, iters >= 1");
  hipLaunchKernelGGL(yapd::mfma_peak_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), out, iters);
  YAPD_LAUNCH_CHECK("mfma_peak_kernel launch");
  return YAPD_OK;
}
