// HiFT vocoder elementwise family on contiguous fp32 [B, C, T] tensors
// (server/kernels.py:35-67): Snake activation, bias / residual adds, the
// three-way resblock mean, and the fused combinations the S3Gen HiFT
// generator uses between its convolutions.
//
// Layout of the work: one workgroup owns kChunk consecutive samples of one
// (b, c) row, so the per-channel alpha / bias values are wave-uniform scalar
// loads made once per workgroup (no per-element index division), and every
// thread moves 16-byte vectors over the 16-byte-aligned middle of its range,
// whatever T is (HiFT's last stage has T = 3 * 6400 + 1 after its reflection
// pad), with at most three elements one by one at either end.  The loads of
// a thread's vectors are all issued before any is used.  Each op is HBM-bound
// (8 to 24 bytes per element against a few dozen VALU operations, sinf
// included), so the roofline is the bytes of the inputs plus the outputs.
#include <cmath>

#include "common.h"
#include "../../include/yapd_vocoder.h"

namespace yapd {
namespace {

constexpr int kVThreads = 256;
constexpr int kVecPer = 2;                            // 16-byte vectors per thread per chunk
constexpr int kChunk = kVThreads * 4 * kVecPer;        // samples per workgroup (2048)

enum VocOp { kOpSnake = 0, kOpResidualBias = 1, kOpResidualBiasSnake = 2, kOpBranchStart = 3 };

struct VocParams {
  const float* x;
  const float* r;     // residual (residual ops) or source (branch start)
  const float* bias;  // per channel, may be NULL for kOpSnake
  const float* a0;    // per channel alphas
  const float* a1;
  const float* a2;
  float* o0;  // snake: out; residual_bias: out; rbs: raw; branch: raw
  float* o1;  // rbs: act; branch: out0
  float* o2;  // branch: out1
  float* o3;  // branch: out2
  int C;
  int64_t T;
  int64_t chunks;  // workgroups per row
  int vec;         // 16-byte path: every pointer 16-byte aligned
};

// Snake with the per-channel constants folded: v + inv * sin(v * a)^2,
// inv = 1 / (a + 1e-9) (the HiFT module's expression; the reference kernel's
// s^2 / (a + 1e-9) differs from it by at most one rounding).
__device__ __forceinline__ float snake(float v, float a, float inv) {
  const float s = sinf(v * a);
  return v + inv * (s * s);
}

template <int OP>
__device__ __forceinline__ void apply(const VocParams& p, float x, float r, float b, const float (&a)[3],
                                      const float (&inv)[3], float (&o)[4]) {
  if constexpr (OP == kOpSnake) {
    o[0] = snake(x + b, a[0], inv[0]);
  } else if constexpr (OP == kOpResidualBias) {
    o[0] = (x + r) + b;
  } else if constexpr (OP == kOpResidualBiasSnake) {
    const float raw = (x + r) + b;
    o[0] = raw;
    o[1] = snake(raw, a[0], inv[0]);
  } else {
    const float raw = x + r;
    o[0] = raw;
    o[1] = snake(raw, a[0], inv[0]);
    o[2] = snake(raw, a[1], inv[1]);
    o[3] = snake(raw, a[2], inv[2]);
  }
}

template <int OP>
__global__ __launch_bounds__(kVThreads) void voc_kernel(const VocParams p) {
  constexpr bool kR = OP != kOpSnake;
  constexpr int kOut = OP == kOpBranchStart ? 4 : OP == kOpResidualBiasSnake ? 2 : 1;
  constexpr int kAlphas = OP == kOpBranchStart ? 3 : OP == kOpResidualBias ? 0 : 1;
  const int64_t wg = blockIdx.x;
  const int64_t row = wg / p.chunks;  // uniform: one (b, c) row per workgroup
  const int64_t t0 = (wg - row * p.chunks) * kChunk;
  const int c = static_cast<int>(row % p.C);
  const float b = (OP != kOpBranchStart && p.bias) ? p.bias[c] : 0.f;
  float a[3] = {0.f, 0.f, 0.f}, inv[3] = {0.f, 0.f, 0.f};
  const float* as[3] = {p.a0, p.a1, p.a2};
#pragma unroll
  for (int j = 0; j < kAlphas; ++j) {
    a[j] = as[j][c];
    inv[j] = 1.0f / (a[j] + 1.0e-9f);
  }
  float* outs[4] = {p.o0, p.o1, p.o2, p.o3};
  // This workgroup's elements, as flat indices [g0, g1) of the [B, C, T] tensors.
  const int64_t g0 = row * p.T + t0;
  const int64_t g1 = row * p.T + (t0 + kChunk < p.T ? t0 + kChunk : p.T);
  auto one = [&](int64_t g) {
    float o[4];
    apply<OP>(p, p.x[g], kR ? p.r[g] : 0.f, b, a, inv, o);
#pragma unroll
    for (int k = 0; k < kOut; ++k) outs[k][g] = o[k];
  };

  if (p.vec) {
    // 16-byte vectors over the aligned middle [v0, v1); at most 3 elements
    // before and after it go one by one.
    const int64_t v0 = (g0 + 3) & ~int64_t{3};
    const int64_t v1 = g1 & ~int64_t{3};
    if (v0 >= v1) {  // a range with no whole aligned vector
      for (int64_t g = g0 + threadIdx.x; g < g1; g += kVThreads) one(g);
      return;
    }
    if (threadIdx.x < v0 - g0) one(g0 + threadIdx.x);
    if (threadIdx.x < g1 - v1) one(v1 + threadIdx.x);
    // Inputs are read once.  residual_bias (one output, a residual input
    // written long before) reads with non-temporal loads: 19 % faster on cold
    // inputs and still 4 % when x was just written.  Snake's only input is
    // usually the output of the convolution just before it, still in the MALL,
    // where non-temporal loads measured 3 % slower; with two or four outputs
    // they measured 4-5 % slower even on cold inputs.
    auto load = [](const float* src) {
      if constexpr (kOut == 1 && kR) {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(src));
      } else {
        return *reinterpret_cast<const f32x4_t*>(src);
      }
    };
    f32x4_t xv[kVecPer], rv[kVecPer];
    int64_t gv[kVecPer];
#pragma unroll
    for (int q = 0; q < kVecPer; ++q) {
      gv[q] = v0 + static_cast<int64_t>(q * kVThreads + threadIdx.x) * 4;
      if (gv[q] < v1) {
        xv[q] = load(p.x + gv[q]);
        if (kR) rv[q] = load(p.r + gv[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < kVecPer; ++q) {
      if (gv[q] >= v1) continue;
      f32x4_t ov[kOut];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float o[4];
        apply<OP>(p, xv[q][e], kR ? rv[q][e] : 0.f, b, a, inv, o);
#pragma unroll
        for (int k = 0; k < kOut; ++k) ov[k][e] = o[k];
      }
#pragma unroll
      for (int k = 0; k < kOut; ++k) *reinterpret_cast<f32x4_t*>(outs[k] + gv[q]) = ov[k];
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4 * kVecPer; ++q) {
      const int64_t g = g0 + q * kVThreads + threadIdx.x;
      if (g >= g1) break;
      one(g);
    }
  }
}

// ((a + b) + c) * (1/3), the reference's operation order, over a flat range;
// with vec, 16-byte vectors up to n & ~3 and the last (n % 4) one by one.
__global__ __launch_bounds__(kVThreads) void mean3_kernel(const float* a, const float* b, const float* c, float* out,
                                                          int64_t n, int vec) {
  constexpr float kThird = 1.0f / 3.0f;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  if (vec) {
    const int64_t nv = n & ~int64_t{3};
#pragma unroll
    for (int q = 0; q < kVecPer; ++q) {
      const int64_t t = t0 + static_cast<int64_t>(q * kVThreads + threadIdx.x) * 4;
      if (t >= nv) continue;
      // read once, one output: non-temporal loads (measured 17 % faster on
      // cold inputs, 7 % with the first input just written)
      const f32x4_t va = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(a + t));
      const f32x4_t vb = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(b + t));
      const f32x4_t vc = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(c + t));
      f32x4_t vo;
#pragma unroll
      for (int e = 0; e < 4; ++e) vo[e] = ((va[e] + vb[e]) + vc[e]) * kThird;
      *reinterpret_cast<f32x4_t*>(out + t) = vo;
    }
    const int64_t t = nv + threadIdx.x;
    if (t0 + kChunk >= n && t < n) out[t] = ((a[t] + b[t]) + c[t]) * kThird;  // the last workgroup
  } else {
#pragma unroll
    for (int q = 0; q < 4 * kVecPer; ++q) {
      const int64_t t = t0 + q * kVThreads + threadIdx.x;
      if (t >= n) break;
      out[t] = ((a[t] + b[t]) + c[t]) * kThird;
    }
  }
}

bool al16f(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_bct(const float* x, int64_t B, int C, int64_t T, const char* op) {
  YAPD_REQUIRE(x != nullptr, "%s: NULL input", op);
  YAPD_REQUIRE(B >= 1 && C >= 1 && T >= 1, "%s: need B, C, T >= 1 (got %lld, %d, %lld)", op,
               static_cast<long long>(B), C, static_cast<long long>(T));
  const int64_t chunks = (T + kChunk - 1) / kChunk;
  YAPD_REQUIRE(B < (int64_t{1} << 31) && B * C < (int64_t{1} << 31) / chunks, "%s: too many workgroups", op);
  return YAPD_OK;
}

template <int OP>
int launch_voc(VocParams p, int64_t B, hipStream_t st, const char* what) {
  p.chunks = (p.T + kChunk - 1) / kChunk;
  const void* ptrs[] = {p.x, p.r, p.o0, p.o1, p.o2, p.o3};
  bool aligned = true;
  for (const void* q : ptrs) aligned = aligned && al16f(q);
  p.vec = aligned;
  const dim3 grid(static_cast<unsigned>(B * p.C * p.chunks)), block(kVThreads);
  hipLaunchKernelGGL((voc_kernel<OP>), grid, block, 0, st, p);
  YAPD_LAUNCH_CHECK(what);
  return YAPD_OK;
}

}  // namespace
}  // namespace yapd

using yapd::VocParams;

extern "C" int yapd_snake(const float* x, const float* alpha, const float* bias, float* out, int64_t B, int C,
                          int64_t T, void* stream) {
  if (int rc = yapd::check_bct(x, B, C, T, "snake")) return rc;
  YAPD_REQUIRE(alpha && out, "snake: NULL alpha or out");
  VocParams p{};
  p.x = x;
  p.bias = bias;
  p.a0 = alpha;
  p.o0 = out;
  p.C = C;
  p.T = T;
  return yapd::launch_voc<yapd::kOpSnake>(p, B, static_cast<hipStream_t>(stream), "snake launch");
}

extern "C" int yapd_residual_bias(const float* x, const float* residual, const float* bias, float* out, int64_t B,
                                  int C, int64_t T, void* stream) {
  if (int rc = yapd::check_bct(x, B, C, T, "residual_bias")) return rc;
  YAPD_REQUIRE(residual && bias && out, "residual_bias: NULL residual, bias or out");
  VocParams p{};
  p.x = x;
  p.r = residual;
  p.bias = bias;
  p.o0 = out;
  p.C = C;
  p.T = T;
  return yapd::launch_voc<yapd::kOpResidualBias>(p, B, static_cast<hipStream_t>(stream), "residual_bias launch");
}

extern "C" int yapd_mean3(const float* a, const float* b, const float* c, float* out, int64_t n, void* stream) {
  YAPD_REQUIRE(a && b && c && out, "mean3: NULL pointer");
  YAPD_REQUIRE(n >= 1, "mean3: n must be >= 1");
  const int64_t wgs = (n + yapd::kChunk - 1) / yapd::kChunk;
  YAPD_REQUIRE(wgs < (int64_t{1} << 31), "mean3: too many elements");
  const int vec = yapd::al16f(a) && yapd::al16f(b) && yapd::al16f(c) && yapd::al16f(out);
  hipLaunchKernelGGL(yapd::mean3_kernel, dim3(static_cast<unsigned>(wgs)), dim3(yapd::kVThreads), 0,
                     static_cast<hipStream_t>(stream), a, b, c, out, n, vec);
  YAPD_LAUNCH_CHECK("mean3 launch");
  return YAPD_OK;
}

extern "C" int yapd_residual_bias_snake(const float* x, const float* residual, const float* bias, const float* alpha,
                                        float* raw_out, float* act_out, int64_t B, int C, int64_t T, void* stream) {
  if (int rc = yapd::check_bct(x, B, C, T, "residual_bias_snake")) return rc;
  YAPD_REQUIRE(residual && bias && alpha && raw_out && act_out, "residual_bias_snake: NULL pointer");
  VocParams p{};
  p.x = x;
  p.r = residual;
  p.bias = bias;
  p.a0 = alpha;
  p.o0 = raw_out;
  p.o1 = act_out;
  p.C = C;
  p.T = T;
  return yapd::launch_voc<yapd::kOpResidualBiasSnake>(p, B, static_cast<hipStream_t>(stream),
                                                      "residual_bias_snake launch");
}

extern "C" int yapd_branch_start(const float* x, const float* source, const float* alpha0, const float* alpha1,
                                 const float* alpha2, float* raw_out, float* out0, float* out1, float* out2,
                                 int64_t B, int C, int64_t T, void* stream) {
  if (int rc = yapd::check_bct(x, B, C, T, "branch_start")) return rc;
  YAPD_REQUIRE(source && alpha0 && alpha1 && alpha2 && raw_out && out0 && out1 && out2,
               "branch_start: NULL pointer");
  VocParams p{};
  p.x = x;
  p.r = source;
  p.a0 = alpha0;
  p.a1 = alpha1;
  p.a2 = alpha2;
  p.o0 = raw_out;
  p.o1 = out0;
  p.o2 = out1;
  p.o3 = out2;
  p.C = C;
  p.T = T;
  return yapd::launch_voc<yapd::kOpBranchStart>(p, B, static_cast<hipStream_t>(stream), "branch_start launch");
}
