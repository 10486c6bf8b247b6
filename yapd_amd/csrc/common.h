// Shared helpers for the gfx950 kernels of the T3 block step.
//
// bf16 values travel as raw uint16_t; conversions are explicit so every
// rounding point is visible (round-to-nearest-even, the same as torch's
// float -> bfloat16 cast).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/yapd_t3.h"

namespace yapd {

// Records a printf-style message for yapd_last_error() (thread-local).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Translates a HIP status into YAPD_OK / YAPD_EHIP with a message.
int check_hip(hipError_t e, const char* what);

}  // namespace yapd

#define YAPD_REQUIRE(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      ::yapd::set_error(__VA_ARGS__);        \
      return YAPD_EINVAL;                    \
    }                                        \
  } while (0)

#define YAPD_LAUNCH_CHECK(what)                                  \
  do {                                                           \
    int _rc = ::yapd::check_hip(hipGetLastError(), (what));      \
    if (_rc != YAPD_OK) return _rc;                              \
  } while (0)

namespace yapd {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

__device__ __forceinline__ float bf16_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// fp32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32, the same
// rounding as torch's float -> bfloat16 cast).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

}  // namespace yapd
