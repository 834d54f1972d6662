// Shared device/host helpers for the gfx950 LTX attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/taomate_ltx.h"

namespace ltx {

// ---------------------------------------------------------------------------
// Error reporting: one message per host thread, returned by ltx_last_error().
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define LTX_REQUIRE(cond, ...)              \
  do {                                      \
    if (!(cond)) {                          \
      ::ltx::set_error(__VA_ARGS__);        \
      return LTX_EINVAL;                    \
    }                                       \
  } while (0)

#define LTX_LAUNCH_CHECK(name)                                                   \
  do {                                                                           \
    hipError_t _e = hipGetLastError();                                           \
    if (_e != hipSuccess) {                                                      \
      ::ltx::set_error("%s: launch failed: %s", name, hipGetErrorString(_e));    \
      return LTX_ELAUNCH;                                                        \
    }                                                                            \
  } while (0)

// ---------------------------------------------------------------------------
// Scalar conversions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// float32 -> bf16 bits, round to nearest even (gfx950 lowers this to
// v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

// Two float32 -> packed bf16x2 (low half = a), one v_cvt_pk_bf16_f32.
typedef __bf16 ltx_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float ltx_f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const ltx_f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ltx_bf16x2_t));
}

// OCP float8_e4m3fn encode: round to nearest even, saturating at +-448,
// NaN -> 0x7F.  Written from the format definition (1 sign, 4 exponent bits
// with bias 7, 3 mantissa bits, no infinities, S.1111.111 = NaN).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  float a = fabsf(x);
  if (!(a == a)) return 0x7Fu;             // NaN
  if (a >= 448.0f) return sign | 0x7Eu;    // saturate
  if (a < 0.015625f) {                     // below 2^-6: subnormal grid of 2^-9
    // a / 2^-9 rounded to nearest even integer in [0, 8]; 8 is the smallest normal.
    float m = __builtin_rintf(a * 512.0f);
    return sign | (uint32_t)m;             // m == 8 encodes 2^-6 exactly (0x08)
  }
  uint32_t ua = __float_as_uint(a);
  // keep 3 mantissa bits with round-to-nearest-even on the dropped 20 bits
  uint32_t lsb = (ua >> 20) & 1u;
  ua += 0x7FFFFu + lsb;
  uint32_t e = (ua >> 23) - 127u + 7u;     // rebias (ua >= 2^-6 so e >= 1)
  uint32_t m = (ua >> 20) & 7u;
  uint32_t code = (e << 3) | m;
  if (code > 0x7Eu) code = 0x7Eu;           // rounding carried past 448
  return sign | code;
}

// OCP float8_e4m3fn decode to float32 (exact).
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t sign = (c & 0x80u) << 24;
  uint32_t e = (c >> 3) & 0xFu;
  uint32_t m = c & 7u;
  float v;
  if (e == 0) {
    v = (float)m * 0.001953125f;  // m * 2^-9
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  if ((c & 0x7Fu) == 0x7Fu) v = __uint_as_float(0x7FC00000u);
  return __uint_as_float(__float_as_uint(v) | sign);
}

template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const uint16_t* p) {
  return bf16_bits_to_f32(*p);
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace ltx
