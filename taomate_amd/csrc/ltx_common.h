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

// fl(x / sc) given r = fl(1 / sc).  fl(x * r) is within 3 ulp of fl(x / sc),
// so both round to the same e4m3 value unless the quotient lies next to a
// rounding midpoint of the e4m3 grid (low 20 mantissa bits near 0x80000) or in
// the e4m3 subnormal range (below 2^-6); only those lanes pay for the exact
// division.  The result is only meant for rounding to e4m3.
__device__ __forceinline__ float quotient_for_e4m3(float x, float sc, float r) {
  const float q = x * r;
  const float a = fabsf(q);
  const uint32_t low = __float_as_uint(a) & 0xFFFFFu;
  if (a < 0.015625f || low - 0x7FFFCu <= 8u) return __fdiv_rn(x, sc);
  return q;
}

// quotient_for_e4m3 for a chunk of N values with one branch per chunk: the
// products x * r are straight-line code, and only a chunk holding a lane near
// a midpoint or in the subnormal range redoes its values with the exact
// division (same results as quotient_for_e4m3 element by element).
template <int N>
__device__ __forceinline__ void quotients_for_e4m3(const float (&x)[N], float sc, float r, float (&q)[N]) {
  bool slow = false;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = x[i] * r;
    const float a = fabsf(q[i]);
    const uint32_t low = __float_as_uint(a) & 0xFFFFFu;
    slow |= (a < 0.015625f) | (low - 0x7FFFCu <= 8u);
  }
  if (slow) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = quotient_for_e4m3(x[i], sc, r);
  }
}

// Four float32 values -> four OCP e4m3fn codes (byte i = value i): clamp to
// +-448, then the gfx950 converter rounds to nearest even.
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  const float m = 448.0f;
  a = __builtin_amdgcn_fmed3f(a, -m, m);
  b = __builtin_amdgcn_fmed3f(b, -m, m);
  c = __builtin_amdgcn_fmed3f(c, -m, m);
  d = __builtin_amdgcn_fmed3f(d, -m, m);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
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
