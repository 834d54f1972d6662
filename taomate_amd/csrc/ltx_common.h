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
// Stores of outputs that the writing launch never reads back, marked
// non-temporal.  A kernel's ordinary stores stay dirty in the writing XCD's
// L2 and are written back when the kernel ends, a phase with no other work;
// streaming stores leave the L2 while the kernel still runs.  Measured at a
// 1152-token chunk of 32 x 128 heads, B = 2: the fp8 K+V quantise 12.9 ->
// 10.4 us, the key-major V append 6.7 -> 5.5 us.  Stores that cover only
// part of a line per instruction got slower this way (the attention output
// written 8 bytes per lane over 32 rows: 159 -> 176 us per call), so the
// attention stages its output to whole rows first; the norm + RoPE rows
// showed no change.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_stream(void* p, uint4 v) {
  const u32x4_t x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void store_stream(void* p, uint2 v) {
  const u32x2_t x = {v.x, v.y};
  __builtin_nontemporal_store(x, reinterpret_cast<u32x2_t*>(p));
}

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

// Frame maxima m >= kCorrectedMinMax quantise with quotient_e4m3_corrected:
// for every bf16 maximum m >= 2^-96 and every bf16 value x with |x| <= m, the
// e4m3 code of quotient_e4m3_corrected(x, sc, fl(1 / sc)), sc = fl(m / 448),
// equals the code of fl(x / sc) (checked exhaustively over all such pairs by
// the CPU tests).  Below it (maxima of 2^-96 and less) the division is exact.
constexpr float kCorrectedMinMax = 0x1p-96f;

// fl(x / sc) up to last bits that cannot change an e4m3 code (see
// kCorrectedMinMax): q = fl(x * r) for r = fl(1 / sc), the negated residual
// q * sc - x in one fused multiply-add (round to nearest even is symmetric, so
// it is exactly minus the residual x - q * sc), then one correction
// q - negated_residual * r (Markstein's correction step).  Written this way a
// zero x keeps its sign (x = -0: q = -0, the negated residual +0, and
// -0 + -0 = -0) without a separate copysign.  Straight line: one multiply
// and two FMAs per value.
__device__ __forceinline__ float quotient_e4m3_corrected(float x, float sc, float r) {
  const float q = __fmul_rn(x, r);
  const float ne = __fmaf_rn(q, sc, -x);
  return __fmaf_rn(-ne, r, q);
}

// Quotients of a chunk of bf16-sourced values for e4m3 rounding: the corrected
// quotient when the frame maximum allows it (a workgroup-uniform choice), the
// exact division otherwise.
template <int N>
__device__ __forceinline__ void quotients_e4m3_bf16(const float (&x)[N], float sc, float r, bool corrected,
                                                    float (&q)[N]) {
  if (corrected) {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = quotient_e4m3_corrected(x[i], sc, r);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = __fdiv_rn(x[i], sc);
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
