// Gated residual update and AdaLN-modulated RMSNorm of the dual-stream block
// (gfx950).
//
// Replaces, per token row of C channels, the bf16 tensor-op chains of
// block_forward_with_cache (ltx_causal/transformer/kv_cache.py:2194-2633):
//   x' = x + y * g            (or x + y)                  -- residual update
//   n  = rms_norm(x') * (1 + scale) + shift  (or rms_norm(x'))  -- next input
// with causal_block.py:94-101's weightless rms_norm.  Every intermediate is
// rounded to bf16 where the reference's bf16 tensor ops round (y*g, the sum,
// the norm, 1 + scale, the product, the shift), so the residual is
// bit-identical and the norm differs only where the float32 sum of squares
// (a different reduction order) flips a rounding.  One workgroup per row,
// C/8 threads, 16-byte loads and stores: one read of x, y and the row's
// modulation vectors, one write of each output.

#include "ltx_common.h"

namespace ltx {

struct AdaArgs {
  const uint16_t* x;
  int64_t x_bs, x_ls;
  const uint16_t* y;      // residual branch output (null: x' = x)
  int64_t y_bs, y_ls;
  const uint16_t* gate;   // per-channel gate (null: x' = x + y)
  int64_t g_bs, g_ls;     // g_ls = 0: one gate row per batch element
  uint16_t* x_out;        // x' (null: not written)
  int64_t xo_bs, xo_ls;
  uint16_t* n_out;        // the normalised row (null: not computed)
  int64_t n_bs, n_ls;
  const uint16_t* scale;  // modulation (null: plain rms_norm)
  int64_t s_bs, s_ls;
  const uint16_t* shift;
  int64_t h_bs, h_ls;
  int64_t L;
  int C;
  float eps;
};

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

struct Bf8 {
  uint4 r;
  __device__ __forceinline__ float get(int i) const {
    const uint32_t w = (&r.x)[i >> 1];
    return bf16_bits_to_f32((i & 1) ? (w >> 16) : (w & 0xFFFFu));
  }
};

__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

__global__ void __launch_bounds__(1024) adaln_kernel(const AdaArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / a.L, l = row % a.L;
  const int c0 = threadIdx.x * 8;
  auto ld = [&](const uint16_t* p, int64_t bs, int64_t ls) {
    Bf8 v;
    v.r = *reinterpret_cast<const uint4*>(p + b * bs + l * ls + c0);
    return v;
  };
  const Bf8 xv = ld(a.x, a.x_bs, a.x_ls);
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = xv.get(i);
  if (a.y != nullptr) {
    const Bf8 yv = ld(a.y, a.y_bs, a.y_ls);
    if (a.gate != nullptr) {
      const Bf8 gv = ld(a.gate, a.g_bs, a.g_ls);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = round_bf16(x[i] + round_bf16(yv.get(i) * gv.get(i)));
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = round_bf16(x[i] + yv.get(i));
    }
  }
  if (a.x_out != nullptr)
    *reinterpret_cast<uint4*>(a.x_out + b * a.xo_bs + l * a.xo_ls + c0) = pack8(x);
  if (a.n_out == nullptr) return;  // uniform across the block

  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    if (off < (int)blockDim.x) ss += __shfl_xor(ss, off, 64);
  __shared__ float red[16];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
  const int nwaves = (blockDim.x + 63) >> 6;
  for (int w = 0; w < nwaves; ++w) tot += red[w];
  const float rs = 1.0f / sqrtf(__fadd_rn(__fdiv_rn(tot, (float)a.C), a.eps));
  float n[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) n[i] = round_bf16(__fmul_rn(x[i], rs));
  if (a.scale != nullptr) {
    const Bf8 sv = ld(a.scale, a.s_bs, a.s_ls), hv = ld(a.shift, a.h_bs, a.h_ls);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float s1 = round_bf16(1.0f + sv.get(i));
      n[i] = round_bf16(round_bf16(n[i] * s1) + hv.get(i));
    }
  }
  *reinterpret_cast<uint4*>(a.n_out + b * a.n_bs + l * a.n_ls + c0) = pack8(n);
}

}  // namespace ltx

using namespace ltx;

extern "C" int ltx_adaln(int64_t B, int64_t L, int64_t C, const void* x, int64_t x_bs, int64_t x_ls,
                         const void* y, int64_t y_bs, int64_t y_ls, const void* gate, int64_t g_bs,
                         int64_t g_ls, void* x_out, int64_t xo_bs, int64_t xo_ls, void* n_out, int64_t n_bs,
                         int64_t n_ls, const void* scale, int64_t s_bs, int64_t s_ls, const void* shift,
                         int64_t h_bs, int64_t h_ls, float eps, void* stream) {
  clear_error();
  LTX_REQUIRE(B >= 1 && L >= 0 && C >= 8 && C % 8 == 0 && C <= 8192, "ltx_adaln: C must be a multiple of 8 in [8, 8192]");
  LTX_REQUIRE(x != nullptr, "ltx_adaln: null x");
  LTX_REQUIRE(gate == nullptr || y != nullptr, "ltx_adaln: a gate needs a residual branch y");
  LTX_REQUIRE((scale == nullptr) == (shift == nullptr), "ltx_adaln: scale and shift go together");
  LTX_REQUIRE(scale == nullptr || n_out != nullptr, "ltx_adaln: modulation needs n_out");
  LTX_REQUIRE(x_out != nullptr || n_out != nullptr, "ltx_adaln: nothing to write");
  LTX_REQUIRE(x_out == nullptr || y != nullptr, "ltx_adaln: x_out without a residual branch");
  LTX_REQUIRE(B * L <= 0x7FFFFFFF, "ltx_adaln: too many rows");
  auto ok = [](const void* p, int64_t bs, int64_t ls) {
    return p == nullptr || (((uintptr_t)p % 16) == 0 && (bs * 2) % 16 == 0 && (ls * 2) % 16 == 0);
  };
  LTX_REQUIRE(ok(x, x_bs, x_ls) && ok(y, y_bs, y_ls) && ok(gate, g_bs, g_ls) && ok(x_out, xo_bs, xo_ls) &&
                  ok(n_out, n_bs, n_ls) && ok(scale, s_bs, s_ls) && ok(shift, h_bs, h_ls),
              "ltx_adaln: rows must be 16-byte aligned");
  if (B * L == 0) return LTX_OK;
  AdaArgs a{(const uint16_t*)x, x_bs, x_ls, (const uint16_t*)y, y_bs, y_ls, (const uint16_t*)gate, g_bs, g_ls,
            (uint16_t*)x_out, xo_bs, xo_ls, (uint16_t*)n_out, n_bs, n_ls, (const uint16_t*)scale, s_bs, s_ls,
            (const uint16_t*)shift, h_bs, h_ls, L, (int)C, eps};
  hipLaunchKernelGGL(adaln_kernel, dim3((unsigned)(B * L)), dim3((unsigned)(C / 8)), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  LTX_LAUNCH_CHECK("ltx_adaln");
  return LTX_OK;
}
