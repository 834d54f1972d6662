// Key-major V append, one 64-token x D tile of one (b, h) per call: the tile
// goes through LDS so both the token-major reads and the key-major writes are
// 16-byte vector accesses.  Shared by the append kernel (kv_cache.hip) and the
// fused norm/RoPE + V append kernel (rope_norm.hip).
#pragma once

#include "ltx_common.h"

namespace ltx {

constexpr int kTransposeTokens = 64;

// LDS elements one tile needs (row stride D + 2: the column reads of the
// write phase spread over banks).
template <int D>
constexpr int transpose_lds_elems() {
  return kTransposeTokens * (D + 2);
}

// Token tile tx (tokens [64 tx, 64 tx + 64) of L), head h, batch b of src
// [B, L, H, D] (bf16 or float, rows 16-byte aligned) into dst, element
// (b, t, h, d) at b*d_bs + h*d_hs + d*d_ds + t.  All threads of the block
// call it (it has one barrier); any block size works.
template <typename TS, int D>
__device__ __forceinline__ void kv_transpose_tile(const TS* __restrict__ src, int64_t s_bs, int64_t s_ls,
                                                  int64_t s_hs, uint16_t* __restrict__ dst, int64_t d_bs,
                                                  int64_t d_hs, int64_t d_ds, int64_t L, int64_t tx, int h, int b,
                                                  uint16_t* tile) {
  constexpr int TT = kTransposeTokens;
  constexpr int RS = D + 2;
  const int64_t l0 = tx * TT;
  const int rows = (int)((L - l0) < TT ? (L - l0) : TT);
  constexpr int CPR = D / 8;
  for (int idx = threadIdx.x; idx < TT * CPR; idx += blockDim.x) {
    const int r = idx / CPR, c = idx % CPR;
    if (r >= rows) continue;
    const TS* sp = src + b * s_bs + (l0 + r) * s_ls + h * s_hs + c * 8;
    uint32_t w[4];
    if constexpr (sizeof(TS) == 2) {
      const uint4 v = *reinterpret_cast<const uint4*>(sp);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const float4 a = reinterpret_cast<const float4*>(sp)[0];
      const float4 bb = reinterpret_cast<const float4*>(sp)[1];
      w[0] = pack_bf16x2(a.x, a.y); w[1] = pack_bf16x2(a.z, a.w);
      w[2] = pack_bf16x2(bb.x, bb.y); w[3] = pack_bf16x2(bb.z, bb.w);
    }
    uint32_t* tp = reinterpret_cast<uint32_t*>(&tile[r * RS + c * 8]);
#pragma unroll
    for (int i = 0; i < 4; ++i) tp[i] = w[i];
  }
  __syncthreads();
  // write: thread -> (d, 8-token chunk)
  for (int idx = threadIdx.x; idx < D * (TT / 8); idx += blockDim.x) {
    const int d = idx / (TT / 8), ch = idx % (TT / 8);
    const int t0 = ch * 8;
    if (t0 >= rows) continue;
    uint16_t* dp = dst + b * d_bs + h * d_hs + d * d_ds + l0 + t0;
    if (t0 + 8 <= rows) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)tile[(t0 + 2 * i) * RS + d] | ((uint32_t)tile[(t0 + 2 * i + 1) * RS + d] << 16);
      store_stream(dp, make_uint4(w[0], w[1], w[2], w[3]));
    } else {
      for (int i = 0; t0 + i < rows; ++i) dp[i] = tile[(t0 + i) * RS + d];
    }
  }
}

}  // namespace ltx
