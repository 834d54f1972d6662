// KV-cache append (copy or fp8-e4m3 quantise) and span gather (compaction).
//
// The reference appends with torch.cat, reallocating and copying the whole cache
// on every commit (ltx_causal/transformer/kv_cache.py:394-398, :2642-2656), and
// evicts by slicing and re-concatenating segment spans (taomate/inference/
// cache.py:28-67).  Here the cache is a preallocated arena: append writes only
// the new tokens into their slots, eviction is slot bookkeeping on the host,
// and gather is the optional physical compaction of the surviving spans.

#include <type_traits>

#include "ltx_common.h"
#include "kv_transpose.h"

namespace ltx {

// One thread moves one 16-byte chunk of a (b, l, h) row.
template <typename TS>
__global__ void kv_copy_kernel(const TS* __restrict__ src, int64_t s_bs, int64_t s_ls, int64_t s_hs,
                               uint16_t* __restrict__ dst, int64_t d_bs, int64_t d_ls, int64_t d_hs,
                               int64_t L, int H, int D) {
  const int cpr = D / 8;  // 8 elements per chunk
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= L * H * cpr) return;
  const int b = blockIdx.y;
  const int c = (int)(gid % cpr);
  const int64_t lh = gid / cpr;
  const int h = (int)(lh % H);
  const int64_t l = lh / H;
  const TS* s = src + b * s_bs + l * s_ls + h * s_hs + c * 8;
  uint16_t* d = dst + b * d_bs + l * d_ls + h * d_hs + c * 8;
  if constexpr (sizeof(TS) == 2) {
    store_stream(d, *reinterpret_cast<const uint4*>(s));
  } else {
    float4 a = reinterpret_cast<const float4*>(s)[0];
    float4 bb = reinterpret_cast<const float4*>(s)[1];
    uint4 o;
    o.x = pack_bf16x2(a.x, a.y);
    o.y = pack_bf16x2(a.z, a.w);
    o.z = pack_bf16x2(bb.x, bb.y);
    o.w = pack_bf16x2(bb.z, bb.w);
    store_stream(d, o);
  }
}

// One workgroup of kQuantThreads per (frame, h, b): absmax over the frame's
// frame_tokens x D values, then quantise.  Each thread keeps its first
// kQuantRegs 8-value chunks in registers between the two passes, so frames of
// up to kQuantThreads * kQuantRegs chunks are read from memory once; chunks
// beyond that are read again in the second pass.
constexpr int kQuantThreads = 1024;
constexpr int kQuantRegs = 8;

// CPR: 8-value chunks per row (D / 8) when known at compile time, 0 otherwise.
template <typename TS, int CPR>
__global__ void __launch_bounds__(kQuantThreads) kv_quant_kernel(
    const TS* __restrict__ src, int64_t s_bs, int64_t s_ls, int64_t s_hs, uint8_t* __restrict__ dst,
    int64_t d_bs, int64_t d_ls, int64_t d_hs, float* __restrict__ scales, int64_t sc_bs,
    int64_t sc_hs, int frame_tokens, int D) {
  const int f = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int cpr = CPR > 0 ? CPR : D / 8;
  const int n = frame_tokens * cpr;  // 8-element chunks in this (frame, head)
  const int64_t l0 = (int64_t)f * frame_tokens;
  const TS* sbase = src + b * s_bs + l0 * s_ls + h * s_hs;
  uint8_t* dbase = dst + b * d_bs + l0 * d_ls + h * d_hs;

  auto load8 = [&](int idx, float* v) {
    const int t = idx / cpr, c = idx % cpr;
    const TS* p = sbase + (int64_t)t * s_ls + c * 8;
    if constexpr (sizeof(TS) == 2) {
      uint4 r = *reinterpret_cast<const uint4*>(p);
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_bits_to_f32(w[i] & 0xFFFFu);
        v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
      }
    } else {
      float4 a = reinterpret_cast<const float4*>(p)[0];
      float4 bb = reinterpret_cast<const float4*>(p)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = bb.x; v[5] = bb.y; v[6] = bb.z; v[7] = bb.w;
    }
  };
  auto store8 = [&](int idx, const float (&v)[8], float sc, float r, bool corrected) {
    float q[8];
    if constexpr (sizeof(TS) == 2)
      quotients_e4m3_bf16(v, sc, r, corrected, q);
    else
      quotients_for_e4m3(v, sc, r, q);
    const uint32_t lo = pack4_e4m3(q[0], q[1], q[2], q[3]);
    const uint32_t hi = pack4_e4m3(q[4], q[5], q[6], q[7]);
    const int t = idx / cpr, c = idx % cpr;
    store_stream(dbase + (int64_t)t * d_ls + c * 8, make_uint2(lo, hi));
  };

  float v[kQuantRegs][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kQuantRegs; ++i) {
    const int idx = threadIdx.x + i * kQuantThreads;
    if (idx < n) {
      load8(idx, v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    }
  }
  for (int idx = threadIdx.x + kQuantRegs * kQuantThreads; idx < n; idx += kQuantThreads) {
    float t[8];
    load8(idx, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(t[e]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  constexpr int kWaves = kQuantThreads / 64;
  __shared__ float red[kWaves];
  __shared__ float scale_s, max_s;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = red[0];
    for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[w]);
    const float sc = m > 0.0f ? __fdiv_rn(m, 448.0f) : 1.0f;
    scale_s = sc;
    max_s = m;
    scales[b * sc_bs + h * sc_hs + f] = sc;
  }
  __syncthreads();
  const float sc = scale_s;
  const float r = __fdiv_rn(1.0f, sc);
  const bool corrected = max_s >= kCorrectedMinMax;
#pragma unroll
  for (int i = 0; i < kQuantRegs; ++i) {
    const int idx = threadIdx.x + i * kQuantThreads;
    if (idx < n) store8(idx, v[i], sc, r, corrected);
  }
  for (int idx = threadIdx.x + kQuantRegs * kQuantThreads; idx < n; idx += kQuantThreads) {
    float t[8];
    load8(idx, t);
    store8(idx, t, sc, r, corrected);
  }
}

// fp8 quantise of bf16 rows: one 1024-thread workgroup per (frame, h, b,
// tensor), each thread holding up to kPairRegs raw 16-byte chunks (8 bf16) of
// its frame between the absmax pass and the quantise pass, so the frame is
// read from memory once (chunks past kPairRegs * 1024 are read again; a 16x24
// frame of a 128-wide head is exactly 6 chunks per thread).  K and V go in one
// launch (blockIdx.z = b + B * tensor): a 16x24 frame of 32 x 128 heads at
// B = 2 is 384 workgroups, one round at two workgroups per CU (56 VGPRs; the
// eighth register pair of an earlier version cost the second workgroup).  The
// quotients are the corrected ones of quotients_e4m3_bf16, the same as
// kv_quant_kernel's for bf16 sources, so codes and scales are bit-identical
// to it for finite inputs.
constexpr int kPairThreads = 1024;
constexpr int kPairRegs = 6;

struct QuantTensor {
  const uint16_t* src;
  int64_t s_bs, s_ls, s_hs;
  uint8_t* dst;
  float* scales;
};
struct QuantPair {
  QuantTensor t[2];
  int64_t d_bs, d_ls, d_hs, sc_bs, sc_hs;
  int B, frame_tokens, D;
};

// OFF32: every element offset of the sources and destinations fits in 31 bits
// (checked on the host), so addresses are computed in 32-bit arithmetic.
template <int CPR, bool OFF32>
__global__ void __launch_bounds__(kPairThreads) kv_quant_pair_kernel(const QuantPair a) {
  using Off = std::conditional_t<OFF32, int32_t, int64_t>;
  const int f = blockIdx.x, h = blockIdx.y;
  const bool second = blockIdx.z >= (unsigned)a.B;
  const int b = blockIdx.z - (second ? a.B : 0);
  // per-tensor fields by scalar selects (no indexing of the kernel-argument array)
  const uint16_t* src = second ? a.t[1].src : a.t[0].src;
  uint8_t* dst = second ? a.t[1].dst : a.t[0].dst;
  float* scales = second ? a.t[1].scales : a.t[0].scales;
  const Off s_ls = (Off)(second ? a.t[1].s_ls : a.t[0].s_ls);
  const Off s_off = (Off)b * (Off)(second ? a.t[1].s_bs : a.t[0].s_bs) + (Off)h * (Off)(second ? a.t[1].s_hs : a.t[0].s_hs);
  const Off d_ls = (Off)a.d_ls;
  const int cpr = CPR > 0 ? CPR : a.D / 8;
  const int n = a.frame_tokens * cpr;
  const Off l0 = (Off)f * a.frame_tokens;
  const uint16_t* sbase = src + (s_off + l0 * s_ls);
  uint8_t* dbase = dst + ((Off)b * (Off)a.d_bs + l0 * d_ls + (Off)h * (Off)a.d_hs);
  auto load = [&](int idx) {
    const int t = idx / cpr, c = idx % cpr;
    return *reinterpret_cast<const uint4*>(sbase + ((Off)t * s_ls + c * 8));
  };
  // absmax as the largest bf16 magnitude, two values per packed 16-bit max
  // (magnitude bits order as the values; a NaN in the frame gives a NaN
  // scale, as a float amax would)
  typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));
  auto amax8 = [&](uint4 r, ushort2_t m) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(ushort2_t, w[i] & 0x7FFF7FFFu));
    return m;
  };
  auto store = [&](int idx, uint4 r, float sc, float rc, bool corrected) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    float x[8], q[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16_bits_to_f32(w[i] & 0xFFFFu);
      x[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
    quotients_e4m3_bf16(x, sc, rc, corrected, q);
    const int t = idx / cpr, c = idx % cpr;
    store_stream(dbase + ((Off)t * d_ls + c * 8),
                 make_uint2(pack4_e4m3(q[0], q[1], q[2], q[3]), pack4_e4m3(q[4], q[5], q[6], q[7])));
  };

  uint4 raw[kPairRegs];
#pragma unroll
  for (int i = 0; i < kPairRegs; ++i) {
    const int idx = threadIdx.x + i * kPairThreads;
    raw[i] = idx < n ? load(idx) : make_uint4(0, 0, 0, 0);
  }
  ushort2_t am = {0, 0};
#pragma unroll
  for (int i = 0; i < kPairRegs; ++i) am = amax8(raw[i], am);
  // keep only the raw chunks live across the reduction (the quantise pass
  // converts them again instead of holding 8 floats per chunk)
#pragma unroll
  for (int i = 0; i < kPairRegs; ++i)
    asm volatile("" : "+v"(raw[i].x), "+v"(raw[i].y), "+v"(raw[i].z), "+v"(raw[i].w));
  for (int idx = threadIdx.x + kPairRegs * kPairThreads; idx < n; idx += kPairThreads) am = amax8(load(idx), am);
  uint32_t mbits = am.x > am.y ? am.x : am.y;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)mbits, off, 64);
    mbits = o > mbits ? o : mbits;
  }
  constexpr int kWaves = kPairThreads / 64;
  __shared__ uint32_t red[kWaves];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mbits;
  __syncthreads();
  uint32_t mb = red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) mb = red[w] > mb ? red[w] : mb;
  const float m = bf16_bits_to_f32(mb);
  const float sc = m == 0.0f ? 1.0f : __fdiv_rn(m, 448.0f);
  if (threadIdx.x == 0) scales[b * a.sc_bs + h * a.sc_hs + f] = sc;
  const float rc = __fdiv_rn(1.0f, sc);
  const bool corrected = m >= kCorrectedMinMax;
#pragma unroll
  for (int i = 0; i < kPairRegs; ++i) {
    const int idx = threadIdx.x + i * kPairThreads;
    if (idx < n) store(idx, raw[i], sc, rc, corrected);
  }
  for (int idx = threadIdx.x + kPairRegs * kPairThreads; idx < n; idx += kPairThreads)
    store(idx, load(idx), sc, rc, corrected);
}

// Whether every element offset the pair kernel forms fits in 31 bits.
inline bool pair_offsets_fit(const QuantPair& a, int ntensors, int64_t L, int64_t H) {
  const int64_t lim = 0x7FFFFFFF;
  auto ok = [&](int64_t bs, int64_t ls, int64_t hs) {
    if (bs < 0 || ls < 0 || hs < 0 || bs > lim || ls > lim || hs > lim) return false;
    return (a.B - 1) * bs + (L - 1) * ls + (H - 1) * hs + a.D <= lim;
  };
  for (int t = 0; t < ntensors; ++t)
    if (!ok(a.t[t].s_bs, a.t[t].s_ls, a.t[t].s_hs)) return false;
  return ok(a.d_bs, a.d_ls, a.d_hs);
}

inline int launch_quant_pair(const QuantPair& a, int ntensors, int64_t L, int64_t H, hipStream_t st) {
  const dim3 grid((unsigned)(L / a.frame_tokens), (unsigned)H, (unsigned)(a.B * ntensors));
  const bool off32 = pair_offsets_fit(a, ntensors, L, H);
#define LTX_QP(CPR)                                                                        \
  do {                                                                                     \
    if (off32)                                                                             \
      hipLaunchKernelGGL((kv_quant_pair_kernel<CPR, true>), grid, dim3(kPairThreads), 0, st, a);  \
    else                                                                                   \
      hipLaunchKernelGGL((kv_quant_pair_kernel<CPR, false>), grid, dim3(kPairThreads), 0, st, a); \
  } while (0)
  if (a.D == 128)
    LTX_QP(16);
  else if (a.D == 64)
    LTX_QP(8);
  else
    LTX_QP(0);
#undef LTX_QP
  return LTX_OK;
}

// Key-major append: one block per 64-token tile of one (b, h) (kv_transpose.h).
template <typename TS, int D>
__global__ void __launch_bounds__(256) kv_transpose_kernel(
    const TS* __restrict__ src, int64_t s_bs, int64_t s_ls, int64_t s_hs, uint16_t* __restrict__ dst,
    int64_t d_bs, int64_t d_hs, int64_t d_ds, int64_t L) {
  __shared__ uint16_t tile[transpose_lds_elems<D>()];
  kv_transpose_tile<TS, D>(src, s_bs, s_ls, s_hs, dst, d_bs, d_hs, d_ds, L, blockIdx.x, blockIdx.y, blockIdx.z,
                           tile);
}

struct SpanTable {
  int64_t src_start[LTX_MAX_SEGMENTS];
  int64_t dst_start[LTX_MAX_SEGMENTS + 1];
  int n;
};

// One thread per 4-byte word of a destination (b, l, h) row.
__global__ void kv_gather_kernel(const uint32_t* __restrict__ src, int64_t s_bs, int64_t s_ls,
                                 int64_t s_hs, uint32_t* __restrict__ dst, int64_t d_bs,
                                 int64_t d_ls, int64_t d_hs, SpanTable spans, int H, int wpr) {
  const int64_t Ltot = spans.dst_start[spans.n];
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= Ltot * H * wpr) return;
  const int b = blockIdx.y;
  const int w = (int)(gid % wpr);
  const int64_t lh = gid / wpr;
  const int h = (int)(lh % H);
  const int64_t l = lh / H;
  int s = 0;
#pragma unroll
  for (int i = 1; i < LTX_MAX_SEGMENTS; ++i)
    if (i < spans.n && l >= spans.dst_start[i]) s = i;
  const int64_t sl = spans.src_start[s] + (l - spans.dst_start[s]);
  dst[b * d_bs + l * d_ls + h * d_hs + w] = src[b * s_bs + sl * s_ls + h * s_hs + w];
}

}  // namespace ltx

using namespace ltx;

extern "C" int ltx_kv_append(int src_dtype, int dst_dtype, int64_t B, int64_t L, int64_t H,
                             int64_t D, const void* src, int64_t s_bs, int64_t s_ls, int64_t s_hs,
                             void* dst, int64_t d_bs, int64_t d_ls, int64_t d_hs, int64_t d_ds,
                             float* scales, int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                             void* stream) {
  clear_error();
  LTX_REQUIRE(src_dtype == LTX_BF16 || src_dtype == LTX_F32, "ltx_kv_append: src_dtype must be BF16 or F32");
  LTX_REQUIRE(dst_dtype == LTX_BF16 || dst_dtype == LTX_F8E4M3,
              "ltx_kv_append: dst_dtype must be BF16 or F8E4M3");
  LTX_REQUIRE(B >= 1 && B <= 65535 && L >= 0 && H >= 1 && H <= 65535 && D >= 8 && D % 8 == 0,
              "ltx_kv_append: bad shape");
  if (L == 0) return LTX_OK;  // nothing to append (an empty tensor may have no storage)
  LTX_REQUIRE(src && dst, "ltx_kv_append: null pointer");
  const int64_t ssz = src_dtype == LTX_BF16 ? 2 : 4;
  const int64_t dsz = dst_dtype == LTX_BF16 ? 2 : 1;
  LTX_REQUIRE(((uintptr_t)src % 16) == 0 && (s_bs * ssz) % 16 == 0 && (s_ls * ssz) % 16 == 0 &&
                  (s_hs * ssz) % 16 == 0,
              "ltx_kv_append: src must be 16-byte aligned per row");
  if (L == 0) return LTX_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (d_ds != 1) {
    LTX_REQUIRE(d_ls == 1 && dst_dtype == LTX_BF16, "ltx_kv_append: dst must be token-major (d_ds == 1) "
                "or bf16 key-major (d_ls == 1)");
    LTX_REQUIRE(D == 64 || D == 128, "ltx_kv_append: key-major append supports D in {64, 128}");
    LTX_REQUIRE(((uintptr_t)dst % 16) == 0 && (d_bs * 2) % 16 == 0 && (d_hs * 2) % 16 == 0 &&
                    (d_ds * 2) % 16 == 0,
                "ltx_kv_append: key-major dst must start on a 16-byte boundary (8-slot aligned)");
    const dim3 grid((unsigned)ceil_div(L, 64), (unsigned)H, (unsigned)B);
#define LTX_TRANSPOSE(TS, DD)                                                                     \
  hipLaunchKernelGGL((kv_transpose_kernel<TS, DD>), grid, dim3(256), 0, st, (const TS*)src, s_bs, s_ls, \
                     s_hs, (uint16_t*)dst, d_bs, d_hs, d_ds, L)
    if (src_dtype == LTX_BF16) {
      if (D == 128) LTX_TRANSPOSE(uint16_t, 128); else LTX_TRANSPOSE(uint16_t, 64);
    } else {
      if (D == 128) LTX_TRANSPOSE(float, 128); else LTX_TRANSPOSE(float, 64);
    }
#undef LTX_TRANSPOSE
    LTX_LAUNCH_CHECK("ltx_kv_append");
    return LTX_OK;
  }
  LTX_REQUIRE(((uintptr_t)dst % 8) == 0 && (d_bs * dsz) % 8 == 0 && (d_ls * dsz) % 8 == 0 &&
                  (d_hs * dsz) % 8 == 0,
              "ltx_kv_append: dst must be 8-byte aligned per row");
  if (dst_dtype == LTX_BF16) {
    LTX_REQUIRE(((uintptr_t)dst % 16) == 0 && (d_bs * 2) % 16 == 0 && (d_ls * 2) % 16 == 0 &&
                    (d_hs * 2) % 16 == 0,
                "ltx_kv_append: bf16 dst must be 16-byte aligned per row");
    const int64_t n = L * H * (D / 8);
    const dim3 grid((unsigned)ceil_div(n, 256), (unsigned)B);
    if (src_dtype == LTX_BF16)
      hipLaunchKernelGGL(kv_copy_kernel<uint16_t>, grid, dim3(256), 0, st, (const uint16_t*)src, s_bs,
                         s_ls, s_hs, (uint16_t*)dst, d_bs, d_ls, d_hs, L, (int)H, (int)D);
    else
      hipLaunchKernelGGL(kv_copy_kernel<float>, grid, dim3(256), 0, st, (const float*)src, s_bs, s_ls,
                         s_hs, (uint16_t*)dst, d_bs, d_ls, d_hs, L, (int)H, (int)D);
  } else {
    LTX_REQUIRE(scales != nullptr, "ltx_kv_append: fp8 needs a scales buffer");
    LTX_REQUIRE(frame_tokens >= 1 && L % frame_tokens == 0,
                "ltx_kv_append: L (%lld) must be a multiple of frame_tokens (%lld)", (long long)L,
                (long long)frame_tokens);
    if (src_dtype == LTX_BF16) {
      QuantPair a{};
      a.t[0] = QuantTensor{(const uint16_t*)src, s_bs, s_ls, s_hs, (uint8_t*)dst, scales};
      a.d_bs = d_bs; a.d_ls = d_ls; a.d_hs = d_hs; a.sc_bs = sc_bs; a.sc_hs = sc_hs;
      a.B = (int)B; a.frame_tokens = (int)frame_tokens; a.D = (int)D;
      launch_quant_pair(a, 1, L, H, st);
      LTX_LAUNCH_CHECK("ltx_kv_append");
      return LTX_OK;
    }
    const dim3 grid((unsigned)(L / frame_tokens), (unsigned)H, (unsigned)B);
    auto launch = [&](auto tag, auto cpr) {
      using TS = decltype(tag);
      hipLaunchKernelGGL((kv_quant_kernel<TS, decltype(cpr)::value>), grid, dim3(kQuantThreads), 0, st,
                         (const TS*)src, s_bs, s_ls, s_hs, (uint8_t*)dst, d_bs, d_ls, d_hs, scales,
                         sc_bs, sc_hs, (int)frame_tokens, (int)D);
    };
    using C16 = std::integral_constant<int, 16>;
    using C8 = std::integral_constant<int, 8>;
    using C0 = std::integral_constant<int, 0>;
    if (src_dtype == LTX_BF16) {
      if (D == 128) launch(uint16_t{}, C16{});
      else if (D == 64) launch(uint16_t{}, C8{});
      else launch(uint16_t{}, C0{});
    } else {
      if (D == 128) launch(float{}, C16{});
      else if (D == 64) launch(float{}, C8{});
      else launch(float{}, C0{});
    }
  }
  LTX_LAUNCH_CHECK("ltx_kv_append");
  return LTX_OK;
}

extern "C" int ltx_kv_gather(int64_t elem_bytes, int64_t B, int64_t H, int64_t D, const void* src,
                             int64_t s_bs, int64_t s_ls, int64_t s_hs, void* dst, int64_t d_bs,
                             int64_t d_ls, int64_t d_hs, int64_t n_spans, const int64_t* starts,
                             const int64_t* lens, void* stream) {
  clear_error();
  LTX_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "ltx_kv_gather: elem_bytes must be 1, 2 or 4");
  LTX_REQUIRE(B >= 1 && B <= 65535 && H >= 1 && D >= 1 && (D * elem_bytes) % 4 == 0,
              "ltx_kv_gather: D*elem_bytes must be a multiple of 4");
  LTX_REQUIRE(n_spans >= 0 && n_spans <= LTX_MAX_SEGMENTS, "ltx_kv_gather: at most %d spans",
              LTX_MAX_SEGMENTS);
  LTX_REQUIRE(src && dst && (n_spans == 0 || (starts && lens)), "ltx_kv_gather: null pointer");
  LTX_REQUIRE(((uintptr_t)src % 4) == 0 && ((uintptr_t)dst % 4) == 0 && (s_bs * elem_bytes) % 4 == 0 &&
                  (s_ls * elem_bytes) % 4 == 0 && (s_hs * elem_bytes) % 4 == 0 &&
                  (d_bs * elem_bytes) % 4 == 0 && (d_ls * elem_bytes) % 4 == 0 &&
                  (d_hs * elem_bytes) % 4 == 0,
              "ltx_kv_gather: rows must be 4-byte aligned");
  SpanTable t{};
  t.n = (int)n_spans;
  t.dst_start[0] = 0;
  for (int i = 0; i < n_spans; ++i) {
    LTX_REQUIRE(starts[i] >= 0 && lens[i] >= 0, "ltx_kv_gather: negative span");
    t.src_start[i] = starts[i];
    t.dst_start[i + 1] = t.dst_start[i] + lens[i];
  }
  const int64_t Ltot = t.dst_start[n_spans];
  if (Ltot == 0) return LTX_OK;
  if (t.n == 0) return LTX_OK;
  // drop empty spans so every span in the table owns at least one token
  SpanTable c{};
  c.dst_start[0] = 0;
  for (int i = 0; i < t.n; ++i) {
    const int64_t len = t.dst_start[i + 1] - t.dst_start[i];
    if (len == 0) continue;
    c.src_start[c.n] = t.src_start[i];
    c.dst_start[c.n + 1] = c.dst_start[c.n] + len;
    c.n++;
  }
  const int wpr = (int)(D * elem_bytes / 4);
  const int64_t w = 4 / elem_bytes;  // elements per word
  const int64_t n = Ltot * H * wpr;
  const dim3 grid((unsigned)ceil_div(n, 256), (unsigned)B);
  hipLaunchKernelGGL(kv_gather_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     (const uint32_t*)src, s_bs / w, s_ls / w, s_hs / w, (uint32_t*)dst, d_bs / w,
                     d_ls / w, d_hs / w, c, (int)H, wpr);
  LTX_LAUNCH_CHECK("ltx_kv_gather");
  return LTX_OK;
}

extern "C" int ltx_kv_append_fp8_pair(int64_t B, int64_t L, int64_t H, int64_t D, int64_t frame_tokens,
                                      const void* k_src, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                                      void* k_dst, float* k_scales, const void* v_src, int64_t v_bs,
                                      int64_t v_ls, int64_t v_hs, void* v_dst, float* v_scales,
                                      int64_t d_bs, int64_t d_ls, int64_t d_hs, int64_t sc_bs,
                                      int64_t sc_hs, void* stream) {
  clear_error();
  LTX_REQUIRE(B >= 1 && B <= 32767 && L >= 0 && H >= 1 && H <= 65535 && D >= 8 && D % 8 == 0,
              "ltx_kv_append_fp8_pair: bad shape");
  LTX_REQUIRE(k_src && v_src && k_dst && v_dst && k_scales && v_scales, "ltx_kv_append_fp8_pair: null pointer");
  LTX_REQUIRE(frame_tokens >= 1 && L % frame_tokens == 0,
              "ltx_kv_append_fp8_pair: L (%lld) must be a multiple of frame_tokens (%lld)", (long long)L,
              (long long)frame_tokens);
  LTX_REQUIRE(L / frame_tokens <= 0x7FFFFFFF, "ltx_kv_append_fp8_pair: too many frames");
  auto al = [](const void* p, uintptr_t n) { return ((uintptr_t)p % n) == 0; };
  LTX_REQUIRE(al(k_src, 16) && al(v_src, 16) && (k_bs * 2) % 16 == 0 && (k_ls * 2) % 16 == 0 &&
                  (k_hs * 2) % 16 == 0 && (v_bs * 2) % 16 == 0 && (v_ls * 2) % 16 == 0 && (v_hs * 2) % 16 == 0,
              "ltx_kv_append_fp8_pair: sources must be 16-byte aligned per row");
  LTX_REQUIRE(al(k_dst, 8) && al(v_dst, 8) && d_bs % 8 == 0 && d_ls % 8 == 0 && d_hs % 8 == 0,
              "ltx_kv_append_fp8_pair: destinations must be 8-byte aligned per row");
  if (L == 0) return LTX_OK;
  QuantPair a{};
  a.t[0] = QuantTensor{(const uint16_t*)k_src, k_bs, k_ls, k_hs, (uint8_t*)k_dst, k_scales};
  a.t[1] = QuantTensor{(const uint16_t*)v_src, v_bs, v_ls, v_hs, (uint8_t*)v_dst, v_scales};
  a.d_bs = d_bs; a.d_ls = d_ls; a.d_hs = d_hs; a.sc_bs = sc_bs; a.sc_hs = sc_hs;
  a.B = (int)B; a.frame_tokens = (int)frame_tokens; a.D = (int)D;
  launch_quant_pair(a, 2, L, H, reinterpret_cast<hipStream_t>(stream));
  LTX_LAUNCH_CHECK("ltx_kv_append_fp8_pair");
  return LTX_OK;
}
