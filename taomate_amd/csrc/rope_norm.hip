// RoPE tables and the fused full-row QK-RMSNorm + SPLIT RoPE kernel (gfx950).
//
// Both kernels are HBM-bound streams: one workgroup owns one token row, loads
// it once with 16-byte vector loads, reduces its sum of squares across the
// workgroup, and writes the normalised, rotated row once.

#include <type_traits>

#include "ltx_common.h"
#include "kv_transpose.h"

namespace ltx {

// ---------------------------------------------------------------------------
// RoPE table (causal_rope.py:139-357, SPLIT branch).
// One thread per (token, global pair index); output [B, H, T, P], P = dim/(2H).
// All position arithmetic is float32 with explicit IEEE ops (no contraction) so
// the angles equal what the reference's float32 tensor ops produce.
// ---------------------------------------------------------------------------
template <typename TOut>
__global__ void rope_table_kernel(TOut* __restrict__ cos_out, TOut* __restrict__ sin_out,
                                  const float* __restrict__ freq_idx, int n_freq,
                                  int num_pos_dims, int grid_h, int grid_w,
                                  int64_t start_frame, int is_audio, float max_t,
                                  float max_h, float max_w, int half_dim, int heads,
                                  int64_t T, int batch) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= T * half_dim) return;
  const int64_t t = gid / half_dim;
  const int g = (int)(gid % half_dim);  // global pair index within the token
  const int pad = half_dim - n_freq * num_pos_dims;
  float c = 1.0f, s = 0.0f;
  if (g >= pad) {
    const int q = g - pad;
    const int fi = q / num_pos_dims;
    const int axis = q % num_pos_dims;
    float frac;
    if (num_pos_dims == 3) {
      const int64_t hw = (int64_t)grid_h * grid_w;
      const int64_t f = t / hw;
      const int64_t rem = t % hw;
      if (axis == 0) {
        // latent frame -> pixel-frame bounds with the causal fix -> seconds
        // (causal_rope.py:264-267), then / max_pos[0] (:275)
        float lt = (float)(start_frame + f);
        float ps = fmaxf(__fadd_rn(__fadd_rn(__fmul_rn(lt, 8.0f), 1.0f), -8.0f), 0.0f);
        float pe = fmaxf(
            __fadd_rn(__fadd_rn(__fmul_rn(__fadd_rn(lt, 1.0f), 8.0f), 1.0f), -8.0f), 0.0f);
        float sec = __fdiv_rn(__fdiv_rn(__fadd_rn(ps, pe), 2.0f), 24.0f);
        frac = __fdiv_rn(sec, max_t);
      } else {
        // spatial pixel midpoints (causal_rope.py:271-277)
        int64_t idx = (axis == 1) ? (rem / grid_w) : (rem % grid_w);
        float px = __fadd_rn(__fmul_rn((float)idx, 32.0f), 16.0f);
        frac = __fdiv_rn(px, axis == 1 ? max_h : max_w);
      }
    } else {
      float lt = (float)(start_frame + t);
      float sec;
      if (is_audio) {
        // mel-frame bounds -> seconds (causal_rope.py:298-300)
        float ms = fmaxf(__fadd_rn(__fadd_rn(__fmul_rn(lt, 4.0f), 1.0f), -4.0f), 0.0f);
        float me = fmaxf(
            __fadd_rn(__fadd_rn(__fmul_rn(__fadd_rn(lt, 1.0f), 4.0f), 1.0f), -4.0f), 0.0f);
        sec = __fdiv_rn(__fmul_rn(__fdiv_rn(__fadd_rn(ms, me), 2.0f), 160.0f), 16000.0f);
      } else {
        float ps = fmaxf(__fadd_rn(__fadd_rn(__fmul_rn(lt, 8.0f), 1.0f), -8.0f), 0.0f);
        float pe = fmaxf(
            __fadd_rn(__fadd_rn(__fmul_rn(__fadd_rn(lt, 1.0f), 8.0f), 1.0f), -8.0f), 0.0f);
        sec = __fdiv_rn(__fdiv_rn(__fadd_rn(ps, pe), 2.0f), 24.0f);
      }
      frac = __fdiv_rn(sec, max_t);
    }
    // freqs = indices * (frac * 2 - 1)   (causal_rope.py:287)
    float ang = __fmul_rn(freq_idx[fi], __fadd_rn(__fmul_rn(frac, 2.0f), -1.0f));
    c = cosf(ang);
    s = sinf(ang);
  }
  const int per_head = half_dim / heads;
  const int h = g / per_head;
  const int j = g % per_head;
  for (int b = 0; b < batch; ++b) {
    int64_t o = (((int64_t)b * heads + h) * T + t) * per_head + j;
    if constexpr (sizeof(TOut) == 2) {
      cos_out[o] = f32_to_bf16_bits(c);
      sin_out[o] = f32_to_bf16_bits(s);
    } else {
      cos_out[o] = c;
      sin_out[o] = s;
    }
  }
}

// Per-axis position -> fraction of max_pos, float32 IEEE ops exactly as in
// rope_table_kernel (causal_rope.py:264-277).
__device__ __forceinline__ float video_frac(int axis, int64_t pos, float max_t, float max_h, float max_w) {
  if (axis == 0) {
    const float lt = (float)pos;
    const float ps = fmaxf(__fadd_rn(__fadd_rn(__fmul_rn(lt, 8.0f), 1.0f), -8.0f), 0.0f);
    const float pe = fmaxf(__fadd_rn(__fadd_rn(__fmul_rn(__fadd_rn(lt, 1.0f), 8.0f), 1.0f), -8.0f), 0.0f);
    const float sec = __fdiv_rn(__fdiv_rn(__fadd_rn(ps, pe), 2.0f), 24.0f);
    return __fdiv_rn(sec, max_t);
  }
  const float px = __fadd_rn(__fmul_rn((float)pos, 32.0f), 16.0f);
  return __fdiv_rn(px, axis == 1 ? max_h : max_w);
}

// ---------------------------------------------------------------------------
// Video (3-D) RoPE table, factorised.  A pair's angle depends only on its
// axis, its frequency index and the token's position along that axis, so a
// latent frame's grid_h x grid_w tokens share few distinct angles: per head,
// the t-axis pairs need one value each, the h-axis pairs grid_h and the w-axis
// pairs grid_w.  One workgroup per (frame, head) computes those cos/sin into
// LDS with the same float32 operations as rope_table_kernel (so every entry
// is bit-identical to it), then writes the frame's [T_frame, P] block of the
// head's table.  The frame's rows are split over blockIdx.z in blocks of
// kRopeRows rows (each block needs all grid_w column values but only its own
// row values), so a 3-frame 16x24 chunk of 32 heads is 384 workgroups.
// About 1/15 of the sines and cosines of rope_table_kernel at that grid.
// ---------------------------------------------------------------------------
constexpr int kRopeRows = 4;

template <typename TOut>
__global__ void __launch_bounds__(256) rope_table_video_kernel(
    TOut* __restrict__ cos_out, TOut* __restrict__ sin_out, const float* __restrict__ freq_idx, int n_freq,
    int grid_h, int grid_w, int64_t start_frame, float max_t, float max_h, float max_w, int half_dim,
    int heads, int64_t T, int batch) {
  extern __shared__ float fac[];  // [1 + kRopeRows + grid_w][P][2]: t, this block's rows, then columns
  const int f = blockIdx.x, h = blockIdx.y;
  const int r0 = blockIdx.z * kRopeRows;
  const int nr = min(kRopeRows, grid_h - r0);
  const int P = half_dim / heads;
  const int pad = half_dim - n_freq * 3;
  const int rows = 1 + kRopeRows + grid_w;
  // entry (row, j): row 0 = this frame (t axis), 1..kRopeRows = rows r0.., then columns
  for (int e = threadIdx.x; e < rows * P; e += blockDim.x) {
    const int row = e / P, j = e % P;
    const int g = h * P + j;
    float c = 1.0f, sn = 0.0f;
    if (g >= pad) {
      const int q = g - pad, fi = q / 3, axis = q % 3;
      const int want = row == 0 ? 0 : (row <= kRopeRows ? 1 : 2);
      if (axis == want && (axis != 1 || row - 1 < nr)) {
        const int64_t pos = axis == 0 ? start_frame + f : (axis == 1 ? r0 + row - 1 : row - 1 - kRopeRows);
        const float frac = video_frac(axis, pos, max_t, max_h, max_w);
        const float ang = __fmul_rn(freq_idx[fi], __fadd_rn(__fmul_rn(frac, 2.0f), -1.0f));
        c = cosf(ang);
        sn = sinf(ang);
      }
    }
    fac[2 * e] = c;
    fac[2 * e + 1] = sn;
  }
  __syncthreads();
  // write: one thread per (token, 8 consecutive pairs), 16-byte (bf16) or
  // 2 x 16-byte (float32) stores per table
  const int64_t t0 = (int64_t)f * grid_h * grid_w + (int64_t)r0 * grid_w;
  const int P8 = P / 8;
  for (int e = threadIdx.x; e < nr * grid_w * P8; e += blockDim.x) {
    const int tl = e / P8, j0 = (e % P8) * 8;
    float c[8], sn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int j = j0 + i, g = h * P + j;
      int row = 0;  // pad entries: identity, stored in every row
      if (g >= pad) {
        const int axis = (g - pad) % 3;
        row = axis == 0 ? 0 : (axis == 1 ? 1 + tl / grid_w : 1 + kRopeRows + tl % grid_w);
      }
      c[i] = fac[2 * (row * P + j)];
      sn[i] = fac[2 * (row * P + j) + 1];
    }
    for (int b = 0; b < batch; ++b) {
      const int64_t o = (((int64_t)b * heads + h) * T + t0 + tl) * P + j0;
      if constexpr (sizeof(TOut) == 2) {
        *reinterpret_cast<uint4*>(cos_out + o) = make_uint4(pack_bf16x2(c[0], c[1]), pack_bf16x2(c[2], c[3]),
                                                            pack_bf16x2(c[4], c[5]), pack_bf16x2(c[6], c[7]));
        *reinterpret_cast<uint4*>(sin_out + o) = make_uint4(pack_bf16x2(sn[0], sn[1]), pack_bf16x2(sn[2], sn[3]),
                                                            pack_bf16x2(sn[4], sn[5]), pack_bf16x2(sn[6], sn[7]));
      } else {
        reinterpret_cast<float4*>(cos_out + o)[0] = make_float4(c[0], c[1], c[2], c[3]);
        reinterpret_cast<float4*>(cos_out + o)[1] = make_float4(c[4], c[5], c[6], c[7]);
        reinterpret_cast<float4*>(sin_out + o)[0] = make_float4(sn[0], sn[1], sn[2], sn[3]);
        reinterpret_cast<float4*>(sin_out + o)[1] = make_float4(sn[4], sn[5], sn[6], sn[7]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The video table of a new start frame from a table of the same grid (any
// start frame).  Only the t-axis entries depend on the start frame: the h and
// w entries of token (f, r, c) are those of (r, c) in every frame, and the pad
// entries are the identity.  One workgroup per (frame, head, token row of
// the grid) computes its frame's t-axis cos/sin with the float32
// operations of rope_table_kernel (so every entry is bit-identical to a fresh
// build) and streams the rows: 16-byte loads of the source entries, the
// t-axis ones replaced, 16-byte stores.  A long stream builds one 3-frame
// table per chunk; this reads and writes it instead of evaluating the h and w
// angles again.  A workgroup lives about one memory round trip, so the
// table is cut into many small workgroups (1536 for a 3-frame 16x24 chunk of
// 32 heads, all resident at once) rather than a few long ones.
// ---------------------------------------------------------------------------
constexpr int kRetimeRows = 1;

template <typename TOut>
__global__ void __launch_bounds__(256) rope_table_retime_kernel(
    TOut* __restrict__ cos_out, TOut* __restrict__ sin_out, const TOut* __restrict__ cos_src,
    const TOut* __restrict__ sin_src, const float* __restrict__ freq_idx, int n_freq, int grid_h, int grid_w,
    int64_t start_frame, float max_t, int half_dim, int heads, int64_t T) {
  extern __shared__ float tfac[];  // [P][2]: this frame's t-axis cos / sin (other entries unused)
  const int f = blockIdx.x, h = blockIdx.y;
  const int r0 = blockIdx.z * kRetimeRows;
  const int nr = min(kRetimeRows, grid_h - r0);
  const int P = half_dim / heads;
  const int pad = half_dim - n_freq * 3;
  constexpr int V = 16 / sizeof(TOut);  // entries per 16-byte vector
  const int64_t t0 = (int64_t)f * grid_h * grid_w + (int64_t)r0 * grid_w;
  const int PV = P / V;
  const int nvec = nr * grid_w * PV;
  auto offset = [&](int e) { return ((int64_t)h * T + t0 + e / PV) * P + (e % PV) * V; };
  // the source vectors are loaded first, so their latency covers the
  // evaluation of the t-axis angles (up to kRetimeRegs vectors per thread;
  // larger rows take the loop below)
  constexpr int kRetimeRegs = 4;
  uint4 cv[kRetimeRegs], sv[kRetimeRegs];
#pragma unroll
  for (int i = 0; i < kRetimeRegs; ++i) {
    const int e = threadIdx.x + i * 256;
    if (e < nvec) {
      cv[i] = *reinterpret_cast<const uint4*>(cos_src + offset(e));
      sv[i] = *reinterpret_cast<const uint4*>(sin_src + offset(e));
    }
  }
  for (int j = threadIdx.x; j < P; j += blockDim.x) {
    const int g = h * P + j;
    float c = 1.0f, sn = 0.0f;
    if (g >= pad && (g - pad) % 3 == 0) {
      const int fi = (g - pad) / 3;
      const float frac = video_frac(0, start_frame + f, max_t, 1.0f, 1.0f);
      const float ang = __fmul_rn(freq_idx[fi], __fadd_rn(__fmul_rn(frac, 2.0f), -1.0f));
      c = cosf(ang);
      sn = sinf(ang);
    }
    tfac[2 * j] = c;
    tfac[2 * j + 1] = sn;
  }
  __syncthreads();
  auto patch_store = [&](int e, uint4 c4, uint4 s4) {
    const int j0 = (e % PV) * V;
    TOut* ce = reinterpret_cast<TOut*>(&c4);
    TOut* se = reinterpret_cast<TOut*>(&s4);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int g = h * P + j0 + i;
      if (g >= pad && (g - pad) % 3 == 0) {
        if constexpr (sizeof(TOut) == 2) {
          ce[i] = f32_to_bf16_bits(tfac[2 * (j0 + i)]);
          se[i] = f32_to_bf16_bits(tfac[2 * (j0 + i) + 1]);
        } else {
          ce[i] = tfac[2 * (j0 + i)];
          se[i] = tfac[2 * (j0 + i) + 1];
        }
      }
    }
    *reinterpret_cast<uint4*>(cos_out + offset(e)) = c4;
    *reinterpret_cast<uint4*>(sin_out + offset(e)) = s4;
  };
#pragma unroll
  for (int i = 0; i < kRetimeRegs; ++i) {
    const int e = threadIdx.x + i * 256;
    if (e < nvec) patch_store(e, cv[i], sv[i]);
  }
  for (int e = threadIdx.x + kRetimeRegs * 256; e < nvec; e += 256)
    patch_store(e, *reinterpret_cast<const uint4*>(cos_src + offset(e)),
                *reinterpret_cast<const uint4*>(sin_src + offset(e)));
}

// ---------------------------------------------------------------------------
// Fused RMSNorm + SPLIT RoPE.  Block = (H*D)/16 threads; thread (h, c) owns the
// 8 elements [c*8, c*8+8) of head h's first half and the matching 8 of its
// second half, i.e. the 8 (x1, x2) rotation pairs j = c*8 .. c*8+7.
// grid: 1-D, see norm_work (row group, batch element, side q = 0 / k = 1).
// ---------------------------------------------------------------------------
struct NormRopeSide {
  const void* in;
  void* out;
  const void* gamma;
  const void* cos;
  const void* sin;
  int64_t len, in_bs, in_ls, out_bs, out_ls, tb, th, tt;
  float eps;
};

template <typename T>
struct Vec8;
template <>
struct Vec8<uint16_t> {
  uint4 raw;
  __device__ __forceinline__ void load(const uint16_t* p) {
    raw = *reinterpret_cast<const uint4*>(p);
  }
  __device__ __forceinline__ void store(uint16_t* p) const {
    *reinterpret_cast<uint4*>(p) = raw;
  }
  __device__ __forceinline__ float get(int i) const {
    uint32_t w = (&raw.x)[i >> 1];
    return bf16_bits_to_f32((i & 1) ? (w >> 16) : (w & 0xFFFFu));
  }
  __device__ __forceinline__ void set(int i, float v) {
    uint32_t& w = (&raw.x)[i >> 1];
    uint32_t b = f32_to_bf16_bits(v);
    w = (i & 1) ? ((w & 0xFFFFu) | (b << 16)) : ((w & 0xFFFF0000u) | b);
  }
};
template <>
struct Vec8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void store(float* p) const {
    reinterpret_cast<float4*>(p)[0] = a;
    reinterpret_cast<float4*>(p)[1] = b;
  }
  __device__ __forceinline__ float get(int i) const {
    return i < 4 ? (&a.x)[i] : (&b.x)[i - 4];
  }
  __device__ __forceinline__ void set(int i, float v) {
    if (i < 4) (&a.x)[i] = v; else (&b.x)[i - 4] = v;
  }
};

// Round a float32 intermediate to the storage type (bf16 rounds, f32 keeps).
template <typename T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (sizeof(T) == 2) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else return v;
}

// Rows handled by one workgroup (all loads of its rows are issued before the
// first reduction).  Measured at 1152 rows x 4096, B = 2, with the division-free
// grid below: 1 row 15.4 us, 2 rows 16.1 us (13.7 / 14.3 with the FAST form).
constexpr int NR_ROWS = 1;

// Norm grid: blockIdx = (row group, batch, side 0 = q / 1 = k), gridDim.x a
// multiple of 8.  Workgroups are dispatched round-robin over the 8 XCDs in
// linear order, so every (batch, side) of row group x runs on XCD x % 8 and
// reads the group's RoPE-table rows from that XCD's L2 after the first.  The
// mapping needs no division: a workgroup lives about one memory round trip,
// and a scalar divide chain ahead of its first load lengthens every one.
inline int64_t norm_grid_x(int64_t rows) { return ceil_div(ceil_div(rows, NR_ROWS), 8) * 8; }

// Per-side fields selected with scalar selects (a reference to one of two
// kernel-argument structs picked at run time makes the compiler reload them).
__device__ __forceinline__ NormRopeSide pick_side(const NormRopeSide& q, const NormRopeSide& k, bool kside) {
  NormRopeSide s;
  s.in = kside ? k.in : q.in;
  s.out = kside ? k.out : q.out;
  s.gamma = kside ? k.gamma : q.gamma;
  s.cos = kside ? k.cos : q.cos;
  s.sin = kside ? k.sin : q.sin;
  s.len = kside ? k.len : q.len;
  s.in_bs = kside ? k.in_bs : q.in_bs;
  s.in_ls = kside ? k.in_ls : q.in_ls;
  s.out_bs = kside ? k.out_bs : q.out_bs;
  s.out_ls = kside ? k.out_ls : q.out_ls;
  s.tb = kside ? k.tb : q.tb;
  s.th = kside ? k.th : q.th;
  s.tt = kside ? k.tt : q.tt;
  s.eps = kside ? k.eps : q.eps;
  return s;
}

// The NR_ROWS rows of row group ``rg`` of (batch b, side); every thread of the
// block calls it (one barrier when normalising).  CPD: D / 16 when known at
// compile time (8 for D = 128, 4 for D = 64), 0 otherwise.  FAST: every side
// has a norm (eps >= 0), a gamma and RoPE tables, and every element offset
// of its rows and tables fits in 31 bits (the host checks both), so the
// loads are issued without flag branches and the addresses are computed in
// 32-bit arithmetic (measured 16.1 -> 14.3 us at 1152 x 4096, B = 2).
template <typename T, typename TT, int CPD, bool FAST>
__device__ __forceinline__ void norm_rope_rows(const NormRopeSide& qs, const NormRopeSide& ks, int H, int D,
                                               int64_t rg, int b, int side) {
  constexpr int R = NR_ROWS;
  using Off = std::conditional_t<FAST, int32_t, int64_t>;
  const NormRopeSide sd = pick_side(qs, ks, side != 0);
  const int64_t row0l = rg * R;
  if (row0l >= sd.len) return;  // uniform across the block
  const int nr = (int)(sd.len - row0l < R ? sd.len - row0l : R);
  const Off row0 = (Off)row0l;
  const Off in_bs = (Off)sd.in_bs, in_ls = (Off)sd.in_ls, out_bs = (Off)sd.out_bs, out_ls = (Off)sd.out_ls;
  const Off tb = (Off)sd.tb, th = (Off)sd.th, tt = (Off)sd.tt;
  const int HD = H * D;
  const int cpd = CPD > 0 ? CPD : D / 16;  // chunks of 8 pairs per head
  const int dh = CPD > 0 ? CPD * 16 : D;
  const int tid = threadIdx.x;
  const int h = tid / cpd;
  const int c = tid % cpd;
  const int e1 = h * dh + c * 8;
  const int e2 = e1 + dh / 2;

  const T* in = reinterpret_cast<const T*>(sd.in) + ((Off)b * in_bs + row0 * in_ls);
  Vec8<T> x1[R], x2[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r < nr) {
      x1[r].load(in + ((Off)r * in_ls + e1));
      x2[r].load(in + ((Off)r * in_ls + e2));
    }
  const bool rope = FAST || sd.cos != nullptr;
  Vec8<TT> cv[R], sv[R];
  if (rope) {
    const Off t0 = (Off)b * tb + (Off)h * th + row0 * tt + c * 8;
    const TT* cp = reinterpret_cast<const TT*>(sd.cos) + t0;
    const TT* sp = reinterpret_cast<const TT*>(sd.sin) + t0;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r < nr) {
        cv[r].load(cp + (Off)r * tt);
        sv[r].load(sp + (Off)r * tt);
      }
  }
  const bool norm = FAST || sd.eps >= 0.0f;
  const bool has_gamma = FAST || (norm && sd.gamma != nullptr);
  Vec8<T> g1, g2;
  if (has_gamma) {
    g1.load(reinterpret_cast<const T*>(sd.gamma) + e1);
    g2.load(reinterpret_cast<const T*>(sd.gamma) + e2);
  }

  float rs[R];  // 1 / rms of each row
  if (norm) {
    float ss[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ss[r] = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float a1 = x1[r].get(i), a2 = x2[r].get(i);
        ss[r] += a1 * a1 + a2 * a2;
      }
    }
    // wavefront reduction then across the block's waves through LDS
    // (xor partners stay inside the block: blocks of 16 or 32 threads use part of a wave)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
      if (off < (int)blockDim.x)
#pragma unroll
        for (int r = 0; r < R; ++r) ss[r] += __shfl_xor(ss[r], off, 64);
    __shared__ float red[R][4];
    const int wave = tid >> 6, lane = tid & 63;
    if (lane == 0)
#pragma unroll
      for (int r = 0; r < R; ++r) red[r][wave] = ss[r];
    __syncthreads();
    const int nwaves = (blockDim.x + 63) >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float tot = 0.0f;
      for (int w = 0; w < nwaves; ++w) tot += red[r][w];
      // y = (x * rsqrt(mean(x^2) + eps)) * gamma in float32, rounded once: the
      // fused rms_norm of PyTorch (bit-identical to torch.nn.functional.rms_norm
      // on bf16 rows, checked against it by the tests)
      rs[r] = 1.0f / sqrtf(__fadd_rn(__fdiv_rn(tot, (float)HD), sd.eps));
    }
  }

  T* out = reinterpret_cast<T*>(sd.out) + ((Off)b * out_bs + row0 * out_ls);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nr) break;
    float v1[8], v2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v1[i] = x1[r].get(i);
      v2[i] = x2[r].get(i);
    }
    if (norm) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float y1 = __fmul_rn(v1[i], rs[r]), y2 = __fmul_rn(v2[i], rs[r]);
        if (has_gamma) {
          y1 = __fmul_rn(y1, g1.get(i));
          y2 = __fmul_rn(y2, g2.get(i));
        }
        v1[i] = rnd<T>(y1);
        v2[i] = rnd<T>(y2);
      }
    }
    if (rope) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float cc = cv[r].get(i), sn = sv[r].get(i);
        // out1 = x1*c ; out1 += (-s)*x2 ; out2 = x2*c ; out2 += s*x1
        // (causal_rope.py:121-126: one rounding after the multiply, one after
        // the float32 multiply-add)
        const float a1 = rnd<T>(__fmul_rn(v1[i], cc));
        const float a2 = rnd<T>(__fmul_rn(v2[i], cc));
        const float o1 = rnd<T>(__fadd_rn(a1, __fmul_rn(-sn, v2[i])));
        const float o2 = rnd<T>(__fadd_rn(a2, __fmul_rn(sn, v1[i])));
        v1[i] = o1;
        v2[i] = o2;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x1[r].set(i, v1[i]);
      x2[r].set(i, v2[i]);
    }
    x1[r].store(out + ((Off)r * out_ls + e1));
    x2[r].store(out + ((Off)r * out_ls + e2));
  }
}

template <typename T, typename TT, int CPD, bool FAST>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(NormRopeSide qs, NormRopeSide ks, int H, int D) {
  norm_rope_rows<T, TT, CPD, FAST>(qs, ks, H, D, blockIdx.x, blockIdx.y, blockIdx.z);
}

// V [B, L, H, DV] bf16 rows into a key-major bf16 store, 64-token tiles.
struct VKeyAppend {
  const uint16_t* src;
  int64_t s_bs, s_ls, s_hs;
  uint16_t* dst;
  int64_t d_bs, d_hs, d_ds, L;
  int H;
};

// One launch for the q/k norm + RoPE rows (blocks [0, n_norm)) and the
// key-major append of the chunk's V (the blocks after, one per (token tile,
// head, batch)): both stream HBM, and the V tiles fill the CUs while the
// norm rows drain instead of waiting for a second launch.
template <typename TT, int DV, bool FAST>
__global__ void __launch_bounds__(256) qk_norm_rope_v_kernel(NormRopeSide qs, NormRopeSide ks, int H, int D,
                                                             int nsides, int64_t v_tiles, VKeyAppend va) {
  __shared__ uint16_t tile[transpose_lds_elems<DV>()];
  if ((int)blockIdx.z < nsides) {  // uniform across the block
    norm_rope_rows<uint16_t, TT, DV / 16, FAST>(qs, ks, H, D, blockIdx.x, blockIdx.y, blockIdx.z);
    return;
  }
  // the z slices after the norm's: V tiles in linear order
  const int64_t t = ((int64_t)(blockIdx.z - nsides) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  if (t >= v_tiles) return;
  const int64_t ntx = (va.L + kTransposeTokens - 1) / kTransposeTokens;
  const int64_t hb = t / ntx;
  kv_transpose_tile<uint16_t, DV>(va.src, va.s_bs, va.s_ls, va.s_hs, va.dst, va.d_bs, va.d_hs, va.d_ds, va.L,
                                  t % ntx, (int)(hb % va.H), (int)(hb / va.H), tile);
}

}  // namespace ltx

using namespace ltx;

extern "C" int ltx_rope_table(void* cos_out, void* sin_out, int out_dtype, const float* freq_idx,
                              int64_t n_freq, int num_pos_dims, int64_t grid_f, int64_t grid_h,
                              int64_t grid_w, int64_t start_frame, int is_audio, float max_pos_t,
                              float max_pos_h, float max_pos_w, int64_t dim, int64_t num_heads,
                              int64_t batch, void* stream) {
  clear_error();
  LTX_REQUIRE(cos_out && sin_out && freq_idx, "ltx_rope_table: null pointer");
  LTX_REQUIRE(num_pos_dims == 1 || num_pos_dims == 3, "ltx_rope_table: num_pos_dims must be 1 or 3");
  LTX_REQUIRE(out_dtype == LTX_F32 || out_dtype == LTX_BF16, "ltx_rope_table: out_dtype must be F32 or BF16");
  LTX_REQUIRE(dim > 0 && dim % 2 == 0 && num_heads > 0 && (dim / 2) % num_heads == 0,
              "ltx_rope_table: dim/2 must be divisible by num_heads");
  LTX_REQUIRE(n_freq >= 0 && n_freq * num_pos_dims <= dim / 2,
              "ltx_rope_table: n_freq*num_pos_dims exceeds dim/2");
  LTX_REQUIRE(grid_f >= 0 && batch >= 1, "ltx_rope_table: bad grid/batch");
  if (num_pos_dims == 3) LTX_REQUIRE(grid_h > 0 && grid_w > 0, "ltx_rope_table: bad spatial grid");
  const int64_t T = num_pos_dims == 3 ? grid_f * grid_h * grid_w : grid_f;
  const int half = (int)(dim / 2);
  const int64_t n = T * half;
  if (n == 0) return LTX_OK;
  const int threads = 256;
  const dim3 grid((unsigned)ceil_div(n, threads));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t fac_bytes = (1 + kRopeRows + grid_w) * (half / num_heads) * 2 * (int64_t)sizeof(float);
  if (num_pos_dims == 3 && (half / num_heads) % 8 == 0 && ((uintptr_t)cos_out % 16) == 0 &&
      ((uintptr_t)sin_out % 16) == 0 && fac_bytes <= 64 * 1024 && grid_f <= 0x7FFFFFFF && num_heads <= 65535 &&
      grid_h * grid_w <= 0x7FFFFFFF / (half / num_heads)) {
    const dim3 vgrid((unsigned)grid_f, (unsigned)num_heads, (unsigned)ceil_div(grid_h, kRopeRows));
    if (out_dtype == LTX_BF16)
      hipLaunchKernelGGL(rope_table_video_kernel<uint16_t>, vgrid, dim3(threads), (size_t)fac_bytes, st,
                         (uint16_t*)cos_out, (uint16_t*)sin_out, freq_idx, (int)n_freq, (int)grid_h,
                         (int)grid_w, start_frame, max_pos_t, max_pos_h, max_pos_w, half, (int)num_heads, T,
                         (int)batch);
    else
      hipLaunchKernelGGL(rope_table_video_kernel<float>, vgrid, dim3(threads), (size_t)fac_bytes, st,
                         (float*)cos_out, (float*)sin_out, freq_idx, (int)n_freq, (int)grid_h, (int)grid_w,
                         start_frame, max_pos_t, max_pos_h, max_pos_w, half, (int)num_heads, T, (int)batch);
    LTX_LAUNCH_CHECK("ltx_rope_table");
    return LTX_OK;
  }
  if (out_dtype == LTX_BF16) {
    hipLaunchKernelGGL(rope_table_kernel<uint16_t>, grid, dim3(threads), 0, st,
                       (uint16_t*)cos_out, (uint16_t*)sin_out, freq_idx, (int)n_freq, num_pos_dims,
                       (int)grid_h, (int)grid_w, start_frame, is_audio, max_pos_t, max_pos_h,
                       max_pos_w, half, (int)num_heads, T, (int)batch);
  } else {
    hipLaunchKernelGGL(rope_table_kernel<float>, grid, dim3(threads), 0, st, (float*)cos_out,
                       (float*)sin_out, freq_idx, (int)n_freq, num_pos_dims, (int)grid_h,
                       (int)grid_w, start_frame, is_audio, max_pos_t, max_pos_h, max_pos_w, half,
                       (int)num_heads, T, (int)batch);
  }
  LTX_LAUNCH_CHECK("ltx_rope_table");
  return LTX_OK;
}

namespace {

// Validated launch of the norm rows: the per-side arguments, block size and
// grid (gx, B, nsides); gx = 0: no rows.
struct NormLaunch {
  NormRopeSide qs, ks;
  int threads, nsides;
  int64_t gx;
  bool fast;  // bf16 rows, every side normalised with gamma and rotated, 31-bit offsets
};

// Whether one side qualifies for the FAST kernel form (see norm_rope_rows).
bool side_is_fast(const NormRopeSide& s, int64_t B, int64_t H, int64_t D) {
  if (s.len == 0) return true;
  if (!s.cos || !s.gamma || !(s.eps >= 0.0f)) return false;
  if (s.in_bs < 0 || s.in_ls < 0 || s.out_bs < 0 || s.out_ls < 0 || s.tb < 0 || s.th < 0 || s.tt < 0)
    return false;
  const int64_t lim = 0x7FFFFFFF;
  auto fits = [&](int64_t v) { return v >= 0 && v <= lim; };
  // strides below 2^31 keep every product below 2^62 (no int64 overflow)
  for (int64_t st : {s.in_bs, s.in_ls, s.out_bs, s.out_ls, s.tb, s.th, s.tt})
    if (!fits(st)) return false;
  return fits((B - 1) * s.in_bs + (s.len - 1) * s.in_ls + H * D) &&
         fits((B - 1) * s.out_bs + (s.len - 1) * s.out_ls + H * D) &&
         fits((B - 1) * s.tb + (H - 1) * s.th + (s.len - 1) * s.tt + D / 2);
}

int norm_setup(int dtype, int64_t B, int64_t H, int64_t D,
                      const void* q_in, int64_t q_len, int64_t q_in_bs, int64_t q_in_ls,
                      void* q_out, int64_t q_out_bs, int64_t q_out_ls,
                      const void* gamma_q, float eps_q,
                      const void* q_cos, const void* q_sin, int64_t q_tb, int64_t q_th,
                      int64_t q_tt,
                      const void* k_in, int64_t k_len, int64_t k_in_bs, int64_t k_in_ls,
                      void* k_out, int64_t k_out_bs, int64_t k_out_ls,
                      const void* gamma_k, float eps_k,
                      const void* k_cos, const void* k_sin, int64_t k_tb, int64_t k_th,
                      int64_t k_tt,
                      int tab_dtype, NormLaunch* nl) {
  LTX_REQUIRE(dtype == LTX_F32 || dtype == LTX_BF16, "ltx_qk_rmsnorm_rope: dtype must be F32 or BF16");
  LTX_REQUIRE(tab_dtype == LTX_F32 || tab_dtype == LTX_BF16,
              "ltx_qk_rmsnorm_rope: tab_dtype must be F32 or BF16");
  LTX_REQUIRE(B >= 1 && B <= 65535 && H >= 1 && D >= 16 && D % 16 == 0,
              "ltx_qk_rmsnorm_rope: need B in [1,65535], D a multiple of 16");
  const int64_t threads = H * D / 16;
  LTX_REQUIRE(threads <= 256 && threads % 64 == 0 || threads == 32 || threads == 16,
              "ltx_qk_rmsnorm_rope: H*D/16 must be 16, 32 or a multiple of 64 up to 256 (H*D=%lld)",
              (long long)(H * D));
  LTX_REQUIRE(q_in && q_out && q_len >= 0, "ltx_qk_rmsnorm_rope: q pointers");
  LTX_REQUIRE(!k_in || (k_out && k_len >= 0), "ltx_qk_rmsnorm_rope: k pointers");
  LTX_REQUIRE((q_cos == nullptr) == (q_sin == nullptr) && (k_cos == nullptr) == (k_sin == nullptr),
              "ltx_qk_rmsnorm_rope: cos and sin must both be given or both NULL");
  const int64_t esz = dtype == LTX_BF16 ? 2 : 4;
  auto aligned16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  LTX_REQUIRE(aligned16(q_in) && aligned16(q_out) && (!k_in || (aligned16(k_in) && aligned16(k_out))),
              "ltx_qk_rmsnorm_rope: tensors must be 16-byte aligned");
  LTX_REQUIRE((q_in_bs * esz) % 16 == 0 && (q_in_ls * esz) % 16 == 0 && (q_out_bs * esz) % 16 == 0 &&
                  (q_out_ls * esz) % 16 == 0,
              "ltx_qk_rmsnorm_rope: q strides must keep rows 16-byte aligned");
  if (k_in)
    LTX_REQUIRE((k_in_bs * esz) % 16 == 0 && (k_in_ls * esz) % 16 == 0 && (k_out_bs * esz) % 16 == 0 &&
                    (k_out_ls * esz) % 16 == 0,
                "ltx_qk_rmsnorm_rope: k strides must keep rows 16-byte aligned");
  const int64_t tsz = tab_dtype == LTX_BF16 ? 2 : 4;
  if (q_cos)
    LTX_REQUIRE(aligned16(q_cos) && aligned16(q_sin) && (q_tb * tsz) % 16 == 0 && (q_th * tsz) % 16 == 0 &&
                    (q_tt * tsz) % 16 == 0,
                "ltx_qk_rmsnorm_rope: q tables must be 16-byte aligned");
  if (k_cos)
    LTX_REQUIRE(aligned16(k_cos) && aligned16(k_sin) && (k_tb * tsz) % 16 == 0 && (k_th * tsz) % 16 == 0 &&
                    (k_tt * tsz) % 16 == 0,
                "ltx_qk_rmsnorm_rope: k tables must be 16-byte aligned");
  if (gamma_q) LTX_REQUIRE(aligned16(gamma_q), "ltx_qk_rmsnorm_rope: gamma_q alignment");
  if (gamma_k) LTX_REQUIRE(aligned16(gamma_k), "ltx_qk_rmsnorm_rope: gamma_k alignment");

  NormRopeSide qs{q_in, q_out, gamma_q, q_cos, q_sin, q_len, q_in_bs, q_in_ls, q_out_bs, q_out_ls,
                  q_tb, q_th, q_tt, eps_q};
  NormRopeSide ks{k_in, k_out, gamma_k, k_cos, k_sin, k_in ? k_len : 0, k_in_bs, k_in_ls, k_out_bs,
                  k_out_ls, k_tb, k_th, k_tt, eps_k};
  const int64_t rows = k_in ? (q_len > k_len ? q_len : k_len) : q_len;
  LTX_REQUIRE(rows <= 0x7FFFFFFF, "ltx_qk_rmsnorm_rope: too many rows");
  nl->qs = qs;
  nl->ks = ks;
  nl->threads = (int)threads;
  nl->nsides = k_in ? 2 : 1;
  nl->gx = rows == 0 ? 0 : norm_grid_x(rows);
  nl->fast = dtype == LTX_BF16 && side_is_fast(qs, B, H, D) && side_is_fast(ks, B, H, D);
  return LTX_OK;
}

}  // namespace

extern "C" int ltx_rope_table_retime(void* cos_out, void* sin_out, const void* cos_src, const void* sin_src,
                                     int out_dtype, const float* freq_idx, int64_t n_freq, int64_t grid_f,
                                     int64_t grid_h, int64_t grid_w, int64_t start_frame, float max_pos_t,
                                     int64_t dim, int64_t num_heads, void* stream) {
  clear_error();
  LTX_REQUIRE(cos_out && sin_out && cos_src && sin_src && freq_idx, "ltx_rope_table_retime: null pointer");
  LTX_REQUIRE(out_dtype == LTX_F32 || out_dtype == LTX_BF16, "ltx_rope_table_retime: out_dtype must be F32 or BF16");
  LTX_REQUIRE(dim > 0 && dim % 2 == 0 && num_heads > 0 && num_heads <= 65535 && (dim / 2) % num_heads == 0,
              "ltx_rope_table_retime: dim/2 must be divisible by num_heads");
  LTX_REQUIRE(n_freq >= 0 && n_freq * 3 <= dim / 2, "ltx_rope_table_retime: n_freq*3 exceeds dim/2");
  LTX_REQUIRE(grid_f >= 0 && grid_f <= 0x7FFFFFFF && grid_h > 0 && grid_w > 0, "ltx_rope_table_retime: bad grid");
  const int half = (int)(dim / 2);
  const int P = half / (int)num_heads;
  const int64_t esz = out_dtype == LTX_BF16 ? 2 : 4;
  LTX_REQUIRE((P * esz) % 16 == 0, "ltx_rope_table_retime: dim/(2 heads) entries must fill 16-byte vectors");
  auto al = [](const void* ptr) { return ((uintptr_t)ptr % 16) == 0; };
  LTX_REQUIRE(al(cos_out) && al(sin_out) && al(cos_src) && al(sin_src),
              "ltx_rope_table_retime: tables must be 16-byte aligned");
  LTX_REQUIRE(grid_h * grid_w <= 0x7FFFFFFF / P, "ltx_rope_table_retime: grid too large");
  const int64_t T = grid_f * grid_h * grid_w;
  if (T == 0) return LTX_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 vgrid((unsigned)grid_f, (unsigned)num_heads, (unsigned)ceil_div(grid_h, kRetimeRows));
  const size_t lds = (size_t)P * 2 * sizeof(float);
  if (out_dtype == LTX_BF16)
    hipLaunchKernelGGL(rope_table_retime_kernel<uint16_t>, vgrid, dim3(256), lds, st, (uint16_t*)cos_out,
                       (uint16_t*)sin_out, (const uint16_t*)cos_src, (const uint16_t*)sin_src, freq_idx,
                       (int)n_freq, (int)grid_h, (int)grid_w, start_frame, max_pos_t, half, (int)num_heads, T);
  else
    hipLaunchKernelGGL(rope_table_retime_kernel<float>, vgrid, dim3(256), lds, st, (float*)cos_out,
                       (float*)sin_out, (const float*)cos_src, (const float*)sin_src, freq_idx, (int)n_freq,
                       (int)grid_h, (int)grid_w, start_frame, max_pos_t, half, (int)num_heads, T);
  LTX_LAUNCH_CHECK("ltx_rope_table_retime");
  return LTX_OK;
}

extern "C" int ltx_qk_rmsnorm_rope(int dtype, int64_t B, int64_t H, int64_t D,
                                   const void* q_in, int64_t q_len, int64_t q_in_bs, int64_t q_in_ls,
                                   void* q_out, int64_t q_out_bs, int64_t q_out_ls,
                                   const void* gamma_q, float eps_q,
                                   const void* q_cos, const void* q_sin, int64_t q_tb, int64_t q_th,
                                   int64_t q_tt,
                                   const void* k_in, int64_t k_len, int64_t k_in_bs, int64_t k_in_ls,
                                   void* k_out, int64_t k_out_bs, int64_t k_out_ls,
                                   const void* gamma_k, float eps_k,
                                   const void* k_cos, const void* k_sin, int64_t k_tb, int64_t k_th,
                                   int64_t k_tt,
                                   int tab_dtype, void* stream) {
  clear_error();
  NormLaunch nl;
  const int rc = norm_setup(dtype, B, H, D, q_in, q_len, q_in_bs, q_in_ls, q_out, q_out_bs, q_out_ls, gamma_q, eps_q, q_cos, q_sin,
                       q_tb, q_th, q_tt, k_in, k_len, k_in_bs, k_in_ls, k_out, k_out_bs, k_out_ls, gamma_k, eps_k,
                       k_cos, k_sin, k_tb, k_th, k_tt, tab_dtype, &nl);
  if (rc != LTX_OK || nl.gx == 0) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)nl.gx, (unsigned)B, (unsigned)nl.nsides), block((unsigned)nl.threads);
  const NormRopeSide &qs = nl.qs, &ks = nl.ks;
#define LTX_NR(T, TT, F)                                                                                     \
  do {                                                                                                       \
    if (D == 128)                                                                                            \
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, TT, 8, F>), grid, block, 0, st, qs, ks, (int)H, (int)D);   \
    else if (D == 64)                                                                                        \
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, TT, 4, F>), grid, block, 0, st, qs, ks, (int)H, (int)D);   \
    else                                                                                                     \
      hipLaunchKernelGGL((qk_norm_rope_kernel<T, TT, 0, F>), grid, block, 0, st, qs, ks, (int)H, (int)D);   \
  } while (0)
  if (dtype == LTX_BF16) {
    if (tab_dtype == LTX_BF16) {
      if (nl.fast) LTX_NR(uint16_t, uint16_t, true); else LTX_NR(uint16_t, uint16_t, false);
    } else {
      if (nl.fast) LTX_NR(uint16_t, float, true); else LTX_NR(uint16_t, float, false);
    }
  } else {
    if (tab_dtype == LTX_BF16) LTX_NR(float, uint16_t, false); else LTX_NR(float, float, false);
  }
#undef LTX_NR
  LTX_LAUNCH_CHECK("ltx_qk_rmsnorm_rope");
  return LTX_OK;
}

extern "C" int ltx_qk_rmsnorm_rope_v(int dtype, int64_t B, int64_t H, int64_t D,
                                     const void* q_in, int64_t q_len, int64_t q_in_bs, int64_t q_in_ls,
                                     void* q_out, int64_t q_out_bs, int64_t q_out_ls,
                                     const void* gamma_q, float eps_q,
                                     const void* q_cos, const void* q_sin, int64_t q_tb, int64_t q_th,
                                     int64_t q_tt,
                                     const void* k_in, int64_t k_len, int64_t k_in_bs, int64_t k_in_ls,
                                     void* k_out, int64_t k_out_bs, int64_t k_out_ls,
                                     const void* gamma_k, float eps_k,
                                     const void* k_cos, const void* k_sin, int64_t k_tb, int64_t k_th,
                                     int64_t k_tt, int tab_dtype,
                                     const void* v_src, int64_t v_len, int64_t v_bs, int64_t v_ls, int64_t v_hs,
                                     void* v_dst, int64_t vd_bs, int64_t vd_hs, int64_t vd_ds, void* stream) {
  clear_error();
  LTX_REQUIRE(dtype == LTX_BF16, "ltx_qk_rmsnorm_rope_v: bf16 rows only");
  LTX_REQUIRE(D == 64 || D == 128, "ltx_qk_rmsnorm_rope_v: head dim must be 64 or 128");
  LTX_REQUIRE(v_len >= 0 && (v_len == 0 || (v_src && v_dst)), "ltx_qk_rmsnorm_rope_v: V pointers");
  if (v_len > 0) {
    LTX_REQUIRE(((uintptr_t)v_src % 16) == 0 && (v_bs * 2) % 16 == 0 && (v_ls * 2) % 16 == 0 &&
                    (v_hs * 2) % 16 == 0,
                "ltx_qk_rmsnorm_rope_v: V rows must be 16-byte aligned");
    LTX_REQUIRE(((uintptr_t)v_dst % 16) == 0 && (vd_bs * 2) % 16 == 0 && (vd_hs * 2) % 16 == 0 &&
                    (vd_ds * 2) % 16 == 0,
                "ltx_qk_rmsnorm_rope_v: key-major V must start on a 16-byte boundary (8-slot aligned)");
  }
  NormLaunch nl;
  const int rc = norm_setup(dtype, B, H, D, q_in, q_len, q_in_bs, q_in_ls, q_out, q_out_bs, q_out_ls, gamma_q, eps_q, q_cos, q_sin,
                       q_tb, q_th, q_tt, k_in, k_len, k_in_bs, k_in_ls, k_out, k_out_bs, k_out_ls, gamma_k, eps_k,
                       k_cos, k_sin, k_tb, k_th, k_tt, tab_dtype, &nl);
  if (rc != LTX_OK) return rc;
  const int64_t v_tiles = ceil_div(v_len, kTransposeTokens) * H * B;
  if (nl.gx == 0 && v_tiles == 0) return LTX_OK;
  // norm slices z < nsides (none without rows), then enough (gx, B) slices
  // for the V tiles
  const int64_t gx = nl.gx > 0 ? nl.gx : 8;
  const int nsides = nl.gx > 0 ? nl.nsides : 0;
  const int64_t vz = ceil_div(v_tiles, gx * B);
  LTX_REQUIRE(gx <= 0x7FFFFFFF && nsides + vz <= 65535, "ltx_qk_rmsnorm_rope_v: grid too large");
  const VKeyAppend va{(const uint16_t*)v_src, v_bs, v_ls, v_hs, (uint16_t*)v_dst, vd_bs, vd_hs, vd_ds, v_len,
                      (int)H};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // the V tiles run with the norm's block size (a multiple of 64 threads up to
  // 256, or 16 / 32): kv_transpose_tile strides by blockDim
  const dim3 grid((unsigned)gx, (unsigned)B, (unsigned)(nsides + vz));
  const dim3 block((unsigned)(nl.gx > 0 ? nl.threads : 256));
#define LTX_NRV(TT, DV)                                                                                           \
  do {                                                                                                            \
    if (nl.fast)                                                                                                  \
      hipLaunchKernelGGL((qk_norm_rope_v_kernel<TT, DV, true>), grid, block, 0, st, nl.qs, nl.ks, (int)H, (int)D, \
                         nsides, v_tiles, va);                                                                    \
    else                                                                                                          \
      hipLaunchKernelGGL((qk_norm_rope_v_kernel<TT, DV, false>), grid, block, 0, st, nl.qs, nl.ks, (int)H,       \
                         (int)D, nsides, v_tiles, va);                                                            \
  } while (0)
  if (tab_dtype == LTX_BF16) {
    if (D == 128) LTX_NRV(uint16_t, 128); else LTX_NRV(uint16_t, 64);
  } else {
    if (D == 128) LTX_NRV(float, 128); else LTX_NRV(float, 64);
  }
#undef LTX_NRV
  LTX_LAUNCH_CHECK("ltx_qk_rmsnorm_rope_v");
  return LTX_OK;
}
