// Flash-style attention forward for gfx950 (CDNA4) over segmented keys.
//
// Replaces F.scaled_dot_product_attention as reached through
// standard_attention_forward (ltx_causal/attention/flex_attention_utils.py:225-276)
// from attention_with_cache (ltx_causal/transformer/kv_cache.py:1531), whose keys
// are torch.cat([cached_k, k], 1) (kv_cache.py:1487-1491).  Here the keys stay
// where they live (anchor | memory | window | current spans of a KV arena) and
// the kernel walks the spans in order.
//
// Work decomposition.  A workgroup of 4 wavefronts owns BM = 128 query rows of
// one (batch, head); each wavefront owns 32 rows.  Keys stream through LDS in
// tiles of BN = 64, double buffered: while the MFMAs consume tile j, the next
// tile is already in registers (global loads issued one tile ahead).
//
// Matrix-core mapping (v_mfma_f32_32x32x16_bf16, lane l, i = l % 32, g = l / 32):
//   S^T = K Q^T: A = K rows (LDS), B = Q^T (registers, loaded once).  The
//   accumulator gives every lane ONE query (i) and 16 keys of each 32-key block,
//   so the softmax row statistics are per-lane scalars plus a single exchange
//   with lane l ^ 32, which holds the other 16 keys of the same query.
//   K rows are stored in LDS with row-index bits 2 and 3 swapped; with that
//   order accumulator register r of block kb holds key kb*32 + 16*(r/8) + 8g +
//   r%8, i.e. each lane's 8-register half is 8 consecutive keys.
//   O^T += V^T P^T: B = P straight from the softmax registers (8 consecutive
//   keys per lane, as above), A = V^T read from a transposed V tile in LDS.
//   The accumulator again gives each lane one query, so the online-softmax
//   rescale is one scalar per lane.
// Softmax: base-2 exponent with log2(e) folded into the logit scale
// (exp(x) = 2^(x*log2 e)), running max / running sum per query (the online
// normaliser of Milakov & Gimelshein 2018, as used by Dao et al. 2022).
// fp8 KV: tiles are decoded to bf16 on their way into LDS; the per-(head,
// frame) scales are folded into the logit scale (K) and into P (V).

#include <mutex>

#include "ltx_common.h"

namespace ltx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

struct FlashParams {
  const uint16_t* q;
  uint16_t* o;
  float* lse;
  const float* mask;
  int64_t q_bs, q_ls, q_hs;
  int64_t o_bs, o_ls, o_hs;
  int o_al16;                        // o and its strides are 16-byte aligned (staged output stores)
  int64_t kv_bs, kv_ls, kv_hs;      // K (and token-major V) strides
  int64_t v_bs, v_hs, v_ds;          // key-major V: element (b, t, h, d) at b*v_bs + h*v_hs + d*v_ds + t
  int64_t sc_bs, sc_hs;
  int64_t mask_bs;
  int64_t Lk;
  // per-batch key counts (n_klen == B, or 0 for none): batch row b attends
  // keys [0, klen[b]) of the concatenated sequence (a key-padding mask that
  // keeps a prefix of each row)
  int n_klen;
  int klen[LTX_MAX_KEYLEN_BATCH];
  int64_t seg_start[LTX_MAX_SEGMENTS + 1];
  const void* k_ptr[LTX_MAX_SEGMENTS];
  const void* v_ptr[LTX_MAX_SEGMENTS];
  const float* k_sc[LTX_MAX_SEGMENTS];
  const float* v_sc[LTX_MAX_SEGMENTS];
  int tile_start[LTX_MAX_SEGMENTS + 1];  // first key tile of each segment (cumulative)
  int B, H, Lq, n_seg, n_qtiles, frame;
  // Balanced tail: the first n_full q-tiles run whole; each of the remaining
  // q-tiles is cut into `split` key ranges run by separate workgroups, whose
  // partial results meet in the workspace and are combined by a second kernel.
  int n_full, split;
  // pair kernel (bf16 key-major V, n_qtiles even): work unit u is q-tiles 2u
  // and 2u + 1, which lie in one (batch, head) and share every K/V tile;
  // n_full and split count units, and the tail q-tiles start at 2 n_full.
  int pair;
  uint16_t* part_o;  // [tail tiles * split][kBM][D] bf16 O / l of the key range (0 where l = 0)
  float* part_ml;     // [tail tiles * split][kBM][2] running max (log2) and sum
  float scale;       // softmax scale applied to q.k
  float scale_log2;  // scale * log2(e)
};

// Max / sum of a lane's value with lane l ^ 32's (the lane holding the other
// 16 keys of the same query): one v_permlane32_swap, no LDS round trip.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int kBM = 128;
constexpr int kBN = 64;
constexpr float kLog2e = 1.4426950408889634f;

// Row r of a K tile is stored at LDS row sig(r): bits 2 and 3 swapped.
__device__ __forceinline__ int sig(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// Blocks are dispatched round-robin over the 8 XCDs (block id % 8).  Give each
// XCD a contiguous range of the (batch*head, q-tile) space so the q-tiles that
// share one head's K/V run on the same XCD and hit the same L2.
__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = nb >> 3, rem = nb & 7;
  return xcd * per + (xcd < rem ? xcd : rem) + slot;
}

template <bool FP8>
struct KVChunk;
template <>
struct KVChunk<false> {
  using raw_t = uint4;  // 8 bf16
  static __device__ __forceinline__ raw_t zero() { return make_uint4(0, 0, 0, 0); }
  static __device__ __forceinline__ raw_t load(const void* base, int64_t off) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
  }
  static __device__ __forceinline__ raw_t bload(__amdgpu_buffer_rsrc_t r, int off) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
  }
  static __device__ __forceinline__ uint4 to_bf16(raw_t r) { return r; }
};
template <>
struct KVChunk<true> {
  using raw_t = uint2;  // 8 fp8
  static __device__ __forceinline__ raw_t zero() { return make_uint2(0, 0); }
  static __device__ __forceinline__ raw_t load(const void* base, int64_t off) {
    return *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(base) + off);
  }
  static __device__ __forceinline__ raw_t bload(__amdgpu_buffer_rsrc_t r, int off) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v[0], v[1]);
  }
  // Exact: every e4m3 value (subnormals included) is representable in bf16,
  // and v_cvt_scalef32_pk_bf16_fp8 with scale 1 decodes two codes (bytes 0-1
  // or 2-3 of the word) into a packed bf16 pair; its output was compared with
  // the e4m3 definition for every code pair on gfx950.
  static __device__ __forceinline__ uint32_t pair(uint32_t w, bool hi) {
    return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                                           : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  }
  static __device__ __forceinline__ uint4 to_bf16(raw_t r) {
    return make_uint4(pair(r.x, false), pair(r.x, true), pair(r.y, false), pair(r.y, true));
  }
};

// Key tiles never cross a segment: each segment is cut into ceil(len / kBN)
// tiles (the last one partial).  The iterator walks them in order with
// wave-uniform (scalar) state, touching the per-segment kernel arguments only
// when it enters a new segment.
struct TileIter {
  int s;
  int64_t row0;  // first token of the tile inside segment s
  int64_t len;   // tokens in segment s
  int64_t key0;  // first token of the tile in the concatenated key sequence
  const void* k;
  const void* v;

  __device__ __forceinline__ void enter(const FlashParams& p, int seg) {
    s = seg;
    row0 = 0;
    key0 = p.seg_start[seg];
    len = p.seg_start[seg + 1] - key0;
    k = p.k_ptr[seg];
    v = p.v_ptr[seg];
  }
  __device__ __forceinline__ void next(const FlashParams& p) {
    row0 += kBN;
    key0 += kBN;
    if (row0 >= len && s + 1 < p.n_seg) enter(p, s + 1);
  }
  __device__ __forceinline__ int nvalid() const {
    return (int)(len - row0 < kBN ? len - row0 : kBN);
  }
  // position on key tile j of the concatenated sequence
  __device__ __forceinline__ void seek(const FlashParams& p, int j) {
    int seg = 0;
    for (int i = 1; i < p.n_seg; ++i) seg = (j >= p.tile_start[i]) ? i : seg;
    enter(p, seg);
    row0 = (int64_t)(j - p.tile_start[seg]) * kBN;
    key0 += row0;
  }
};

// Key tiles of the concatenated sequence that hold keys below `lim` (the
// tiles a batch row with a per-batch key count attends; bf16 tiling).
__device__ __forceinline__ int tiles_below(const FlashParams& p, int lim) {
  int t = p.tile_start[p.n_seg];
  for (int i = p.n_seg - 1; i >= 0; --i)
    if (lim <= p.seg_start[i + 1]) {
      const int64_t in = lim - p.seg_start[i];
      t = p.tile_start[i] + (int)((in > 0 ? in : 0) + kBN - 1) / kBN;
    }
  return t;
}

// Which q-tile and key-tile range block `bid` owns.  Blocks below n_full take
// whole q-tiles; the rest take 1/split of a tail q-tile's key tiles.  Each
// group is spread over the 8 XCDs on its own (dispatch is round-robin by
// block id), and inside a group consecutive work shares an XCD's L2.
struct WorkItem {
  int qtile;   // linear (b*H + h) * n_qtiles + qt
  int j0, j1;  // key tiles [j0, j1)
  int piece;   // -1: whole q-tile; else index into the partial buffers
  int tail;    // tail q-tile index (piece >= 0)
};
__device__ __forceinline__ WorkItem work_item(const FlashParams& p, int bid, int ntiles) {
  WorkItem w;
  if (bid < p.n_full) {
    w.qtile = xcd_remap(bid, p.n_full);
    w.j0 = 0;
    w.j1 = ntiles;
    w.piece = -1;
    w.tail = -1;
  } else {
    const int ntail = gridDim.x - p.n_full;
    const int t = xcd_remap(bid - p.n_full, ntail);
    w.tail = t / p.split;
    const int part = t % p.split;
    w.qtile = p.n_full + w.tail;
    w.j0 = (int)((int64_t)ntiles * part / p.split);
    w.j1 = (int)((int64_t)ntiles * (part + 1) / p.split);
    w.piece = t;
  }
  return w;
}

// Work of group grp of pair workgroup `bid`: q-tile 2u + grp of unit u
// (units below n_full run whole, the rest 1/split of their key tiles; a
// split unit's two q-tiles are tail q-tiles 2 tu and 2 tu + 1).
__device__ __forceinline__ WorkItem pair_work(const FlashParams& p, int bid, int grp, int ntiles) {
  WorkItem w;
  int u;
  if (bid < p.n_full) {
    u = xcd_remap(bid, p.n_full);
    w.j0 = 0;
    w.j1 = ntiles;
    w.piece = -1;
    w.tail = -1;
  } else {
    const int ntail = gridDim.x - p.n_full;
    const int t = xcd_remap(bid - p.n_full, ntail);
    const int tu = t / p.split, part = t % p.split;
    u = p.n_full + tu;
    w.j0 = (int)((int64_t)ntiles * part / p.split);
    w.j1 = (int)((int64_t)ntiles * (part + 1) / p.split);
    w.tail = 2 * tu + grp;
    w.piece = w.tail * p.split + part;
  }
  w.qtile = 2 * u + grp;
  return w;
}

// Epilogue shared by the kernels: normalise and store a whole q-tile, or
// store a key range's partial result (unnormalised O, running max and sum).  oacc holds O^T fragments (lane: query li,
// d = db*32 + 8*(r/4) + 4*hg + r%4); m_run / l_tot are per query.
//
// stage (the pipelined kernels): this wave's 32 x (D + 8) bf16 region of LDS,
// free once every wave is past its last K/V tile.  The wave's 32 rows go
// through it so that each store writes 16 bytes per lane and a store
// instruction covers whole rows (four 256-byte rows at D = 128) instead of 16
// bytes of each of 32 rows 8 KB apart: an eighth of the memory requests.
// The stores are streaming ones (whole rows now, so they leave the L2 as
// full lines while the kernel runs): 156.3 -> 154.0 us for the staging and
// 152.6 us with streaming stores at the 1152 x 4608 chunk, and the launch
// after it 1.5 us faster.  Every wave of the workgroup calls it (two
// barriers inside), with one path for the whole workgroup (a whole q-tile or
// a key range, and o_al16).
template <int D>
__device__ __forceinline__ void finish_tile(const FlashParams& p, const WorkItem& w, int b, int h,
                                            int qt, int row, const f32x16_t (&oacc)[D / 32], float m_run,
                                            float l_tot, uint16_t* stage = nullptr) {
  constexpr int DB = D / 32;
  const int hg = (threadIdx.x & 63) >> 5;  // row: this lane's query inside the q-tile
  const int qi = qt * kBM + row;
  if (stage != nullptr && (w.piece >= 0 || p.o_al16)) {
    constexpr int RS = D + 8;   // staging row stride (elements)
    constexpr int CPR = D / 8;  // 16-byte chunks per row
    const int li = threadIdx.x & 31, lane = threadIdx.x & 63;
    const int row0 = row - li;  // the wave's first row in the q-tile
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    __syncthreads();  // every wave is done reading the K/V tiles
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        uint2 v;
        v.x = pack_bf16x2(oacc[d][4 * g4] * inv, oacc[d][4 * g4 + 1] * inv);
        v.y = pack_bf16x2(oacc[d][4 * g4 + 2] * inv, oacc[d][4 * g4 + 3] * inv);
        *reinterpret_cast<uint2*>(stage + li * RS + d * 32 + 8 * g4 + 4 * hg) = v;
      }
    __syncthreads();
    if (w.piece < 0) {
      const int64_t obase = b * p.o_bs + h * p.o_hs;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const int c = i * 64 + lane, r = c / CPR, cc = c % CPR;
        const int q = qt * kBM + row0 + r;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + r * RS + cc * 8);
        if (q < p.Lq) store_stream(p.o + obase + (int64_t)q * p.o_ls + cc * 8, v);
      }
      if (p.lse != nullptr && hg == 0 && qi < p.Lq)
        p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = (m_run + __log2f(l_tot)) / kLog2e;
    } else {
      uint16_t* po = p.part_o + ((int64_t)w.piece * kBM + row0) * D;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) {
        const int c = i * 64 + lane, r = c / CPR, cc = c % CPR;
        store_stream(po + r * D + cc * 8, *reinterpret_cast<const uint4*>(stage + r * RS + cc * 8));
      }
      if (hg == 0) *reinterpret_cast<float2*>(p.part_ml + ((int64_t)w.piece * kBM + row) * 2) = make_float2(m_run, l_tot);
    }
    return;
  }
  if (w.piece < 0) {
    if (qi < p.Lq) {
      const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      uint16_t* op = p.o + b * p.o_bs + (int64_t)qi * p.o_ls + h * p.o_hs;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          uint2 v;
          v.x = pack_bf16x2(oacc[d][4 * g4] * inv, oacc[d][4 * g4 + 1] * inv);
          v.y = pack_bf16x2(oacc[d][4 * g4 + 2] * inv, oacc[d][4 * g4 + 3] * inv);
          *reinterpret_cast<uint2*>(op + d * 32 + 8 * g4 + 4 * hg) = v;
        }
      }
      if (p.lse != nullptr && hg == 0) p.lse[((int64_t)b * p.H + h) * p.Lq + qi] = (m_run + __log2f(l_tot)) / kLog2e;
    }
    return;
  }
  // ---- partial result of one key range: combined by flash_combine_kernel.
  // O is stored normalised by the range's own sum and rounded to bf16 (the
  // output's precision), so the partials cost a quarter of fp32 O traffic;
  // the combine weighs each range by its sum and maximum. ----
  uint16_t* po = p.part_o + ((int64_t)w.piece * kBM + row) * D;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      uint2 v;
      v.x = pack_bf16x2(oacc[d][4 * g4] * inv, oacc[d][4 * g4 + 1] * inv);
      v.y = pack_bf16x2(oacc[d][4 * g4 + 2] * inv, oacc[d][4 * g4 + 3] * inv);
      *reinterpret_cast<uint2*>(po + d * 32 + 8 * g4 + 4 * hg) = v;
    }
  if (hg == 0) *reinterpret_cast<float2*>(p.part_ml + ((int64_t)w.piece * kBM + row) * 2) = make_float2(m_run, l_tot);
}

constexpr int kMaxSplit = 8;  // key ranges a tail q-tile may be cut into

// Combines the `split` partial results of every tail q-tile, launched after the
// attention kernel on the same stream: out = sum_i w_i o_i / sum_i w_i with
// w_i = l_i 2^(m_i - max m) and o_i the range's normalised output.  One thread
// per (query row, 8 output columns): every piece's (max, sum) and 16-byte O
// chunk are loaded up front, so each thread waits for one round of loads.
// The output is written as two 8-byte halves (the entry point guarantees
// 8-byte aligned output rows); the workspace partials are 16-byte aligned.
constexpr int kCombineCols = 8;
template <int D>
constexpr int combine_wg_per_tile() { return kBM / (256 / (D / kCombineCols)); }

template <int D>
__global__ void __launch_bounds__(256) flash_combine_kernel(const FlashParams p) {
  constexpr int CG = D / kCombineCols;  // 8-column groups per row
  constexpr int ROWS = 256 / CG;        // rows per workgroup
  constexpr int WG_PER_TILE = kBM / ROWS;
  static_assert(WG_PER_TILE == combine_wg_per_tile<D>() && ROWS * WG_PER_TILE == kBM, "combine grid");
  const int tail = blockIdx.x / WG_PER_TILE;
  const int r = (blockIdx.x % WG_PER_TILE) * ROWS + threadIdx.x / CG;
  const int cg = threadIdx.x % CG;
  const int qtile = (p.pair ? 2 * p.n_full : p.n_full) + tail;
  const int qt = qtile % p.n_qtiles;
  const int bh = qtile / p.n_qtiles;
  const int b = bh / p.H, h = bh % p.H;
  const int q = qt * kBM + r;
  if (q >= p.Lq) return;
  const int64_t first = (int64_t)tail * p.split;
  f32x2_t ml[kMaxSplit];
  uint4 o[kMaxSplit];
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i) {
    if (i < p.split) {
      ml[i] = *reinterpret_cast<const f32x2_t*>(p.part_ml + ((first + i) * kBM + r) * 2);
      o[i] = *reinterpret_cast<const uint4*>(p.part_o + ((first + i) * kBM + r) * D + cg * kCombineCols);
    }
  }
  float mmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i)
    if (i < p.split) mmax = fmaxf(mmax, ml[i][0]);
  float lsum = 0.0f;
  float acc[kCombineCols] = {};
#pragma unroll
  for (int i = 0; i < kMaxSplit; ++i) {
    if (i < p.split) {
      const float wgt = ml[i][0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[i][0] - mmax) * ml[i][1];
      lsum += wgt;
      const uint32_t w[4] = {o[i].x, o[i].y, o[i].z, o[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += wgt * bf16_bits_to_f32(w[e] & 0xFFFFu);
        acc[2 * e + 1] += wgt * bf16_bits_to_f32(w[e] >> 16);
      }
    }
  }
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  uint16_t* dst = p.o + b * p.o_bs + (int64_t)q * p.o_ls + h * p.o_hs + cg * kCombineCols;
  *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(acc[0] * inv, acc[1] * inv),
                                              pack_bf16x2(acc[2] * inv, acc[3] * inv));
  *reinterpret_cast<uint2*>(dst + 4) = make_uint2(pack_bf16x2(acc[4] * inv, acc[5] * inv),
                                                  pack_bf16x2(acc[6] * inv, acc[7] * inv));
  if (p.lse != nullptr && cg == 0) p.lse[((int64_t)b * p.H + h) * p.Lq + q] = (mmax + __log2f(lsum)) / kLog2e;
}

template <int D, bool FP8, bool MASK>
__global__ void __launch_bounds__(256, 2) flash_fwd_kernel(const FlashParams p) {
  constexpr int BM = kBM, BN = kBN;
  constexpr int KS = D + 8;                // K tile LDS row stride (elements)
  constexpr int VS = BN + 8;               // V^T tile LDS row stride
  constexpr int KBUF = BN * KS;
  constexpr int VBUF = D * VS;
  constexpr int NKC = D / 8;               // 8-element chunks per K row
  constexpr int KROWS_PER_PASS = 256 / NKC;
  constexpr int K_LOADS = BN / KROWS_PER_PASS;
  constexpr int NVP = (BN / 4) * (D / 8);  // (4-key group, 8-d chunk) pairs
  constexpr int DB = D / 32;
  constexpr int QS = D / 16;
  using Chunk = KVChunk<FP8>;
  using raw_t = typename Chunk::raw_t;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (KBUF + VBUF)];
  __shared__ float mask_s[MASK ? 2 : 1][MASK ? BN : 1];

  const WorkItem wi = work_item(p, blockIdx.x, p.tile_start[p.n_seg]);
  const int qt = wi.qtile % p.n_qtiles;
  const int bh = wi.qtile / p.n_qtiles;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, hg = lane >> 5;
  const int qi = qt * BM + wave * 32 + li;
  const int ntiles = wi.j1 - wi.j0;

  // ---- Q^T fragments, resident for the whole key loop ----
  bf16x8_t qf[QS];
  {
    const bool ok = qi < p.Lq;
    const uint16_t* qp = p.q + b * p.q_bs + (int64_t)(ok ? qi : 0) * p.q_ls + h * p.q_hs + hg * 8;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint4 v = ok ? *reinterpret_cast<const uint4*>(qp + s * 16) : make_uint4(0, 0, 0, 0);
      qf[s] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  const int64_t kv_off = b * p.kv_bs + h * p.kv_hs;
  // rows this thread moves in every tile, as loop-invariant byte offsets from
  // the tile's first row (buffer loads return 0 past the tile's valid rows)
  const int kc = tid % NKC;
  const int kr0 = tid / NKC;
  const int vkg = tid % 16, vdc = tid / 16;
  const bool vthread = tid < NVP;
  constexpr int ESZ = FP8 ? 1 : 2;
  const int row_bytes = (int)(p.kv_ls * ESZ);
  int koff[K_LOADS], voff[4];
#pragma unroll
  for (int i = 0; i < K_LOADS; ++i) koff[i] = (kr0 + i * KROWS_PER_PASS) * row_bytes + kc * 8 * ESZ;
#pragma unroll
  for (int e = 0; e < 4; ++e) voff[e] = (vkg * 4 + e) * row_bytes + vdc * 8 * ESZ;

  // ---- global -> register prefetch of one K/V tile ----
  raw_t kreg[K_LOADS];
  raw_t vreg[4];
  float mreg = 0.0f;
  TileIter ld;
  ld.seek(p, wi.j0);
  auto load_tile = [&]() {
    const int64_t base = (kv_off + ld.row0 * p.kv_ls) * ESZ;
    const int nbytes = ld.nvalid() * row_bytes;
    const auto kr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(ld.k) + base), (short)0, nbytes, 0x00020000);
    const auto vr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(ld.v) + base), (short)0, nbytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) kreg[i] = Chunk::bload(kr, koff[i]);
    if (vthread) {
#pragma unroll
      for (int e = 0; e < 4; ++e) vreg[e] = Chunk::bload(vr, voff[e]);
    }
    if constexpr (MASK) {
      if (tid < BN) mreg = tid < ld.nvalid() ? p.mask[b * p.mask_bs + ld.key0 + tid] : 0.0f;
    }
    ld.next(p);
  };

  // ---- register -> LDS store (K rows permuted, V transposed) ----
  auto store_tile = [&](int buf) {
    uint16_t* ks = smem + buf * (KBUF + VBUF);
    uint16_t* vs = ks + KBUF;
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int r = kr0 + i * KROWS_PER_PASS;
      *reinterpret_cast<uint4*>(ks + sig(r) * KS + kc * 8) = Chunk::to_bf16(kreg[i]);
    }
    if (vthread) {
      uint4 v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = Chunk::to_bf16(vreg[e]);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t a0 = (&v[0].x)[w], a1 = (&v[1].x)[w], a2 = (&v[2].x)[w], a3 = (&v[3].x)[w];
        // d = vdc*8 + 2w (low halves) and 2w+1 (high halves); keys vkg*4 .. +3
        uint2 lo, hi;
        lo.x = __builtin_amdgcn_perm(a1, a0, 0x05040100u);
        lo.y = __builtin_amdgcn_perm(a3, a2, 0x05040100u);
        hi.x = __builtin_amdgcn_perm(a1, a0, 0x07060302u);
        hi.y = __builtin_amdgcn_perm(a3, a2, 0x07060302u);
        *reinterpret_cast<uint2*>(vs + (vdc * 8 + 2 * w) * VS + vkg * 4) = lo;
        *reinterpret_cast<uint2*>(vs + (vdc * 8 + 2 * w + 1) * VS + vkg * 4) = hi;
      }
    }
    if constexpr (MASK) {
      if (tid < BN) mask_s[buf][tid] = mreg;
    }
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16_t{};
  // Running max in the base-2 logit domain.  It is only raised when a new
  // maximum exceeds it by more than kLazy (then O and l are rescaled); in
  // between, P = 2^(x - m) may reach 2^kLazy, which float32 sums and bf16 P
  // represent exactly enough.  Exact: O and l always share the same m.
  constexpr float kLazy = 8.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;  // sum over this lane's 16-key halves

  if (ntiles > 0) {
    load_tile();
    store_tile(0);
    if (ntiles > 1) load_tile();
    __syncthreads();
  }
  TileIter cp;
  cp.seek(p, wi.j0);

  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    if (j + 1 < ntiles) {
      store_tile(buf ^ 1);
      if (j + 2 < ntiles) load_tile();
    }
    const uint16_t* ks = smem + buf * (KBUF + VBUF);
    const uint16_t* vs = ks + KBUF;
    const int nvalid = cp.nvalid();

    // per-tile logit scale (and V scale for fp8)
    float c_log2 = p.scale_log2;
    float v_scale = 1.0f;
    if constexpr (FP8) {
      const int64_t f = cp.row0 / p.frame;
      c_log2 *= p.k_sc[cp.s][b * p.sc_bs + h * p.sc_hs + f];
      v_scale = p.v_sc[cp.s][b * p.sc_bs + h * p.sc_hs + f];
    }

    // ---- S^T = K Q^T, fragments read one k-step ahead ----
    f32x16_t sacc[2] = {f32x16_t{}, f32x16_t{}};
    const uint16_t* kfrag = ks + li * KS + hg * 8;
    bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(kfrag);
    bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(kfrag + 32 * KS);
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      bf16x8_t n0 = a0, n1 = a1;
      if (s + 1 < QS) {
        n0 = *reinterpret_cast<const bf16x8_t*>(kfrag + (s + 1) * 16);
        n1 = *reinterpret_cast<const bf16x8_t*>(kfrag + 32 * KS + (s + 1) * 16);
      }
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[s], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[s], sacc[1], 0, 0, 0);
      a0 = n0;
      a1 = n1;
    }
    // first V^T fragments, in flight during the softmax
    const uint16_t* vfrag = vs + li * VS + hg * 8;
    bf16x8_t va = *reinterpret_cast<const bf16x8_t*>(vfrag);
    bf16x8_t vb = *reinterpret_cast<const bf16x8_t*>(vfrag + 16);

    // ---- online softmax on the accumulators (base-2 domain) ----
    if constexpr (MASK) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * 32 + 16 * (r >> 3) + 8 * hg + (r & 7);
          sacc[kb][r] = fmaxf((sacc[kb][r] * p.scale + mask_s[buf][key]) * kLog2e, -3.0e38f);
        }
    }
    if (nvalid < BN) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb * 32 + 16 * (r >> 3) + 8 * hg + (r & 7);
          if (key >= nvalid) sacc[kb][r] = -INFINITY;
        }
    }
    float mt = sacc[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
    mt = pair_max(mt);
    // logits are x = s * c (c > 0), so max(x) = max(s) * c
    const float c = MASK ? 1.0f : c_log2;
    const float m_tile = mt * c;
    const bool raise = m_tile > m_run + kLazy;
    if (__builtin_amdgcn_ballot_w64(raise)) {
      const float m_new = fmaxf(m_run, m_tile);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
    }
    // all keys masked so far: keep the exponent finite
    const float neg_m = (m_run == -INFINITY) ? 0.0f : -m_run;

    float psum = 0.0f;
    bf16x8_t pf[4];
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const int kb = ks4 >> 1, t = ks4 & 1;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][8 * t + e], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][8 * t + e + 1], c, neg_m));
        psum += p0 + p1;
        w[e >> 1] = FP8 ? pack_bf16x2(p0 * v_scale, p1 * v_scale) : pack_bf16x2(p0, p1);
      }
      pf[ks4] = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
    }
    l_run += psum;

    // ---- O^T += V^T P^T, fragments read one step ahead ----
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int ks4 = 0; ks4 < 4; ks4 += 2) {
        bf16x8_t na = va, nb = vb;
        const int nd = (ks4 + 2 < 4) ? d : d + 1;
        const int nk = (ks4 + 2 < 4) ? ks4 + 2 : 0;
        if (nd < DB) {
          na = *reinterpret_cast<const bf16x8_t*>(vfrag + nd * 32 * VS + nk * 16);
          nb = *reinterpret_cast<const bf16x8_t*>(vfrag + nd * 32 * VS + (nk + 1) * 16);
        }
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pf[ks4], oacc[d], 0, 0, 0);
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, pf[ks4 + 1], oacc[d], 0, 0, 0);
        va = na;
        vb = nb;
      }
    }
    cp.next(p);
    __syncthreads();
  }

  // ---- epilogue: combine the two lane halves' sums, then store or publish ----
  finish_tile<D>(p, wi, b, h, qt, (int)(threadIdx.x >> 6) * 32 + (int)(threadIdx.x & 31), oacc, m_run,
                 pair_sum(l_run));
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// ---------------------------------------------------------------------------
// Software-pipelined direct kernel (bf16; K token-major, V key-major in HBM).
//
// K and V^T tiles go HBM -> LDS with buffer_load ... lds (gfx950 writes 16
// bytes per lane straight into LDS: lane L of an instruction lands at base +
// 16*L), so no VGPRs and no VALU work go into staging.  Each instruction
// covers 64 consecutive 16-byte LDS chunks of a padded tile: a K row is 16
// data chunks plus 1 pad chunk (272-byte rows), a V^T row (one head-dim
// channel, 64 keys) 8 data chunks plus 1 pad; lanes that fall on a pad chunk
// re-read a valid chunk.  The K-row order swap and the V transpose both
// happen in the address each lane reads from.  V must be stored key-major
// (the KV arena's V layout); a segment's last 8-token chunk is read whole and
// its keys past the segment end are masked out of the softmax.
//
// The per-tile vector work is cut down and moved under the matrix cores:
//
// * P = 2^(S*c - m) (c = scale*log2 e) is one v_fma and one v_exp per score:
//   no tile maximum is taken on the common path.
// * The row sum (fp32 adds of the P values) doubles as the overflow check:
//   m is not raised every tile.  While the per-lane sum of a tile stays at or below 2^16, every P
//   of that tile is at most 2^16, which fp32 sums and bf16 P carry as exactly
//   as P <= 1.  When a lane's sum goes above it, the tile maximum is taken
//   and m, O and l are rescaled before P is redone (the online normaliser of
//   Milakov & Gimelshein 2018).  The first tile sets m from its own maximum,
//   so the sums never underflow.  Logits stay fp32-exact (Q is not rescaled).
// * Pipeline: iteration j computes O += V(j-1)^T P(j-1) on the matrix cores
//   while the vector unit turns S(j) into P(j), then S(j+1) = K(j+1) Q^T.
//   K is loaded two tiles ahead and V one tile ahead of their use; one
//   barrier per tile frees the buffers read in the previous iteration.
//
// fp8 K/V (token-major e4m3 codes with per-(batch, head, frame) scales) use
// the same slot program (tiles cut at frame boundaries, see KeyStreamT).
// Their tiles are staged through registers instead:
// each thread loads 8-byte chunks of the next tiles from HBM one iteration
// ahead, and decodes them (exactly) to bf16 into the LDS buffers the barrier
// freed, K rows in the swapped order and V transposed with v_perm, so every
// code is decoded once per workgroup.  The decode and the next loads are
// spread over the slot program of the tile, under its matrix work.  A tile never crosses a frame
// (KeyStreamT<true>), so its scales are two scalars: the K scale joins
// the logit scale, c_j = c * sk_j, and the V scale joins the exponent,
// P' = 2^(S c_j - m + log2 sv_j) = sv_j P, so the PV MFMAs read plain codes;
// the row sum and the overflow check use sum(P') / sv_j.
// ---------------------------------------------------------------------------

// One operand (K or V) of the concatenated segments, walked tile by tile with
// wave-uniform state: the segment, the keys it has left from the current
// tile on, and the byte address of the current tile's first key (segment base
// + the (b, h) offset + the rows already passed).  Total keys < 2^31 (checked
// on the host).
//
// FRAMED (fp8 K/V, one scale per frame): tiles never cross a frame.  A frame
// of F tokens is cut into ceil(F / 64) tiles, the last one partial when F is
// not a multiple of 64, and a segment's last frame may itself be partial; a
// segment starts on a frame boundary (frame-aligned arena spans).  frem holds
// the keys of the current frame from the current tile on.
template <bool FRAMED>
struct KeyStreamT {
  int s, rem, frem;
  int lim = 0x7FFFFFFF;  // keys past this index of the concatenated sequence are not part of the stream
  const char* ptr;
  __device__ __forceinline__ void enter(const void* const* base, int64_t head, const FlashParams& p, int seg) {
    s = seg;
    rem = (int)((p.seg_start[seg + 1] < lim ? p.seg_start[seg + 1] : (int64_t)lim) - p.seg_start[seg]);
    ptr = reinterpret_cast<const char*>(base[seg]) + head;
    if constexpr (FRAMED) frem = p.frame;
  }
  __device__ __forceinline__ void seek(const void* const* base, int64_t head, int64_t tile_bytes,
                                       const FlashParams& p, int j) {
    int seg = 0;
    for (int i = 1; i < p.n_seg; ++i) seg = (j >= p.tile_start[i]) ? i : seg;
    enter(base, head, p, seg);
    const int t = j - p.tile_start[seg];
    if constexpr (FRAMED) {
      const int tpf = (p.frame + kBN - 1) / kBN;  // tiles per frame
      const int fr = t / tpf, k = t - fr * tpf;
      const int pos = fr * p.frame + k * kBN;
      frem = p.frame - k * kBN;
      rem -= pos;
      ptr += (int64_t)pos * (tile_bytes / kBN);
    } else {
      rem -= t * kBN;
      ptr += t * tile_bytes;
    }
  }
  __device__ __forceinline__ void next(const void* const* base, int64_t head, int64_t tile_bytes,
                                       const FlashParams& p) {
    if constexpr (FRAMED) {
      const int len = nvalid();
      rem -= len;
      ptr += (int64_t)len * (tile_bytes / kBN);
      frem -= len;
      if (frem == 0) frem = p.frame;
    } else {
      rem -= kBN;
      ptr += tile_bytes;
    }
    if (rem <= 0 && s + 1 < p.n_seg) enter(base, head, p, s + 1);
  }
  __device__ __forceinline__ int nvalid() const {
    const int n = rem < kBN ? rem : kBN;
    if constexpr (FRAMED) return frem < n ? frem : n;
    return n;
  }
  // first key of the current tile, counted from its segment's start
  __device__ __forceinline__ int row0(const FlashParams& p) const {
    return (int)(p.seg_start[s + 1] - p.seg_start[s]) - rem;
  }
};

// The pipelined kernels' body.  FRAMED (fp8 only): frames that are not a
// whole number of 64-key tiles, cut at frame boundaries (KeyStreamT<true>,
// its own kernel); frames of 64k tokens take the plain tiling, which never
// crosses a frame either and keeps the hot kernel's scalar state and
// registers as they were (the framed state costs the D = 128 instance
// register spills).
//
// PAIR: 8-wave workgroups of two groups of 4 waves (waves w and w + 4
// share a SIMD) that own two q-tiles of one head (pair_work) and read one
// K/V stream.  bf16: only group 0 issues the tile loads, so group 1's waves
// run their slot programs while group 0's wait on the load pipe.  fp8:
// group 0 stages (loads and decodes) the K tiles and group 1 the V tiles,
// so each thread stages half of what a 4-wave workgroup's does for the
// same two q-tiles.  The groups meet at every per-tile barrier: the two
// waves of a SIMD finish together, where two 4-wave workgroups on one CU do
// not (the older one's waves win the issue arbitration and finish about a
// quarter earlier, leaving the CU half busy until the other ends).
template <int D, bool FP8, bool FRAMED, bool PAIR = false>
__device__ __forceinline__ void flash_pipe_body(const FlashParams& p) {
  static_assert(FP8 || !FRAMED, "frame tiling is an fp8 feature");
  static_assert(!(PAIR && FRAMED), "pair workgroups take the plain tiling");
  constexpr int BM = kBM, BN = kBN;
  constexpr int NKC = D / 8;
  constexpr int KS = D + 8;
  // V^T tile rows (one head-dim channel, BN keys = 8 chunks of 16 bytes):
  // with D = 128 two rows share one pad chunk (17 chunks per pair, 17 load
  // instructions per tile), else each row has its own (9 chunks).  Either
  // way 16 consecutive rows' same chunk covers 16 distinct 16-byte bank
  // groups, so a fragment read is conflict-free.
  constexpr bool VPAIR = (D / 2) * 17 % 64 == 0;
  constexpr int VS = BN + 8;                      // row stride without pairing
  constexpr int VPS = 2 * BN + 8;                 // pair stride with pairing
  constexpr int KBUF = BN * KS;
  constexpr int VBUF = VPAIR ? (D / 2) * VPS : D * VS;
  constexpr int KINS = BN * (NKC + 1) / 64;
  constexpr int VINS = VPAIR ? (D / 2) * 17 / 64 : D * 9 / 64;
  constexpr int KSLOT = (KINS + 3) / 4;
  constexpr int VSLOT = (VINS + 3) / 4;
  constexpr int DB = D / 32;
  constexpr int QS = D / 16;
  constexpr float kOver = 65536.0f;  // largest per-lane tile sum kept without raising m
  static_assert(BN * (NKC + 1) % 64 == 0 && (VPAIR || D * 9 % 64 == 0), "tile does not split into whole instructions");
  // element offset of V^T row r in a V buffer
  auto vrow = [](int r) { return VPAIR ? (r >> 1) * VPS + (r & 1) * BN : r * VS; };

  __shared__ __attribute__((aligned(16))) uint16_t kbuf[2][KBUF];
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[2][VBUF];

  const int grp = PAIR ? (__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) >> 2) : 0;
  const WorkItem wi = PAIR ? pair_work(p, blockIdx.x, grp, p.tile_start[p.n_seg])
                           : work_item(p, blockIdx.x, p.tile_start[p.n_seg]);
  const bool loader = !PAIR || grp == 0;  // issues the K/V tile loads
  const int qt = wi.qtile % p.n_qtiles;
  const int bh = wi.qtile / p.n_qtiles;
  const int b = bh / p.H, h = bh % p.H;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) & 3;
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, hg = lane >> 5;
  const int qi = qt * BM + wave * 32 + li;
  // a per-batch key count ends this row's key tiles early (the streams stop
  // at it, so its last tile is partial and masked like a segment's last)
  const int klim = (!FP8 && p.n_klen) ? p.klen[b] : 0x7FFFFFFF;
  int jend = wi.j1;
  if (!FP8 && p.n_klen) {
    const int tb = tiles_below(p, klim);
    jend = jend < tb ? jend : tb;
  }
  const int ntiles = jend > wi.j0 ? jend - wi.j0 : 0;

  // ---- per-lane load offsets (bytes from a tile's first key), loop invariant ----
  const int row_bytes = (int)(p.kv_ls * (FP8 ? 1 : 2));
  const int vrow_bytes = (int)(p.v_ds * 2);
  auto kpos = [&](int i, int& r, int& c) {
    const int pch = (wave + 4 * i) * 64 + lane;
    r = sig(pch / (NKC + 1));
    c = pch % (NKC + 1);
    c = c < NKC ? c : 0;
  };
  // the (channel, 16-byte chunk) load slot i of this lane fills; a pad slot
  // re-reads a valid chunk
  auto vpos = [&](int i, int& d, int& c) {
    const int pch = (wave + 4 * i) * 64 + lane;
    if constexpr (VPAIR) {
      const int q = pch % 17;
      d = 2 * (pch / 17) + (q < 16 ? q >> 3 : 0);
      c = q < 16 ? (q & 7) : 0;
    } else {
      d = pch / 9;
      d = d < D ? d : 0;
      c = pch % 9;
      c = c < 8 ? c : 0;
    }
  };
  int koff[KSLOT], voff[VSLOT];
#pragma unroll
  for (int i = 0; i < KSLOT; ++i) {
    int r, c;
    kpos(i, r, c);
    koff[i] = r * row_bytes + c * 16;
  }
#pragma unroll
  for (int i = 0; i < VSLOT; ++i) {
    int d, c;
    vpos(i, d, c);
    voff[i] = d * vrow_bytes + c * 16;
  }

  const int64_t k_head = (b * p.kv_bs + h * p.kv_hs) * (FP8 ? 1 : 2);
  const int64_t v_head = FP8 ? k_head : (b * p.v_bs + h * p.v_hs) * 2;
  const int64_t k_tile = (int64_t)BN * row_bytes;
  const int64_t v_tile = FP8 ? k_tile : BN * 2;
  KeyStreamT<FRAMED> kit, vit;
  kit.lim = klim;
  vit.lim = klim;
  kit.seek(p.k_ptr, k_head, k_tile, p, wi.j0);
  vit.seek(p.v_ptr, v_head, v_tile, p, wi.j0);
  // LDS address of this wave's first load slot in a buffer; the empty asm
  // keeps the compiler from holding every (buffer, slot) address in its own
  // scalar register across the loop (they cost one s_add each instead)
  auto lds_slot0 = [&](uint16_t* buf0) {
    uint32_t a = (uint32_t)(uintptr_t)(lds_ptr_t)(buf0 + wave * 512);
    asm volatile("" : "+s"(a));
    return a;
  };
  // One load instruction ("slot" i of this wave) of a K or V tile.  rs is the
  // tile's buffer resource, l0 this wave's first LDS chunk of the buffer and
  // nv the tile's valid keys.  K rows past a segment's end lie outside the
  // partial tile's buffer range (issue_k): those lanes load zeros, and their
  // scores are masked out of the softmax.  V (8-key chunks of key-major rows)
  // re-reads the segment's last chunk for the positions past its end.
  auto k_load = [&](__amdgpu_buffer_rsrc_t rs, uint32_t l0, int i) {
    if (loader && i < KSLOT && wave + 4 * i < KINS)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(uintptr_t)(l0 + i * 4096), 16, koff[i], 0, 0, 0);
  };
  auto v_load = [&](__amdgpu_buffer_rsrc_t rs, uint32_t l0, int nv, int i) {
    if (loader && i < VSLOT && wave + 4 * i < VINS) {
      int off = voff[i];
      if (nv < BN) {
        int d, c;
        vpos(i, d, c);
        off = d * vrow_bytes + min(c, (nv + 7) / 8 - 1) * 16;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(uintptr_t)(l0 + i * 4096), 16, off, 0, 0, 0);
    }
  };
  auto rsrc = [&](const char* ptr) { return __builtin_amdgcn_make_buffer_rsrc((void*)ptr, (short)0, 0x7FFFFFFF, 0x00020000); };
  // whole tiles (every tile but a segment's last) take one branch and issue
  // their loads from the precomputed offsets; a K tile's buffer range ends at
  // its last valid row (a whole tile's is left open), so the partial tile
  // issues the same loads
  auto issue_k = [&](int buf) {
    const int nv = kit.nvalid();
    const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)kit.ptr, (short)0, nv == BN ? 0x7FFFFFFF : nv * row_bytes,
                                                      0x00020000);
    const uint32_t l0 = lds_slot0(kbuf[buf]);
#pragma unroll
    for (int i = 0; i < KSLOT; ++i) k_load(rs, l0, i);
    kit.next(p.k_ptr, k_head, k_tile, p);
  };
  auto issue_v = [&](int buf) {
    const auto rs = rsrc(vit.ptr);
    const uint32_t l0 = lds_slot0(vbuf[buf]);
    const int nv = vit.nvalid();
    if (nv == BN) {
#pragma unroll
      for (int i = 0; i < VSLOT; ++i) v_load(rs, l0, BN, i);
    } else {
#pragma unroll
      for (int i = 0; i < VSLOT; ++i) v_load(rs, l0, nv, i);
    }
    vit.next(p.v_ptr, v_head, v_tile, p);
  };

  // ---- fp8: register staging of the next K and V tiles ----
  // K: thread t moves 8-code chunk t % NKC of rows t / NKC + FROWS * i.
  // V: thread t (< NVP) moves 8-channel chunk t / 16 of keys 4 * (t % 16) .. +3
  // and writes them transposed (4 keys of 8 channel rows); 16 consecutive
  // lanes fill one 128-byte V^T row segment, so the LDS writes are
  // conflict-free.  Loads past a partial tile's last key return 0 (buffer
  // range check).
  constexpr int FROWS = 256 / NKC;
  constexpr int FKL = BN / FROWS;
  constexpr int NVP = (BN / 4) * NKC;
  const int tid = threadIdx.x & 255;  // thread index within the group
  const int fkc = tid % NKC, fkr = tid / NKC;
  const int fvg = tid % 16, fvc = tid / 16;
  const bool fv_on = tid < NVP;
  const bool stage_k = !PAIR || grp == 0, stage_v = !PAIR || grp == 1;  // wave-uniform
  uint2 kreg[FP8 ? FKL : 1], vreg[FP8 ? 4 : 1];
  auto load_k8 = [&]() {
    if (!stage_k) return;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)kit.ptr, (short)0, kit.nvalid() * row_bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < FKL; ++i) kreg[i] = KVChunk<true>::bload(rs, (fkr + FROWS * i) * row_bytes + fkc * 8);
    kit.next(p.k_ptr, k_head, k_tile, p);
  };
  auto load_v8 = [&]() {
    if (!stage_v) return;
    const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)vit.ptr, (short)0, vit.nvalid() * row_bytes, 0x00020000);
    if (fv_on) {
#pragma unroll
      for (int e = 0; e < 4; ++e) vreg[e] = KVChunk<true>::bload(rs, (fvg * 4 + e) * row_bytes + fvc * 8);
    }
    vit.next(p.v_ptr, v_head, v_tile, p);
  };
  auto store_k8_row = [&](int buf, int i) {
    if (!stage_k) return;
    *reinterpret_cast<uint4*>(&kbuf[buf][sig(fkr + FROWS * i) * KS + fkc * 8]) = KVChunk<true>::to_bf16(kreg[i]);
  };
  auto store_k8 = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FKL; ++i) store_k8_row(buf, i);
  };
  auto store_v8_half = [&](int buf, int half) {
    if constexpr (FP8) {   // vreg holds the four staged code chunks only in the fp8 instances
      if (!stage_v || !fv_on) return;
      const uint32_t d0 = half ? vreg[0].y : vreg[0].x, d1 = half ? vreg[1].y : vreg[1].x;
      const uint32_t d2 = half ? vreg[2].y : vreg[2].x, d3 = half ? vreg[3].y : vreg[3].x;
      // channels 4*half + {0, 1} and {2, 3} of keys (0, 1) and (2, 3)
      const uint32_t k01a = __builtin_amdgcn_perm(d1, d0, 0x05010400u), k23a = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
      const uint32_t k01b = __builtin_amdgcn_perm(d1, d0, 0x07030602u), k23b = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
      const int r0 = fvc * 8 + 4 * half;
      uint16_t* vb = &vbuf[buf][fvg * 4];
      *reinterpret_cast<uint2*>(vb + vrow(r0)) = make_uint2(KVChunk<true>::pair(k01a, false), KVChunk<true>::pair(k23a, false));
      *reinterpret_cast<uint2*>(vb + vrow(r0 + 1)) = make_uint2(KVChunk<true>::pair(k01a, true), KVChunk<true>::pair(k23a, true));
      *reinterpret_cast<uint2*>(vb + vrow(r0 + 2)) = make_uint2(KVChunk<true>::pair(k01b, false), KVChunk<true>::pair(k23b, false));
      *reinterpret_cast<uint2*>(vb + vrow(r0 + 3)) = make_uint2(KVChunk<true>::pair(k01b, true), KVChunk<true>::pair(k23b, true));
    }
  };
  // V(j) to LDS: the codes are interleaved by key before decoding: one v_perm
  // puts channels c and c + 1 of keys 2i and 2i + 1 into one word, whose low
  // and high byte pairs decode into the (key 2i, key 2i + 1) bf16 pairs of the
  // two V^T rows.  8 perms and 16 decodes per thread, where decoding first and
  // transposing the bf16 pairs takes 16 of each.
  auto store_v8 = [&](int buf) {
    store_v8_half(buf, 0);
    store_v8_half(buf, 1);
  };
  // the tile the softmax works on: its valid keys and (fp8) its scales
  KeyStreamT<FRAMED> cit;
  if constexpr (FP8) cit.seek(p.k_ptr, 0, 0, p, wi.j0);
  struct TileScale { float c, off, inv; };  // logit scale, exponent offset log2 sv, 1 / sv
  auto tile_scale = [&]() -> TileScale {
    if constexpr (FP8) {
      const int64_t o = b * p.sc_bs + h * p.sc_hs + cit.row0(p) / p.frame;
      const float sk = p.k_sc[cit.s][o];
      const float sv = p.v_sc[cit.s][o];
      return TileScale{p.scale_log2 * sk, __log2f(sv), 1.0f / sv};
    } else {
      return TileScale{p.scale_log2, 0.0f, 1.0f};
    }
  };

  // ---- Q^T fragments, resident for the whole key loop ----
  bf16x8_t qf[QS];
  auto load_q = [&]() {
    const bool ok = qi < p.Lq;
    const uint16_t* qp = p.q + b * p.q_bs + (int64_t)(ok ? qi : 0) * p.q_ls + h * p.q_hs + hg * 8;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      uint4 v = ok ? *reinterpret_cast<const uint4*>(qp + s * 16) : make_uint4(0, 0, 0, 0);
      qf[s] = __builtin_bit_cast(bf16x8_t, v);
    }
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) oacc[d] = f32x16_t{};
  float m_run = -INFINITY;  // per query, base-2 logit units
  float l_run = 0.0f;       // this lane's share of the row sum
  const ltx_bf16x2_t ones = __builtin_bit_cast(ltx_bf16x2_t, 0x3F803F80u);  // bf16 pair (1, 1)

  // keys past a partial tile's valid count drop out of the softmax (the
  // lane's key is kb*32 + 16*(r/8) + 8*hg + r%8: compare its constant part
  // with one per-lane limit so no key index is kept in registers)
  auto mask_tail = [&](f32x16_t (&s)[2], int nvalid) {
    const int lim = nvalid - 8 * hg;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb * 32 + 16 * (r >> 3) + (r & 7) >= lim) s[kb][r] = -INFINITY;
  };
  // largest base-2 logit of a tile for this lane's query (c > 0)
  auto tile_max = [&](const f32x16_t (&s)[2], float c) {
    float mt = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    return pair_max(mt) * c;
  };
  // P = 2^(S*c + off) packed to bf16 pairs (pw[i] holds scores 2i, 2i+1 in
  // accumulator order); returns this lane's sum.  Used outside the slot
  // program (first tile, rescale).
  auto exp_all = [&](const f32x16_t (&s)[2], uint32_t (&pw)[16], float c, float neg_m) {
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
      const int kb = i >> 4, r = i & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], c, neg_m));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r + 1], c, neg_m));
      pw[i >> 1] = pack_bf16x2(p0, p1);
      ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ltx_bf16x2_t, pw[i >> 1]), ones, ps, false);
    }
    return ps;
  };
  // S = K Q^T of a whole tile from kbuf[buf] (first tile only)
  auto qk_tile = [&](int buf, f32x16_t (&s)[2]) {
    const f32x16_t zero = f32x16_t{};
    const uint16_t* kf = &kbuf[buf][li * KS + hg * 8];
#pragma unroll
    for (int k = 0; k < QS; ++k) {
      const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(kf + k * 16);
      const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(kf + 32 * KS + k * 16);
      s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, qf[k], k == 0 ? zero : s[0], 0, 0, 0);
      s[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, qf[k], k == 0 ? zero : s[1], 0, 0, 0);
    }
  };
  // O^T += V^T P^T of a whole tile from vbuf[buf] (last tile only)
  auto pv_tile = [&](int buf, const uint32_t (&pw)[16]) {
    const uint16_t* vf = &vbuf[buf][vrow(li) + hg * 8];
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const bf16x8_t pf =
          __builtin_bit_cast(bf16x8_t, make_uint4(pw[4 * k4], pw[4 * k4 + 1], pw[4 * k4 + 2], pw[4 * k4 + 3]));
#pragma unroll
      for (int d = 0; d < DB; ++d)
        oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            *reinterpret_cast<const bf16x8_t*>(vf + vrow(d * 32) + k4 * 16), pf, oacc[d], 0, 0, 0);
    }
  };
  // bf16: the tile loads go straight to LDS and are counted by vmcnt, so
  // they must land before the barrier publishes them.  fp8: the staged tiles
  // reach LDS through ds_writes (the barrier waits for those), and the
  // loads in flight only fill registers that the next slot program decodes
  // (the compiler waits for each before its use), so they stay in flight
  // across the barrier: 194.5 -> 192.8 us at 1152 x 4608.
  auto publish = [&]() {
    if constexpr (!FP8) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  // ---- the slot program of one tile ----
  // NS matrix-core slots: PV(j-1) (4*DB MFMAs over vbuf[vb]) then S(j+1)
  // (2*QS MFMAs over kbuf[kbf]).  Each slot issues its MFMA, the LDS read
  // of the fragment PREF slots ahead, and a slice of the softmax of S(j).
  // With 32 slots (D = 128) that is one score per slot: score i has its fma
  // at slot i, its exp at i + 1 and its row-sum add at i + 2, and pair q its
  // bf16 pack at 2q + 3 (whole pairs per slot, fma of both at 2q and the
  // rest at 2q + 1 and 2q + 3, measured 1 % slower: the odd slots then carry
  // two exps, the adds and the pack).  With 16 slots (D = 64) score pair p
  // has its fma at slot p, its exp at p + 1 and its pack and adds at p + 3.  A
  // scheduling fence closes every slot, so the exp work stays spread under
  // the MFMAs (each 32x32x16 MFMA leaves room for about two exp and two
  // other VALU instructions of the same SIMD).  The row sum adds the fp32 P
  // values: v_dot2c_f32_bf16 over the packed pair (one instruction instead
  // of two) waits for the SIMD's matrix pipeline on gfx950, about one MFMA
  // per instruction while the other wave's MFMAs run, where adds issue
  // beside them (fp8 at 1152 x 4608: 199.0 -> 191.0 us with the adds).
  // The fully unrolled slot program of the fp8 instances is larger than
  // LLVM's default limit for a pragma-requested full unroll; the library is
  // built with a higher one (-pragma-unroll-threshold), without which the
  // loop stays rolled and its per-slot arrays go to scratch memory.
  constexpr int NS = 4 * DB + 2 * QS;
  constexpr int PREF = 3;
  // fp8 staging inside the slot program: one unit (a K row chunk, a V half,
  // a load) every kStageStride slots from kStageSlot0 on
  constexpr int kStageSlot0 = 0, kStageStride = 1;
  const uint16_t* vf0 = &vbuf[0][vrow(li) + hg * 8];
  const uint16_t* kf0 = &kbuf[0][li * KS + hg * 8];
  auto tile = [&](int vb, int kbf, const f32x16_t (&scur)[2], f32x16_t (&snext)[2], const uint32_t (&pprev)[16],
                  uint32_t (&pcur)[16], float& ps0, float& ps1, float c, float neg_m, auto&& slot_work) {
    const f32x16_t zero = f32x16_t{};
    const uint16_t* vf = vf0 + vb * VBUF;
    const uint16_t* kf = kf0 + kbf * KBUF;
    auto frag = [&](int t) -> bf16x8_t {
      if (t < 4 * DB) return *reinterpret_cast<const bf16x8_t*>(vf + vrow((t % DB) * 32) + (t / DB) * 16);
      const int u = t - 4 * DB;
      return *reinterpret_cast<const bf16x8_t*>(kf + (u & 1) * 32 * KS + (u >> 1) * 16);
    };
    bf16x8_t ring[PREF + 1];
#pragma unroll
    for (int t = 0; t < PREF; ++t) ring[t] = frag(t);
    float e0[16], e1[16];
    ps0 = 0.0f;
    ps1 = 0.0f;
#pragma unroll
    for (int t = 0; t < NS + 2; ++t) {
      if (t < NS) {
        if (t + PREF < NS) ring[(t + PREF) % (PREF + 1)] = frag(t + PREF);
        const bf16x8_t a = ring[t % (PREF + 1)];
        if (t < 4 * DB) {
          const int k4 = t / DB, d = t % DB;
          const bf16x8_t pf = __builtin_bit_cast(
              bf16x8_t, make_uint4(pprev[4 * k4], pprev[4 * k4 + 1], pprev[4 * k4 + 2], pprev[4 * k4 + 3]));
          oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, oacc[d], 0, 0, 0);
        } else {
          const int u = t - 4 * DB, kb = u & 1, kk = u >> 1;  // the two key blocks' chains alternate
          snext[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], kk == 0 ? zero : snext[kb], 0, 0, 0);
        }
      }
      slot_work(t);
      if constexpr (NS == 32) {
        // one score per slot: its fma at slot i, its exp at i + 1, its
        // row-sum add at i + 2, and the bf16 pack of pair q at 2q + 3, so
        // every slot carries the same vector work
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int q = i >> 1, kb = q >> 3, r = (q & 7) * 2 + (i & 1);
          float* e = (i & 1) ? e1 : e0;
          if (t == i) e[q] = __builtin_fmaf(scur[kb][r], c, neg_m);
          if (t == i + 1) e[q] = __builtin_amdgcn_exp2f(e[q]);
          if (t == i + 2) {
            float& ps = (i & 1) ? ps1 : ps0;
            ps = ps + e[q];
          }
        }
#pragma unroll
        for (int q = 0; q < 16; ++q)
          if (t == 2 * q + 3) {
            pcur[q] = pack_bf16x2(e0[q], e1[q]);
            asm volatile("" : "+v"(pcur[q]));
          }
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int kb = q >> 3, r = (q & 7) * 2;
          if ((2 * q * NS) / 32 == t) {
            e0[q] = __builtin_fmaf(scur[kb][r], c, neg_m);
            e1[q] = __builtin_fmaf(scur[kb][r + 1], c, neg_m);
          }
          if ((2 * q * NS) / 32 + 1 == t) {
            e0[q] = __builtin_amdgcn_exp2f(e0[q]);
            e1[q] = __builtin_amdgcn_exp2f(e1[q]);
          }
          if ((2 * q * NS) / 32 + 3 == t || (q == 15 && t == NS + 1 && (2 * q * NS) / 32 + 3 > NS + 1)) {
            pcur[q] = pack_bf16x2(e0[q], e1[q]);
            float& ps = (q & 1) ? ps1 : ps0;
            ps = ps + e0[q];
            ps = ps + e1[q];
            // with no use left in this slot the compiler would sink the pack
            // to the next tile's PV and issue all sixteen back to back after
            // the slot program; pin it here, under this slot's MFMA
            asm volatile("" : "+v"(pcur[q]));
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (ntiles > 0) {
    f32x16_t sa[2], sb[2];
    uint32_t pa[16], pb[16];  // P(j) of even / odd j
    // ---- prologue: S(0) sets m from its own maximum; P(0); S(1) ----
    int nv0;
    if constexpr (FP8) {
      // K(0), V(0), K(1) decoded into LDS; K(2) and V(1) left in registers
      nv0 = cit.nvalid();
      load_k8();
      load_v8();
      load_q();
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      store_k8(0);
      store_v8(0);
      if (ntiles > 1) {
        load_k8();
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        store_k8(1);
        load_v8();
      }
      if (ntiles > 2) load_k8();
      publish();
    } else {
      issue_k(0);
      if (ntiles > 1) issue_k(1);
      nv0 = vit.nvalid();  // valid keys of tile 0 (the V stream is at tile j before V(j) is issued)
      issue_v(0);
      load_q();  // its latency overlaps the first tiles' loads
      publish();
    }
    qk_tile(0, sa);
    if (nv0 < BN) mask_tail(sa, nv0);
    {
      const TileScale ts = tile_scale();
      m_run = tile_max(sa, ts.c);
      l_run = exp_all(sa, pa, ts.c, ts.off - m_run) * ts.inv;
      if constexpr (FP8) cit.next(p.k_ptr, 0, 0, p);
    }
    if (ntiles > 1) qk_tile(1, sb);
    if (ntiles > 2) {
      __syncthreads();  // every wave is done with K(0)
      if constexpr (FP8) {
        store_k8(0);                   // K(2)
        if (ntiles > 3) load_k8();     // K(3)
      } else {
        issue_k(0);                    // K(2)
      }
    }
    // ---- iteration j (1 <= j < ntiles): the slot program computes
    //      O += V(j-1)^T P(j-1), S(j+1) = K(j+1) Q^T and P(j) = 2^(S(j)c - m).
    //      On the last tile S(j+1) is computed from stale LDS and dropped. ----
    auto step = [&](int j, f32x16_t (&scur)[2], f32x16_t (&snext)[2], const uint32_t (&pprev)[16],
                    uint32_t (&pcur)[16]) {
      int nv;
      if constexpr (FP8) {
        // registers hold K(j+2) and V(j); LDS holds K(j+1) and V(j-1)
        publish();  // the buffers of K(j) and V(j-2) are free
        nv = cit.nvalid();
      } else {
        publish();  // K(j+1) and V(j-1) have landed; the buffers of K(j) and V(j-2) are free
        if (j + 2 < ntiles) issue_k(j & 1);  // K(j+2)
        nv = vit.nvalid();                   // valid keys of tile j
        issue_v(j & 1);                      // V(j)
      }
      if (nv < BN) mask_tail(scur, nv);
      const TileScale ts = tile_scale();
      float ps0, ps1;
      // fp8: the decode of K(j+2) and V(j) into the free buffers and the
      // loads of K(j+3) and V(j+1) into the freed registers ride in the slot
      // program, under the matrix work of tile j
      tile((j - 1) & 1, (j + 1) & 1, scur, snext, pprev, pcur, ps0, ps1, ts.c, ts.off - m_run, [&](int t) {
        if constexpr (FP8) {
#pragma unroll
          for (int i = 0; i < FKL; ++i)
            if (t == kStageSlot0 + kStageStride * i && j + 2 < ntiles) store_k8_row(j & 1, i);  // K(j+2)
          if (t == kStageSlot0 + kStageStride * FKL && j + 3 < ntiles) load_k8();               // K(j+3)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            if (t == kStageSlot0 + kStageStride * (FKL + 1 + hh)) store_v8_half(j & 1, hh);     // V(j)
          if (t == kStageSlot0 + kStageStride * (FKL + 3) && j + 1 < ntiles) load_v8();         // V(j+1)
        }
      });
      float ps = (ps0 + ps1) * ts.inv;
      if (__builtin_amdgcn_ballot_w64(ps > kOver)) {
        // raise m to the tile maximum, rescale O and l, redo P(j) from S(j)
        const float m_new = fmaxf(m_run, tile_max(scur, ts.c));
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < DB; ++d) oacc[d] *= alpha;
        ps = exp_all(scur, pcur, ts.c, ts.off - m_run) * ts.inv;
      }
      l_run += ps;
      if constexpr (FP8) cit.next(p.k_ptr, 0, 0, p);
    };
    int j = 1;
    for (; j + 1 < ntiles; j += 2) {
      step(j, sb, sa, pa, pb);
      step(j + 1, sa, sb, pb, pa);
    }
    if (j < ntiles) step(j, sb, sa, pa, pb);
    // ---- epilogue: O += V(n-1)^T P(n-1) ----
    publish();
    if ((ntiles - 1) & 1)
      pv_tile(1, pb);
    else
      pv_tile(0, pa);
  }

  // output staging: waves 0-3 in the K buffers, the pair kernel's group 1 in the V buffers
  static_assert(4 * 32 * (D + 8) <= 2 * KBUF && 4 * 32 * (D + 8) <= 2 * VBUF, "output staging region");
  const int owave = PAIR ? wave : (int)(threadIdx.x >> 6);
  uint16_t* stage = (PAIR && grp == 1 ? &vbuf[0][0] : &kbuf[0][0]) + owave * 32 * (D + 8);
  finish_tile<D>(p, wi, b, h, qt, owave * 32 + (int)(threadIdx.x & 31), oacc, m_run, pair_sum(l_run), stage);
}

template <int D, bool FP8>
__global__ void __launch_bounds__(256, 2) flash_fwd_pipe_kernel(const FlashParams p) {
  flash_pipe_body<D, FP8, false>(p);
}

// bf16 key-major V, or fp8 K/V in frames of whole 64-key tiles, with an even
// number of q-tiles per head: pair workgroups
template <int D, bool FP8>
__global__ void __launch_bounds__(512, 1) flash_fwd_pair_kernel(const FlashParams p) {
  flash_pipe_body<D, FP8, false, true>(p);
}

// fp8 frames that are not a whole number of 64-key tiles
template <int D>
__global__ void __launch_bounds__(256, 2) flash_fwd_pipe_framed_kernel(const FlashParams p) {
  flash_pipe_body<D, true, true>(p);
}

template <int D>
int launch_combine(const FlashParams& p, hipStream_t st) {
  if (p.split <= 1) return LTX_OK;
  const int64_t tail = (int64_t)p.B * p.H * p.n_qtiles - (p.pair ? 2 * (int64_t)p.n_full : p.n_full);
  const int64_t wg_per_tile = combine_wg_per_tile<D>();
  hipLaunchKernelGGL((flash_combine_kernel<D>), dim3((unsigned)(tail * wg_per_tile)), dim3(256), 0, st, p);
  LTX_LAUNCH_CHECK("ltx_flash_attn_fwd (combine)");
  return LTX_OK;
}

// Grid: whole q-tiles (pair kernel: units of two) first, then the key-range
// pieces of the tail ones.
inline int64_t grid_blocks(const FlashParams& p) {
  const int64_t nq = (int64_t)p.B * p.H * p.n_qtiles / (p.pair ? 2 : 1);
  return p.n_full + (nq - p.n_full) * p.split;
}

template <int D, bool FP8, bool FRAMED = false>
int launch_flash_pipe(const FlashParams& p, hipStream_t st) {
  static_assert(FP8 || !FRAMED, "frame tiling is an fp8 feature");
  const int64_t nblocks = grid_blocks(p);
  LTX_REQUIRE(nblocks <= 0x7FFFFFFF, "ltx_flash_attn_fwd: grid too large");
  if constexpr (FRAMED)
    hipLaunchKernelGGL((flash_fwd_pipe_framed_kernel<D>), dim3((unsigned)nblocks), dim3(256), 0, st, p);
  else if (p.pair)
    hipLaunchKernelGGL((flash_fwd_pair_kernel<D, FP8>), dim3((unsigned)nblocks), dim3(512), 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_pipe_kernel<D, FP8>), dim3((unsigned)nblocks), dim3(256), 0, st, p);
  LTX_LAUNCH_CHECK("ltx_flash_attn_fwd");
  return launch_combine<D>(p, st);
}

template <int D, bool FP8, bool MASK>
int launch_flash(const FlashParams& p, hipStream_t st) {
  const int64_t nblocks = grid_blocks(p);
  LTX_REQUIRE(nblocks <= 0x7FFFFFFF, "ltx_flash_attn_fwd: grid too large");
  hipLaunchKernelGGL((flash_fwd_kernel<D, FP8, MASK>), dim3((unsigned)nblocks), dim3(256), 0, st, p);
  LTX_LAUNCH_CHECK("ltx_flash_attn_fwd");
  return launch_combine<D>(p, st);
}

}  // namespace ltx

using namespace ltx;

// Resident workgroups the device holds for this kernel (CUs x occupancy),
// computed once per device under a once-flag (calls from several host
// threads may race to fill it); one table per kernel (each instantiation of
// the template has its own).
constexpr int kMaxDevices = 64;
struct Slots {
  int slots;   // resident workgroups (0: unknown, no split is planned)
  int pieces;  // key-range pieces a split tail aims for (see plan_split)
};
template <auto Kernel>
Slots resident_slots(int threads = 256) {
  static std::once_flag once[kMaxDevices];
  static Slots slots[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return Slots{0, 1};
  std::call_once(once[dev], [&]() {
    int cus = 0, occ = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, Kernel, threads, 0) != hipSuccess) {
      slots[dev] = Slots{0, 1};
      return;
    }
    occ = occ > 0 ? occ : 1;
    slots[dev] = Slots{cus * occ, cus};  // pieces: one per CU until flash_slots says otherwise
  });
  return slots[dev];
}

// Tail q-tiles (those past the last whole round of resident slots) and how
// many key ranges each is cut into: about s.pieces pieces in all.  For the
// bf16 pipelined kernel that is one per CU.  Of the workgroups one CU holds,
// the oldest one's waves win the issue arbitration: with two of its 4-wave
// workgroups per CU the older finishes its q-tile about a quarter before the
// younger, so one slot per CU frees early.  Pieces that fill just those
// slots run beside the younger workgroups' last stretch; pieces for every
// slot (twice as many, half as long) leave their second half to start only
// when the younger workgroups end, with a CU half busy until they drain
// (193.7 against 184.8 us for the bf16 step at 1152 x 4608, 8 against 4
// pieces per tail q-tile).  The fp8 kernel measured the other way round
// (194-196 against 200-202 us) while its per-tile barrier also waited for
// the register-staged loads; without that wait it gains from one piece per
// CU too (187.6 against 180.4 us).  The staged kernel's pieces fill every
// slot.  Each piece keeps >= 4 key tiles behind a whole round.  A grid
// that is a single partial round (fewer q-tiles than slots: the 75-query
// audio and V2A calls, 64 q-tiles at B = 2 and 32 heads) is split too, into
// pieces of >= 2 key tiles, so its few workgroups spread over the CUs: V2A
// 75 x 1152 16.0 -> 12.5 us, audio self-attention 75 x 675 14.2 -> 12.6 us.
// Zero tail tiles: no split.
inline void plan_split(int64_t nq, int ntiles, Slots s, int64_t* n_full, int* split) {
  *n_full = nq;
  *split = 1;
  const int slots = s.slots;
  if (slots <= 0 || nq % slots == 0) return;
  const int64_t full = (nq / slots) * slots;
  const int64_t tail = nq - full;
  int sp = (int)(s.pieces / tail);
  if (sp > kMaxSplit) sp = kMaxSplit;
  // pieces keep >= 4 key tiles behind a whole round, >= 2 when the grid is
  // a single partial round (its few workgroups would leave most CUs idle)
  const int min_tiles = full > 0 ? 4 : 2;
  if (sp > ntiles / min_tiles) sp = ntiles / min_tiles;
  if (sp < 2) return;
  *n_full = full;
  *split = sp;
}

inline int64_t workspace_bytes_for(int64_t tail, int split, int64_t D) {
  return tail * split * kBM * (2 * 4 + D * 2);  // (max, sum) fp32 + bf16 O row
}

inline int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

// Resident slots of the kernel a call with head size D takes: for
// key-major bf16 V (vkey) the pair kernel when the q-tiles per head are
// even (pair), else the pipelined kernel; for fp8 K/V the same choice (the
// framed kernel shares the pipelined kernel's occupancy); else the staged
// kernel (its masked instance for a key mask).
inline Slots flash_slots(int64_t D, bool vkey, bool fp8, bool mask, bool pair) {
  Slots s;
  if (D == 128)
    s = vkey && pair ? resident_slots<flash_fwd_pair_kernel<128, false>>(512)
        : vkey       ? resident_slots<flash_fwd_pipe_kernel<128, false>>()
        : fp8 && pair ? resident_slots<flash_fwd_pair_kernel<128, true>>(512)
        : fp8        ? resident_slots<flash_fwd_pipe_kernel<128, true>>()
        : mask       ? resident_slots<flash_fwd_kernel<128, false, true>>()
                     : resident_slots<flash_fwd_kernel<128, false, false>>();
  else
    s = vkey && pair ? resident_slots<flash_fwd_pair_kernel<64, false>>(512)
        : vkey       ? resident_slots<flash_fwd_pipe_kernel<64, false>>()
        : fp8 && pair ? resident_slots<flash_fwd_pair_kernel<64, true>>(512)
        : fp8        ? resident_slots<flash_fwd_pipe_kernel<64, true>>()
        : mask       ? resident_slots<flash_fwd_kernel<64, false, true>>()
                     : resident_slots<flash_fwd_kernel<64, false, false>>();
  // pieces: one per CU for the pipelined kernels (and the pair kernel, one
  // workgroup per CU), one per slot for the staged kernel (plan_split)
  if (!vkey && !fp8) s.pieces = s.slots;
  return s;
}

// fp8 K/V in frames of whole 64-key tiles with an odd number (>= 3) of
// q-tiles per head runs as two launches: the first n_qtiles - 1 q-tiles of
// every head as pair workgroups (each thread stages half of a K/V tile that
// two q-tiles share), then the last q-tile of every head on the 4-wave
// kernel, cut into key ranges so that its workgroups fill every slot (they
// start on an empty GPU, so two per CU beat one), merged by the combine
// kernel.  At 1152 queries over 4608 keys (B = 2, 32 heads) that is 256 pair
// units in one round and 64 q-tiles in 8 ranges of 9 key tiles.  SplitPlan
// holds both launches' split plans and their partial buffers' offsets.
struct SplitPlan {
  int64_t n_full[2];
  int split[2];
  int64_t off[2], bytes[2];
  int64_t total;
};

inline SplitPlan plan_fp8_split_launch(int64_t B, int64_t H, int64_t nqt, int ntiles, int64_t D) {
  SplitPlan sp{};
  // launch 0: pair units over the first nqt - 1 q-tiles of every head
  const int64_t nu0 = B * H * (nqt - 1) / 2;
  plan_split(nu0, ntiles, flash_slots(D, false, true, false, true), &sp.n_full[0], &sp.split[0]);
  sp.bytes[0] = sp.split[0] > 1 ? workspace_bytes_for((nu0 - sp.n_full[0]) * 2, sp.split[0], D) : 0;
  // launch 1: the last q-tile of every head, one piece per slot
  const int64_t nu1 = B * H;
  const Slots s1 = flash_slots(D, false, true, false, false);
  sp.n_full[1] = nu1;
  sp.split[1] = 1;
  if (s1.slots > 0 && nu1 < s1.slots) {
    int k = (int)(s1.slots / nu1);
    k = k > kMaxSplit ? kMaxSplit : k;
    k = k > ntiles / 2 ? ntiles / 2 : k;   // pieces of >= 2 key tiles
    if (k >= 2) {
      sp.n_full[1] = 0;
      sp.split[1] = k;
    }
  }
  sp.bytes[1] = sp.split[1] > 1 ? workspace_bytes_for(nu1 - sp.n_full[1], sp.split[1], D) : 0;
  sp.off[0] = 0;
  sp.off[1] = round256(sp.bytes[0]);
  sp.total = sp.off[1] + sp.bytes[1];
  return sp;
}

extern "C" int ltx_flash_attn_workspace_size(int64_t B, int64_t Lq, int64_t H, int64_t D,
                                             int64_t* bytes) {
  clear_error();
  LTX_REQUIRE(bytes != nullptr && B >= 1 && H >= 1 && Lq >= 0 && (D == 64 || D == 128),
              "ltx_flash_attn_workspace_size: bad arguments");
  // the largest partial buffer any of the kernels for this D may plan (the
  // pair kernel plans over units of two q-tiles)
  const int64_t nqt = (Lq + kBM - 1) / kBM;
  const int64_t nq = B * H * nqt;
  const bool pair = nqt % 2 == 0;
  int64_t need = 0;
  // kernels: staged, pipelined (key-major V), fp8 pipelined (framed or
  // not), fp8 pair (frames of whole tiles), masked staged
  for (int k = 0; k < 5; ++k) {
    const bool vk = k == 1, f8 = k == 2 || k == 3, mk = k == 4;
    const bool kp = (k == 1 || k == 3) && pair;
    const int64_t nu = kp ? nq / 2 : nq;
    int64_t n_full;
    int split;
    // with an unbounded key count the planned split is the largest any call of this shape plans
    plan_split(nu, 1 << 30, flash_slots(D, vk, f8, mk, kp), &n_full, &split);
    const int64_t b = split > 1 ? workspace_bytes_for((nu - n_full) * (kp ? 2 : 1), split, D) : 0;
    need = b > need ? b : need;
  }
  // the two-launch fp8 plan for an odd q-tile count
  if (nqt >= 3 && nqt % 2 == 1) {
    const int64_t b = plan_fp8_split_launch(B, H, nqt, 1 << 30, D).total;
    need = b > need ? b : need;
  }
  *bytes = need;
  return LTX_OK;
}

// The body of both attention entry points.  `strict_ws`: a planned split
// whose partials do not fit the workspace is an error (the no-allocation
// entry point, whose workspace is the fixed scratch array) instead of a
// fallback to whole q-tiles.
static int flash_attn_fwd_impl(const void* q, int64_t B, int64_t Lq, int64_t H, int64_t D,
                               int64_t q_bs, int64_t q_ls, int64_t q_hs, int64_t n_segments,
                               const void* const* k_ptrs, const void* const* v_ptrs,
                               const int64_t* seg_lens, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                               int64_t v_bs, int64_t v_ls, int64_t v_hs, int64_t v_ds, int kv_dtype,
                               const float* const* k_scales, const float* const* v_scales,
                               int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                               const float* key_mask, int64_t mask_bs, const int64_t* key_lens, void* out,
                               int64_t o_bs, int64_t o_ls, int64_t o_hs, float* lse, float scale,
                               void* workspace, int64_t workspace_bytes, bool strict_ws, void* stream) {
  LTX_REQUIRE(q && out, "ltx_flash_attn_fwd: null q/out");
  LTX_REQUIRE(D == 64 || D == 128, "ltx_flash_attn_fwd: head dim %lld unsupported (64 or 128)",
              (long long)D);
  LTX_REQUIRE(B >= 1 && H >= 1 && Lq >= 0 && Lq <= 0x7FFFFFFF, "ltx_flash_attn_fwd: bad B/H/Lq");
  LTX_REQUIRE(n_segments >= 0 && n_segments <= LTX_MAX_SEGMENTS,
              "ltx_flash_attn_fwd: n_segments must be in [0, %d]", LTX_MAX_SEGMENTS);
  LTX_REQUIRE(kv_dtype == LTX_BF16 || kv_dtype == LTX_F8E4M3, "ltx_flash_attn_fwd: kv_dtype must be BF16 or F8E4M3");
  LTX_REQUIRE(n_segments == 0 || (k_ptrs && v_ptrs && seg_lens), "ltx_flash_attn_fwd: null segment arrays");
  const bool fp8 = kv_dtype == LTX_F8E4M3;
  const bool vkey = v_ds != 1;  // key-major V
  LTX_REQUIRE(!vkey || v_ls == 1, "ltx_flash_attn_fwd: V must be token-major (v_ds == 1) or key-major (v_ls == 1)");
  LTX_REQUIRE(!vkey || (!fp8 && key_mask == nullptr),
              "ltx_flash_attn_fwd: key-major V is bf16 without a key mask");
  const int64_t esz = fp8 ? 1 : 2;
  auto al = [](const void* ptr, uintptr_t a) { return ((uintptr_t)ptr % a) == 0; };
  LTX_REQUIRE(al(q, 16) && (q_bs * 2) % 16 == 0 && (q_ls * 2) % 16 == 0 && (q_hs * 2) % 16 == 0,
              "ltx_flash_attn_fwd: q rows must be 16-byte aligned");
  LTX_REQUIRE(al(out, 8) && (o_bs * 2) % 8 == 0 && (o_ls * 2) % 8 == 0 && (o_hs * 2) % 8 == 0,
              "ltx_flash_attn_fwd: out rows must be 8-byte aligned");
  LTX_REQUIRE((k_bs * esz) % 16 == 0 && (k_ls * esz) % 16 == 0 && (k_hs * esz) % 16 == 0,
              "ltx_flash_attn_fwd: K strides must keep 16-byte rows");
  if (vkey)
    LTX_REQUIRE((v_bs * 2) % 16 == 0 && (v_hs * 2) % 16 == 0 && (v_ds * 2) % 16 == 0 &&
                    v_ds * D * 2 < ((int64_t)1 << 31),
                "ltx_flash_attn_fwd: key-major V strides must keep 16-byte rows");
  else
    LTX_REQUIRE(v_bs == k_bs && v_ls == k_ls && v_hs == k_hs,
                "ltx_flash_attn_fwd: token-major V must share K's strides");

  FlashParams p{};
  p.q = (const uint16_t*)q;
  p.o = (uint16_t*)out;
  p.lse = lse;
  p.mask = key_mask;
  p.q_bs = q_bs; p.q_ls = q_ls; p.q_hs = q_hs;
  p.o_bs = o_bs; p.o_ls = o_ls; p.o_hs = o_hs;
  p.o_al16 = ((uintptr_t)out % 16 == 0 && o_bs % 8 == 0 && o_ls % 8 == 0 && o_hs % 8 == 0) ? 1 : 0;
  p.kv_bs = k_bs; p.kv_ls = k_ls; p.kv_hs = k_hs;
  p.v_bs = v_bs; p.v_hs = v_hs; p.v_ds = v_ds;
  p.sc_bs = sc_bs; p.sc_hs = sc_hs;
  p.mask_bs = mask_bs;
  p.B = (int)B; p.H = (int)H; p.Lq = (int)Lq;
  p.frame = (int)(frame_tokens > 0 ? frame_tokens : 1);
  p.scale = scale > 0.0f ? scale : 1.0f / sqrtf((float)D);
  p.scale_log2 = p.scale * kLog2e;
  // drop empty segments
  int n = 0;
  p.seg_start[0] = 0;
  p.tile_start[0] = 0;
  for (int64_t i = 0; i < n_segments; ++i) {
    LTX_REQUIRE(seg_lens[i] >= 0, "ltx_flash_attn_fwd: negative segment length");
    if (seg_lens[i] == 0) continue;
    LTX_REQUIRE(k_ptrs[i] && v_ptrs[i], "ltx_flash_attn_fwd: null segment %lld", (long long)i);
    LTX_REQUIRE(al(k_ptrs[i], 16) && al(v_ptrs[i], 16), "ltx_flash_attn_fwd: segment %lld not 16-byte aligned",
                (long long)i);
    if (fp8) {
      LTX_REQUIRE(k_scales && v_scales && k_scales[i] && v_scales[i],
                  "ltx_flash_attn_fwd: fp8 segment %lld needs k/v scales", (long long)i);
      LTX_REQUIRE(frame_tokens > 0 && frame_tokens <= 0x7FFFFFFF,
                  "ltx_flash_attn_fwd: fp8 needs frame_tokens > 0 (got %lld)", (long long)frame_tokens);
      p.k_sc[n] = k_scales[i];
      p.v_sc[n] = v_scales[i];
    }
    p.k_ptr[n] = k_ptrs[i];
    p.v_ptr[n] = v_ptrs[i];
    p.seg_start[n + 1] = p.seg_start[n] + seg_lens[i];
    // fp8: tiles never cross a frame (ceil(F / 64) per frame, the segment's
    // last frame possibly partial); bf16: ceil(len / 64)
    const int64_t seg_tiles =
        fp8 ? (seg_lens[i] / frame_tokens) * ((frame_tokens + kBN - 1) / kBN) +
                  (seg_lens[i] % frame_tokens + kBN - 1) / kBN
            : (seg_lens[i] + kBN - 1) / kBN;
    const int64_t tiles = p.tile_start[n] + seg_tiles;
    LTX_REQUIRE(tiles <= 0x7FFFFFFF, "ltx_flash_attn_fwd: too many keys");
    p.tile_start[n + 1] = (int)tiles;
    ++n;
  }
  p.n_seg = n;
  p.Lk = p.seg_start[n];
  if (key_mask) LTX_REQUIRE(!fp8, "ltx_flash_attn_fwd: key mask with fp8 KV is not built");
  if (key_lens) {
    LTX_REQUIRE(vkey && !fp8 && key_mask == nullptr,
                "ltx_flash_attn_fwd: key_lens needs bf16 key-major V and no key mask");
    LTX_REQUIRE(B <= LTX_MAX_KEYLEN_BATCH, "ltx_flash_attn_fwd: key_lens supports at most %d batch rows",
                LTX_MAX_KEYLEN_BATCH);
    for (int64_t b = 0; b < B; ++b) {
      LTX_REQUIRE(key_lens[b] >= 0 && key_lens[b] <= p.Lk,
                  "ltx_flash_attn_fwd: key_lens[%lld] = %lld outside [0, %lld]", (long long)b,
                  (long long)key_lens[b], (long long)p.Lk);
      p.klen[b] = (int)key_lens[b];
    }
    p.n_klen = (int)B;
  }
  LTX_REQUIRE(k_ls * esz * kBN < (int64_t)1 << 31 && k_ls >= D,
              "ltx_flash_attn_fwd: kv token stride %lld out of range", (long long)k_ls);
  p.n_qtiles = (int)((Lq + kBM - 1) / kBM);
  if (Lq == 0) return LTX_OK;
  LTX_REQUIRE(n > 0, "ltx_flash_attn_fwd: no keys (Lk == 0)");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // fp8 K/V, frames of whole tiles, an odd q-tile count >= 3: two launches
  // (plan_fp8_split_launch), each over its own rows of q and out (q and out
  // offset, Lq cut), so only without lse, whose rows are Lq apart.  A plan
  // whose partials do not fit the workspace takes the one-launch path below.
  if (fp8 && frame_tokens % kBN == 0 && p.n_qtiles >= 3 && p.n_qtiles % 2 == 1 && lse == nullptr &&
      workspace != nullptr) {
    const SplitPlan sp = plan_fp8_split_launch(B, H, p.n_qtiles, p.tile_start[n], D);
    if (sp.total <= workspace_bytes) {
      LTX_REQUIRE(al(workspace, 256), "ltx_flash_attn_fwd: workspace must be 256-byte aligned");
      const int64_t lq0 = (int64_t)(p.n_qtiles - 1) * kBM;
      FlashParams lp[2] = {p, p};
      lp[0].Lq = (int)lq0;
      lp[0].n_qtiles = p.n_qtiles - 1;
      lp[0].pair = 1;
      lp[1].q = p.q + lq0 * q_ls;
      lp[1].o = p.o + lq0 * o_ls;
      lp[1].o_al16 = ((uintptr_t)lp[1].o % 16 == 0 && o_bs % 8 == 0 && o_ls % 8 == 0 && o_hs % 8 == 0) ? 1 : 0;
      lp[1].Lq = (int)(Lq - lq0);
      lp[1].n_qtiles = 1;
      lp[1].pair = 0;
      for (int i = 0; i < 2; ++i) {
        lp[i].n_full = (int)sp.n_full[i];
        lp[i].split = sp.split[i];
        if (sp.split[i] > 1) {
          const int64_t tail = (i == 0 ? 2 * ((int64_t)B * H * lp[0].n_qtiles / 2 - sp.n_full[0])
                                       : (int64_t)B * H - sp.n_full[1]);
          lp[i].part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + sp.off[i]);
          lp[i].part_o = reinterpret_cast<uint16_t*>(lp[i].part_ml + tail * sp.split[i] * kBM * 2);
        }
        const int rc = D == 128 ? launch_flash_pipe<128, true>(lp[i], st) : launch_flash_pipe<64, true>(lp[i], st);
        if (rc != LTX_OK) return rc;
      }
      return LTX_OK;
    }
  }
  // balanced tail (needs a workspace; without one every q-tile runs whole).
  // Key-major bf16 V, or fp8 K/V in frames of whole 64-key tiles, with an
  // even number of q-tiles per head runs the pair kernel, whose grid counts
  // units of two q-tiles (two partial results per split unit).
  {
    const int64_t nq = (int64_t)B * H * p.n_qtiles;
    LTX_REQUIRE(nq <= 0x7FFFFFFF, "ltx_flash_attn_fwd: grid too large");
    p.pair = (vkey || (fp8 && frame_tokens % kBN == 0)) && p.n_qtiles % 2 == 0 ? 1 : 0;
    const int64_t nu = p.pair ? nq / 2 : nq;
    const int per_unit = p.pair ? 2 : 1;
    int64_t n_full = nu;
    int split = 1;
    if (workspace != nullptr) {
      plan_split(nu, p.tile_start[n], flash_slots(D, vkey, fp8, key_mask != nullptr, p.pair != 0), &n_full,
                 &split);
      if (split > 1 && workspace_bytes_for((nu - n_full) * per_unit, split, D) > workspace_bytes) {
        LTX_REQUIRE(!strict_ws,
                    "ltx_flash_attn_fwd_noalloc: this call's split partials need %lld bytes, more than the "
                    "%lld-byte scratch array",
                    (long long)workspace_bytes_for((nu - n_full) * per_unit, split, D), (long long)workspace_bytes);
        n_full = nu;
        split = 1;
      }
    }
    p.n_full = (int)n_full;
    p.split = split;
    if (split > 1) {
      LTX_REQUIRE(al(workspace, 256), "ltx_flash_attn_fwd: workspace must be 256-byte aligned");
      const int64_t tail = (nu - n_full) * per_unit;
      p.part_ml = static_cast<float*>(workspace);
      p.part_o = reinterpret_cast<uint16_t*>(p.part_ml + tail * split * kBM * 2);
    }
  }
  if (vkey) {
    if (D == 128) return launch_flash_pipe<128, false>(p, st);
    return launch_flash_pipe<64, false>(p, st);
  }
  if (fp8) {
    // the framed instances share the plain ones' occupancy (same registers
    // and LDS), so the split plan above holds for them too
    if (frame_tokens % kBN != 0) {
      if (D == 128) return launch_flash_pipe<128, true, true>(p, st);
      return launch_flash_pipe<64, true, true>(p, st);
    }
    if (D == 128) return launch_flash_pipe<128, true>(p, st);
    return launch_flash_pipe<64, true>(p, st);
  }
  if (D == 128) {
    if (key_mask) return launch_flash<128, false, true>(p, st);
    return launch_flash<128, false, false>(p, st);
  } else {
    if (key_mask) return launch_flash<64, false, true>(p, st);
    return launch_flash<64, false, false>(p, st);
  }
}

extern "C" int ltx_flash_attn_fwd(const void* q, int64_t B, int64_t Lq, int64_t H, int64_t D,
                                  int64_t q_bs, int64_t q_ls, int64_t q_hs, int64_t n_segments,
                                  const void* const* k_ptrs, const void* const* v_ptrs,
                                  const int64_t* seg_lens, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                                  int64_t v_bs, int64_t v_ls, int64_t v_hs, int64_t v_ds, int kv_dtype,
                                  const float* const* k_scales, const float* const* v_scales,
                                  int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                                  const float* key_mask, int64_t mask_bs, const int64_t* key_lens, void* out,
                                  int64_t o_bs, int64_t o_ls, int64_t o_hs, float* lse, float scale,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  return flash_attn_fwd_impl(q, B, Lq, H, D, q_bs, q_ls, q_hs, n_segments, k_ptrs, v_ptrs, seg_lens, k_bs,
                             k_ls, k_hs, v_bs, v_ls, v_hs, v_ds, kv_dtype, k_scales, v_scales, sc_bs, sc_hs,
                             frame_tokens, key_mask, mask_bs, key_lens, out, o_bs, o_ls, o_hs, lse, scale,
                             workspace, workspace_bytes, false, stream);
}

// ---------------------------------------------------------------------------
// No-allocation variant: the split partials live in a fixed device array.
//
// `scratch` holds the partial results of the split tail q-tiles (per piece:
// 128 rows of (max, sum) in float32 and an O row in bf16).  The partial
// results are at most two per CU (pieces <= resident slots, two 4-wave
// workgroups per CU; the pair kernel's units hold two q-tiles at one
// workgroup per CU), so a launch needs at most 2 CUs x 128 x (8 + 2 D) bytes:
// 17.3 MB for D = 128 at 256 CUs (the fp8 two-launch plan keeps both
// launches' partials in the array and is taken only when they fit).  Every piece writes its whole partial before the
// combine kernel reads it, so nothing needs clearing between calls.  Each
// device holds its own copy of the array for the life of the process; its
// device address is looked up once per device (hipGetSymbolAddress) and
// only that address is handed to kernels.  Calls that overlap in time on one
// device share the array and race.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = LTX_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch` (nullptr and an error message on failure).
static void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("ltx_flash_attn_fwd_noalloc: no current HIP device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("ltx_flash_attn_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

extern "C" int ltx_flash_attn_fwd_noalloc(const void* q, int64_t B, int64_t Lq, int64_t H, int64_t D,
                                          int64_t q_bs, int64_t q_ls, int64_t q_hs, int64_t n_segments,
                                          const void* const* k_ptrs, const void* const* v_ptrs,
                                          const int64_t* seg_lens, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                                          int64_t v_bs, int64_t v_ls, int64_t v_hs, int64_t v_ds,
                                          int kv_dtype, const float* const* k_scales,
                                          const float* const* v_scales, int64_t sc_bs, int64_t sc_hs,
                                          int64_t frame_tokens, const float* key_mask, int64_t mask_bs,
                                          const int64_t* key_lens, void* out, int64_t o_bs, int64_t o_ls,
                                          int64_t o_hs, float* lse, float scale, void* stream) {
  clear_error();
  void* ws = scratch_for_current_device();
  if (ws == nullptr) return LTX_ELAUNCH;
  return flash_attn_fwd_impl(q, B, Lq, H, D, q_bs, q_ls, q_hs, n_segments, k_ptrs, v_ptrs, seg_lens, k_bs,
                             k_ls, k_hs, v_bs, v_ls, v_hs, v_ds, kv_dtype, k_scales, v_scales, sc_bs, sc_hs,
                             frame_tokens, key_mask, mask_bs, key_lens, out, o_bs, o_ls, o_hs, lse, scale, ws,
                             kScratchBytes, true, stream);
}
