/*
 * taomate_ltx.h -- C ABI of the MI355X (gfx950) chunked causal LTX attention path.
 *
 * The reference (TaoMate `ltx_causal`) is pure PyTorch: its hot path is
 * `attention_with_cache` (ltx_causal/transformer/kv_cache.py:1148-1547), which runs
 * q/k RMSNorm -> SPLIT RoPE -> torch.cat(cache, new) -> SDPA.  Each entry point
 * below replaces one of the PyTorch operations that path reaches; the reference
 * function each one stands in for is cited next to it.
 *
 * Conventions (all entry points):
 *   - plain device pointers, int64 element strides (not bytes), dtype enums;
 *   - return 0 (LTX_OK) or a negative ltx_status; never throw, never allocate
 *     device memory, never synchronise; work is enqueued on `stream`;
 *   - the message of the last failure on the calling thread is ltx_last_error();
 *   - tensors follow the reference's [B, L, H, D] layout with D contiguous;
 *   - key/value "segments": the logical key sequence is the concatenation of up
 *     to LTX_MAX_SEGMENTS device spans (anchor | memory | window... | current),
 *     which is what `torch.cat([cached_k, k], 1)` (kv_cache.py:1487-1491) builds
 *     physically in the reference; here the spans are read in place.
 */
#ifndef TAOMATE_LTX_H
#define TAOMATE_LTX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LTX_ABI_VERSION 2
#define LTX_MAX_SEGMENTS 16
#define LTX_MAX_KEYLEN_BATCH 16   /* batch rows ltx_flash_attn_fwd's key_lens covers */

typedef enum {
  LTX_F32 = 0,
  LTX_BF16 = 1,
  LTX_F8E4M3 = 2 /* OCP float8_e4m3fn (max 448, no inf) */
} ltx_dtype;

typedef enum {
  LTX_OK = 0,
  LTX_EINVAL = -1,       /* bad pointer, shape, stride or dtype */
  LTX_EUNSUPPORTED = -2, /* valid request this build has no kernel for */
  LTX_ELAUNCH = -3       /* the HIP launch itself failed */
} ltx_status;

/* ABI version this library implements (LTX_ABI_VERSION). */
int ltx_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). */
const char* ltx_last_error(void);

/*
 * RoPE cos/sin table, SPLIT layout [B, H, T, dim/(2H)].
 * Replaces causal_precompute_freqs_cis (ltx_causal/rope/causal_rope.py:139-357),
 * SPLIT branch (:323-341), for the video 3-D (F,H,W) grid (:258-288), the audio
 * 1-D grid (:295-300) and the video-time 1-D grid (:302-306).
 *   freq_idx: device float32[n_freq], the generate_freq_grid values
 *             (causal_rope.py:45-80; n_freq = dim / (2*num_pos_dims)).
 *   num_pos_dims 3: grid (grid_f, grid_h, grid_w); 1: grid_f only, is_audio picks
 *   the audio (mel) or video (pixel-frame) time conversion.
 *   max_pos_*: normalisers (reference defaults 20, 2048, 2048).
 *   out_dtype: LTX_F32 or LTX_BF16 (values computed in float32, rounded once).
 *   The B batch rows are identical copies (the reference builds one per batch).
 */
int ltx_rope_table(void* cos_out, void* sin_out, int out_dtype, const float* freq_idx,
                   int64_t n_freq, int num_pos_dims, int64_t grid_f, int64_t grid_h,
                   int64_t grid_w, int64_t start_frame, int is_audio, float max_pos_t,
                   float max_pos_h, float max_pos_w, int64_t dim, int64_t num_heads,
                   int64_t batch, void* stream);

/*
 * The SPLIT video (3-D) table of ltx_rope_table for a new start frame, from a
 * table of the same grid, dim, heads and frequencies built for any other start
 * frame (also causal_precompute_freqs_cis, causal_rope.py:139-357: the same
 * values, built another way).  Only the t-axis entries depend on the start
 * frame (causal_rope.py:264-267, 284-288); the h, w and pad entries are read
 * from the source table.  Every entry is bit-identical to ltx_rope_table's.
 *   cos_out/sin_out, cos_src/sin_src: [1, H, T, dim/(2H)], T = grid_f *
 *   grid_h * grid_w, 16-byte aligned, dim/(2H) entries a multiple of 16 bytes;
 *   the source and output must not overlap.
 *   max_pos_t: the time normaliser (reference default 20).
 */
int ltx_rope_table_retime(void* cos_out, void* sin_out, const void* cos_src, const void* sin_src,
                          int out_dtype, const float* freq_idx, int64_t n_freq, int64_t grid_f,
                          int64_t grid_h, int64_t grid_w, int64_t start_frame, float max_pos_t,
                          int64_t dim, int64_t num_heads, void* stream);

/*
 * Fused full-row RMSNorm + SPLIT RoPE on q and k rows.
 * Replaces, in order: q_norm/k_norm = nn.RMSNorm(H*D, eps)
 * (ltx_causal/attention/causal_attention.py:105-106, applied at
 * kv_cache.py:1406-1407) and apply_split_rotary_emb (causal_rope.py:102-132,
 * called through CausalLTXAttention._apply_rope, causal_attention.py:326-338,
 * at kv_cache.py:1415-1417).
 *   x rows: [B, L, H*D] with (b_stride, l_stride) in elements, H*D contiguous.
 *   The k output may point into a KV arena (that is the "append" of new keys).
 *   gamma_*: [H*D] in `dtype`, or NULL for gamma = 1.
 *   eps_* < 0 skips the norm (RoPE only); cos_* == NULL skips RoPE (norm only).
 *   Tables: [Bt, H, T, D/2] in tab_dtype with strides (tb, th, tt) in elements;
 *   tb may be 0 to broadcast one table row over the batch.
 *   Rounding (bf16): (x * rsqrt(mean x^2 + eps)) * gamma in float32 -> round
 *   (PyTorch's fused rms_norm); then x1*c -> round -> +/-(s*x2) in float32 ->
 *   round (the mul / addcmul_ pair of causal_rope.py:121-126).
 *   k_in == NULL processes q only.
 */
int ltx_qk_rmsnorm_rope(int dtype, int64_t B, int64_t H, int64_t D,
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
                        int tab_dtype, void* stream);

/*
 * ltx_qk_rmsnorm_rope and the key-major bf16 append of the chunk's V in one
 * launch: the q/k rows as above (dtype LTX_BF16, D 64 or 128) and
 * v_src [B, v_len, H, D] bf16 (strides v_bs, v_ls, v_hs; D contiguous; rows
 * 16-byte aligned) transposed into v_dst, element (b, t, h, d) at
 * v_dst + b*vd_bs + h*vd_hs + d*vd_ds + t (the arena's V layout, as
 * ltx_kv_append with d_ls == 1).  Replaces, in one pass over HBM, the q/k
 * norm + RoPE (kv_cache.py:1406-1417) and the V half of the cache append
 * (_cat_cache, kv_cache.py:394-398) of attention_with_cache.
 */
int ltx_qk_rmsnorm_rope_v(int dtype, int64_t B, int64_t H, int64_t D,
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
                          void* v_dst, int64_t vd_bs, int64_t vd_hs, int64_t vd_ds, void* stream);

/*
 * KV append into a preallocated arena (copy, transpose or fp8 quantise).
 * Replaces _cat_cache / torch.cat (ltx_causal/transformer/kv_cache.py:394-398,
 * block cache update :2642-2656): the new tokens are written once into their
 * arena slots instead of reallocating the whole cache.
 *   src: [B, L, H, D] `src_dtype` (LTX_BF16 or LTX_F32), strides (bs, ls, hs),
 *   D contiguous.
 *   dst: element (b, l, h, d) at dst + b*d_bs + l*d_ls + h*d_hs + d*d_ds.
 *     d_ds == 1: token-major; dst_dtype LTX_BF16 copies, LTX_F8E4M3 quantises
 *       with one scale per (b, h, frame) of `frame_tokens` tokens:
 *       scale = absmax / 448 (1 if absmax == 0), q = rne_sat(x / scale).
 *     d_ls == 1: key-major (the arena's V layout, [B, H, D, slots]); LTX_BF16
 *       only: the tokens are transposed on the way in.
 *   scales: float32 [B, H, n_frames] with strides (sbs, shs), frame index f
 *   at scales[b*sbs + h*shs + f]; only used for LTX_F8E4M3. L must be a
 *   multiple of frame_tokens for LTX_F8E4M3.
 */
int ltx_kv_append(int src_dtype, int dst_dtype, int64_t B, int64_t L, int64_t H,
                  int64_t D, const void* src, int64_t s_bs, int64_t s_ls, int64_t s_hs,
                  void* dst, int64_t d_bs, int64_t d_ls, int64_t d_hs, int64_t d_ds,
                  float* scales, int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                  void* stream);

/*
 * fp8 append of a chunk's K and V in one launch.
 * Replaces the two _cat_cache appends of one commit (ltx_causal/transformer/
 * kv_cache.py:394-398, :2642-2656) for an fp8 arena (the reference has no fp8
 * cache: an extension of this library).  Same quantisation as ltx_kv_append
 * with dst_dtype LTX_F8E4M3 (bit-identical codes and scales), for bf16
 * sources:
 *   k_src / v_src: bf16 [B, L, H, D] with their own strides (D contiguous);
 *   k_dst / v_dst: uint8 codes sharing the strides (d_bs, d_ls, d_hs);
 *   k_scales / v_scales: float32 sharing the strides (sc_bs, sc_hs), frame f of
 *   (b, h) at scales[b*sc_bs + h*sc_hs + f].  L must be a multiple of
 *   frame_tokens.
 */
int ltx_kv_append_fp8_pair(int64_t B, int64_t L, int64_t H, int64_t D, int64_t frame_tokens,
                           const void* k_src, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                           void* k_dst, float* k_scales, const void* v_src, int64_t v_bs,
                           int64_t v_ls, int64_t v_hs, void* v_dst, float* v_scales,
                           int64_t d_bs, int64_t d_ls, int64_t d_hs, int64_t sc_bs,
                           int64_t sc_hs, void* stream);

/*
 * Span gather (cache compaction).
 * Replaces _slice_tensor/_slice_cache (taomate/inference/cache.py:28-56) and
 * _slice_kv_tensor (taomate/inference/streaming_runtime.py:431-442) when a
 * physically contiguous copy is wanted (eviction itself is index-only).
 *   Copies n_spans token ranges src[:, starts[i]:starts[i]+lens[i]] back to back
 *   into dst[:, 0:sum(lens)].  starts/lens are host arrays.  src and dst must
 *   not overlap.  elem_bytes: 1 (fp8), 2 (bf16) or 4 (f32); D*elem_bytes must
 *   be a multiple of 4.
 */
int ltx_kv_gather(int64_t elem_bytes, int64_t B, int64_t H, int64_t D, const void* src,
                  int64_t s_bs, int64_t s_ls, int64_t s_hs, void* dst, int64_t d_bs,
                  int64_t d_ls, int64_t d_hs, int64_t n_spans, const int64_t* starts,
                  const int64_t* lens, void* stream);

/*
 * Flash attention forward over segmented keys.
 * Replaces standard_attention_forward -> F.scaled_dot_product_attention
 * (ltx_causal/attention/flex_attention_utils.py:225-276, called at
 * kv_cache.py:1531): out = softmax(q k^T * scale + mask) v over the keys of all
 * segments in order; no causal mask (causality is what the segments contain).
 *   q, out: [B, Lq, H, D] bf16, strides (bs, ls, hs).  D in {64, 128}.
 *   Segment i: k_ptrs[i], v_ptrs[i] point at its first token (b=0, h=0, d=0);
 *   seg_lens[i] tokens.  K element (b, t, h, d) at k + b*k_bs + t*k_ls + h*k_hs
 *   + d; V element at v + b*v_bs + t*v_ls + h*v_hs + d*v_ds, either token-major
 *   (v_ds == 1) or key-major (v_ls == 1, bf16 only).  All segments share the
 *   strides.  Key-major V is read in 8-token (16-byte) chunks: a segment's
 *   start must be 16-byte aligned and its values may be read up to the next
 *   multiple of 8 tokens past its end; those extra values must be finite (they
 *   get weight 0).  The KV arena guarantees both.
 *   kv_dtype LTX_BF16, or LTX_F8E4M3 (token-major) with per-(b, h, frame)
 *   float32 scales: k_scales[i], v_scales[i] for segment i, index b*sc_bs +
 *   h*sc_hs + (t/frame) where t counts tokens from the segment start (a
 *   segment starts on a frame boundary; any frame_tokens >= 1, a frame that
 *   is not a multiple of 64 tokens being cut into 64-key tiles at its
 *   boundaries).
 *   key_mask: NULL or float32 additive mask [B, Lk_total] with batch stride
 *   mask_bs (the reference's `(m - 1) * finfo.max` padding mask,
 *   ltx_causal/transformer/causal_model.py:551-562); token-major V only.
 *   key_lens: NULL, or a host array of B key counts (B <= LTX_MAX_KEYLEN_BATCH):
 *   batch row b attends keys [0, key_lens[b]) of the concatenated sequence
 *   only, each count in [0, Lk_total].  This is that padding mask when every
 *   row keeps a prefix of its keys (the masked keys' weights are exactly 0 in
 *   float32), run on the pipelined kernel; bf16 key-major V, no key_mask.  A
 *   row with no keys gets a zero output.
 *   lse: NULL or float32 [B, H, Lq] natural-log sum-exp of the scaled logits.
 *   scale <= 0 selects 1/sqrt(D) (SDPA's default).
 *   workspace: NULL, or workspace_bytes >= ltx_flash_attn_workspace_size() of
 *   device memory, 256-byte aligned.  With it the q-tiles that do not fill a
 *   whole round of the device's resident workgroups are split along the keys
 *   and recombined by a second kernel on `stream`, so the grid ends together;
 *   without it they run whole.  Calls that overlap in time must use different
 *   workspaces.
 *   Host arrays (k_ptrs, v_ptrs, seg_lens, scales, key_lens) are read during the call only.
 */
int ltx_flash_attn_fwd(const void* q, int64_t B, int64_t Lq, int64_t H, int64_t D,
                       int64_t q_bs, int64_t q_ls, int64_t q_hs, int64_t n_segments,
                       const void* const* k_ptrs, const void* const* v_ptrs,
                       const int64_t* seg_lens, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                       int64_t v_bs, int64_t v_ls, int64_t v_hs, int64_t v_ds, int kv_dtype,
                       const float* const* k_scales, const float* const* v_scales,
                       int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                       const float* key_mask, int64_t mask_bs, const int64_t* key_lens, void* out,
                       int64_t o_bs, int64_t o_ls, int64_t o_hs, float* lse, float scale, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * ltx_flash_attn_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 *   Same arguments, semantics and results as ltx_flash_attn_fwd with a
 *   sufficient workspace; the split partials go to a fixed device array of
 *   LTX_NOALLOC_SCRATCH_BYTES inside the library (one per device, kept until
 *   the process ends).  Allocates nothing: no hipMalloc / hipFree, no
 *   allocating library call.  A call whose split would need more scratch
 *   than that returns LTX_EINVAL with a message (at most two partial
 *   results per CU, 512 x 128 rows x (8 + 2 D) bytes, are ever planned on
 *   MI355X: 17.3 MB for D = 128).  Calls that overlap in time on one device share the
 *   array and race: serialise them (one stream, or events).
 */
#define LTX_NOALLOC_SCRATCH_BYTES (24ll << 20)
int ltx_flash_attn_fwd_noalloc(const void* q, int64_t B, int64_t Lq, int64_t H, int64_t D,
                               int64_t q_bs, int64_t q_ls, int64_t q_hs, int64_t n_segments,
                               const void* const* k_ptrs, const void* const* v_ptrs,
                               const int64_t* seg_lens, int64_t k_bs, int64_t k_ls, int64_t k_hs,
                               int64_t v_bs, int64_t v_ls, int64_t v_hs, int64_t v_ds, int kv_dtype,
                               const float* const* k_scales, const float* const* v_scales,
                               int64_t sc_bs, int64_t sc_hs, int64_t frame_tokens,
                               const float* key_mask, int64_t mask_bs, const int64_t* key_lens, void* out,
                               int64_t o_bs, int64_t o_ls, int64_t o_hs, float* lse, float scale, void* stream);

/*
 * Workspace bytes ltx_flash_attn_fwd can use for a [B, Lq, H, D] query on the
 * current device (0: no split is ever planned for this shape).
 * No counterpart in the reference (its SDPA call has no workspace).
 */
int ltx_flash_attn_workspace_size(int64_t B, int64_t Lq, int64_t H, int64_t D, int64_t* bytes);

/*
 * Gated residual update and AdaLN-modulated RMSNorm, bf16 [B, L, C] rows.
 * Replaces the bf16 tensor-op chains of block_forward_with_cache
 * (ltx_causal/transformer/kv_cache.py:2194-2633) around each attention and
 * feed-forward: x' = x + y * gate (x + y without a gate; x when y is null),
 * then n = rms_norm(x') * (1 + scale) + shift (rms_norm of
 * ltx_causal/transformer/causal_block.py:94-101; plain rms_norm(x') without
 * scale/shift), rounding to bf16 where the reference's tensor ops do.
 *   Every tensor is given by a pointer and (batch, row) element strides with
 *   the C channels contiguous; gate/scale/shift rows are per batch element
 *   (row stride 0) or per row.  x_out (may equal x) receives x' when y is
 *   given; n_out (may be null) receives n.  C must be a multiple of 8, at
 *   most 8192; rows 16-byte aligned.
 */
int ltx_adaln(int64_t B, int64_t L, int64_t C, const void* x, int64_t x_bs, int64_t x_ls,
              const void* y, int64_t y_bs, int64_t y_ls, const void* gate, int64_t g_bs, int64_t g_ls,
              void* x_out, int64_t xo_bs, int64_t xo_ls, void* n_out, int64_t n_bs, int64_t n_ls,
              const void* scale, int64_t s_bs, int64_t s_ls, const void* shift, int64_t h_bs,
              int64_t h_ls, float eps, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TAOMATE_LTX_H */
