"""fp32 restatement of the dual-stream block step (oracle; test
infrastructure only).

Follows, op for op:
  timestep embedding, AdaLayerNormSingle   ltx_causal/transformer/compat.py:76-275
  _prepare_timestep / cross timestep       ltx_causal/transformer/causal_model.py:426-496
  get_ada_values / get_av_ca_ada_values    ltx_causal/transformer/causal_block.py:434-481
  block_forward_with_cache (sync branch)   ltx_causal/transformer/kv_cache.py:2145-2656
  text cross-attention                     kv_cache.py:1090-1141 (without prompt AdaLN,
                                           and the LTX-2.3 prompt AdaLN when the
                                           blocks hold prompt_scale_shift_table;
                                           prompt timestep kv_cache.py:2876-2895)
  _process_output                          causal_model.py:568-599
  learned-memory adapters (optional)       causal_block.py:108-193, 489-505;
                                           placement kv_cache.py:2217-2330;
                                           encoders kv_cache.py:529-559
with the attention calls of ``oracle.attention`` (attention_with_cache for
self / cross-modal attention, text_cross_attention for the text keys).
Weights are plain dicts of float32 CPU tensors keyed by the reference's
parameter names.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import attention as OA
from . import cache as OC


def rms_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """causal_block.py:94-101 (no weight)."""
    return F.rms_norm(x, (x.shape[-1],), None, eps)


def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: int = 10000) -> torch.Tensor:
    """compat.py:76-106, flip_sin_to_cos=True, downscale_freq_shift=0."""
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32) / half
    emb = t[:, None].float() * torch.exp(exponent)[None, :]
    return torch.cat([torch.cos(emb), torch.sin(emb)], dim=-1)


def adaln_single(p: Dict[str, torch.Tensor], prefix: str, t: torch.Tensor):
    """compat.py:212-275: (linear(silu(emb)), emb), emb = MLP(sinusoid(t))."""
    e = timestep_embedding(t)
    e = F.linear(e, p[prefix + "emb.timestep_embedder.linear_1.weight"],
                 p[prefix + "emb.timestep_embedder.linear_1.bias"])
    e = F.linear(F.silu(e), p[prefix + "emb.timestep_embedder.linear_2.weight"],
                 p[prefix + "emb.timestep_embedder.linear_2.bias"])
    return F.linear(F.silu(e), p[prefix + "linear.weight"], p[prefix + "linear.bias"]), e


def ada_values(table: torch.Tensor, batch: int, ts: torch.Tensor, idx: slice):
    """causal_block.py:434-452."""
    n = table.shape[0]
    return (table[idx][None, None] + ts.reshape(batch, ts.shape[1], n, -1)[:, :, idx, :]).unbind(dim=2)


def av_ca_values(table: torch.Tensor, batch: int, ss: torch.Tensor, gate: torch.Tensor):
    """causal_block.py:454-481."""
    return (*ada_values(table[:4], batch, ss, slice(None)), *ada_values(table[4:], batch, gate, slice(None)))


def attn_weights(p: Dict[str, torch.Tensor], prefix: str, heads: int, dim_head: int) -> OA.AttnWeights:
    g = lambda n: p[prefix + n]
    return OA.AttnWeights(g("to_q.weight"), g("to_q.bias"), g("to_k.weight"), g("to_k.bias"), g("to_v.weight"),
                          g("to_v.bias"), g("to_out.0.weight"), g("to_out.0.bias"), g("q_norm.weight"),
                          g("k_norm.weight"), heads, dim_head)


def feed_forward(p: Dict[str, torch.Tensor], prefix: str, x: torch.Tensor) -> torch.Tensor:
    """compat.py:46-71: Linear -> tanh-GELU -> Linear."""
    h = F.gelu(F.linear(x, p[prefix + "net.0.proj.weight"], p[prefix + "net.0.proj.bias"]), approximate="tanh")
    return F.linear(h, p[prefix + "net.2.weight"], p[prefix + "net.2.bias"])


def memory_attention(p: Dict[str, torch.Tensor], prefix: str, x: torch.Tensor, memory: torch.Tensor,
                     heads: int) -> torch.Tensor:
    """LearnedMemoryAttention.forward (causal_block.py:136-160): q from x,
    k / v from the memory tokens, SDPA with scale 1/sqrt(head), out linear."""
    if memory.shape[0] == 1 and x.shape[0] > 1:
        memory = memory.expand(x.shape[0], -1, -1)
    q = F.linear(x, p[prefix + "to_q.weight"])
    k = F.linear(memory, p[prefix + "to_k.weight"])
    v = F.linear(memory, p[prefix + "to_v.weight"])
    B, L, md = q.shape
    d = md // heads
    split = lambda t: t.reshape(B, t.shape[1], heads, d)
    out = OA.standard_attention_forward(split(q), split(k), split(v), scale=1.0 / math.sqrt(d))
    return F.linear(out.reshape(B, L, md), p[prefix + "to_out.weight"], p[prefix + "to_out.bias"])


def color_film(p: Dict[str, torch.Tensor], prefix: str, x: torch.Tensor, color: torch.Tensor) -> torch.Tensor:
    """LearnedMemoryColorFiLM.forward (causal_block.py:179-193)."""
    if color.shape[0] == 1 and x.shape[0] > 1:
        color = color.expand(x.shape[0], -1)
    h = F.silu(F.linear(color, p[prefix + "net.0.weight"], p[prefix + "net.0.bias"]))
    scale, shift = F.linear(h, p[prefix + "net.2.weight"], p[prefix + "net.2.bias"]).chunk(2, dim=-1)
    return x * scale[:, None] + shift[:, None]


def _memory_steps(p, prefix, cfg, stream: str, memory, color):
    """The adapters of one stream in this block, as (callable, argument) pairs."""
    if prefix + f"{stream}_memory_attn.to_q.weight" not in p:
        return []
    steps = []
    if memory is not None:
        steps.append((lambda x, m: memory_attention(p, prefix + f"{stream}_memory_attn.", x, m,
                                                    cfg.learned_memory_heads), memory))
    if stream == "video" and color is not None and prefix + "video_color_film.net.0.weight" in p:
        steps.append((lambda x, c: color_film(p, prefix + "video_color_film.", x, c), color))
    return steps


def _apply_steps(x, steps, eps):
    """x + adapter(rms_norm(x), arg) for each step (causal_block.py:489-505)."""
    for fn, arg in steps:
        x = x + fn(rms_norm(x, eps), arg)
    return x


def text_cross(p, prefix: str, attn: str, table: str, prompt_table: str, B: int, ts, prompt_ts, x, ctx, mask,
               heads: int, d_head: int, eps: float):
    """_apply_text_cross_attention_for_inference (kv_cache.py:1090-1141).
    Without prompt AdaLN: attention of rms_norm(x) over the context.  With it
    (the block holds ``prompt_table``): the query input is rms_norm(x) *
    (1 + scale) + shift from rows 6..8 of the block's table (shift, scale,
    gate), the context is modulated by (shift, scale) = prompt table + prompt
    timestep, and the output is scaled by the gate."""
    w = attn_weights(p, prefix + attn, heads, d_head)
    if prefix + prompt_table not in p:
        return OA.text_cross_attention(w, rms_norm(x, eps), ctx, mask)
    sh_q, sc_q, g = ada_values(p[prefix + table], B, ts, slice(6, 9))
    kv = p[prefix + prompt_table][None, None] + prompt_ts.reshape(B, prompt_ts.shape[1], 2, -1)
    sh_kv, sc_kv = kv.unbind(dim=2)
    return OA.text_cross_attention(w, rms_norm(x, eps) * (1 + sc_q) + sh_q, ctx * (1 + sc_kv) + sh_kv, mask) * g


def block_forward(p: Dict[str, torch.Tensor], prefix: str, cfg, vx, ax, v_ts, a_ts, video_pe, audio_pe,
                  video_cross_pe, audio_cross_pe, video_ctx, audio_ctx, video_mask, audio_mask, v_ss, v_gate,
                  a_ss, a_gate, cache: Dict[str, Optional[torch.Tensor]], video_memory=None, audio_memory=None,
                  color_memory=None, v_prompt=None, a_prompt=None):
    """kv_cache.py:2145-2656, synchronous branch.  ``cache`` holds dense
    video_self_k/v, audio_self_k/v, a2v_k/v, v2a_k/v (or None).  Returns
    (vx, ax, new_cache): new_cache holds each field with this chunk's K/V
    appended (the cache update of kv_cache.py:2642-2656, _cat_cache :394-398)."""
    eps = cfg.norm_eps
    B = vx.shape[0]
    vh, vdh, ah, adh = cfg.video_heads, cfg.video_d_head, cfg.audio_heads, cfg.audio_d_head
    mode = getattr(cfg, "learned_memory_mode", None)
    v_steps = _memory_steps(p, prefix, cfg, "video", video_memory, color_memory)
    a_steps = _memory_steps(p, prefix, cfg, "audio", audio_memory, None)
    t = lambda n: p[prefix + n]
    sh, sc, g = ada_values(t("scale_shift_table"), B, v_ts, slice(0, 3))
    out, vs_k, vs_v = OA.attention_with_cache(attn_weights(p, prefix + "attn1.", vh, vdh),
                                              rms_norm(vx, eps) * (1 + sc) + sh, None, video_pe, None,
                                              cache.get("video_self_k"), cache.get("video_self_v"))
    vx = vx + out * g
    if mode == "memory_kv_side_branch":
        vx = _apply_steps(vx, v_steps, eps)
    v_text = text_cross(p, prefix, "attn2.", "scale_shift_table", "prompt_scale_shift_table", B, v_ts, v_prompt, vx,
                        video_ctx, video_mask, vh, vdh, eps)
    sh, sc, g = ada_values(t("audio_scale_shift_table"), B, a_ts, slice(0, 3))
    out, as_k, as_v = OA.attention_with_cache(attn_weights(p, prefix + "audio_attn1.", ah, adh),
                                              rms_norm(ax, eps) * (1 + sc) + sh, None, audio_pe, None,
                                              cache.get("audio_self_k"), cache.get("audio_self_v"))
    ax = ax + out * g
    if mode == "memory_kv_side_branch":
        ax = _apply_steps(ax, a_steps, eps)
    a_text = text_cross(p, prefix, "audio_attn2.", "audio_scale_shift_table", "audio_prompt_scale_shift_table", B,
                        a_ts, a_prompt, ax, audio_ctx, audio_mask, ah, adh, eps)
    vx = vx + v_text
    ax = ax + a_text
    if mode == "cross_attn_adapter":
        vx = _apply_steps(vx, v_steps, eps)
        ax = _apply_steps(ax, a_steps, eps)
    vn, an = rms_norm(vx, eps), rms_norm(ax, eps)
    sc_a_a2v, sh_a_a2v, sc_a_v2a, sh_a_v2a, gate_v2a = av_ca_values(t("scale_shift_table_a2v_ca_audio"), B, a_ss,
                                                                     a_gate)
    sc_v_a2v, sh_v_a2v, sc_v_v2a, sh_v_v2a, gate_a2v = av_ca_values(t("scale_shift_table_a2v_ca_video"), B, v_ss,
                                                                     v_gate)
    a2v, a2v_k, a2v_v = OA.attention_with_cache(attn_weights(p, prefix + "audio_to_video_attn.", ah, adh),
                                        vn * (1 + sc_v_a2v) + sh_v_a2v, an * (1 + sc_a_a2v) + sh_a_a2v,
                                        video_cross_pe, audio_cross_pe, cache.get("a2v_k"), cache.get("a2v_v"))
    vx = vx + a2v * gate_a2v
    v2a, v2a_k, v2a_v = OA.attention_with_cache(attn_weights(p, prefix + "video_to_audio_attn.", ah, adh),
                                        an * (1 + sc_a_v2a) + sh_a_v2a, vn * (1 + sc_v_v2a) + sh_v_v2a,
                                        audio_cross_pe, video_cross_pe, cache.get("v2a_k"), cache.get("v2a_v"))
    ax = ax + v2a * gate_v2a
    sh, sc, g = ada_values(t("scale_shift_table"), B, v_ts, slice(3, 6))
    vx = vx + feed_forward(p, prefix + "ff.", rms_norm(vx, eps) * (1 + sc) + sh) * g
    sh, sc, g = ada_values(t("audio_scale_shift_table"), B, a_ts, slice(3, 6))
    ax = ax + feed_forward(p, prefix + "audio_ff.", rms_norm(ax, eps) * (1 + sc) + sh) * g
    new = {"video_self_k": vs_k, "video_self_v": vs_v, "audio_self_k": as_k, "audio_self_v": as_v,
           "a2v_k": a2v_k, "a2v_v": a2v_v, "v2a_k": v2a_k, "v2a_v": v2a_v}
    return vx, ax, {f: OC.cat_cache(cache.get(f), t) for f, t in new.items()}


def per_token(t: torch.Tensor, tokens: int) -> torch.Tensor:
    """_expand_per_frame_to_per_token (causal_model.py:1365-1392): [B, F, X] rows
    of F equal frames repeated over their tokens; [B, 1, X] and one row per
    token stay as they are."""
    B, F_, X = t.shape
    if F_ <= 1 or F_ == tokens:
        return t
    return t[:, :, None, :].expand(B, F_, tokens // F_, X).reshape(B, tokens, X)


def forward_chunk(p: Dict[str, torch.Tensor], cfg, video_latent, audio_latent, sigma, video_ctx, audio_ctx,
                  video_mask, audio_mask, video_pe, audio_pe, video_cross_pe, audio_cross_pe,
                  caches: List[Dict[str, Optional[torch.Tensor]]], learned_memory_video=None,
                  learned_memory_audio=None, learned_memory_color=None, audio_sigma=None,
                  return_caches: bool = False):
    """One denoising step: patchify, timestep modulation (causal_model.py:426-496),
    the block loop, the output heads (causal_model.py:568-599).  ``sigma`` is
    [B] or per latent frame [B, F] (expanded to the frames' tokens,
    kv_cache.py:2895-2903); ``audio_sigma`` defaults to ``sigma``.  Returns
    (video, audio) outputs, and with ``return_caches`` also every layer's cache
    with the chunk appended."""
    B = video_latent.shape[0]
    vx = F.linear(video_latent, p["patchify_proj.weight"], p["patchify_proj.bias"])
    ax = F.linear(audio_latent, p["audio_patchify_proj.weight"], p["audio_patchify_proj.bias"])
    s = (sigma * cfg.timestep_scale_multiplier).flatten()
    sa = ((sigma if audio_sigma is None else audio_sigma) * cfg.timestep_scale_multiplier).flatten()
    factor = cfg.av_ca_timestep_scale_multiplier / cfg.timestep_scale_multiplier
    v_ts, v_emb = adaln_single(p, "adaln_single.", s)
    a_ts, a_emb = adaln_single(p, "audio_adaln_single.", sa)
    v_ss, _ = adaln_single(p, "av_ca_video_scale_shift_adaln_single.", s)
    a_ss, _ = adaln_single(p, "av_ca_audio_scale_shift_adaln_single.", sa)
    v_gate, _ = adaln_single(p, "av_ca_a2v_gate_adaln_single.", s * factor)
    a_gate, _ = adaln_single(p, "av_ca_v2a_gate_adaln_single.", sa * factor)
    vm = am = cm = None
    if getattr(cfg, "learned_memory_enabled", False):
        if learned_memory_video is not None:
            vm = F.linear(learned_memory_video, p["learned_memory_video_encoder.weight"],
                          p["learned_memory_video_encoder.bias"])
        if learned_memory_audio is not None:
            am = F.linear(learned_memory_audio, p["learned_memory_audio_encoder.weight"],
                          p["learned_memory_audio_encoder.bias"])
        if learned_memory_color is not None and cfg.learned_memory_color_film_enabled:
            cm = learned_memory_color
    vview = lambda x: per_token(x.view(B, -1, x.shape[-1]), vx.shape[1])
    aview = lambda x: per_token(x.view(B, -1, x.shape[-1]), ax.shape[1])
    v_ts, v_emb, a_ts, a_emb = vview(v_ts), vview(v_emb), aview(a_ts), aview(a_emb)
    v_ss, a_ss, v_gate, a_gate = vview(v_ss), aview(a_ss), vview(v_gate), aview(a_gate)
    v_prompt = a_prompt = None
    if "prompt_adaln_single.linear.weight" in p:
        # LTX-2.3 prompt timestep (kv_cache.py:2876-2895): one value per sample,
        # the mean of per-frame / per-token sigmas
        vs = sigma.mean(dim=-1, keepdim=True) if sigma.dim() == 2 else sigma
        as_ = sigma if audio_sigma is None else audio_sigma
        as_ = as_.mean(dim=-1, keepdim=True) if as_.dim() == 2 else as_
        v_prompt = adaln_single(p, "prompt_adaln_single.", (vs * cfg.timestep_scale_multiplier).flatten())[0]
        a_prompt = adaln_single(p, "audio_prompt_adaln_single.", (as_ * cfg.timestep_scale_multiplier).flatten())[0]
        v_prompt, a_prompt = v_prompt.view(B, -1, v_prompt.shape[-1]), a_prompt.view(B, -1, a_prompt.shape[-1])
    new_caches = []
    for i in range(cfg.num_layers):
        vx, ax, nc = block_forward(p, f"transformer_blocks.{i}.", cfg, vx, ax, v_ts, a_ts, video_pe, audio_pe,
                                   video_cross_pe, audio_cross_pe, video_ctx, audio_ctx, video_mask, audio_mask,
                                   v_ss, v_gate, a_ss, a_gate, caches[i], vm, am, cm, v_prompt, a_prompt)
        new_caches.append(nc)

    def head(table, proj, x, emb):
        v = table[None, None] + emb[:, :, None]
        shift, scale = v[:, :, 0], v[:, :, 1]
        return F.linear(F.layer_norm(x, (x.shape[-1],), eps=1e-6) * (1 + scale) + shift, p[proj + ".weight"],
                        p[proj + ".bias"])

    out = (head(p["scale_shift_table"], "proj_out", vx, v_emb),
           head(p["audio_scale_shift_table"], "audio_proj_out", ax, a_emb))
    return (*out, new_caches) if return_caches else out
