"""The dual-stream (video + audio) causal DiT around the attention path: one
denoising step of a chunk through the block stack, on the gfx950 attention
kernels.

Host mirror, with the reference's module and parameter names so state dicts
line up:
  FeedForward / GELUApprox            ltx_causal/transformer/compat.py:28-71
  Timesteps / TimestepEmbedding /
  AdaLayerNormSingle                  compat.py:76-275
  CausalAVTransformerBlock (params)   ltx_causal/transformer/causal_block.py:196-376
  get_ada_values / get_av_ca_ada_values  causal_block.py:434-481
  block_forward_with_cache            ltx_causal/transformer/kv_cache.py:2145-2656
  _apply_text_cross_attention_for_inference  kv_cache.py:1090-1141
  _prepare_timestep / _prepare_cross_attention_timestep  causal_model.py:426-496
  _process_output                     causal_model.py:568-599

Built: the shipped inference configuration (no text-cross AdaLN, no gated
attention, captions already at the model width as in the 22B checkpoints),
with the learned long-memory adapters as an option (``AVConfig.learned_memory_*``):
  LearnedMemoryAttention / ColorFiLM  causal_block.py:108-193
  their placement in the block        kv_cache.py:2217-2330 (_apply_learned_memory,
                                      causal_block.py:489-505)
  memory encoders                     causal_model.py:253-268, kv_cache.py:529-559  The q/k/v/out projections, FFNs and the timestep
MLPs are PyTorch-ROCm GEMMs; every attention (video self, text cross, audio
self, text cross, A2V, V2A) and every residual update + (modulated) RMSNorm
pair between them runs through this package's kernels.
"""
from __future__ import annotations

import math
import weakref
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
from .attention import CausalLTXAttention, attention_with_cache, standard_attention_forward
from .kv_cache import LayerKVCache, _cat_cache


def rms_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """causal_block.py:94-101: RMSNorm over the last dim without a weight."""
    return F.rms_norm(x, (x.shape[-1],), weight=None, eps=eps)


class GELUApprox(nn.Module):
    def __init__(self, dim_in: int, dim_out: int):
        super().__init__()
        self.proj = nn.Linear(dim_in, dim_out)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and x.dtype == torch.bfloat16 and self.proj.bias is not None and not torch.is_grad_enabled():
            # the GEMM's GELU-bias epilogue: tanh-GELU of the float32
            # accumulator + bias, rounded to bf16 once, instead of a second
            # pass over the bf16 [tokens, 4·dim] output
            y = torch._addmm_activation(self.proj.bias, x.reshape(-1, x.shape[-1]), self.proj.weight.t(),
                                        use_gelu=True)
            return y.view(*x.shape[:-1], y.shape[-1])
        return F.gelu(self.proj(x), approximate="tanh")


class FeedForward(nn.Module):
    """compat.py:46-71: Linear -> tanh-GELU -> Linear, inner width mult * dim."""

    def __init__(self, dim: int, dim_out: int, mult: int = 4):
        super().__init__()
        inner = int(dim * mult)
        self.net = nn.Sequential(GELUApprox(dim, inner), nn.Identity(), nn.Linear(inner, dim_out))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x)


def timestep_embedding(t: torch.Tensor, dim: int = 256, max_period: int = 10000) -> torch.Tensor:
    """compat.py:76-106 with flip_sin_to_cos=True, downscale_freq_shift=0: [cos | sin]."""
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32, device=t.device) / half
    emb = t[:, None].float() * torch.exp(exponent)[None, :]
    return torch.cat([torch.cos(emb), torch.sin(emb)], dim=-1)


class TimestepEmbedding(nn.Module):
    def __init__(self, in_channels: int, dim: int):
        super().__init__()
        self.linear_1 = nn.Linear(in_channels, dim)
        self.act = nn.SiLU()
        self.linear_2 = nn.Linear(dim, dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.linear_2(self.act(self.linear_1(x)))


class _CombinedEmbedding(nn.Module):
    def __init__(self, dim: int):
        super().__init__()
        self.timestep_embedder = TimestepEmbedding(256, dim)

    def forward(self, t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        return self.timestep_embedder(timestep_embedding(t).to(dtype))


class AdaLayerNormSingle(nn.Module):
    """compat.py:212-275: timestep -> (coefficient * dim modulation, dim embedding)."""

    def __init__(self, dim: int, coefficient: int = 6):
        super().__init__()
        self.emb = _CombinedEmbedding(dim)
        self.silu = nn.SiLU()
        self.linear = nn.Linear(dim, coefficient * dim)

    def forward(self, t: torch.Tensor, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        e = self.emb(t, dtype)
        return self.linear(self.silu(e)), e


@dataclass
class AVConfig:
    """causal_model.py:97-190 defaults (22B inference configuration)."""
    num_layers: int = 48
    video_dim: int = 4096
    audio_dim: int = 2048
    video_heads: int = 32
    audio_heads: int = 32
    video_d_head: int = 128
    audio_d_head: int = 64
    in_channels: int = 128
    out_channels: int = 128
    norm_eps: float = 1e-6
    timestep_scale_multiplier: float = 1000.0
    av_ca_timestep_scale_multiplier: float = 1.0
    apply_gated_attention: bool = False   # per-head output gates (to_gate_logits)
    # LTX-2.3 text cross-attention AdaLN (causal_model.py:180-184): 9-row
    # modulation tables, prompt tables and prompt_adaln_single modules
    cross_attention_adaln: bool = False
    # learned long-memory adapters (causal_model.py:194-203), off by default
    learned_memory_enabled: bool = False
    learned_memory_mode: str = "cross_attn_adapter"   # or "memory_kv_side_branch"
    learned_memory_layer_interval: int = 4
    learned_memory_video_dim: int = 512
    learned_memory_audio_dim: int = 256
    learned_memory_heads: int = 8
    learned_memory_color_film_enabled: bool = False
    learned_memory_color_condition_dim: int = 512
    learned_memory_color_film_hidden_dim: int = 256


class LearnedMemoryAttention(nn.Module):
    """Cross-attention of the stream's tokens over the memory tokens
    (causal_block.py:108-160): q from the stream (query_dim -> memory_dim),
    k / v from the memory, ``heads`` heads of memory_dim / heads, out back to
    query_dim.  The attention runs on the flash kernels; a head size of 32
    (the audio adapter's 256 / 8) is zero-padded to 64, which leaves q.k and
    the first 32 output columns unchanged."""

    def __init__(self, query_dim: int, memory_dim: int, heads: int):
        super().__init__()
        heads = max(1, int(heads))
        if memory_dim % heads != 0:
            raise ValueError(f"learned memory dim ({memory_dim}) must be divisible by heads ({heads})")
        self.heads = heads
        self.head_dim = memory_dim // heads
        if self.head_dim not in (32, 64, 128):
            raise ValueError(f"learned memory head size {self.head_dim} is not built (32, 64 or 128)")
        self.to_q = nn.Linear(query_dim, memory_dim, bias=False)
        self.to_k = nn.Linear(memory_dim, memory_dim, bias=False)
        self.to_v = nn.Linear(memory_dim, memory_dim, bias=False)
        self.to_out = nn.Linear(memory_dim, query_dim, bias=True)

    def forward(self, x: torch.Tensor, memory: Optional[torch.Tensor]) -> torch.Tensor:
        if memory is None or memory.numel() == 0:
            return x.new_zeros(x.shape)
        B, L, _ = x.shape
        if memory.shape[0] == 1 and B > 1:
            memory = memory.expand(B, -1, -1)
        memory = memory.to(device=x.device, dtype=x.dtype)
        h, d = self.heads, self.head_dim
        q = self.to_q(x).view(B, L, h, d)
        k = self.to_k(memory).view(B, memory.shape[1], h, d)
        v = self.to_v(memory).view(B, memory.shape[1], h, d)
        if d == 32:
            pad = lambda t: F.pad(t, (0, 32))
            q, k, v = pad(q), pad(k), pad(v)
        out = standard_attention_forward(q, k, v, scale=1.0 / math.sqrt(d))
        return self.to_out(out[..., :d].reshape(B, L, h * d))


class LearnedMemoryColorFiLM(nn.Module):
    """x * scale + shift from the colour-memory vector through a SiLU MLP
    (causal_block.py:163-193)."""

    def __init__(self, condition_dim: int, query_dim: int, hidden_dim: int):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(int(condition_dim), max(1, int(hidden_dim))), nn.SiLU(),
                                 nn.Linear(max(1, int(hidden_dim)), query_dim * 2))

    def forward(self, x: torch.Tensor, color: Optional[torch.Tensor]) -> torch.Tensor:
        if color is None or color.numel() == 0:
            return x.new_zeros(x.shape)
        if color.shape[0] == 1 and x.shape[0] > 1:
            color = color.expand(x.shape[0], -1)
        scale, shift = self.net(color.to(device=x.device, dtype=x.dtype)).chunk(2, dim=-1)
        return x * scale.unsqueeze(1) + shift.unsqueeze(1)


class AVBlock(nn.Module):
    """Parameters of CausalAVTransformerBlock (causal_block.py:211-376), same
    names; block ``idx`` carries the memory adapters when learned memory is on
    and (idx + 1) is a multiple of the layer interval (causal_model.py:341-359)."""

    def __init__(self, cfg: AVConfig, idx: int = 0):
        super().__init__()
        self.idx = idx
        vd, ad = cfg.video_dim, cfg.audio_dim
        self.norm_eps = cfg.norm_eps
        gated = cfg.apply_gated_attention
        self.attn1 = CausalLTXAttention(vd, heads=cfg.video_heads, dim_head=cfg.video_d_head, norm_eps=cfg.norm_eps,
                                        apply_gated_attention=gated)
        self.attn2 = CausalLTXAttention(vd, context_dim=vd, heads=cfg.video_heads, dim_head=cfg.video_d_head,
                                        norm_eps=cfg.norm_eps, apply_gated_attention=gated)
        self.ff = FeedForward(vd, vd)
        coeff = 9 if cfg.cross_attention_adaln else 6   # causal_block.py:248-255
        self.cross_attention_adaln = bool(cfg.cross_attention_adaln)
        self.scale_shift_table = nn.Parameter(torch.empty(coeff, vd))
        self.audio_attn1 = CausalLTXAttention(ad, heads=cfg.audio_heads, dim_head=cfg.audio_d_head,
                                              norm_eps=cfg.norm_eps, apply_gated_attention=gated)
        self.audio_attn2 = CausalLTXAttention(ad, context_dim=ad, heads=cfg.audio_heads, dim_head=cfg.audio_d_head,
                                              norm_eps=cfg.norm_eps, apply_gated_attention=gated)
        self.audio_ff = FeedForward(ad, ad)
        self.audio_scale_shift_table = nn.Parameter(torch.empty(coeff, ad))
        if cfg.cross_attention_adaln:   # causal_block.py:343-348
            self.prompt_scale_shift_table = nn.Parameter(torch.empty(2, vd))
            self.audio_prompt_scale_shift_table = nn.Parameter(torch.empty(2, ad))
        self.audio_to_video_attn = CausalLTXAttention(vd, context_dim=ad, heads=cfg.audio_heads,
                                                      dim_head=cfg.audio_d_head, norm_eps=cfg.norm_eps,
                                                      apply_gated_attention=gated)
        self.video_to_audio_attn = CausalLTXAttention(ad, context_dim=vd, heads=cfg.audio_heads,
                                                      dim_head=cfg.audio_d_head, norm_eps=cfg.norm_eps,
                                                      apply_gated_attention=gated)
        self.scale_shift_table_a2v_ca_audio = nn.Parameter(torch.empty(5, ad))
        self.scale_shift_table_a2v_ca_video = nn.Parameter(torch.empty(5, vd))
        memory_here = (cfg.learned_memory_enabled and cfg.learned_memory_layer_interval > 0
                       and (idx + 1) % cfg.learned_memory_layer_interval == 0)
        self.learned_memory_mode = str(cfg.learned_memory_mode) if memory_here else None
        if memory_here and self.learned_memory_mode not in ("cross_attn_adapter", "memory_kv_side_branch"):
            raise ValueError(f"learned_memory_mode must be cross_attn_adapter or memory_kv_side_branch, "
                             f"got {self.learned_memory_mode!r}")
        self.video_memory_attn = LearnedMemoryAttention(vd, cfg.learned_memory_video_dim,
                                                        cfg.learned_memory_heads) if memory_here else None
        self.audio_memory_attn = LearnedMemoryAttention(ad, cfg.learned_memory_audio_dim,
                                                        cfg.learned_memory_heads) if memory_here else None
        self.video_color_film = LearnedMemoryColorFiLM(
            cfg.learned_memory_color_condition_dim, vd, cfg.learned_memory_color_film_hidden_dim) \
            if memory_here and cfg.learned_memory_color_film_enabled else None

    @staticmethod
    def get_ada_values(table: torch.Tensor, batch: int, timestep: torch.Tensor, idx: slice):
        """causal_block.py:434-452."""
        n = table.shape[0]
        return (table[idx].unsqueeze(0).unsqueeze(0).to(device=timestep.device, dtype=timestep.dtype)
                + timestep.reshape(batch, timestep.shape[1], n, -1)[:, :, idx, :]).unbind(dim=2)

    def get_av_ca_ada_values(self, table: torch.Tensor, batch: int, ss_t: torch.Tensor, gate_t: torch.Tensor):
        """causal_block.py:454-481: 4 scale/shift values then the gate."""
        ss = self.get_ada_values(table[:4, :], batch, ss_t, slice(None, None))
        gate = self.get_ada_values(table[4:, :], batch, gate_t, slice(None, None))
        return (*ss, *gate)


def _modulate(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_norm(x) * (1 + scale) + shift in one pass (ltx_adaln)."""
    n = torch.empty_like(x)
    kernels.adaln(x, n_out=n, scale=scale, shift=shift, eps=eps)
    return n


def _residual(x: torch.Tensor, y: torch.Tensor, gate: Optional[torch.Tensor] = None, norm: bool = False,
              scale: Optional[torch.Tensor] = None, shift: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """x + y * gate (x + y without a gate) and, with ``norm``, the next input
    rms_norm(x') [* (1 + scale) + shift] in the same pass (ltx_adaln)."""
    xo = torch.empty_like(x)
    n = torch.empty_like(x) if norm else None
    kernels.adaln(x, y=y, gate=gate, x_out=xo, n_out=n, scale=scale, shift=shift, eps=eps)
    return xo, n


def _apply_memory(x: torch.Tensor, n: Optional[torch.Tensor], steps, eps: float, need_norm: bool):
    """x + adapter(rms_norm(x), arg) for each (adapter, arg) in ``steps``
    (causal_block.py:489-505), each residual fused with the next norm.  ``n``
    is rms_norm(x) when already known.  Returns (x, rms_norm(x) or None)."""
    steps = [(m, a) for m, a in steps if m is not None and a is not None]
    for i, (mod, arg) in enumerate(steps):
        if n is None:
            n = torch.empty_like(x)
            kernels.adaln(x, n_out=n, eps=eps)
        x, n = _residual(x, mod(n, arg), norm=need_norm or i + 1 < len(steps), eps=eps)
    if need_norm and n is None:
        n = torch.empty_like(x)
        kernels.adaln(x, n_out=n, eps=eps)
    return x, n


def _all_blocks_ada(blocks, batch: int, v_ts, a_ts, v_ss, v_gate, a_ss, a_gate) -> List[Optional[Dict[str, tuple]]]:
    """Every block's modulation values (AVBlock.get_ada_values /
    get_av_ca_ada_values, causal_block.py:434-481) with one add per table kind
    over the stacked tables of all blocks instead of eight small adds per
    block: the same elementwise table + timestep sums.  Only for one timestep
    row per sample ([B, 1, n*D]): with per-token rows the stacked values of all
    blocks would be [L, B, T, n, D] at once (gigabytes at a 1152-token chunk),
    so each block then computes its own inside the block loop (None here)."""
    if any(t.shape[1] != 1 for t in (v_ts, a_ts, v_ss, v_gate, a_ss, a_gate)):
        return [None] * len(blocks)

    def stacked(name, ts, rows):
        tab = torch.stack([getattr(b, name)[rows] for b in blocks]).to(device=ts.device, dtype=ts.dtype)
        n = tab.shape[1]
        vals = tab[:, None, None] + ts.reshape(batch, ts.shape[1], n, -1)[None]
        return [v.unbind(dim=2) for v in vals]
    v = stacked("scale_shift_table", v_ts, slice(None))
    a = stacked("audio_scale_shift_table", a_ts, slice(None))
    a_ss4 = stacked("scale_shift_table_a2v_ca_audio", a_ss, slice(0, 4))
    a_g = stacked("scale_shift_table_a2v_ca_audio", a_gate, slice(4, 5))
    v_ss4 = stacked("scale_shift_table_a2v_ca_video", v_ss, slice(0, 4))
    v_g = stacked("scale_shift_table_a2v_ca_video", v_gate, slice(4, 5))
    return [{"v": v[i], "a": a[i], "a_ca": (*a_ss4[i], *a_g[i]), "v_ca": (*v_ss4[i], *v_g[i])}
            for i in range(len(blocks))]


def _text_cross(block: AVBlock, attn: CausalLTXAttention, x: torch.Tensor, xn: torch.Tensor, ctx: torch.Tensor,
                mask: Optional[torch.Tensor], ts: torch.Tensor, prompt_ts: Optional[torch.Tensor],
                table: torch.Tensor, prompt_table: Optional[torch.Tensor], ada_q: Optional[tuple]) -> torch.Tensor:
    """_apply_text_cross_attention_for_inference (kv_cache.py:1090-1141).
    ``xn`` is rms_norm(x).  Without prompt AdaLN the query input is xn.  With
    it (LTX-2.3): (shift, scale, gate) from rows 6..8 of the block's table,
    the query input rms_norm(x) * (1 + scale) + shift, the context modulated
    by (shift, scale) = prompt table + prompt timestep, and the output scaled
    by the gate (the residual adds it ungated, as without AdaLN)."""
    if prompt_table is None:
        return attn(xn, context=ctx, mask=mask)   # kv_cache.py:1134-1141
    B = x.shape[0]
    sh_q, sc_q, g = ada_q if ada_q is not None else block.get_ada_values(table, B, ts, slice(6, 9))
    kv = (prompt_table[None, None].to(device=x.device, dtype=x.dtype)
          + prompt_ts.reshape(B, prompt_ts.shape[1], 2, -1)).unbind(dim=2)
    ctx_mod = ctx * (1 + kv[1]) + kv[0]
    return attn(_modulate(x, sc_q, sh_q, block.norm_eps), context=ctx_mod, mask=mask) * g


def block_forward_with_cache(block: AVBlock, vx: torch.Tensor, ax: torch.Tensor, v_ts: torch.Tensor,
                             a_ts: torch.Tensor, video_pe, audio_pe, video_cross_pe, audio_cross_pe,
                             video_ctx: torch.Tensor, audio_ctx: torch.Tensor, video_mask: Optional[torch.Tensor],
                             audio_mask: Optional[torch.Tensor], v_cross_ss: torch.Tensor, v_cross_gate: torch.Tensor,
                             a_cross_ss: torch.Tensor, a_cross_gate: torch.Tensor, cache: LayerKVCache,
                             video_memory: Optional[torch.Tensor] = None, audio_memory: Optional[torch.Tensor] = None,
                             color_memory: Optional[torch.Tensor] = None, ada: Optional[Dict[str, tuple]] = None,
                             v_prompt: Optional[torch.Tensor] = None, a_prompt: Optional[torch.Tensor] = None,
                             audio_stream: Optional[torch.cuda.Stream] = None):
    """kv_cache.py:2145-2656 (synchronous branch): video self -> video text ->
    audio self -> audio text -> A2V -> V2A -> video FFN -> audio FFN.
    Returns (vx, ax, cache with the chunk's K/V appended).

    The residual updates and the (modulated) RMSNorms between the attentions
    and FFNs are fused pairwise into ltx_adaln passes with the reference's
    bf16 rounding; each stream's text residual is applied before the
    cross-modal norms as in the reference (the audio stream does not read the
    video residual before that point, so the order of the two streams'
    updates does not matter).

    With ``audio_stream`` the audio ops are queued on that HIP stream and the
    video ops on the current one, in the same order and with the same inputs:
    the two modalities only exchange their modulated inputs of A2V and V2A,
    which each side waits for (the caller forks ``audio_stream`` from the
    current stream before the first block and joins it after the last).  The
    audio stream's small, latency-bound kernels then run beside the video
    stream's large GEMMs; every result is unchanged.

    With memory adapters (``block.learned_memory_mode``): the video memory
    attention and colour FiLM, and the audio memory attention, are applied
    after the streams' self-attention residuals ("memory_kv_side_branch") or
    after their text residuals ("cross_attn_adapter"), kv_cache.py:2217-2330."""
    eps = block.norm_eps
    B = vx.shape[0]
    mode = getattr(block, "learned_memory_mode", None)
    v_steps = ((getattr(block, "video_memory_attn", None), video_memory),
               (getattr(block, "video_color_film", None), color_memory))
    a_steps = ((getattr(block, "audio_memory_attn", None), audio_memory),)
    side, after_text = mode == "memory_kv_side_branch", mode == "cross_attn_adapter"
    v_mem = any(m is not None and a is not None for m, a in v_steps)
    a_mem = any(m is not None and a is not None for m, a in a_steps)
    main = torch.cuda.current_stream(vx.device) if audio_stream is not None else None

    def on_audio():
        return torch.cuda.stream(audio_stream) if audio_stream is not None else _NoStream()

    # video self-attention, then its residual fused with the text-cross norm
    sh, sc, g = ada["v"][0:3] if ada else block.get_ada_values(block.scale_shift_table, B, v_ts, slice(0, 3))
    out, vs_k, vs_v = attention_with_cache(block.attn1, _modulate(vx, sc, sh, eps), None, video_pe, None,
                                           cache.video_self_k, cache.video_self_v)
    vx, vn = _residual(vx, out, g, norm=True, eps=eps)
    if side:
        vx, vn = _apply_memory(vx, vn, v_steps, eps, need_norm=True)
    v_text = _text_cross(block, block.attn2, vx, vn, video_ctx, video_mask, v_ts, v_prompt,
                         block.scale_shift_table, getattr(block, "prompt_scale_shift_table", None),
                         ada["v"][6:9] if ada and block.cross_attention_adaln else None)
    # audio self-attention and text cross-attention
    with on_audio():
        sh, sc, g = ada["a"][0:3] if ada else block.get_ada_values(block.audio_scale_shift_table, B, a_ts,
                                                                   slice(0, 3))
        out, as_k, as_v = attention_with_cache(block.audio_attn1, _modulate(ax, sc, sh, eps), None, audio_pe, None,
                                               cache.audio_self_k, cache.audio_self_v)
        ax, an = _residual(ax, out, g, norm=True, eps=eps)
        if side:
            ax, an = _apply_memory(ax, an, a_steps, eps, need_norm=True)
        a_text = _text_cross(block, block.audio_attn2, ax, an, audio_ctx, audio_mask, a_ts, a_prompt,
                             block.audio_scale_shift_table, getattr(block, "audio_prompt_scale_shift_table", None),
                             ada["a"][6:9] if ada and block.cross_attention_adaln else None)
    vx, vn = _residual(vx, v_text, norm=after_text and v_mem, eps=eps)
    with on_audio():
        ax, an = _residual(ax, a_text, norm=after_text and a_mem, eps=eps)
    if after_text:
        vx, _ = _apply_memory(vx, vn, v_steps, eps, need_norm=False)
        with on_audio():
            ax, _ = _apply_memory(ax, an, a_steps, eps, need_norm=False)
    # cross-modal: both read the norms taken before either update
    with on_audio():
        sc_a_a2v, sh_a_a2v, sc_a_v2a, sh_a_v2a, gate_v2a = ada["a_ca"] if ada else block.get_av_ca_ada_values(
            block.scale_shift_table_a2v_ca_audio, B, a_cross_ss, a_cross_gate)
        a_a2v_kv = _modulate(ax, sc_a_a2v, sh_a_a2v, eps)
        a_v2a_q = _modulate(ax, sc_a_v2a, sh_a_v2a, eps)
    sc_v_a2v, sh_v_a2v, sc_v_v2a, sh_v_v2a, gate_a2v = ada["v_ca"] if ada else block.get_av_ca_ada_values(
        block.scale_shift_table_a2v_ca_video, B, v_cross_ss, v_cross_gate)
    v_a2v_q = _modulate(vx, sc_v_a2v, sh_v_a2v, eps)
    v_v2a_kv = _modulate(vx, sc_v_v2a, sh_v_v2a, eps)
    if audio_stream is not None:
        # each side waits for the other's modulated input (and only what was
        # queued before it); the reading stream is recorded on the tensor so
        # its memory is not handed out again before that stream has read it
        main.wait_stream(audio_stream)
        audio_stream.wait_stream(main)
        a_a2v_kv.record_stream(main)
        v_v2a_kv.record_stream(audio_stream)
    a2v, a2v_k, a2v_v = attention_with_cache(block.audio_to_video_attn, v_a2v_q, a_a2v_kv, video_cross_pe,
                                             audio_cross_pe, cache.a2v_k, cache.a2v_v)
    with on_audio():
        v2a, v2a_k, v2a_v = attention_with_cache(block.video_to_audio_attn, a_v2a_q, v_v2a_kv, audio_cross_pe,
                                                 video_cross_pe, cache.v2a_k, cache.v2a_v)
    # cross-modal residuals fused with the feed-forward input norms
    sh, sc, g = ada["v"][3:6] if ada else block.get_ada_values(block.scale_shift_table, B, v_ts, slice(3, 6))
    vx, vn = _residual(vx, a2v, gate_a2v, norm=True, scale=sc, shift=sh, eps=eps)
    vx, _ = _residual(vx, block.ff(vn), g, eps=eps)
    with on_audio():
        sh, sc, g = ada["a"][3:6] if ada else block.get_ada_values(block.audio_scale_shift_table, B, a_ts,
                                                                   slice(3, 6))
        ax, an = _residual(ax, v2a, gate_v2a, norm=True, scale=sc, shift=sh, eps=eps)
        ax, _ = _residual(ax, block.audio_ff(an), g, eps=eps)
    new_cache = LayerKVCache(
        video_self_k=_cat_cache(cache.video_self_k, vs_k), video_self_v=_cat_cache(cache.video_self_v, vs_v),
        audio_self_k=_cat_cache(cache.audio_self_k, as_k), audio_self_v=_cat_cache(cache.audio_self_v, as_v),
        a2v_k=_cat_cache(cache.a2v_k, a2v_k), a2v_v=_cat_cache(cache.a2v_v, a2v_v),
        v2a_k=_cat_cache(cache.v2a_k, v2a_k), v2a_v=_cat_cache(cache.v2a_v, v2a_v))
    return vx, ax, new_cache


# AVModel -> {device index: the stream its audio ops run on}
_AUDIO_STREAMS: "weakref.WeakKeyDictionary[nn.Module, Dict[int, torch.cuda.Stream]]" = weakref.WeakKeyDictionary()


def _tensors(x) -> Tuple[torch.Tensor, ...]:
    """The tensors of a RoPE table argument: a (cos, sin) pair, one tensor or None."""
    if x is None:
        return ()
    if isinstance(x, torch.Tensor):
        return (x,)
    return tuple(t for t in x if isinstance(t, torch.Tensor))


class _NoStream:
    """A context that leaves the current stream as it is."""

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


class AVModel(nn.Module):
    """The block stack with its timestep modulation and output heads
    (causal_model.py:211-391 parameter names)."""

    def __init__(self, cfg: AVConfig):
        super().__init__()
        self.cfg = cfg
        vd, ad = cfg.video_dim, cfg.audio_dim
        self.patchify_proj = nn.Linear(cfg.in_channels, vd)
        self.audio_patchify_proj = nn.Linear(cfg.in_channels, ad)
        coeff = 9 if cfg.cross_attention_adaln else 6   # causal_model.py:246-283
        self.adaln_single = AdaLayerNormSingle(vd, coeff)
        self.audio_adaln_single = AdaLayerNormSingle(ad, coeff)
        self.prompt_adaln_single = AdaLayerNormSingle(vd, 2) if cfg.cross_attention_adaln else None
        self.audio_prompt_adaln_single = AdaLayerNormSingle(ad, 2) if cfg.cross_attention_adaln else None
        self.av_ca_video_scale_shift_adaln_single = AdaLayerNormSingle(vd, 4)
        self.av_ca_audio_scale_shift_adaln_single = AdaLayerNormSingle(ad, 4)
        self.av_ca_a2v_gate_adaln_single = AdaLayerNormSingle(vd, 1)
        self.av_ca_v2a_gate_adaln_single = AdaLayerNormSingle(ad, 1)
        self.transformer_blocks = nn.ModuleList([AVBlock(cfg, i) for i in range(cfg.num_layers)])
        if cfg.learned_memory_enabled:   # causal_model.py:253-268
            self.learned_memory_video_encoder = nn.Linear(cfg.in_channels, cfg.learned_memory_video_dim)
            self.learned_memory_audio_encoder = nn.Linear(cfg.in_channels, cfg.learned_memory_audio_dim)
        else:
            self.learned_memory_video_encoder = None
            self.learned_memory_audio_encoder = None
        self.scale_shift_table = nn.Parameter(torch.empty(2, vd))
        self.norm_out = nn.LayerNorm(vd, elementwise_affine=False, eps=1e-6)
        self.proj_out = nn.Linear(vd, cfg.out_channels)
        self.audio_scale_shift_table = nn.Parameter(torch.empty(2, ad))
        self.audio_norm_out = nn.LayerNorm(ad, elementwise_affine=False, eps=1e-6)
        self.audio_proj_out = nn.Linear(ad, cfg.out_channels)
        self._overlap_audio = True   # the audio ops on their own stream (overlap_audio_)

    def init_kv_cache(self, plan=None):
        """CausalLTX2DiffusionWrapper.init_kv_cache (wrapper.py:15-20): an empty
        LayerKVCache per block.  With an ``integration.ArenaPlan`` every block's
        four cached attentions start their caches in arenas of that size."""
        from .integration import init_kv_cache_for
        return init_kv_cache_for(self, plan)

    def fuse_qkv_(self) -> "AVModel":
        """Pack the q/k/v projections of every self-attention (video and audio)
        into one GEMM each; parameter names, values and memory are unchanged
        (CausalLTXAttention.fuse_qkv_)."""
        for m in self.modules():
            if isinstance(m, CausalLTXAttention):
                m.fuse_qkv_()
        return self

    def overlap_audio_(self, enabled: bool = True) -> "AVModel":
        """Queue each block's audio ops on a second HIP stream (default
        priority) beside the video ops on the current stream; the two meet at
        the A2V / V2A inputs and at the end of forward_chunk.  The results
        are the same as with one stream.  On by default on a GPU: the audio
        stream's kernels are small and latency-bound (75-token rows), and
        beside the video stream's GEMMs they take 84 instead of 89 ms of the
        48-block step at the 512x768 chunk."""
        self._overlap_audio = bool(enabled)
        return self

    def _audio_stream_for(self, device: torch.device) -> Optional[torch.cuda.Stream]:
        # kept outside the module's own attributes, so that copies and pickles
        # of the model carry no stream (each copy makes its own on first use)
        if not getattr(self, "_overlap_audio", False) or device.type != "cuda":
            return None
        streams = _AUDIO_STREAMS.setdefault(self, {})
        if device.index not in streams:
            streams[device.index] = torch.cuda.Stream(device=device)
        return streams[device.index]

    def cache_text_kv_(self, enabled: bool = True, size: int = 4) -> "AVModel":
        """Keep each block's text cross-attention K/V (video and audio) across
        calls with the same context tensor (CausalLTXAttention.cache_text_kv_;
        kv_cache.py:707-760, off by default as there)."""
        for blk in self.transformer_blocks:
            blk.attn2.cache_text_kv_(enabled, size)
            blk.audio_attn2.cache_text_kv_(enabled, size)
        return self

    @staticmethod
    def _per_token(t: torch.Tensor, tokens: int) -> torch.Tensor:
        """_expand_per_frame_to_per_token (causal_model.py:1365-1392): [B, F, X]
        per-frame rows repeated over the F equal frames of ``tokens`` tokens;
        one row ([B, 1, X]) broadcasts and stays as it is."""
        B, F, X = t.shape
        if F <= 1 or F == tokens:
            return t
        if tokens % F:
            raise ValueError(f"{tokens} tokens are not {F} equal frames")
        return t.unsqueeze(2).expand(B, F, tokens // F, X).reshape(B, tokens, X)

    def _timestep(self, sigma: torch.Tensor, adaln: AdaLayerNormSingle, batch: int, dtype):
        """causal_model.py:426-455."""
        ts, emb = adaln((sigma * self.cfg.timestep_scale_multiplier).flatten(), dtype)
        return ts.view(batch, -1, ts.shape[-1]), emb.view(batch, -1, emb.shape[-1])

    def _cross_timestep(self, sigma: torch.Tensor, ss: AdaLayerNormSingle, gate: AdaLayerNormSingle, batch: int,
                        dtype):
        """causal_model.py:457-496."""
        scaled = (sigma * self.cfg.timestep_scale_multiplier).flatten()
        factor = self.cfg.av_ca_timestep_scale_multiplier / self.cfg.timestep_scale_multiplier
        s, _ = ss(scaled, dtype)
        g, _ = gate(scaled * factor, dtype)
        return s.view(batch, -1, s.shape[-1]), g.view(batch, -1, g.shape[-1])

    @staticmethod
    def _process_output(table, norm, proj, x, emb):
        """causal_model.py:568-599."""
        v = table[None, None].to(device=x.device, dtype=x.dtype) + emb[:, :, None]
        shift, scale = v[:, :, 0], v[:, :, 1]
        return proj(norm(x) * (1 + scale) + shift)

    def forward_chunk(self, video_latent: torch.Tensor, audio_latent: torch.Tensor, sigma: torch.Tensor,
                      video_ctx: torch.Tensor, audio_ctx: torch.Tensor, video_mask: Optional[torch.Tensor],
                      audio_mask: Optional[torch.Tensor], video_pe, audio_pe, video_cross_pe, audio_cross_pe,
                      caches: List[LayerKVCache], commit: bool = False,
                      learned_memory_video: Optional[torch.Tensor] = None,
                      learned_memory_audio: Optional[torch.Tensor] = None,
                      learned_memory_color: Optional[torch.Tensor] = None, kv_cache_only: bool = False,
                      audio_sigma: Optional[torch.Tensor] = None):
        """One denoising step of a chunk (the block loop of
        model_forward_inference, kv_cache.py:2681-3365): returns the video and
        audio outputs [B, T, out_channels] and, with ``commit``, the caches
        with the chunk's keys appended (a denoise step leaves them as given).
        ``sigma`` is one value per sample [B] or one per latent frame [B, F]
        (the reference's ``timesteps``; a conditioning frame carries 0,
        model_runtime.py:897-910), expanded to the frame's tokens
        (kv_cache.py:2895-2903); ``audio_sigma`` ([B] or one per audio token)
        defaults to ``sigma`` when that is per sample.
        The learned-memory tensors ([B, N, in_channels] tokens, [B, 4C] colour
        vector, from ``LearnedMemoryState.with_conditional_memory``) are used
        when the model has memory adapters.  ``kv_cache_only`` is the clean
        commit pass (kv_cache.py:3302-3309): it commits and returns
        (None, None, caches) without the output heads."""
        commit = commit or kv_cache_only
        B = video_latent.shape[0]
        dt = self.patchify_proj.weight.dtype
        vm = am = cm = None
        if self.cfg.learned_memory_enabled:   # kv_cache.py:529-559
            dev = video_latent.device
            if learned_memory_video is not None:
                vm = self.learned_memory_video_encoder(learned_memory_video.to(device=dev, dtype=dt))
            if learned_memory_audio is not None:
                am = self.learned_memory_audio_encoder(learned_memory_audio.to(device=dev, dtype=dt))
            if learned_memory_color is not None and self.cfg.learned_memory_color_film_enabled:
                cm = learned_memory_color.to(device=dev, dtype=dt)
        vx = self.patchify_proj(video_latent)
        ax = self.audio_patchify_proj(audio_latent)
        if audio_sigma is None:
            if sigma.dim() == 2 and sigma.shape[1] > 1:
                raise ValueError("per-frame video sigma needs its own audio_sigma ([B] or [B, audio tokens])")
            audio_sigma = sigma
        Lv, La = vx.shape[1], ax.shape[1]
        v_ts, v_emb = self._timestep(sigma, self.adaln_single, B, dt)
        a_ts, a_emb = self._timestep(audio_sigma, self.audio_adaln_single, B, dt)
        v_ss, v_gate = self._cross_timestep(sigma, self.av_ca_video_scale_shift_adaln_single,
                                            self.av_ca_a2v_gate_adaln_single, B, dt)
        a_ss, a_gate = self._cross_timestep(audio_sigma, self.av_ca_audio_scale_shift_adaln_single,
                                            self.av_ca_v2a_gate_adaln_single, B, dt)
        v_ts, v_emb, v_ss, v_gate = (self._per_token(t, Lv) for t in (v_ts, v_emb, v_ss, v_gate))
        a_ts, a_emb, a_ss, a_gate = (self._per_token(t, La) for t in (a_ts, a_emb, a_ss, a_gate))
        v_prompt = a_prompt = None
        if self.cfg.cross_attention_adaln:
            # LTX-2.3 prompt timestep (kv_cache.py:2876-2895): one value per
            # sample, the mean of per-frame / per-token sigmas
            vs = sigma.mean(dim=-1, keepdim=True) if sigma.dim() == 2 else sigma
            as_ = audio_sigma.mean(dim=-1, keepdim=True) if audio_sigma.dim() == 2 else audio_sigma
            v_prompt, _ = self._timestep(vs, self.prompt_adaln_single, B, dt)
            a_prompt, _ = self._timestep(as_, self.audio_prompt_adaln_single, B, dt)
        new_caches = []
        ada = _all_blocks_ada(self.transformer_blocks, B, v_ts, a_ts, v_ss, v_gate, a_ss, a_gate)
        astream = self._audio_stream_for(vx.device)
        if astream is not None:
            # fork: the audio stream starts after everything queued so far,
            # and the audio inputs made on the current stream are recorded on
            # it (their memory is not reused before it has read them)
            main = torch.cuda.current_stream(vx.device)
            astream.wait_stream(main)
            for t in (ax, a_ts, a_ss, a_gate, audio_ctx, audio_mask, a_prompt, am, *_tensors(audio_pe),
                      *_tensors(audio_cross_pe), *_tensors(video_cross_pe)):
                if isinstance(t, torch.Tensor) and t.is_cuda:
                    t.record_stream(astream)
        try:
            for blk, cache, blk_ada in zip(self.transformer_blocks, caches, ada):
                vx, ax, nc = block_forward_with_cache(blk, vx, ax, v_ts, a_ts, video_pe, audio_pe, video_cross_pe,
                                                      audio_cross_pe, video_ctx, audio_ctx, video_mask, audio_mask,
                                                      v_ss, v_gate, a_ss, a_gate, cache, vm, am, cm, ada=blk_ada,
                                                      v_prompt=v_prompt, a_prompt=a_prompt, audio_stream=astream)
                new_caches.append(nc if commit else cache)
                del nc
        finally:
            if astream is not None:
                # join (also when a block raised): the current stream waits
                # for everything queued on the audio stream
                main.wait_stream(astream)
                ax.record_stream(main)
        if kv_cache_only:
            return None, None, new_caches
        vo = self._process_output(self.scale_shift_table, self.norm_out, self.proj_out, vx, v_emb)
        ao = self._process_output(self.audio_scale_shift_table, self.audio_norm_out, self.audio_proj_out, ax, a_emb)
        return vo, ao, new_caches


def init_random_(model: nn.Module, seed: int, std: float = 0.02) -> None:
    """Seeded random weights in place: linear weights ~N(0, std^2), biases 0,
    modulation tables ~N(0, 1)/sqrt(width) (the reference's table init)."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("bias"):
                p.zero_()
            elif "scale_shift_table" in name:
                p.copy_(torch.randn(p.shape, generator=g, device=dev) / math.sqrt(p.shape[-1]))
            elif name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.copy_(torch.randn(p.shape, generator=g, device=dev) * std)


def build_model(cfg: AVConfig, device, seed: int = 3, dtype=torch.bfloat16) -> AVModel:
    """The model constructed directly on ``device`` in ``dtype`` (no host copy
    of the weights), then seeded."""
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device(device):
            m = AVModel(cfg)
    finally:
        torch.set_default_dtype(prev)
    init_random_(m, seed)
    return m.eval()
