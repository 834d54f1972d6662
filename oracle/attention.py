"""Attention-path restatement (oracle; test infrastructure only).

Follows:
  nn.RMSNorm(H*D) q/k norm       ltx_causal/attention/causal_attention.py:105-106
  standard_attention_forward     ltx_causal/attention/flex_attention_utils.py:225-276
  attention_with_cache (SP=1)    ltx_causal/transformer/kv_cache.py:1388-1547
  _finish_attention_output...    ltx_causal/transformer/kv_cache.py:1680-1700
  _prepare_attention_mask        ltx_causal/transformer/causal_model.py:551-562
  CausalLTXAttention.forward     ltx_causal/attention/causal_attention.py:224-324
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

from .rope import apply_split_rotary_emb


@dataclass
class AttnWeights:
    """Weights of one CausalLTXAttention (causal_attention.py:100-118)."""
    wq: torch.Tensor
    bq: torch.Tensor
    wk: torch.Tensor
    bk: torch.Tensor
    wv: torch.Tensor
    bv: torch.Tensor
    wo: torch.Tensor
    bo: torch.Tensor
    gq: torch.Tensor            # q_norm weight [H*D]
    gk: torch.Tensor            # k_norm weight [H*D]
    heads: int
    dim_head: int
    eps: float = 1e-6
    wg: Optional[torch.Tensor] = None   # to_gate_logits weight [H, query_dim]
    bg: Optional[torch.Tensor] = None

    def to(self, **kw) -> "AttnWeights":
        conv = {k: (v.to(**kw) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return AttnWeights(**conv)


def rms_norm_full_row(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float) -> torch.Tensor:
    """nn.RMSNorm(H*D, eps) over the full H*D row (causal_attention.py:105-106)."""
    return F.rms_norm(x, (x.shape[-1],), weight, eps)


def rms_norm_f64(x: np.ndarray, weight: Optional[np.ndarray], eps: float) -> np.ndarray:
    """Textbook RMSNorm in float64: x / sqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, dtype=np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y if weight is None else y * np.asarray(weight, dtype=np.float64)


def standard_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               mask: Optional[torch.Tensor] = None,
                               scale: Optional[float] = None) -> torch.Tensor:
    """flex_attention_utils.py:225-276: [B,L,H,D] in, [B,L,H,D] out through SDPA."""
    qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    am = None
    if mask is not None:
        if mask.dtype == torch.bool:
            am = torch.zeros_like(mask, dtype=q.dtype)
            am.masked_fill_(~mask, float("-inf"))
        else:
            am = mask
        if am.ndim == 2:
            am = am.unsqueeze(0).unsqueeze(0)
        elif am.ndim == 3:
            am = am.unsqueeze(1)
    out = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=am, scale=scale,
                                         dropout_p=0.0, is_causal=False)
    return out.transpose(1, 2)


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                  key_mask: Optional[np.ndarray] = None, scale: Optional[float] = None) -> np.ndarray:
    """Brute-force float64 softmax attention, [B,L,H,D] layout; key_mask [B,Lk] additive."""
    q = np.asarray(q, np.float64); k = np.asarray(k, np.float64); v = np.asarray(v, np.float64)
    d = q.shape[-1]
    sc = 1.0 / np.sqrt(d) if scale is None else scale
    s = np.einsum("bqhd,bkhd->bhqk", q, k) * sc
    if key_mask is not None:
        s = s + np.asarray(key_mask, np.float64)[:, None, None, :]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", p, v)


def prepare_attention_mask(mask: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """causal_model.py:551-562: 0/1 key mask -> additive (m-1)*finfo.max, [B,1,1,Lk]."""
    if torch.is_floating_point(mask):
        return mask
    return (mask - 1).to(dtype).reshape(mask.shape[0], 1, -1, mask.shape[-1]) * torch.finfo(dtype).max


def project_qkv(w: AttnWeights, x: torch.Tensor, ctx: torch.Tensor):
    """to_q/to_k/to_v Linear layers (causal_attention.py:100-102)."""
    return F.linear(x, w.wq, w.bq), F.linear(ctx, w.wk, w.bk), F.linear(ctx, w.wv, w.bv)


def norm_rope_qk(w: AttnWeights, q: torch.Tensor, k: torch.Tensor, pe, k_pe):
    """q_norm/k_norm then SPLIT RoPE (kv_cache.py:1406-1417)."""
    q = rms_norm_full_row(q, w.gq, w.eps)
    k = rms_norm_full_row(k, w.gk, w.eps)
    if pe is not None:
        q = apply_split_rotary_emb(q, *pe)
        kp = k_pe if k_pe is not None else pe
        k = apply_split_rotary_emb(k, *kp)
    return q, k


def finish_output(w: AttnWeights, out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """kv_cache.py:1680-1700: reshape, optional per-head gate 2*sigmoid, to_out."""
    B = x.shape[0]
    out = out.reshape(B, -1, w.heads * w.dim_head)
    if w.wg is not None:
        g = F.linear(x, w.wg, w.bg)
        b, t, _ = out.shape
        out = (out.view(b, t, w.heads, w.dim_head) * (2.0 * torch.sigmoid(g)).unsqueeze(-1))
        out = out.view(b, t, w.heads * w.dim_head)
    return F.linear(out, w.wo, w.bo)


def attention_with_cache(w: AttnWeights, x: torch.Tensor, context: Optional[torch.Tensor], pe, k_pe,
                         cached_k: Optional[torch.Tensor], cached_v: Optional[torch.Tensor],
                         logit_log_scale: Optional[torch.Tensor] = None,
                         new_kv_real_len: Optional[int] = None
                         ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """kv_cache.py:1148-1547, single-GPU synchronous branch (:1401-1428, :1474-1547)."""
    B = x.shape[0]
    ctx = x if context is None else context
    q, k, v = project_qkv(w, x, ctx)
    q, k = norm_rope_qk(w, q, k, pe, k_pe)
    if logit_log_scale is not None:
        q = q * logit_log_scale
    q = q.view(B, -1, w.heads, w.dim_head)
    k = k.view(B, -1, w.heads, w.dim_head)
    v = v.view(B, -1, w.heads, w.dim_head)
    if new_kv_real_len is not None and new_kv_real_len < k.shape[1]:
        k = k[:, :new_kv_real_len].contiguous()
        v = v[:, :new_kv_real_len].contiguous()
    new_k, new_v = k, v
    if cached_k is not None:
        full_k = torch.cat([cached_k, k], dim=1)
        full_v = torch.cat([cached_v, v], dim=1)
    else:
        full_k, full_v = k, v
    out = standard_attention_forward(q, full_k, full_v, mask=None)
    return finish_output(w, out, x), new_k, new_v


def text_cross_attention(w: AttnWeights, x: torch.Tensor, context: torch.Tensor,
                         mask: Optional[torch.Tensor]) -> torch.Tensor:
    """CausalLTXAttention.forward without RoPE (causal_attention.py:224-324), as
    text cross-attention calls it (kv_cache.py:764-785): q/k norm, no RoPE,
    additive key-padding mask, gate, to_out."""
    B = x.shape[0]
    q, k, v = project_qkv(w, x, context)
    q, k = norm_rope_qk(w, q, k, None, None)
    q = q.view(B, -1, w.heads, w.dim_head)
    k = k.view(B, -1, w.heads, w.dim_head)
    v = v.view(B, -1, w.heads, w.dim_head)
    out = standard_attention_forward(q, k, v, mask)
    return finish_output(w, out, x)
