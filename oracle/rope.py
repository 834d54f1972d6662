"""RoPE restatement (oracle; test infrastructure only).

Follows ltx_causal/rope/causal_rope.py:
  generate_freq_grid           :45-80
  apply_split_rotary_emb       :102-132
  causal_precompute_freqs_cis  :139-357 (SPLIT branch :323-341)
plus float64 closed forms used to pin the float32 restatement.
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np
import torch

VIDEO_TEMPORAL_SCALE = 8   # causal_rope.py:33
VIDEO_SPATIAL_SCALE = 32   # :34
VIDEO_FPS = 24             # :35
AUDIO_DOWNSAMPLE = 4       # :36
AUDIO_HOP = 160            # :37
AUDIO_SR = 16000           # :38


def generate_freq_grid(theta: float, max_pos_count: int, inner_dim: int) -> torch.Tensor:
    """causal_rope.py:45-80 -- theta ** linspace(log_theta(1), 1, n) * pi/2, float32."""
    n_elem = 2 * max_pos_count
    idx = theta ** torch.linspace(math.log(1, theta), math.log(theta, theta),
                                  inner_dim // n_elem, dtype=torch.float32)
    return idx * math.pi / 2


def ntk_theta(theta: float, dim: int, grid_f: int, start_frame: int, is_audio: bool,
              rope_extrapolation: str, rope_train_max_seconds: float) -> float:
    """causal_rope.py:213-246 -- NTK-aware theta scaling (off by default)."""
    if rope_extrapolation == "off":
        return float(theta)
    if rope_extrapolation != "ntk":
        raise ValueError(f"rope_extrapolation must be 'off' or 'ntk', got {rope_extrapolation!r}")
    max_abs = int(start_frame) + int(grid_f)
    if max_abs <= 0:
        return float(theta)
    if is_audio:
        t_max = max(0.0, max_abs * AUDIO_DOWNSAMPLE + 1 - AUDIO_DOWNSAMPLE) * AUDIO_HOP / AUDIO_SR
    else:
        t_max = max(0.0, max_abs * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE) / VIDEO_FPS
    ratio = max(1.0, t_max / max(float(rope_train_max_seconds), 1e-6))
    if ratio > 1.0:
        return float(theta) * ratio ** (float(dim) / max(float(dim - 2), 1.0))
    return float(theta)


def _fractional_positions(grid: Tuple[int, ...], start_frame: int, is_audio: bool,
                          max_pos: List[int]) -> torch.Tensor:
    """causal_rope.py:258-311 -- [T, num_pos_dims] float32 fractional positions."""
    if len(grid) == 3:
        f, h, w = grid
        lt = torch.arange(start_frame, start_frame + f, dtype=torch.float32)
        ps = (lt * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE).clamp(min=0)
        pe = ((lt + 1) * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE).clamp(min=0)
        t_sec = (ps + pe) / 2.0 / VIDEO_FPS
        hp = torch.arange(h, dtype=torch.float32) * VIDEO_SPATIAL_SCALE + VIDEO_SPATIAL_SCALE / 2.0
        wp = torch.arange(w, dtype=torch.float32) * VIDEO_SPATIAL_SCALE + VIDEO_SPATIAL_SCALE / 2.0
        gt, gh, gw = torch.meshgrid(t_sec / max_pos[0], hp / max_pos[1], wp / max_pos[2], indexing="ij")
        return torch.stack([gt, gh, gw], dim=-1).reshape(f * h * w, 3)
    (f,) = grid
    lt = torch.arange(start_frame, start_frame + f, dtype=torch.float32)
    if is_audio:
        ms = (lt * AUDIO_DOWNSAMPLE + 1 - AUDIO_DOWNSAMPLE).clamp(min=0)
        me = ((lt + 1) * AUDIO_DOWNSAMPLE + 1 - AUDIO_DOWNSAMPLE).clamp(min=0)
        t_sec = (ms + me) / 2.0 * AUDIO_HOP / AUDIO_SR
    else:
        ps = (lt * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE).clamp(min=0)
        pe = ((lt + 1) * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE).clamp(min=0)
        t_sec = (ps + pe) / 2.0 / VIDEO_FPS
    return (t_sec / max_pos[0]).unsqueeze(-1)


def rope_angles(grid: Tuple[int, ...], dim: int, theta: float = 10000.0,
                max_pos: Optional[List[int]] = None, start_frame: int = 0,
                is_audio: bool = False, rope_extrapolation: str = "off",
                rope_train_max_seconds: float = 8.0) -> Tuple[torch.Tensor, int]:
    """causal_rope.py:249-321: float32 angles [T, n*ndim] interleaved
    [f0_t, f0_h, f0_w, f1_t, ...] (before the SPLIT pad), and the pad size."""
    if max_pos is None:
        max_pos = [20, 2048, 2048]
    ndim = len(grid)
    th = ntk_theta(theta, dim, grid[0], start_frame, is_audio, rope_extrapolation,
                   rope_train_max_seconds)
    ind = generate_freq_grid(th, ndim, dim)                        # [n]
    frac = _fractional_positions(grid, start_frame, is_audio, max_pos)  # [T, ndim]
    freqs = ind * (frac.unsqueeze(-1) * 2 - 1)                     # [T, ndim, n]
    freqs = freqs.transpose(-1, -2).flatten(1)                      # [T, n*ndim]
    return freqs, dim // 2 - freqs.shape[-1]


def causal_precompute_freqs_cis(grid: Tuple[int, ...], dim: int, theta: float = 10000.0,
                                max_pos: Optional[List[int]] = None, start_frame: int = 0,
                                dtype: torch.dtype = torch.float32, is_audio: bool = False,
                                num_attention_heads: int = 32, batch: int = 1,
                                rope_extrapolation: str = "off",
                                rope_train_max_seconds: float = 8.0):
    """causal_rope.py:139-357, SPLIT branch.  Returns (cos, sin) [batch, H, T, dim/(2H)].

    The reference loops over batch rows of ``grid_sizes`` (:254-321) and stacks
    them; every row here uses the same grid, and ``batch`` copies are returned
    so a B=2 input pairs with a B=2 table (the reference's split helper reshapes
    x with the *table's* batch, :111-115).
    """
    freqs, pad = rope_angles(grid, dim, theta, max_pos, start_frame, is_audio,
                             rope_extrapolation, rope_train_max_seconds)
    cos, sin = freqs.cos(), freqs.sin()
    if pad > 0:
        cos = torch.cat([torch.ones_like(cos[:, :pad]), cos], dim=-1)
        sin = torch.cat([torch.zeros_like(sin[:, :pad]), sin], dim=-1)
    T = cos.shape[0]
    cos = cos.reshape(T, num_attention_heads, -1).swapaxes(0, 1)
    sin = sin.reshape(T, num_attention_heads, -1).swapaxes(0, 1)
    cos = cos.unsqueeze(0).expand(batch, -1, -1, -1).contiguous()
    sin = sin.unsqueeze(0).expand(batch, -1, -1, -1).contiguous()
    return cos.to(dtype), sin.to(dtype)


def freqs_closed_form_f64(grid: Tuple[int, ...], dim: int, theta: float = 10000.0,
                          max_pos: Optional[List[int]] = None, start_frame: int = 0,
                          is_audio: bool = False, num_attention_heads: int = 32) -> np.ndarray:
    """Float64 angle table [H, T, dim/(2H)] written from the formulas, no torch.

    Pad entries hold angle 0.  Used only to pin the float32 restatement.
    """
    if max_pos is None:
        max_pos = [20, 2048, 2048]
    ndim = len(grid)
    n = dim // (2 * ndim)
    ind = np.array([theta ** (i / (n - 1)) if n > 1 else 1.0 for i in range(n)]) * math.pi / 2
    rows = []
    if ndim == 3:
        F, Hh, W = grid
        for f in range(F):
            lf = start_frame + f
            t = (max(0, 8 * lf - 7) + max(0, 8 * lf + 1)) / 2 / 24
            for hi in range(Hh):
                for wi in range(W):
                    pos = (t / max_pos[0], (32 * hi + 16) / max_pos[1], (32 * wi + 16) / max_pos[2])
                    rows.append([ind[k] * (2 * pos[a] - 1) for k in range(n) for a in range(3)])
    else:
        (F,) = grid
        for f in range(F):
            lf = start_frame + f
            if is_audio:
                t = (max(0, 4 * lf - 3) + max(0, 4 * lf + 1)) / 2 * 160 / 16000
            else:
                t = (max(0, 8 * lf - 7) + max(0, 8 * lf + 1)) / 2 / 24
            rows.append([ind[k] * (2 * t / max_pos[0] - 1) for k in range(n)])
    ang = np.array(rows, dtype=np.float64)
    pad = dim // 2 - ang.shape[1]
    ang = np.concatenate([np.zeros((ang.shape[0], pad)), ang], axis=1)
    T = ang.shape[0]
    return ang.reshape(T, num_attention_heads, -1).transpose(1, 0, 2)


def apply_split_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """causal_rope.py:102-132.  x [B, T, H*D] with cos/sin [B, H, T, D/2].

    Same op sequence as the reference: ``out = x * cos`` (one rounding), then
    ``out1.addcmul_(-sin, x2)`` / ``out2.addcmul_(sin, x1)``.
    """
    squeeze = False
    if x.ndim != 4 and cos.ndim == 4:
        b, h, t, _ = cos.shape
        x = x.reshape(b, t, h, -1).swapaxes(1, 2)
        squeeze = True
    d2 = x.shape[-1] // 2
    split = x.reshape(*x.shape[:-1], 2, d2)
    first, second = split[..., :1, :], split[..., 1:, :]
    out = split * cos.unsqueeze(-2)
    out[..., :1, :].addcmul_(-sin.unsqueeze(-2), second)
    out[..., 1:, :].addcmul_(sin.unsqueeze(-2), first)
    out = out.reshape(*x.shape)
    if squeeze:
        out = out.swapaxes(1, 2).reshape(b, t, -1)
    return out
