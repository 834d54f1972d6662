"""RoPE tables and SPLIT rotation on gfx950 (host mirror of ltx_causal/rope/causal_rope.py).

``causal_precompute_freqs_cis`` keeps the reference signature (causal_rope.py:139-152)
and returns the SPLIT ``(cos, sin)`` pair ``[B, H, T, dim/(2H)]``; the table is
built on the device by ``ltx_rope_table``.  ``apply_split_rotary_emb`` keeps
causal_rope.py:102 and runs the fused kernel with the norm switched off.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from enum import Enum
from typing import List, Optional, Tuple, Union

import torch

from . import kernels

VIDEO_TEMPORAL_SCALE = 8
VIDEO_FPS = 24
AUDIO_DOWNSAMPLE_FACTOR = 4
AUDIO_HOP_LENGTH = 160
AUDIO_SAMPLE_RATE = 16000


class CausalRopeType(Enum):
    """causal_rope.py:20-23."""
    INTERLEAVED = "interleaved"
    SPLIT = "split"


_FREQ_CACHE: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_TABLE_CACHE: "OrderedDict[tuple, Tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()
_TABLE_CACHE_SIZE = 16
# one built video table per layout (everything but the start frame, with the
# theta actually used): a table for a new start frame is derived from it by
# ltx_rope_table_retime, which recomputes only the t-axis entries
_VIDEO_TEMPLATES: "OrderedDict[tuple, Tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()


def generate_freq_grid(theta: float, max_pos_count: int, inner_dim: int,
                       device: Union[torch.device, str] = "cuda") -> torch.Tensor:
    """causal_rope.py:45-80.  The n = inner_dim // (2*max_pos_count) frequencies
    ``theta**linspace(0, 1, n) * pi/2`` are evaluated once on the host in float32
    (the same expression the reference evaluates) and kept on the device."""
    dev = torch.device(device)
    key = (float(theta), int(max_pos_count), int(inner_dim), str(dev))
    hit = _FREQ_CACHE.get(key)
    if hit is not None:
        return hit
    n = inner_dim // (2 * max_pos_count)
    idx = theta ** torch.linspace(math.log(1, theta), math.log(theta, theta), n, dtype=torch.float32)
    idx = (idx * math.pi / 2).to(dev)
    _FREQ_CACHE[key] = idx
    if len(_FREQ_CACHE) > 64:
        _FREQ_CACHE.popitem(last=False)
    return idx


def _ntk_theta(theta, dim, max_latent_f, start_frame, is_audio, mode, train_max_s) -> float:
    """causal_rope.py:213-246 (NTK-aware scaling, host scalar math)."""
    if mode == "off":
        return float(theta)
    if mode != "ntk":
        raise ValueError(f"rope_extrapolation must be 'off' or 'ntk', got {mode!r}")
    max_abs = int(start_frame) + int(max_latent_f)
    if max_abs <= 0:
        return float(theta)
    if is_audio:
        t_max = max(0.0, max_abs * AUDIO_DOWNSAMPLE_FACTOR + 1 - AUDIO_DOWNSAMPLE_FACTOR) \
            * AUDIO_HOP_LENGTH / AUDIO_SAMPLE_RATE
    else:
        t_max = max(0.0, max_abs * VIDEO_TEMPORAL_SCALE + 1 - VIDEO_TEMPORAL_SCALE) / VIDEO_FPS
    ratio = max(1.0, t_max / max(float(train_max_s), 1e-6))
    if ratio > 1.0:
        return float(theta) * ratio ** (float(dim) / max(float(dim - 2), 1.0))
    return float(theta)


def causal_precompute_freqs_cis(
    grid_sizes: torch.Tensor,
    dim: int,
    theta: float = 10000.0,
    max_pos: Optional[List[int]] = None,
    start_frame: int = 0,
    rope_type: CausalRopeType = CausalRopeType.SPLIT,
    device: Union[torch.device, str] = "cuda",
    dtype: torch.dtype = torch.float32,
    is_audio: bool = False,
    rope_extrapolation: str = "off",
    rope_train_max_seconds: float = 8.0,
    num_attention_heads: int = 32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """causal_rope.py:139-357, SPLIT layout, built by ltx_rope_table.

    Every batch row of ``grid_sizes`` must describe the same grid (the
    reference stacks per-row tables, which requires equal lengths anyway).
    Tables are cached by their integer layout (grid, start frame, dims, dtype),
    which is exact: they depend on nothing else (kv_cache.py:562-652).
    """
    if rope_type != CausalRopeType.SPLIT:
        raise NotImplementedError("only SPLIT RoPE is built (TaoMate's configured rope_type)")
    if dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"RoPE tables are built in float32 or bfloat16, not {dtype}")
    if max_pos is None:
        max_pos = [20, 2048, 2048]
    gs = torch.as_tensor(grid_sizes)
    if gs.ndim == 3:
        gs = (gs[..., 0] + gs[..., 1]) / 2.0
    rows = [tuple(int(v) for v in r) for r in gs.tolist()]
    if not rows or any(r != rows[0] for r in rows):
        raise NotImplementedError("all batch rows of grid_sizes must be equal")
    grid = rows[0]
    nd = len(grid)
    if nd not in (1, 3):
        raise ValueError(f"Unsupported num_pos_dims: {nd}")
    batch = len(rows)
    dev = torch.device(device)
    key = (grid, int(dim), float(theta), tuple(int(m) for m in max_pos[:nd]), int(start_frame),
           str(dev), str(dtype), bool(is_audio), rope_extrapolation, float(rope_train_max_seconds),
           int(num_attention_heads), batch)
    hit = _TABLE_CACHE.get(key)
    if hit is not None:
        _TABLE_CACHE.move_to_end(key)
        return hit
    th = _ntk_theta(theta, dim, grid[0], start_frame, is_audio, rope_extrapolation,
                    rope_train_max_seconds)
    freq = generate_freq_grid(th, nd, dim, dev)
    # every batch row has the same grid, so one row of the table is built and
    # the batch dimension is a stride-0 expansion: the values are the
    # reference's [B, H, T, dim/(2H)] tables, and the kernels that read them
    # see one copy (shared through the cache hierarchy) instead of B
    tkey = (grid, int(dim), float(th), tuple(int(m) for m in max_pos[:nd]), str(dev), str(dtype),
            int(num_attention_heads)) if nd == 3 else None
    tmpl = _VIDEO_TEMPLATES.get(tkey) if tkey is not None else None
    per = dim // 2 // num_attention_heads
    if tmpl is not None:
        cos, sin = kernels.rope_table_retime(tmpl, freq, grid, start_frame, float(max_pos[0]), dim,
                                             num_attention_heads)
    else:
        cos, sin = kernels.rope_table(freq, grid, start_frame, is_audio, [float(m) for m in max_pos[:nd]],
                                      dim, num_attention_heads, 1, dtype)
        if tkey is not None and (per * cos.element_size()) % 16 == 0:
            _VIDEO_TEMPLATES[tkey] = (cos, sin)
            while len(_VIDEO_TEMPLATES) > _TABLE_CACHE_SIZE:
                _VIDEO_TEMPLATES.popitem(last=False)
    out = (cos.expand(batch, -1, -1, -1), sin.expand(batch, -1, -1, -1))
    _TABLE_CACHE[key] = out
    while len(_TABLE_CACHE) > _TABLE_CACHE_SIZE:
        _TABLE_CACHE.popitem(last=False)
    return out


def apply_split_rotary_emb(input_tensor: torch.Tensor, cos_freqs: torch.Tensor,
                           sin_freqs: torch.Tensor) -> torch.Tensor:
    """causal_rope.py:102-132 for x [B, T, H*D] and tables [B, H, T, D/2]."""
    if input_tensor.ndim != 3 or cos_freqs.ndim != 4:
        raise NotImplementedError("apply_split_rotary_emb takes x [B, T, H*D] with 4-D tables")
    B, T, HD = input_tensor.shape
    H = cos_freqs.shape[1]
    D = HD // H
    x = input_tensor if input_tensor.stride(-1) == 1 else input_tensor.contiguous()
    out = torch.empty_like(x)
    kernels.qk_rmsnorm_rope(x, out, None, None, (cos_freqs, sin_freqs), H, D)
    return out
