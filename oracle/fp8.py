"""fp8-e4m3 KV quantisation restatement (oracle; test infrastructure only).

The reference has no fp8 KV cache (its only fp8 use is weight dtypes,
ltx_causal/tensor_parallel.py:43-59); this is the build-side extension the
long-stream workload asks for: one scale per (batch, head, frame) of
``frame_tokens`` tokens, ``scale = absmax / 448`` (1 when absmax is 0),
codes ``= e4m3fn(x / scale)`` with round-to-nearest-even and saturation at 448.
torch's float8_e4m3fn cast (RNE) is the encoder after clamping to +-448.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0


def quantize_kv(x: torch.Tensor, frame_tokens: int):
    """x [B, L, H, D] float -> (codes uint8 [B, L, H, D], scales float32 [B, H, L/frame])."""
    B, L, H, D = x.shape
    assert L % frame_tokens == 0
    xf = x.to(torch.float32)
    fr = xf.reshape(B, L // frame_tokens, frame_tokens, H, D)
    amax = fr.abs().amax(dim=(2, 4))                              # [B, nF, H]
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = fr / scale[:, :, None, :, None]
    q = q.clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    codes = q.view(torch.uint8).reshape(B, L, H, D)
    return codes, scale.permute(0, 2, 1).contiguous()            # [B, H, nF]


def dequantize_kv(codes: torch.Tensor, scales: torch.Tensor, frame_tokens: int) -> torch.Tensor:
    """Inverse of quantize_kv: float32 [B, L, H, D]."""
    B, L, H, D = codes.shape
    v = codes.view(torch.float8_e4m3fn).to(torch.float32).reshape(B, L // frame_tokens, frame_tokens, H, D)
    s = scales.permute(0, 2, 1)[:, :, None, :, None]
    return (v * s).reshape(B, L, H, D)


def e4m3_value(code: int) -> float:
    """Decode one e4m3fn code from the format definition (float64)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 7
    if e == 0xF and m == 7:
        return float("nan")
    if e == 0:
        return s * m * 2.0 ** -9
    return s * (1 + m / 8) * 2.0 ** (e - 7)
