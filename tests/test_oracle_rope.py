"""Pins the RoPE oracle (CPU) against float64 closed forms, special cases and invariants."""
import math

import numpy as np
import pytest
import torch

from oracle import rope as OR

GRIDS = [
    ((3, 16, 24), 4096, 32, 12, False, [20, 2048, 2048]),
    ((2, 8, 12), 512, 8, 10, False, [20, 2048, 2048]),
    ((75,), 2048, 32, 600, True, [20]),
    ((3,), 2048, 32, 12, False, [20]),
    ((4, 16, 24), 4096, 32, 0, False, [20, 2048, 2048]),
]


def _closed(grid, dim, heads, sf, audio, mp):
    f = OR.freqs_closed_form_f64(grid, dim, start_frame=sf, is_audio=audio, max_pos=mp,
                                 num_attention_heads=heads)
    return f.transpose(1, 0, 2).reshape(f.shape[1], -1)  # [T, dim/2] incl. pad


@pytest.mark.parametrize("case", GRIDS, ids=lambda c: f"{c[0]}_{c[1]}")
def test_angles_match_float64_closed_form(case):
    grid, dim, heads, sf, audio, mp = case
    ang, pad = OR.rope_angles(grid, dim, start_frame=sf, is_audio=audio, max_pos=mp)
    ref = _closed(grid, dim, heads, sf, audio, mp)[:, pad:]
    rel = np.abs(ang.double().numpy() - ref) / np.maximum(np.abs(ref), 1e-3)
    assert rel.max() < 1e-6  # a few float32 ulps through pow/div/mul


@pytest.mark.parametrize("case", GRIDS, ids=lambda c: f"{c[0]}_{c[1]}")
def test_table_layout_and_pad(case):
    grid, dim, heads, sf, audio, mp = case
    cos, sin = OR.causal_precompute_freqs_cis(grid, dim, start_frame=sf, is_audio=audio, max_pos=mp,
                                              num_attention_heads=heads, batch=2)
    T = math.prod(grid)
    assert cos.shape == (2, heads, T, dim // 2 // heads)
    assert torch.equal(cos[0], cos[1])
    pad = dim // 2 - (dim // (2 * len(grid))) * len(grid)
    flat_c = cos[0].permute(1, 0, 2).reshape(T, -1)
    flat_s = sin[0].permute(1, 0, 2).reshape(T, -1)
    assert torch.all(flat_c[:, :pad] == 1) and torch.all(flat_s[:, :pad] == 0)
    ref = _closed(grid, dim, heads, sf, audio, mp)
    # |d cos| <= |d angle|: the float32 angle error bound carries over
    tol = np.abs(ref) * 1e-6 + 1e-6
    assert np.all(np.abs(flat_c.double().numpy() - np.cos(ref)) <= tol + 2e-7)
    assert np.all(np.abs(flat_s.double().numpy() - np.sin(ref)) <= tol + 2e-7)


def test_known_positions():
    # ind[0] = pi/2 and ind[-1] = theta * pi/2; geometric spacing
    f = OR.generate_freq_grid(10000.0, 3, 4096).double()
    assert f.numel() == 682
    assert abs(f[0].item() - math.pi / 2) < 1e-6
    assert abs(f[-1].item() / (math.pi / 2 * 10000) - 1) < 1e-6
    ratio = (f[1:] / f[:-1]).numpy()
    assert np.allclose(ratio, 10000 ** (1 / 681), rtol=1e-5)
    # video frame 0: pixel frames [0, 1) -> midpoint 0.5 / 24 s (causal fix clamps -7 to 0)
    frac = OR._fractional_positions((1, 1, 1), 0, False, [20, 2048, 2048])
    assert abs(frac[0, 0].item() - 0.5 / 24 / 20) < 1e-9
    assert abs(frac[0, 1].item() - 16 / 2048) < 1e-9
    # frame 12: pixel frames [89, 97) -> 93 / 24 s
    frac = OR._fractional_positions((1, 2, 3), 12, False, [20, 2048, 2048])
    assert abs(frac[0, 0].item() - 93 / 24 / 20) < 1e-7
    assert abs(frac[5, 2].item() - (32 * 2 + 16) / 2048) < 1e-9
    # audio latent frame 600: mel [2397, 2401) -> 2399 * 160 / 16000 s
    frac = OR._fractional_positions((1,), 600, True, [20])
    assert abs(frac[0, 0].item() - 2399 * 0.01 / 20) < 1e-7


def test_split_rotation_is_complex_multiply_and_keeps_norms():
    g = torch.Generator().manual_seed(0)
    B, T, H, D = 2, 48, 4, 64
    x = torch.randn(B, T, H * D, generator=g, dtype=torch.float64)
    cos, sin = OR.causal_precompute_freqs_cis((1, T, 1), H * D, start_frame=5, num_attention_heads=H,
                                              batch=B, dtype=torch.float64)
    y = OR.apply_split_rotary_emb(x, cos, sin)
    xr = x.view(B, T, H, D)
    yr = y.view(B, T, H, D)
    c = cos.permute(0, 2, 1, 3)
    s = sin.permute(0, 2, 1, 3)
    z = torch.complex(xr[..., :D // 2], xr[..., D // 2:]) * torch.complex(c, s)
    assert torch.allclose(yr[..., :D // 2], z.real, atol=1e-12)
    assert torch.allclose(yr[..., D // 2:], z.imag, atol=1e-12)
    n0 = xr[..., :D // 2] ** 2 + xr[..., D // 2:] ** 2
    n1 = yr[..., :D // 2] ** 2 + yr[..., D // 2:] ** 2
    assert torch.allclose(n0, n1, atol=1e-10)
    # sin = 0, cos = 1 is the identity
    assert torch.equal(OR.apply_split_rotary_emb(x, torch.ones_like(cos), torch.zeros_like(sin)), x)


def test_planted_sign_mistake_is_caught():
    """Flipping the sign of the sin term (a plausible mistake) breaks the complex-multiply check."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 8, 128, generator=g, dtype=torch.float64)
    cos, sin = OR.causal_precompute_freqs_cis((1, 8, 1), 128, start_frame=3, num_attention_heads=2,
                                              dtype=torch.float64)
    bad = OR.apply_split_rotary_emb(x, cos, -sin)
    good = OR.apply_split_rotary_emb(x, cos, sin)
    assert (bad - good).abs().max() > 1e-2


def test_ntk_theta():
    assert OR.ntk_theta(10000.0, 4096, 3, 12, False, "off", 8.0) == 10000.0
    # 15 latent frames -> pixel end 113 -> 4.708 s < 8 s: unchanged
    assert OR.ntk_theta(10000.0, 4096, 3, 12, False, "ntk", 8.0) == 10000.0
    t = OR.ntk_theta(10000.0, 4096, 3, 97, False, "ntk", 8.0)   # 100 frames -> 793/24 s
    r = (100 * 8 + 1 - 8) / 24 / 8.0
    assert abs(t / (10000.0 * r ** (4096 / 4094)) - 1) < 1e-12
    with pytest.raises(ValueError):
        OR.ntk_theta(10000.0, 4096, 3, 0, False, "yarn", 8.0)
