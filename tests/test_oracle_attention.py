"""Pins the attention oracle (CPU) against float64 textbook formulas and invariants."""
import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import rope as OR


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_rms_norm_full_row_vs_textbook():
    g = _g(0)
    x = torch.randn(2, 17, 512, generator=g) * 3
    w = 1 + 0.1 * torch.randn(512, generator=g)
    y = OA.rms_norm_full_row(x, w, 1e-6)
    ref = OA.rms_norm_f64(x.numpy(), w.numpy(), 1e-6)
    assert np.allclose(y.numpy(), ref, rtol=2e-6, atol=2e-6)
    # the norm runs over the full H*D row, not per head
    per_head = OA.rms_norm_f64(x.view(2, 17, 8, 64).numpy(), None, 1e-6).reshape(2, 17, 512)
    assert not np.allclose(OA.rms_norm_f64(x.numpy(), None, 1e-6), per_head, atol=1e-3)


@pytest.mark.parametrize("shape", [(1, 5, 2, 16, 7), (2, 64, 4, 64, 130), (1, 192, 8, 64, 768)])
def test_sdpa_vs_bruteforce_f64(shape):
    B, Lq, H, D, Lk = shape
    g = _g(1)
    q = torch.randn(B, Lq, H, D, generator=g)
    k = torch.randn(B, Lk, H, D, generator=g)
    v = torch.randn(B, Lk, H, D, generator=g)
    out = OA.standard_attention_forward(q, k, v)
    ref = OA.attention_f64(q.numpy(), k.numpy(), v.numpy())
    assert np.allclose(out.numpy(), ref, atol=2e-5)


def test_sdpa_planted_transpose_is_caught():
    """Using V in place of K (a swapped operand) must fail the brute-force check."""
    g = _g(2)
    q = torch.randn(1, 16, 2, 32, generator=g)
    k = torch.randn(1, 24, 2, 32, generator=g)
    v = torch.randn(1, 24, 2, 32, generator=g)
    ref = OA.attention_f64(q.numpy(), k.numpy(), v.numpy())
    bad = OA.standard_attention_forward(q, v, v)
    assert np.abs(bad.numpy() - ref).max() > 1e-2


def test_key_permutation_invariance_and_mask_equals_removal():
    g = _g(3)
    q = torch.randn(2, 32, 4, 64, generator=g)
    k = torch.randn(2, 100, 4, 64, generator=g)
    v = torch.randn(2, 100, 4, 64, generator=g)
    perm = torch.randperm(100, generator=g)
    a = OA.standard_attention_forward(q, k, v)
    b = OA.standard_attention_forward(q, k[:, perm], v[:, perm])
    assert torch.allclose(a, b, atol=1e-5)
    keep = torch.ones(2, 100, dtype=torch.int64)
    keep[:, 80:] = 0
    for dt in (torch.float32, torch.bfloat16):
        m = OA.prepare_attention_mask(keep, dt).float()        # (m-1)*finfo.max, [B,1,1,Lk]
        assert m.shape == (2, 1, 1, 100)
        masked = OA.standard_attention_forward(q, k, v, m)
        removed = OA.standard_attention_forward(q, k[:, :80], v[:, :80])
        assert torch.allclose(masked, removed, atol=1e-5)
    bm = keep.bool().view(2, 1, 1, 100)
    assert torch.allclose(OA.standard_attention_forward(q, k, v, bm),
                          OA.standard_attention_forward(q, k[:, :80], v[:, :80]), atol=1e-5)


def _weights(d, H, Dh, seed, gate=False):
    g = _g(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.02
    z = lambda n: torch.zeros(n)
    HD = H * Dh
    return OA.AttnWeights(r(HD, d), z(HD), r(HD, d), z(HD), r(HD, d), z(HD), r(d, HD), z(d),
                          torch.ones(HD), torch.ones(HD), H, Dh,
                          wg=r(H, d) if gate else None, bg=z(H) if gate else None)


def test_attention_with_cache_equals_full_attention():
    """cat(cache, new) attention equals attending over the concatenation computed directly,
    and the returned new K/V are the post-norm/post-RoPE keys at the chunk's positions."""
    H, Dh, d = 4, 64, 256
    w = _weights(d, H, Dh, 4, gate=True)
    g = _g(5)
    x_old = torch.randn(1, 2 * 12, d, generator=g)
    x_new = torch.randn(1, 12, d, generator=g)
    pe_old = OR.causal_precompute_freqs_cis((2, 3, 4), d, start_frame=0, num_attention_heads=H)
    pe_new = OR.causal_precompute_freqs_cis((1, 3, 4), d, start_frame=2, num_attention_heads=H)
    _, ck, cv = OA.attention_with_cache(w, x_old, None, pe_old, None, None, None)
    out, nk, nv = OA.attention_with_cache(w, x_new, None, pe_new, None, ck, cv)
    # direct: project / norm / rope the new chunk, attend over [old keys, new keys]
    q, k, v = OA.project_qkv(w, x_new, x_new)
    q, k = OA.norm_rope_qk(w, q, k, pe_new, None)
    assert torch.allclose(nk, k.view(1, 12, H, Dh)) and torch.allclose(nv, v.view(1, 12, H, Dh))
    att = OA.attention_f64(q.view(1, 12, H, Dh).numpy(), torch.cat([ck, nk], 1).numpy(),
                           torch.cat([cv, nv], 1).numpy())
    ref = OA.finish_output(w, torch.from_numpy(att).float(), x_new)
    assert torch.allclose(out, ref, atol=1e-5)
    # causality comes from the cache contents: no future chunk can be seen
    out_nocache, _, _ = OA.attention_with_cache(w, x_new, None, pe_new, None, None, None)
    assert not torch.allclose(out, out_nocache, atol=1e-4)


def test_gate_is_two_sigmoid():
    H, Dh, d = 2, 32, 64
    w = _weights(d, H, Dh, 6, gate=True)
    w.wg.zero_()   # zero-initialised gate -> 2*sigmoid(0) = 1: identity
    w0 = OA.AttnWeights(**{**w.__dict__, "wg": None, "bg": None})
    x = torch.randn(1, 5, d, generator=_g(7))
    o = torch.randn(1, 5, H, Dh, generator=_g(8))
    assert torch.allclose(OA.finish_output(w, o, x), OA.finish_output(w0, o, x))
