"""CPU checks of the learned long-memory state: the oracle's pooling,
resampling and gate against what their definitions fix, then the product's
PyTorch state machine (StreamingMemory settings) against the float64 oracle
over a short stream of chunks."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import memory as OM
from taomate_amd.memory import LearnedMemoryState, StreamingMemory, summarize_audio_memory, \
    summarize_video_memory


def test_oracle_pooling_and_resampling_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 3, 16, 24))
    # divisible sizes: block means
    ref = x.reshape(2, 3, 4, 4, 6, 4).mean(axis=(3, 5))
    assert np.allclose(OM.adaptive_avg_pool_2d(x, 4, 6), ref, atol=1e-12)
    # 1-D non-divisible: windows [floor(i n/m), ceil((i+1) n/m)) of 5 -> 3: [0,2) [1,4) [3,5)
    v = np.arange(5.0)
    assert np.allclose(OM.adaptive_avg_pool_1d(v, 3), [0.5, 2.0, 3.5])
    # bilinear of a plane a*i + b*j (align_corners=False): interior samples are exact,
    # edges clamp to the first/last source sample
    g = np.add.outer(2.0 * np.arange(4), 3.0 * np.arange(4))[None, None]
    up = OM.bilinear(g, 8, 8)[0, 0]
    for i in range(1, 7):
        for j in range(1, 7):
            si, sj = (i + 0.5) / 2 - 0.5, (j + 0.5) / 2 - 0.5
            assert abs(up[i, j] - (2 * si + 3 * sj)) < 1e-12
    assert up[0, 0] == g[0, 0, 0, 0]
    # a planted off-by-half in the sample position is caught
    bad = OM._bilinear_axis(np.arange(4.0)[None], 8)
    assert not np.allclose(bad, np.clip((np.arange(8) + 0.5) / 2, 0, 3) * 1.0)


def test_oracle_gate_and_ema_closed_forms():
    assert OM.gate(0.05, 0.05, 0.1, 0.1) == pytest.approx(0.1 + 0.9 * 0.5)
    assert OM.gate(10.0, 0.05, 0.1, 0.1) == pytest.approx(1.0)
    assert OM.gate(-10.0, 0.05, 0.1, 0.1) == pytest.approx(0.1)
    assert OM.gate(0.0, 0.05, 0.0, 0.3) == 0.3
    prev, anc, cur = np.full(3, 2.0), np.zeros(3), np.full(3, 4.0)
    # (2 * 0.85 + 4 * 0.15) * 0.8 + 0 * 0.2
    assert np.allclose(OM.ema(prev, anc, cur, 0.15, 0.2), 1.84)
    assert np.allclose(OM.ema(None, anc, cur, 0.15, 0.2), cur)


def test_oracle_token_summaries_properties():
    rng = np.random.default_rng(1)
    lat = rng.standard_normal((2, 3, 8, 16, 24)) * 3 + 5
    tok = OM.video_tokens(lat)
    assert tok.shape == (2, 24, 8)
    # pooling preserves the mean of the standardised map: every channel's tokens average to 0
    assert np.allclose(tok.mean(axis=1), 0.0, atol=1e-12)
    # a constant latent: the std clamps at eps and every token is 0
    assert np.allclose(OM.video_tokens(np.ones((1, 2, 4, 8, 8))), 0.0)
    aud = rng.standard_normal((2, 100, 8))
    at = OM.audio_tokens(aud, 64)
    assert at.shape == (2, 64, 8)
    assert np.allclose(OM.audio_tokens(aud, 100), (aud - aud.mean(1, keepdims=True)) / aud.std(1, keepdims=True))
    # cosine of a tensor with itself is 1, with its negation -1
    assert OM.token_cosine(tok, tok, 1e-6) == pytest.approx(1.0)
    assert OM.token_cosine(tok, -tok, 1e-6) == pytest.approx(-1.0)


def test_summaries_match_oracle():
    g = torch.Generator().manual_seed(2)
    lat = torch.randn(2, 3, 128, 16, 24, generator=g) * 2 + 1
    aud = torch.randn(2, 25, 128, generator=g)
    assert torch.allclose(summarize_video_memory(lat).double(), torch.from_numpy(OM.video_tokens(lat.numpy())),
                          atol=2e-5)
    assert torch.allclose(summarize_audio_memory(aud).double(), torch.from_numpy(OM.audio_tokens(aud.numpy())),
                          atol=2e-5)


def test_streaming_memory_matches_oracle_over_a_stream():
    g = torch.Generator().manual_seed(3)
    prod, orc = StreamingMemory(), OM.MemoryOracle()
    base = torch.randn(1, 1, 128, 16, 24, generator=g)
    gates = []
    for i in range(5):
        v = base + 0.3 * i * torch.randn(2, 3, 128, 16, 24, generator=g)
        a = torch.randn(2, 25, 128, generator=g)
        if i == 0:
            prod.set_reference(v, a)
            orc.set_reference(v.numpy(), a.numpy())
        cv = prod.apply_color_memory(v)
        assert torch.allclose(cv.double(), torch.from_numpy(orc.apply_color(v.numpy())), atol=5e-5)
        prod.update(v, a)
        orc.update(v.numpy(), a.numpy())
        gates.append(prod.video_last_update_gate)
        assert prod.video_last_update_gate == pytest.approx(orc.last_gate, abs=1e-5)
        cond = prod.with_conditional_memory({"prompt": 1})
        ref = orc.conditioning()
        assert cond["prompt"] == 1
        for key in ("learned_memory_video", "learned_memory_audio", "learned_memory_color"):
            assert torch.allclose(cond[key].double(), torch.from_numpy(ref[key]), atol=5e-5), (i, key)
    assert cond["learned_memory_video"].shape == (2, 48, 128)   # identity anchor 24 + EMA 24
    assert cond["learned_memory_audio"].shape == (2, 64, 128)
    assert cond["learned_memory_color"].shape == (2, 512)
    assert min(gates) < 1.0   # the drift gate engaged as the chunks moved away from the anchor


def test_disabled_state_is_inert():
    s = LearnedMemoryState()
    s.update(torch.randn(1, 2, 4, 8, 8), torch.randn(1, 5, 4))
    assert s.video is None and s.with_conditional_memory({"a": 1}) == {"a": 1}
    assert s.apply_color_memory(torch.ones(1)) is not None
