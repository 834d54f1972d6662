"""Pins of the dual-stream block oracle's building blocks against closed forms
and special cases (CPU).  Each check is chosen so that a plausible slip in the
restatement fails it:

* timestep sinusoid (compat.py:76-106, flip_sin_to_cos=True,
  downscale_freq_shift=0): cosines first; at t = 0 the cosines are 1 and the
  sines 0; the first frequency is 1 and the last max_period^-(half-1)/half
  (a shift of 1 would make it 1/max_period);
* feed-forward (compat.py:46-71): tanh-approximated GELU, whose value at 1 is
  0.8411919906 (exact GELU gives 0.8413447461);
* learned-memory attention (causal_block.py:136-160): over one memory token
  the softmax weight is 1, so every query's output is to_out(W_v m) whatever
  the queries and W_q, W_k are; swapped key / value projections fail it;
* colour FiLM (causal_block.py:179-193): the projection splits into (scale,
  shift) in that order, applied as x * scale + shift.
"""
import math

import torch

from oracle import dit as OD


def test_timestep_embedding_closed_forms():
    half = 128
    e0 = OD.timestep_embedding(torch.zeros(3))
    assert e0.shape == (3, 2 * half)
    assert torch.equal(e0[:, :half], torch.ones(3, half))
    assert torch.equal(e0[:, half:], torch.zeros(3, half))
    t = torch.tensor([1.0, 250.0, 999.0])
    e = OD.timestep_embedding(t).double()
    for i, tv in enumerate(t.tolist()):
        assert abs(e[i, 0].item() - math.cos(tv)) < 1e-5
        assert abs(e[i, half].item() - math.sin(tv)) < 1e-5
        f_last = 10000.0 ** (-(half - 1) / half)
        assert abs(e[i, half - 1].item() - math.cos(tv * f_last)) < 1e-4
        assert abs(e[i, 2 * half - 1].item() - math.sin(tv * f_last)) < 1e-4


def test_feed_forward_is_tanh_gelu():
    d = 4
    eye = torch.eye(d)
    p = {"ff.net.0.proj.weight": eye, "ff.net.0.proj.bias": torch.zeros(d), "ff.net.2.weight": eye,
         "ff.net.2.bias": torch.zeros(d)}
    x = torch.tensor([[1.0, 0.0, -1.0, 3.0]])
    y = OD.feed_forward(p, "ff.", x)
    assert abs(y[0, 0].item() - 0.8411919906) < 1e-6
    assert y[0, 1].item() == 0.0
    assert abs(y[0, 2].item() - (0.8411919906 - 1.0)) < 1e-6   # gelu(-x) = gelu(x) - x
    assert abs(y[0, 0].item() - 0.8413447461) > 1e-4           # not the exact erf form


def test_memory_attention_over_one_token_is_the_value_projection():
    g = torch.Generator().manual_seed(5)
    B, L, qd, md, heads = 2, 7, 48, 64, 8
    r = lambda *s: torch.randn(*s, generator=g)
    p = {"m.to_q.weight": r(md, qd), "m.to_k.weight": r(md, md), "m.to_v.weight": r(md, md),
         "m.to_out.weight": r(qd, md), "m.to_out.bias": r(qd)}
    x, mem = r(B, L, qd), r(B, 1, md)
    y = OD.memory_attention(p, "m.", x, mem, heads)
    want = (mem[:, 0] @ p["m.to_v.weight"].T) @ p["m.to_out.weight"].T + p["m.to_out.bias"]
    torch.testing.assert_close(y, want[:, None].expand(B, L, qd), rtol=1e-5, atol=1e-5)
    # a one-token memory shared by the batch broadcasts
    y1 = OD.memory_attention(p, "m.", x, mem[:1], heads)
    torch.testing.assert_close(y1[1], want[0].expand(L, qd), rtol=1e-5, atol=1e-5)


def test_color_film_scale_then_shift():
    d, cd, hd = 6, 4, 5
    p = {"f.net.0.weight": torch.zeros(hd, cd), "f.net.0.bias": torch.zeros(hd),
         "f.net.2.weight": torch.zeros(2 * d, hd),
         "f.net.2.bias": torch.cat([torch.full((d,), 2.0), torch.full((d,), 3.0)])}
    x = torch.randn(2, 3, d)
    y = OD.color_film(p, "f.", x, torch.randn(2, cd))
    torch.testing.assert_close(y, 2.0 * x + 3.0)
