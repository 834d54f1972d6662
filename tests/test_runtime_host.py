"""CPU checks of the stream loop's host arithmetic: the denoising schedule
(ltx_core/components/schedulers.py:21-57, model.py:11-19) pinned by its special
cases, the product's schedule and helpers against the oracle, and the
patchify layout round trip."""
import math

import pytest
import torch

from oracle import runtime as ORT
from taomate_amd import runtime as RT


def test_schedule_special_cases():
    """First value 1, last non-zero value the terminal 0.1, then 0; strictly
    decreasing; the un-stretched midpoint is sigmoid(shift), with shift 2.05
    at 4096 tokens and 0.95 at 1024 (a slip in the shift line or the stretch
    moves these)."""
    s = ORT.schedule(40).double()
    assert s[0].item() == 1.0 and s[-1].item() == 0.0
    assert abs(s[-2].item() - 0.1) < 1e-6
    assert bool((s[1:] < s[:-1]).all())
    for tokens, shift in ((4096, 2.05), (1024, 0.95)):
        raw = ORT.schedule(2, tokens=tokens, terminal=0.0).double()   # terminal 0: stretch leaves 1 - z unscaled
        # with 2 steps: values at t = 1, 0.5, 0; stretch divides 1 - s by (1 - s_mid) / 1
        mid = 1.0 / (1.0 + math.exp(-shift))
        assert raw[0].item() == 1.0 and abs(raw[1].item()) < 1e-7   # stretched to the terminal 0
        s40 = ORT.schedule(40, tokens=tokens).double()
        z = 1.0 - s40[:-1]
        # before the stretch, 1 - s at t = 0.5 is 1 - sigmoid(shift); the stretch is a common scale
        unstretched_mid = 1.0 - math.exp(shift) / (math.exp(shift) + 1.0)
        unstretched_last = 1.0 - math.exp(shift) / (math.exp(shift) + 39.0)
        assert abs(z[20].item() / z[-1].item() - unstretched_mid / unstretched_last) < 1e-6
        assert abs(mid - (1.0 - unstretched_mid)) < 1e-12
    sig = ORT.denoising_sigmas()
    assert sig[0].item() == 1.0 and sig[-1].item() == 0.0
    full = ORT.schedule(40)
    for t, v in zip((757, 522), sig[1:3].tolist()):
        assert abs(v - t / 1000.0) == min(abs(x - t / 1000.0) for x in full.tolist())


def test_product_schedule_and_helpers_match_oracle():
    torch.testing.assert_close(RT.ltx2_schedule(), ORT.schedule(), rtol=0, atol=1e-6)
    torch.testing.assert_close(RT.denoising_sigmas(), ORT.denoising_sigmas(), rtol=0, atol=1e-6)
    g = torch.Generator().manual_seed(1)
    x0, n, v = (torch.randn(2, 3, 4, 5, 6, generator=g) for _ in range(3))
    s = torch.tensor([0.25, 0.75])
    torch.testing.assert_close(RT.add_noise(x0, n, s), ORT.add_noise(x0, n, s))
    torch.testing.assert_close(RT.velocity_to_x0(x0, v, s), ORT.velocity_to_x0(x0, v, s))
    assert torch.allclose(RT.add_noise(x0, n, torch.zeros(2)), x0) and torch.allclose(RT.add_noise(x0, n, torch.ones(2)), n)
    anchor = ORT.channel_stats(n)
    got = RT.apply_renorm(x0, anchor, 1.0)
    torch.testing.assert_close(got, ORT.apply_renorm(x0, anchor, 1.0))
    m, sd = ORT.channel_stats(got)
    torch.testing.assert_close(m, anchor[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(sd, anchor[1], rtol=1e-5, atol=1e-5)


def test_patchify_layout_round_trip():
    """[B, F, C, H, W] -> tokens in (frame, row, column) order with channels last,
    as forward_inference's permute/reshape (kv_cache.py:2770-2772), and back."""
    B, F, C, H, W = 2, 3, 4, 5, 6
    lat = torch.arange(B * F * C * H * W, dtype=torch.float32).view(B, F, C, H, W)
    tok = RT.video_tokens(lat)
    ref = lat.permute(0, 2, 1, 3, 4).reshape(B, C, -1).permute(0, 2, 1)
    assert torch.equal(tok, ref)
    assert torch.equal(tok[1, (2 * H + 3) * W + 4], lat[1, 2, :, 3, 4])
    assert torch.equal(RT.video_latent(tok, F, (H, W)), lat)


def test_mask_preparation():
    m = torch.tensor([[1, 1, 0]])
    out = RT.prepare_attention_mask(m, torch.bfloat16)
    assert out.shape == (1, 1, 1, 3) and out[0, 0, 0, 0].item() == 0.0
    assert out[0, 0, 0, 2].item() == -torch.finfo(torch.bfloat16).max
    f = torch.zeros(1, 1, 1, 3)
    assert RT.prepare_attention_mask(f, torch.bfloat16) is f


def test_prepared_mask_kept_per_mask_tensor():
    """The loop prepares a conditioning mask once: the same object while the
    mask tensor is unchanged, a new one after an in-place change."""
    gen = RT.StreamingGenerator(object(), (4, 6))
    m = torch.tensor([[1, 1, 0, 0]])
    a = gen._prepared_mask(m, torch.bfloat16)
    assert gen._prepared_mask(m, torch.bfloat16) is a
    torch.testing.assert_close(a, RT.prepare_attention_mask(m, torch.bfloat16))
    m[0, 2] = 1
    b = gen._prepared_mask(m, torch.bfloat16)
    assert b is not a and b[0, 0, 0, 2].item() == 0.0
    assert gen._prepared_mask(None, torch.bfloat16) is None


def _cpu_kernels(monkeypatch):
    """Shape-correct stand-ins for the HIP entry points, so the loop's cache
    bookkeeping runs on the CPU (values are not checked here)."""
    from taomate_amd import kernels

    def rope_table(freq, grid, start, audio, max_pos, dim, heads, batch, dtype):
        T_ = math.prod(grid)
        per = dim // 2 // heads
        return torch.ones(batch, heads, T_, per, dtype=dtype), torch.zeros(batch, heads, T_, per, dtype=dtype)

    def qk(q_in, q_out, *a, k_in=None, k_out=None, v_in=None, v_out=None, **kw):
        q_out.copy_(q_in)
        if k_out is not None:
            k_out.copy_(k_in.view(k_out.shape))
        if v_out is not None:
            v_out.copy_(v_in.view(v_out.shape))

    def adaln(x, y=None, gate=None, x_out=None, n_out=None, **kw):
        if x_out is not None:
            x_out.copy_(x if y is None else x + y)
        if n_out is not None:
            n_out.copy_(x)

    monkeypatch.setattr(kernels, "rope_table", rope_table)
    monkeypatch.setattr(kernels, "rope_table_retime", lambda src, *a, **k: (src[0].clone(), src[1].clone()))
    monkeypatch.setattr(kernels, "qk_rmsnorm_rope", qk)
    monkeypatch.setattr(kernels, "flash_attn", lambda q, segs, out, **kw: out.zero_())
    monkeypatch.setattr(kernels, "adaln", adaln)
    monkeypatch.setattr(kernels, "kv_append", lambda src, dst, *a, **k: dst.copy_(src))


def test_stream_loop_arena_bookkeeping_on_cpu(monkeypatch):
    """Four windows of the loop on module arenas: after the first window all 16
    frames are cached; in the next windows every retention leaves exactly the
    sink block and the 2 most recent blocks' slots busy (no slot is pinned by
    a view nobody holds), segments follow the eviction rule, and the caller's
    cache object is left as it was."""
    import taomate_amd as T
    from taomate_amd import dit as D
    _cpu_kernels(monkeypatch)
    cfg = D.AVConfig(num_layers=1, video_dim=128, audio_dim=64, video_heads=2, audio_heads=1, video_d_head=64,
                     audio_d_head=64)
    model = D.build_model(cfg, "cpu", seed=7)
    grid = (2, 4)
    hw = grid[0] * grid[1]
    gen = RT.StreamingGenerator(model, grid, noise=lambda s, d, t: torch.zeros(s, dtype=t),
                                arena_plan=T.ArenaPlan.for_stream(grid))
    keep = torch.ones(1, 4, dtype=torch.int64)
    cond = dict(video_context=torch.zeros(1, 4, 128, dtype=torch.bfloat16),
                audio_context=torch.zeros(1, 4, 64, dtype=torch.bfloat16), video_context_mask=keep,
                audio_context_mask=keep)
    arena = lambda: model.transformer_blocks[0].attn1.__dict__["_ltx_arena"]
    busy = lambda: sum(b - a for a, b in arena().live_intervals())
    with torch.no_grad():
        gen.generate_first_window((1, 16, 128, *grid), (1, 126, 128), cond, None)
        cache = gen.last_cache
        assert [s["block_idx"] for s in cache.segments] == [0, 1, 2, 3, 4]
        assert busy() == 16 * hw
        real = RT.retain_streaming_context
        seen = []

        def rec(c):
            out = real(c)
            seen.append(([s["block_idx"] for s in out.segments], out.layers[0].video_self_k.shape[1]))
            return out

        monkeypatch.setattr(RT, "retain_streaming_context", rec)
        for w in range(3):
            before = [s["block_idx"] for s in cache.segments]
            gen.generate_next_window((1, 15, 128, *grid), (1, 125, 128), cond, None, cache, 5 + 5 * w)
            assert [s["block_idx"] for s in cache.segments] == before     # caller's object untouched
            gen.last_cache, cache = None, gen.last_cache
            assert busy() == (4 + 3 + 3) * hw                              # sink + 2 recent only
    for i, (blocks, vlen) in enumerate(seen):
        b = 5 + i
        assert blocks == [0, b - 1, b] and vlen == (4 + 6) * hw
