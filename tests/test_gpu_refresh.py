"""GPU parity of the prompt-change refresh of a retained cache
(_refresh_conditioning_cache, taomate/inference/runtime.py:386-470) at a
reduced width on the 16x24 grid, B = 1: after a first window under prompt A
and the retention of the sink block and the 2 most recent blocks, the cache
is refreshed under prompt B.  The refreshed audio self, A2V and V2A K/V
equal a fresh fp32 prefill of those blocks under prompt B at their global
positions; the video self K/V are the same views, bit for bit."""
import pytest
import torch

import taomate_amd as T
from oracle import runtime as ORT
from taomate_amd import dit as D
from taomate_amd import runtime as RT

from .helpers import cosine
from .test_gpu_runtime import NoiseTape

pytestmark = pytest.mark.gpu

GRID, C = (16, 24), 128
FIELDS = ("audio_self_k", "audio_self_v", "a2v_k", "a2v_v", "v2a_k", "v2a_v")


def _cond(cfg, seed, dev=None):
    g = torch.Generator().manual_seed(seed)
    keep = torch.ones(1, 16, dtype=torch.int64)
    keep[:, -3:] = 0
    c = dict(video_context=torch.randn(1, 16, cfg.video_dim, generator=g).to(torch.bfloat16).float(),
             audio_context=torch.randn(1, 16, cfg.audio_dim, generator=g).to(torch.bfloat16).float(),
             video_context_mask=keep, audio_context_mask=keep)
    if dev is None:
        return c
    return {k: (v.to(dev, torch.bfloat16) if torch.is_floating_point(v) else v.to(dev)) for k, v in c.items()}


def _dense(t):
    return t.materialize() if isinstance(t, T.KVSpanView) else t


@pytest.mark.timeout(900)
def test_prompt_change_refresh_matches_fresh_prefill(dev):
    cfg = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                     audio_d_head=64)
    model = D.build_model(cfg, dev, seed=9)
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    gen = RT.StreamingGenerator(model, GRID, noise=NoiseTape(8), arena_plan=T.ArenaPlan.for_stream(GRID))
    lat = {}
    with torch.no_grad():
        gen.generate_first_window((1, 16, C, *GRID), (1, 126, C), _cond(cfg, 81, dev), None,
                                  block_callback=lambda v, a, b: lat.__setitem__(b.block_idx, (v, a)))
        cache = T.retain_streaming_context(gen.last_cache)
    gen.last_cache = None
    assert [s["block_idx"] for s in cache.segments] == [0, 3, 4]
    prefix_v = torch.cat([lat[i][0] for i in (0, 3, 4)], dim=1)
    prefix_a = torch.cat([lat[i][1] for i in (0, 3, 4)], dim=1)
    assert prefix_v.shape[1] == 10 and prefix_a.shape[1] == 76
    before = [{f: _dense(getattr(l, f)).clone() for f in ("video_self_k", "video_self_v") + FIELDS}
              for l in cache.layers]
    views = [(l.video_self_k, l.video_self_v) for l in cache.layers]
    cond_b = _cond(cfg, 82)
    with torch.no_grad():
        out = gen.refresh_conditioning_cache(cache, _cond(cfg, 82, dev), prefix_v, prefix_a, (1, 15, C, *GRID))
    torch.cuda.synchronize()
    assert out is cache and [s["block_idx"] for s in cache.segments] == [0, 3, 4]
    orc = ORT.StreamOracle(params, cfg, GRID, noise=None)
    ref = orc.rebuild_for_prompt(cache.segments, cond_b, prefix_v.float().cpu(), prefix_a.float().cpu(), 15)
    for i, l in enumerate(cache.layers):
        # video self: the same views and bytes (pinned)
        assert l.video_self_k is views[i][0] and l.video_self_v is views[i][1]
        assert torch.equal(_dense(l.video_self_k), before[i]["video_self_k"])
        assert torch.equal(_dense(l.video_self_v), before[i]["video_self_v"])
        for f in FIELDS:
            got = _dense(getattr(l, f)).float().cpu()
            want = ref[i][f]
            assert got.shape == want.shape, (i, f)
            c = cosine(got, want)
            err = (got - want).abs().max().item()
            print(f"layer {i} {f}: cosine {c:.6f} max-abs {err:.3e}", flush=True)
            assert c >= 0.9999, (i, f, c)
            assert err <= 2e-2 * max(1.0, want.abs().max().item()), (i, f, err)
            # the new prompt reaches every refreshed field but layer 0's audio
            # self K/V, which come before any text cross-attention
            moved = (got - before[i][f].float().cpu()).abs().max().item()
            if i > 0 or not f.startswith("audio_self"):
                assert moved > 1e-3, (i, f, moved)
