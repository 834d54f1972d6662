"""GPU parity of the model-level stream loop against the fp32 oracle loop at a
reduced width (2 blocks, video 8 x 64 heads, audio 4 x 64, learned-memory
adapters on block 1) on the 16x24 latent grid, B = 1:

* the first window: block 0 (4 frames, 26 audio) denoised in 3 steps on an
  empty cache, then blocks 1-4 (3 frames, 25 audio), each committed clean with
  no pruning (16 frames, 6144 video keys cached);
* the next window: blocks 5-9 at their global positions, each denoised over
  the retained context, committed, fed to the memory and cut back to the sink
  block plus the 2 most recent.

Every block's latents are compared with the oracle's, the segment list after
each retention bit for bit with the committed eviction plan, and the final
caches with the oracle's."""
import json
import os

import pytest
import torch

import taomate_amd as T
from oracle import memory as OM
from oracle import runtime as ORT
from taomate_amd import dit as D
from taomate_amd import runtime as RT

from .helpers import cosine

pytestmark = pytest.mark.gpu

GRID = (16, 24)
C = 128


class NoiseTape:
    """The same Gaussian sequence for both loops (bf16-representable values)."""

    def __init__(self, seed):
        self.g = torch.Generator().manual_seed(seed)

    def __call__(self, shape, device=None, dtype=None):
        x = torch.randn(shape, generator=self.g).to(torch.bfloat16)
        return x.to(device) if device is not None else x.float()


def _seg(s):
    return {k: s[k] for k in ("block_idx", "video_tokens", "audio_tokens")}


@pytest.mark.timeout(900)
def test_two_windows_match_oracle(dev):
    cfg = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                     audio_d_head=64, learned_memory_enabled=True, learned_memory_layer_interval=2,
                     learned_memory_color_film_enabled=True)
    model = D.build_model(cfg, dev, seed=7)
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    g = torch.Generator().manual_seed(71)
    keep = torch.ones(1, 16, dtype=torch.int64)
    keep[:, -4:] = 0
    cond_cpu = dict(video_context=torch.randn(1, 16, cfg.video_dim, generator=g).to(torch.bfloat16).float(),
                    audio_context=torch.randn(1, 16, cfg.audio_dim, generator=g).to(torch.bfloat16).float(),
                    video_context_mask=keep, audio_context_mask=keep)
    cond = {k: (v.to(dev, torch.bfloat16) if torch.is_floating_point(v) else v.to(dev)) for k, v in cond_cpu.items()}

    gen = RT.StreamingGenerator(model, GRID, noise=NoiseTape(5), arena_plan=T.ArenaPlan.for_stream(GRID))
    orc = ORT.StreamOracle(params, cfg, GRID, noise=NoiseTape(5), memory=OM.MemoryOracle())
    memory = T.StreamingMemory()
    got = []
    cb = lambda v, a, blk: got.append((blk.block_idx, v.float().cpu(), a.float().cpu()))

    print("loop: first window", flush=True)
    gen.generate_first_window((1, 16, C, *GRID), (1, 126, C), cond, memory, block_callback=cb)
    ref = orc.first_window(1, C, cond_cpu)
    cache = gen.last_cache
    assert [_seg(s) for s in cache.segments] == orc.segments
    assert all(s["kind"] == "generated" and s["window_slot"] == i for i, s in enumerate(cache.segments))
    assert cache.layers[0].video_self_k.shape[1] == 16 * GRID[0] * GRID[1]       # no pruning
    assert isinstance(cache.layers[0].video_self_k, T.KVSpanView)                 # arena-backed from block 0

    print("loop: next window", flush=True)
    retained = []
    real_retain = RT.retain_streaming_context

    def recording(c):
        out = real_retain(c)
        retained.append(([_seg(s) for s in out.segments], out.layers[0].video_self_k.shape[1]))
        return out

    RT.retain_streaming_context = recording
    try:
        gen.generate_next_window((1, 15, C, *GRID), (1, 125, C), cond, memory, cache, 5, block_callback=cb)
    finally:
        RT.retain_streaming_context = real_retain
    ref += orc.next_window(1, C, cond_cpu, 5)

    with open(os.path.join(os.path.dirname(__file__), "golden", "eviction_plan_16x24_60.json")) as f:
        plan = json.load(f)
    assert len(retained) == 5
    for i, (segs, vlen) in enumerate(retained):
        assert segs == plan[5 + i]["segments"], 5 + i
        assert vlen == plan[5 + i]["video_len"], 5 + i
    assert [_seg(s) for s in gen.last_cache.segments] == orc.segments

    assert [b for b, _, _ in got] == list(range(10))
    worst = 1.0
    for (bi, v, a), (blk, rv, ra) in zip(got, ref):
        assert blk[0] == bi and v.shape == rv.shape and a.shape == ra.shape
        cv, ca = cosine(v, rv), cosine(a, ra)
        worst = min(worst, cv, ca)
        print(f"block {bi}: cosine video {cv:.6f} audio {ca:.6f}", flush=True)
        assert cv >= 0.999 and ca >= 0.999, (bi, cv, ca)
        # and elementwise: within 3 % of the block's range (bf16 GEMMs and
        # attention over three denoise steps and the commit)
        for out, r in ((v, rv), (a, ra)):
            err = (out.float() - r).abs().max().item()
            assert err <= 3e-2 * r.abs().max().item(), (bi, err)
    last = gen.last_cache.layers[1]
    for f in ("video_self_k", "video_self_v", "audio_self_k", "a2v_v", "v2a_k"):
        t = getattr(last, f)
        t = t.materialize() if isinstance(t, T.KVSpanView) else t
        assert t.shape == orc.layers[1][f].shape, f
        assert cosine(t, orc.layers[1][f]) >= 0.999, f
    print(f"loop: worst block cosine {worst:.6f}", flush=True)
