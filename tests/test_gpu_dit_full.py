"""The dual-stream denoising step at its real widths and shape: one
full-width block against the fp32 oracle, and the 48-block step's properties.

Shape (the 512x768 chunk, B = 2): video 4096 wide (32 x 128 heads), audio
2048 wide (32 x 64), 4x GELU FFNs; 1152 video queries (3 frames of 16x24)
over 3456 cached + 1152 keys, 75 audio queries over 600 cached + 75, 1024
text keys with the last 20 % padding for both streams, A2V 1152 x 75 and
V2A 75 x 1152 over the chunk's own tokens."""
import gc

import pytest
import torch

import taomate_amd as T
from oracle import attention as OA
from oracle import dit as OD
from oracle import rope as OR
from taomate_amd import dit as D
from taomate_amd import kernels
from taomate_amd.kv_cache import KVSpanView

from .helpers import cosine

pytestmark = pytest.mark.gpu

B, GH, GW, NF, F0 = 2, 16, 24, 3, 12
HW = GH * GW
LQ, LV_CACHE = NF * HW, 9 * HW            # 1152 queries over 3456 cached video keys
LA, LA_CACHE, A0, LT = 75, 600, 600, 1024


def _pes(cfg, dev=None):
    """(video, audio, video cross, audio cross) RoPE tables at the chunk's
    absolute positions; the oracle's fp32 tables when dev is None."""
    cross = cfg.audio_heads * cfg.audio_d_head
    if dev is None:
        pe = lambda grid, dim, heads, f0, audio=False: OR.causal_precompute_freqs_cis(
            grid, dim, start_frame=f0, num_attention_heads=heads, batch=B, is_audio=audio)
    else:
        pe = lambda grid, dim, heads, f0, audio=False: T.causal_precompute_freqs_cis(
            torch.tensor([list(grid)] * B), dim, start_frame=f0, device=dev, dtype=torch.bfloat16,
            num_attention_heads=heads, is_audio=audio)
    vcross = [t.repeat_interleave(HW, dim=2).contiguous() for t in pe((NF,), cross, cfg.audio_heads, F0)]
    return (pe((NF, GH, GW), cfg.video_dim, cfg.video_heads, F0),
            pe((LA,), cfg.audio_dim, cfg.audio_heads, A0, True), vcross,
            pe((LA,), cross, cfg.audio_heads, A0, True))


def _inputs(cfg, seed, layers):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).float()
    x = dict(video=r(B, LQ, cfg.in_channels), audio=r(B, LA, cfg.in_channels),
             sigma=torch.rand(B, generator=g), vctx=r(B, LT, cfg.video_dim), actx=r(B, LT, cfg.audio_dim))
    keep = torch.ones(B, LT, dtype=torch.int64)
    keep[:, int(0.8 * LT):] = 0
    x["mask"] = OA.prepare_attention_mask(keep, torch.bfloat16)
    x["cache"] = [dict(video_self_k=r(B, LV_CACHE, cfg.video_heads, cfg.video_d_head),
                       video_self_v=r(B, LV_CACHE, cfg.video_heads, cfg.video_d_head),
                       audio_self_k=r(B, LA_CACHE, cfg.audio_heads, cfg.audio_d_head),
                       audio_self_v=r(B, LA_CACHE, cfg.audio_heads, cfg.audio_d_head))
                  for _ in range(layers)]
    return x


def _arena_caches(dev, cfg, dense):
    """Each layer's dense caches in its own arenas, room for two more chunks."""
    specs = {"video_self": T.ArenaSpec(LV_CACHE + 2 * LQ, cfg.video_heads, cfg.video_d_head),
             "audio_self": T.ArenaSpec(LA_CACHE + 2 * LA + 16, cfg.audio_heads, cfg.audio_d_head)}
    kvc = T.init_kv_cache(len(dense), B, specs, dev)
    caches = []
    for lay, c in zip(kvc.layers, dense):
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        for arena, n, kk, vv in ((va, LV_CACHE, "video_self_k", "video_self_v"),
                                 (aa, LA_CACHE, "audio_self_k", "audio_self_v")):
            arena.slots("k", 0, n).copy_(c[kk].to(dev, torch.bfloat16))
            arena.slots("v", 0, n).copy_(c[vv].to(dev, torch.bfloat16))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, LV_CACHE)]),
                                     video_self_v=KVSpanView(va, "v", [(0, LV_CACHE)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, LA_CACHE)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, LA_CACHE)])))
    return caches


@pytest.mark.timeout(900)
def test_full_width_block_matches_oracle(dev):
    """One full-width block (about 0.47 B parameters) with the model's
    timestep modulation and output heads, against the fp32 oracle."""
    cfg = D.AVConfig(num_layers=1)
    model = D.build_model(cfg, dev, seed=3).fuse_qkv_()
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs(cfg, 61, 1)
    print("full-width block: oracle", flush=True)
    ref_v, ref_a = OD.forward_chunk(params, cfg, x["video"], x["audio"], x["sigma"], x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(cfg), x["cache"])
    caches = _arena_caches(dev, cfg, x["cache"])
    bf = lambda t: t.to(dev, torch.bfloat16)
    with torch.no_grad():
        vo, ao, _ = model.forward_chunk(bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]),
                                        bf(x["actx"]), bf(x["mask"]), bf(x["mask"]), *_pes(cfg, dev), caches)
    torch.cuda.synchronize()
    assert vo.shape == (B, LQ, cfg.out_channels) and ao.shape == (B, LA, cfg.out_channels)
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    rel = [((out.float().cpu() - ref).abs().max() / ref.abs().max()).item() for out, ref in ((vo, ref_v), (ao, ref_a))]
    print(f"full-width block: cosine video {cv:.6f} audio {ca:.6f}; max-abs / max |ref| {rel[0]:.2e} {rel[1]:.2e}",
          flush=True)
    # bf16 activations and weights against the fp32 oracle: measured cosines
    # 0.999975 / 0.999984 and largest errors 0.75 % / 0.43 % of the largest
    # output, so the bars leave a 4x margin on 1 - cos and 2x on the error
    assert cv >= 0.9999 and ca >= 0.9999, (cv, ca)
    for r in rel:
        assert r <= 1.5e-2, rel
    del model, caches
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_48_block_step_properties(dev):
    """The 48-block model (about 18.8 B parameters, bf16, random weights):
    one denoising step attends 288 times (6 attentions per block), its outputs
    are finite and leave the caches as given; the clean commit pass then
    appends exactly one chunk to every layer's caches (video 1152 and audio
    75 self keys, 75 A2V and 1152 V2A keys) and returns no outputs."""
    cfg = D.AVConfig()
    model = D.build_model(cfg, dev, seed=3).fuse_qkv_()
    assert len(model.transformer_blocks) == 48
    x = _inputs(cfg, 62, 1)
    dense = x["cache"] * cfg.num_layers          # the same cached keys in every layer
    caches = _arena_caches(dev, cfg, dense)
    bf = lambda t: t.to(dev, torch.bfloat16)
    args = (bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]),
            bf(x["mask"]), *_pes(cfg, dev))
    calls = []
    real = kernels.flash_attn

    def counting(q, segments, out, **kw):
        calls.append((tuple(q.shape), sum(s.k.shape[1] for s in segments)))
        return real(q, segments, out, **kw)

    kernels.flash_attn = counting
    try:
        with torch.no_grad():
            vo, ao, kept = model.forward_chunk(*args, caches)
            n_step = len(calls)
            _, _, committed = model.forward_chunk(*args[:2], torch.zeros_like(args[2]), *args[3:], caches,
                                                  kv_cache_only=True)
    finally:
        kernels.flash_attn = real
    torch.cuda.synchronize()
    assert n_step == 6 * 48, n_step
    per_block = sorted(set(calls[:6]))
    assert ((B, LQ, 32, 128), LV_CACHE + LQ) in per_block            # video self over cache + chunk
    assert ((B, LQ, 32, 128), int(0.8 * LT)) in per_block            # video text over the kept prefix
    assert ((B, LA, 32, 64), LA_CACHE + LA) in per_block             # audio self
    assert ((B, LQ, 32, 64), LA) in per_block and ((B, LA, 32, 64), LQ) in per_block   # A2V, V2A
    assert torch.isfinite(vo).all() and torch.isfinite(ao).all()
    assert all(k is c for k, c in zip(kept, caches))
    assert len(committed) == 48
    for c in committed:
        assert c.video_self_k.shape[1] == LV_CACHE + LQ and c.video_self_v.shape[1] == LV_CACHE + LQ
        assert c.audio_self_k.shape[1] == LA_CACHE + LA and c.audio_self_v.shape[1] == LA_CACHE + LA
        assert c.a2v_k.shape == (B, LA, 32, 64) and c.v2a_k.shape == (B, LQ, 32, 64)
    del model, caches, committed, kept
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.timeout(900)
def test_audio_stream_overlap_bit_identical(dev):
    """forward_chunk with the audio ops on their own HIP stream
    (AVModel.overlap_audio_) gives the one-stream outputs and committed
    caches bit for bit: 4 full-width blocks, a denoise step then a clean
    commit, each on fresh caches, the overlapped pass run twice."""
    cfg = D.AVConfig(num_layers=4)
    model = D.build_model(cfg, dev, seed=3).fuse_qkv_()
    x = _inputs(cfg, 63, 1)
    dense = x["cache"] * cfg.num_layers
    bf = lambda t: t.to(dev, torch.bfloat16)
    args = (bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]),
            bf(x["mask"]), *_pes(cfg, dev))
    fields = ("video_self_k", "video_self_v", "audio_self_k", "audio_self_v", "a2v_k", "a2v_v", "v2a_k", "v2a_v")

    def run(overlap):
        model.overlap_audio_(overlap)
        caches = _arena_caches(dev, cfg, dense)
        with torch.no_grad():
            vo, ao, _ = model.forward_chunk(*args, caches)
            _, _, committed = model.forward_chunk(*args[:2], torch.zeros_like(args[2]), *args[3:], caches,
                                                  kv_cache_only=True)
        torch.cuda.synchronize()
        dense_of = lambda t: t.materialize() if hasattr(t, "materialize") else t.clone()
        return vo, ao, [[dense_of(getattr(c, f)) for f in fields] for c in committed]

    ref = run(False)
    for i in range(2):
        print(f"audio stream overlap: pass {i}", flush=True)
        got = run(True)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), f"pass {i}: outputs differ"
        for layer, (g, r) in enumerate(zip(got[2], ref[2])):
            for f, a, b in zip(fields, g, r):
                assert torch.equal(a, b), f"pass {i}: layer {layer} {f} differs"
    model.overlap_audio_(False)
    del model
    gc.collect()
    torch.cuda.empty_cache()
