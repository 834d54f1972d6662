"""GPU parity of the dual-stream block stack (AdaLN-modulated video self,
video text, audio self, audio text, A2V, V2A attention and the GELU FFNs,
timestep modulation and output heads) against the fp32 oracle restatement,
at a reduced width: 2 blocks, video 8 x 64 heads, audio 4 x 64 heads, a
4x6 latent grid, 3-frame chunk over 6 cached frames, 10 audio tokens over 40
cached, 16 text tokens with the last 4 masked, B = 2."""
import pytest
import torch

from oracle import attention as OA
from oracle import dit as OD
from oracle import rope as OR
import taomate_amd as T
from taomate_amd import dit as D
from taomate_amd.kv_cache import KVSpanView

from .helpers import cosine

pytestmark = pytest.mark.gpu

CFG = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                 audio_d_head=64)
B, GH, GW, NF, F0, NCACHE_F = 2, 4, 6, 3, 6, 6
LA, LA_CACHE, A0, LT = 10, 40, 60, 16


def _inputs(CFG=CFG):
    g = torch.Generator().manual_seed(33)
    r = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16).float()
    hw = GH * GW
    vd, ad = CFG.video_dim, CFG.audio_dim
    x = dict(video=r(B, NF * hw, CFG.in_channels), audio=r(B, LA, CFG.in_channels),
             sigma=torch.rand(B, generator=g), vctx=r(B, LT, vd), actx=r(B, LT, ad))
    keep = torch.ones(B, LT, dtype=torch.int64)
    keep[:, -4:] = 0
    x["mask"] = OA.prepare_attention_mask(keep, torch.bfloat16)
    x["cache"] = [dict(video_self_k=r(B, NCACHE_F * hw, CFG.video_heads, CFG.video_d_head),
                       video_self_v=r(B, NCACHE_F * hw, CFG.video_heads, CFG.video_d_head),
                       audio_self_k=r(B, LA_CACHE, CFG.audio_heads, CFG.audio_d_head),
                       audio_self_v=r(B, LA_CACHE, CFG.audio_heads, CFG.audio_d_head))
                  for _ in range(CFG.num_layers)]
    return x


def _pes(dev=None, CFG=CFG):
    """(video, audio, video cross, audio cross) RoPE tables; oracle when dev is None."""
    vd, cross = CFG.video_dim, CFG.audio_heads * CFG.audio_d_head
    hw = GH * GW
    if dev is None:
        pe = lambda grid, dim, heads, f0, audio=False: OR.causal_precompute_freqs_cis(
            grid, dim, start_frame=f0, num_attention_heads=heads, batch=B, is_audio=audio)
    else:
        pe = lambda grid, dim, heads, f0, audio=False: T.causal_precompute_freqs_cis(
            torch.tensor([list(grid)] * B), dim, start_frame=f0, device=dev, dtype=torch.bfloat16,
            num_attention_heads=heads, is_audio=audio)
    vcross = [t.repeat_interleave(hw, dim=2).contiguous() for t in pe((NF,), cross, CFG.audio_heads, F0)]
    return (pe((NF, GH, GW), vd, CFG.video_heads, F0), pe((LA,), CFG.audio_dim, CFG.audio_heads, A0, True),
            vcross, pe((LA,), cross, CFG.audio_heads, A0, True))


@pytest.mark.parametrize("packed", [False, True], ids=["qkv3", "qkv_packed"])
def test_block_stack_matches_oracle(dev, packed):
    model = D.build_model(CFG, dev, seed=3)
    if packed:
        model.fuse_qkv_()   # video and audio self-attentions: one q/k/v GEMM each
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs()
    ref_v, ref_a = OD.forward_chunk(params, CFG, x["video"], x["audio"], x["sigma"], x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(), x["cache"])
    hw = GH * GW
    # room for two chunks past the cache: the committed step's and the clean commit pass's
    specs = {"video_self": T.ArenaSpec((NCACHE_F + 2 * NF) * hw, CFG.video_heads, CFG.video_d_head),
             "audio_self": T.ArenaSpec(LA_CACHE + 2 * LA + 8, CFG.audio_heads, CFG.audio_d_head)}
    kvc = T.init_kv_cache(CFG.num_layers, B, specs, dev)
    caches = []
    for lay, c in zip(kvc.layers, x["cache"]):
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        nv, na = c["video_self_k"].shape[1], c["audio_self_k"].shape[1]
        va.slots("k", 0, nv).copy_(c["video_self_k"].to(dev, torch.bfloat16))
        va.slots("v", 0, nv).copy_(c["video_self_v"].to(dev, torch.bfloat16))
        aa.slots("k", 0, na).copy_(c["audio_self_k"].to(dev, torch.bfloat16))
        aa.slots("v", 0, na).copy_(c["audio_self_v"].to(dev, torch.bfloat16))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, nv)]),
                                     video_self_v=KVSpanView(va, "v", [(0, nv)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, na)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, na)])))
    bf = lambda t: t.to(dev, torch.bfloat16)
    with torch.no_grad():
        vo, ao, kept = model.forward_chunk(bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]),
                                           bf(x["actx"]), bf(x["mask"]), bf(x["mask"]), *_pes(dev), caches)
        # a committed step appends the chunk's keys to every self-attention cache
        _, _, committed = model.forward_chunk(bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev),
                                              bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]), bf(x["mask"]),
                                              *_pes(dev), caches, commit=True)
        # the clean commit pass: same caches, no outputs
        nv_, na_, kv_only = model.forward_chunk(bf(x["video"]), bf(x["audio"]), torch.zeros_like(x["sigma"]).to(dev),
                                                bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]), bf(x["mask"]),
                                                *_pes(dev), caches, kv_cache_only=True)
    torch.cuda.synchronize()
    assert nv_ is None and na_ is None
    assert kv_only[0].video_self_k.shape[1] == (NCACHE_F + NF) * hw
    assert kept is not caches and all(k is c for k, c in zip(kept, caches))
    assert committed[0].video_self_k.shape[1] == (NCACHE_F + NF) * hw
    assert committed[1].audio_self_k.shape[1] == LA_CACHE + LA
    assert torch.isfinite(vo).all() and torch.isfinite(ao).all()
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err


@pytest.mark.parametrize("mode", ["cross_attn_adapter", "memory_kv_side_branch"])
def test_block_stack_with_learned_memory_matches_oracle(dev, mode):
    """The same stack with learned-memory adapters on block 1 (interval 2):
    video memory attention (512 = 8 x 64) and colour FiLM, audio memory
    attention (256 = 8 x 32, the zero-padded head path), in both placements;
    48 video and 64 audio memory tokens, a 512-wide colour vector."""
    cfg = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                     audio_d_head=64, learned_memory_enabled=True, learned_memory_mode=mode,
                     learned_memory_layer_interval=2, learned_memory_color_film_enabled=True)
    model = D.build_model(cfg, dev, seed=5)
    assert model.transformer_blocks[1].video_memory_attn is not None
    assert model.transformer_blocks[0].video_memory_attn is None
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs()
    g = torch.Generator().manual_seed(44)
    mem = dict(learned_memory_video=torch.randn(B, 48, cfg.in_channels, generator=g),
               learned_memory_audio=torch.randn(B, 64, cfg.in_channels, generator=g),
               learned_memory_color=torch.randn(B, 512, generator=g) * 0.5)
    mem = {k: v.to(torch.bfloat16).float() for k, v in mem.items()}
    dense = lambda c: {k: v for k, v in c.items()}
    ref_v, ref_a = OD.forward_chunk(params, cfg, x["video"], x["audio"], x["sigma"], x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(), [dense(c) for c in x["cache"]],
                                    **mem)
    hw = GH * GW
    specs = {"video_self": T.ArenaSpec((NCACHE_F + NF) * hw, cfg.video_heads, cfg.video_d_head),
             "audio_self": T.ArenaSpec(LA_CACHE + LA + 8, cfg.audio_heads, cfg.audio_d_head)}
    kvc = T.init_kv_cache(cfg.num_layers, B, specs, dev)
    caches = []
    for lay, c in zip(kvc.layers, x["cache"]):
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        nv, na = c["video_self_k"].shape[1], c["audio_self_k"].shape[1]
        va.slots("k", 0, nv).copy_(c["video_self_k"].to(dev, torch.bfloat16))
        va.slots("v", 0, nv).copy_(c["video_self_v"].to(dev, torch.bfloat16))
        aa.slots("k", 0, na).copy_(c["audio_self_k"].to(dev, torch.bfloat16))
        aa.slots("v", 0, na).copy_(c["audio_self_v"].to(dev, torch.bfloat16))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, nv)]),
                                     video_self_v=KVSpanView(va, "v", [(0, nv)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, na)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, na)])))
    bf = lambda t: t.to(dev, torch.bfloat16)
    with torch.no_grad():
        args = (bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]),
                bf(x["mask"]), *_pes(dev), caches)
        vo, ao, _ = model.forward_chunk(*args, **{k: bf(v) for k, v in mem.items()})
        vo0, ao0, _ = model.forward_chunk(*args)
    torch.cuda.synchronize()
    assert torch.isfinite(vo).all() and torch.isfinite(ao).all()
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err
    # the memory reached both streams
    assert (vo - vo0).abs().max().item() > 1e-2 and (ao - ao0).abs().max().item() > 1e-2


@pytest.mark.parametrize("L", [300, 2304])
def test_ffn_gelu_epilogue(dev, L):
    """The first FFN GEMM with its tanh-GELU epilogue (bf16, no grad) against
    float32 tanh-GELU(x W^T + b), and no further from it than the two-pass
    bf16 form (linear, then gelu) the reference runs."""
    torch.manual_seed(5)
    m = D.GELUApprox(512, 2048).to(dev, torch.bfloat16)
    x = torch.randn(2, L, 512, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y = m(x)
        two = torch.nn.functional.gelu(m.proj(x), approximate="tanh")
    ref = torch.nn.functional.gelu(torch.nn.functional.linear(x.float(), m.proj.weight.float(), m.proj.bias.float()),
                                   approximate="tanh")
    assert y.shape == two.shape and y.dtype == torch.bfloat16
    e_epi = (y.float() - ref).abs()
    e_two = (two.float() - ref).abs()
    assert e_epi.max().item() <= 2e-2 and e_epi.mean().item() <= 2e-3
    assert e_epi.mean().item() <= e_two.mean().item() * 1.05


def _arena_caches(dev, cfg, dense_caches):
    """The dense per-layer caches copied into one arena per layer and kind,
    with room for two more chunks."""
    hw = GH * GW
    specs = {"video_self": T.ArenaSpec((NCACHE_F + 2 * NF) * hw, cfg.video_heads, cfg.video_d_head),
             "audio_self": T.ArenaSpec(LA_CACHE + 2 * LA + 8, cfg.audio_heads, cfg.audio_d_head)}
    kvc = T.init_kv_cache(cfg.num_layers, B, specs, dev)
    caches = []
    for lay, c in zip(kvc.layers, dense_caches):
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        nv, na = c["video_self_k"].shape[1], c["audio_self_k"].shape[1]
        for arena, n, kk, vv in ((va, nv, "video_self_k", "video_self_v"), (aa, na, "audio_self_k", "audio_self_v")):
            arena.slots("k", 0, n).copy_(c[kk].to(dev, torch.bfloat16))
            arena.slots("v", 0, n).copy_(c[vv].to(dev, torch.bfloat16))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, nv)]),
                                     video_self_v=KVSpanView(va, "v", [(0, nv)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, na)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, na)])))
    return caches


def test_per_frame_sigma_matches_oracle(dev):
    """One sigma per latent frame with frame 1 a clean conditioning frame
    (sigma 0, model_runtime.py:897-910), expanded over the frame's tokens
    (kv_cache.py:2895-2903), and a per-sample audio sigma, against the oracle."""
    model = D.build_model(CFG, dev, seed=3)
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs()
    g = torch.Generator().manual_seed(9)
    sigma = torch.rand(B, NF, generator=g)
    sigma[:, 1] = 0.0
    a_sigma = torch.rand(B, generator=g)
    ref_v, ref_a = OD.forward_chunk(params, CFG, x["video"], x["audio"], sigma, x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(), x["cache"], audio_sigma=a_sigma)
    # the conditioning frame changes the result: per-frame sigma is not the per-sample one
    ref_u, _ = OD.forward_chunk(params, CFG, x["video"], x["audio"], sigma[:, 0], x["vctx"], x["actx"],
                                x["mask"].float(), x["mask"].float(), *_pes(), x["cache"], audio_sigma=a_sigma)
    assert (ref_u - ref_v).abs().max().item() > 1e-2
    caches = _arena_caches(dev, CFG, x["cache"])
    bf = lambda t: t.to(dev, torch.bfloat16)
    with torch.no_grad():
        vo, ao, _ = model.forward_chunk(bf(x["video"]), bf(x["audio"]), sigma.to(dev), bf(x["vctx"]), bf(x["actx"]),
                                        bf(x["mask"]), bf(x["mask"]), *_pes(dev), caches, audio_sigma=a_sigma.to(dev))
        with pytest.raises(ValueError, match="audio_sigma"):
            model.forward_chunk(bf(x["video"]), bf(x["audio"]), sigma.to(dev), bf(x["vctx"]), bf(x["actx"]),
                                bf(x["mask"]), bf(x["mask"]), *_pes(dev), caches)
    torch.cuda.synchronize()
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err


def test_loaded_checkpoint_matches_oracle(dev, tmp_path):
    """Weights that came through the disk format: a generator saved in the
    load_model_generator layout (taomate/inference/model_runtime.py:182-425),
    loaded with load_generator onto the GPU (configuration detected from the
    tensors), runs forward_chunk; the oracle runs on the tensors read back
    from the same file."""
    from taomate_amd import checkpoint as C
    src = D.build_model(CFG, dev, seed=11)
    path = str(tmp_path / "gen.pt")
    C.save_generator(src, path)
    del src
    model = C.load_generator(path, device=dev, dtype=torch.bfloat16, video_d_head=CFG.video_d_head,
                             audio_d_head=CFG.audio_d_head)
    assert model.cfg.num_layers == CFG.num_layers and model.cfg.video_heads == CFG.video_heads
    params = {n: p.float() for n, p in C.read_generator_state(path).items()}
    x = _inputs()
    ref_v, ref_a = OD.forward_chunk(params, CFG, x["video"], x["audio"], x["sigma"], x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(), x["cache"])
    hw = GH * GW
    bf = lambda t: t.to(dev, torch.bfloat16)
    caches = [T.LayerKVCache(video_self_k=bf(c["video_self_k"]), video_self_v=bf(c["video_self_v"]),
                             audio_self_k=bf(c["audio_self_k"]), audio_self_v=bf(c["audio_self_v"]))
              for c in x["cache"]]
    with torch.no_grad():
        vo, ao, _ = model.forward_chunk(bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]),
                                        bf(x["actx"]), bf(x["mask"]), bf(x["mask"]), *_pes(dev), caches)
    torch.cuda.synchronize()
    assert vo.shape == (B, NF * hw, CFG.out_channels)
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err


@pytest.mark.timeout(600)
def test_48_block_stack_matches_oracle(dev):
    """All 48 blocks of the model's depth composed, at a reduced width (video
    8 x 64, audio 4 x 64): one denoising step over dense caches against the
    fp32 oracle's 48-block forward (the full-width 48-block step is checked
    for its properties in test_gpu_dit_full.py; its fp32 oracle would need
    75 GB of weights)."""
    cfg = D.AVConfig(num_layers=48, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4,
                     video_d_head=64, audio_d_head=64)
    model = D.build_model(cfg, dev, seed=13).fuse_qkv_()
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs(cfg)
    ref_v, ref_a = OD.forward_chunk(params, cfg, x["video"], x["audio"], x["sigma"], x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(None, cfg), x["cache"])
    bf = lambda t: t.to(dev, torch.bfloat16)
    caches = [T.LayerKVCache(video_self_k=bf(c["video_self_k"]), video_self_v=bf(c["video_self_v"]),
                             audio_self_k=bf(c["audio_self_k"]), audio_self_v=bf(c["audio_self_v"]))
              for c in x["cache"]]
    with torch.no_grad():
        vo, ao, _ = model.forward_chunk(bf(x["video"]), bf(x["audio"]), x["sigma"].to(dev), bf(x["vctx"]),
                                        bf(x["actx"]), bf(x["mask"]), bf(x["mask"]), *_pes(dev, cfg), caches)
    torch.cuda.synchronize()
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err


@pytest.mark.parametrize("per_frame", [False, True], ids=["per_sample_sigma", "per_frame_sigma"])
def test_ltx23_text_adaln_matches_oracle(dev, per_frame):
    """The LTX-2.3 text cross-attention AdaLN (9-row modulation tables, prompt
    tables, prompt_adaln_single modules; kv_cache.py:1090-1141, prompt
    timestep :2876-2895) through the 2-block stack against the oracle, with a
    sigma per sample and per latent frame (the prompt timestep then takes
    the frames' mean), both streams' text keys 25 % padded."""
    cfg = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                     audio_d_head=64, cross_attention_adaln=True, apply_gated_attention=True)
    model = D.build_model(cfg, dev, seed=17)
    assert model.transformer_blocks[0].scale_shift_table.shape == (9, 512)
    params = {n: p.detach().float().cpu() for n, p in model.named_parameters()}
    x = _inputs(cfg)
    g = torch.Generator().manual_seed(19)
    sigma = torch.rand(B, NF, generator=g) if per_frame else x["sigma"]
    a_sigma = torch.rand(B, generator=g) if per_frame else None
    ref_v, ref_a = OD.forward_chunk(params, cfg, x["video"], x["audio"], sigma, x["vctx"], x["actx"],
                                    x["mask"].float(), x["mask"].float(), *_pes(None, cfg), x["cache"],
                                    audio_sigma=a_sigma)
    caches = _arena_caches(dev, cfg, x["cache"])
    bf = lambda t: t.to(dev, torch.bfloat16)
    with torch.no_grad():
        vo, ao, _ = model.forward_chunk(bf(x["video"]), bf(x["audio"]), sigma.to(dev), bf(x["vctx"]),
                                        bf(x["actx"]), bf(x["mask"]), bf(x["mask"]), *_pes(dev, cfg), caches,
                                        audio_sigma=None if a_sigma is None else a_sigma.to(dev))
    torch.cuda.synchronize()
    cv, ca = cosine(vo, ref_v), cosine(ao, ref_a)
    assert cv >= 0.999 and ca >= 0.999, (cv, ca)
    for out, ref in ((vo, ref_v), (ao, ref_a)):
        err = (out.float().cpu() - ref).abs().max().item()
        assert err <= 3e-2 * ref.abs().max().item(), err


def _small_arena_caches(dev, cfg, x):
    hw = GH * GW
    specs = {"video_self": T.ArenaSpec((NCACHE_F + 2 * NF) * hw, cfg.video_heads, cfg.video_d_head),
             "audio_self": T.ArenaSpec(LA_CACHE + 2 * LA + 16, cfg.audio_heads, cfg.audio_d_head)}
    kvc = T.init_kv_cache(cfg.num_layers, B, specs, dev)
    caches = []
    for lay, c in zip(kvc.layers, x["cache"]):
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        nv, na = c["video_self_k"].shape[1], c["audio_self_k"].shape[1]
        va.slots("k", 0, nv).copy_(c["video_self_k"].to(dev, torch.bfloat16))
        va.slots("v", 0, nv).copy_(c["video_self_v"].to(dev, torch.bfloat16))
        aa.slots("k", 0, na).copy_(c["audio_self_k"].to(dev, torch.bfloat16))
        aa.slots("v", 0, na).copy_(c["audio_self_v"].to(dev, torch.bfloat16))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, nv)]),
                                     video_self_v=KVSpanView(va, "v", [(0, nv)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, na)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, na)])))
    return caches


@pytest.mark.parametrize("mode", [None, "cross_attn_adapter", "memory_kv_side_branch"])
@pytest.mark.parametrize("per_frame", [False, True], ids=["per_sample_sigma", "per_frame_sigma"])
def test_audio_stream_overlap_bit_identical(dev, mode, per_frame):
    """The audio ops on their own stream (the model's default) against one
    stream, bit for bit: outputs of a denoise step and the caches a clean
    commit leaves, with and without learned-memory adapters (both
    placements), with one sigma per sample (every block's modulation values
    precomputed) and one per latent frame (each block computes its own on its
    stream); the overlapped pass runs twice."""
    mem_on = mode is not None
    cfg = D.AVConfig(num_layers=2, video_dim=512, audio_dim=256, video_heads=8, audio_heads=4, video_d_head=64,
                     audio_d_head=64, learned_memory_enabled=mem_on,
                     learned_memory_mode=mode or "cross_attn_adapter", learned_memory_layer_interval=2,
                     learned_memory_color_film_enabled=mem_on)
    model = D.build_model(cfg, dev, seed=6)
    x = _inputs(cfg)
    g = torch.Generator().manual_seed(45)
    bf = lambda t: t.to(dev, torch.bfloat16)
    kw = {}
    if mem_on:
        kw = dict(learned_memory_video=bf(torch.randn(B, 48, cfg.in_channels, generator=g)),
                  learned_memory_audio=bf(torch.randn(B, 64, cfg.in_channels, generator=g)),
                  learned_memory_color=bf(torch.randn(B, 512, generator=g) * 0.5))
    if per_frame:
        sigma = torch.rand(B, NF, generator=g).to(dev)
        kw["audio_sigma"] = torch.rand(B, generator=g).to(dev)
    else:
        sigma = x["sigma"].to(dev)
    args = (bf(x["video"]), bf(x["audio"]), sigma, bf(x["vctx"]), bf(x["actx"]), bf(x["mask"]), bf(x["mask"]),
            *_pes(dev, cfg))
    fields = ("video_self_k", "video_self_v", "audio_self_k", "audio_self_v", "a2v_k", "a2v_v", "v2a_k", "v2a_v")

    def run(overlap):
        model.overlap_audio_(overlap)
        caches = _small_arena_caches(dev, cfg, x)
        with torch.no_grad():
            vo, ao, _ = model.forward_chunk(*args, caches, **kw)
            _, _, committed = model.forward_chunk(*args[:2], torch.zeros_like(sigma), *args[3:], caches,
                                                  kv_cache_only=True, **kw)
        torch.cuda.synchronize()
        dense_of = lambda t: t.materialize() if hasattr(t, "materialize") else t.clone()
        return vo, ao, [[dense_of(getattr(c, f)) for f in fields] for c in committed]

    ref = run(False)
    for i in range(2):
        got = run(True)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), f"pass {i}: outputs differ"
        for layer, (gl, rl) in enumerate(zip(got[2], ref[2])):
            for f, a, b in zip(fields, gl, rl):
                assert torch.equal(a, b), f"pass {i}: layer {layer} {f} differs"
