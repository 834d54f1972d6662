"""Benchmark of the chunked causal LTX attention hot path on one MI355X.

One step = one pass of the path over one chunk, with its inputs (the q/k/v
projection outputs and a populated KV arena) resident in HBM:
  1. fused full-row q/k RMSNorm + 3-D SPLIT RoPE, new K written into its arena slots
  2. V append into the arena
  3. flash attention of the 1152-query chunk over anchor | memory | window | current
     (384 + 768 + 2304 + 1152 = 4608 keys), B=2 (cond/uncond), 32 heads x 128, bf16.
The q/k/v/out projections are hipBLASLt GEMMs outside this path and not timed.

Prints one JSON line.  `--gpus N` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "query-tokens/sec + TFLOP/s (% bf16 MFMA peak) for 1152q×4608k chunk attn"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E

# 512x768 output: 16x24 latent grid = 384 tokens per latent frame
GRID_H, GRID_W = 16, 24
FRAME = GRID_H * GRID_W
B, H, D = 2, 32, 128
HD = H * D
LQ = 3 * FRAME                                   # 3-frame chunk
SEGMENTS = [("anchor", 0, 1), ("memory", 1, 2), ("window", 6, 6)]  # (name, first frame, frames)
CUR_FRAME0 = 12
LK = FRAME * (1 + 2 + 6) + LQ                    # 4608


def attn_flops() -> float:
    return 4.0 * B * H * LQ * LK * D


def attn_bytes(kv_bytes: int = 2) -> float:
    """Algorithmic HBM bytes of one attention launch: q and out once, K and V once."""
    return B * H * D * (2 * LQ * 2 + 2 * LK * kv_bytes)


def norm_rope_bytes() -> float:
    """q and k rows read + written once (bf16), gammas, and the bf16 cos/sin table once."""
    return 2 * (2 * B * LQ * HD * 2) + 2 * HD * 2 + 2 * (H * LQ * (D // 2) * 2)


def append_bytes(kv_dtype: str = "bf16") -> float:
    """bf16 arena: V read and written key-major.  fp8 arena: the bf16 K and V
    rows read, their e4m3 codes and one float32 scale per (batch, head, frame)
    of each written."""
    if kv_dtype == "fp8":
        return 2 * B * LQ * HD * 2 + 2 * B * LQ * HD + 2 * B * H * (LQ // FRAME) * 4
    return 2 * B * LQ * HD * 2


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "attention_b2_h32_d128_1152q_4608k_hbm_traffic.md")


def measured_traffic(kv_dtype: str):
    """HBM bytes per attention call (attention + combine kernels) for this
    workload, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (line `traffic_bytes_per_call[<kv>]: N`); None when not profiled."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                key = f"traffic_bytes_per_call[{kv_dtype}]:"
                if line.strip().startswith(key):
                    return int(line.split(":", 1)[1].strip().strip("`"))
    except OSError:
        pass
    return None


def build_workload(dev, kv_dtype: str = "bf16"):
    from taomate_amd import kernels
    from taomate_amd.kv_cache import KVArena
    from taomate_amd.rope import causal_precompute_freqs_cis

    g = torch.Generator(device=dev)
    g.manual_seed(1)
    cached = FRAME * 9
    arena = KVArena(B, cached + 2 * LQ, H, D, dev, kv_dtype, frame_tokens=FRAME, name="bench")
    # cached anchor | memory | window spans: post-norm keys ~ N(0,1), values ~ N(0,1)
    spans, pos = [], 0
    for _, _, nf in SEGMENTS:
        n = nf * FRAME
        k = torch.randn(B, n, H, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn(B, n, H, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
        if arena.fp8:
            kernels.kv_append(k, arena.slots("k", pos, n), arena.scale_slots("k", pos, n), FRAME)
            kernels.kv_append(v, arena.slots("v", pos, n), arena.scale_slots("v", pos, n), FRAME)
        else:
            arena.slots("k", pos, n).copy_(k)
            arena.slots("v", pos, n).copy_(v)
        spans.append((pos, n))
        pos += n
    # projection outputs of the current chunk (hidden ~ N(0,1), W ~ N(0, 0.02^2) => ~N(0, 1.64))
    sd = 0.02 * math.sqrt(HD)
    q_lin = (torch.randn(B, LQ, HD, generator=g, device=dev) * sd).to(torch.bfloat16)
    k_lin = (torch.randn(B, LQ, HD, generator=g, device=dev) * sd).to(torch.bfloat16)
    v_lin = (torch.randn(B, LQ, HD, generator=g, device=dev) * sd).to(torch.bfloat16)
    gq = torch.ones(HD, device=dev, dtype=torch.bfloat16)
    gk = torch.ones(HD, device=dev, dtype=torch.bfloat16)
    grid = torch.tensor([[3, GRID_H, GRID_W]] * B)
    pe = causal_precompute_freqs_cis(grid, HD, start_frame=CUR_FRAME0, device=dev,
                                     dtype=torch.bfloat16, num_attention_heads=H)
    return dict(arena=arena, spans=spans, q_lin=q_lin, k_lin=k_lin, v_lin=v_lin, gq=gq, gk=gk,
                pe=pe, slot=pos, q=torch.empty_like(q_lin),
                out=torch.empty(B, LQ, H, D, device=dev, dtype=torch.bfloat16))


def make_step(w, attn_queries: int = LQ):
    """Returns (step, attn_only, norm_only, append_only, prep) closures over the
    workload; prep is the step's first part: the fused q/k norm + RoPE + V
    append launch (bf16 arena) or norm then the fp8 pair append.  attn_queries:
    the attention call takes the chunk's first attn_queries queries (all by
    default)."""
    from taomate_amd import kernels
    from taomate_amd.kernels import KVSegment

    a = w["arena"]
    slot = w["slot"]
    kd, vd = a.slots("k", slot, LQ), a.slots("v", slot, LQ)
    ks, vs = a.scale_slots("k", slot, LQ), a.scale_slots("v", slot, LQ)
    segs = []
    for s, n in w["spans"] + [(slot, LQ)]:
        segs.append(KVSegment(a.slots("k", s, n), a.slots("v", s, n),
                              a.scale_slots("k", s, n), a.scale_slots("v", s, n)))
    frame = FRAME if a.fp8 else 0
    kbf = torch.empty(B, LQ, H, D, device=a.device, dtype=torch.bfloat16) if a.fp8 else kd
    q4 = w["q"].view(B, LQ, H, D)

    def norm():
        kernels.qk_rmsnorm_rope(w["q_lin"], w["q"], w["gq"], 1e-6, w["pe"], H, D,
                                w["k_lin"], kbf, w["gk"], 1e-6, w["pe"])

    def append():
        if a.fp8:
            kernels.kv_append_fp8_pair(kbf, kd, ks, w["v_lin"].view(B, LQ, H, D), vd, vs, FRAME)
        else:
            kernels.kv_append(w["v_lin"].view(B, LQ, H, D), vd)

    qa, oa = q4[:, :attn_queries], w["out"][:, :attn_queries]

    def attn():
        kernels.flash_attn(qa, segs, oa, frame_tokens=frame)

    def prep():
        if a.fp8:
            norm()
            append()
        else:
            kernels.qk_rmsnorm_rope(w["q_lin"], w["q"], w["gq"], 1e-6, w["pe"], H, D,
                                    w["k_lin"], kbf, w["gk"], 1e-6, w["pe"],
                                    v_in=w["v_lin"].view(B, LQ, H, D), v_out=vd)

    def step():
        prep()
        attn()

    return step, attn, norm, append, prep


def stream_bench(dev, n_chunks: int = 60, kv_dtype: str = "fp8", warm_chunks: int = 60, fuse_qkv: bool = True):
    """Sustained rate of the long stream: one video self-attention layer at the
    512x768 chunk shape (B=2, 32 heads x 128, d=4096, weights ~N(0, 0.02^2),
    inputs ~N(0, 1), seed 4) run through ``n_chunks`` 3-frame chunks with the
    anchor (1 frame) pinned, 2 memory frames re-prefilled every 4 chunks and a
    12-frame rolling window (steady state: 384 + 768 + 4608 cached keys + the
    chunk's own 1152), K/V in the fp8-e4m3 arena.  Each chunk is the whole
    layer: q/k/v projections, fused norm+RoPE, K/V quantise into the arena,
    attention, output projection, eviction and (every 4th) the memory
    re-prefill.  Timed from the first chunk to the last, synchronised at both
    ends; the prefill of anchor and memory is not timed."""
    import taomate_amd as T
    from taomate_amd.streaming import ChunkStream

    g = torch.Generator(device=dev)
    g.manual_seed(4)
    attn = T.CausalLTXAttention(HD, heads=H, dim_head=D).to(dev, torch.bfloat16)
    with torch.no_grad():
        for lin in (attn.to_q, attn.to_k, attn.to_v, attn.to_out[0]):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g, device=dev) * 0.02)
            lin.bias.zero_()
    if fuse_qkv:
        attn.fuse_qkv_()
    # eight distinct chunk inputs, used in turn
    xs = [torch.randn(B, LQ, HD, generator=g, device=dev).to(torch.bfloat16) for _ in range(8)]
    xa = torch.randn(B, FRAME, HD, generator=g, device=dev).to(torch.bfloat16)
    xm = torch.randn(B, 2 * FRAME, HD, generator=g, device=dev).to(torch.bfloat16)

    def run(n):
        st = ChunkStream(attn, (GRID_H, GRID_W), B, dev, kv_dtype=kv_dtype)
        st.prefill(xa, xm)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for c in range(n):
            st.step(xs[c % len(xs)])
        torch.cuda.synchronize()
        return time.perf_counter() - t0, st

    with torch.no_grad():
        run(warm_chunks)
        secs, st = run(n_chunks)
    keys = st.k.shape[1]
    return {"query_tokens_per_s": n_chunks * B * LQ / secs, "unit": "query-tokens/s",
            "ms_per_chunk": secs / n_chunks * 1e3, "chunks": n_chunks, "kv_dtype": kv_dtype,
            "memory_refreshes": st.memory_version, "cached_keys_after_last_chunk": keys,
            "qkv_projection": "one packed GEMM" if fuse_qkv else "three GEMMs",
            "workload": "one 32x128 video self-attention layer (d=4096, B=2) over 60 chunks of 3 frames at "
                        "16x24: anchor 1 frame pinned | memory 2 frames refreshed every 4 chunks | 12-frame "
                        "window | current chunk, whole layer per chunk (projections included)"}


def c3_bench(dev, iters: int = 200) -> dict:
    """The audio and cross-attention calls of one block at the chunk shape,
    B = 2, inputs ~N(0, 1), seed 2: audio self-attention (75 queries, 32 x 64,
    over 600 cached + 75 current audio keys), A2V (1152 video queries over the
    chunk's 75 audio keys, 32 x 64), V2A (75 audio queries over the chunk's 1152
    video keys, 32 x 64) and the text cross-attention (1152 queries, 32 x 128,
    over 1024 text keys of which each row keeps its first 820: 20 % padding, the
    per-row key counts of the pipelined kernel).  V is key-major, as the layer
    stores it (arena, or the key-major copy of a plain-tensor cache).  Each call
    timed back to back between HIP events; FLOPs count the attended keys."""
    from taomate_amd import kernels
    from taomate_amd.kernels import KVSegment
    from taomate_amd.kv_cache import KVArena

    g = torch.Generator(device=dev)
    g.manual_seed(2)

    def rnd(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)

    def arena_segs(lens, Hh, Dh):
        a = KVArena(B, sum(lens) + 8 * len(lens), Hh, Dh, dev, "bf16", name="c3")
        segs, pos = [], 0
        for n in lens:
            a.slots("k", pos, n).copy_(rnd(B, n, Hh, Dh))
            a.slots("v", pos, n).copy_(rnd(B, n, Hh, Dh))
            segs.append(KVSegment(a.slots("k", pos, n), a.slots("v", pos, n)))
            pos += -(-n // 8) * 8
        return a, segs

    calls = {}
    for name, lq, lens, Dh, klen in (("audio_self", 75, [600, 75], 64, None),
                                     ("a2v", LQ, [75], 64, None),
                                     ("v2a", 75, [LQ], 64, None),
                                     ("text_cross", LQ, [1024], 128, [820, 820])):
        a, segs = arena_segs(lens, H, Dh)
        q = rnd(B, lq, H, Dh)
        out = torch.empty_like(q)
        fn = (lambda q=q, segs=segs, out=out, klen=klen: kernels.flash_attn(q, segs, out, key_lens=klen))
        for _ in range(20):
            fn()
        ms = time_region(fn, iters)
        keys = (sum(klen) / B) if klen else sum(lens)
        fl = 4.0 * B * H * lq * keys * Dh
        calls[name] = {"queries": lq, "keys": int(keys), "head_dim": Dh, "us": ms * 1e3,
                       "TFLOP/s": fl / (ms * 1e-3) / 1e12, "frac_bf16_peak": fl / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
        del a, segs, q, out
    calls["what"] = ("B = 2, 32 heads; each call back to back between HIP events; small calls are bound by "
                     "latency (launch and one round of loads), not by the matrix cores")
    return calls


def dit_bench(dev, steps: int = 5, warmup: int = 2, learned_memory: bool = False, fuse_qkv: bool = True):
    """One denoising step of the 48-block dual-stream model (video 32 x 128,
    d = 4096; audio 32 x 64, d = 2048; 4x GELU FFNs; AdaLN modulation) for one
    512x768 chunk at B = 2: 1152 video tokens over the 3456 cached keys of the
    chunk workload above, 75 audio tokens over 600 cached, 1024 text tokens
    (20 % masked) for both streams, A2V / V2A over the chunk's own tokens.
    Random bf16 weights (seed 3), sigma ~ U(0, 1).  Timed with HIP events
    around whole steps, with the audio ops on their own stream (the model's
    default) and again on one stream; the attention share is the summed
    duration of every attention call (events around each, one stream) over
    the one-stream step time.
    With ``learned_memory`` every 4th block carries the memory adapters
    (video 8 x 64 over 48 tokens + colour FiLM, audio 8 x 32 over 64 tokens),
    fed by a StreamingMemory updated once with the chunk's latents."""
    from taomate_amd import dit as Dm
    from taomate_amd import kernels
    import taomate_amd as T
    from taomate_amd.kv_cache import KVSpanView
    from taomate_amd.rope import causal_precompute_freqs_cis

    cfg = Dm.AVConfig(learned_memory_enabled=learned_memory, learned_memory_color_film_enabled=learned_memory)
    model = Dm.build_model(cfg, dev, seed=3)
    if fuse_qkv:
        model.fuse_qkv_()
    n_params = sum(p.numel() for p in model.parameters())
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    r = lambda *sh: torch.randn(*sh, generator=g, device=dev).to(torch.bfloat16)
    LT, LA, LA_C = 1024, 75, 600
    vlat, alat = r(B, LQ, cfg.in_channels), r(B, LA, cfg.in_channels)
    sigma = torch.rand(B, generator=g, device=dev)
    vctx, actx = r(B, LT, cfg.video_dim), r(B, LT, cfg.audio_dim)
    mask = torch.zeros(B, 1, 1, LT, dtype=torch.bfloat16, device=dev)
    mask[..., int(0.8 * LT):] = torch.finfo(torch.bfloat16).min
    cached = LK - LQ
    specs = {"video_self": T.ArenaSpec(cached + LQ, H, D), "audio_self": T.ArenaSpec(LA_C + LA + 8, 32, 64)}
    kvc = T.init_kv_cache(cfg.num_layers, B, specs, dev)
    caches = []
    for lay in kvc.layers:
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        va.slots("k", 0, cached).copy_(r(B, cached, H, D))
        va.slots("v", 0, cached).copy_(r(B, cached, H, D))
        aa.slots("k", 0, LA_C).copy_(r(B, LA_C, 32, 64))
        aa.slots("v", 0, LA_C).copy_(r(B, LA_C, 32, 64))
        caches.append(T.LayerKVCache(video_self_k=KVSpanView(va, "k", [(0, cached)]),
                                     video_self_v=KVSpanView(va, "v", [(0, cached)]),
                                     audio_self_k=KVSpanView(aa, "k", [(0, LA_C)]),
                                     audio_self_v=KVSpanView(aa, "v", [(0, LA_C)])))
    pe = lambda grid, dim, heads, f0, audio=False: causal_precompute_freqs_cis(
        torch.tensor([list(grid)] * B), dim, start_frame=f0, device=dev, dtype=torch.bfloat16,
        num_attention_heads=heads, is_audio=audio)
    vpe = pe((3, GRID_H, GRID_W), cfg.video_dim, H, CUR_FRAME0)
    ape = pe((LA,), cfg.audio_dim, 32, LA_C, True)
    vcross = [t.repeat_interleave(FRAME, dim=2).contiguous() for t in pe((3,), 2048, 32, CUR_FRAME0)]
    across = pe((LA,), 2048, 32, LA_C, True)

    attn_events = []
    real_flash = kernels.flash_attn

    def timed_flash(*a, **kw):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        real_flash(*a, **kw)
        e1.record()
        attn_events.append((e0, e1))

    mem = {}
    if learned_memory:
        state = T.StreamingMemory()
        lat5 = vlat.view(B, 3, GRID_H, GRID_W, cfg.in_channels).permute(0, 1, 4, 2, 3)
        state.set_reference(lat5, alat)
        state.update(lat5, alat)
        mem = state.with_conditional_memory({}, device=dev, dtype=torch.bfloat16)

    def step():
        return model.forward_chunk(vlat, alat, sigma, vctx, actx, mask, mask, vpe, ape, vcross, across, caches,
                                   **mem)

    def timed_steps():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            out = step()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / steps, out

    with torch.no_grad():
        # every op on one stream first (the audio stream's kernels between the
        # video stream's), then the model's default with the audio ops beside
        # them on their own stream
        model.overlap_audio_(False)
        ms_one, _ = timed_steps()
        # attention share (one stream, so that each call's events hold only
        # that call): three more steps with events around every attention
        # call; the fastest of them (a host stall only lengthens a step) gives
        # the step time and its attention calls' summed time
        kernels.flash_attn = timed_flash
        best = None
        try:
            for _ in range(3):
                attn_events.clear()
                s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s0.record()
                step()
                s1.record()
                s1.synchronize()
                cur = (s0.elapsed_time(s1), sum(a.elapsed_time(b) for a, b in attn_events), len(attn_events))
                best = cur if best is None or cur[0] < best[0] else best
        finally:
            kernels.flash_attn = real_flash
            model.overlap_audio_(True)
        ms_inst, ms_attn, n_attn = best
        ms, (vo, ao, _) = timed_steps()
        finite = bool(torch.isfinite(vo).all() and torch.isfinite(ao).all())
        # the same steps with the text cross-attention's K/V kept across steps
        # (the reference's exact text K/V cache, off by default there and in
        # the figure above): the first call projects, the timed ones reuse
        model.cache_text_kv_()
        ms_tkv, _ = timed_steps()
        model.cache_text_kv_(False)
    res = {"ms_per_step": ms, "chunk_query_tokens_per_s": B * LQ / (ms * 1e-3), "params": n_params,
           "audio_stream": "the audio ops on a second HIP stream beside the video ops (overlap_audio_)",
           "ms_per_step_one_stream": ms_one,
           "ms_per_step_text_kv_cached": ms_tkv,
           "attention_ms": ms_attn, "attention_share": ms_attn / ms_inst, "attention_calls": n_attn,
           "outputs_finite": finite, "learned_memory": learned_memory,
           "qkv_projection": "one packed GEMM per self-attention" if fuse_qkv else "three GEMMs",
           "workload": "48 dual-stream blocks (video 32x128 d=4096, audio 32x64 d=2048, 4x GELU FFNs, AdaLN), "
                       "one denoising step of a 512x768 chunk at B=2: 1152 video queries over 3456 cached + 1152 "
                       "keys, 75 audio over 600 + 75, 1024 text keys (20% masked), A2V 1152x75, V2A 75x1152"
                       + ("; memory adapters on every 4th block" if learned_memory else "")}
    del model, caches, kvc
    torch.cuda.empty_cache()
    return res


def time_region(fn, iters: int) -> float:
    """Average device ms per call over `iters` back-to-back calls, HIP events on
    the launching stream (the attention-only profiling mode and the standalone
    rates of the norm and append kernels; the step figures come from the timed
    step loop).  The calls are queued behind a bounded device spin so that the
    host's launch cost stays out of the interval: the start event must still
    be pending once the last call is queued, else the spin is lengthened and
    the measurement repeated (a short kernel launched from Python otherwise
    times the host, not the kernel)."""
    st = torch.cuda.current_stream()
    cycles = 1 << 20
    for attempt in range(6):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        torch.cuda._sleep(cycles)
        e0.record(st)
        for _ in range(iters):
            fn()
        ahead = not e0.query()
        e1.record(st)
        e1.synchronize()
        if ahead:
            return e0.elapsed_time(e1) / iters
        cycles *= 4
    print("time_region: the host could not queue ahead of the device; the figure includes launch cost",
          file=sys.stderr)
    return e0.elapsed_time(e1) / iters


def cpu_baseline(seconds_budget: float = 20.0):
    """The oracle (op-for-op PyTorch CPU restatement of the reference path) on the
    host cores, fp32: RMSNorm -> SPLIT RoPE -> cat -> SDPA for the same chunk.
    Sample: one batch element (B=1) of the same shape, repeated while inside the
    time budget; the rate is scaled to query-tokens/s."""
    from oracle import attention as OA
    from oracle import rope as OR

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator()
    g.manual_seed(1)
    sd = 0.02 * math.sqrt(HD)
    q_lin = torch.randn(1, LQ, HD, generator=g) * sd
    k_lin = torch.randn(1, LQ, HD, generator=g) * sd
    cached_k = torch.randn(1, LK - LQ, H, D, generator=g)
    cached_v = torch.randn(1, LK - LQ, H, D, generator=g)
    v = torch.randn(1, LQ, H, D, generator=g)
    cos, sin = OR.causal_precompute_freqs_cis((3, GRID_H, GRID_W), HD, start_frame=CUR_FRAME0,
                                              num_attention_heads=H, batch=1)
    ones = torch.ones(HD)

    def once():
        q = OR.apply_split_rotary_emb(OA.rms_norm_full_row(q_lin, ones, 1e-6), cos, sin)
        k = OR.apply_split_rotary_emb(OA.rms_norm_full_row(k_lin, ones, 1e-6), cos, sin)
        fk = torch.cat([cached_k, k.view(1, LQ, H, D)], 1)
        fv = torch.cat([cached_v, v], 1)
        return OA.standard_attention_forward(q.view(1, LQ, H, D), fk, fv)

    once()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < seconds_budget and len(times) < 200):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": LQ / med, "unit": "query-tokens/s", "cores": cores, "kind": "port",
            "sample": f"fp32 CPU oracle, one batch element (B=1) of the 1152q x 4608k chunk, "
                      f"median of {len(times)} runs ({med * 1e3:.0f} ms each); "
                      f"torch {torch.__version__}, {platform.processor() or platform.machine()}"}


def cold_rates(w, copies: int = 6) -> dict:
    """The step's HBM kernels with their inputs rotated over ``copies`` sets of
    q/k/v projection outputs (6 x 56.6 MB, more than the 256 MB last-level
    cache), so every call reads its inputs from HBM: the rates of the
    standalone loops (one input set, back to back) are flattered by that
    cache."""
    from taomate_amd import kernels

    a = w["arena"]
    slot = w["slot"]
    kd, vd = a.slots("k", slot, LQ), a.slots("v", slot, LQ)
    ks, vs = a.scale_slots("k", slot, LQ), a.scale_slots("v", slot, LQ)
    sets = [(w["q_lin"].clone(), w["k_lin"].clone(), w["v_lin"].clone()) for _ in range(copies)]
    kbf = torch.empty(B, LQ, H, D, device=a.device, dtype=torch.bfloat16) if a.fp8 else kd
    it = {"i": 0}

    def nxt():
        it["i"] = (it["i"] + 1) % copies
        return sets[it["i"]]

    def norm():
        ql, kl, _ = nxt()
        kernels.qk_rmsnorm_rope(ql, w["q"], w["gq"], 1e-6, w["pe"], H, D, kl, kbf, w["gk"], 1e-6, w["pe"])

    def append():
        _, kl, vl = nxt()
        if a.fp8:
            kernels.kv_append_fp8_pair(kl.view(B, LQ, H, D), kd, ks, vl.view(B, LQ, H, D), vd, vs, FRAME)
        else:
            kernels.kv_append(vl.view(B, LQ, H, D), vd)

    def prep():
        ql, kl, vl = nxt()
        if a.fp8:
            kernels.qk_rmsnorm_rope(ql, w["q"], w["gq"], 1e-6, w["pe"], H, D, kl, kbf, w["gk"], 1e-6, w["pe"])
            kernels.kv_append_fp8_pair(kbf, kd, ks, vl.view(B, LQ, H, D), vd, vs, FRAME)
        else:
            kernels.qk_rmsnorm_rope(ql, w["q"], w["gq"], 1e-6, w["pe"], H, D, kl, kbf, w["gk"], 1e-6, w["pe"],
                                    v_in=vl.view(B, LQ, H, D), v_out=vd)

    for f in (norm, append, prep):
        for _ in range(copies):
            f()
    out = {"norm_ms": time_region(norm, 60), "append_ms": time_region(append, 60), "prep_ms": time_region(prep, 60),
           "copies": copies, "what": f"inputs rotated over {copies} copies of the q/k/v projection outputs "
                                     f"({copies * 3 * B * LQ * HD * 2 / 1e6:.0f} MB, beyond the last-level cache)"}
    del sets
    return out


def measure_steps(step, attn, norm, append, prep, steps: int, warmup: int, settle_seconds: float) -> dict:
    """The C2 step timings for one workload: settle, warm-up, the K timed steps
    (events only at the two ends of the region), an instrumented pass of K
    steps with events around each step's two parts, and the two HBM kernels
    and the step's first part on their own."""
    # Settle phase (reported as its own field, outside warmup and steps): the
    # step runs back to back for --settle-seconds of wall time so that the
    # card leaves its idle clock state before the warm-up and timed steps; a
    # cold card runs its first milliseconds of work at a lower clock.
    settle_steps = 0
    torch.cuda.synchronize()
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < settle_seconds:
        for _ in range(20):
            step()
        settle_steps += 20
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle
    for _ in range(warmup):
        step()
    # Timed region: the K steps the driver asks for, bracketed by
    # synchronisations, with HIP events only at its two ends.  (On this
    # runtime an event recorded between two kernels holds the second one back
    # by about 5 us, so per-call events inside this loop would add about
    # 15 us to every step.)
    st = torch.cuda.current_stream()
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record(st)
    for i in range(steps):
        step()
    t_enq = time.perf_counter() - t0   # host time to queue the K steps
    e_end.record(st)
    e_end.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e_start.elapsed_time(e_end) / steps
    # Instrumented pass: K more steps with events on the launching stream
    # around each step's two parts (q/k norm + RoPE + V append, attention),
    # for the per-step distributions and the in-step split.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        e = ev[i]
        e[0].record(st)
        prep()
        e[1].record(st)
        attn()
        e[2].record(st)
    torch.cuda.synchronize()
    prep_ms = [e[0].elapsed_time(e[1]) for e in ev]
    attn_ms = [e[1].elapsed_time(e[2]) for e in ev]
    step_ms = [e[0].elapsed_time(e[2]) for e in ev]
    ms_prep = sum(prep_ms) / steps
    # The attention call's average duration inside the step (the roofline's
    # kernel_ms): events around each call in the instrumented pass.  The same
    # calls back to back, with no other kernel between them, measured 1-2 %
    # slower (170-173 against 169-170 us at the 512x768 chunk), so that figure
    # is reported beside it.
    ms_attn = sum(attn_ms) / steps
    ms_attn_b2b = time_region(attn, steps)
    # the two HBM kernels on their own (after the timed region), for their rates
    for _ in range(10):
        norm()
        append()
    ms_norm = time_region(norm, 50)
    ms_app = time_region(append, 50)
    # the step's first part on its own: as launched in the step, and as the
    # two separate launches (norm, then append) it replaces
    ms_prep_alone = time_region(prep, 50)
    ms_prep_two = time_region(lambda: (norm(), append()), 50)
    return dict(ms_step=ms_step, ms_attn=ms_attn, ms_attn_b2b=ms_attn_b2b, ms_prep=ms_prep, ms_norm=ms_norm,
                ms_app=ms_app, ms_prep_alone=ms_prep_alone, ms_prep_two=ms_prep_two, step_ms=step_ms,
                attn_ms=attn_ms, prep_ms=prep_ms, settle_s=settle_s, settle_steps=settle_steps, wall=wall,
                t_enq=t_enq)


def fp8_step_bench(dev, steps: int, warmup: int, settle_seconds: float) -> dict:
    """The same C2 step on an fp8-e4m3 arena (per-(batch, head, frame) scales),
    measured in the same run and the same way as the headline line: q/k norm +
    RoPE (K to a bf16 buffer), the K and V quantise into the arena (one
    launch), then attention over the dequantised-in-kernel cache."""
    w = build_workload(dev, "fp8")
    step, attn, norm, append, prep = make_step(w)
    m = measure_steps(step, attn, norm, append, prep, steps, warmup, settle_seconds)
    cold = cold_rates(w)
    del step, attn, norm, append, prep, w
    fl = attn_flops()
    ach = fl / (m["ms_attn"] * 1e-3) / 1e12
    prep_bytes = norm_rope_bytes() + append_bytes("fp8")
    return {
        "query_tokens_per_s": B * LQ / (m["ms_step"] * 1e-3),
        "ms_per_step": m["ms_step"],
        "attention": {"kernel": "flash_fwd_pair_kernel<128, true> (q-tiles 0-7 of every head) + "
                                "flash_fwd_pipe_kernel<128, true> (q-tile 8, key ranges) + flash_combine_kernel<128>",
                      "kernel_ms": m["ms_attn"], "kernel_ms_back_to_back": m["ms_attn_b2b"],
                      "tflops": ach, "frac_bf16_peak": ach / PEAK_BF16_TFLOPS,
                      "algorithmic_bytes": attn_bytes(1), "traffic": measured_traffic("fp8")},
        "quantise": {"ms": m["ms_app"], "GB/s": append_bytes("fp8") / (m["ms_app"] * 1e-3) / 1e9,
                     "frac_hbm": append_bytes("fp8") / (m["ms_app"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                     "what": "K and V quantised to e4m3 into the arena (one launch, run on its own)"},
        "norm_rope": {"ms": m["ms_norm"], "GB/s": norm_rope_bytes() / (m["ms_norm"] * 1e-3) / 1e9,
                      "frac_hbm": norm_rope_bytes() / (m["ms_norm"] * 1e-3) / 1e9 / PEAK_HBM_GBPS},
        "step_prep": {"ms": m["ms_prep"], "alone_ms": m["ms_prep_alone"],
                      "GB/s": prep_bytes / (m["ms_prep"] * 1e-3) / 1e9,
                      "frac_hbm": prep_bytes / (m["ms_prep"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                      "what": "q/k norm + RoPE, then the fp8 pair append (in the step)"},
        "hbm_cold": {**cold,
                     "norm_rope_frac_hbm": norm_rope_bytes() / (cold["norm_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                     "quantise_frac_hbm": append_bytes("fp8") / (cold["append_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                     "prep_frac_hbm": prep_bytes / (cold["prep_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS},
        "per_step_ms_median": {"step": statistics.median(m["step_ms"]),
                               "attention": statistics.median(m["attn_ms"]),
                               "prep": statistics.median(m["prep_ms"])},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--kv", choices=["bf16", "fp8"], default="bf16")
    ap.add_argument("--settle-seconds", type=float, default=2.0,
                    help="seconds of back-to-back steps before the warm-up (reported in the 'settle' field)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--attn-only", action="store_true", help="loop only the attention kernel (profiling)")
    ap.add_argument("--attn-queries", type=int, default=LQ,
                    help="--attn-only: attend the chunk's first N queries (1024: 8 q-tiles per head, the pair kernel)")
    ap.add_argument("--no-fp8", action="store_true", help="skip the same step on the fp8-e4m3 arena (its own object)")
    ap.add_argument("--no-c3", action="store_true",
                    help="skip the audio self / A2V / V2A / text cross-attention calls (their own object)")
    ap.add_argument("--no-stream", action="store_true", help="skip the 60-chunk long-stream measurement")
    ap.add_argument("--stream-only", action="store_true", help="run only the 60-chunk long-stream measurement")
    ap.add_argument("--no-dit", action="store_true", help="skip the 48-block denoising-step measurement")
    ap.add_argument("--dit-only", action="store_true", help="run only the 48-block denoising-step measurement")
    ap.add_argument("--no-fuse-qkv", action="store_true",
                    help="stream and 48-block step: three q/k/v GEMMs instead of one packed GEMM per self-attention")
    ap.add_argument("--dit-learned-memory", action="store_true",
                    help="the 48-block step with learned-memory adapters on every 4th block")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 256 MiB device copy (scale reference for HBM byte counters)")
    ap.add_argument("--copy-bandwidth", action="store_true",
                    help="time plain device copies of 64 MiB - 4 GiB (the practical HBM ceiling of a streaming kernel)")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="time hipBLASLt bf16 GEMMs of 4096^3 - 16384^3 (the sustained matrix-core rate of a "
                         "vendor kernel on this part)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the hot path on one GPU; --gpus must be 1 "
              "(multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 64 * 1024 * 1024
        x = torch.ones(n, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "launches": 3}))
        return
    if args.stream_only:
        print(json.dumps(stream_bench(dev, fuse_qkv=not args.no_fuse_qkv)))
        return
    if args.dit_only:
        print(json.dumps(dit_bench(dev, learned_memory=args.dit_learned_memory, fuse_qkv=not args.no_fuse_qkv)))
        return
    if args.copy_bandwidth:
        for mib in (64, 256, 1024, 4096):
            n = mib * 1024 * 1024 // 4
            x = torch.ones(n, device=dev)
            y = torch.empty_like(x)
            for _ in range(10):
                y.copy_(x)
            ms = time_region(lambda: y.copy_(x), 50)
            print(json.dumps({"copy_MiB": mib, "ms": round(ms, 4),
                              "TB/s (read + write)": round(2 * n * 4 / (ms * 1e-3) / 1e12, 3)}))
            del x, y
        return
    if args.gemm_ceiling:
        for n in (4096, 8192, 16384):
            a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
            bm = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
            c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
            gemm = lambda: torch.matmul(a, bm, out=c)  # noqa: E731
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 1.0:  # leave the idle clock state
                for _ in range(4):
                    gemm()
                torch.cuda.synchronize()
            reps = max(10, int(2e14 / (2 * n ** 3)))
            ms = time_region(gemm, reps)
            tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
            print(json.dumps({"gemm_bf16": f"{n}x{n}x{n}", "ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                              "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 3), "reps": reps}))
            del a, bm, c
        return
    w = build_workload(dev, args.kv)
    if not 1 <= args.attn_queries <= LQ:
        print(f"bench.py: --attn-queries must be in [1, {LQ}]", file=sys.stderr)
        sys.exit(2)
    step, attn, norm, append, prep = make_step(w, args.attn_queries if args.attn_only else LQ)
    if args.attn_only:
        prep()  # the chunk's normalised q and new K/V: the attention inputs of a step
        torch.cuda.synchronize()
        t_settle = time.perf_counter()
        while time.perf_counter() - t_settle < args.settle_seconds:
            for _ in range(20):
                attn()
            torch.cuda.synchronize()
        for _ in range(args.warmup):
            attn()
        ms = time_region(attn, args.steps)
        flops = attn_flops() * args.attn_queries / LQ
        print(json.dumps({"attn_only_ms": ms, "queries": args.attn_queries, "tflops": flops / ms / 1e9}))
        return
    m = measure_steps(step, attn, norm, append, prep, args.steps, args.warmup, args.settle_seconds)
    cold = cold_rates(w)
    del step, attn, norm, append, prep, w
    ms_step, ms_attn, ms_attn_b2b, ms_prep = m["ms_step"], m["ms_attn"], m["ms_attn_b2b"], m["ms_prep"]
    ms_norm, ms_app, ms_prep_alone, ms_prep_two = m["ms_norm"], m["ms_app"], m["ms_prep_alone"], m["ms_prep_two"]
    step_ms, attn_ms, prep_ms = m["step_ms"], m["attn_ms"], m["prep_ms"]
    settle_s, settle_steps, wall, t_enq = m["settle_s"], m["settle_steps"], m["wall"], m["t_enq"]

    def dist(xs):
        return {"min": min(xs), "median": statistics.median(xs), "max": max(xs)}
    kvb = 1 if args.kv == "fp8" else 2
    fl = attn_flops()
    ach = fl / (ms_attn * 1e-3) / 1e12
    res = {
        "metric": METRIC,
        "value": B * LQ / (ms_step * 1e-3),
        "unit": "query-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "video self-attention chunk at 512x768: B=2 (cond/uncond), 32 heads x 128, "
                               "1152 queries (3 frames of 16x24) over 4608 keys = anchor 384 | memory 768 | "
                               "window 2304 | current 1152; step = fused q/k RMSNorm+RoPE (new K into arena) "
                               "+ V append + flash attention",
                   "kv_dtype": args.kv, "global_batch": B, "seq_len": LQ, "keys": LK,
                   "heads": H, "head_dim": D, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": ach, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": ach / PEAK_BF16_TFLOPS, "traffic": measured_traffic(args.kv),
                     "kernel_ms_back_to_back": ms_attn_b2b,
                     "timing": "kernel_ms: the attention calls of a second pass of K steps, a HIP event on "
                               "the launching stream before and after each call (the interval holds the "
                               "about 5 us the event before it adds); kernel_ms_back_to_back: K calls with "
                               "no other kernel between them, between two events",
                     "kernel": ("flash_fwd_pipe_kernel<128, false> + flash_combine_kernel<128>" if args.kv == "bf16"
                                else "flash_fwd_pair_kernel<128, true> (q-tiles 0-7 of every head) + "
                                     "flash_fwd_pipe_kernel<128, true> (q-tile 8, key ranges) + "
                                     "flash_combine_kernel<128>"),
                     "kernel_ms": ms_attn,
                     "algorithmic_flops": fl, "algorithmic_bytes": attn_bytes(kvb)},
        "attention_tflops": ach,
        "attention_query_tokens_per_s": B * LQ / (ms_attn * 1e-3),
        "norm_rope": {"ms": ms_norm, "GB/s": norm_rope_bytes() / (ms_norm * 1e-3) / 1e9,
                      "frac_hbm": norm_rope_bytes() / (ms_norm * 1e-3) / 1e9 / PEAK_HBM_GBPS},
        "kv_append": {"ms": ms_app, "GB/s": append_bytes(args.kv) / (ms_app * 1e-3) / 1e9,
                      "frac_hbm": append_bytes(args.kv) / (ms_app * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                      "what": "V transposed into the key-major arena" if args.kv == "bf16"
                      else "K and V quantised to e4m3 into the arena (one launch)"},
        "hbm_cold": {**cold,
                     "norm_rope_frac_hbm": norm_rope_bytes() / (cold["norm_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                     "append_frac_hbm": append_bytes(args.kv) / (cold["append_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBPS,
                     "prep_frac_hbm": (norm_rope_bytes() + append_bytes(args.kv)) / (cold["prep_ms"] * 1e-3) / 1e9
                     / PEAK_HBM_GBPS},
        "step_prep": {"ms": ms_prep,
                      "GB/s": (norm_rope_bytes() + append_bytes(args.kv)) / (ms_prep * 1e-3) / 1e9,
                      "alone_ms": ms_prep_alone, "two_launches_ms": ms_prep_two,
                      "what": "fused q/k norm + RoPE + V append (one launch)" if args.kv == "bf16"
                      else "q/k norm + RoPE, then the fp8 pair append"},
        "per_step_ms": {"step": dist(step_ms), "attention": dist(attn_ms), "prep": dist(prep_ms),
                        "what": "a second pass of K steps with an event before, between and after the two "
                                "parts of each step (the events add their own gaps)"},
        "settle": {"seconds": settle_s, "steps": settle_steps,
                   "what": "back-to-back steps before the warm-up, so the card leaves its idle clock state"},
        "wall_s_timed_region": wall,
        "host_enqueue_ms_per_step": t_enq * 1e3 / args.steps,
    }
    if args.kv == "bf16" and not args.no_fp8:
        res["fp8"] = fp8_step_bench(dev, args.steps, args.warmup, args.settle_seconds)
    if args.kv == "bf16" and not args.no_c3:
        res["c3"] = c3_bench(dev)
    if not args.no_stream:
        res["long_stream"] = stream_bench(dev, fuse_qkv=not args.no_fuse_qkv)
    if not args.no_dit:
        res["dit_step"] = dit_bench(dev, learned_memory=args.dit_learned_memory, fuse_qkv=not args.no_fuse_qkv)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
