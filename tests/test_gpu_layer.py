"""GPU parity of the drop-in attention surface against the fp32 CPU oracle:
attention_with_cache over an arena cache (anchor | memory | window | current),
the audio / cross-modal / text-cross attentions, and the streaming loop."""
import gc
import math

import pytest
import torch

import taomate_amd as T
from oracle import attention as OA
from oracle import rope as OR

from .helpers import BF16_MAX_ABS, BF16_MEAN_ABS, assert_bf16_close, cosine, diff_stats

pytestmark = pytest.mark.gpu


def make_layer(dev, d, H, Dh, seed, context_dim=None, gate=False):
    """Seeded weights ~N(0, 0.02^2), zero biases, unit norm weights; the module
    in bf16 on the GPU and the same values in fp32 for the oracle."""
    g = torch.Generator().manual_seed(seed)
    m = T.CausalLTXAttention(d, context_dim=context_dim, heads=H, dim_head=Dh, apply_gated_attention=gate)
    with torch.no_grad():
        lins = [m.to_q, m.to_k, m.to_v, m.to_out[0]] + ([m.to_gate_logits] if gate else [])
        for lin in lins:
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.02)
            lin.bias.zero_()
    c = lambda t: t.detach().clone().float()
    w = OA.AttnWeights(c(m.to_q.weight), c(m.to_q.bias), c(m.to_k.weight), c(m.to_k.bias),
                       c(m.to_v.weight), c(m.to_v.bias), c(m.to_out[0].weight), c(m.to_out[0].bias),
                       c(m.q_norm.weight), c(m.k_norm.weight), H, Dh,
                       wg=c(m.to_gate_logits.weight) if gate else None,
                       bg=c(m.to_gate_logits.bias) if gate else None)
    return m.to(dev, torch.bfloat16), w


def gpu_pe(dev, grid, dim, heads, start, B, audio=False):
    return T.causal_precompute_freqs_cis(torch.tensor([list(grid)] * B), dim, start_frame=start, device=dev,
                                         dtype=torch.bfloat16, num_attention_heads=heads, is_audio=audio)


def ora_pe(grid, dim, heads, start, B, audio=False):
    return OR.causal_precompute_freqs_cis(grid, dim, start_frame=start, num_attention_heads=heads, batch=B,
                                          is_audio=audio)


# (name, B, grid_h, grid_w, heads, dim_head, seed, kv_dtype)
LAYERS = [
    ("8x12grid_8x64", 1, 8, 12, 8, 64, 0, "bf16"),
    ("16x24grid_32x128_B2", 2, 16, 24, 32, 128, 1, "bf16"),
    ("16x24grid_32x128_B2_fp8", 2, 16, 24, 32, 128, 1, "fp8"),
]
# anchor frame 0 | memory frames | window frames | current chunk frames
SEGS_SMALL = [("anchor", 0, 1), ("memory", 1, 1), ("window", 6, 4)]
SEGS_FULL = [("anchor", 0, 1), ("memory", 1, 2), ("window", 6, 6)]


_ORACLE = {}


def _layer_reference(B, gh, gw, H, Dh, seed, w):
    """fp32 oracle: prefill every segment at its absolute frames, then the chunk
    over cat(cache, new).  Cached: the bf16 and fp8 cases share it."""
    key = (B, gh, gw, H, Dh, seed)
    if key not in _ORACLE:
        d, hw = H * Dh, gh * gw
        segs = SEGS_SMALL if H == 8 else SEGS_FULL
        cur_f0, cur_nf = (10, 2) if H == 8 else (12, 3)
        g = torch.Generator().manual_seed(seed + 100)
        xs = [torch.randn(B, nf * hw, d, generator=g) for _, _, nf in segs]
        xc = torch.randn(B, cur_nf * hw, d, generator=g)
        ck = cv = None
        for (nm, f0, nf), x in zip(segs, xs):
            _, k, v = OA.attention_with_cache(w, x, None, ora_pe((nf, gh, gw), d, H, f0, B), None, None, None)
            ck = k if ck is None else torch.cat([ck, k], 1)
            cv = v if cv is None else torch.cat([cv, v], 1)
        ref, ref_k, _ = OA.attention_with_cache(w, xc, None, ora_pe((cur_nf, gh, gw), d, H, cur_f0, B), None,
                                                ck, cv)
        _ORACLE[key] = (xs, xc, ref, ref_k)
    return _ORACLE[key]


@pytest.mark.parametrize("packed", [False, True], ids=["qkv3", "qkv_packed"])
@pytest.mark.parametrize("case", LAYERS, ids=[c[0] for c in LAYERS])
def test_attention_with_cache_layer(dev, case, packed):
    """packed: the q/k/v projections run as one GEMM (fuse_qkv_), whose three
    column views (row stride 3·H·D) feed the norm / RoPE and append kernels."""
    name, B, gh, gw, H, Dh, seed, kvd = case
    d = H * Dh
    hw = gh * gw
    segs = SEGS_SMALL if H == 8 else SEGS_FULL
    cur_f0, cur_nf = (10, 2) if H == 8 else (12, 3)
    attn, w = make_layer(dev, d, H, Dh, seed)
    if packed:
        attn.fuse_qkv_()
        assert attn._packed_qkv() is not None
    xs, xc, ref, ref_k = _layer_reference(B, gh, gw, H, Dh, seed, w)
    # GPU: same calls through an arena cache
    total = sum(nf for _, _, nf in segs) * hw + cur_nf * hw
    spec = {"video_self": T.ArenaSpec(total, H, Dh, kvd, frame_tokens=hw)}
    cache = T.init_kv_cache(1, B, spec, dev)
    lay = cache.layers[0]
    kc, vc = lay.video_self_k, lay.video_self_v
    with torch.no_grad():
        for (nm, f0, nf), x in zip(segs, xs):
            _, nk, nv = T.attention_with_cache(attn, x.to(dev, torch.bfloat16), None,
                                               gpu_pe(dev, (nf, gh, gw), d, H, f0, B), None, kc, vc)
            kc, vc = T._cat_cache(kc, nk), T._cat_cache(vc, nv)
        out, nk, nv = T.attention_with_cache(attn, xc.to(dev, torch.bfloat16), None,
                                             gpu_pe(dev, (cur_nf, gh, gw), d, H, cur_f0, B), None, kc, vc)
    torch.cuda.synchronize()
    assert isinstance(nk, T.KVSpanView) and nk.shape == (B, cur_nf * hw, H, Dh)
    assert kc.shape[1] == total - cur_nf * hw
    if kvd == "bf16":
        assert_bf16_close(out, ref, name)
        assert cosine(nk.materialize(), ref_k) >= 0.9999
    else:
        assert diff_stats(out, ref)[0] <= BF16_MAX_ABS
    c = cosine(out, ref)
    assert c >= (0.999 if kvd == "fp8" else 0.9999), c


@pytest.mark.parametrize("case", LAYERS[:2], ids=[c[0] for c in LAYERS[:2]])
def test_dense_cache_layer(dev, case):
    """Plain-tensor caches (no arena plan: the reference's torch.cat caches,
    kv_cache.py:394-398).  At the 16x24 chunk shape the cached and new V go
    into one key-major store for the pipelined kernel (1152 queries over
    3456 + 1152 keys); the 8x12 case (192 queries) concatenates as the
    reference does.  Both match the fp32 oracle."""
    name, B, gh, gw, H, Dh, seed, kvd = case
    d = H * Dh
    segs = SEGS_SMALL if H == 8 else SEGS_FULL
    cur_f0, cur_nf = (10, 2) if H == 8 else (12, 3)
    attn, w = make_layer(dev, d, H, Dh, seed)
    xs, xc, ref, ref_k = _layer_reference(B, gh, gw, H, Dh, seed, w)
    kc = vc = None
    with torch.no_grad():
        for (nm, f0, nf), x in zip(segs, xs):
            _, nk, nv = T.attention_with_cache(attn, x.to(dev, torch.bfloat16), None,
                                               gpu_pe(dev, (nf, gh, gw), d, H, f0, B), None, kc, vc)
            kc, vc = T._cat_cache(kc, nk), T._cat_cache(vc, nv)
        out, nk, nv = T.attention_with_cache(attn, xc.to(dev, torch.bfloat16), None,
                                             gpu_pe(dev, (cur_nf, gh, gw), d, H, cur_f0, B), None, kc, vc)
    torch.cuda.synchronize()
    assert not isinstance(kc, T.KVSpanView) and kc.is_contiguous() and vc.is_contiguous()
    assert nk.shape == (B, cur_nf * gh * gw, H, Dh) and nv.stride(3) == 1
    assert_bf16_close(out, ref, name + " dense")
    assert cosine(out, ref) >= 0.9999
    assert cosine(nk, ref_k) >= 0.9999


def test_audio_and_cross_modal_attention(dev):
    """Audio self-attention (75 queries over 600 cached + 75 new audio keys, 32 x 64,
    1-D audio RoPE) and the A2V / V2A cross-modal attentions (1152 video tokens
    <-> 75 audio tokens, projected to 32 x 64, 1-D cross RoPE)."""
    B, Hh, Dh = 1, 32, 64
    da, dv = 2048, 4096
    g = torch.Generator().manual_seed(2)
    # audio self: 24 cached blocks of 25 frames at latent frames 0..599, chunk at 600..674
    attn, w = make_layer(dev, da, Hh, Dh, 20)
    xa_old = torch.randn(B, 600, da, generator=g)
    xa = torch.randn(B, 75, da, generator=g)
    _, ck, cv = OA.attention_with_cache(w, xa_old, None, ora_pe((600,), da, Hh, 0, B, True), None, None, None)
    ref, _, _ = OA.attention_with_cache(w, xa, None, ora_pe((75,), da, Hh, 600, B, True), None, ck, cv)
    cache = T.init_kv_cache(1, B, {"audio_self": T.ArenaSpec(700, Hh, Dh)}, dev)
    lay = cache.layers[0]
    with torch.no_grad():
        _, nk, nv = T.attention_with_cache(attn, xa_old.to(dev, torch.bfloat16), None,
                                           gpu_pe(dev, (600,), da, Hh, 0, B, True), None,
                                           lay.audio_self_k, lay.audio_self_v)
        kc, vc = T._cat_cache(lay.audio_self_k, nk), T._cat_cache(lay.audio_self_v, nv)
        out, _, _ = T.attention_with_cache(attn, xa.to(dev, torch.bfloat16), None,
                                           gpu_pe(dev, (75,), da, Hh, 600, B, True), None, kc, vc)
    assert_bf16_close(out, ref, "audio self")
    assert cosine(out, ref) >= 0.9999

    # cross-modal: video 3 frames x 384 tokens at frames 12..14, audio 75 frames at 100..174
    xv = torch.randn(B, 1152, dv, generator=g)
    xa = torch.randn(B, 75, da, generator=g)
    vpe_o = [t.repeat_interleave(384, dim=2) for t in ora_pe((3,), 2048, Hh, 12, B)]
    ape_o = ora_pe((75,), 2048, Hh, 100, B, True)
    vpe_g = [t.repeat_interleave(384, dim=2).contiguous() for t in gpu_pe(dev, (3,), 2048, Hh, 12, B)]
    ape_g = gpu_pe(dev, (75,), 2048, Hh, 100, B, True)
    a2v, wa2v = make_layer(dev, dv, Hh, Dh, 21, context_dim=da)   # video queries, audio keys
    v2a, wv2a = make_layer(dev, da, Hh, Dh, 22, context_dim=dv)   # audio queries, video keys
    ref_a2v, _, _ = OA.attention_with_cache(wa2v, xv, xa, vpe_o, ape_o, None, None)
    ref_v2a, _, _ = OA.attention_with_cache(wv2a, xa, xv, ape_o, vpe_o, None, None)
    with torch.no_grad():
        o_a2v, _, _ = T.attention_with_cache(a2v, xv.to(dev, torch.bfloat16), xa.to(dev, torch.bfloat16),
                                             vpe_g, ape_g, None, None)
        o_v2a, _, _ = T.attention_with_cache(v2a, xa.to(dev, torch.bfloat16), xv.to(dev, torch.bfloat16),
                                             ape_g, vpe_g, None, None)
    assert_bf16_close(o_a2v, ref_a2v, "A2V")
    assert_bf16_close(o_v2a, ref_v2a, "V2A")
    assert cosine(o_a2v, ref_a2v) >= 0.9999 and cosine(o_v2a, ref_v2a) >= 0.9999


def test_text_cross_attention_with_padding_mask(dev):
    """1152 video queries against 1024 text keys of dim 4096 (32 x 128), 20% of the
    keys padding, through CausalLTXAttention.forward with the reference's
    prepared additive mask (causal_model.py:551-562), gated output."""
    B, H, Dh, d = 1, 32, 128, 4096
    attn, w = make_layer(dev, d, H, Dh, 30, context_dim=d, gate=True)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, 1152, d, generator=g)
    ctx = torch.randn(B, 1024, d, generator=g)
    keep = torch.ones(B, 1024, dtype=torch.int64)
    keep[:, 819:] = 0
    m = OA.prepare_attention_mask(keep, torch.bfloat16)
    ref = OA.text_cross_attention(w, x, ctx, m.float())
    with torch.no_grad():
        out = attn(x.to(dev, torch.bfloat16), context=ctx.to(dev, torch.bfloat16), mask=m.to(dev))
    assert_bf16_close(out, ref, "text cross")
    assert cosine(out, ref) >= 0.9999


def test_text_kv_cache_keeps_key_major_v(dev, monkeypatch):
    """A cache hit of the text K/V attends the cached key-major V as it is: no
    V transposition runs on the hit (the pipelined kernel's path: >= 256
    queries, a key-padding mask that keeps the same prefix in every row), and
    the output equals the uncached one bit for bit."""
    from taomate_amd import kernels as K
    B, H, Dh, d = 2, 8, 128, 1024
    attn, w = make_layer(dev, d, H, Dh, 37, context_dim=d, gate=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, 384, d, generator=g).to(dev, torch.bfloat16)
    ctx = torch.randn(B, 200, d, generator=g).to(dev, torch.bfloat16)
    keep = torch.ones(B, 200, dtype=torch.int64)
    keep[:, 160:] = 0
    m = OA.prepare_attention_mask(keep, torch.bfloat16).to(dev)
    calls = []
    real = K.kv_append
    monkeypatch.setattr(K, "kv_append", lambda *a, **k: (calls.append(1), real(*a, **k))[1])
    with torch.no_grad():
        plain = attn(x, context=ctx, mask=m)
        assert len(calls) == 1                      # the uncached call transposes V once
        attn.cache_text_kv_()
        first = attn(x, context=ctx, mask=m)        # fills the entry (one transposition)
        n_fill = len(calls)
        again = attn(x, context=ctx, mask=m)        # hit: nothing transposed
        assert len(calls) == n_fill == 2
        attn.cache_text_kv_(False)
    torch.cuda.synchronize()
    assert torch.equal(first, plain) and torch.equal(again, plain)


def test_text_kv_cache_is_exact(dev):
    """cache_text_kv_: calls with the same context tensor reuse its K/V and give
    bit-identical outputs to projecting again; an in-place change of the
    context or of a K/V weight, or another context tensor, projects again."""
    B, H, Dh, d = 2, 8, 64, 512
    attn, w = make_layer(dev, d, H, Dh, 31, context_dim=d, gate=True)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, 96, d, generator=g).to(dev, torch.bfloat16)
    ctx = torch.randn(B, 40, d, generator=g).to(dev, torch.bfloat16)
    keep = torch.ones(B, 40, dtype=torch.int64)
    keep[1, 30:] = 0
    m = OA.prepare_attention_mask(keep, torch.bfloat16).to(dev)
    with torch.no_grad():
        plain = attn(x, context=ctx, mask=m)
        attn.cache_text_kv_()
        first = attn(x, context=ctx, mask=m)
        again = attn(x, context=ctx, mask=m)
        assert len(attn._text_kv_cache) == 1
        assert torch.equal(first, plain) and torch.equal(again, plain)
        ctx.add_(0.25)                                   # in place: a new version, projected again
        moved = attn(x, context=ctx, mask=m)
        attn.cache_text_kv_(False)
        assert torch.equal(moved, attn(x, context=ctx, mask=m))
        attn.cache_text_kv_()
        attn(x, context=ctx, mask=m)
        attn.to_v.weight.mul_(0.5)                       # a K/V parameter changed in place
        halved = attn(x, context=ctx, mask=m)
        attn.cache_text_kv_(False)
        assert torch.equal(halved, attn(x, context=ctx, mask=m))
        attn.cache_text_kv_(size=2)
        ctxs = [ctx.clone() for _ in range(3)]           # three live tensors: LRU of 2
        for c in ctxs:
            attn(x, context=c, mask=m)
        assert len(attn._text_kv_cache) == 2
        # a freed context whose address and version a new tensor reuses is no
        # hit: the entry's weak reference no longer points at the caller's tensor
        del ctxs
        fresh = ctx.clone().mul_(-1.0)
        attn.cache_text_kv_(False)
        want = attn(x, context=fresh, mask=m)
        attn.cache_text_kv_(size=2)
        for _ in range(2):
            tmp = ctx.clone()
            attn(x, context=tmp, mask=m)
            del tmp
        assert torch.equal(attn(x, context=fresh, mask=m), want)
    torch.cuda.synchronize()


def test_denoise_steps_do_not_commit(dev):
    """Three denoise-step calls on a snapshot, then the commit: the committed cache
    holds only the commit pass's keys, and step outputs equal the oracle's."""
    B, H, Dh, d, hw = 1, 8, 64, 512, 96
    attn, w = make_layer(dev, d, H, Dh, 40)
    g = torch.Generator().manual_seed(41)
    x0 = torch.randn(B, 4 * hw, d, generator=g)
    pe0 = (ora_pe((4, 8, 12), d, H, 0, B), gpu_pe(dev, (4, 8, 12), d, H, 0, B))
    pe1 = (ora_pe((3, 8, 12), d, H, 4, B), gpu_pe(dev, (3, 8, 12), d, H, 4, B))
    _, ck, cv = OA.attention_with_cache(w, x0, None, pe0[0], None, None, None)
    cache = T.init_kv_cache(1, B, {"video_self": T.ArenaSpec(10 * hw, H, Dh)}, dev)
    lay = cache.layers[0]
    with torch.no_grad():
        _, nk, nv = T.attention_with_cache(attn, x0.to(dev, torch.bfloat16), None, pe0[1], None,
                                           lay.video_self_k, lay.video_self_v)
        cache.layers = [T.LayerKVCache(video_self_k=T._cat_cache(lay.video_self_k, nk),
                                       video_self_v=T._cat_cache(lay.video_self_v, nv))]
        del nk, nv, lay
        snapshot = list(cache.layers)
        for step in range(3):
            cache.layers = list(snapshot)
            xs = torch.randn(B, 3 * hw, d, generator=g)
            ref, _, _ = OA.attention_with_cache(w, xs, None, pe1[0], None, ck, cv)
            out, sk, sv = T.attention_with_cache(attn, xs.to(dev, torch.bfloat16), None, pe1[1], None,
                                                 snapshot[0].video_self_k, snapshot[0].video_self_v)
            cache.layers = [T.LayerKVCache(video_self_k=T._cat_cache(snapshot[0].video_self_k, sk),
                                           video_self_v=T._cat_cache(snapshot[0].video_self_v, sv))]
            assert_bf16_close(out, ref, f"step {step}")
            del out, sk, sv
        cache.layers = list(snapshot)
        gc.collect()
        xc = torch.randn(B, 3 * hw, d, generator=g)
        _, rk, rv = OA.attention_with_cache(w, xc, None, pe1[0], None, ck, cv)
        _, nk, nv = T.attention_with_cache(attn, xc.to(dev, torch.bfloat16), None, pe1[1], None,
                                           snapshot[0].video_self_k, snapshot[0].video_self_v)
        committed = T._cat_cache(snapshot[0].video_self_k, nk)
    full = committed.materialize().float().cpu()
    assert full.shape[1] == 7 * hw
    assert cosine(full[:, 4 * hw:], rk) >= 0.9999
    assert cosine(full[:, :4 * hw], ck) >= 0.9999


@pytest.mark.parametrize("kind", ["common_prefix", "per_row_prefix", "holes", "soft_bias", "bool_prefix"])
def test_standard_attention_mask_forms(dev, kind):
    """Key-padding masks through standard_attention_forward: a prefix kept in
    every row is attended as the prefix alone and row-dependent prefixes as
    per-row key counts (both on the pipelined kernel over a key-major V copy);
    other forms (holes, finite biases) take the masked kernel.  All against
    the oracle with the same additive mask."""
    B, Lq, Lk, H, D = 2, 384, 700, 8, 128
    g = torch.Generator().manual_seed(61)
    q = torch.randn(B, Lq, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    keep = torch.ones(B, Lk, dtype=torch.int64)
    if kind in ("common_prefix", "bool_prefix"):
        keep[:, 555:] = 0
    elif kind == "per_row_prefix":
        keep[0, 555:] = 0
        keep[1, 610:] = 0
    elif kind == "holes":
        keep[:, 100:180] = 0
        keep[1, 400:] = 0
    if kind == "soft_bias":
        add = (torch.randn(B, 1, 1, Lk, generator=g) * 2.0).to(torch.bfloat16)
    else:
        add = OA.prepare_attention_mask(keep, torch.bfloat16)
    ref = OA.standard_attention_forward(q.float(), k.float(), v.float(), add.float())
    m = keep.bool().view(B, 1, 1, Lk).to(dev) if kind == "bool_prefix" else add.to(dev)
    with torch.no_grad():
        out = T.standard_attention_forward(q.to(dev), k.to(dev), v.to(dev), mask=m)
        again = T.standard_attention_forward(q.to(dev), k.to(dev), v.to(dev), mask=m)  # cached decision
    torch.cuda.synchronize()
    assert_bf16_close(out, ref, kind)
    assert torch.equal(out, again)
    assert cosine(out, ref) >= 0.9999


def test_text_cross_per_row_prefixes_take_the_pipelined_kernel(dev, monkeypatch):
    """Cond / uncond prompts of different lengths: 1152 queries against 1024
    text keys (32 x 128) with batch row 0 keeping 1024 keys and row 1 keeping
    700 (the reference's additive mask, causal_model.py:551-562, applied at
    kv_cache.py:764-827).  The call goes to the pipelined kernel with per-row
    key counts (no float mask, key-major V) and matches the oracle."""
    from taomate_amd import kernels as K
    B, Lq, Lk, H, D = 2, 1152, 1024, 32, 128
    g = torch.Generator().manual_seed(67)
    q = torch.randn(B, Lq, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Lk, H, D, generator=g).to(torch.bfloat16)
    keep = torch.ones(B, Lk, dtype=torch.int64)
    keep[1, 700:] = 0
    add = OA.prepare_attention_mask(keep, torch.bfloat16)
    ref = OA.standard_attention_forward(q.float(), k.float(), v.float(), add.float())
    seen = []
    real = K.flash_attn

    def spy(qq, segs, out, **kw):
        seen.append((kw.get("key_mask"), kw.get("key_lens"), segs[0].v.stride(1)))
        return real(qq, segs, out, **kw)

    monkeypatch.setattr(K, "flash_attn", spy)
    with torch.no_grad():
        out = T.standard_attention_forward(q.to(dev), k.to(dev), v.to(dev), mask=add.to(dev))
    torch.cuda.synchronize()
    assert len(seen) == 1 and seen[0][0] is None and tuple(seen[0][1]) == (1024, 700) and seen[0][2] == 1
    assert_bf16_close(out, ref, "per-row prefixes")
    assert cosine(out, ref) >= 0.9999


@pytest.mark.parametrize("Lq", [1152, 1024, 300], ids=["split_tail", "pair", "one_round"])
def test_flash_attn_key_lens_over_segments(dev, Lq):
    """ltx_flash_attn_fwd's key_lens over two key-major segments: row 0 stops
    inside the first segment (mid-tile), row 1 inside the second; the split
    tail (1152 queries), the pair kernel (1024) and a single round (300)
    against the oracle attending each row's keys alone."""
    from taomate_amd import kernels as K
    from taomate_amd.attention import _key_major
    B, H, D = 2, 32, 128
    L1, L2 = 1000, 1500
    lens = (613, 1000 + 877)
    g = torch.Generator().manual_seed(71)
    q = torch.randn(B, Lq, H, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, L1 + L2, H, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, L1 + L2, H, D, generator=g).to(torch.bfloat16)
    kd, vd = kc.to(dev), _key_major(vc.to(dev))     # segments share strides: views of one store
    segs = [K.KVSegment(kd[:, :L1], vd[:, :L1]), K.KVSegment(kd[:, L1:], vd[:, L1:])]
    out = torch.empty(B, Lq, H, D, device=dev, dtype=torch.bfloat16)
    K.flash_attn(q.to(dev), segs, out, key_lens=lens)
    torch.cuda.synchronize()
    for b in range(B):
        n = lens[b]
        ref = OA.standard_attention_forward(q[b:b + 1].float(), kc[b:b + 1, :n].float(), vc[b:b + 1, :n].float())
        assert_bf16_close(out[b:b + 1], ref, f"row {b} keeps {n}")
        assert cosine(out[b:b + 1], ref) >= 0.9999


def test_flash_attn_key_lens_rejections(dev):
    from taomate_amd import kernels as K
    q = torch.zeros(2, 128, 8, 128, device=dev, dtype=torch.bfloat16)
    k = torch.zeros(2, 64, 8, 128, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    with pytest.raises(ValueError, match="key_lens"):
        K.flash_attn(q, [K.KVSegment(k, k)], out, key_lens=(64, 65))
    # token-major V: the entry point refuses per-row counts
    from taomate_amd import _native as N
    with pytest.raises(N.NativeCallError, match="key_lens"):
        K.flash_attn(q, [K.KVSegment(k, k.clone())], out, key_lens=(64, 10))
