"""Pins of the oracle's projection, output, modulation and block composition
against closed forms and special cases (CPU).  Every check is also run on a
planted mistake (a mutant of the oracle function) and must fail there:

* project_qkv (causal_attention.py:100-102): with x != ctx, q comes from x
  and K/V only from ctx; distinct scalar weights give exact values, and a
  swapped W_k / W_v is caught;
* finish_output (kv_cache.py:1680-1700): a per-head gate 2*sigmoid(logit)
  doubles exactly the head whose logit is large and leaves a head with
  logit 0 unchanged; a gate applied to the wrong head axis is caught;
* ada_values / av_ca_values (causal_block.py:434-481): one-hot table rows
  and per-row timestep constants land each value in its known slot; a
  transposed timestep reshape is caught;
* block_forward (kv_cache.py:2145-2656): with every attention's output
  projection zeroed the block is its two FFN paths in closed form; with one
  video and one audio token every attention is over a single key, so each
  returns to_out(to_v(context)) and the whole block has a closed form that
  fixes the order of the residuals, in particular that V2A reads the video
  norm taken before the A2V update (kv_cache.py:2588-2590) and that the
  text residuals land before the cross-modal norms (:2530-2540).
"""
import math
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as OA
from oracle import dit as OD


def _eye_weights(d, heads, wq=1.0, wk=2.0, wv=3.0, wo=1.0, gate=None):
    eye = torch.eye(d)
    z = torch.zeros(d)
    return OA.AttnWeights(wq * eye, z + 0.5, wk * eye, z - 0.25, wv * eye, z + 1.0, wo * eye, z, torch.ones(d),
                          torch.ones(d), heads, d // heads,
                          wg=None if gate is None else gate[0], bg=None if gate is None else gate[1])


def _check_project(fn) -> bool:
    g = torch.Generator().manual_seed(1)
    x, ctx = torch.randn(2, 5, 8, generator=g), torch.randn(2, 3, 8, generator=g)
    w = _eye_weights(8, 2)
    q, k, v = fn(w, x, ctx)
    ok = torch.allclose(q, x + 0.5) and torch.allclose(k, 2 * ctx - 0.25) and torch.allclose(v, 3 * ctx + 1.0)
    q2, k2, v2 = fn(w, x + 7.0, ctx)     # K/V must not depend on x
    return ok and torch.equal(k2, k) and torch.equal(v2, v) and not torch.equal(q2, q)


def test_project_qkv_pins():
    assert _check_project(OA.project_qkv)

    def swapped(w, x, ctx):
        return F.linear(x, w.wq, w.bq), F.linear(ctx, w.wv, w.bv), F.linear(ctx, w.wk, w.bk)

    def from_x(w, x, ctx):
        return F.linear(x, w.wq, w.bq), F.linear(x[:, :ctx.shape[1]], w.wk, w.bk), F.linear(ctx, w.wv, w.bv)

    assert not _check_project(swapped)
    assert not _check_project(from_x)


def _check_finish(fn) -> bool:
    H, Dh, B, L = 4, 3, 2, 5
    d = H * Dh
    g = torch.Generator().manual_seed(2)
    out = torch.randn(B, L, H, Dh, generator=g)
    x = torch.randn(B, L, d, generator=g)
    wg = torch.zeros(H, d)
    bg = torch.tensor([0.0, 60.0, 0.0, -60.0])      # heads 1 and 3: gate 2 and 0
    w = _eye_weights(d, H, gate=(wg, bg))
    y = fn(w, out, x).view(B, L, H, Dh)
    want = out.clone()
    want[:, :, 1] *= 2.0
    want[:, :, 3] = 0.0
    return torch.allclose(y, want, atol=1e-6)


def test_finish_output_gate_pins():
    assert _check_finish(OA.finish_output)

    def wrong_axis(w, out, x):
        B = x.shape[0]
        o = out.reshape(B, -1, w.heads * w.dim_head)
        g = 2.0 * torch.sigmoid(F.linear(x, w.wg, w.bg))
        b, t, _ = o.shape
        o = (o.view(b, t, w.dim_head, w.heads) * g.unsqueeze(-2)).reshape(b, t, -1)
        return F.linear(o, w.wo, w.bo)

    assert not _check_finish(wrong_axis)


def _check_ada(fn_ada, fn_ca) -> bool:
    B, T, D = 2, 3, 5
    n = 6
    table = torch.zeros(n, D)
    for i in range(n):
        table[i, i % D] = 1.0                          # one-hot rows
    ts = torch.zeros(B, T, n, D)
    for i in range(n):
        ts[:, :, i, :] = 10.0 * (i + 1)               # per-row constants
    vals = fn_ada(table, B, ts.reshape(B, T, n * D), slice(0, n))
    ok = len(vals) == n
    for i, v in enumerate(vals):
        want = torch.full((B, T, D), 10.0 * (i + 1))
        want[..., i % D] += 1.0
        ok = ok and torch.equal(v, want)
    sub = fn_ada(table, B, ts.reshape(B, T, n * D), slice(3, 6))
    ok = ok and torch.equal(sub[0], vals[3]) and torch.equal(sub[2], vals[5])
    # av_ca: 4 scale/shift rows from ss, the gate row from its own timestep
    tab5 = table[:5]
    ss = ts[:, :, :4].reshape(B, T, 4 * D)
    gate = torch.full((B, T, D), -7.0)
    ca = fn_ca(tab5, B, ss, gate)
    ok = ok and len(ca) == 5 and torch.equal(ca[2], vals[2])
    want_g = torch.full((B, T, D), -7.0)
    want_g[..., 4 % D] += 1.0
    return ok and torch.equal(ca[4], want_g)


def test_ada_values_pins():
    assert _check_ada(OD.ada_values, OD.av_ca_values)

    def transposed(table, batch, ts, idx):
        n = table.shape[0]
        t = ts.reshape(batch, ts.shape[1], -1, n).transpose(-1, -2)
        return (table[idx][None, None] + t[:, :, idx, :]).unbind(dim=2)

    def ca_with(fn):
        return lambda table, batch, ss, gate: (*fn(table[:4], batch, ss, slice(None)),
                                               *fn(table[4:], batch, gate, slice(None)))

    assert not _check_ada(transposed, ca_with(transposed))

    def gate_from_ss(table, batch, ss, gate):
        return (*OD.ada_values(table[:4], batch, ss, slice(None)),
                *OD.ada_values(table[4:], batch, ss[..., :gate.shape[-1]], slice(None)))

    assert not _check_ada(OD.ada_values, gate_from_ss)


# ---------------------------------------------------------------------------
# block composition
# ---------------------------------------------------------------------------

def _cfg(vd=16, ad=8, vh=2, ah=2):
    return SimpleNamespace(norm_eps=1e-6, video_heads=vh, video_d_head=vd // vh, audio_heads=ah,
                           audio_d_head=ad // ah, learned_memory_mode=None)


ATTNS = [("attn1.", "v", "v"), ("attn2.", "v", "v"), ("audio_attn1.", "a", "a"), ("audio_attn2.", "a", "a"),
         ("audio_to_video_attn.", "v", "a"), ("video_to_audio_attn.", "a", "v")]


def _block_params(vd, ad, g, zero_out=False):
    """Random weights for one block; cross-modal attentions project into the
    audio width (causal_block.py:353-372)."""
    r = lambda *s: torch.randn(*s, generator=g) * 0.3
    p = {}
    dims = {"v": vd, "a": ad}
    for name, qs, ks in ATTNS:
        inner = ad if name in ("audio_to_video_attn.", "video_to_audio_attn.") else dims[qs]
        p[name + "to_q.weight"], p[name + "to_q.bias"] = r(inner, dims[qs]), r(inner)
        p[name + "to_k.weight"], p[name + "to_k.bias"] = r(inner, dims[ks]), r(inner)
        p[name + "to_v.weight"], p[name + "to_v.bias"] = r(inner, dims[ks]), r(inner)
        p[name + "q_norm.weight"], p[name + "k_norm.weight"] = 1 + r(inner), 1 + r(inner)
        p[name + "to_out.0.weight"] = torch.zeros(dims[qs], inner) if zero_out else r(dims[qs], inner)
        p[name + "to_out.0.bias"] = torch.zeros(dims[qs]) if zero_out else r(dims[qs])
    for pre, d in (("ff.", vd), ("audio_ff.", ad)):
        p[pre + "net.0.proj.weight"], p[pre + "net.0.proj.bias"] = r(4 * d, d), r(4 * d)
        p[pre + "net.2.weight"], p[pre + "net.2.bias"] = r(d, 4 * d), r(d)
    p["scale_shift_table"], p["audio_scale_shift_table"] = r(6, vd), r(6, ad)
    p["scale_shift_table_a2v_ca_video"], p["scale_shift_table_a2v_ca_audio"] = r(5, vd), r(5, ad)
    return p


def _inputs(B, Lv, La, vd, ad, g, Lctx=1):
    r = lambda *s: torch.randn(*s, generator=g)
    return dict(vx=r(B, Lv, vd), ax=r(B, La, ad), v_ts=r(B, 1, 6 * vd) * 0.2, a_ts=r(B, 1, 6 * ad) * 0.2,
                v_ss=r(B, 1, 4 * vd) * 0.2, v_gate=r(B, 1, vd) * 0.2, a_ss=r(B, 1, 4 * ad) * 0.2,
                a_gate=r(B, 1, ad) * 0.2, vctx=r(B, Lctx, vd), actx=r(B, Lctx, ad))


def _run_block(p, cfg, x, vpe=None, ape=None, vcpe=None, acpe=None):
    vx, ax, _ = OD.block_forward(p, "", cfg, x["vx"], x["ax"], x["v_ts"], x["a_ts"], vpe, ape, vcpe, acpe,
                                 x["vctx"], x["actx"], None, None, x["v_ss"], x["v_gate"], x["a_ss"],
                                 x["a_gate"], {})
    return vx, ax


def _ffn_path(p, x, eps=1e-6):
    """Both streams with every attention output zero: x + FFN(rms(x)(1+sc)+sh)*g,
    (sh, sc, g) the table rows 3..5 plus their timestep slices."""
    B = x["vx"].shape[0]
    out = []
    for s, tab, ts, ff in (("vx", "scale_shift_table", "v_ts", "ff."), ("ax", "audio_scale_shift_table", "a_ts",
                                                                         "audio_ff.")):
        d = x[s].shape[-1]
        t = p[tab][None, None] + x[ts].reshape(B, 1, p[tab].shape[0], d)
        sh, sc, g = t[:, :, 3], t[:, :, 4], t[:, :, 5]
        out.append(x[s] + OD.feed_forward(p, ff, OD.rms_norm(x[s], eps) * (1 + sc) + sh) * g)
    return out


def test_block_with_zero_attention_outputs_is_its_ffn_path():
    g = torch.Generator().manual_seed(3)
    vd, ad = 16, 8
    cfg = _cfg(vd, ad)
    p = _block_params(vd, ad, g, zero_out=True)
    x = _inputs(2, 6, 4, vd, ad, g, Lctx=5)
    vx, ax = _run_block(p, cfg, x)
    wv, wa = _ffn_path(p, x)
    torch.testing.assert_close(vx, wv, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ax, wa, rtol=1e-5, atol=1e-5)


def _one_key(p, name, ctx):
    """Attention over a single key: softmax weight 1, so the output is
    to_out(to_v(ctx)) whatever the queries (no gate)."""
    v = F.linear(ctx, p[name + "to_v.weight"], p[name + "to_v.bias"])
    return F.linear(v, p[name + "to_out.0.weight"], p[name + "to_out.0.bias"])


def _one_token_block(p, x, eps=1e-6, v2a_after_a2v=False, text=None):
    """The block for one video and one audio token written from the
    reference's order (kv_cache.py:2194-2633) with every attention over one
    key.  ``v2a_after_a2v`` plants a mistake: V2A reading the video norm taken
    after the A2V residual.  ``text``: the two text terms, when not the plain
    to_out(to_v(context)) (the prompt-AdaLN ones)."""
    B = x["vx"].shape[0]
    vd, ad = x["vx"].shape[-1], x["ax"].shape[-1]
    rms = lambda t: OD.rms_norm(t, eps)
    nv, na = p["scale_shift_table"].shape[0], p["audio_scale_shift_table"].shape[0]
    vt = p["scale_shift_table"][None, None] + x["v_ts"].reshape(B, 1, nv, vd)
    at = p["audio_scale_shift_table"][None, None] + x["a_ts"].reshape(B, 1, na, ad)
    vx, ax = x["vx"], x["ax"]
    vx = vx + _one_key(p, "attn1.", rms(vx) * (1 + vt[:, :, 1]) + vt[:, :, 0]) * vt[:, :, 2]
    v_text = _one_key(p, "attn2.", x["vctx"]) if text is None else text[0]
    ax = ax + _one_key(p, "audio_attn1.", rms(ax) * (1 + at[:, :, 1]) + at[:, :, 0]) * at[:, :, 2]
    a_text = _one_key(p, "audio_attn2.", x["actx"]) if text is None else text[1]
    vx, ax = vx + v_text, ax + a_text
    vca = p["scale_shift_table_a2v_ca_video"][None, None] + torch.cat(
        [x["v_ss"].reshape(B, 1, 4, vd), x["v_gate"].reshape(B, 1, 1, vd)], 2)
    aca = p["scale_shift_table_a2v_ca_audio"][None, None] + torch.cat(
        [x["a_ss"].reshape(B, 1, 4, ad), x["a_gate"].reshape(B, 1, 1, ad)], 2)
    vn, an = rms(vx), rms(ax)
    a2v = _one_key(p, "audio_to_video_attn.", an * (1 + aca[:, :, 0]) + aca[:, :, 1])
    vx = vx + a2v * vca[:, :, 4]
    vn_v2a = rms(vx) if v2a_after_a2v else vn
    v2a = _one_key(p, "video_to_audio_attn.", vn_v2a * (1 + vca[:, :, 2]) + vca[:, :, 3])
    ax = ax + v2a * aca[:, :, 4]
    return _ffn_path(p, dict(x, vx=vx, ax=ax), eps)


def test_block_over_single_keys_has_the_reference_order():
    g = torch.Generator().manual_seed(4)
    vd, ad = 16, 8
    cfg = _cfg(vd, ad)
    p = _block_params(vd, ad, g)
    x = _inputs(2, 1, 1, vd, ad, g, Lctx=1)
    vx, ax = _run_block(p, cfg, x)
    wv, wa = _one_token_block(p, x)
    torch.testing.assert_close(vx, wv, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ax, wa, rtol=1e-5, atol=1e-5)
    # the planted ordering mistake gives a different audio stream
    _, bad_a = _one_token_block(p, x, v2a_after_a2v=True)
    assert (bad_a - wa).abs().max().item() > 1e-3


def test_block_returns_the_committed_cache():
    """block_forward's new cache is each field with this chunk's K/V appended:
    the video self K is the chunk's normalised keys after the cached ones."""
    g = torch.Generator().manual_seed(5)
    vd, ad = 16, 8
    cfg = _cfg(vd, ad)
    p = _block_params(vd, ad, g)
    x = _inputs(1, 3, 2, vd, ad, g, Lctx=2)
    _, _, c1 = OD.block_forward(p, "", cfg, x["vx"], x["ax"], x["v_ts"], x["a_ts"], None, None, None, None,
                                x["vctx"], x["actx"], None, None, x["v_ss"], x["v_gate"], x["a_ss"], x["a_gate"], {})
    assert c1["video_self_k"].shape == (1, 3, 2, 8) and c1["audio_self_v"].shape == (1, 2, 2, 4)
    assert c1["a2v_k"].shape == (1, 2, 2, 4) and c1["v2a_k"].shape == (1, 3, 2, 4)
    _, _, c2 = OD.block_forward(p, "", cfg, x["vx"], x["ax"], x["v_ts"], x["a_ts"], None, None, None, None,
                                x["vctx"], x["actx"], None, None, x["v_ss"], x["v_gate"], x["a_ss"], x["a_gate"], c1)
    assert c2["video_self_k"].shape == (1, 6, 2, 8)
    assert torch.equal(c2["video_self_k"][:, :3], c1["video_self_k"])
    assert torch.equal(c2["video_self_k"][:, 3:], c1["video_self_k"])   # same inputs, same keys


def test_memory_ema_rule_special_cases():
    """_ema_update (learned_memory.py:231-249): beta 0 keeps the state, beta 1
    takes the new frames, tether 1 returns the anchor, and one step with the
    streaming settings (0.15, 0.20) is the two-stage closed form; a tether
    applied before the EMA (a plausible slip) differs."""
    from oracle import stream as OS
    g = torch.Generator().manual_seed(6)
    prev, anchor, cur = (torch.randn(2, 5, 4, generator=g) for _ in range(3))
    assert torch.equal(OS.ema_update(prev, None, cur, 0.0, 0.0), prev)
    assert torch.equal(OS.ema_update(prev, None, cur, 1.0, 0.0), cur)
    torch.testing.assert_close(OS.ema_update(prev, anchor, cur, 0.3, 1.0), anchor)
    got = OS.ema_update(prev, anchor, cur, 0.15, 0.20)
    want = 0.8 * (0.85 * prev + 0.15 * cur) + 0.2 * anchor
    torch.testing.assert_close(got, want)
    slip = 0.85 * (0.8 * prev + 0.2 * anchor) + 0.15 * cur
    assert (got - slip).abs().max().item() > 1e-3


def _adaln_text_case(g, vd=16, ad=8, B=2):
    """One block with the LTX-2.3 prompt AdaLN: 9-row tables, prompt tables,
    prompt timesteps; one video and one audio token, one text key each."""
    p = _block_params(vd, ad, g)
    r = lambda *s: torch.randn(*s, generator=g) * 0.3
    p["scale_shift_table"], p["audio_scale_shift_table"] = r(9, vd), r(9, ad)
    p["prompt_scale_shift_table"], p["audio_prompt_scale_shift_table"] = r(2, vd), r(2, ad)
    x = _inputs(B, 1, 1, vd, ad, g, Lctx=1)
    x["v_ts"], x["a_ts"] = r(B, 1, 9 * vd), r(B, 1, 9 * ad)
    x["v_prompt"], x["a_prompt"] = r(B, 1, 2 * vd), r(B, 1, 2 * ad)
    return p, x


def _adaln_text_closed_form(p, x, stream="v", slip=None):
    """The text cross-attention term of one stream over a single text key
    (kv_cache.py:1090-1141): softmax weight 1, so the output is
    to_out(to_v(ctx * (1 + scale_kv) + shift_kv)) * gate, (shift_kv, scale_kv)
    = prompt table + prompt timestep in that order, gate = row 8 of the block's
    table + its timestep slice.  ``slip``: "kv_order" swaps shift and scale,
    "no_gate" drops the gate, "rows_3_5" takes the gate from row 5."""
    B = x["vx"].shape[0]
    tab, ptab, ts, pts, ctx, attn = (("scale_shift_table", "prompt_scale_shift_table", "v_ts", "v_prompt", "vctx",
                                      "attn2.") if stream == "v" else
                                     ("audio_scale_shift_table", "audio_prompt_scale_shift_table", "a_ts",
                                      "a_prompt", "actx", "audio_attn2."))
    d = x[ctx].shape[-1]
    kv = p[ptab][None, None] + x[pts].reshape(B, 1, 2, d)
    sh, sc = kv[:, :, 0], kv[:, :, 1]
    if slip == "kv_order":
        sh, sc = sc, sh
    t9 = p[tab][None, None] + x[ts].reshape(B, 1, 9, d)
    gate = t9[:, :, 5] if slip == "rows_3_5" else t9[:, :, 8]
    out = _one_key(p, attn, x[ctx] * (1 + sc) + sh)
    return out if slip == "no_gate" else out * gate


def test_adaln_text_cross_over_one_key():
    """With the LTX-2.3 prompt AdaLN the text term of each stream is the closed
    form above; the planted slips (shift / scale of the context swapped, the
    gate dropped, the gate taken from the feed-forward rows) all differ."""
    g = torch.Generator().manual_seed(9)
    p, x = _adaln_text_case(g)
    B, vd, ad = 2, 16, 8
    for stream in ("v", "a"):
        d = vd if stream == "v" else ad
        xs = x["vx"] if stream == "v" else x["ax"]
        got = OD.text_cross(p, "", "attn2." if stream == "v" else "audio_attn2.",
                            "scale_shift_table" if stream == "v" else "audio_scale_shift_table",
                            "prompt_scale_shift_table" if stream == "v" else "audio_prompt_scale_shift_table", B,
                            x["v_ts"] if stream == "v" else x["a_ts"], x["v_prompt"] if stream == "v" else x["a_prompt"],
                            xs, x["vctx"] if stream == "v" else x["actx"], None, 2, d // 2, 1e-6)
        want = _adaln_text_closed_form(p, x, stream)
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
        for slip in ("kv_order", "no_gate", "rows_3_5"):
            assert (got - _adaln_text_closed_form(p, x, stream, slip)).abs().max().item() > 1e-3, (stream, slip)
    # and inside the block: the one-token block with the text terms replaced by these
    vx, ax, _ = OD.block_forward(p, "", _cfg(vd, ad), x["vx"], x["ax"], x["v_ts"], x["a_ts"], None, None, None,
                                 None, x["vctx"], x["actx"], None, None, x["v_ss"], x["v_gate"], x["a_ss"],
                                 x["a_gate"], {}, v_prompt=x["v_prompt"], a_prompt=x["a_prompt"])
    text = (_adaln_text_closed_form(p, x, "v"), _adaln_text_closed_form(p, x, "a"))
    wv, wa = _one_token_block(p, x, text=text)
    torch.testing.assert_close(vx, wv, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ax, wa, rtol=1e-5, atol=1e-5)
