"""Packed q/k/v projections (CausalLTXAttention.fuse_qkv_) on the CPU: the
packing keeps every parameter's name and value, the one GEMM equals the three
(kv_cache.py:1406-1408), and anything that replaces a parameter ends the
packing instead of leaving the GEMM on stale weights."""
import os

import pytest
import torch

import taomate_amd as T
from taomate_amd import dit as D
from taomate_amd.attention import _project_qkv
from taomate_amd.checkpoint import load_generator, save_generator


def _module(seed=0, **kw):
    torch.manual_seed(seed)
    m = T.CausalLTXAttention(64, heads=2, dim_head=32, **kw)
    with torch.no_grad():
        for lin in (m.to_q, m.to_k, m.to_v):
            lin.bias.normal_()
    return m


def test_packing_keeps_values_and_matches_three_gemms():
    m = _module()
    before = {k: v.clone() for k, v in m.state_dict().items()}
    x = torch.randn(2, 5, 64)
    want = (m.to_q(x), m.to_k(x), m.to_v(x))
    m.fuse_qkv_()
    after = m.state_dict()
    assert before.keys() == after.keys()
    for k in before:
        assert torch.equal(before[k], after[k]), k
    w, b = m._packed_qkv()
    assert w.shape == (3 * 64, 64) and b.shape == (3 * 64,)
    assert m.to_k.weight.data_ptr() == w[64].data_ptr()   # a view, not a copy
    got = _project_qkv(m, x, x)
    assert got[0].stride(1) == 3 * 64                      # column views of one [B, L, 3n] output
    for g_, w_ in zip(got, want):
        torch.testing.assert_close(g_, w_, rtol=1e-6, atol=1e-6)
    # in-place updates of a projection reach the packed GEMM
    with torch.no_grad():
        m.to_v.weight.mul_(2.0)
    torch.testing.assert_close(_project_qkv(m, x, x)[2], m.to_v(x), rtol=1e-6, atol=1e-6)


def test_replacing_a_parameter_ends_the_packing():
    m = _module().fuse_qkv_()
    sd = {k: v.clone() * 3 for k, v in m.state_dict().items()}
    m.load_state_dict(sd, assign=True)
    assert m._packed_qkv() is None and m._qkv_packed is None
    x = torch.randn(1, 4, 64)
    for g_, w_ in zip(_project_qkv(m, x, x), (m.to_q(x), m.to_k(x), m.to_v(x))):
        assert torch.equal(g_, w_)
    m2 = _module().fuse_qkv_().to(torch.float64)
    assert m2._packed_qkv() is None


def test_cross_attention_and_foreign_context_stay_unpacked():
    m = T.CausalLTXAttention(64, context_dim=32, heads=2, dim_head=32).fuse_qkv_()
    assert getattr(m, "_qkv_packed", None) is None
    s = _module().fuse_qkv_()
    x, ctx = torch.randn(1, 3, 64), torch.randn(1, 7, 64)
    q, k, v = _project_qkv(s, x, ctx)   # K / V from another tensor: three GEMMs
    assert k.shape[1] == 7 and torch.equal(k, s.to_k(ctx))


def test_model_packs_every_self_attention_and_saves(tmp_path):
    cfg = D.AVConfig(num_layers=2, video_dim=128, audio_dim=64, video_heads=2, audio_heads=1, video_d_head=64,
                     audio_d_head=64, in_channels=8)
    model = D.AVModel(cfg)
    with torch.no_grad():   # the constructor leaves some tables uninitialised (possibly NaN)
        for p in model.parameters():
            p.normal_()
    before = {k: v.clone() for k, v in model.state_dict().items()}
    model.fuse_qkv_()
    packed = [n for n, m in model.named_modules() if isinstance(m, T.CausalLTXAttention) and m._packed_qkv()]
    assert sorted(packed) == sorted(f"transformer_blocks.{i}.{a}" for i in range(2) for a in ("attn1", "audio_attn1"))
    for ext in (".safetensors", ".pt"):
        path = os.path.join(tmp_path, "g" + ext)
        save_generator(model, path)
        back = load_generator(path, device="cpu", dtype=torch.float32)
        sd = back.state_dict()
        for k, v in before.items():
            assert torch.equal(sd[k], v), k


def test_all_blocks_modulation_equals_per_block():
    """_all_blocks_ada (one add per table kind over the stacked tables of every
    block) gives bit for bit the values of each block's get_ada_values /
    get_av_ca_ada_values (causal_block.py:434-481), in bf16 as the step runs."""
    cfg = D.AVConfig(num_layers=3, video_dim=128, audio_dim=64, video_heads=2, audio_heads=1, video_d_head=64,
                     audio_d_head=64, in_channels=8)
    torch.manual_seed(4)
    model = D.AVModel(cfg).to(torch.bfloat16)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_()
    B, T = 2, 1
    r = lambda *s: torch.randn(*s).to(torch.bfloat16)
    v_ts, a_ts = r(B, T, 6 * 128), r(B, T, 6 * 64)
    v_ss, v_gate, a_ss, a_gate = r(B, T, 4 * 128), r(B, T, 128), r(B, T, 4 * 64), r(B, T, 64)
    ada = D._all_blocks_ada(model.transformer_blocks, B, v_ts, a_ts, v_ss, v_gate, a_ss, a_gate)
    for blk, got in zip(model.transformer_blocks, ada):
        want = {"v": blk.get_ada_values(blk.scale_shift_table, B, v_ts, slice(0, 6)),
                "a": blk.get_ada_values(blk.audio_scale_shift_table, B, a_ts, slice(0, 6)),
                "a_ca": blk.get_av_ca_ada_values(blk.scale_shift_table_a2v_ca_audio, B, a_ss, a_gate),
                "v_ca": blk.get_av_ca_ada_values(blk.scale_shift_table_a2v_ca_video, B, v_ss, v_gate)}
        for k in want:
            assert len(got[k]) == len(want[k]), k
            for g_, w_ in zip(got[k], want[k]):
                assert g_.dtype == w_.dtype and torch.equal(g_, w_), k
        assert all(torch.equal(g_, w_) for g_, w_ in zip(got["v"][3:6],
                                                         blk.get_ada_values(blk.scale_shift_table, B, v_ts,
                                                                            slice(3, 6))))


def test_per_token_modulation_is_not_stacked_over_blocks():
    """With per-token timestep rows (a per-frame sigma expanded to the chunk's
    tokens) the values of all blocks are not built at once: _all_blocks_ada
    hands every block None, and each block's own get_ada_values gives the
    per-token values."""
    cfg = D.AVConfig(num_layers=2, video_dim=128, audio_dim=64, video_heads=2, audio_heads=1, video_d_head=64,
                     audio_d_head=64, in_channels=8)
    model = D.AVModel(cfg).to(torch.bfloat16)
    B, T = 2, 12
    r = lambda *s: torch.randn(*s).to(torch.bfloat16)
    ts = [r(B, T, 6 * 128), r(B, T, 6 * 64), r(B, T, 4 * 128), r(B, T, 128), r(B, T, 4 * 64), r(B, T, 64)]
    assert D._all_blocks_ada(model.transformer_blocks, B, *ts) == [None, None]


def test_per_frame_sigma_expands_to_tokens():
    """_expand_per_frame_to_per_token (causal_model.py:1365-1392): each frame's
    row repeated over its tokens; one row, or one row per token, unchanged."""
    t = torch.arange(2 * 3 * 4, dtype=torch.float32).view(2, 3, 4)
    e = D.AVModel._per_token(t, 12)
    assert e.shape == (2, 12, 4)
    for f in range(3):
        for i in range(4):
            assert torch.equal(e[:, 4 * f + i], t[:, f])
    assert D.AVModel._per_token(t, 3) is t
    one = t[:, :1]
    assert D.AVModel._per_token(one, 12) is one
    with pytest.raises(ValueError):
        D.AVModel._per_token(t, 10)


def test_audio_stream_switch_and_copies():
    """The audio-stream overlap is on by default, off on the CPU (no stream
    is made for a CPU device), switchable, and kept outside the module's
    attributes: a deep copy or a state dict of the model carries no stream."""
    import copy
    cfg = D.AVConfig(num_layers=1, video_dim=64, audio_dim=64, video_heads=1, audio_heads=1, video_d_head=64,
                     audio_d_head=64)
    m = D.AVModel(cfg)
    assert m._overlap_audio is True
    assert m._audio_stream_for(torch.device("cpu")) is None
    assert m.overlap_audio_(False) is m and m._overlap_audio is False
    m.overlap_audio_()
    m2 = copy.deepcopy(m)
    assert m2._overlap_audio is True
    assert not any(isinstance(v, dict) and v and all(hasattr(s, "cuda_stream") for s in v.values())
                   for v in vars(m2).values())
    assert set(m2.state_dict()) == set(m.state_dict())
