"""Pins the cache-bookkeeping and fp8 oracles (CPU): the reference's own known answers,
brute force over token ids, and the e4m3 format definition."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import cache as OC
from oracle import fp8 as OF

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _spans(blocks):
    return [(b.video_start, b.video_end, b.audio_start, b.audio_end) for b in blocks]


def test_av_blocks_reference_known_answers():
    # ltx_causal/attention/mask_builder.py:129-134 (OmniForcing 4-3-3-3, 16 frames)
    assert _spans(OC.compute_av_blocks(16, num_frame_per_block_first=4)) == [
        (0, 4, 0, 26), (4, 7, 26, 51), (7, 10, 51, 76), (10, 13, 76, 101), (13, 16, 101, 126)]
    # mask_builder.py:136-140 (legacy 1-3-3-3)
    assert _spans(OC.compute_av_blocks(16))[:3] == [(0, 1, 0, 1), (1, 4, 1, 26), (4, 7, 26, 51)]
    # mask_builder.py:252-255: 126 aligned audio frames in both layouts
    assert OC.compute_aligned_audio_frames(16, num_frame_per_block_first=4) == 126
    assert OC.compute_aligned_audio_frames(16) == 126
    # partial last block gets proportional audio (25 * 2 // 3 = 16)
    assert _spans(OC.compute_av_blocks(9, num_frame_per_block_first=4))[-1] == (7, 9, 51, 67)


@pytest.mark.parametrize("recent", [0, 1, 2, 3])
def test_retain_is_sink_plus_recent_bruteforce(recent):
    hw = (2, 3)
    for n in range(1, 9):
        plan = OC.streaming_plan(n, hw, recent_blocks=recent)
        blocks = OC.compute_av_blocks(4 + (n - 1) * 3, num_frame_per_block_first=4)[:n]
        # brute force: ids of block 0 plus the last `recent` committed blocks, in order
        keep = sorted({0} | set(range(max(1, n - recent), n)) if recent else {0})
        vid = [i for b in keep for i in range(blocks[b].video_start * 6, blocks[b].video_end * 6)]
        aid = [i for b in keep for i in range(blocks[b].audio_start, blocks[b].audio_end)]
        assert plan[-1]["video_ids"] == vid
        assert plan[-1]["audio_ids"] == aid
        assert [s["block_idx"] for s in plan[-1]["segments"]] == keep


def test_eviction_plan_golden():
    """Committed fixture of the 16x24-grid eviction plan (60 blocks): the plan
    reproduces it exactly (ids of every kept token after each commit)."""
    with open(os.path.join(GOLDEN, "eviction_plan_16x24_60.json")) as f:
        gold = json.load(f)
    plan = OC.streaming_plan(60, (16, 24))
    assert len(plan) == len(gold) == 60
    for got, exp in zip(plan, gold):
        assert got["segments"] == exp["segments"]
        assert got["video_ids"][:3] == exp["video_head"] and len(got["video_ids"]) == exp["video_len"]
        assert sum(got["video_ids"]) == exp["video_sum"] and sum(got["audio_ids"]) == exp["audio_sum"]


def test_e4m3_codes_roundtrip_and_format():
    codes = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).to(torch.float64)
    defn = torch.tensor([OF.e4m3_value(c) for c in range(256)], dtype=torch.float64)
    nan = torch.isnan(defn)
    assert nan.sum() == 2 and torch.isnan(vals[nan]).all()
    assert torch.equal(vals[~nan], defn[~nan])
    assert defn[~nan].abs().max() == 448 and OF.e4m3_value(0x08) == 2 ** -6 and OF.e4m3_value(1) == 2 ** -9
    # every finite code survives an encode of its own value
    back = vals[~nan].to(torch.float32).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(back, codes[~nan])


def test_e4m3_rounding_is_nearest_even():
    pos = sorted({OF.e4m3_value(c) for c in range(0x7F)})
    for a, b in zip(pos[:-1], pos[1:]):
        mid = torch.tensor([(a + b) / 2], dtype=torch.float32)
        got = mid.to(torch.float8_e4m3fn).to(torch.float64).item()
        ca = [c for c in range(0x7F) if OF.e4m3_value(c) == a][0]
        assert got == (a if ca % 2 == 0 else b)   # ties go to the even code
        assert torch.tensor([a + (b - a) * 0.26]).to(torch.float8_e4m3fn).to(torch.float64).item() == a


def test_quantize_kv_scales_and_error_bound():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 768, 4, 64, generator=g) * 3
    x[1, :384, 2] = 0
    codes, sc = OF.quantize_kv(x, 384)
    assert sc.shape == (2, 4, 2)
    amax = x.view(2, 2, 384, 4, 64).abs().amax(dim=(2, 4)).permute(0, 2, 1)
    assert torch.equal(sc[1, 2, 0], torch.tensor(1.0))
    nz = amax > 0
    assert torch.equal(sc[nz], (amax / 448)[nz])
    y = OF.dequantize_kv(codes, sc, 384)
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 for normals; abs <= 2^-10 * scale below
    s_tok = sc.permute(0, 2, 1).repeat_interleave(384, 1).unsqueeze(-1)
    err = (y - x).abs()
    assert torch.all(err <= x.abs() * 2 ** -4 + s_tok * 2 ** -10 + 1e-12)


def test_fp8_reciprocal_fast_path_argument():
    """The fp8 quantiser multiplies by r = fl(1/scale) and divides exactly only
    when fl(x*r) lies within 4 ulp of an e4m3 rounding midpoint (low 20
    mantissa bits in [0x7FFFC, 0x80004]) or below 2^-6.  Emulated here in
    float32 on quotients placed at and around every midpoint under awkward
    scales: the e4m3 codes equal those of fl(x/scale)."""
    g = torch.Generator().manual_seed(3)
    grid = sorted({OF.e4m3_value(c) for c in range(0x7F)})
    g64 = torch.tensor(grid, dtype=torch.float64)
    mids = ((g64[1:] + g64[:-1]) / 2).float()
    inf = torch.tensor(float("inf"))
    for m in torch.rand(200, generator=g) * 1e3 + 1e-4:
        sc = (m.float() / 448.0).float()
        x = (mids * sc).float()
        for _ in range(int(torch.randint(0, 6, (1,), generator=g))):
            x = torch.nextafter(x, inf if torch.rand(1, generator=g) < 0.5 else -inf)
        x = torch.cat([x, -x, torch.randn(4096, generator=g) * m])
        q = x / sc
        r = (torch.tensor(1.0) / sc).float()
        qf = x * r
        a = qf.abs()
        low = a.view(torch.int32) & 0xFFFFF
        near = (a < 2.0 ** -6) | ((low >= 0x7FFFC) & (low <= 0x80004))
        qf = torch.where(near, q, qf)
        c_exact = q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        c_fast = qf.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(c_exact, c_fast)
    # a window that is too narrow is caught (planted mistake)
    sc = torch.tensor(3.7 / 448.0, dtype=torch.float32)
    x = (mids * sc).float()
    q, qf = x / sc, x * (torch.tensor(1.0) / sc).float()
    assert not torch.equal(q.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8),
                           qf.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8))


@pytest.mark.parametrize("window_frames,memory_frames,refresh", [(12, 2, 4), (6, 1, 2), (3, 0, 0), (9, 2, 1)])
def test_stream_plan_bruteforce(window_frames, memory_frames, refresh):
    """The anchor | memory | window plan equals its definition written out
    directly: the anchor frames, the memory frames and the newest
    window_frames / 3 chunks, in frame order; the memory version counts the
    refreshes so far."""
    hw = (2, 3)
    per = 6
    for n in range(1, 11):
        plan = OC.streaming_plan_window(n, hw, anchor_frames=1, memory_frames=memory_frames,
                                        window_frames=window_frames, refresh_every=refresh)
        last = plan[-1]
        keep_chunks = list(range(max(0, n - window_frames // 3), n))
        frames = [0] + [1 + i for i in range(memory_frames)]
        for c in keep_chunks:
            f0 = 1 + memory_frames + 3 * c
            frames += [f0, f0 + 1, f0 + 2]
        assert last["video_ids"] == [f * per + t for f in frames for t in range(per)]
        assert [s["kind"] for s in last["segments"]] == ["prefix", "memory"] + ["generated"] * len(keep_chunks)
        assert [s.get("window_slot") for s in last["segments"][2:]] == keep_chunks
        assert last["memory_version"] == (n // refresh if refresh else 0)


def test_stream_plan_golden():
    """Committed fixture of the 16x24 anchor | memory | window stream (60 chunks)."""
    with open(os.path.join(GOLDEN, "stream_plan_16x24_60.json")) as f:
        gold = json.load(f)
    plan = OC.streaming_plan_window(60, (16, 24))
    assert len(plan) == len(gold) == 60
    for got, exp in zip(plan, gold):
        assert got["segments"] == exp["segments"] and got["memory_version"] == exp["memory_version"]
        v = got["video_ids"]
        assert v[:3] == exp["video_head"] and v[-3:] == exp["video_tail"] and len(v) == exp["video_len"]
        assert sum(v) == exp["video_sum"]
    # steady state: anchor 384 + memory 768 + window 4608 keys before each chunk's own 1152
    assert gold[-1]["video_len"] == 384 + 768 + 4608
