"""GPU parity of the 60-chunk anchor | memory | window | current stream (one
attention layer, 8 heads x 64, 3-frame chunks, 12-frame window, 2 memory
frames re-prefilled every 4 chunks) against the fp32 oracle replay of the same
policy: every chunk's output, the final cache contents and the segment list.
bf16 and fp8-e4m3 K/V on the 8x12 latent grid (96-token frames: the fp8
kernel cuts its 64-key tiles at frame boundaries, 64 + 32 per frame), fp8
also on 8x16 (128-token frames, two whole tiles)."""
import pytest
import torch

from oracle import stream as OS
from taomate_amd.streaming import ChunkStream

from .helpers import BF16_MAX_ABS, FP8_COSINE, assert_bf16_close, cosine, diff_stats
from .test_gpu_layer import make_layer

pytestmark = pytest.mark.gpu

B, H, DH, N_CHUNKS = 1, 8, 64, 60


def _inputs_and_reference(w, grid):
    """Seeded inputs (bf16-representable, so both sides read the same values)
    and the oracle's outputs."""
    g = torch.Generator().manual_seed(51)
    hw, d = grid[0] * grid[1], H * DH
    r = lambda nf: torch.randn(B, nf * hw, d, generator=g).to(torch.bfloat16).float()
    xa, xm = r(1), r(2)
    chunks = [r(3) for _ in range(N_CHUNKS)]
    return xa, xm, chunks, OS.run_stream(w, grid, xa, xm, chunks)


@pytest.mark.parametrize("kv_dtype,grid", [("bf16", (8, 12)), ("fp8", (8, 12)), ("fp8", (8, 16))],
                         ids=["bf16_8x12", "fp8_8x12", "fp8_8x16"])
def test_chunk_stream_60_chunks(dev, kv_dtype, grid):
    attn, w = make_layer(dev, H * DH, H, DH, 50)
    if kv_dtype == "fp8":
        attn.fuse_qkv_()   # packed q/k/v GEMM, memory re-prefill included (bf16 keeps three GEMMs)
    xa, xm, chunks, (ref_outs, ref_k, ref_v, ref_segs) = _inputs_and_reference(w, grid)
    st = ChunkStream(attn, grid, B, dev, kv_dtype=kv_dtype)
    worst = 1.0
    with torch.no_grad():
        st.prefill(xa.to(dev, torch.bfloat16), xm.to(dev, torch.bfloat16))
        for c, x in enumerate(chunks):
            out = st.step(x.to(dev, torch.bfloat16))
            cs = cosine(out, ref_outs[c])
            worst = min(worst, cs)
            if kv_dtype == "bf16":
                assert_bf16_close(out, ref_outs[c], f"chunk {c}")
                assert cs >= 0.9999, (c, cs)
            else:
                assert cs >= FP8_COSINE, (c, cs)
                assert diff_stats(out, ref_outs[c])[0] <= BF16_MAX_ABS, c
    assert st.segments == ref_segs
    assert st.memory_version == N_CHUNKS // 4
    bar = 0.9999 if kv_dtype == "bf16" else FP8_COSINE
    assert cosine(st.k.materialize(), ref_k) >= bar
    assert cosine(st.v.materialize(), ref_v) >= bar
    print(f"{kv_dtype}: worst per-chunk cosine {worst:.6f}")


@pytest.mark.timeout(1200)
def test_chunk_stream_60_chunks_full_size_fp8(dev):
    """The long-stream workload at its real shape: one 32 x 128 video
    self-attention layer (d = 4096, B = 2) on the 16x24 latent grid, fp8-e4m3
    K/V, 60 chunks of 3 frames, anchor 1 frame | memory 2 frames re-prefilled
    every 4 chunks | 12-frame window (6912 keys at the steady state), packed
    q/k/v.  Every 4th chunk's output (and the last) against the fp32 oracle
    replay at cosine >= 0.999; the segment list after every chunk bit-exact
    against the committed plan fixture; the final cache and memory version."""
    import json
    import os
    Bf, Hf, Df, grid = 2, 32, 128, (16, 24)
    hw, d = grid[0] * grid[1], Hf * Df
    attn, w = make_layer(dev, d, Hf, Df, 52)
    attn.fuse_qkv_()
    g = torch.Generator().manual_seed(53)
    r = lambda nf: torch.randn(Bf, nf * hw, d, generator=g).to(torch.bfloat16).float()
    xa, xm = r(1), r(2)
    chunks = [r(3) for _ in range(N_CHUNKS)]
    checked = lambda c: c % 4 == 3 or c == N_CHUNKS - 1
    print("full-size stream: oracle replay", flush=True)
    ref_outs, ref_k, ref_v, ref_segs = OS.run_stream(w, grid, xa, xm, chunks, outputs_for=checked)
    with open(os.path.join(os.path.dirname(__file__), "golden", "stream_plan_16x24_60.json")) as f:
        plan = json.load(f)
    st = ChunkStream(attn, grid, Bf, dev, kv_dtype="fp8")
    worst = 1.0
    with torch.no_grad():
        st.prefill(xa.to(dev, torch.bfloat16), xm.to(dev, torch.bfloat16))
        for c, x in enumerate(chunks):
            out = st.step(x.to(dev, torch.bfloat16))
            assert st.segments == plan[c]["segments"], c
            assert st.memory_version == plan[c]["memory_version"], c
            assert st.k.shape[1] == plan[c]["video_len"], c
            if checked(c):
                cs = cosine(out, ref_outs[c])
                worst = min(worst, cs)
                assert cs >= FP8_COSINE, (c, cs)
                assert diff_stats(out, ref_outs[c])[0] <= BF16_MAX_ABS, c
    assert st.segments == ref_segs
    assert st.k.shape[1] == (1 + 2 + 12) * hw     # anchor | memory | window: 5760 cached keys
    assert cosine(st.k.materialize(), ref_k) >= FP8_COSINE
    assert cosine(st.v.materialize(), ref_v) >= FP8_COSINE
    print(f"full-size fp8 stream: worst checked-chunk cosine {worst:.6f}", flush=True)
