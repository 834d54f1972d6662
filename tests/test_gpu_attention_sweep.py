"""Seeded sweep of the attention entry point over many small shapes against an
fp32 reference: batch rows, heads, head dim 64 / 128, query counts on and off
the 32 / 128-query boundaries, one to six key segments of ragged lengths with
gaps between their spans, token-major and key-major V, per-row key counts,
and fp8 K/V with frames of 25, 64, 96 and 384 tokens.  The shapes take every
launch plan of the kernels: a single partial round (cut into key ranges or
not), whole rounds with a split tail, the staged, pipelined and framed
kernels.  The configurations come from a fixed generator, so the sweep is the
same on every run."""
import math
import random

import pytest
import torch

from oracle import fp8 as OF
from taomate_amd import kernels
from taomate_amd.kernels import KVSegment

from .helpers import assert_bf16_close, gen, randn

pytestmark = pytest.mark.gpu

EDGE_LQ = [1, 31, 32, 33, 75, 127, 128, 129, 255, 256, 257, 640]
EDGE_LEN = [1, 7, 8, 9, 63, 64, 65, 100, 127, 128, 129, 384, 700]


def _cases():
    rnd = random.Random(20261202)
    cases = []
    i = 0
    while len(cases) < 120:
        i += 1
        kind = "fp8" if i % 4 == 3 else ("key" if i % 2 else "token")
        D = rnd.choice([64, 128])
        H = rnd.choice([1, 2, 4, 8, 8, 32]) if i % 9 else 32
        B = rnd.choice([1, 2, 2, 3])
        Lq = rnd.choice(EDGE_LQ) if rnd.random() < 0.6 else rnd.randint(1, 700)
        nseg = rnd.randint(1, 6)
        frame = 0
        if kind == "fp8":
            frame = rnd.choice([25, 64, 96, 384])
            # segments of whole frames, the last one possibly ending mid-frame
            lens = [frame * rnd.randint(1, 3 if frame < 384 else 1) for _ in range(nseg)]
            lens[-1] -= rnd.randint(0, frame - 1) if frame > 1 else 0
            lens = [max(1, n) for n in lens]
        else:
            lens = [rnd.choice(EDGE_LEN) if rnd.random() < 0.5 else rnd.randint(1, 600) for _ in range(nseg)]
        key_lens = None
        if kind == "key" and rnd.random() < 0.4:
            lk = sum(lens)
            key_lens = [rnd.randint(1, lk) for _ in range(B)]
        if B * H * Lq * sum(lens) * D > 1.5e9:   # keep the fp32 CPU reference to a fraction of a second
            continue
        cases.append((len(cases), kind, B, Lq, H, D, tuple(lens), frame, key_lens))
    return cases


CASES = _cases()


def _ref(q, K, V, key_lens=None):
    """fp32 softmax(q K^T / sqrt(D)) V per (batch, head); key_lens limits row b's keys."""
    B, Lq, H, D = q.shape
    out = torch.empty(B, Lq, H, D)
    for b in range(B):
        n = K.shape[1] if key_lens is None else key_lens[b]
        qb = q[b].float().transpose(0, 1)                       # [H, Lq, D]
        kb = K[b, :n].float().transpose(0, 1)
        vb = V[b, :n].float().transpose(0, 1)
        p = torch.softmax(qb @ kb.transpose(1, 2) / math.sqrt(D), -1)
        out[b] = (p @ vb).transpose(0, 1)
    return out


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-{c[1]}-B{c[2]}-q{c[3]}-H{c[4]}-D{c[5]}-s{len(c[6])}" +
                                               (f"-f{c[7]}" if c[7] else "") + ("-klen" if c[8] else "")
                                               for c in CASES])
def test_attention_sweep(dev, case):
    idx, kind, B, Lq, H, D, lens, frame, key_lens = case
    g = gen(1000 + idx)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    ks = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    if kind == "fp8":
        # each segment in its own frame-aligned span, a free frame between spans
        nfr = [-(-n // frame) for n in lens]
        cap = (sum(nfr) + len(lens)) * frame
        kc = torch.zeros(B, cap, H, D, dtype=torch.uint8, device=dev)
        vc = torch.zeros_like(kc)
        ksc = torch.ones(B, H, cap // frame, dtype=torch.float32, device=dev)
        vsc = torch.ones_like(ksc)
        segs, kd, vd, f0 = [], [], [], 0
        for n, nf, kk, vv in zip(lens, nfr, ks, vs):
            pad = nf * frame - n
            kq, kqs = OF.quantize_kv(torch.cat([kk.float(), torch.zeros(B, pad, H, D)], 1), frame)
            vq, vqs = OF.quantize_kv(torch.cat([vv.float(), torch.zeros(B, pad, H, D)], 1), frame)
            p0 = f0 * frame
            kc[:, p0:p0 + nf * frame] = kq.to(dev)
            vc[:, p0:p0 + nf * frame] = vq.to(dev)
            ksc[:, :, f0:f0 + nf] = kqs.to(dev)
            vsc[:, :, f0:f0 + nf] = vqs.to(dev)
            segs.append(KVSegment(kc[:, p0:p0 + n], vc[:, p0:p0 + n], ksc[:, :, f0:f0 + nf], vsc[:, :, f0:f0 + nf]))
            kd.append(OF.dequantize_kv(kq, kqs, frame)[:, :n])
            vd.append(OF.dequantize_kv(vq, vqs, frame)[:, :n])
            f0 += nf + 1
        kernels.flash_attn(q.to(dev), segs, out, frame_tokens=frame)
        torch.cuda.synchronize()
        # the decode is exact, so against the dequantised cache only bf16 rounding is left
        assert_bf16_close(out, _ref(q, torch.cat(kd, 1), torch.cat(vd, 1)), f"{case}")
        return
    cap = -(-(sum(lens) + 40 * len(lens) + 64) // 8) * 8
    ka = torch.zeros(B, cap, H, D, dtype=torch.bfloat16, device=dev)
    va = torch.zeros_like(ka) if kind == "token" else \
        torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=dev).permute(0, 3, 1, 2)
    segs, pos = [], 0
    for kk, vv in zip(ks, vs):
        n = kk.shape[1]
        ka[:, pos:pos + n] = kk.to(dev)
        va[:, pos:pos + n] = vv.to(dev)
        segs.append(KVSegment(ka[:, pos:pos + n], va[:, pos:pos + n]))
        pos = -(-(pos + n + 29) // 8) * 8          # a gap, then the next 8-slot boundary
    kernels.flash_attn(q.to(dev), segs, out, key_lens=key_lens)
    torch.cuda.synchronize()
    assert_bf16_close(out, _ref(q, torch.cat(ks, 1), torch.cat(vs, 1), key_lens), f"{case}")
