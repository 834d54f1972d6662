"""HIP graph capture of the chunk step (q/k norm + RoPE, V append, split-tail
attention with its combine kernel) at the 512x768 chunk shape: every replay,
with eager work and synchronisations in between, must reproduce the eager
outputs bit for bit (the kernels are deterministic and allocate nothing)."""
import math

import pytest
import torch

from taomate_amd import kernels
from taomate_amd.kernels import KVSegment
from taomate_amd.kv_cache import KVArena
from taomate_amd.rope import causal_precompute_freqs_cis

pytestmark = pytest.mark.gpu


def _workload(dev):
    B, H, D, hw = 2, 32, 128, 384
    HD, LQ = H * D, 3 * hw
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    arena = KVArena(B, 9 * hw + 2 * LQ, H, D, dev, "bf16", frame_tokens=hw, name="graph")
    spans, pos = [], 0
    for nf in (1, 2, 6):
        n = nf * hw
        arena.slots("k", pos, n).copy_(torch.randn(B, n, H, D, generator=g, device=dev).to(torch.bfloat16))
        arena.slots("v", pos, n).copy_(torch.randn(B, n, H, D, generator=g, device=dev).to(torch.bfloat16))
        spans.append((pos, n))
        pos += n
    sd = 0.02 * math.sqrt(HD)
    lin = [(torch.randn(B, LQ, HD, generator=g, device=dev) * sd).to(torch.bfloat16) for _ in range(3)]
    gam = torch.ones(HD, device=dev, dtype=torch.bfloat16)
    pe = causal_precompute_freqs_cis(torch.tensor([[3, 16, 24]] * B), HD, start_frame=12, device=dev,
                                     dtype=torch.bfloat16, num_attention_heads=H)
    q = torch.empty_like(lin[0])
    out = torch.empty(B, LQ, H, D, device=dev, dtype=torch.bfloat16)
    kd, vd = arena.slots("k", pos, LQ), arena.slots("v", pos, LQ)
    segs = [KVSegment(arena.slots("k", s, n), arena.slots("v", s, n)) for s, n in spans + [(pos, LQ)]]

    def step():
        kernels.qk_rmsnorm_rope(lin[0], q, gam, 1e-6, pe, H, D, lin[1], kd, gam, 1e-6, pe)
        kernels.kv_append(lin[2].view(B, LQ, H, D), vd)
        kernels.flash_attn(q.view(B, LQ, H, D), segs, out)

    return step, (q, kd, vd, out), lin


def test_step_graph_replays_match_eager(dev):
    step, outs, lin = _workload(dev)
    step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    for rep in range(3):
        for t in outs:       # poison the outputs eagerly between replays
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("q", "k slots", "v slots", "out"), outs, eager):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager step"
        lin[0].add_(0)       # eager work on the inputs between replays
