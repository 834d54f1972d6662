"""ltx_flash_attn_fwd_noalloc (split partials in the library's fixed scratch
array) against ltx_flash_attn_fwd (caller's workspace): two calls in a row,
the second smaller, both with a split tail, results bit-identical."""
import ctypes

import pytest
import torch

from taomate_amd import _native, kernels
from taomate_amd.kernels import KVSegment

from .helpers import assert_bf16_close, gen, randn
from .test_gpu_kernels import _ref_attn

pytestmark = pytest.mark.gpu


def _arena_segments(dev, B, H, D, lens, g):
    """K token-major and V key-major spans of one arena (the product layout)."""
    ks = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    cap = -(-(sum(lens) + 16 * len(lens)) // 8) * 8
    ka = torch.zeros(B, cap, H, D, dtype=torch.bfloat16, device=dev)
    va = torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=dev).permute(0, 3, 1, 2)
    segs, pos = [], 0
    for kk, vv in zip(ks, vs):
        n = kk.shape[1]
        ka[:, pos:pos + n] = kk.to(dev)
        va[:, pos:pos + n] = vv.to(dev)
        segs.append(KVSegment(ka[:, pos:pos + n], va[:, pos:pos + n]))
        pos = -(-(pos + n + 5) // 8) * 8
    return segs, torch.cat(ks, 1), torch.cat(vs, 1)


@pytest.mark.parametrize("first,second", [
    # (B, Lq, H, D, segment lengths): 576 then 520 q-tiles of 128 on 512 resident slots
    ((2, 1152, 32, 128, [384, 768, 2304, 1152]), (1, 1664, 40, 128, [512, 1536])),
    # even q-tile counts per head (the pair kernel): 320 then 280 units of two q-tiles on 256
    ((2, 1280, 32, 128, [1024, 1024]), (1, 1792, 40, 128, [512, 1536])),
])
def test_noalloc_matches_workspace_entry_point(dev, first, second):
    g = gen(21)
    for i, (B, Lq, H, D, lens) in enumerate((first, second)):
        print(f"noalloc call {i}: B={B} Lq={Lq} H={H} D={D} keys={lens}", flush=True)
        ws = ctypes.c_int64(0)
        _native.call("ltx_flash_attn_workspace_size", B, Lq, H, D, ctypes.byref(ws))
        assert ws.value > 0, "the shape must plan a split tail"
        assert ws.value <= _native.NOALLOC_SCRATCH_BYTES
        segs, K, V = _arena_segments(dev, B, H, D, lens, g)
        q = randn((B, Lq, H, D), g, torch.bfloat16).to(dev)
        ref_out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
        out = torch.full((B, Lq, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
        ref_lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
        lse = torch.full((B, H, Lq), float("nan"), dtype=torch.float32, device=dev)
        kernels.flash_attn(q, segs, ref_out, lse=ref_lse)
        kernels.flash_attn(q, segs, out, lse=lse, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"call {i}: noalloc output differs from the workspace entry point"
        assert torch.equal(lse, ref_lse), f"call {i}: noalloc lse differs"
        if i == 0:
            assert_bf16_close(out, _ref_attn(q.cpu(), K, V), "noalloc vs fp32")


def _fp8_segments(dev, B, H, D, lens, frame, g):
    """fp8 K/V spans (frame-aligned, codes and per-frame scales) and the
    dequantised K/V they hold."""
    from oracle import fp8 as OF
    n = sum(lens)
    kc, ksc = OF.quantize_kv(randn((B, n, H, D), g, torch.float32), frame)
    vc, vsc = OF.quantize_kv(randn((B, n, H, D), g, torch.float32), frame)
    kcd, vcd, kscd, vscd = kc.to(dev), vc.to(dev), ksc.to(dev), vsc.to(dev)
    segs, pos = [], 0
    for m in lens:   # spans of one store (shared strides), whole frames each
        f0, nf = pos // frame, m // frame
        segs.append(KVSegment(kcd[:, pos:pos + m], vcd[:, pos:pos + m], kscd[:, :, f0:f0 + nf],
                              vscd[:, :, f0:f0 + nf]))
        pos += m
    return segs, OF.dequantize_kv(kc, ksc, frame), OF.dequantize_kv(vc, vsc, frame)


@pytest.mark.parametrize("first,second", [
    # fp8 K/V in 384-token frames, even q-tile counts per head (the pair
    # workgroups: group 0 stages K, group 1 V): 320 then 280 units on 256
    ((2, 1280, 32, 128, [384, 768, 1152]), (1, 1792, 40, 128, [384, 1152])),
    # odd q-tile counts (9, then 11 per head): pair workgroups over all but
    # the last q-tile of every head, then the last ones cut into key ranges
    ((2, 1152, 32, 128, [384, 768, 1152]), (1, 1408, 40, 128, [384, 1152])),
])
def test_noalloc_fp8_pair_matches_workspace_entry_point(dev, first, second):
    g = gen(22)
    frame = 384
    for i, (B, Lq, H, D, lens) in enumerate((first, second)):
        print(f"noalloc fp8 call {i}: B={B} Lq={Lq} H={H} D={D} keys={lens}", flush=True)
        segs, K, V = _fp8_segments(dev, B, H, D, lens, frame, g)
        q = randn((B, Lq, H, D), g, torch.bfloat16).to(dev)
        ref_out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
        out = torch.full((B, Lq, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
        kernels.flash_attn(q, segs, ref_out, frame_tokens=frame)
        kernels.flash_attn(q, segs, out, frame_tokens=frame, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"call {i}: noalloc output differs from the workspace entry point"
        if i == 0:
            assert_bf16_close(out, _ref_attn(q.cpu(), K, V), "noalloc fp8 vs the dequantised cache")
