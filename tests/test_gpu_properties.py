"""Size-independent properties of the attention kernels at the full chunk
workload (B = 2, 32 heads x 128, 1152 queries over anchor 384 | memory 768 |
window 2304 | current 1152 keys, the tail q-tiles split and merged), where the
fp32 oracle comparisons of the other tests run at reduced or single-call
sizes.  Each property follows from the arithmetic, not from a second
implementation:

* scaling V by 2 scales every product, every fp32 partial sum, every split
  partial and the merge by 2 exactly, so the bf16 output doubles bit for bit;
* attention is linear in V for fixed Q and K;
* a batch row computed alone (a grid with no split tail) equals the same row
  of the two-row call (split tail and merge) up to rounding;
* attention depends on the set of keys, not on their order: reversed
  segments give the same output up to rounding;
* every key twice halves each weight and leaves the output as it was;
* one vector added to every key shifts all of a query's logits by the same
  amount, which the softmax removes.
"""
import pytest
import torch

from taomate_amd import kernels
from taomate_amd.kernels import KVSegment
from taomate_amd.kv_cache import KVArena

from .helpers import cosine, diff_stats, gen, randn

pytestmark = pytest.mark.gpu

FRAME = 384                     # 16x24 latent grid
LQ = 3 * FRAME                  # the chunk's queries and its own keys
SEG_FRAMES = (1, 2, 6)          # anchor, memory, window (frames)


def _arena(dev, kv, H, D, k_parts, v_parts):
    """An arena holding the given [B, n, H, D] K/V parts as consecutive spans
    (fp8: quantised per frame by the append kernel); returns the segments."""
    B = k_parts[0].shape[0]
    total = sum(p.shape[1] for p in k_parts)
    a = KVArena(B, total + FRAME, H, D, dev, kv, frame_tokens=FRAME, name="props")
    segs, pos = [], 0
    for k, v in zip(k_parts, v_parts):
        n = k.shape[1]
        if a.fp8:
            kernels.kv_append(k.to(dev), a.slots("k", pos, n), a.scale_slots("k", pos, n), FRAME)
            kernels.kv_append(v.to(dev), a.slots("v", pos, n), a.scale_slots("v", pos, n), FRAME)
        else:
            a.slots("k", pos, n).copy_(k.to(dev))
            a.slots("v", pos, n).copy_(v.to(dev))
        segs.append(KVSegment(a.slots("k", pos, n), a.slots("v", pos, n),
                              a.scale_slots("k", pos, n), a.scale_slots("v", pos, n)))
        pos += n
    return a, segs


def _parts(g, B, H, D):
    lens = [f * FRAME for f in SEG_FRAMES] + [LQ]
    ks = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.float32) for n in lens]
    return ks, vs


def _attend(dev, kv, q, ks, vs, H, D):
    a, segs = _arena(dev, kv, H, D, ks, vs)
    out = torch.empty(q.shape[0], q.shape[1], H, D, dtype=torch.bfloat16, device=dev)
    kernels.flash_attn(q, segs, out, frame_tokens=FRAME if kv == "fp8" else 0)
    torch.cuda.synchronize()
    del a
    return out


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_output_doubles_with_v(dev, kv):
    """out(2V) = 2 out(V): bit for bit with bf16 K/V (the whole path is exact
    under a power-of-two scale, the split-tail merge included); with fp8 K/V
    the doubled frame scale enters the exponent through its logarithm, so
    the two calls round apart in the last bits."""
    B, H, D = 2, 32, 128
    g = gen(41)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    ks, vs = _parts(g, B, H, D)
    v1 = [v.to(torch.bfloat16) for v in vs]
    v2 = [(2 * v).to(torch.bfloat16) for v in vs]          # exactly 2 x v1
    assert all(torch.equal(b, 2 * a) for a, b in zip(v1, v2))
    o1 = _attend(dev, kv, q, ks, v1, H, D)
    o2 = _attend(dev, kv, q, ks, v2, H, D)
    assert torch.isfinite(o1.float()).all()
    print(f"doubling V ({kv}): max-abs {diff_stats(o2, 2 * o1)[0]:.3e}", flush=True)
    if kv == "bf16":
        assert torch.equal(o2, 2 * o1), diff_stats(o2, 2 * o1)
    else:
        mx, mn = diff_stats(o2, 2 * o1)
        ref = o1.float().abs().max().item()
        assert cosine(o2, 2 * o1) >= 0.99999 and mx <= 2 ** -6 * 2 * ref, (cosine(o2, 2 * o1), mx, ref)


def test_output_linear_in_v(dev):
    """out(V1 + V2) = out(V1) + out(V2) for fixed Q and K, up to the bf16
    roundings of V1 + V2 and of the three outputs."""
    B, H, D = 2, 32, 128
    g = gen(42)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    ks, va = _parts(g, B, H, D)
    _, vb = _parts(g, B, H, D)
    v1 = [v.to(torch.bfloat16) for v in va]
    v2 = [v.to(torch.bfloat16) for v in vb]
    v12 = [(a.float() + b.float()).to(torch.bfloat16) for a, b in zip(v1, v2)]
    o1 = _attend(dev, "bf16", q, ks, v1, H, D).float()
    o2 = _attend(dev, "bf16", q, ks, v2, H, D).float()
    o12 = _attend(dev, "bf16", q, ks, v12, H, D).float()
    mx, mn = diff_stats(o12, o1 + o2)
    scale = (o1 + o2).abs().max().item()
    print(f"linearity: max-abs {mx:.3e} mean-abs {mn:.3e} scale {scale:.3e} cos {cosine(o12, o1 + o2):.7f}", flush=True)
    # measured 1.2e-3 and 7.8e-5 at a largest output of 0.34: bounds with a 3x margin
    assert mx <= 1e-2 * scale and mn <= 1e-3 * scale, (mx, mn, scale)
    assert cosine(o12, o1 + o2) >= 0.99999


def test_batch_row_alone_matches_two_row_call(dev):
    """Batch row 1 attended alone (288 q-tiles: one partial round, no split
    tail) against row 1 of the two-row call (576 q-tiles: the tail q-tiles cut
    into key ranges and merged)."""
    B, H, D = 2, 32, 128
    g = gen(43)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    ks, vs = _parts(g, B, H, D)
    vs = [v.to(torch.bfloat16) for v in vs]
    both = _attend(dev, "bf16", q, ks, vs, H, D)
    alone = _attend(dev, "bf16", q[1:].contiguous(), [k[1:] for k in ks], [v[1:] for v in vs], H, D)
    mx, mn = diff_stats(alone[0], both[1])
    print(f"batch row alone vs in the pair: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    # measured 9.8e-4 / 1.1e-5: bounds with a 4x margin
    assert mx <= 4e-3 and mn <= 5e-5, (mx, mn)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_segment_order_does_not_matter(dev, kv):
    """Attention is a function of the key set: the four segments (whole
    frames each) in reverse order give the same output up to the order of the
    fp32 sums and of the running maximum's updates."""
    B, H, D = 2, 32, 128
    g = gen(44)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    ks, vs = _parts(g, B, H, D)
    vs = [v.to(torch.bfloat16) for v in vs]
    fwd = _attend(dev, kv, q, ks, vs, H, D)
    rev = _attend(dev, kv, q, ks[::-1], vs[::-1], H, D)
    mx, mn = diff_stats(rev, fwd)
    scale = fwd.float().abs().max().item()
    print(f"segment order ({kv}): max-abs {mx:.3e} mean-abs {mn:.3e} scale {scale:.3e}", flush=True)
    assert torch.isfinite(fwd.float()).all()
    # measured (both K/V types) max-abs 9.8e-4 and mean-abs 4.3e-5 at a largest output of 0.17
    assert cosine(rev, fwd) >= 0.99999 and mx <= 2 ** -6 * scale and mn <= 2 ** -11 * scale, (mx, mn, scale)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_duplicated_keys_leave_output_unchanged(dev, kv):
    """Every key twice (eight segments: the four, then the four again): each
    softmax weight halves and the output is the same, up to rounding; the
    row sums reach twice the single set's."""
    B, H, D = 2, 32, 128
    g = gen(45)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    ks, vs = _parts(g, B, H, D)
    vs = [v.to(torch.bfloat16) for v in vs]
    once = _attend(dev, kv, q, ks, vs, H, D)
    twice = _attend(dev, kv, q, ks + ks, vs + vs, H, D)
    mx, mn = diff_stats(twice, once)
    scale = once.float().abs().max().item()
    print(f"duplicated keys ({kv}): max-abs {mx:.3e} mean-abs {mn:.3e} scale {scale:.3e}", flush=True)
    # measured max-abs 4.9e-4 (bf16) / 9.8e-4 (fp8), mean-abs 6.1e-6, at a largest output of 0.25
    assert cosine(twice, once) >= 0.99999 and mx <= 2 ** -6 * scale and mn <= 2 ** -11 * scale, (mx, mn, scale)


def test_uniform_logit_offset_leaves_output_unchanged(dev):
    """K + u for one vector u shared by every key adds q.u to all of a query's
    logits, which the softmax removes.  K and u sit on a 1/16 grid small
    enough that K + u is exact in bf16, and u is large (6 to 8 per channel,
    random signs), so a query's logits move by about 10 log2 units on
    average and by over 40 at the extremes."""
    B, H, D = 2, 32, 128
    g = gen(46)
    q = randn((B, LQ, H, D), g, torch.bfloat16).to(dev)
    lens = [f * FRAME for f in SEG_FRAMES] + [LQ]
    ks = [(torch.randint(-64, 65, (B, n, H, D), generator=g).float() / 16).to(torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    u = (torch.randint(96, 129, (1, 1, H, D), generator=g).float() / 16) * torch.where(
        torch.rand(1, 1, H, D, generator=g) < 0.5, -1.0, 1.0)
    ku = [(k.float() + u).to(torch.bfloat16) for k in ks]
    assert all(torch.equal(a.float(), k.float() + u) for a, k in zip(ku, ks)), "K + u must be exact"
    base = _attend(dev, "bf16", q, ks, vs, H, D)
    moved = _attend(dev, "bf16", q, ku, vs, H, D)
    off = (q.float().cpu() * u).sum(-1) / D ** 0.5 / torch.log(torch.tensor(2.0))
    mx, mn = diff_stats(moved, base)
    scale = base.float().abs().max().item()
    print(f"logit offset up to {off.abs().max().item():.1f} (log2): max-abs {mx:.3e} mean-abs {mn:.3e} "
          f"scale {scale:.3e}", flush=True)
    assert off.abs().max().item() > 20.0
    # measured max-abs 3.9e-3 and mean-abs 3.3e-7 at a largest output of 2.9 (offsets up to 43)
    assert cosine(moved, base) >= 0.99999 and mx <= 2 ** -6 * scale and mn <= 2 ** -11 * scale, (mx, mn, scale)
