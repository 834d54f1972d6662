"""GPU parity of each kernel against the CPU oracle (run on an MI355X)."""
import ctypes
import math

import pytest
import torch

from oracle import attention as OA
from oracle import fp8 as OF
from oracle import rope as OR
from taomate_amd import _native, kernels
from taomate_amd.kernels import KVSegment
from taomate_amd.rope import causal_precompute_freqs_cis, generate_freq_grid

from .helpers import (BF16_MAX_ABS, BF16_MEAN_ABS, FP8_COSINE, assert_bf16_close, bf16_ulp_diff,
                      cosine, diff_stats, gen, randn)

pytestmark = pytest.mark.gpu

ROPE_CASES = [
    # (grid, dim, heads, start_frame, is_audio, max_pos)
    ((2, 8, 12), 512, 8, 10, False, [20, 2048, 2048]),      # 8x12 latent grid, 8 x 64 heads
    ((3, 16, 24), 4096, 32, 12, False, [20, 2048, 2048]),   # 16x24 grid, 32 x 128 heads
    ((75,), 2048, 32, 600, True, [20]),                     # audio 1-D, 32 x 64
    ((3,), 2048, 32, 12, False, [20]),                      # video-time 1-D (cross-modal)
    ((4, 16, 24), 4096, 32, 0, False, [20, 2048, 2048]),    # frame 0 (causal fix clamp)
    ((1, 8, 130), 4096, 32, 3, False, [20, 2048, 2048]),    # rows too wide for the per-block LDS tables
    ((2, 18, 20), 4096, 32, 7, False, [20, 2048, 2048]),    # row count not a multiple of the row block
]


@pytest.mark.parametrize("case", ROPE_CASES, ids=lambda c: f"grid{c[0]}_dim{c[1]}")
def test_rope_table_matches_oracle(dev, case):
    grid, dim, heads, sf, audio, mp = case
    gs = torch.tensor([list(grid)])
    cos, sin = causal_precompute_freqs_cis(gs, dim, max_pos=mp, start_frame=sf, device=dev,
                                           dtype=torch.float32, is_audio=audio,
                                           num_attention_heads=heads)
    rc, rs = OR.causal_precompute_freqs_cis(grid, dim, max_pos=mp, start_frame=sf, is_audio=audio,
                                            num_attention_heads=heads)
    assert cos.shape == rc.shape
    # float32 tables: only the final cos/sin evaluation may differ (<= a few ulp)
    assert (cos.cpu() - rc).abs().max().item() <= 2e-6
    assert (sin.cpu() - rs).abs().max().item() <= 2e-6
    # bf16 tables: rounding of those values; at most 1 bf16 ulp apart, nearly all equal
    cb, sb = causal_precompute_freqs_cis(gs, dim, max_pos=mp, start_frame=sf, device=dev,
                                         dtype=torch.bfloat16, is_audio=audio,
                                         num_attention_heads=heads)
    u = bf16_ulp_diff(cb, rc.to(torch.bfloat16))
    assert u.max() <= 1 and (u == 0).mean() >= 0.999
    u = bf16_ulp_diff(sb, rs.to(torch.bfloat16))
    assert u.max() <= 1 and (u == 0).mean() >= 0.999


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("grid,dim,heads", [((3, 16, 24), 4096, 32), ((2, 8, 12), 512, 8), ((2, 18, 20), 4096, 32)],
                         ids=["16x24_32x128", "8x12_8x64", "18x20"])
def test_rope_table_retime_bit_identical(dev, grid, dim, heads, dtype):
    """A video table derived for a new start frame from one built for another
    (ltx_rope_table_retime: h, w and pad entries copied, t entries recomputed)
    equals the table built directly for that frame bit for bit, for start
    frames around the causal clamp (0, 1) and far along a stream; and
    causal_precompute_freqs_cis, which derives every table after the first of
    a layout, returns those tables."""
    from taomate_amd import kernels as K
    from taomate_amd import rope as R
    mp = [20.0, 2048.0, 2048.0]
    freq = generate_freq_grid(10000.0, 3, dim, dev)
    src = K.rope_table(freq, grid, 5, False, mp, dim, heads, 1, dtype)
    for sf in (0, 1, 5, 13, 186, 4000):
        want = K.rope_table(freq, grid, sf, False, mp, dim, heads, 1, dtype)
        got = K.rope_table_retime(src, freq, grid, sf, mp[0], dim, heads)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1]), sf
    R._TABLE_CACHE.clear()
    R._VIDEO_TEMPLATES.clear()
    gs = torch.tensor([list(grid)] * 2)
    for sf in (3, 9, 4000):
        cos, sin = causal_precompute_freqs_cis(gs, dim, start_frame=sf, device=dev, dtype=dtype,
                                               num_attention_heads=heads)
        want = K.rope_table(freq, grid, sf, False, mp, dim, heads, 1, dtype)
        assert cos.shape[0] == 2 and torch.equal(cos[1], want[0][0]) and torch.equal(sin[0], want[1][0]), sf
    assert len(R._VIDEO_TEMPLATES) == 1


def test_freq_grid_is_reference_expression(dev):
    f = generate_freq_grid(10000.0, 3, 4096, dev).cpu()
    assert torch.equal(f, OR.generate_freq_grid(10000.0, 3, 4096))


NORM_CASES = [
    # (B, L, H, D, dtype)
    (1, 192, 8, 64, torch.bfloat16),
    (2, 1152, 32, 128, torch.bfloat16),
    (1, 75, 32, 64, torch.bfloat16),
    (1, 192, 8, 64, torch.float32),
    (2, 37, 16, 64, torch.float32),
]


@pytest.mark.parametrize("case", NORM_CASES, ids=lambda c: f"B{c[0]}L{c[1]}H{c[2]}D{c[3]}{str(c[4])[6:]}")
def test_qk_rmsnorm_rope_matches_oracle(dev, case):
    B, L, H, D, dt = case
    g = gen(11)
    HD = H * D
    q = randn((B, L, HD), g, dt, 3.0)
    k = randn((B, L, HD), g, dt, 0.5)
    gq = (1 + 0.1 * randn((HD,), g)).to(dt)
    gk = (1 + 0.1 * randn((HD,), g)).to(dt)
    grid = (1, L, 1)
    cos, sin = OR.causal_precompute_freqs_cis(grid, HD, start_frame=3, num_attention_heads=H,
                                              batch=B, dtype=dt)
    # oracle in the same dtype (the reference's composite op order) and in fp32
    rq = OR.apply_split_rotary_emb(OA.rms_norm_full_row(q, gq, 1e-6), cos, sin)
    rk = OR.apply_split_rotary_emb(OA.rms_norm_full_row(k, gk, 1e-6), cos, sin)
    f = lambda t: t.float()
    rq32 = OR.apply_split_rotary_emb(OA.rms_norm_full_row(f(q), f(gq), 1e-6), f(cos), f(sin))
    qd, kd = q.to(dev), k.to(dev)
    qo, ko = torch.empty_like(qd), torch.empty_like(kd)
    kernels.qk_rmsnorm_rope(qd, qo, gq.to(dev), 1e-6, (cos.to(dev), sin.to(dev)), H, D,
                            kd, ko, gk.to(dev), 1e-6, (cos.to(dev), sin.to(dev)))
    torch.cuda.synchronize()
    if dt == torch.bfloat16:
        # same rounding sequence as torch's bf16 ops: bit-identical except where
        # the float32 sum of squares (a different reduction order) flips a rounding
        for out, ref in ((qo, rq), (ko, rk)):
            out = out.cpu()
            exact = (out == ref).float().mean().item()
            d = (out.float() - ref.float()).abs().max().item()
            assert exact >= 0.995 and d <= 2 ** -6 * ref.float().abs().max().item(), (exact, d)
        assert_bf16_close(qo, rq32, "q vs fp32", max_abs=0.05, mean_abs=2e-3)
    else:
        assert diff_stats(qo, rq)[0] <= 1e-5
        assert diff_stats(ko, rk)[0] <= 1e-5


@pytest.mark.parametrize("B,L,H,D", [(2, 1152, 32, 128), (1, 192, 8, 64), (2, 37, 16, 64)])
def test_qk_rmsnorm_rope_shared_table_path(dev, B, L, H, D):
    """q and k through one RoPE table with a stride-0 batch (the shared-table
    kernel: one workgroup per positions, all q/k rows) equal, bit for bit, the
    per-side kernel run on separate per-batch copies of the same table."""
    g = gen(12)
    HD = H * D
    q = randn((B, L, HD), g, torch.bfloat16, 3.0).to(dev)
    k = randn((B, L, HD), g, torch.bfloat16, 0.5).to(dev)
    gq = (1 + 0.1 * randn((HD,), g)).to(torch.bfloat16).to(dev)
    gk = (1 + 0.1 * randn((HD,), g)).to(torch.bfloat16).to(dev)
    cos, sin = OR.causal_precompute_freqs_cis((1, L, 1), HD, start_frame=5, num_attention_heads=H,
                                              batch=1, dtype=torch.bfloat16)
    cs, ss = cos.to(dev).expand(B, -1, -1, -1), sin.to(dev).expand(B, -1, -1, -1)
    qa, ka = torch.empty_like(q), torch.empty_like(k)
    kernels.qk_rmsnorm_rope(q, qa, gq, 1e-6, (cs, ss), H, D, k, ka, gk, 1e-6, (cs, ss))
    qb, kb = torch.empty_like(q), torch.empty_like(k)
    kernels.qk_rmsnorm_rope(q, qb, gq, 1e-6, (cs.contiguous(), ss.contiguous()), H, D,
                            k, kb, gk, 1e-6, (cs.contiguous(), ss.contiguous()))
    torch.cuda.synchronize()
    assert torch.equal(qa, qb) and torch.equal(ka, kb)


@pytest.mark.parametrize("B,L,H,D,Lv", [(2, 1152, 32, 128, 1152), (1, 192, 8, 64, 192), (2, 37, 16, 64, 37),
                                         (1, 64, 8, 128, 0), (2, 5, 32, 128, 200)])
def test_qk_rmsnorm_rope_v_fused_equals_separate(dev, B, L, H, D, Lv):
    """The fused launch (q/k norm + RoPE rows and the key-major V tiles in one
    grid) writes exactly what the two separate kernels write, including the
    V store's untouched slots; V lengths that are not a multiple of the 64-token
    tile, no V at all, and more V tokens than q/k rows."""
    g = gen(21)
    HD = H * D
    q = randn((B, L, HD), g, torch.bfloat16, 3.0).to(dev)
    k = randn((B, L, HD), g, torch.bfloat16, 0.5).to(dev)
    v = randn((B, Lv, H, D), g, torch.bfloat16).to(dev)
    gq = (1 + 0.1 * randn((HD,), g)).to(torch.bfloat16).to(dev)
    gk = (1 + 0.1 * randn((HD,), g)).to(torch.bfloat16).to(dev)
    cos, sin = OR.causal_precompute_freqs_cis((1, L, 1), HD, start_frame=3, num_attention_heads=H,
                                              batch=1, dtype=torch.bfloat16)
    tab = (cos.to(dev), sin.to(dev))
    slots = -(-(Lv + 72) // 8) * 8
    outs = []
    for fused in (False, True):
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        store = torch.zeros(B, H, D, slots, dtype=torch.bfloat16, device=dev)
        vview = store.permute(0, 3, 1, 2)[:, 64:64 + Lv]
        if fused:
            kernels.qk_rmsnorm_rope(q, qo, gq, 1e-6, tab, H, D, k, ko, gk, 1e-6, tab, v_in=v, v_out=vview)
        else:
            kernels.qk_rmsnorm_rope(q, qo, gq, 1e-6, tab, H, D, k, ko, gk, 1e-6, tab)
            kernels.kv_append(v, vview)
        outs.append((qo, ko, store))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert torch.equal(outs[1][2].permute(0, 3, 1, 2)[:, 64:64 + Lv], v)


def test_norm_only_and_rope_only(dev):
    g = gen(5)
    B, L, H, D = 1, 64, 4, 64
    x = randn((B, L, H * D), g, torch.bfloat16)
    cos, sin = OR.causal_precompute_freqs_cis((1, L, 1), H * D, num_attention_heads=H, dtype=torch.bfloat16)
    xd = x.to(dev)
    y = torch.empty_like(xd)
    kernels.qk_rmsnorm_rope(xd, y, None, 1e-6, None, H, D)
    ref = OA.rms_norm_full_row(x, None, 1e-6)
    assert (y.cpu() == ref).float().mean().item() >= 0.995
    kernels.qk_rmsnorm_rope(xd, y, None, None, (cos.to(dev), sin.to(dev)), H, D)
    ref = OR.apply_split_rotary_emb(x, cos, sin)
    assert torch.equal(y.cpu(), ref)  # RoPE alone: the same three roundings, bit-exact


def test_kv_append_copy_bit_exact(dev):
    g = gen(3)
    B, L, H, D = 2, 100, 32, 128
    src = randn((B, L, H, D), g, torch.bfloat16).to(dev)
    arena = torch.zeros(B, 300, H, D, dtype=torch.bfloat16, device=dev)
    kernels.kv_append(src, arena[:, 57:57 + L])
    torch.cuda.synchronize()
    assert torch.equal(arena[:, 57:57 + L], src)
    assert torch.count_nonzero(arena[:, :57]) == 0 and torch.count_nonzero(arena[:, 157:]) == 0


@pytest.mark.parametrize("L,D,src_dt", [(100, 128, torch.bfloat16), (37, 64, torch.bfloat16),
                                        (1152, 128, torch.float32)])
def test_kv_append_key_major_bit_exact(dev, L, D, src_dt):
    """Transposing append into a key-major [B, H, D, slots] store (the arena's V layout)."""
    g = gen(12)
    B, H = 2, 8
    src = randn((B, L, H, D), g, src_dt).to(dev)
    store = torch.zeros(B, H, D, -(-(L + 120) // 8) * 8, dtype=torch.bfloat16, device=dev)
    view = store.permute(0, 3, 1, 2)                 # [B, slots, H, D], token stride 1
    kernels.kv_append(src, view[:, 56:56 + L])
    torch.cuda.synchronize()
    assert torch.equal(view[:, 56:56 + L], src.to(torch.bfloat16))
    assert torch.count_nonzero(store[..., :56]) == 0 and torch.count_nonzero(store[..., 56 + L:]) == 0


@pytest.mark.parametrize("shape,frame", [((2, 1152, 32, 128), 384), ((1, 96, 8, 64), 96),
                                          ((1, 50, 32, 64), 25)])
def test_kv_append_fp8_bit_exact(dev, shape, frame):
    g = gen(4)
    B, L, H, D = shape
    src = randn(shape, g, torch.bfloat16, 2.0)
    src[0, :frame, 0] = 0  # an all-zero (b, h, frame): scale 1
    codes_ref, sc_ref = OF.quantize_kv(src.float(), frame)
    dst = torch.zeros(B, L, H, D, dtype=torch.uint8, device=dev)
    sc = torch.zeros(B, H, L // frame, dtype=torch.float32, device=dev)
    kernels.kv_append(src.to(dev), dst, sc, frame)
    torch.cuda.synchronize()
    assert torch.equal(sc.cpu(), sc_ref)
    assert torch.equal(dst.cpu(), codes_ref)


@pytest.mark.parametrize("shape,frame", [((2, 1152, 32, 128), 384), ((1, 128, 8, 64), 64),
                                          ((1, 1024, 4, 128), 512), ((2, 150, 32, 64), 25),
                                          ((1, 96, 3, 128), 96)])
def test_kv_append_fp8_pair_bit_exact(dev, shape, frame):
    """K and V of a chunk quantised in one launch into arena slot views (offset
    spans of a larger store, V read through a strided projection view): codes
    and scales equal the oracle quantiser and the single-tensor append."""
    g = gen(14)
    B, L, H, D = shape
    k = randn(shape, g, torch.bfloat16, 2.0)
    v_rows = randn((B, L, H * D + 64), g, torch.bfloat16, 0.5)           # row stride H*D + 64
    v = v_rows[..., 32:32 + H * D].unflatten(-1, (H, D))
    k[0, :frame, 1] = 0
    kd_store = torch.zeros(B, L + 2 * frame, H, D, dtype=torch.uint8, device=dev)
    vd_store = torch.zeros_like(kd_store)
    nf = L // frame
    ks_store = torch.zeros(B, H, nf + 2, dtype=torch.float32, device=dev)
    vs_store = torch.zeros_like(ks_store)
    kd, vd = kd_store[:, frame:frame + L], vd_store[:, frame:frame + L]
    ks, vs = ks_store[:, :, 1:1 + nf], vs_store[:, :, 1:1 + nf]
    kernels.kv_append_fp8_pair(k.to(dev), kd, ks, v.to(dev), vd, vs, frame)
    torch.cuda.synchronize()
    for got_c, got_s, x in ((kd, ks, k), (vd, vs, v)):
        codes_ref, sc_ref = OF.quantize_kv(x.float(), frame)
        assert torch.equal(got_s.cpu(), sc_ref)
        assert torch.equal(got_c.cpu(), codes_ref)
    # slots and scales outside the spans are untouched
    assert torch.count_nonzero(kd_store[:, :frame]) == 0 and torch.count_nonzero(vd_store[:, frame + L:]) == 0
    assert torch.count_nonzero(ks_store[:, :, 0]) == 0 and torch.count_nonzero(vs_store[:, :, 1 + nf:]) == 0
    one_c = torch.zeros(B, L, H, D, dtype=torch.uint8, device=dev)
    one_s = torch.zeros(B, H, nf, dtype=torch.float32, device=dev)
    kernels.kv_append(v.to(dev), one_c, one_s, frame)
    torch.cuda.synchronize()
    assert torch.equal(one_c, vd) and torch.equal(one_s, vs)


def _frames_to_src(frames, D=64):
    """Pack 1-D float32 frames into a [1, n*F, 1, D] source, F tokens per frame."""
    F = max(math.ceil(len(f) / D) for f in frames)
    out = torch.zeros(len(frames), F * D, dtype=torch.float32)
    for i, f in enumerate(frames):
        out[i, :len(f)] = f
    return out.view(1, len(frames) * F, 1, D), F


def test_kv_append_fp8_rounding_ties(dev):
    """Quotients exactly on, and one float32 ulp either side of, every e4m3
    value and every midpoint between neighbours (ties go to even), subnormals
    included; then the same grid scaled by awkward per-frame scales so x/scale
    lands within a few ulp of midpoints."""
    grid = sorted({OF.e4m3_value(c) for c in range(0x7F)})
    g64 = torch.tensor(grid, dtype=torch.float64)
    base = torch.cat([g64, (g64[1:] + g64[:-1]) / 2]).float()
    inf = torch.tensor(float("inf"))
    vals = torch.cat([base, torch.nextafter(base, inf), torch.nextafter(base, -inf)])
    vals = vals.clamp(max=448.0)
    vals[1::2] *= -1
    frames = [torch.cat([vals, torch.tensor([448.0])])]           # scale exactly 1
    gen_ = torch.Generator().manual_seed(11)
    for m in (3.7, 0.0131, 1234.5, 1e-3, 7.0, 0.3):
        sc = torch.tensor(m, dtype=torch.float32) / 448.0
        t = base[base <= 440.0]
        x = (t * sc).float()
        # perturb by -3..3 ulp so quotients straddle the midpoints
        k = torch.randint(-3, 4, x.shape, generator=gen_)
        for _ in range(3):
            x = torch.where(k > 0, torch.nextafter(x, inf), torch.where(k < 0, torch.nextafter(x, -inf), x))
            k = k - k.sign()
        x[1::2] *= -1
        frames.append(torch.cat([x, torch.tensor([m], dtype=torch.float32)]))
    src, F = _frames_to_src(frames)
    codes_ref, sc_ref = OF.quantize_kv(src, F)
    dst = torch.zeros(src.shape, dtype=torch.uint8, device=dev)
    sc = torch.zeros(1, 1, len(frames), dtype=torch.float32, device=dev)
    kernels.kv_append(src.to(dev), dst, sc, F)
    torch.cuda.synchronize()
    assert torch.equal(sc.cpu(), sc_ref)
    assert torch.equal(dst.cpu(), codes_ref)


def test_kv_append_fp8_many_scales(dev):
    """16.7M bf16 values under per-head scales from 1e-3 to 1e3: every lane
    of the reciprocal fast path and of the exact-division fallback agrees
    with the float32 division of the reference quantiser."""
    g = gen(12)
    B, L, H, D, frame = 1, 4096, 32, 128, 512
    mag = 10.0 ** (torch.rand(1, 1, H, 1, generator=g) * 6 - 3)
    src = (torch.randn(B, L, H, D, generator=g) * mag).to(torch.bfloat16)
    codes_ref, sc_ref = OF.quantize_kv(src.float(), frame)
    dst = torch.empty(B, L, H, D, dtype=torch.uint8, device=dev)
    sc = torch.empty(B, H, L // frame, dtype=torch.float32, device=dev)
    kernels.kv_append(src.to(dev), dst, sc, frame)
    torch.cuda.synchronize()
    assert torch.equal(sc.cpu(), sc_ref)
    assert torch.equal(dst.cpu(), codes_ref)


def test_kv_gather_bit_exact(dev):
    g = gen(6)
    B, L, H, D = 2, 500, 8, 64
    src = randn((B, L, H, D), g, torch.bfloat16).to(dev)
    spans = [(0, 96), (300, 0), (200, 150), (480, 20)]
    dst = torch.empty(B, 266, H, D, dtype=torch.bfloat16, device=dev)
    kernels.kv_gather(src, dst, spans)
    ref = torch.cat([src[:, s:s + n] for s, n in spans], dim=1)
    assert torch.equal(dst, ref)
    u8 = torch.randint(0, 256, (B, L, H, D), dtype=torch.uint8, generator=g).to(dev)
    d8 = torch.empty(B, 266, H, D, dtype=torch.uint8, device=dev)
    kernels.kv_gather(u8, d8, spans)
    assert torch.equal(d8, torch.cat([u8[:, s:s + n] for s, n in spans], dim=1))


def _ref_attn(q, k, v, mask=None):
    return OA.standard_attention_forward(q.float().cpu(), k.float().cpu(), v.float().cpu(),
                                         None if mask is None else mask.cpu().view(mask.shape[0], 1, 1, -1))


ATTN_CASES = [
    # (B, Lq, H, D, segment lengths)
    (1, 192, 8, 64, [96, 96, 384, 192]),          # 8x12 grid: anchor|memory|window|current
    (2, 1152, 32, 128, [384, 768, 2304, 1152]),   # 16x24 grid full shape
    (1, 75, 32, 64, [600, 75]),                   # audio self
    (1, 1152, 32, 64, [75]),                      # A2V
    (1, 75, 32, 64, [1152]),                      # V2A
    (2, 130, 4, 128, [1, 63, 65, 7]),             # ragged tails, tiny segments
    (1, 1, 2, 128, [5]),                          # single query / few keys
    # the 16-segment maximum (after the two empty ones are dropped), ragged
    (1, 64, 4, 128, [8, 0, 17, 64, 1, 130, 9, 33, 0, 64, 2, 71, 5, 40, 16, 3, 7, 11]),
    (1, 128, 8, 128, [40000, 128]),               # long key range: 627 key tiles
    # two q-tiles per head (key-major V: the two-q-tile workgroup kernel), the
    # second one ragged, at the segment maximum and over a long key range
    (1, 200, 4, 128, [8, 0, 17, 64, 1, 130, 9, 33, 0, 64, 2, 71, 5, 40, 16, 3, 7, 11]),
    (1, 250, 8, 128, [40000, 128]),
]


def test_flash_attn_segment_limits(dev):
    """More than 16 non-empty segments, or none with keys, is refused before
    any launch."""
    q = torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(q)
    ka = torch.zeros(1, 17 * 8, 2, 64, dtype=torch.bfloat16, device=dev)
    segs = [KVSegment(ka[:, 8 * i:8 * i + 8], ka[:, 8 * i:8 * i + 8]) for i in range(17)]
    with pytest.raises(ValueError, match="segments"):
        kernels.flash_attn(q, segs, out)
    with pytest.raises(ValueError, match="no keys"):
        kernels.flash_attn(q, [KVSegment(ka[:, :0], ka[:, :0])], out)
    kernels.flash_attn(q, segs[:16], out)   # the maximum itself runs
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))   # V = 0


@pytest.mark.parametrize("vlayout", ["token", "key"])
@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"B{c[0]}q{c[1]}H{c[2]}D{c[3]}k{sum(c[4])}")
def test_flash_attn_bf16_vs_fp32(dev, case, vlayout):
    """Segments scattered over one arena (gaps between spans).  token: V shares K's
    [B, slots, H, D] layout (register-staged kernel); key: V in a key-major
    [B, H, D, slots] store with 8-slot-aligned spans (direct-to-LDS kernel)."""
    B, Lq, H, D, lens = case
    g = gen(7)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    ks = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    cap = -(-(sum(lens) + 64 * len(lens) + 64) // 8) * 8
    ka = torch.zeros(B, cap, H, D, dtype=torch.bfloat16, device=dev)
    if vlayout == "token":
        va = torch.zeros_like(ka)
    else:
        va = torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=dev).permute(0, 3, 1, 2)
    segs, pos = [], 0
    for kk, vv in zip(ks, vs):
        n = kk.shape[1]
        ka[:, pos:pos + n] = kk.to(dev)
        va[:, pos:pos + n] = vv.to(dev)
        segs.append(KVSegment(ka[:, pos:pos + n], va[:, pos:pos + n]))
        pos += n + 37
        pos = -(-pos // 8) * 8   # spans start on 8-slot boundaries
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    kernels.flash_attn(q.to(dev), segs, out, lse=lse)
    torch.cuda.synchronize()
    K, V = torch.cat(ks, 1), torch.cat(vs, 1)
    ref = _ref_attn(q, K, V)
    assert_bf16_close(out, ref, f"attn {case} {vlayout}")
    s_ = torch.einsum("bqhd,bkhd->bhqk", q.float(), K.float()) / math.sqrt(D)
    assert (lse.cpu() - torch.logsumexp(s_, -1)).abs().max().item() < 1e-2


def test_flash_attn_fp8_odd_qtiles_lse_takes_one_launch(dev):
    """fp8 K/V at 1152 queries (9 q-tiles per head): without lse the call runs
    as two launches (pair workgroups, then the last q-tile of every head),
    with lse as one (the 4-wave kernel, whose lse rows are Lq apart).  The
    two agree to bf16 rounding (they cut different q-tiles into key ranges;
    the rest run the same arithmetic and match bit for bit), and lse matches
    the log-sum-exp of the dequantised logits."""
    B, Lq, H, D, frame, lens = 2, 1152, 32, 128, 384, [384, 768, 1152]
    g = gen(10)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    K = randn((B, sum(lens), H, D), g, torch.bfloat16)
    V = randn((B, sum(lens), H, D), g, torch.bfloat16)
    kc, ksc = OF.quantize_kv(K.float(), frame)
    vc, vsc = OF.quantize_kv(V.float(), frame)
    kd, vd, kscd, vscd = kc.to(dev), vc.to(dev), ksc.to(dev), vsc.to(dev)
    segs, pos = [], 0
    for n in lens:
        f0, nf = pos // frame, n // frame
        segs.append(KVSegment(kd[:, pos:pos + n], vd[:, pos:pos + n], kscd[:, :, f0:f0 + nf], vscd[:, :, f0:f0 + nf]))
        pos += n
    two = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    one = torch.empty_like(two)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    kernels.flash_attn(q.to(dev), segs, two, frame_tokens=frame)
    kernels.flash_attn(q.to(dev), segs, one, frame_tokens=frame, lse=lse)
    torch.cuda.synchronize()
    same = (two == one).float().mean().item()
    print(f"fp8 odd q-tiles: two launches vs one: {same:.4f} of the outputs bit-identical", flush=True)
    assert_bf16_close(two, one, "two launches vs one")
    assert same >= 0.8, same
    Kd = OF.dequantize_kv(kc, ksc, frame)
    s_ = torch.einsum("bqhd,bkhd->bhqk", q.float(), Kd.float()) / math.sqrt(D)
    assert (lse.cpu() - torch.logsumexp(s_, -1)).abs().max().item() < 1e-2


@pytest.mark.parametrize("vlayout", ["token", "key"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("scales", [(1, 6, 1, 12), (12, 1, 6, 1)], ids=["rising", "falling"])
def test_flash_attn_logit_range(dev, D, scales, vlayout):
    """Logit maxima that rise far above (or fall far below) the first tile's:
    K segments scaled so later tiles exceed the running maximum by tens of
    base-2 units, which forces the rescale of O, l and m mid-stream."""
    B, Lq, H = 1, 130, 2
    lens = [64, 100, 64, 77]
    g = gen(11)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    ks = [randn((B, n, H, D), g, torch.bfloat16, scale=s) for n, s in zip(lens, scales)]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    cap = -(-(sum(lens) + 64 * len(lens) + 64) // 8) * 8
    ka = torch.zeros(B, cap, H, D, dtype=torch.bfloat16, device=dev)
    if vlayout == "token":
        va = torch.zeros_like(ka)
    else:
        va = torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=dev).permute(0, 3, 1, 2)
    segs, pos = [], 0
    for kk, vv in zip(ks, vs):
        n = kk.shape[1]
        ka[:, pos:pos + n] = kk.to(dev)
        va[:, pos:pos + n] = vv.to(dev)
        segs.append(KVSegment(ka[:, pos:pos + n], va[:, pos:pos + n]))
        pos = -(-(pos + n + 13) // 8) * 8
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, Lq, dtype=torch.float32, device=dev)
    kernels.flash_attn(q.to(dev), segs, out, lse=lse)
    torch.cuda.synchronize()
    K, V = torch.cat(ks, 1), torch.cat(vs, 1)
    assert_bf16_close(out, _ref_attn(q, K, V), f"logit range {scales} D{D} {vlayout}")
    s_ = torch.einsum("bqhd,bkhd->bhqk", q.float(), K.float()) / math.sqrt(D)
    ref_lse = torch.logsumexp(s_, -1)
    assert ((lse.cpu() - ref_lse).abs() / ref_lse.abs().clamp_min(1)).max().item() < 1e-3


def test_flash_attn_key_mask(dev):
    """Text cross-attention: 1152 queries, 1024 keys, 20% masked with the
    reference's (m-1)*finfo.max additive mask."""
    g = gen(8)
    B, Lq, Lk, H, D = 1, 1152, 1024, 32, 128
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    k = randn((B, Lk, H, D), g, torch.bfloat16)
    v = randn((B, Lk, H, D), g, torch.bfloat16)
    keep = torch.ones(B, Lk, dtype=torch.int64)
    keep[:, -int(0.2 * Lk):] = 0
    add = OA.prepare_attention_mask(keep, torch.bfloat16)          # [B,1,1,Lk] bf16
    ref = OA.standard_attention_forward(q.float(), k.float(), v.float(), add.float())
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    kernels.flash_attn(q.to(dev), [KVSegment(k.to(dev), v.to(dev))], out,
                       key_mask=add.view(B, Lk).float().to(dev))
    torch.cuda.synchronize()
    assert_bf16_close(out, ref, "masked attn")
    # masking equals dropping the masked keys
    kept = int(keep.sum())
    ref2 = OA.standard_attention_forward(q.float(), k[:, :kept].float(), v[:, :kept].float())
    assert_bf16_close(out, ref2, "masked == removed")


@pytest.mark.parametrize("case", [(2, 1152, 32, 128, 384, [384, 768, 2304, 1152]),
                                  (1, 192, 8, 64, 64, [128, 64, 384, 192]),
                                  (1, 192, 8, 64, 96, [96, 96, 384, 192]),
                                  (2, 192, 8, 128, 96, [96, 96, 384, 192]),
                                  (1, 75, 32, 64, 25, [600, 75]),
                                  (1, 128, 4, 128, 64, [64]),
                                  (1, 128, 4, 128, 64, [128]),
                                  (1, 128, 4, 128, 64, [192]),
                                  (2, 96, 4, 64, 64, [64, 64, 64]),
                                  (2, 1280, 32, 128, 384, [384, 768, 1152]),
                                  (1, 1024, 8, 64, 64, [256, 512, 1024]),
                                  (1, 300, 8, 128, 64, [128, 256, 320]),
                                  (2, 1152, 8, 64, 64, [256, 512, 1152])],
                         ids=["16x24grid", "64tok_frames", "8x12grid_96tok_frames", "8x12grid_96tok_D128",
                              "audio_25tok_frames", "1_tile", "2_tiles", "3_tiles", "3_segments_of_1_tile",
                              "pair_split_tail_1280q", "pair_one_round_D64", "odd_3_qtiles_partial_last",
                              "odd_9_qtiles_D64"])
def test_flash_attn_fp8_kv(dev, case):
    """fp8 K/V with one scale per (batch, head, frame); frames of 96 and 25
    tokens are cut into 64-key tiles at frame boundaries (64 + 32, and one
    partial tile per frame).  One to three key tiles exercise the staging
    prologue and the last iterations of the tile loop.  Even q-tile counts
    with frames of whole tiles take the pair workgroups (group 0 stages K,
    group 1 V): 1280 queries at B = 2 and 32 heads give 320 units, 256 whole
    and 64 cut into key ranges and merged; 1024 queries over 8 heads one
    partial round.  Odd q-tile counts >= 3 with frames of whole tiles run
    the pair workgroups over all but the last q-tile of every head and then
    the last ones, cut into key ranges, as a second launch: 1152 queries (9
    q-tiles, D = 128 and 64) and 300 (3, the last one partial)."""
    B, Lq, H, D, frame, lens = case
    g = gen(9)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    K = randn((B, sum(lens), H, D), g, torch.bfloat16)
    V = randn((B, sum(lens), H, D), g, torch.bfloat16)
    kc, ksc = OF.quantize_kv(K.float(), frame)
    vc, vsc = OF.quantize_kv(V.float(), frame)
    kc, vc, ksc, vsc = kc.to(dev), vc.to(dev), ksc.to(dev), vsc.to(dev)
    segs, pos = [], 0
    for n in lens:
        f0, nf = pos // frame, n // frame
        segs.append(KVSegment(kc[:, pos:pos + n], vc[:, pos:pos + n], ksc[:, :, f0:f0 + nf],
                              vsc[:, :, f0:f0 + nf]))
        pos += n
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    kernels.flash_attn(q.to(dev), segs, out, frame_tokens=frame)
    torch.cuda.synchronize()
    ref = _ref_attn(q, K, V)
    c = cosine(out, ref)
    assert c >= FP8_COSINE, c
    # against the dequantised cache the only error left is bf16 rounding
    Kd = OF.dequantize_kv(kc.cpu(), ksc.cpu(), frame)
    Vd = OF.dequantize_kv(vc.cpu(), vsc.cpu(), frame)
    assert_bf16_close(out, _ref_attn(q, Kd, Vd), "fp8 vs dequantised")


@pytest.mark.parametrize("frame", [64, 96])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("scales", [(1, 1, 1, 1), (1, 6, 1, 12), (12, 1, 6, 1)], ids=["flat", "rising", "falling"])
def test_flash_attn_fp8_ragged_segments(dev, D, scales, frame):
    """fp8 K/V in frame-aligned spans with gaps, segments ending mid-tile
    (partial last frames), per-frame scales spread over two orders of
    magnitude so later tiles raise the running maximum (rescale path).
    With scaled segments the softmax is so peaked that e4m3 rounding of K
    alone moves the fp32 answer (the oracle's own dequantised attention is at
    cosine 0.995 there), so those cases are held to the dequantised cache."""
    B, Lq, H = 2, 130, 2
    lens = [64, 100, 37, 192] if frame == 64 else [96, 150, 37, 288]
    g = gen(13)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    ks = [randn((B, n, H, D), g, torch.bfloat16, scale=s) for n, s in zip(lens, scales)]
    vs = [randn((B, n, H, D), g, torch.bfloat16, scale=s) for n, s in zip(lens, scales)]
    nfr = [-(-n // frame) for n in lens]
    cap = (sum(nfr) + len(lens)) * frame
    kc = torch.zeros(B, cap, H, D, dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    ksc = torch.ones(B, H, cap // frame, dtype=torch.float32, device=dev)
    vsc = torch.ones_like(ksc)
    segs, kd, vd, pos = [], [], [], 0
    for kk, vv, n, nf in zip(ks, vs, lens, nfr):
        pad = nf * frame - n
        kq, kq_s = OF.quantize_kv(torch.nn.functional.pad(kk.float(), (0, 0, 0, 0, 0, pad)), frame)
        vq, vq_s = OF.quantize_kv(torch.nn.functional.pad(vv.float(), (0, 0, 0, 0, 0, pad)), frame)
        f0 = pos // frame
        kc[:, pos:pos + n] = kq[:, :n].to(dev)
        vc[:, pos:pos + n] = vq[:, :n].to(dev)
        ksc[:, :, f0:f0 + nf] = kq_s.to(dev)
        vsc[:, :, f0:f0 + nf] = vq_s.to(dev)
        segs.append(KVSegment(kc[:, pos:pos + n], vc[:, pos:pos + n], ksc[:, :, f0:f0 + nf], vsc[:, :, f0:f0 + nf]))
        kd.append(OF.dequantize_kv(kq, kq_s, frame)[:, :n])
        vd.append(OF.dequantize_kv(vq, vq_s, frame)[:, :n])
        pos += (nf + 1) * frame   # one free frame between spans
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    kernels.flash_attn(q.to(dev), segs, out, frame_tokens=frame)
    torch.cuda.synchronize()
    K, V = torch.cat(ks, 1), torch.cat(vs, 1)
    if max(scales) == 1:
        assert cosine(out, _ref_attn(q, K, V)) >= FP8_COSINE
    assert_bf16_close(out, _ref_attn(q, torch.cat(kd, 1), torch.cat(vd, 1)), f"fp8 ragged {scales} D{D}",
                      max_abs=2e-2 * max(scales), mean_abs=2e-3 * max(scales))


@pytest.mark.parametrize("C,L,per_row", [(4096, 1152, False), (2048, 75, True), (512, 33, False)])
def test_adaln_matches_torch_ops(dev, C, L, per_row):
    """ltx_adaln against the reference's bf16 tensor ops on the GPU: the gated
    residual x + y * g is bit-identical; rms_norm(x') * (1 + scale) + shift
    rounds the same way (equal except where the float32 sum of squares, summed
    in another order, flips a rounding)."""
    g = gen(21)
    B = 2
    x = randn((B, L, C), g, torch.bfloat16, 2.0).to(dev)
    y = randn((B, L, C), g, torch.bfloat16, 0.5).to(dev)
    rows = L if per_row else 1
    tab = randn((B, rows, 3, C), g, torch.bfloat16, 0.3).to(dev)   # shift / scale / gate rows, strided
    sh, sc, gt = tab.unbind(dim=2)
    F = torch.nn.functional
    x1 = x + y * gt
    ref_mod = F.rms_norm(x1, (C,), None, 1e-6) * (1 + sc) + sh
    ref_plain = F.rms_norm(x1, (C,), None, 1e-6)
    xo, n1, n2 = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)
    kernels.adaln(x, y=y, gate=gt, x_out=xo, n_out=n1, scale=sc, shift=sh)
    kernels.adaln(x, y=y, gate=gt, x_out=x, n_out=n2)        # in place, plain norm
    r = torch.empty_like(x)
    kernels.adaln(xo, y=y, x_out=r)                           # ungated residual only
    torch.cuda.synchronize()
    assert torch.equal(xo, x1) and torch.equal(x, x1)
    assert torch.equal(r, x1 + y)
    for out, ref in ((n1, ref_mod), (n2, ref_plain)):
        exact = (out == ref).float().mean().item()
        d = (out.float() - ref.float()).abs().max().item()
        assert exact >= 0.995 and d <= 2 ** -6 * ref.float().abs().max().item(), (exact, d)


@pytest.mark.parametrize("vlayout", ["token", "key"])
@pytest.mark.parametrize("D,Lq,H", [(64, 1152, 64), (64, 1280, 64), (128, 1280, 32)])
def test_flash_attn_split_tail(dev, vlayout, D, Lq, H):
    """Enough q-tiles to leave a partial last round and 32 key tiles, so the
    tail q-tiles are cut into key ranges and merged by the combine kernel;
    both V layouts against fp32.  1152 queries (9 q-tiles per head) run the
    4-wave kernels; 1280 (10 per head) with key-major V runs the pair kernel,
    whose split units each leave two q-tiles' partials."""
    B, lens = 2, [1024, 1024]
    ws = ctypes.c_int64(0)
    _native.call("ltx_flash_attn_workspace_size", B, Lq, H, D, ctypes.byref(ws))
    assert ws.value > 0, "the shape must plan a split tail"
    g = gen(17)
    q = randn((B, Lq, H, D), g, torch.bfloat16)
    ks = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    vs = [randn((B, n, H, D), g, torch.bfloat16) for n in lens]
    cap = sum(lens) + 64
    ka = torch.zeros(B, cap, H, D, dtype=torch.bfloat16, device=dev)
    va = torch.zeros_like(ka) if vlayout == "token" else \
        torch.zeros(B, H, D, cap, dtype=torch.bfloat16, device=dev).permute(0, 3, 1, 2)
    segs, pos = [], 0
    for kk, vv in zip(ks, vs):
        n = kk.shape[1]
        ka[:, pos:pos + n] = kk.to(dev)
        va[:, pos:pos + n] = vv.to(dev)
        segs.append(KVSegment(ka[:, pos:pos + n], va[:, pos:pos + n]))
        pos += n + 32
    out = torch.empty(B, Lq, H, D, dtype=torch.bfloat16, device=dev)
    kernels.flash_attn(q.to(dev), segs, out)
    torch.cuda.synchronize()
    assert_bf16_close(out, _ref_attn(q, torch.cat(ks, 1), torch.cat(vs, 1)), f"D{D} Lq{Lq} split tail {vlayout}")
