"""Typed wrappers over the C ABI: torch device tensors in, kernels enqueued on the
current HIP stream.  Shapes and strides are checked here before any launch so a
malformed call raises instead of reaching the GPU."""
from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Sequence, Tuple

import torch

from . import _native as N

_DT = {torch.float32: N.F32, torch.bfloat16: N.BF16, torch.uint8: N.F8E4M3,
       torch.float8_e4m3fn: N.F8E4M3}


def _code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_gpu(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("taomate_amd kernels take device tensors (got a CPU tensor)")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def rope_table(freq_idx: torch.Tensor, grid: Tuple[int, ...], start_frame: int, is_audio: bool,
               max_pos: Sequence[float], dim: int, num_heads: int, batch: int,
               dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    """ltx_rope_table -> (cos, sin) [batch, H, T, dim/(2H)] on freq_idx's device."""
    _need_gpu(freq_idx)
    assert freq_idx.dtype == torch.float32 and freq_idx.is_contiguous()
    nd = len(grid)
    T = math.prod(grid)
    per = dim // 2 // num_heads
    cos = torch.empty(batch, num_heads, T, per, device=freq_idx.device, dtype=dtype)
    sin = torch.empty_like(cos)
    gf = grid[0]
    gh = grid[1] if nd == 3 else 1
    gw = grid[2] if nd == 3 else 1
    mp = list(max_pos) + [1.0] * (3 - len(max_pos))
    N.call("ltx_rope_table", cos.data_ptr(), sin.data_ptr(), _code(cos), freq_idx.data_ptr(),
           freq_idx.numel(), nd, gf, gh, gw, int(start_frame), int(bool(is_audio)),
           float(mp[0]), float(mp[1]), float(mp[2]), dim, num_heads, batch, _stream(freq_idx))
    return cos, sin


def rope_table_retime(src: Tuple[torch.Tensor, torch.Tensor], freq_idx: torch.Tensor, grid: Tuple[int, int, int],
                      start_frame: int, max_pos_t: float, dim: int, num_heads: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """ltx_rope_table_retime: the video table of ``grid`` at ``start_frame``
    from ``src`` = (cos, sin) [1, H, T, dim/(2H)] of the same grid built for
    another start frame."""
    cs, ss = src
    _need_gpu(freq_idx, cs, ss)
    T = math.prod(grid)
    per = dim // 2 // num_heads
    for t in (cs, ss):
        if t.shape != (1, num_heads, T, per) or not t.is_contiguous() or t.dtype != cs.dtype:
            raise ValueError(f"rope_table_retime: source tables must be contiguous [1, {num_heads}, {T}, {per}]")
    cos = torch.empty_like(cs)
    sin = torch.empty_like(ss)
    N.call("ltx_rope_table_retime", cos.data_ptr(), sin.data_ptr(), cs.data_ptr(), ss.data_ptr(), _code(cos),
           freq_idx.data_ptr(), freq_idx.numel(), grid[0], grid[1], grid[2], int(start_frame), float(max_pos_t),
           dim, num_heads, _stream(freq_idx))
    return cos, sin


def _rows(t: torch.Tensor, HD: int) -> Tuple[int, int, int]:
    """(len, b_stride, l_stride) of a [B, L, H*D] (or [B, L, H, D]) row tensor."""
    if t.dim() == 4:
        B, L, H, D = t.shape
        if t.stride(3) != 1 or t.stride(2) != D:
            raise ValueError("rows must be contiguous over (H, D)")
        return L, t.stride(0), t.stride(1)
    if t.dim() != 3 or t.shape[-1] != HD or t.stride(2) != 1:
        raise ValueError(f"expected [B, L, {HD}] rows with a contiguous last dim, got {tuple(t.shape)}")
    return t.shape[1], t.stride(0), t.stride(1)


def _table(tab, H: int, D: int, L: int, B: int):
    if tab is None:
        return None, None, 0, 0, 0, None
    cos, sin = tab
    if cos.shape != sin.shape or cos.stride() != sin.stride() or cos.dtype != sin.dtype:
        raise ValueError("cos/sin tables must share shape, strides and dtype")
    if cos.dim() != 4 or cos.shape[1] != H or cos.shape[3] != D // 2 or cos.shape[2] < L:
        raise ValueError(f"RoPE table {tuple(cos.shape)} does not match H={H} D/2={D // 2} T>={L}")
    if cos.stride(3) != 1:
        raise ValueError("RoPE table last dim must be contiguous")
    if cos.shape[0] not in (1, B):
        raise ValueError(f"RoPE table batch {cos.shape[0]} vs input batch {B}")
    tb = 0 if cos.shape[0] == 1 else cos.stride(0)
    return cos, sin, tb, cos.stride(1), cos.stride(2), cos.dtype


def qk_rmsnorm_rope(q_in: torch.Tensor, q_out: torch.Tensor, gamma_q: Optional[torch.Tensor],
                    eps_q: Optional[float], q_tab, H: int, D: int,
                    k_in: Optional[torch.Tensor] = None, k_out: Optional[torch.Tensor] = None,
                    gamma_k: Optional[torch.Tensor] = None, eps_k: Optional[float] = None,
                    k_tab=None, v_in: Optional[torch.Tensor] = None, v_out: Optional[torch.Tensor] = None) -> None:
    """ltx_qk_rmsnorm_rope.  eps None skips the norm; a None table skips RoPE.
    With ``v_in`` [B, L, H, D] and a key-major bf16 ``v_out`` view of the same
    shape (the arena's V slots), the V append rides in the same launch
    (ltx_qk_rmsnorm_rope_v)."""
    _need_gpu(q_in, q_out, k_in, k_out, gamma_q, gamma_k, v_in, v_out)
    HD = H * D
    B = q_in.shape[0]
    dt = q_in.dtype
    for t in (q_out, k_in, k_out, gamma_q, gamma_k):
        if t is not None and t.dtype != dt:
            raise TypeError("q/k inputs, outputs and gammas must share one dtype")
    ql, qbs, qls = _rows(q_in, HD)
    qol, qobs, qols = _rows(q_out, HD)
    if qol != ql or q_out.shape[0] != B:
        raise ValueError("q_out shape mismatch")
    qc, qs, qtb, qth, qtt, qtd = _table(q_tab, H, D, ql, B)
    if k_in is not None:
        kl, kbs, kls = _rows(k_in, HD)
        kol, kobs, kols = _rows(k_out, HD)
        if kol != kl or k_in.shape[0] != B or k_out.shape[0] != B:
            raise ValueError("k_out shape mismatch")
        kc, ks, ktb, kth, ktt, ktd = _table(k_tab, H, D, kl, B)
    else:
        kl = kbs = kls = kobs = kols = 0
        kc = ks = None
        ktb = kth = ktt = 0
        ktd = None
    tds = {d for d in (qtd, ktd) if d is not None}
    if len(tds) > 1:
        raise TypeError("q and k RoPE tables must share a dtype")
    tab_code = _DT[tds.pop()] if tds else N.BF16
    for g in (gamma_q, gamma_k):
        if g is not None and (g.numel() != HD or not g.is_contiguous()):
            raise ValueError("gamma must be a contiguous [H*D] vector")
    args = (_code(q_in), B, H, D,
            q_in.data_ptr(), ql, qbs, qls, q_out.data_ptr(), qobs, qols,
            _ptr(gamma_q), -1.0 if eps_q is None else float(eps_q),
            _ptr(qc), _ptr(qs), qtb, qth, qtt,
            _ptr(k_in), kl, kbs, kls, _ptr(k_out), kobs, kols,
            _ptr(gamma_k), -1.0 if eps_k is None else float(eps_k),
            _ptr(kc), _ptr(ks), ktb, kth, ktt, tab_code)
    if v_in is None and v_out is None:
        N.call("ltx_qk_rmsnorm_rope", *args, _stream(q_in))
        return
    if v_in is None or v_out is None:
        raise ValueError("v_in and v_out go together")
    if v_in.dim() != 4 or v_out.shape != v_in.shape or v_in.shape[0] != B or v_in.shape[2:] != (H, D):
        raise ValueError(f"V {tuple(v_in.shape)} -> {tuple(v_out.shape)} does not match B={B} H={H} D={D}")
    if v_in.dtype != torch.bfloat16 or v_out.dtype != torch.bfloat16 or v_in.stride(3) != 1:
        raise ValueError("V must be bf16 with a contiguous head dim")
    if v_out.stride(1) != 1:
        raise ValueError("v_out must be key-major (token stride 1)")
    N.call("ltx_qk_rmsnorm_rope_v", *args, v_in.data_ptr(), v_in.shape[1], v_in.stride(0), v_in.stride(1),
           v_in.stride(2), v_out.data_ptr(), v_out.stride(0), v_out.stride(2), v_out.stride(3), _stream(q_in))


def kv_append(src: torch.Tensor, dst: torch.Tensor, scales: Optional[torch.Tensor] = None,
              frame_tokens: int = 1) -> None:
    """ltx_kv_append: src [B, L, H, D] -> dst [B, L, H, D] view.

    A token-major dst (head dim contiguous) is a bf16 copy or an fp8 quantise
    (``scales`` float32 [B, H, L/frame_tokens], frame index contiguous); a
    key-major dst (token stride 1, the arena's V layout) is a bf16 transpose."""
    _need_gpu(src, dst, scales)
    if src.dim() != 4 or dst.shape != src.shape:
        raise ValueError(f"kv_append: shapes {tuple(src.shape)} vs {tuple(dst.shape)}")
    if src.stride(3) != 1:
        raise ValueError("kv_append: src head dim must be contiguous")
    B, L, H, D = src.shape
    key_major = dst.stride(3) != 1
    if key_major and (dst.stride(1) != 1 or _code(dst) != N.BF16):
        raise ValueError("kv_append: dst must be token-major or bf16 key-major")
    sc_bs = sc_hs = 0
    if _code(dst) == N.F8E4M3:
        if scales is None or scales.dtype != torch.float32:
            raise ValueError("kv_append: fp8 destination needs float32 scales")
        if L % frame_tokens != 0 or scales.shape != (B, H, L // frame_tokens) or (
                L and scales.stride(2) != 1):
            raise ValueError(f"kv_append: scales {tuple(scales.shape)} for L={L}, frame={frame_tokens}")
        sc_bs, sc_hs = scales.stride(0), scales.stride(1)
    N.call("ltx_kv_append", _code(src), _code(dst), B, L, H, D, src.data_ptr(),
           src.stride(0), src.stride(1), src.stride(2), dst.data_ptr(), dst.stride(0),
           dst.stride(1), dst.stride(2), dst.stride(3), _ptr(scales), sc_bs, sc_hs,
           int(frame_tokens), _stream(src))


def kv_append_fp8_pair(k: torch.Tensor, k_dst: torch.Tensor, k_scales: torch.Tensor, v: torch.Tensor,
                       v_dst: torch.Tensor, v_scales: torch.Tensor, frame_tokens: int) -> None:
    """ltx_kv_append_fp8_pair: a chunk's bf16 K and V [B, L, H, D] quantised into
    fp8 arena slots in one launch (codes and scales as ``kv_append``)."""
    _need_gpu(k, k_dst, k_scales, v, v_dst, v_scales)
    if k.dim() != 4 or v.shape != k.shape or k_dst.shape != k.shape or v_dst.shape != k.shape:
        raise ValueError(f"kv_append_fp8_pair: shapes {tuple(k.shape)}, {tuple(v.shape)}, "
                         f"{tuple(k_dst.shape)}, {tuple(v_dst.shape)}")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("kv_append_fp8_pair: K and V must be bf16")
    if _code(k_dst) != N.F8E4M3 or _code(v_dst) != N.F8E4M3:
        raise TypeError("kv_append_fp8_pair: destinations must be fp8 (uint8 codes)")
    if k.stride(3) != 1 or v.stride(3) != 1 or k_dst.stride(3) != 1 or v_dst.stride(3) != 1:
        raise ValueError("kv_append_fp8_pair: head dim must be contiguous")
    if k_dst.stride() != v_dst.stride():
        raise ValueError("kv_append_fp8_pair: K and V destinations must share strides")
    B, L, H, D = k.shape
    if L % frame_tokens != 0:
        raise ValueError(f"kv_append_fp8_pair: L={L} is not a whole number of {frame_tokens}-token frames")
    for sc in (k_scales, v_scales):
        if sc.dtype != torch.float32 or sc.shape != (B, H, L // frame_tokens) or (L and sc.stride(2) != 1):
            raise ValueError(f"kv_append_fp8_pair: scales {tuple(sc.shape)} for L={L}, frame={frame_tokens}")
    if k_scales.stride() != v_scales.stride():
        raise ValueError("kv_append_fp8_pair: K and V scales must share strides")
    N.call("ltx_kv_append_fp8_pair", B, L, H, D, int(frame_tokens),
           k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), k_dst.data_ptr(), k_scales.data_ptr(),
           v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), v_dst.data_ptr(), v_scales.data_ptr(),
           k_dst.stride(0), k_dst.stride(1), k_dst.stride(2), k_scales.stride(0), k_scales.stride(1),
           _stream(k))


def kv_gather(src: torch.Tensor, dst: torch.Tensor, spans: Sequence[Tuple[int, int]]) -> None:
    """ltx_kv_gather: dst[:, 0:sum(len)] = cat(src[:, s:s+len] for s, len in spans)."""
    _need_gpu(src, dst)
    if src.dtype != dst.dtype or src.dim() != 4 or dst.dim() != 4 or src.shape[0] != dst.shape[0] \
            or src.shape[2:] != dst.shape[2:]:
        raise ValueError("kv_gather: src/dst layout mismatch")
    if src.stride(3) != 1 or dst.stride(3) != 1:
        raise ValueError("kv_gather: head dim must be contiguous")
    total = sum(int(n) for _, n in spans)
    if total > dst.shape[1]:
        raise ValueError(f"kv_gather: {total} tokens do not fit dst ({dst.shape[1]})")
    for s, n in spans:
        if s < 0 or n < 0 or s + n > src.shape[1]:
            raise ValueError(f"kv_gather: span ({s}, {n}) outside src ({src.shape[1]})")
    B, _, H, D = src.shape
    starts = N.i64_array([s for s, _ in spans])
    lens = N.i64_array([n for _, n in spans])
    N.call("ltx_kv_gather", src.element_size(), B, H, D, src.data_ptr(), src.stride(0),
           src.stride(1), src.stride(2), dst.data_ptr(), dst.stride(0), dst.stride(1),
           dst.stride(2), len(spans), ctypes.cast(starts, ctypes.c_void_p),
           ctypes.cast(lens, ctypes.c_void_p), _stream(src))


_WS_SIZE: dict = {}
_WS: dict = {}


def _flash_workspace(q: torch.Tensor, B: int, Lq: int, H: int, D: int):
    """Device workspace for the balanced-tail split (partial results), one per
    (device, stream) so overlapping launches never share one; grown on demand."""
    key = (q.device.index, B, Lq, H, D)
    need = _WS_SIZE.get(key)
    if need is None:
        out = ctypes.c_int64(0)
        N.call("ltx_flash_attn_workspace_size", B, Lq, H, D, ctypes.byref(out))
        need = _WS_SIZE[key] = int(out.value)
    if need == 0:
        return None, 0
    skey = (q.device.index, _stream(q))
    ws = _WS.get(skey)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        _WS[skey] = ws
    return ws, ws.numel()


class KVSegment:
    """One key/value span for flash_attn: k, v [B, L, H, D] views sharing strides;
    for fp8, k_scales / v_scales are float32 [B, H, L/frame] views."""
    __slots__ = ("k", "v", "k_scales", "v_scales")

    def __init__(self, k, v, k_scales=None, v_scales=None):
        self.k, self.v, self.k_scales, self.v_scales = k, v, k_scales, v_scales


def flash_attn(q: torch.Tensor, segments: List[KVSegment], out: torch.Tensor,
               key_mask: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
               scale: Optional[float] = None, frame_tokens: int = 0, noalloc: bool = False,
               key_lens: Optional[Sequence[int]] = None) -> None:
    """ltx_flash_attn_fwd.  q/out [B, Lq, H, D] bf16; key_mask float32 [B, Lk] additive.
    ``key_lens`` (B host ints): batch row b attends keys [0, key_lens[b]) only
    (a prefix-per-row padding mask, bf16 key-major V, on the pipelined kernel).
    ``noalloc`` calls ltx_flash_attn_fwd_noalloc instead: no workspace tensor,
    the split partials go to the library's fixed per-device scratch array
    (calls overlapping on one device race on it)."""
    _need_gpu(q, out, key_mask, lse)
    if q.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise TypeError("flash_attn: q and out must be bf16")
    if q.dim() != 4 or out.shape != q.shape or q.stride(3) != 1 or out.stride(3) != 1:
        raise ValueError("flash_attn: q/out must be [B, Lq, H, D] with contiguous D")
    B, Lq, H, D = q.shape
    segs = [s for s in segments if s.k.shape[1] > 0]
    if not segs:
        raise ValueError("flash_attn: no keys")
    if len(segs) > N.MAX_SEGMENTS:
        raise ValueError(f"flash_attn: {len(segs)} segments > {N.MAX_SEGMENTS}")
    kv_code = _code(segs[0].k)
    kst = vst = None
    lk = 0
    for s in segs:
        for t, which in ((s.k, "k"), (s.v, "v")):
            _need_gpu(t)
            if t.dim() != 4 or t.shape[0] != B or t.shape[2] != H or t.shape[3] != D:
                raise ValueError(f"flash_attn: segment {tuple(t.shape)} vs q {tuple(q.shape)}")
            if _code(t) != kv_code:
                raise ValueError("flash_attn: segments must share one dtype")
        if s.k.stride(3) != 1:
            raise ValueError("flash_attn: K head dim must be contiguous")
        if s.v.stride(3) != 1 and s.v.stride(1) != 1:
            raise ValueError("flash_attn: V must be token-major or key-major")
        ks = (s.k.stride(0), s.k.stride(1), s.k.stride(2))
        vs = (s.v.stride(0), s.v.stride(1), s.v.stride(2), s.v.stride(3))
        if kst is None:
            kst, vst = ks, vs
        elif ks != kst or vs != vst:
            raise ValueError("flash_attn: all K/V segments must share strides")
        if s.v.shape[1] != s.k.shape[1]:
            raise ValueError("flash_attn: k/v segment lengths differ")
        lk += s.k.shape[1]
    fp8 = kv_code == N.F8E4M3
    sc_bs = sc_hs = 0
    if fp8:
        sst = None
        for s in segs:
            for sc in (s.k_scales, s.v_scales):
                if sc is None or sc.dtype != torch.float32 or sc.shape[0] != B or sc.shape[1] != H:
                    raise ValueError("flash_attn: fp8 segments need float32 [B, H, nF] scales")
                if sc.shape[2] * frame_tokens < s.k.shape[1] or (sc.shape[2] > 1 and sc.stride(2) != 1):
                    raise ValueError("flash_attn: fp8 scales do not cover the segment")
                if sst is None:
                    sst = (sc.stride(0), sc.stride(1))
                elif (sc.stride(0), sc.stride(1)) != sst:
                    raise ValueError("flash_attn: fp8 scale tensors must share strides")
        sc_bs, sc_hs = sst
    mask_bs = 0
    if key_mask is not None:
        if key_mask.dtype != torch.float32 or key_mask.dim() != 2 or key_mask.shape[1] != lk or \
                key_mask.shape[0] not in (1, B) or key_mask.stride(1) != 1:
            raise ValueError(f"flash_attn: key_mask must be float32 [B, {lk}] with contiguous keys")
        mask_bs = 0 if key_mask.shape[0] == 1 else key_mask.stride(0)
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (B, H, Lq) or not lse.is_contiguous()):
        raise ValueError("flash_attn: lse must be contiguous float32 [B, H, Lq]")
    kl = None
    if key_lens is not None:
        if len(key_lens) != B or any(not 0 <= int(n) <= lk for n in key_lens):
            raise ValueError(f"flash_attn: key_lens must hold {B} counts in [0, {lk}]")
        kl = N.i64_array([int(n) for n in key_lens])
    kp = N.ptr_array([s.k.data_ptr() for s in segs])
    vp = N.ptr_array([s.v.data_ptr() for s in segs])
    lens = N.i64_array([s.k.shape[1] for s in segs])
    ksp = N.ptr_array([s.k_scales.data_ptr() for s in segs]) if fp8 else None
    vsp = N.ptr_array([s.v_scales.data_ptr() for s in segs]) if fp8 else None
    args = (q.data_ptr(), B, Lq, H, D, q.stride(0), q.stride(1), q.stride(2),
            len(segs), ctypes.cast(kp, ctypes.c_void_p), ctypes.cast(vp, ctypes.c_void_p),
            ctypes.cast(lens, ctypes.c_void_p), kst[0], kst[1], kst[2], vst[0], vst[1], vst[2], vst[3],
            kv_code,
            ctypes.cast(ksp, ctypes.c_void_p) if fp8 else None,
            ctypes.cast(vsp, ctypes.c_void_p) if fp8 else None, sc_bs, sc_hs,
            int(frame_tokens), _ptr(key_mask), mask_bs,
            ctypes.cast(kl, ctypes.c_void_p) if kl is not None else None, out.data_ptr(), out.stride(0), out.stride(1),
            out.stride(2), _ptr(lse), float(scale) if scale is not None else 0.0)
    if noalloc:
        N.call("ltx_flash_attn_fwd_noalloc", *args, _stream(q))
        return
    ws, ws_bytes = _flash_workspace(q, B, Lq, H, D)
    N.call("ltx_flash_attn_fwd", *args, _ptr(ws), ws_bytes, _stream(q))


def adaln(x: torch.Tensor, y: Optional[torch.Tensor] = None, gate: Optional[torch.Tensor] = None,
          x_out: Optional[torch.Tensor] = None, n_out: Optional[torch.Tensor] = None,
          scale: Optional[torch.Tensor] = None, shift: Optional[torch.Tensor] = None, eps: float = 1e-6) -> None:
    """ltx_adaln on bf16 [B, L, C] rows: x_out = x + y * gate (x + y without a
    gate), n_out = rms_norm(x_out or x) * (1 + scale) + shift (plain rms_norm
    without scale/shift).  gate/scale/shift are [B, 1 or L, C]."""
    _need_gpu(x, y, gate, x_out, n_out, scale, shift)
    if x.dim() != 3 or x.dtype != torch.bfloat16:
        raise ValueError("adaln: x must be bf16 [B, L, C]")
    B, L, C = x.shape

    def rows(t, name, per_row_ok=True):
        if t is None:
            return None, 0, 0
        if t.dtype != torch.bfloat16 or t.dim() != 3 or t.shape[0] != B or t.shape[2] != C or t.stride(2) != 1:
            raise ValueError(f"adaln: {name} must be bf16 [B, L or 1, C] with contiguous channels")
        if t.shape[1] == L:
            return t.data_ptr(), t.stride(0), (t.stride(1) if L > 1 else 0)
        if t.shape[1] == 1 and per_row_ok:
            return t.data_ptr(), t.stride(0), 0
        raise ValueError(f"adaln: {name} rows {t.shape[1]} vs L={L}")

    args = [rows(x, "x"), rows(y, "y"), rows(gate, "gate"), rows(x_out, "x_out"), rows(n_out, "n_out"),
            rows(scale, "scale"), rows(shift, "shift")]
    for t, name in ((y, "y"), (x_out, "x_out"), (n_out, "n_out")):
        if t is not None and t.shape[1] != L:
            raise ValueError(f"adaln: {name} must have L={L} rows")
    flat = [v for a in args for v in a]
    N.call("ltx_adaln", B, L, C, *flat, float(eps), _stream(x))
