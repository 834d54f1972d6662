"""Drop-in attention surface on gfx950 kernels.

Host mirror of:
  CausalLTXAttention            ltx_causal/attention/causal_attention.py:61-338
  standard_attention_forward    ltx_causal/attention/flex_attention_utils.py:225-276
  attention_with_cache          ltx_causal/transformer/kv_cache.py:1148-1547 (single GPU)
  _finish_attention_output...   ltx_causal/transformer/kv_cache.py:1680-1700

Projections (to_q/to_k/to_v/to_out, to_gate_logits) stay ``nn.Linear`` GEMMs on
PyTorch-ROCm (hipBLASLt).  Everything between them runs in this package's HIP
kernels: fused full-row q/k RMSNorm + SPLIT RoPE (writing new keys straight into
their KV-arena slots), the V append, and flash attention over the cached spans
plus the new chunk.  Activations are bf16, as on the reference's GPU path.
"""
from __future__ import annotations

import collections
import weakref
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from . import _native as N
from . import kernels
from .kernels import KVSegment
from .kv_cache import KVSpanView, module_arena
from .rope import CausalRopeType, apply_split_rotary_emb


class CausalLTXAttention(nn.Module):
    """causal_attention.py:61-118: weight-compatible module (same attribute names)."""

    def __init__(self, query_dim: int, context_dim: Optional[int] = None, heads: int = 8,
                 dim_head: int = 64, norm_eps: float = 1e-6,
                 rope_type: CausalRopeType = CausalRopeType.SPLIT,
                 apply_gated_attention: bool = False, local_attn_size: int = -1,
                 sink_size: int = 1):
        super().__init__()
        self.rope_type = rope_type
        self.heads = heads
        self.dim_head = dim_head
        self.inner_dim = heads * dim_head
        self.is_cross_attention = context_dim is not None
        context_dim = query_dim if context_dim is None else context_dim
        self.to_q = nn.Linear(query_dim, self.inner_dim, bias=True)
        self.to_k = nn.Linear(context_dim, self.inner_dim, bias=True)
        self.to_v = nn.Linear(context_dim, self.inner_dim, bias=True)
        self.q_norm = nn.RMSNorm(self.inner_dim, eps=norm_eps)
        self.k_norm = nn.RMSNorm(self.inner_dim, eps=norm_eps)
        self.to_gate_logits = nn.Linear(query_dim, heads, bias=True) if apply_gated_attention else None
        self.to_out = nn.Sequential(nn.Linear(self.inner_dim, query_dim, bias=True), nn.Identity())

    def fuse_qkv_(self) -> "CausalLTXAttention":
        """Re-home to_q / to_k / to_v's weights and biases in one packed
        [3·inner, dim] buffer, the three parameters becoming row views of it
        (no extra memory; names, values and state_dict unchanged), so that a
        self-attention projects q, k and v with one GEMM.  A no-op for
        cross-attention (K and V come from the context).  Anything that
        re-creates a parameter afterwards (``load_state_dict(assign=True)``,
        ``.to()``, assignment) ends the packing and the three GEMMs run again."""
        if self.is_cross_attention:
            return self
        lins = (self.to_q, self.to_k, self.to_v)
        with torch.no_grad():
            w = torch.cat([lin.weight.detach() for lin in lins], 0)
            b = torch.cat([lin.bias.detach() for lin in lins], 0)
        n = self.inner_dim
        for i, lin in enumerate(lins):
            lin.weight = nn.Parameter(w[i * n:(i + 1) * n], requires_grad=lin.weight.requires_grad)
            lin.bias = nn.Parameter(b[i * n:(i + 1) * n], requires_grad=lin.bias.requires_grad)
        self._qkv_packed = (w, b)
        return self

    def _packed_qkv(self) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """The packed (weight, bias) while the three projections still alias it."""
        pk = getattr(self, "_qkv_packed", None)
        if pk is None:
            return None
        w, b = pk
        n = self.inner_dim
        for i, lin in enumerate((self.to_q, self.to_k, self.to_v)):
            if lin.weight.data_ptr() != w[i * n].data_ptr() or lin.bias is None or \
                    lin.bias.data_ptr() != b[i * n:].data_ptr() or lin.weight.shape != w[i * n:(i + 1) * n].shape:
                self._qkv_packed = None   # a parameter was replaced: drop the stale buffer
                return None
        return w, b

    def cache_text_kv_(self, enabled: bool = True, size: int = 4) -> "CausalLTXAttention":
        """Keep the normalised K and the V of the last ``size`` contexts
        (_get_cached_text_cross_kv, kv_cache.py:707-760: the exact,
        inference-only LRU of the text cross-attention's projections, off by
        default there too).  A hit needs the same context tensor object,
        unmodified since (its version counter), and unchanged K/V parameters;
        anything else projects again."""
        self._text_kv_cache = collections.OrderedDict() if enabled else None
        self._text_kv_size = int(size)
        return self

    def _cached_text_kv(self, ctx: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """k = k_norm(to_k(ctx)) [B, L, H*D] and v = to_v(ctx) as a [B, L, H, D]
        view of a key-major store (the layout the pipelined kernel streams into
        LDS, made once when the entry is filled instead of on every call), from
        the cache when it holds them."""
        params = tuple((p.data_ptr(), p._version) for p in (self.to_k.weight, self.to_k.bias, self.to_v.weight,
                                                              self.to_v.bias, self.k_norm.weight) if p is not None)
        key = (id(ctx), ctx.data_ptr(), tuple(ctx.shape), tuple(ctx.stride()), ctx.dtype, str(ctx.device),
               ctx._version, params)
        cache = self._text_kv_cache
        hit = cache.get(key)
        if hit is not None and hit[0]() is ctx:
            cache.move_to_end(key)
            return hit[1], hit[2]
        k = _norm_one(self.k_norm, self.to_k(ctx), None, self.heads, self.dim_head)
        v_lin = self.to_v(ctx)
        v = _key_major(v_lin.view(v_lin.shape[0], -1, self.heads, self.dim_head)) \
            if self.dim_head in (64, 128) else v_lin
        cache[key] = (weakref.ref(ctx), k, v)
        while len(cache) > self._text_kv_size:
            cache.popitem(last=False)
        return k, v

    def _apply_rope(self, x: torch.Tensor, freqs_cis: Tuple[torch.Tensor, torch.Tensor]) -> torch.Tensor:
        """causal_attention.py:326-338 (SPLIT only)."""
        if self.rope_type != CausalRopeType.SPLIT:
            raise NotImplementedError("only SPLIT RoPE is built")
        return apply_split_rotary_emb(x, *freqs_cis)

    def forward(self, x: torch.Tensor, context: Optional[torch.Tensor] = None,
                mask: Optional[torch.Tensor] = None, pe=None, k_pe=None, block_mask=None,
                cross_causal_mask=None, logit_log_scale: Optional[torch.Tensor] = None,
                sp_context_sharded: bool = True) -> torch.Tensor:
        """causal_attention.py:120-324 on the inference path (no block masks, SP off).

        This is the route text cross-attention takes (kv_cache.py:764-785): q/k
        norm, optional RoPE, an optional key-padding mask, gate and to_out.
        """
        if block_mask is not None or cross_causal_mask is not None:
            raise NotImplementedError("training block masks are not part of the inference path")
        B = x.shape[0]
        ctx = x if context is None else context
        if context is not None and pe is None and k_pe is None and getattr(self, "_text_kv_cache", None) is not None \
                and not torch.is_grad_enabled():
            k, v = self._cached_text_kv(context)
            q = _norm_one(self.q_norm, self.to_q(x), None, self.heads, self.dim_head)
        else:
            q_lin, k_lin, v = self.to_q(x), self.to_k(ctx), self.to_v(ctx)
            q, k = _norm_rope(self, q_lin, k_lin, pe, k_pe, None)
        if logit_log_scale is not None:
            q = q * logit_log_scale
        H, D = self.heads, self.dim_head
        q4 = q.view(B, -1, H, D)
        k4 = k.view(B, -1, H, D)
        v4 = v if v.dim() == 4 else v.view(B, -1, H, D)
        out = standard_attention_forward(q4, k4, v4, mask=mask)
        return _finish(self, out, x)


def _check_bf16(*ts):
    for t in ts:
        if t is not None and t.dtype != torch.bfloat16:
            raise TypeError(f"the gfx950 attention path runs bf16 activations, got {t.dtype}")


def packed_qkv(attn: nn.Module) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """The packed q/k/v (weight, bias) of a module packed by ``fuse_qkv_``;
    None for any other module, including one built by the reference
    (causal_attention.py:61-118), which carries only the three Linears."""
    fn = getattr(attn, "_packed_qkv", None)
    return fn() if fn is not None else None


def _project_qkv(attn: nn.Module, x: torch.Tensor, ctx: torch.Tensor):
    """to_q(x), to_k(ctx), to_v(ctx) (kv_cache.py:1406-1408).  A self-attention
    packed by ``fuse_qkv_`` runs one GEMM and returns three column views of its
    [B, L, 3·inner] output (row stride 3·inner), which the norm / RoPE and
    append kernels read in place."""
    packed = packed_qkv(attn) if ctx is x else None
    if packed is None:
        return attn.to_q(x), attn.to_k(ctx), attn.to_v(ctx)
    y = torch.nn.functional.linear(x, *packed)
    n = attn.inner_dim
    return y[..., :n], y[..., n:2 * n], y[..., 2 * n:]


def _norm_rope(attn: CausalLTXAttention, q_lin: torch.Tensor, k_lin: torch.Tensor, pe, k_pe,
               k_out: Optional[torch.Tensor], v_in: Optional[torch.Tensor] = None,
               v_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """q = rope(q_norm(q_lin)), k = rope(k_norm(k_lin)) in one launch
    (kv_cache.py:1406-1417).  ``k_out`` may be an arena slot view [B, L, H, D];
    with ``v_in`` / ``v_out`` (the arena's key-major V slots) the V append
    rides in the same launch."""
    _check_bf16(q_lin, k_lin)
    H, D = attn.heads, attn.dim_head
    q = torch.empty_like(q_lin)
    k = torch.empty_like(k_lin) if k_out is None else k_out
    kp = k_pe if k_pe is not None else pe
    gq = attn.q_norm.weight if attn.q_norm.weight is not None else None
    gk = attn.k_norm.weight if attn.k_norm.weight is not None else None
    _check_bf16(gq, gk)
    eq = attn.q_norm.eps if attn.q_norm.eps is not None else torch.finfo(q_lin.dtype).eps
    ek = attn.k_norm.eps if attn.k_norm.eps is not None else torch.finfo(k_lin.dtype).eps
    kernels.qk_rmsnorm_rope(q_lin, q, gq, eq, pe, H, D, k_lin, k, gk, ek, kp, v_in=v_in, v_out=v_out)
    return q, k


def _norm_one(norm: nn.RMSNorm, x_lin: torch.Tensor, pe, H: int, D: int) -> torch.Tensor:
    """rope(norm(x_lin)) for one side (the same per-row arithmetic as the q/k launch)."""
    g = norm.weight
    _check_bf16(x_lin, g)
    eps = norm.eps if norm.eps is not None else torch.finfo(x_lin.dtype).eps
    out = torch.empty_like(x_lin)
    kernels.qk_rmsnorm_rope(x_lin, out, g, eps, pe, H, D)
    return out


def _finish(attn: CausalLTXAttention, out: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """kv_cache.py:1680-1700: reshape, optional per-head gate 2*sigmoid(.), to_out."""
    B = x.shape[0]
    out = out.reshape(B, -1, attn.inner_dim)
    if attn.to_gate_logits is not None:
        g = attn.to_gate_logits(x)
        b, t, _ = out.shape
        out = (out.view(b, t, attn.heads, attn.dim_head) * (2.0 * torch.sigmoid(g)).unsqueeze(-1))
        out = out.view(b, t, attn.inner_dim)
    return attn.to_out(out)


def _key_padding_mask(mask: Optional[torch.Tensor], B: int, Lk: int) -> Optional[torch.Tensor]:
    """Reduce the reference's mask forms (flex_attention_utils.py:250-264) to the
    additive float32 [B or 1, Lk] key mask the kernel takes.  Masks that vary
    per query are not on the inference path."""
    if mask is None:
        return None
    m = mask
    if m.dtype == torch.bool:
        m = torch.zeros(m.shape, dtype=torch.float32, device=m.device).masked_fill_(~m, float("-inf"))
    if m.ndim == 4:
        if m.shape[1] != 1 or m.shape[2] != 1:
            raise NotImplementedError("only key-padding masks [B,1,1,Lk] are supported")
        m = m[:, 0, 0, :]
    elif m.ndim == 3:
        if m.shape[1] != 1:
            raise NotImplementedError("only key-padding masks [B,1,Lk] are supported")
        m = m[:, 0, :]
    elif m.ndim == 2:
        if m.shape[0] != 1 and m.shape[0] != B:
            raise NotImplementedError("2-D masks must be [1 or B, Lk] key-padding masks")
    else:
        raise NotImplementedError(f"mask of shape {tuple(mask.shape)}")
    if m.shape[-1] != Lk:
        raise ValueError(f"mask covers {m.shape[-1]} keys, attention has {Lk}")
    return m.to(torch.float32).contiguous()


# A key-padding mask whose kept keys are a prefix of each batch row, with
# every other key at or below -1e30 (the reference's (m - 1) * finfo.max form),
# gives those keys a weight of exactly 0 in float32: attending each row's
# prefix alone is the same computation.  A prefix common to every row is a
# shorter key range; prefixes of different lengths are per-row key counts for
# the pipelined kernel.  The check needs the mask's values on the host, so
# its result is kept per mask tensor (dropped when the tensor dies, recomputed
# after an in-place change) and a mask reused across blocks and steps costs
# one synchronisation.
_PREFIX: Dict[int, Tuple[int, Optional[Tuple[int, ...]]]] = {}


def _kept_prefixes(mask: torch.Tensor, km: torch.Tensor) -> Optional[Tuple[int, ...]]:
    """Per mask row, the length of the kept prefix, when every row keeps a
    non-empty prefix and drops the rest; else None."""
    key = id(mask)
    hit = _PREFIX.get(key)
    if hit is not None and hit[0] == mask._version:
        return hit[1]
    kept, dropped = km == 0, km <= -1e30
    n: Optional[Tuple[int, ...]] = None
    if bool((kept | dropped).all()):
        counts = kept.sum(dim=1)
        # a prefix: no kept key after the first dropped one
        first_drop = torch.where(dropped.any(dim=1), dropped.int().argmax(dim=1),
                                 torch.full_like(counts, km.shape[1]))
        if bool((counts == first_drop).all()) and bool((counts > 0).all()):
            n = tuple(int(c) for c in counts.tolist())
    if hit is None:
        weakref.finalize(mask, _PREFIX.pop, key, None)
    _PREFIX[key] = (mask._version, n)
    return n


def _key_major(v: torch.Tensor) -> torch.Tensor:
    """V [B, L, H, D] copied into a key-major store [B, H, D, L rounded up to 8]
    (zero tail), returned as its [B, L, H, D] view: the layout the pipelined
    kernel streams straight into LDS."""
    B, L, H, D = v.shape
    store = torch.empty(B, H, D, -(-L // 8) * 8, dtype=v.dtype, device=v.device)
    if store.shape[-1] > L:
        store[..., L:].zero_()
    view = store.permute(0, 3, 1, 2)[:, :L]
    kernels.kv_append(v, view)
    return view


def standard_attention_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               mask: Optional[torch.Tensor] = None,
                               scale: Optional[float] = None) -> torch.Tensor:
    """flex_attention_utils.py:225-276: [B, L, H, D] in, [B, L, H, D] out."""
    _check_bf16(q, k, v)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    B, Lq, H, D = q.shape
    qq = q if q.stride(3) == 1 else q.contiguous()
    kk = k if k.stride(3) == 1 else k.contiguous()
    # a V that is already a key-major view (the text K/V cache keeps V that
    # way) is attended as it is; a token-major V shares K's strides
    key_major = D in (64, 128) and v.stride(1) == 1 and v.stride(3) != 1
    vv = v
    if not key_major:
        vv = v if v.stride() == kk.stride() else v.contiguous()
        if kk.stride() != vv.stride():
            kk = kk.contiguous()
            vv = vv.contiguous()
    km = _key_padding_mask(mask, B, k.shape[1])
    key_lens = None
    if km is not None:
        lens = _kept_prefixes(mask, km)
        if lens is not None and len(set(lens)) == 1:
            n = lens[0]
            kk, vv, km = kk[:, :n], vv[:, :n], None
        elif lens is not None and B <= N.MAX_KEYLEN_BATCH and D in (64, 128) and Lq >= 256:
            # prefixes of different lengths: per-row key counts on the pipelined
            # kernel (with fewer queries the masked kernel, whatever V's layout,
            # so a cached key-major V gives the same result as a fresh one)
            key_lens, km = lens, None
            if not key_major:
                vv = _key_major(vv)
                key_major = True
    if km is not None and key_major:
        # the masked kernel reads token-major V with K's strides
        kk = kk.contiguous()
        vv = vv.contiguous()
    elif km is None and not key_major and D in (64, 128) and Lq >= 256 and kk.shape[1] >= 64:
        vv = _key_major(vv)
    kernels.flash_attn(qq, [KVSegment(kk, vv)], out, key_mask=km, scale=scale, key_lens=key_lens)
    return out


def _dense_segments(segs: List[KVSegment], new_k: torch.Tensor, new_v: torch.Tensor,
                    n_queries: int) -> List[KVSegment]:
    """Segments for a plain-tensor cache (the reference's torch.cat caches) plus
    the new chunk.  K is concatenated as the reference does (kv_cache.py:
    1487-1491) when the cache tensor's strides differ from the chunk's.  V goes
    into one key-major store instead of a token-major concatenation, the same
    bytes moved, so the attention runs on the pipelined kernel rather than the
    staged one (measured at 1152 queries over 3456 cached + 1152 new keys,
    B = 2, 32 x 128: 236 us staged, 180 us pipelined)."""
    if not segs:
        return [KVSegment(new_k, new_v)]
    old = segs[0]
    B, Lc, H, D = old.v.shape
    Ln = new_v.shape[1]
    same = old.k.stride() == new_k.stride()
    if D not in (64, 128) or n_queries < 256 or Lc + Ln < 64 or Lc % 8:
        if same and old.v.stride() == new_v.stride():
            return segs + [KVSegment(new_k, new_v)]
        return [KVSegment(torch.cat([old.k, new_k], dim=1), torch.cat([old.v, new_v], dim=1))]
    store = torch.empty(B, H, D, -(-(Lc + Ln) // 8) * 8, dtype=new_v.dtype, device=new_v.device)
    if store.shape[-1] > Lc + Ln:
        store[..., Lc + Ln:].zero_()
    vkm = store.permute(0, 3, 1, 2)
    kernels.kv_append(old.v, vkm[:, :Lc])
    kernels.kv_append(new_v, vkm[:, Lc:Lc + Ln])
    if same:
        return [KVSegment(old.k, vkm[:, :Lc]), KVSegment(new_k, vkm[:, Lc:Lc + Ln])]
    return [KVSegment(torch.cat([old.k, new_k], dim=1), vkm[:, :Lc + Ln])]


def _cached_segments(cached_k, cached_v) -> Tuple[List[KVSegment], int]:
    """Key segments of the cache (arena spans or one dense tensor) and the
    fp8 frame size (0 for bf16)."""
    if cached_k is None:
        return [], 0
    if isinstance(cached_k, KVSpanView):
        if not (isinstance(cached_v, KVSpanView) and cached_v.arena is cached_k.arena
                and cached_v.spans == cached_k.spans):
            raise ValueError("cached_k / cached_v must be views of one arena with equal spans")
        segs = []
        for (k, ks), (v, vs) in zip(cached_k.pieces(), cached_v.pieces()):
            segs.append(KVSegment(k, v, ks, vs))
        return segs, (cached_k.arena.frame_tokens if cached_k.arena.fp8 else 0)
    _check_bf16(cached_k, cached_v)
    return [KVSegment(cached_k, cached_v)], 0


def attention_with_cache(
    attn: CausalLTXAttention,
    x: torch.Tensor,
    context: Optional[torch.Tensor],
    pe: Optional[Tuple[torch.Tensor, torch.Tensor]],
    k_pe: Optional[Tuple[torch.Tensor, torch.Tensor]],
    cached_k,
    cached_v,
    logit_log_scale: Optional[torch.Tensor] = None,
    pyramid_policy=None,
    layer_idx: Optional[int] = None,
    modality: Optional[str] = None,
    frame_seqlen: Optional[int] = None,
    sp_context_sharded: bool = True,
    new_kv_real_len: Optional[int] = None,
    profile_name: Optional[str] = None,
):
    """kv_cache.py:1148-1547 (single-GPU synchronous branch).

    Returns ``(out [B, L, Dq], new_k, new_v)``.  When ``cached_k``/``cached_v``
    are arena views the new K/V are written into free arena slots and returned
    as views, so ``_cat_cache(cached_k, new_k)`` is free; otherwise they are
    dense [B, L_new, H, D] tensors as in the reference.  Keys attended are
    cached (in order) followed by the new chunk, with no mask: causality is
    what the cache holds (kv_cache.py:1525-1531).
    """
    if pyramid_policy is not None:
        raise NotImplementedError("PyramidKVPolicy is never constructed on the inference path")
    B, L, _ = x.shape
    ctx = x if context is None else context
    H, D = attn.heads, attn.dim_head
    q_lin, k_lin, v_lin = _project_qkv(attn, x, ctx)
    _check_bf16(q_lin, k_lin, v_lin)
    Lk_new = k_lin.shape[1]
    real = Lk_new if new_kv_real_len is None else min(int(new_kv_real_len), Lk_new)
    k_lin = k_lin[:, :real]
    v_lin = v_lin[:, :real]

    arena = cached_k.arena if isinstance(cached_k, KVSpanView) else None
    if cached_k is None and cached_v is None:
        # an empty field of the reference's init_kv_cache(): a module with an
        # arena plan starts its cache in that arena (None: dense tensors)
        arena = module_arena(attn, B, x.device)
    segs, frame = _cached_segments(cached_k, cached_v)
    if arena is not None and arena.fp8:
        frame = arena.frame_tokens
    if arena is not None and not arena.fp8:
        slot = arena.alloc(real)
        k_dst = arena.slots("k", slot, real)
        q, _ = _norm_rope(attn, q_lin, k_lin, pe, k_pe, k_dst, v_lin.view(B, real, H, D),
                          arena.slots("v", slot, real))
        new_k = KVSpanView(arena, "k", [(slot, real)])
        new_v = KVSpanView(arena, "v", [(slot, real)])
        segs.append(KVSegment(k_dst, arena.slots("v", slot, real)))
    elif arena is not None:
        # fp8 arena: the new chunk is quantised into its slots and attended in fp8
        q, k = _norm_rope(attn, q_lin, k_lin, pe, k_pe, None)
        slot = arena.alloc(real)
        kd, vd = arena.slots("k", slot, real), arena.slots("v", slot, real)
        ks, vs = arena.scale_slots("k", slot, real), arena.scale_slots("v", slot, real)
        kernels.kv_append_fp8_pair(k.view(B, real, H, D), kd, ks, v_lin.view(B, real, H, D), vd, vs,
                                   arena.frame_tokens)
        new_k = KVSpanView(arena, "k", [(slot, real)])
        new_v = KVSpanView(arena, "v", [(slot, real)])
        segs.append(KVSegment(kd, vd, ks, vs))
    else:
        q, k = _norm_rope(attn, q_lin, k_lin, pe, k_pe, None)
        new_k = k.view(B, real, H, D)
        new_v = v_lin.view(B, real, H, D)
        if not new_v.is_contiguous() or (segs and segs[0].k.stride() != new_k.stride()):
            new_v = new_v.contiguous()
            new_k = new_k.contiguous()
        segs = _dense_segments(segs, new_k, new_v, L)
    if logit_log_scale is not None:
        q = q * logit_log_scale
    out = torch.empty(B, L, H, D, dtype=q.dtype, device=q.device)
    kernels.flash_attn(q.view(B, L, H, D), segs, out, frame_tokens=frame)
    return _finish(attn, out, x), new_k, new_v
