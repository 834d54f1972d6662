"""Arena-backed KV cache with the reference's LayerKVCache / KVCache surface.

Reference: ltx_causal/transformer/kv_cache.py:321-358 (LayerKVCache, KVCache),
:394-398 (_cat_cache), ltx_causal/wrapper.py:15-20 (init_kv_cache).

The reference stores each cache field as a [B, L, H, D] tensor, appends with
``torch.cat`` (a full reallocation and copy per commit) and evicts by slicing and
re-concatenating.  Here every (layer, attention kind) owns one preallocated
``KVArena`` on the device holding K and V side by side, and a cache field is a
``KVSpanView``: the ordered list of arena slot spans that make up its logical
[B, L, H, D] sequence.

* Append writes only the new tokens into free slots (the fused norm/RoPE kernel
  writes K there directly).  ``_cat_cache`` of two views of one arena is span
  concatenation: no bytes move.
* Eviction slices spans (index-only).  ``retain_streaming_context`` therefore
  moves zero bytes; ``KVSpanView.materialize`` compacts on demand.
* Views are immutable and the functional semantics of the reference are kept:
  a slot is never handed out while any live view (a snapshot, a retained
  cache, a denoise-step cache) still covers it.  Liveness is tracked with
  weak references, so dropping the last reference to a view -- e.g. restoring
  the pre-block snapshot before the next denoise step -- frees its slots.
* bf16 arenas keep K token-major [B, slots, H, D] and V key-major
  [B, H, D, slots] (the attention kernel loads V^T tiles straight into LDS);
  appends start on 8-slot boundaries.
* fp8-e4m3 arenas store codes plus one float32 scale per (batch, head, frame)
  of ``frame_tokens`` slots (both token-major); spans are frame aligned.
"""
from __future__ import annotations

import itertools
import weakref
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from . import kernels

Span = Tuple[int, int]  # (slot start, length)


class KVArenaFull(RuntimeError):
    """No free slot range is large enough for an append."""


def _merge(spans: Sequence[Span]) -> Tuple[Span, ...]:
    out: List[List[int]] = []
    for s, n in spans:
        s, n = int(s), int(n)
        if n <= 0:
            continue
        if out and out[-1][0] + out[-1][1] == s:
            out[-1][1] += n
        else:
            out.append([s, n])
    return tuple((s, n) for s, n in out)


class KVArena:
    """Device storage for one K/V pair: k, v [B, capacity, H, D]."""

    def __init__(self, batch: int, capacity: int, heads: int, dim_head: int,
                 device="cuda", kv_dtype: str = "bf16", frame_tokens: int = 1,
                 name: str = ""):
        if kv_dtype not in ("bf16", "fp8"):
            raise ValueError(f"kv_dtype must be 'bf16' or 'fp8', got {kv_dtype!r}")
        self.B, self.H, self.D = int(batch), int(heads), int(dim_head)
        # whole 8-slot groups: key-major V is read in 8-token chunks
        self.cap = -(-int(capacity) // 8) * 8
        self.kv_dtype = kv_dtype
        self.fp8 = kv_dtype == "fp8"
        self.frame_tokens = int(frame_tokens) if self.fp8 else 1
        if self.fp8 and int(capacity) % self.frame_tokens:
            raise ValueError("fp8 arena capacity must be a whole number of frames")
        self.name = name
        self.device = torch.device(device)
        store = torch.uint8 if self.fp8 else torch.bfloat16
        self.k = torch.empty(self.B, self.cap, self.H, self.D, dtype=store, device=self.device)
        if self.fp8:
            self.v = torch.empty_like(self.k)
        else:
            # bf16 V is stored key-major, [B, H, D, slots]: the attention kernel
            # streams V^T tiles straight into LDS; self.v is its [B, slots, H, D]
            # view.  Zero-filled: the kernel reads a span's last 8-slot group
            # whole, so never-written slots must hold finite values.
            self.v_store = torch.zeros(self.B, self.H, self.D, self.cap, dtype=store, device=self.device)
            self.v = self.v_store.permute(0, 3, 1, 2)
        if self.fp8:
            nf = self.cap // self.frame_tokens
            self.k_scales = torch.ones(self.B, self.H, nf, dtype=torch.float32, device=self.device)
            self.v_scales = torch.ones_like(self.k_scales)
        else:
            self.k_scales = self.v_scales = None
        self._live: Dict[int, Tuple[Span, ...]] = {}
        self._ids = itertools.count()

    # ---- liveness ----
    def _register(self, spans: Tuple[Span, ...]) -> int:
        key = next(self._ids)
        self._live[key] = spans
        return key

    def _release(self, key: int) -> None:
        self._live.pop(key, None)

    def live_intervals(self) -> List[Span]:
        iv = sorted((s, s + n) for spans in self._live.values() for s, n in spans)
        out: List[List[int]] = []
        for a, b in iv:
            if out and a <= out[-1][1]:
                out[-1][1] = max(out[-1][1], b)
            else:
                out.append([a, b])
        return [(a, b) for a, b in out]

    @property
    def align(self) -> int:
        """Slot alignment of appends: whole frames for fp8 (one scale per frame),
        8 slots for bf16 (16-byte rows of the key-major V store)."""
        return self.frame_tokens if self.fp8 else 8

    def alloc(self, n: int) -> int:
        """First free slot range of n tokens (aligned to ``align``) not covered
        by any live view."""
        n = int(n)
        al = self.align
        if self.fp8 and n % al:
            raise ValueError(f"append of {n} tokens is not a whole number of {al}-token frames")
        pos = 0
        for a, b in self.live_intervals() + [(self.cap, self.cap)]:
            start = -(-pos // al) * al
            if start + n <= a:
                return start
            pos = max(pos, b)
        raise KVArenaFull(
            f"KV arena {self.name or ''} full: {n} tokens requested, capacity {self.cap}, "
            f"live {self.live_intervals()}")

    # ---- views ----
    def empty_view(self, which: str) -> "KVSpanView":
        return KVSpanView(self, which, ())

    def slots(self, which: str, start: int, n: int) -> torch.Tensor:
        store = self.k if which == "k" else self.v
        return store[:, start:start + n]

    def scale_slots(self, which: str, start: int, n: int) -> Optional[torch.Tensor]:
        if not self.fp8:
            return None
        sc = self.k_scales if which == "k" else self.v_scales
        f0 = start // self.frame_tokens
        return sc[:, :, f0:f0 + -(-n // self.frame_tokens)]


class KVSpanView:
    """Logical [B, L, H, D] cache tensor = concatenation of arena slot spans.

    Supports what the reference's cache code does with its tensors: ``.shape``,
    ``.size()``, ``[:, a:b]`` slicing (index-only), ``_cat_cache`` (span
    concatenation) and ``materialize()`` for a dense copy.
    """
    __slots__ = ("arena", "which", "spans", "_key", "__weakref__")

    def __init__(self, arena: KVArena, which: str, spans: Sequence[Span]):
        if which not in ("k", "v"):
            raise ValueError("which must be 'k' or 'v'")
        self.arena = arena
        self.which = which
        self.spans = _merge(spans)
        self._key = arena._register(self.spans)
        weakref.finalize(self, arena._release, self._key)

    # tensor-like metadata
    @property
    def shape(self) -> torch.Size:
        a = self.arena
        return torch.Size((a.B, sum(n for _, n in self.spans), a.H, a.D))

    def size(self, dim: Optional[int] = None):
        return self.shape if dim is None else self.shape[dim]

    @property
    def ndim(self) -> int:
        return 4

    def dim(self) -> int:
        return 4

    @property
    def dtype(self) -> torch.dtype:
        return torch.bfloat16

    @property
    def device(self) -> torch.device:
        return self.arena.device

    def __len__(self) -> int:
        return self.arena.B

    def __repr__(self) -> str:
        return (f"KVSpanView({self.which}, shape={tuple(self.shape)}, spans={list(self.spans)}, "
                f"kv_dtype={self.arena.kv_dtype})")

    def __getitem__(self, idx):
        if not (isinstance(idx, tuple) and len(idx) == 2 and idx[0] == slice(None)
                and isinstance(idx[1], slice) and idx[1].step in (None, 1)):
            raise TypeError("KVSpanView supports [:, start:end] slicing only; materialize() for more")
        L = self.shape[1]
        a, b, _ = idx[1].indices(L)
        return KVSpanView(self.arena, self.which, self._subspans(a, max(a, b)))

    def _subspans(self, a: int, b: int) -> List[Span]:
        out, pos = [], 0
        for s, n in self.spans:
            lo, hi = max(a, pos), min(b, pos + n)
            if lo < hi:
                out.append((s + lo - pos, hi - lo))
            pos += n
        return out

    # kernel-facing pieces
    def pieces(self) -> List[Tuple[torch.Tensor, Optional[torch.Tensor]]]:
        """(slot tensor [B, n, H, D], scales [B, H, nF] or None) per span."""
        a = self.arena
        return [(a.slots(self.which, s, n), a.scale_slots(self.which, s, n)) for s, n in self.spans]

    def materialize(self) -> torch.Tensor:
        """Dense contiguous bf16 copy [B, L, H, D] (ltx_kv_gather; fp8 is dequantised)."""
        a = self.arena
        B, L, H, D = self.shape
        store = a.k if self.which == "k" else a.v
        if self.which == "v" and not a.fp8:
            # key-major V store: slice the spans of the [B, slots, H, D] view
            if not L:
                return torch.empty(B, 0, H, D, dtype=torch.bfloat16, device=a.device)
            return torch.cat([store[:, s:s + n] for s, n in self.spans], dim=1).contiguous()
        dense = torch.empty(B, L, H, D, dtype=store.dtype, device=a.device)
        if L:
            kernels.kv_gather(store, dense, list(self.spans))
        if not a.fp8:
            return dense
        # fp8: gather scales per span and expand per token (interop path, not the hot loop)
        sc = torch.cat([p[1] for p in self.pieces()], dim=2) if L else None
        vals = dense.view(torch.float8_e4m3fn).to(torch.float32)
        per_tok = sc.repeat_interleave(a.frame_tokens, dim=2)[:, :, :L].permute(0, 2, 1)
        return (vals * per_tok.unsqueeze(-1)).to(torch.bfloat16)


def _is_view(x: Any) -> bool:
    return isinstance(x, KVSpanView)


def _dense(x):
    return x.materialize() if _is_view(x) else x


def _cat_cache(old, new):
    """kv_cache.py:394-398.  Views of one arena concatenate their spans (no copy);
    plain tensors concatenate like the reference; mixed inputs are densified."""
    if old is None:
        return new
    if _is_view(old) and _is_view(new) and old.arena is new.arena and old.which == new.which:
        return KVSpanView(old.arena, old.which, old.spans + new.spans)
    return torch.cat([_dense(old), _dense(new)], dim=1)


@dataclass
class LayerKVCache:
    """kv_cache.py:321-351: per-layer cache for the four cached attention kinds.

    Fields hold ``KVSpanView`` (arena-backed), plain [B, L, H, D] tensors, or None.
    """
    video_self_k: Optional[Any] = None
    video_self_v: Optional[Any] = None
    audio_self_k: Optional[Any] = None
    audio_self_v: Optional[Any] = None
    a2v_k: Optional[Any] = None
    a2v_v: Optional[Any] = None
    v2a_k: Optional[Any] = None
    v2a_v: Optional[Any] = None


@dataclass
class KVCache:
    """kv_cache.py:354-358 plus the segment metadata the runtime attaches
    (taomate/inference/cache.py:7-12, streaming_runtime.py ``_interactive_segments``)."""
    layers: List[LayerKVCache] = field(default_factory=list)
    layerwise_cpu_offload: bool = False
    segments: List[Dict[str, Any]] = field(default_factory=list)


@dataclass(frozen=True)
class ArenaSpec:
    """Capacity and head layout of one attention kind's arena."""
    capacity: int
    heads: int
    dim_head: int
    kv_dtype: str = "bf16"
    frame_tokens: int = 1


KIND_FIELDS = {
    "video_self": ("video_self_k", "video_self_v"),
    "audio_self": ("audio_self_k", "audio_self_v"),
    "a2v": ("a2v_k", "a2v_v"),
    "v2a": ("v2a_k", "v2a_v"),
}


def init_kv_cache(num_layers: int, batch: int, specs: Dict[str, ArenaSpec],
                  device="cuda") -> KVCache:
    """wrapper.py:15-20 with preallocated arenas: each layer gets one arena per
    attention kind in ``specs`` and starts with empty views of it; kinds not in
    ``specs`` stay None (plain-tensor behaviour)."""
    layers = []
    for li in range(num_layers):
        kw = {}
        for kind, spec in specs.items():
            if kind not in KIND_FIELDS:
                raise ValueError(f"unknown cache kind {kind!r}")
            arena = KVArena(batch, spec.capacity, spec.heads, spec.dim_head, device,
                            spec.kv_dtype, spec.frame_tokens, name=f"layer{li}.{kind}")
            fk, fv = KIND_FIELDS[kind]
            kw[fk] = arena.empty_view("k")
            kw[fv] = arena.empty_view("v")
        layers.append(LayerKVCache(**kw))
    return KVCache(layers=layers)


# ---------------------------------------------------------------------------
# Arenas attached to attention modules.
#
# The reference starts every stream from ``init_kv_cache()`` with no
# arguments (wrapper.py:15-20): each LayerKVCache field is None until the
# first append.  An attention module that carries an arena plan gets its own
# KVArena, created on its first call (the batch and device come from that
# call), so the first append of a None field already lands in arena slots and
# every later cache of that field is a KVSpanView of it.
# ---------------------------------------------------------------------------

def attach_arena(attn, capacity: int, kv_dtype: str = "bf16", frame_tokens: int = 1, name: str = "") -> None:
    """Give ``attn`` (any module with ``heads`` / ``dim_head``) an arena plan of
    ``capacity`` tokens; the arena itself is allocated on first use."""
    if kv_dtype not in ("bf16", "fp8"):
        raise ValueError(f"kv_dtype must be 'bf16' or 'fp8', got {kv_dtype!r}")
    attn.__dict__["_ltx_arena_plan"] = ArenaSpec(int(capacity), int(attn.heads), int(attn.dim_head), kv_dtype,
                                                 int(frame_tokens))
    attn.__dict__["_ltx_arena_name"] = name
    attn.__dict__.pop("_ltx_arena", None)


def detach_arena(attn) -> None:
    for k in ("_ltx_arena_plan", "_ltx_arena_name", "_ltx_arena"):
        attn.__dict__.pop(k, None)


def module_arena(attn, batch: int, device) -> Optional[KVArena]:
    """The arena of ``attn`` for this batch and device (created on first use,
    replaced when either changes; views of the old arena keep it alive), or
    None when ``attn`` carries no plan."""
    spec = attn.__dict__.get("_ltx_arena_plan")
    if spec is None:
        return None
    dev = torch.device(device)
    arena = attn.__dict__.get("_ltx_arena")
    if arena is None or arena.B != int(batch) or arena.device != dev:
        arena = KVArena(batch, spec.capacity, spec.heads, spec.dim_head, dev, spec.kv_dtype, spec.frame_tokens,
                        name=attn.__dict__.get("_ltx_arena_name", ""))
        attn.__dict__["_ltx_arena"] = arena
    return arena


# attention module of each cached kind in a dual-stream block
# (causal_block.py:260-376): its keys/values come from the stream named
BLOCK_CACHE_MODULES = {
    "video_self": ("attn1", "video"),
    "audio_self": ("audio_attn1", "audio"),
    "a2v": ("audio_to_video_attn", "audio"),
    "v2a": ("video_to_audio_attn", "video"),
}


def attach_block_arenas(blocks, video_tokens: int, audio_tokens: int, kv_dtype: str = "bf16",
                        video_frame_tokens: int = 1) -> None:
    """Arena plans for the four cached attentions of every block: video-keyed
    kinds (video_self, v2a) hold ``video_tokens``, audio-keyed kinds
    (audio_self, a2v) ``audio_tokens``.  ``kv_dtype`` "fp8" applies to the
    video-keyed kinds (frame-aligned appends of ``video_frame_tokens``); the
    audio kinds stay bf16 (audio latent frames are single tokens)."""
    for i, blk in enumerate(blocks):
        for kind, (attr, stream) in BLOCK_CACHE_MODULES.items():
            attn = getattr(blk, attr, None)
            if attn is None:
                continue
            if stream == "video":
                attach_arena(attn, video_tokens, kv_dtype, video_frame_tokens if kv_dtype == "fp8" else 1,
                             name=f"layer{i}.{kind}")
            else:
                attach_arena(attn, audio_tokens, "bf16", 1, name=f"layer{i}.{kind}")


def empty_kv_cache(num_layers: int) -> KVCache:
    """The reference's empty cache (wrapper.py:15-20): one LayerKVCache with
    every field None per layer."""
    return KVCache(layers=[LayerKVCache() for _ in range(int(num_layers))])
