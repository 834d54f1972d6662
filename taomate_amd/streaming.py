"""The anchor | memory | window | current chunk stream of one attention layer.

Host mirror of the window loop of ``generate_next_window``
(taomate/inference/model.py:166-248): each chunk attends over what the cache
holds plus itself (kv_cache.py:1525-1531), its keys and values are committed
into the cache (``_cat_cache``, kv_cache.py:394-398) with a segment record
(streaming_runtime.py:354-387), and eviction slices the cache by segments
(``_prune_clean_kv_to_sink_recent``, streaming_runtime.py:612-662).

The layout widens the reference's sink-plus-recent policy:

* anchor -- the first ``anchor_frames`` latent frames, kind "prefix", pinned;
* memory -- ``memory_frames`` frames at fixed positions right after the anchor,
  kind "memory", pinned, and re-prefilled every ``refresh_every`` chunks from
  an evolving state at those original positions (the re-prefill of retained
  segments at their global positions, taomate/inference/runtime.py:386-470).
  The state evolves by the reference's memory rule, an EMA with an identity
  tether (_ema_update, taomate/runtime_support/learned_memory.py:231-249):
  state <- ((1 - beta) state + beta new) (1 - tether) + tether anchor, where
  new is the newest chunk's last memory frames, anchor the state the stream
  started from, and beta / tether the streaming settings 0.15 / 0.20
  (video_beta, video_anchor_tether, taomate/inference/memory.py:4-29);
* window -- the newest generated chunks whose frames fit in ``window_frames``;
* current -- the chunk being generated (``chunk_frames`` frames).

All K/V live in one preallocated arena (bf16 or fp8-e4m3 with per-(head,
frame) scales); commit writes only the chunk's tokens, eviction and the memory
swap are span edits that move no bytes.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Dict, List, Optional, Tuple

import torch

from . import kernels
from .attention import CausalLTXAttention, _check_bf16, attention_with_cache, packed_qkv
from .cache import _segment_offsets, _slice_tensor
from .kv_cache import KVArena, KVSpanView, _cat_cache
from .rope import causal_precompute_freqs_cis

PINNED_KINDS = ("prefix", "memory")


def retain_pinned_recent(segments: List[Dict], recent_blocks: int, pinned_kinds=PINNED_KINDS) -> List[int]:
    """Indices of the segments kept: every pinned segment and the newest
    ``recent_blocks`` others, in list (chronological) order."""
    pinned = [i for i, s in enumerate(segments) if s.get("kind") in pinned_kinds]
    others = [i for i in range(len(segments)) if i not in pinned]
    recent = others[-recent_blocks:] if recent_blocks > 0 else []
    return sorted(set(pinned + recent))


def prefill_kv(attn: CausalLTXAttention, x: torch.Tensor, pe, arena: KVArena) -> Tuple[KVSpanView, KVSpanView]:
    """K and V of ``x`` written into fresh arena slots (projection, full-row k
    RMSNorm, SPLIT RoPE at the positions of ``pe``): the cache-only prefill of
    a segment, with no attention output."""
    B, L, _ = x.shape
    H, D = attn.heads, attn.dim_head
    packed = packed_qkv(attn)
    if packed is None:
        k_lin, v_lin = attn.to_k(x), attn.to_v(x)
    else:   # the K and V rows of a packed q/k/v weight (fuse_qkv_): one GEMM
        n = attn.inner_dim
        kv = torch.nn.functional.linear(x, packed[0][n:], packed[1][n:])
        k_lin, v_lin = kv[..., :n], kv[..., n:]
    _check_bf16(k_lin, v_lin)
    gk = attn.k_norm.weight
    ek = attn.k_norm.eps if attn.k_norm.eps is not None else torch.finfo(k_lin.dtype).eps
    slot = arena.alloc(L)
    kd, vd = arena.slots("k", slot, L), arena.slots("v", slot, L)
    if arena.fp8:
        k = torch.empty_like(k_lin)
        kernels.qk_rmsnorm_rope(k_lin, k, gk, ek, pe, H, D)
        kernels.kv_append_fp8_pair(k.view(B, L, H, D), kd, arena.scale_slots("k", slot, L), v_lin.view(B, L, H, D),
                                   vd, arena.scale_slots("v", slot, L), arena.frame_tokens)
    else:
        kernels.qk_rmsnorm_rope(k_lin, kd, gk, ek, pe, H, D, v_in=v_lin.view(B, L, H, D), v_out=vd)
    return KVSpanView(arena, "k", [(slot, L)]), KVSpanView(arena, "v", [(slot, L)])


class ChunkStream:
    """One layer's anchor | memory | window | current stream on the device."""

    def __init__(self, attn: CausalLTXAttention, video_hw: Tuple[int, int], batch: int, device="cuda",
                 anchor_frames: int = 1, memory_frames: int = 2, chunk_frames: int = 3,
                 window_frames: int = 12, refresh_every: int = 4, kv_dtype: str = "fp8",
                 theta: float = 10000.0, memory_beta: float = 0.15, memory_tether: float = 0.20):
        if window_frames % chunk_frames:
            raise ValueError("window_frames must be a whole number of chunks")
        self.attn = attn
        self.hw = int(video_hw[0]) * int(video_hw[1])
        self.grid = (int(video_hw[0]), int(video_hw[1]))
        self.B = int(batch)
        self.device = torch.device(device)
        self.anchor_frames, self.memory_frames = int(anchor_frames), int(memory_frames)
        self.chunk_frames, self.window_frames = int(chunk_frames), int(window_frames)
        self.recent = self.window_frames // self.chunk_frames
        self.refresh_every = int(refresh_every)
        self.theta = float(theta)
        self.memory_beta = min(max(float(memory_beta), 0.0), 1.0)
        self.memory_tether = min(max(float(memory_tether), 0.0), 1.0)
        # live at most: anchor + two memory versions (during a swap) + window
        # + the chunk being committed and the next; one chunk of slack for
        # first-fit fragmentation
        frames = self.anchor_frames + 2 * self.memory_frames + self.window_frames + 3 * self.chunk_frames
        self.arena = KVArena(self.B, frames * self.hw, attn.heads, attn.dim_head, self.device, kv_dtype,
                             frame_tokens=self.hw, name="stream")
        self.k: KVSpanView = self.arena.empty_view("k")
        self.v: KVSpanView = self.arena.empty_view("v")
        self.segments: List[Dict] = []
        self.memory_state: Optional[torch.Tensor] = None
        self.memory_anchor: Optional[torch.Tensor] = None
        self.memory_version = 0
        self.chunks_done = 0
        self._pe_cache: "OrderedDict[Tuple[int, int], tuple]" = OrderedDict()

    # ---- positions ----
    def chunk_start_frame(self, c: int) -> int:
        return self.anchor_frames + self.memory_frames + c * self.chunk_frames

    def _pe(self, f0: int, nf: int):
        key = (f0, nf)
        hit = self._pe_cache.get(key)
        if hit is None:
            hit = causal_precompute_freqs_cis(torch.tensor([[nf, *self.grid]] * self.B), self.attn.inner_dim,
                                              theta=self.theta, start_frame=f0, device=self.device,
                                              dtype=torch.bfloat16, num_attention_heads=self.attn.heads)
            self._pe_cache[key] = hit
            while len(self._pe_cache) > 8:
                self._pe_cache.popitem(last=False)
        return hit

    def _segment(self, kind: str, block_idx: int, frames: int, window_slot: Optional[int] = None) -> Dict:
        seg = {"kind": kind, "block_idx": int(block_idx), "video_tokens": int(frames * self.hw), "audio_tokens": 0}
        if window_slot is not None:
            seg["window_slot"] = int(window_slot)
        return seg

    # ---- device work ----
    def _prefill_segment(self, x: torch.Tensor, f0: int, nf: int) -> Tuple[KVSpanView, KVSpanView]:
        """K/V of ``nf`` frames of hidden states at absolute frames f0.. in new
        arena slots."""
        return prefill_kv(self.attn, x, self._pe(f0, nf), self.arena)

    def _attend(self, x: torch.Tensor, f0: int, nf: int):
        """The chunk at frames f0.. over the cache plus itself: (out, new k, new v)."""
        return attention_with_cache(self.attn, x, None, self._pe(f0, nf), None, self.k, self.v)

    # ---- cache edits (span-only) ----
    def _keep(self, indices: List[int]) -> None:
        offs = _segment_offsets(self.segments)
        spans = [(offs[i][0], offs[i][1]) for i in indices]
        self.k = _slice_tensor(self.k, spans)
        self.v = _slice_tensor(self.v, spans)
        self.segments = [dict(self.segments[i]) for i in indices]

    def prefill(self, x_anchor: torch.Tensor, x_memory: Optional[torch.Tensor]) -> None:
        """Cache-only prefill of the anchor (frames 0..) and the memory (the
        frames after it); ``x_memory`` also seeds the evolving memory state."""
        if self.segments:
            raise RuntimeError("prefill of a stream that already holds segments")
        self.k, self.v = self._prefill_segment(x_anchor, 0, self.anchor_frames)
        self.segments = [self._segment("prefix", 0, self.anchor_frames)]
        if self.memory_frames:
            if x_memory is None:
                raise ValueError("memory frames configured but no memory hidden states given")
            self.memory_state = x_memory.float().clone()
            self.memory_anchor = self.memory_state.clone()
            km, vm = self._prefill_segment(x_memory, self.anchor_frames, self.memory_frames)
            self.k, self.v = _cat_cache(self.k, km), _cat_cache(self.v, vm)
            self.segments.append(self._segment("memory", 1, self.memory_frames))

    def refresh_memory(self, x_recent: torch.Tensor) -> None:
        """Evolve the fp32 memory state with the last memory_frames frames of
        ``x_recent`` (EMA, then the tether to the starting state), re-prefill
        it at the memory's own positions and swap it into the cache in place."""
        n = self.memory_frames * self.hw
        tail = x_recent[:, -n:]
        # (1 - t) ((1 - b) m + b x) + t a in place, three float32 passes
        # (the bf16 frames are widened inside the add) instead of seven
        b, t = self.memory_beta, self.memory_tether if self.memory_tether > 0.0 else 0.0
        ema = self.memory_state.mul_((1.0 - b) * (1.0 - t)).add_(tail, alpha=b * (1.0 - t))
        if t > 0.0:
            ema.add_(self.memory_anchor, alpha=t)
        self.memory_state = ema
        km, vm = self._prefill_segment(self.memory_state.to(x_recent.dtype), self.anchor_frames,
                                       self.memory_frames)
        mi = next(i for i, s in enumerate(self.segments) if s["kind"] == "memory")
        offs = _segment_offsets(self.segments)
        before = [(offs[i][0], offs[i][1]) for i in range(mi)]
        after = [(offs[i][0], offs[i][1]) for i in range(mi + 1, len(self.segments))]
        def join(*parts):
            out = None
            for part in parts:
                if part is not None:
                    out = _cat_cache(out, part)
            return out
        k = join(_slice_tensor(self.k, before), km, _slice_tensor(self.k, after))
        v = join(_slice_tensor(self.v, before), vm, _slice_tensor(self.v, after))
        self.k, self.v = k, v
        self.memory_version += 1

    def step(self, x_chunk: torch.Tensor) -> torch.Tensor:
        """Attend the chunk over anchor | memory | window plus itself, commit
        its K/V, evict, and re-prefill the memory when due.  Returns the
        layer output [B, chunk tokens, d]."""
        c = self.chunks_done
        out, nk, nv = self._attend(x_chunk, self.chunk_start_frame(c), self.chunk_frames)
        self.k, self.v = _cat_cache(self.k, nk), _cat_cache(self.v, nv)
        del nk, nv
        self.segments.append(self._segment("generated", c + 2, self.chunk_frames, window_slot=c))
        keep = retain_pinned_recent(self.segments, self.recent)
        if keep != list(range(len(self.segments))):
            self._keep(keep)
        if self.memory_frames and self.refresh_every > 0 and (c + 1) % self.refresh_every == 0:
            self.refresh_memory(x_chunk)
        self.chunks_done += 1
        return out

    def cache_frames(self) -> List[Tuple[str, int, int]]:
        """(kind, first frame, frames) of every cached segment, in cache order."""
        out = []
        for s in self.segments:
            nf = s["video_tokens"] // self.hw
            if s["kind"] == "prefix":
                f0 = 0
            elif s["kind"] == "memory":
                f0 = self.anchor_frames
            else:
                f0 = self.chunk_start_frame(s["window_slot"])
            out.append((s["kind"], f0, nf))
        return out
