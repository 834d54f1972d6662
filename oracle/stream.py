"""fp32 restatement of the anchor | memory | window | current stream (oracle;
test infrastructure only).

One attention layer over dense [B, L, H, D] caches, with the reference's own
operations: attention_with_cache (ltx_causal/transformer/kv_cache.py:1148-1547)
for every chunk, torch.cat commit (_cat_cache, kv_cache.py:394-398), segment
slicing for eviction (taomate/inference/cache.py:28-56) with the pinned
{anchor, memory} + newest-window policy of ``cache.retain_pinned_recent``,
and the memory re-prefilled at its own positions every ``refresh_every``
chunks (runtime.py:386-470) from a state evolved by the reference's memory
rule, _ema_update (taomate/runtime_support/learned_memory.py:231-249):
``ema = state (1 - beta) + new beta``, then ``ema (1 - tether) + anchor tether``,
with ``new`` the chunk's last memory frames, ``anchor`` the starting state and
the streaming settings beta 0.15, tether 0.20 (taomate/inference/memory.py:4-29).
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence, Tuple

import torch

from . import attention as OA
from . import cache as OC
from . import rope as OR


def _pe(grid_hw, nf: int, dim: int, heads: int, start: int, batch: int):
    return OR.causal_precompute_freqs_cis((nf, grid_hw[0], grid_hw[1]), dim, start_frame=start,
                                          num_attention_heads=heads, batch=batch)


def _kv_only(w: OA.AttnWeights, x: torch.Tensor, pe) -> Tuple[torch.Tensor, torch.Tensor]:
    """K/V of a cache-only prefill (the attention output is not needed)."""
    _, new_k, new_v = OA.attention_with_cache(w, x, None, pe, None, None, None)
    return new_k, new_v


def ema_update(prev: torch.Tensor, anchor: Optional[torch.Tensor], current: torch.Tensor, beta: float,
               tether: float) -> torch.Tensor:
    """learned_memory.py:231-249 (with a previous state): EMA, then the tether."""
    beta, tether = min(max(beta, 0.0), 1.0), min(max(tether, 0.0), 1.0)
    ema = prev * (1.0 - beta) + current * beta
    if anchor is not None and tether > 0.0:
        ema = ema * (1.0 - tether) + anchor * tether
    return ema


def run_stream(w: OA.AttnWeights, grid_hw: Tuple[int, int], x_anchor: torch.Tensor,
               x_memory: Optional[torch.Tensor], chunks: Sequence[torch.Tensor], anchor_frames: int = 1,
               memory_frames: int = 2, chunk_frames: int = 3, window_frames: int = 12, refresh_every: int = 4,
               memory_beta: float = 0.15, memory_tether: float = 0.20,
               outputs_for: Optional[Callable[[int], bool]] = None):
    """Layer outputs of every chunk in order, and the final K/V caches with
    their segment list: ``(outs, k, v, segments)``.  ``outputs_for(c)`` False
    skips chunk c's output (its K/V are still computed and committed); its
    entry in ``outs`` is None."""
    B = x_anchor.shape[0]
    hw = grid_hw[0] * grid_hw[1]
    dim, heads = w.heads * w.dim_head, w.heads
    recent = window_frames // chunk_frames
    anchor, memory, chunk_seg = OC.stream_segments_layout(grid_hw, anchor_frames, memory_frames, chunk_frames)
    ck, cv = _kv_only(w, x_anchor, _pe(grid_hw, anchor_frames, dim, heads, 0, B))
    segments = [dict(anchor)]
    state = None
    mem_pe = _pe(grid_hw, memory_frames, dim, heads, anchor_frames, B) if memory_frames else None
    if memory_frames:
        state = x_memory.clone()
        start = state.clone()
        mk, mv = _kv_only(w, state, mem_pe)
        ck, cv = OC.cat_cache(ck, mk), OC.cat_cache(cv, mv)
        segments.append(dict(memory))
    outs = []
    for c, x in enumerate(chunks):
        f0 = OC.chunk_start_frame(c, anchor_frames, memory_frames, chunk_frames)
        pe = _pe(grid_hw, chunk_frames, dim, heads, f0, B)
        if outputs_for is None or outputs_for(c):
            out, nk, nv = OA.attention_with_cache(w, x, None, pe, None, ck, cv)
        else:
            out, (nk, nv) = None, _kv_only(w, x, pe)
        outs.append(out)
        ck, cv = OC.cat_cache(ck, nk), OC.cat_cache(cv, nv)
        segments.append(chunk_seg(c))
        keep = OC.retain_pinned_recent(segments, recent)
        if keep != list(range(len(segments))):
            offs = OC.segment_offsets(segments)
            spans = [(offs[i][0], offs[i][1]) for i in keep]
            ck, cv = OC.slice_tensor(ck, spans), OC.slice_tensor(cv, spans)
            segments = [dict(segments[i]) for i in keep]
        if memory_frames and refresh_every > 0 and (c + 1) % refresh_every == 0:
            state = ema_update(state, start, x[:, -memory_frames * hw:], memory_beta, memory_tether)
            mk, mv = _kv_only(w, state, mem_pe)
            mi = next(i for i, s in enumerate(segments) if s["kind"] == "memory")
            offs = OC.segment_offsets(segments)
            a, b = offs[mi][0], offs[mi][1]
            ck = torch.cat([ck[:, :a], mk, ck[:, b:]], dim=1)
            cv = torch.cat([cv[:, :a], mv, cv[:, b:]], dim=1)
    return outs, ck, cv, segments
