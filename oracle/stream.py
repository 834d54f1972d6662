"""fp32 restatement of the anchor | memory | window | current stream (oracle;
test infrastructure only).

One attention layer over dense [B, L, H, D] caches, with the reference's own
operations: attention_with_cache (ltx_causal/transformer/kv_cache.py:1148-1547)
for every chunk, torch.cat commit (_cat_cache, kv_cache.py:394-398), segment
slicing for eviction (taomate/inference/cache.py:28-56) with the pinned
{anchor, memory} + newest-window policy of ``cache.retain_pinned_recent``,
and the memory re-prefilled at its own positions every ``refresh_every``
chunks (runtime.py:386-470) from the state update
``state <- mix * state + (1 - mix) * last memory frames of the chunk``.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

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


def run_stream(w: OA.AttnWeights, grid_hw: Tuple[int, int], x_anchor: torch.Tensor,
               x_memory: Optional[torch.Tensor], chunks: Sequence[torch.Tensor], anchor_frames: int = 1,
               memory_frames: int = 2, chunk_frames: int = 3, window_frames: int = 12, refresh_every: int = 4,
               memory_mix: float = 0.5):
    """Layer outputs of every chunk in order, and the final K/V caches with
    their segment list: ``(outs, k, v, segments)``."""
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
        mk, mv = _kv_only(w, state, mem_pe)
        ck, cv = OC.cat_cache(ck, mk), OC.cat_cache(cv, mv)
        segments.append(dict(memory))
    outs = []
    for c, x in enumerate(chunks):
        f0 = OC.chunk_start_frame(c, anchor_frames, memory_frames, chunk_frames)
        out, nk, nv = OA.attention_with_cache(w, x, None, _pe(grid_hw, chunk_frames, dim, heads, f0, B), None,
                                              ck, cv)
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
            state = state * memory_mix + x[:, -memory_frames * hw:] * (1.0 - memory_mix)
            mk, mv = _kv_only(w, state, mem_pe)
            mi = next(i for i, s in enumerate(segments) if s["kind"] == "memory")
            offs = OC.segment_offsets(segments)
            a, b = offs[mi][0], offs[mi][1]
            ck = torch.cat([ck[:, :a], mk, ck[:, b:]], dim=1)
            cv = torch.cat([cv[:, :a], mv, cv[:, b:]], dim=1)
    return outs, ck, cv, segments
