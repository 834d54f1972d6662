"""Segment metadata and eviction (host mirror of taomate/inference/cache.py:1-67 and
taomate/inference/streaming_runtime.py:409-662).

Eviction keeps the sink block (``block_idx == 0``, the pinned anchor) plus the
newest non-sink blocks, in chronological order.  On arena-backed caches every
slice is index-only: the surviving spans are re-listed and nothing is copied.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

from .kv_cache import KVCache, KVSpanView, LayerKVCache


def cache_segments(cache: KVCache) -> List[Dict[str, Any]]:
    """cache.py:7-8."""
    return [dict(item) for item in cache.segments]


def attach_segments(cache: KVCache, segments: List[Dict[str, Any]]) -> KVCache:
    """cache.py:10-12."""
    cache.segments = [dict(item) for item in segments]
    return cache


def _segment_offsets(segments: List[Dict[str, Any]]) -> List[Tuple[int, int, int, int]]:
    """cache.py:14-26 (missing/negative counts read as 0, streaming_runtime.py:409-428)."""
    vo = ao = 0
    offsets = []
    for seg in segments:
        ve = vo + max(0, int(seg.get("video_tokens") or 0))
        ae = ao + max(0, int(seg.get("audio_tokens") or 0))
        offsets.append((vo, ve, ao, ae))
        vo, ao = ve, ae
    return offsets


def _slice_tensor(tensor, spans: Sequence[Tuple[int, int]]):
    """cache.py:28-32 / streaming_runtime.py:431-442.  Views slice by index."""
    if tensor is None:
        return None
    pieces = [tensor[:, a:b] for a, b in spans if b > a]
    if not pieces:
        return None
    if len(pieces) == 1:
        return pieces[0]
    if isinstance(tensor, KVSpanView):
        return KVSpanView(tensor.arena, tensor.which, [s for p in pieces for s in p.spans])
    return torch.cat(pieces, dim=1)


_VIDEO = ("video_self_k", "video_self_v", "v2a_k", "v2a_v")
_AUDIO = ("audio_self_k", "audio_self_v", "a2v_k", "a2v_v")


def _slice_layers(layers: List[LayerKVCache], segments, indices: List[int]) -> List[LayerKVCache]:
    offsets = _segment_offsets(segments)
    vsp = [(offsets[i][0], offsets[i][1]) for i in indices]
    asp = [(offsets[i][2], offsets[i][3]) for i in indices]
    out = []
    for layer in layers:
        kw = {f: _slice_tensor(getattr(layer, f), vsp) for f in _VIDEO}
        kw.update({f: _slice_tensor(getattr(layer, f), asp) for f in _AUDIO})
        out.append(LayerKVCache(**kw))
    return out


def _slice_cache(cache: KVCache, indices: List[int]) -> KVCache:
    """cache.py:34-56."""
    segments = cache_segments(cache)
    return attach_segments(KVCache(layers=_slice_layers(cache.layers, segments, indices)),
                           [segments[i] for i in indices])


def retain_streaming_context(cache: KVCache) -> KVCache:
    """cache.py:58-67: keep the sink block and the 2 newest non-sink blocks."""
    segments = cache_segments(cache)
    if not segments:
        raise RuntimeError("Cached inference did not attach block metadata.")
    sink = next(i for i, s in enumerate(segments) if int(s["block_idx"]) == 0)
    non_sink = [i for i in range(len(segments)) if i != sink]
    keep = sorted([sink, *non_sink[-2:]])
    return cache if keep == list(range(len(segments))) else _slice_cache(cache, keep)


def prune_clean_kv_to_sink_recent(cache: KVCache, *, recent_blocks: int) -> Optional[KVCache]:
    """streaming_runtime.py:612-662: sink (if any) + ``recent_blocks`` newest blocks."""
    if cache is None:
        return None
    segments = cache_segments(cache)
    if not segments:
        return None
    sink = next((i for i, s in enumerate(segments) if int(s.get("block_idx", -1)) == 0), None)
    non_sink = [i for i in range(len(segments)) if i != sink]
    k = max(0, int(recent_blocks))
    keep = sorted(set(([sink] if sink is not None else []) + (non_sink[-k:] if k > 0 else [])))
    if keep == list(range(len(segments))):
        return cache
    return _slice_cache(cache, keep)
