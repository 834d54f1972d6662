"""KV-cache bookkeeping restatement (oracle; test infrastructure only).

Follows:
  _cat_cache                       ltx_causal/transformer/kv_cache.py:394-398
  LayerKVCache fields              ltx_causal/transformer/kv_cache.py:321-358
  _segment_offsets/_slice_tensor/_slice_cache/retain_streaming_context
                                   taomate/inference/cache.py:14-67
  _prune_clean_kv_to_sink_recent   taomate/inference/streaming_runtime.py:612-662
  compute_av_blocks / compute_aligned_audio_frames
                                   ltx_causal/attention/mask_builder.py:102-266
  _cache_segment                   taomate/inference/model.py:131-136
A layer cache here is a dict field-name -> tensor [B, L, H, D] (or None).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

FIELDS = ("video_self_k", "video_self_v", "audio_self_k", "audio_self_v",
          "a2v_k", "a2v_v", "v2a_k", "v2a_v")
VIDEO_FIELDS = ("video_self_k", "video_self_v", "v2a_k", "v2a_v")

AUDIO_FRAMES_PER_BLOCK = 25   # mask_builder.py:97
AUDIO_FRAMES_FIRST_BLOCK = 26  # mask_builder.py:99


def cat_cache(old: Optional[torch.Tensor], new: torch.Tensor) -> torch.Tensor:
    """kv_cache.py:394-398."""
    return new if old is None else torch.cat([old, new], dim=1)


def segment_offsets(segments: List[Dict[str, int]]) -> List[Tuple[int, int, int, int]]:
    """cache.py:14-26 -- cumulative (video_start, video_end, audio_start, audio_end)."""
    vo = ao = 0
    out = []
    for s in segments:
        ve = vo + int(s["video_tokens"])
        ae = ao + int(s["audio_tokens"])
        out.append((vo, ve, ao, ae))
        vo, ao = ve, ae
    return out


def slice_tensor(t: Optional[torch.Tensor], spans: List[Tuple[int, int]]) -> Optional[torch.Tensor]:
    """cache.py:28-32."""
    if t is None:
        return None
    pieces = [t[:, a:b] for a, b in spans if b > a]
    return pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=1)


def slice_cache(layers: List[Dict[str, torch.Tensor]], segments: List[Dict[str, int]],
                indices: List[int]):
    """cache.py:34-56: keep the given segment indices in chronological order."""
    offs = segment_offsets(segments)
    vsp = [(offs[i][0], offs[i][1]) for i in indices]
    asp = [(offs[i][2], offs[i][3]) for i in indices]
    new_layers = []
    for layer in layers:
        new_layers.append({f: slice_tensor(layer.get(f), vsp if f in VIDEO_FIELDS else asp)
                           for f in FIELDS})
    return new_layers, [dict(segments[i]) for i in indices]


def retain_indices(segments: List[Dict[str, int]], recent_blocks: int = 2) -> List[int]:
    """cache.py:58-67 (recent=2) / streaming_runtime.py:612-662: sink + newest non-sink."""
    if not segments:
        raise RuntimeError("Cached inference did not attach block metadata.")
    sink = next((i for i, s in enumerate(segments) if int(s["block_idx"]) == 0), None)
    non_sink = [i for i in range(len(segments)) if i != sink]
    recent = non_sink[-recent_blocks:] if recent_blocks > 0 else []
    return sorted(set(([sink] if sink is not None else []) + recent))


def retain_streaming_context(layers, segments, recent_blocks: int = 2):
    """cache.py:58-67: returns (layers, segments), unchanged when nothing is evicted."""
    keep = retain_indices(segments, recent_blocks)
    if keep == list(range(len(segments))):
        return layers, segments
    return slice_cache(layers, segments, keep)


@dataclass
class AVBlock:
    """mask_builder.py AVBlock: video/audio latent-frame ranges of one block."""
    block_idx: int
    video_start: int
    video_end: int
    audio_start: int
    audio_end: int

    @property
    def video_frames(self) -> int:
        return self.video_end - self.video_start

    @property
    def audio_frames(self) -> int:
        return self.audio_end - self.audio_start


def compute_av_blocks(total_video_latent_frames: int, num_frame_per_block: int = 3,
                      num_frame_per_block_first: int = 0) -> List[AVBlock]:
    """mask_builder.py:102-233 (OmniForcing 4-3-3-3 when first > 0, else 1-3-3-3)."""
    first = num_frame_per_block_first
    if first > 0:
        assert total_video_latent_frames >= first
        blocks = [AVBlock(0, 0, first, 0, AUDIO_FRAMES_FIRST_BLOCK)]
        vi, ai = first, AUDIO_FRAMES_FIRST_BLOCK
    else:
        assert total_video_latent_frames >= 1
        blocks = [AVBlock(0, 0, 1, 0, 1)]
        vi, ai = 1, 1
    bi = 1
    while vi < total_video_latent_frames:
        ve = min(vi + num_frame_per_block, total_video_latent_frames)
        nf = ve - vi
        ae = ai + (AUDIO_FRAMES_PER_BLOCK if nf == num_frame_per_block
                   else (AUDIO_FRAMES_PER_BLOCK * nf) // num_frame_per_block)
        blocks.append(AVBlock(bi, vi, ve, ai, ae))
        vi, ai, bi = ve, ae, bi + 1
    return blocks


def compute_aligned_audio_frames(total_video_latent_frames: int, num_frame_per_block: int = 3,
                                 num_frame_per_block_first: int = 0) -> int:
    """mask_builder.py:236-266."""
    b = compute_av_blocks(total_video_latent_frames, num_frame_per_block, num_frame_per_block_first)
    return b[-1].audio_end if b else 0


def cache_segment(block: AVBlock, video_hw: Tuple[int, int]) -> Dict[str, int]:
    """model.py:131-136."""
    return {"block_idx": int(block.block_idx),
            "video_tokens": int(block.video_frames * video_hw[0] * video_hw[1]),
            "audio_tokens": int(block.audio_frames)}


def streaming_plan(n_blocks: int, video_hw: Tuple[int, int], recent_blocks: int = 2,
                   first: int = 4) -> List[dict]:
    """Replay the commit/evict loop of generate_next_window (model.py:202-246) on
    token-id tensors, one entry per committed block: the absolute video and audio
    token ids held after eviction.  This is the bit-exact eviction plan."""
    total = first + (n_blocks - 1) * 3
    blocks = compute_av_blocks(total, num_frame_per_block_first=first)[:n_blocks]
    hw = video_hw[0] * video_hw[1]
    layer = {f: None for f in FIELDS}
    segments: List[Dict[str, int]] = []
    plan = []
    for blk in blocks:
        vid = torch.arange(blk.video_start * hw, blk.video_end * hw, dtype=torch.int64).view(1, -1, 1, 1)
        aid = torch.arange(blk.audio_start, blk.audio_end, dtype=torch.int64).view(1, -1, 1, 1)
        layer = {f: cat_cache(layer[f], vid if f in VIDEO_FIELDS else aid) for f in FIELDS}
        segments.append(cache_segment(blk, video_hw))
        layers, segments = retain_streaming_context([layer], segments, recent_blocks)
        layer = layers[0]
        plan.append({"block_idx": blk.block_idx,
                     "segments": [dict(s) for s in segments],
                     "video_ids": layer["video_self_k"].flatten().tolist(),
                     "audio_ids": layer["audio_self_k"].flatten().tolist()})
    return plan
