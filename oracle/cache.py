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


# ---------------------------------------------------------------------------
# The anchor | memory | window | current stream (the long-stream steady state).
#
# Same mechanics as generate_next_window's commit/evict loop (model.py:202-246,
# segments as _make_interactive_kv_segment builds them, streaming_runtime.py:
# 354-387, eviction as _prune_clean_kv_to_sink_recent, :612-662), with the
# pinned set widened from the sink block to {anchor ("prefix"), memory} and the
# recent set sized by a frame cap: the window keeps the newest generated
# blocks whose frames fit in ``window_frames``.  The memory segment keeps its
# positions (frames anchor_frames .. anchor_frames + memory_frames - 1) and is
# re-prefilled at them every ``refresh_every`` commits (the re-prefill of
# retained segments at their original global positions, runtime.py:386-470);
# its content version counts the refreshes.
# ---------------------------------------------------------------------------
PINNED_KINDS = ("prefix", "memory")


def retain_pinned_recent(segments: List[Dict], recent_blocks: int,
                         pinned_kinds=PINNED_KINDS) -> List[int]:
    """Indices kept: every pinned segment plus the newest ``recent_blocks``
    other segments, in chronological (list) order."""
    pinned = [i for i, s in enumerate(segments) if s.get("kind") in pinned_kinds]
    others = [i for i in range(len(segments)) if i not in pinned]
    recent = others[-recent_blocks:] if recent_blocks > 0 else []
    return sorted(set(pinned + recent))


def stream_segments_layout(video_hw: Tuple[int, int], anchor_frames: int = 1, memory_frames: int = 2,
                           chunk_frames: int = 3):
    """Segment dicts of the anchor and memory, and of generated chunk c."""
    hw = video_hw[0] * video_hw[1]
    anchor = {"kind": "prefix", "block_idx": 0, "video_tokens": anchor_frames * hw, "audio_tokens": 0}
    memory = {"kind": "memory", "block_idx": 1, "video_tokens": memory_frames * hw, "audio_tokens": 0}

    def chunk(c: int) -> Dict:
        return {"kind": "generated", "block_idx": c + 2, "video_tokens": chunk_frames * hw, "audio_tokens": 0,
                "window_slot": c}
    return anchor, memory, chunk


def chunk_start_frame(c: int, anchor_frames: int = 1, memory_frames: int = 2, chunk_frames: int = 3) -> int:
    """Absolute latent frame of chunk c's first frame."""
    return anchor_frames + memory_frames + c * chunk_frames


def streaming_plan_window(n_chunks: int, video_hw: Tuple[int, int], anchor_frames: int = 1,
                          memory_frames: int = 2, chunk_frames: int = 3, window_frames: int = 12,
                          refresh_every: int = 4) -> List[dict]:
    """Replay of the stream on token-id tensors.  Entry c describes the cache
    after chunk c is committed, evicted and (when due) the memory refreshed:
    the kept segments, the absolute video token ids in cache order, and the
    memory content version."""
    hw = video_hw[0] * video_hw[1]
    recent = window_frames // chunk_frames
    anchor, memory, chunk = stream_segments_layout(video_hw, anchor_frames, memory_frames, chunk_frames)
    ids = lambda f0, nf: torch.arange(f0 * hw, (f0 + nf) * hw, dtype=torch.int64).view(1, -1, 1, 1)
    layer = {"video_self_k": cat_cache(ids(0, anchor_frames), ids(anchor_frames, memory_frames))}
    segments = [dict(anchor), dict(memory)]
    version = 0
    plan = []
    for c in range(n_chunks):
        f0 = chunk_start_frame(c, anchor_frames, memory_frames, chunk_frames)
        layer["video_self_k"] = cat_cache(layer["video_self_k"], ids(f0, chunk_frames))
        segments.append(chunk(c))
        keep = retain_pinned_recent(segments, recent)
        if keep != list(range(len(segments))):
            offs = segment_offsets(segments)
            layer["video_self_k"] = slice_tensor(layer["video_self_k"], [(offs[i][0], offs[i][1]) for i in keep])
            segments = [dict(segments[i]) for i in keep]
        if refresh_every > 0 and (c + 1) % refresh_every == 0:
            # re-prefill the memory at its own positions: same token ids, new version
            version += 1
        plan.append({"chunk": c, "segments": [dict(s) for s in segments],
                     "video_ids": layer["video_self_k"].flatten().tolist(), "memory_version": version})
    return plan
