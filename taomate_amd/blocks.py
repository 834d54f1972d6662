"""Audio/video block layout (host mirror of ltx_causal/attention/mask_builder.py:85-266).

The block table gives every chunk its RoPE start frames and the segment token
counts that drive eviction.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List

AUDIO_FRAMES_PER_BLOCK = 25    # mask_builder.py:97  (1 s = 3 video : 25 audio)
AUDIO_FRAMES_FIRST_BLOCK = 26  # mask_builder.py:99


@dataclass(frozen=True)
class AVBlock:
    """mask_builder.py AVBlock: [video_start, video_end) / [audio_start, audio_end) latent frames."""
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
    """mask_builder.py:102-233: 4-3-3-3 (OmniForcing) when first > 0, else 1-3-3-3.

    A partial last block gets ``25 * frames // num_frame_per_block`` audio frames.
    """
    first = int(num_frame_per_block_first)
    total = int(total_video_latent_frames)
    if first > 0:
        if total < first:
            raise ValueError(f"Need >= {first} video frames, got {total}")
        blocks = [AVBlock(0, 0, first, 0, AUDIO_FRAMES_FIRST_BLOCK)]
        v, a = first, AUDIO_FRAMES_FIRST_BLOCK
    else:
        if total < 1:
            raise ValueError(f"Need at least 1 video latent frame, got {total}")
        blocks = [AVBlock(0, 0, 1, 0, 1)]
        v, a = 1, 1
    idx = 1
    while v < total:
        ve = min(v + num_frame_per_block, total)
        n = ve - v
        ae = a + (AUDIO_FRAMES_PER_BLOCK if n == num_frame_per_block
                  else (AUDIO_FRAMES_PER_BLOCK * n) // num_frame_per_block)
        blocks.append(AVBlock(idx, v, ve, a, ae))
        v, a, idx = ve, ae, idx + 1
    return blocks


def compute_aligned_audio_frames(total_video_latent_frames: int, num_frame_per_block: int = 3,
                                 num_frame_per_block_first: int = 0) -> int:
    """mask_builder.py:236-266."""
    blocks = compute_av_blocks(total_video_latent_frames, num_frame_per_block,
                               num_frame_per_block_first)
    return blocks[-1].audio_end if blocks else 0


def global_block_at_index(block_idx: int, num_frame_per_block: int = 3,
                          num_frame_per_block_first: int = 4) -> AVBlock:
    """streaming_runtime.py:976-1000: one block by absolute index."""
    if block_idx < 0:
        raise ValueError(f"block_idx must be >= 0, got {block_idx}")
    total = num_frame_per_block_first + block_idx * num_frame_per_block
    blocks = compute_av_blocks(total, num_frame_per_block, num_frame_per_block_first)
    if block_idx >= len(blocks):
        raise RuntimeError(f"Failed to reconstruct global block {block_idx}")
    return blocks[block_idx]
