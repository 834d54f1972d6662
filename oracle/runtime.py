"""fp32 restatement of the model-level stream loop (oracle; test
infrastructure only).

Follows, step for step:
  LTX2Scheduler.execute                 ltx_core/components/schedulers.py:21-57
  compute_denoising_sigmas              taomate/inference/model.py:11-19
  add_noise                             taomate/inference/model_runtime.py:123-134
  _velocity_to_x0                       model_runtime.py:681-687
  _channel_stats / _apply_renorm /
  _maybe_renorm_block                   model_runtime.py:24-46, 732-770
  _denoise_block_with_kv                model_runtime.py:772-964 (no conditioning frames)
  _commit_clean_block                   model.py:88-129
  generate, first window                model_runtime.py:1008-1342
  generate_next_window                  model.py:166-248
with the dual-stream step of ``oracle.dit`` over dense caches (one dict of
[B, L, H, D] tensors per layer), the learned memory of ``oracle.memory`` and
the retention rule of ``oracle.cache``.
"""
from __future__ import annotations

import math
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import attention as OA
from . import cache as OC
from . import dit as OD
from . import rope as OR

DENOISING_STEPS = (1000, 757, 522, 0)


def schedule(steps: int = 40, tokens: int = 4096, max_shift: float = 2.05, base_shift: float = 0.95,
             terminal: float = 0.1) -> torch.Tensor:
    """schedulers.py:21-57: linspace(1, 0) shifted by exp(shift) / (exp(shift) +
    1/s - 1) with shift linear in the token count (0.95 at 1024 tokens, 2.05 at
    4096), the non-zero values stretched so the last one is ``terminal``."""
    s = torch.linspace(1.0, 0.0, steps + 1, dtype=torch.float64)
    m = (max_shift - base_shift) / (4096 - 1024)
    shift = tokens * m + base_shift - m * 1024
    out = torch.zeros_like(s)
    nz = s != 0
    out[nz] = math.exp(shift) / (math.exp(shift) + (1.0 / s[nz] - 1.0))
    z = 1.0 - out[nz]
    out[nz] = 1.0 - z / (z[-1] / (1.0 - terminal))
    return out.float()


def denoising_sigmas() -> torch.Tensor:
    sch = schedule()
    return torch.stack([sch[int((sch - t / 1000.0).abs().argmin())] for t in DENOISING_STEPS])


def add_noise(x0, noise, sigma):
    s = sigma.reshape(*sigma.shape, *([1] * (x0.dim() - sigma.dim())))
    return (1 - s) * x0 + s * noise


def velocity_to_x0(x, v, sigma):
    s = sigma.reshape(*sigma.shape, *([1] * (x.dim() - sigma.dim())))
    return x - v * s


def channel_stats(latent):
    return latent.mean(dim=(1, 3, 4), keepdim=True), latent.std(dim=(1, 3, 4), keepdim=True).clamp_min(1e-6)


def apply_renorm(latent, anchor, alpha):
    mean, std = channel_stats(latent)
    tm = (1 - alpha) * mean + alpha * anchor[0]
    ts = (1 - alpha) * std + alpha * anchor[1]
    return ((latent - mean) / std) * ts + tm


def compute_blocks(total_frames: int) -> List[Tuple[int, int, int, int, int]]:
    """(block_idx, video_start, video_end, audio_start, audio_end) of the 4-3-3-...
    frame blocks (oracle.cache.compute_av_blocks, mask_builder.py:97-233)."""
    return [(b.block_idx, b.video_start, b.video_end, b.audio_start, b.audio_end)
            for b in OC.compute_av_blocks(total_frames, num_frame_per_block_first=4)]


class StreamOracle:
    """One stream's loop state: dense per-layer caches, their segments, the
    renorm anchor.  ``noise(shape)`` supplies the Gaussians in the loop's order
    (per block: initial video, initial audio; per step but the last: video
    then audio re-noise)."""

    def __init__(self, params: Dict[str, torch.Tensor], cfg, video_hw: Tuple[int, int], noise: Callable,
                 memory=None, renorm: bool = True, alpha: float = 1.0, sigmas: Optional[torch.Tensor] = None):
        self.p, self.cfg, self.hw = params, cfg, (int(video_hw[0]), int(video_hw[1]))
        self.noise, self.memory = noise, memory
        self.renorm, self.alpha = renorm, alpha
        self.sigmas = denoising_sigmas() if sigmas is None else sigmas.float()
        self.layers: Optional[List[dict]] = None
        self.segments: List[dict] = []
        self.anchor = None

    def _rope(self, blk, B):
        cfg = self.cfg
        _, vs, ve, as_, ae = blk
        F_, Fa = ve - vs, ae - as_
        H, W = self.hw
        cross = cfg.audio_heads * cfg.audio_d_head
        pe = lambda grid, dim, heads, f0, audio=False: OR.causal_precompute_freqs_cis(
            grid, dim, start_frame=f0, num_attention_heads=heads, batch=B, is_audio=audio)
        vc = [t.repeat_interleave(H * W, dim=2) for t in pe((F_,), cross, cfg.audio_heads, vs)]
        return (pe((F_, H, W), cfg.video_dim, cfg.video_heads, vs),
                pe((Fa,), cfg.audio_dim, cfg.audio_heads, as_, True), vc, pe((Fa,), cross, cfg.audio_heads, as_, True))

    def _cond(self, cond):
        out = dict(cond)
        if self.memory is not None:
            for k, v in self.memory.conditioning().items():
                out[k] = torch.from_numpy(np.asarray(v)).float()
        return out

    def _forward(self, blk, video, audio, sigma, cond, layers):
        """(video velocity [B, F, C, H, W], audio velocity, layers with the block appended)."""
        B, F_, C, H, W = video.shape
        tokens = video.permute(0, 1, 3, 4, 2).reshape(B, F_ * H * W, C)
        mv = OA.prepare_attention_mask(cond["video_context_mask"], torch.bfloat16).float()
        ma = OA.prepare_attention_mask(cond["audio_context_mask"], torch.bfloat16).float()
        vo, ao, new = OD.forward_chunk(self.p, self.cfg, tokens, audio, sigma, cond["video_context"],
                                       cond["audio_context"], mv, ma, *self._rope(blk, B),
                                       layers if layers is not None else [{} for _ in range(self.cfg.num_layers)],
                                       learned_memory_video=cond.get("learned_memory_video"),
                                       learned_memory_audio=cond.get("learned_memory_audio"),
                                       learned_memory_color=cond.get("learned_memory_color"), return_caches=True)
        return vo.view(B, F_, H, W, C).permute(0, 1, 4, 2, 3), ao, new

    def _denoise(self, blk, B, C, c, pre):
        """_denoise_block_with_kv (model_runtime.py:847-962): pure noise, then per
        step the prefix-only cache (``pre``, restored every step), x0 = x - v*sigma,
        and re-noise with the NEXT sigma while it is above 0."""
        _, vs, ve, as_, ae = blk
        H, W = self.hw
        video = self.noise((B, ve - vs, C, H, W))
        audio = self.noise((B, ae - as_, C))
        sig = self.sigmas
        for si in range(len(sig) - 1):
            s = sig[si].expand(B)
            v_vel, a_vel, _ = self._forward(blk, video, audio, s, c, pre)     # attends the prefix only
            video, audio = velocity_to_x0(video, v_vel, s), velocity_to_x0(audio, a_vel, s)
            if float(sig[si + 1]) > 0.0:
                n = sig[si + 1].expand(B)
                video = add_noise(video, self.noise(tuple(video.shape)), n)
                audio = add_noise(audio, self.noise(tuple(audio.shape)), n)
        return video, audio

    def _stabilize(self, bi, video):
        """_maybe_renorm_block (model_runtime.py:732-770), anchor block 0, video only."""
        if self.renorm:
            if bi == 0:
                self.anchor = channel_stats(video)
            elif self.anchor is not None:
                video = apply_renorm(video, self.anchor, self.alpha)
        return video

    def _commit(self, blk, video, audio, c, pre, first_of_stream: bool):
        """_commit_clean_block (model.py:88-129): sigma 0 over the block's final
        latents, appended to the pre-block layers (a fresh cache for block 0)."""
        B = video.shape[0]
        _, _, self.layers = self._forward(blk, video, audio, torch.zeros(B), c, None if first_of_stream else pre)

    def _block(self, blk, B, C, cond, first_of_stream: bool):
        """One block in the reference's order (model.py:200-243;
        model_runtime.py:1160-1325): conditioning from the memory, denoise,
        renorm, colour correction, clean commit, then set_reference (block 0)
        and update."""
        bi = blk[0]
        c = self._cond(cond)
        pre = self.layers
        video, audio = self._denoise(blk, B, C, c, pre)
        video = self._stabilize(bi, video)
        if self.memory is not None:
            video = torch.from_numpy(self.memory.apply_color(video.double().numpy())).float()
        self._commit(blk, video, audio, c, pre, first_of_stream)
        if self.memory is not None:
            if first_of_stream:
                self.memory.set_reference(video.double().numpy(), audio.double().numpy())
            self.memory.update(video.double().numpy(), audio.double().numpy())
        return video, audio

    def first_window(self, B: int, C: int, cond, frames: int = 16):
        """Blocks of 4, 3, 3, ... frames from an empty cache, no pruning."""
        out = []
        self.segments = []
        for i, blk in enumerate(compute_blocks(frames)):
            v, a = self._block(blk, B, C, cond, first_of_stream=blk[0] == 0)
            self.segments.append({"block_idx": blk[0], "video_tokens": (blk[2] - blk[1]) * self.hw[0] * self.hw[1],
                                  "audio_tokens": blk[4] - blk[3]})
            out.append((blk, v, a))
        return out

    def next_window(self, B: int, C: int, cond, first_block_index: int, n_blocks: int = 5):
        """5 blocks at their global positions; after each commit the cache keeps
        the sink block and the 2 most recent (cache.py:58-67)."""
        total = 4 + (first_block_index + n_blocks - 1) * 3
        out = []
        for blk in compute_blocks(total)[first_block_index:first_block_index + n_blocks]:
            v, a = self._block(blk, B, C, cond, first_of_stream=False)
            self.segments.append({"block_idx": blk[0], "video_tokens": (blk[2] - blk[1]) * self.hw[0] * self.hw[1],
                                  "audio_tokens": blk[4] - blk[3]})
            layers, self.segments = OC.retain_streaming_context(self.layers, self.segments, 2)
            self.layers = layers
            out.append((blk, v, a))
        return out

    def rebuild_for_prompt(self, segments, cond, prefix_video, prefix_audio, next_frames: int):
        """_refresh_conditioning_cache (taomate/inference/runtime.py:386-470):
        the retained segments' latents (cache order) re-run at sigma 0 under
        ``cond`` at their global block positions, from an empty cache.
        Returns the rebuilt layers (the caller keeps their audio self, A2V and
        V2A fields)."""
        layers = None
        for lb, gb in refresh_selection(segments, prefix_video.shape[1], next_frames):
            video = prefix_video[:, lb[1]:lb[2]]
            audio = prefix_audio[:, lb[3]:lb[4]]
            B = video.shape[0]
            _, _, layers = self._forward(gb, video, audio, torch.zeros(B), self._cond(cond), layers)
        return layers


def global_block(k: int):
    """_global_block (taomate/inference/runtime.py:365-371): block k of a stream
    of 4 + 3k frames."""
    return compute_blocks(4 + int(k) * 3)[int(k)]


def refresh_selection(segments, prefix_frames: int, next_frames: int):
    """The (local prefix block, global block) pairs _refresh_conditioning_cache
    re-runs (taomate/inference/runtime.py:400-414, 427): the prefix's blocks
    among those of prefix + next frames; the sink block first when the cache
    holds block 0, then the last ``warm`` prefix blocks; each paired with the
    global block of its segment's block index."""
    prefix_blocks = [b for b in compute_blocks(int(prefix_frames) + int(next_frames)) if b[2] <= prefix_frames]
    has_sink = int(segments[0]["block_idx"]) == 0
    warm = len(segments) - int(has_sink)
    cands = prefix_blocks[1:] if has_sink else prefix_blocks
    selected = ([prefix_blocks[0]] if has_sink else []) + (cands[-warm:] if warm else [])
    if len(selected) != len(segments):
        raise RuntimeError("The retained latent prefix does not match the cache layout.")
    return [(lb, global_block(seg["block_idx"])) for lb, seg in zip(selected, segments)]
