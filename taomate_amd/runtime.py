"""The model-level stream loop: denoising a block over the cached context,
committing its clean K/V, and keeping the window.

Host mirror of:
  compute_denoising_sigmas        taomate/inference/model.py:11-19, with the
                                  schedule of LTX2Scheduler.execute
                                  (ltx_core/components/schedulers.py:21-57)
  add_noise                       taomate/inference/model_runtime.py:123-134
  _velocity_to_x0                 model_runtime.py:681-687
  _channel_stats / _apply_renorm /
  _maybe_renorm_block             model_runtime.py:24-46, 732-770
  _denoise_block_with_kv          model_runtime.py:772-964
  _commit_clean_block             taomate/inference/model.py:88-129
  generate (first window)         model_runtime.py:1008-1342: block 0 on an
                                  empty cache, later blocks appended without
                                  pruning
  generate_next_window            model.py:166-248: per block, denoise, commit,
                                  memory update, retain (sink + 2 recent)
  _refresh_conditioning_cache     taomate/inference/runtime.py:386-470: on a
                                  prompt change, the retained blocks re-run at
                                  sigma 0 under the new conditioning at their
                                  global positions; their audio self, A2V and
                                  V2A K/V replace the cache's, video self stays

Every attention, norm and cache kernel runs through ``AVModel.forward_chunk``
on this package's HIP library; the loop itself only moves latents and cache
views.  The cache keeps the reference's functional semantics: a denoising step
attends the pre-block layers plus the block and leaves them as they were (the
snapshot/restore of model_runtime.py:847-895 holds trivially), and the clean
commit appends the block's sigma-0 keys to those same pre-block layers.
"""
from __future__ import annotations

import math
import weakref
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import torch

from .blocks import AVBlock, compute_aligned_audio_frames, compute_av_blocks, global_block_at_index
from .cache import attach_segments, cache_segments, retain_streaming_context
from .kv_cache import KVCache, LayerKVCache
from .rope import causal_precompute_freqs_cis

DENOISING_STEPS = (1000, 757, 522, 0)
FIRST_BLOCK_FRAMES = 4
FRAMES_PER_BLOCK = 3
WINDOW_BLOCKS = 5


def ltx2_schedule(steps: int = 40, tokens: int = 4096, max_shift: float = 2.05, base_shift: float = 0.95,
                  terminal: float = 0.1) -> torch.Tensor:
    """LTX2Scheduler.execute (schedulers.py:21-57) without a latent: the
    shifted flow-matching schedule from 1 to 0 in ``steps`` steps, its
    non-zero values stretched so the last one equals ``terminal``."""
    s = torch.linspace(1.0, 0.0, steps + 1)
    slope = (max_shift - base_shift) / (4096 - 1024)
    shift = tokens * slope + (base_shift - slope * 1024)
    e = math.exp(shift)
    s = torch.where(s != 0, e / (e + (1.0 / s - 1.0)), torch.zeros_like(s))
    nz = s != 0
    one_minus = 1.0 - s[nz]
    s[nz] = 1.0 - one_minus / (one_minus[-1] / (1.0 - terminal))
    return s.to(torch.float32)


def denoising_sigmas(steps: Sequence[int] = DENOISING_STEPS, device="cpu") -> torch.Tensor:
    """compute_denoising_sigmas (model.py:11-19): for each step t of
    DENOISING_STEPS the schedule value nearest to t / 1000."""
    schedule = ltx2_schedule()
    out = [schedule[int((schedule - t / 1000.0).abs().argmin())] for t in steps]
    return torch.stack(out).to(device)


def add_noise(x0: torch.Tensor, noise: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """x_t = (1 - sigma) x0 + sigma noise (model_runtime.py:123-134); sigma
    [B] or [B, F] broadcast over the remaining dims."""
    s = sigma.reshape(*sigma.shape, *([1] * (x0.dim() - sigma.dim()))).to(x0.dtype)
    return ((1 - s) * x0 + s * noise).to(x0.dtype)


def velocity_to_x0(sample: torch.Tensor, velocity: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """x0 = sample - velocity sigma in float32 (model_runtime.py:681-687)."""
    s = sigma.reshape(*sigma.shape, *([1] * (sample.dim() - sigma.dim()))).to(torch.float32)
    return (sample.to(torch.float32) - velocity.to(torch.float32) * s).to(sample.dtype)


def channel_stats(latent: torch.Tensor, video: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-sample, per-channel mean and (unbiased) std over frames and space
    for a [B, F, C, H, W] video latent (model_runtime.py:24-31)."""
    dims = (1, 3, 4) if video else (1,)
    return latent.mean(dim=dims, keepdim=True), latent.std(dim=dims, keepdim=True).clamp_min(1e-6)


def apply_renorm(latent: torch.Tensor, anchor: Tuple[torch.Tensor, torch.Tensor], alpha: float) -> torch.Tensor:
    """Moves each channel's statistics to (1 - alpha) current + alpha anchor
    (model_runtime.py:34-46)."""
    mean, std = channel_stats(latent)
    tm = (1.0 - alpha) * mean + alpha * anchor[0].to(mean.dtype)
    ts = (1.0 - alpha) * std + alpha * anchor[1].to(std.dtype)
    return (((latent - mean) / std) * ts + tm).to(latent.dtype)


def prepare_attention_mask(mask: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
    """causal_model.py:551-562: a 0/1 key mask becomes the additive
    (m - 1) * finfo(dtype).max of shape [B, 1, 1, L]; a float mask is used as
    given."""
    if mask is None or torch.is_floating_point(mask):
        return mask
    return (mask - 1).to(dtype).reshape(mask.shape[0], 1, -1, mask.shape[-1]) * torch.finfo(dtype).max


def video_tokens(latent: torch.Tensor) -> torch.Tensor:
    """[B, F, C, H, W] -> [B, F*H*W, C] in (frame, row, column) order, the
    patchify layout of forward_inference (kv_cache.py:2770-2772)."""
    B, F, C, H, W = latent.shape
    return latent.permute(0, 1, 3, 4, 2).reshape(B, F * H * W, C)


def video_latent(tokens: torch.Tensor, frames: int, hw: Tuple[int, int]) -> torch.Tensor:
    """Inverse of ``video_tokens``."""
    B, _, C = tokens.shape
    return tokens.view(B, frames, hw[0], hw[1], C).permute(0, 1, 4, 2, 3)


NoiseFn = Callable[[Tuple[int, ...], torch.device, torch.dtype], torch.Tensor]


def refresh_selection(segments: Sequence[Dict[str, Any]], prefix_frames: int,
                      next_frames: int) -> List[Tuple[AVBlock, AVBlock]]:
    """The (prefix block, global block) pairs a prompt-change refresh re-runs
    (taomate/inference/runtime.py:400-414, 427): the prefix's blocks among the
    4-3-3 blocks of prefix + next frames; the sink block first when the cache
    holds block 0, then the last ``len(segments) - sink`` prefix blocks, each
    paired with the global block of its segment's index.  A prefix holding
    fewer blocks than the cache's segments is an error."""
    local = compute_av_blocks(int(prefix_frames) + int(next_frames), FRAMES_PER_BLOCK, FIRST_BLOCK_FRAMES)
    prefix_blocks = [b for b in local if b.video_end <= prefix_frames]
    has_sink = int(segments[0]["block_idx"]) == 0
    warm = len(segments) - int(has_sink)
    candidates = prefix_blocks[1:] if has_sink else prefix_blocks
    selected = ([prefix_blocks[0]] if has_sink else []) + (candidates[-warm:] if warm else [])
    if len(selected) != len(segments):
        raise RuntimeError("The retained latent prefix does not match the cache layout.")
    return [(lb, global_block_at_index(int(seg["block_idx"]), FRAMES_PER_BLOCK, FIRST_BLOCK_FRAMES))
            for lb, seg in zip(selected, segments)]


class StreamingGenerator:
    """Block loop of one stream on an ``AVModel`` (taomate/inference/model.py:33-248).

    ``noise(shape, device, dtype)`` draws every Gaussian the loop needs, in the
    reference's order: per block the initial video then audio noise, then per
    denoising step but the last the video then audio re-noise.  The default
    draws from ``torch.randn`` with a generator seeded by ``seed``.
    ``prefix_renorm`` (on, alpha 1, anchor block 0, as the shipped runtime,
    runtime.py:165-166) moves each block's video statistics to block 0's.
    ``arena_plan`` gives the caches of ``init_kv_cache`` KV arenas."""

    def __init__(self, model, video_hw: Tuple[int, int], *, sigmas: Optional[torch.Tensor] = None,
                 prefix_renorm: bool = True, renorm_alpha: float = 1.0, renorm_anchor_block: int = 0,
                 arena_plan=None, noise: Optional[NoiseFn] = None, seed: int = 0):
        self.model = model
        self.video_hw = (int(video_hw[0]), int(video_hw[1]))
        self.sigmas = (denoising_sigmas() if sigmas is None else sigmas).detach().to("cpu", torch.float32)
        self.prefix_renorm = bool(prefix_renorm)
        self.renorm_alpha = float(renorm_alpha)
        self.renorm_anchor_block = int(renorm_anchor_block)
        self._anchor_v: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self.arena_plan = arena_plan
        self._gen: Optional[torch.Generator] = None
        self._seed = int(seed)
        self.noise = noise if noise is not None else self._randn
        self.last_cache: Optional[KVCache] = None
        self._pe_cache: Dict[Tuple, tuple] = {}
        self._mask_cache: Dict[Tuple, tuple] = {}

    # ---- pieces ----
    def _randn(self, shape, device, dtype) -> torch.Tensor:
        dev = torch.device(device)
        if self._gen is None or self._gen.device != dev:
            self._gen = torch.Generator(device=dev)
            self._gen.manual_seed(self._seed)
        return torch.randn(shape, generator=self._gen, device=dev, dtype=torch.float32).to(dtype)

    def init_kv_cache(self) -> KVCache:
        return self.model.init_kv_cache(self.arena_plan)

    def _prepared_mask(self, mask: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
        """prepare_attention_mask, kept per conditioning mask tensor (same
        object, unmodified since): every forward of the stream then passes the
        same additive mask tensor, whose kept-prefix test (one host
        synchronisation per new mask tensor) runs once per stream instead of
        once per denoising step."""
        if mask is None or torch.is_floating_point(mask):
            return mask
        key = (id(mask), mask._version, dtype)
        hit = self._mask_cache.get(key)
        if hit is not None and hit[0]() is mask:
            return hit[1]
        out = prepare_attention_mask(mask, dtype)
        if len(self._mask_cache) > 8:
            self._mask_cache.clear()
        self._mask_cache[key] = (weakref.ref(mask), out)
        return out

    def block_rope(self, block: AVBlock, batch: int, device):
        """The four RoPE tables of a block at its absolute frames
        (kv_cache.py:2906-3027): video 3-D, audio 1-D, and the 1-D time tables
        of the cross-modal attentions, the video one repeated over each
        frame's tokens."""
        cfg = self.model.cfg
        key = (block.video_start, block.video_frames, block.audio_start, block.audio_frames, batch, str(device))
        hit = self._pe_cache.get(key)
        if hit is not None:
            return hit
        H, W = self.video_hw
        F, Fa = block.video_frames, block.audio_frames
        cross = cfg.audio_heads * cfg.audio_d_head

        def pe(grid, dim, heads, f0, audio=False):
            return causal_precompute_freqs_cis(torch.tensor([list(grid)] * batch), dim, start_frame=f0,
                                               device=device, dtype=torch.bfloat16, num_attention_heads=heads,
                                               is_audio=audio)
        vcross = tuple(t.repeat_interleave(H * W, dim=2).contiguous()
                       for t in pe((F,), cross, cfg.audio_heads, block.video_start))
        out = (pe((F, H, W), cfg.video_dim, cfg.video_heads, block.video_start),
               pe((Fa,), cfg.audio_dim, cfg.audio_heads, block.audio_start, True), vcross,
               pe((Fa,), cross, cfg.audio_heads, block.audio_start, True))
        if len(self._pe_cache) > 16:
            self._pe_cache.clear()
        self._pe_cache[key] = out
        return out

    def forward(self, block: AVBlock, video: torch.Tensor, audio: torch.Tensor, sigma_v: torch.Tensor,
                sigma_a: torch.Tensor, cond: Dict[str, Any], cache: KVCache, kv_cache_only: bool = False):
        """forward_inference for one block (kv_cache.py:2681-3365): video
        [B, F, C, H, W] and audio [B, Fa, C] latents, per-frame sigmas.
        Returns the velocities in the latents' layouts; with ``kv_cache_only``
        the cache's layers become the committed ones and (None, None) is
        returned."""
        B = video.shape[0]
        dt = self.model.patchify_proj.weight.dtype
        vpe, ape, vcpe, acpe = self.block_rope(block, B, video.device)
        mask_v = self._prepared_mask(cond.get("video_context_mask"), dt)
        mask_a = self._prepared_mask(cond.get("audio_context_mask"), dt)
        vo, ao, layers = self.model.forward_chunk(
            video_tokens(video).to(dt), audio.to(dt), sigma_v, cond["video_context"].to(dt),
            cond["audio_context"].to(dt), mask_v, mask_a, vpe, ape, vcpe, acpe, list(cache.layers),
            learned_memory_video=cond.get("learned_memory_video"),
            learned_memory_audio=cond.get("learned_memory_audio"),
            learned_memory_color=cond.get("learned_memory_color"), kv_cache_only=kv_cache_only,
            audio_sigma=sigma_a)
        if kv_cache_only:
            cache.layers = layers
            return None, None
        return video_latent(vo, video.shape[1], self.video_hw).to(video.dtype), ao.to(audio.dtype)

    def _renorm(self, block_idx: int, video: torch.Tensor) -> torch.Tensor:
        """_maybe_renorm_block (model_runtime.py:732-770), video only."""
        if not self.prefix_renorm or block_idx < self.renorm_anchor_block:
            return video
        if block_idx == self.renorm_anchor_block:
            self._anchor_v = tuple(t.detach() for t in channel_stats(video))
            return video
        return apply_renorm(video, self._anchor_v, self.renorm_alpha) if self._anchor_v is not None else video

    def denoise_block(self, block: AVBlock, B: int, video_tail_shape: Tuple[int, ...], audio_channels: int,
                      cond: Dict[str, Any], cache: KVCache, device, dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """_denoise_block_with_kv (model_runtime.py:772-964) without conditioning
        frames: start from noise, and at each sigma but the last predict the
        velocity over the pre-block cache, take x0 = x - v sigma and re-noise
        it to the next sigma."""
        pre = list(cache.layers)
        video = self.noise((B, block.video_frames, *video_tail_shape), device, dtype)
        audio = self.noise((B, block.audio_frames, audio_channels), device, dtype)
        sig = self.sigmas
        for si in range(len(sig) - 1):
            cache.layers = list(pre)   # every step attends the prefix only
            # one sigma for every frame of the block: the per-frame [B, F]
            # values of the reference are equal, so one per sample is the same
            s = sig[si].to(device).expand(B)
            v_vel, a_vel = self.forward(block, video, audio, s, s, cond, cache)
            video = velocity_to_x0(video, v_vel, s)
            audio = velocity_to_x0(audio, a_vel, s)
            nxt = sig[si + 1]
            if float(nxt) > 0.0:
                n = nxt.to(device).expand(B)
                video = add_noise(video, self.noise(tuple(video.shape), device, dtype), n)
                audio = add_noise(audio, self.noise(tuple(audio.shape), device, dtype), n)
        cache.layers = pre
        return video, audio

    def commit_clean_block(self, block: AVBlock, video: torch.Tensor, audio: torch.Tensor, cond: Dict[str, Any],
                           cache: Optional[KVCache], previous_layers: Optional[List[LayerKVCache]]) -> KVCache:
        """_commit_clean_block (model.py:88-129): the sigma-0 pass over the
        clean block appends its K/V to the pre-block layers (or to a fresh
        cache for the first block)."""
        if previous_layers is None or cache is None:
            cache = self.init_kv_cache()
        else:
            cache.layers = list(previous_layers)
        z = torch.zeros(video.shape[0], device=video.device, dtype=torch.float32)
        self.forward(block, video, audio, z, z, cond, cache, kv_cache_only=True)
        return cache

    def segment(self, block: AVBlock, window_slot: Optional[int] = None) -> Dict[str, Any]:
        """The block's cache segment record (model.py:131-137,
        model_runtime.py:1056-1069)."""
        seg = {"block_idx": int(block.block_idx),
               "video_tokens": int(block.video_frames * self.video_hw[0] * self.video_hw[1]),
               "audio_tokens": int(block.audio_frames)}
        if window_slot is not None:
            seg.update(kind="generated", window_slot=int(window_slot), include_audio_sinks=False)
        return seg

    def _with_memory(self, memory, cond, device, dtype):
        return memory.with_conditional_memory(cond, device=device, dtype=dtype) if memory is not None else cond

    # ---- windows ----
    @torch.no_grad()
    def generate_first_window(self, video_shape: Tuple[int, ...], audio_shape: Tuple[int, ...],
                              cond: Dict[str, Any], memory=None,
                              block_callback: Optional[Callable] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """The first window (model_runtime.py:1008-1342 as called by
        model.py:139-159): block 0 (4 frames) denoised on an empty cache, then
        blocks 1..4 (3 frames each), every block's clean K/V appended with no
        pruning (16 frames cached at the end).  Returns the window's video
        [B, F, C, H, W] and audio [B, Fa, C] latents; the cache and its
        segments are ``self.last_cache``."""
        dev = cond["video_context"].device
        dtype = torch.bfloat16
        B, F_total = int(video_shape[0]), int(video_shape[1])
        blocks = compute_av_blocks(F_total, FRAMES_PER_BLOCK, FIRST_BLOCK_FRAMES)
        video = torch.zeros(video_shape, device=dev, dtype=dtype)
        audio = torch.zeros(audio_shape, device=dev, dtype=dtype)
        segments: List[Dict[str, Any]] = []
        cache: Optional[KVCache] = None
        self._anchor_v = None
        for i, block in enumerate(blocks):
            bc = self._with_memory(memory, cond, dev, dtype)
            if block.block_idx == 0:
                cache = self.init_kv_cache()
                prev = None
            else:
                prev = list(cache.layers)
            bv, ba = self.denoise_block(block, B, tuple(video_shape[2:]), int(audio_shape[2]), bc, cache, dev, dtype)
            bv = self._renorm(block.block_idx, bv)
            if memory is not None:
                bv = memory.apply_color_memory(bv)
            video[:, block.video_start:block.video_end] = bv
            audio[:, block.audio_start:block.audio_end] = ba
            if block_callback is not None:
                block_callback(bv, ba, block)
            cache = self.commit_clean_block(block, bv, ba, bc, cache, prev)
            segments.append(self.segment(block, window_slot=i))
            if memory is not None:
                if block.block_idx == 0:
                    memory.set_reference(bv, ba)
                memory.update(bv, ba)
        attach_segments(cache, segments)
        self.last_cache = cache
        return video, audio

    @torch.no_grad()
    def generate_next_window(self, video_shape: Tuple[int, ...], audio_shape: Tuple[int, ...],
                             cond: Dict[str, Any], memory, cache: KVCache, first_block_index: int,
                             block_callback: Optional[Callable] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """generate_next_window (model.py:166-248): 5 blocks of 3 frames at
        their global positions; each is denoised over the retained context,
        committed clean from the pre-block layers, fed to the memory, and the
        cache is cut back to the sink block plus the 2 most recent blocks."""
        dev = cond["video_context"].device
        dtype = torch.bfloat16
        B = int(video_shape[0])
        total = FIRST_BLOCK_FRAMES + (int(first_block_index) + WINDOW_BLOCKS - 1) * FRAMES_PER_BLOCK
        blocks = compute_av_blocks(total, FRAMES_PER_BLOCK, FIRST_BLOCK_FRAMES)[
            first_block_index:first_block_index + WINDOW_BLOCKS]
        if len(blocks) != WINDOW_BLOCKS:
            raise RuntimeError("Unable to construct continuous block positions.")
        video = torch.zeros(video_shape, device=dev, dtype=dtype)
        audio = torch.zeros(audio_shape, device=dev, dtype=dtype)
        segments = cache_segments(cache)
        # The reference's first commit re-assigns the layers of the object it
        # was given (model.py:100-103) and retention then returns a new one, so
        # the caller's object would keep every block committed so far alive
        # for the whole window.  With arena-backed caches that pins evicted
        # slots; the loop therefore works on its own shallow copy (same views,
        # same results) and leaves the caller's object as it was.
        cache = KVCache(layers=list(cache.layers), segments=[dict(s) for s in segments])
        vo = ao = 0
        for block in blocks:
            prev = list(cache.layers)
            bc = self._with_memory(memory, cond, dev, dtype)
            bv, ba = self.denoise_block(block, B, tuple(video_shape[2:]), int(audio_shape[2]), bc, cache, dev, dtype)
            bv = self._renorm(block.block_idx, bv)
            if memory is not None:
                bv = memory.apply_color_memory(bv)
            video[:, vo:vo + block.video_frames] = bv
            audio[:, ao:ao + block.audio_frames] = ba
            if block_callback is not None:
                block_callback(bv, ba, block)
            cache = self.commit_clean_block(block, bv, ba, bc, cache, prev)
            if memory is not None:
                memory.update(bv, ba)
            segments.append(self.segment(block))
            attach_segments(cache, segments)
            cache = retain_streaming_context(cache)
            segments = cache_segments(cache)
            vo += block.video_frames
            ao += block.audio_frames
        self.last_cache = cache
        return video, audio

    @torch.no_grad()
    def refresh_conditioning_cache(self, cache: KVCache, cond: Dict[str, Any], prefix_video: torch.Tensor,
                                   prefix_audio: torch.Tensor, next_video_shape: Tuple[int, ...],
                                   memory=None) -> KVCache:
        """_refresh_conditioning_cache (taomate/inference/runtime.py:386-470).

        ``prefix_video`` [B, F, C, H, W] / ``prefix_audio`` [B, Fa, C] are the
        retained blocks' latents in cache order (sink block, then the recent
        blocks).  Each cached segment's latents go through the sigma-0
        cache-only pass with the new ``cond`` at the segment's global block
        positions, building a fresh cache; the retained layers then take that
        cache's audio self, A2V and V2A K/V, while their video self K/V stay
        as they are (pinned).  The layers are updated in place, as in the
        reference, and ``cache`` is returned with its segments."""
        segments = cache_segments(cache)
        if not segments:
            raise RuntimeError("The retained cache has no block metadata.")
        if prefix_audio is None or int(prefix_audio.shape[1]) != compute_aligned_audio_frames(
                int(prefix_video.shape[1]), FRAMES_PER_BLOCK, FIRST_BLOCK_FRAMES):
            raise RuntimeError(f"Prefix alignment mismatch: {prefix_video.shape[1]} video frames, "
                               f"{None if prefix_audio is None else prefix_audio.shape[1]} audio frames.")
        pairs = refresh_selection(segments, int(prefix_video.shape[1]), int(next_video_shape[1]))
        dev = cond["video_context"].device
        dtype = self.model.patchify_proj.weight.dtype
        rebuilt = self.init_kv_cache()
        for lb, gb in pairs:
            video = prefix_video[:, lb.video_start:lb.video_end].to(device=dev, dtype=dtype)
            audio = prefix_audio[:, lb.audio_start:lb.audio_end].to(device=dev, dtype=dtype)
            bc = self._with_memory(memory, cond, dev, dtype)
            z = torch.zeros(video.shape[0], device=dev, dtype=torch.float32)
            self.forward(gb, video, audio, z, z, bc, rebuilt, kv_cache_only=True)
        if len(rebuilt.layers) != len(cache.layers):
            raise RuntimeError("Conditioning cache refresh failed.")
        for kept, new in zip(cache.layers, rebuilt.layers):
            kept.audio_self_k, kept.audio_self_v = new.audio_self_k, new.audio_self_v
            kept.a2v_k, kept.a2v_v = new.a2v_k, new.a2v_v
            kept.v2a_k, kept.v2a_v = new.v2a_k, new.v2a_v
        return attach_segments(cache, segments)
