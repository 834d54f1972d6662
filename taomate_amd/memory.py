"""Learned long-memory state: the detached summaries of generated latents that
condition later chunks through the blocks' memory adapters.

Host-side PyTorch on small tensors (a chunk's latents are [B, F, 128, H, W]
with H x W = 16 x 24 at 512 x 768; the memory is 48 video tokens and 64 audio
tokens of 128 channels), run on the latents' device.  The adapters that read
the memory inside the blocks are in ``taomate_amd.dit``.

Behaviour follows taomate/runtime_support/learned_memory.py:
  video / audio token summaries         :192-229
  EMA update with an anchor tether      :231-249
  drift gate (pooled cosine, sigmoid)   :120-166, :414-428
  colour memory (channel statistics,
  low-frequency prototype, correction)  :35-103, :169-189, :430-487
  LearnedMemoryState / update /
  with_conditional_memory               :252-591
and the production settings of taomate/inference/memory.py:4-29
(``StreamingMemory``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn.functional as F

__all__ = ["LearnedMemoryState", "StreamingMemory", "summarize_video_memory", "summarize_audio_memory",
           "apply_color_memory_snapshot"]


def _unit(x: float) -> float:
    """Clamp to [0, 1]."""
    return min(1.0, max(0.0, float(x)))


def _standardize(x: torch.Tensor, dims: Tuple[int, ...], eps: float) -> torch.Tensor:
    """(x - mean) / max(std, eps) over ``dims`` (population std)."""
    mu = x.mean(dim=dims, keepdim=True)
    sd = x.std(dim=dims, keepdim=True, unbiased=False).clamp_min(eps)
    return (x - mu) / sd


def summarize_video_memory(video_latent: Optional[torch.Tensor], *, downsample: int = 4,
                           eps: float = 1e-6) -> Optional[torch.Tensor]:
    """[B, F, C, H, W] latents -> [B, (H/d)(W/d), C] tokens: the frame mean,
    standardised over the spatial grid per channel, average-pooled by d."""
    if video_latent is None or video_latent.numel() == 0:
        return None
    if video_latent.dim() != 5:
        raise ValueError(f"video_latent must be [B,F,C,H,W], got {tuple(video_latent.shape)}")
    x = _standardize(video_latent.detach().float().mean(dim=1), (-2, -1), eps)
    d = max(1, int(downsample))
    gh, gw = max(1, x.shape[-2] // d), max(1, x.shape[-1] // d)
    x = F.adaptive_avg_pool2d(x, (gh, gw))
    B, C = x.shape[:2]
    return x.flatten(2).transpose(1, 2).contiguous().view(B, gh * gw, C)


def summarize_audio_memory(audio_latent: Optional[torch.Tensor], *, num_tokens: int = 64,
                           eps: float = 1e-6) -> Optional[torch.Tensor]:
    """[B, F, C] latents -> [B, num_tokens, C]: standardised over time per
    channel, average-pooled to ``num_tokens`` steps."""
    if audio_latent is None or audio_latent.numel() == 0:
        return None
    if audio_latent.dim() != 3:
        raise ValueError(f"audio_latent must be [B,F,C], got {tuple(audio_latent.shape)}")
    x = _standardize(audio_latent.detach().float().transpose(1, 2), (-1,), eps)
    return F.adaptive_avg_pool1d(x, max(1, int(num_tokens))).transpose(1, 2).contiguous()


def _channel_stats(latent: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per (batch, channel) mean and population std over frames and pixels."""
    x = latent.detach().float()
    return x.mean(dim=(1, 3, 4)), x.std(dim=(1, 3, 4), unbiased=False).clamp_min(eps)


def _lowfreq_proto(latent: torch.Tensor, grid: int) -> torch.Tensor:
    """[B, C, g, g]: the frame mean average-pooled to a g x g grid."""
    g = max(1, int(grid))
    return F.adaptive_avg_pool2d(latent.detach().float().mean(dim=1), (g, g))


def _renorm_channels(latent: torch.Tensor, ref: Tuple[torch.Tensor, torch.Tensor], alpha: float,
                     eps: float) -> torch.Tensor:
    """Blend ``alpha`` of the latents moved to the reference channel statistics."""
    alpha = _unit(alpha)
    if alpha <= 0.0:
        return latent
    mu, sd = _channel_stats(latent, eps)
    rmu = ref[0].to(device=latent.device, dtype=torch.float32)
    rsd = ref[1].to(device=latent.device, dtype=torch.float32).clamp_min(eps)
    bc = lambda t: t[:, None, :, None, None]
    x = latent.float()
    moved = (x - bc(mu)) / bc(sd).clamp_min(eps) * bc(rsd) + bc(rmu)
    return (x * (1.0 - alpha) + moved * alpha).to(latent.dtype)


def _pull_lowfreq(latent: torch.Tensor, proto: Optional[torch.Tensor], alpha: float, max_correction: float,
                  eps: float) -> torch.Tensor:
    """Add ``alpha`` of the (clamped, bilinearly upsampled) difference between
    a target low-frequency prototype and the latents' own."""
    alpha = _unit(alpha)
    if alpha <= 0.0 or proto is None:
        return latent
    delta = proto.to(device=latent.device, dtype=torch.float32) - _lowfreq_proto(latent, int(proto.shape[-1]))
    if max_correction > 0.0:
        lim = _channel_stats(latent, eps)[1].float().mean(dim=0).view(1, -1, 1, 1) * float(max_correction)
        delta = torch.maximum(torch.minimum(delta, lim), -lim)
    delta = F.interpolate(delta, size=tuple(latent.shape[-2:]), mode="bilinear", align_corners=False)
    return (latent.float() + alpha * delta[:, None]).to(latent.dtype)


def apply_color_memory_snapshot(video_latent: Optional[torch.Tensor],
                                snapshot: Optional[Dict[str, Any]]) -> Optional[torch.Tensor]:
    """Colour correction of generated latents from a memory snapshot
    (channel statistics, then the low-frequency prototype)."""
    if video_latent is None or not snapshot:
        return video_latent
    eps = float(snapshot.get("eps", 1e-6))
    out = video_latent
    if float(snapshot.get("color_alpha", 0.0)) > 0.0 and snapshot.get("color_stats") is not None:
        out = _renorm_channels(out, snapshot["color_stats"], float(snapshot["color_alpha"]), eps)
    if float(snapshot.get("color_proto_alpha", 0.0)) > 0.0:
        out = _pull_lowfreq(out, snapshot.get("color_proto"), float(snapshot["color_proto_alpha"]),
                            float(snapshot.get("color_max_correction", 0.5)), eps)
    return out


def _stats_drift(stats, anchor, eps: float) -> float:
    """Mean |Δmean| / anchor std plus 0.1 x mean |log(std ratio)|."""
    mu, sd = stats
    amu, asd = anchor[0].to(mu.device).float(), anchor[1].to(sd.device).float().clamp_min(eps)
    mean_term = ((mu.float() - amu).abs() / asd).mean()
    std_term = torch.log(sd.float().clamp_min(eps) / asd).abs().mean()
    return float((mean_term + 0.1 * std_term).detach().cpu())


def _token_cosine(current: torch.Tensor, anchor: torch.Tensor, eps: float) -> float:
    """Mean over the batch of the cosine between the flattened token grids
    (the common leading tokens when the counts differ)."""
    cur = current.detach().float()
    anc = anchor.detach().to(device=cur.device, dtype=torch.float32)
    if cur.dim() != 3 or anc.dim() != 3:
        return 1.0
    n = min(cur.shape[1], anc.shape[1])
    if n <= 0:
        return 1.0
    a = F.normalize(cur[:, :n].flatten(1), dim=-1, eps=eps)
    b = F.normalize(anc[:, :n].flatten(1), dim=-1, eps=eps)
    return float((a * b).sum(-1).mean().detach().cpu())


def _gate(score: float, threshold: float, temperature: float, floor: float) -> float:
    """floor + (1 - floor) * sigmoid((score - threshold) / temperature); a
    step at the threshold when the temperature is 0."""
    floor = _unit(floor)
    if temperature <= 0.0:
        return 1.0 if score >= threshold else floor
    z = (float(score) - float(threshold)) / max(float(temperature), 1e-6)
    s = 1.0 if z >= 50.0 else 0.0 if z <= -50.0 else 1.0 / (1.0 + math.exp(-z))
    return floor + (1.0 - floor) * s


def _blend(prev: Optional[torch.Tensor], anchor: Optional[torch.Tensor], cur: torch.Tensor, beta: float,
           tether: float) -> torch.Tensor:
    """EMA step prev (1 - beta) + cur beta, then pulled ``tether`` of the way
    back to the anchor; the first step takes the current tokens."""
    cur = cur.detach().contiguous()
    if prev is None:
        return cur.clone()
    beta, tether = _unit(beta), _unit(tether)
    out = prev.detach().to(device=cur.device, dtype=cur.dtype) * (1.0 - beta) + cur * beta
    if anchor is not None and tether > 0.0:
        out = out * (1.0 - tether) + anchor.detach().to(device=cur.device, dtype=cur.dtype) * tether
    return out.detach().contiguous()


@dataclass
class LearnedMemoryState:
    """EMA memory of generated chunks (video tokens, audio tokens, colour
    statistics) with a frozen first-chunk anchor; field names and defaults
    of learned_memory.py:252-277."""
    enabled: bool = False
    video_downsample: int = 4
    audio_tokens: int = 64
    video_beta: float = 0.15
    audio_beta: float = 0.10
    video_anchor_tether: float = 0.20
    audio_anchor_tether: float = 0.10
    identity_anchor_enabled: bool = False
    identity_anchor_scale: float = 1.0
    drift_gate_enabled: bool = False
    drift_gate_threshold: float = 0.05
    drift_gate_temperature: float = 0.10
    drift_gate_min: float = 0.10
    drift_gate_apply_to_color: bool = True
    color_enabled: bool = False
    color_alpha: float = 0.0
    color_proto_alpha: float = 0.0
    color_update_beta: float = 0.05
    color_anchor_tether: float = 0.40
    color_proto_grid: int = 4
    color_drift_threshold: float = 2.5
    color_max_correction: float = 0.5
    color_film_enabled: bool = False
    reference_anchor_enabled: bool = False
    eps: float = 1e-6
    # evolving state
    video: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    audio: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    video_anchor: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    audio_anchor: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    color_stats: Optional[Tuple[torch.Tensor, torch.Tensor]] = field(default=None, init=False, repr=False)
    color_anchor_stats: Optional[Tuple[torch.Tensor, torch.Tensor]] = field(default=None, init=False, repr=False)
    color_proto: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    color_anchor_proto: Optional[torch.Tensor] = field(default=None, init=False, repr=False)
    color_last_drift: Optional[float] = field(default=None, init=False)
    color_last_updated: bool = field(default=False, init=False)
    video_last_anchor_cosine: Optional[float] = field(default=None, init=False)
    video_last_update_gate: Optional[float] = field(default=None, init=False)
    reference_initialized: bool = field(default=False, init=False)

    def __post_init__(self) -> None:
        for name in ("video_beta", "audio_beta", "video_anchor_tether", "audio_anchor_tether", "drift_gate_min",
                     "color_alpha", "color_proto_alpha", "color_update_beta", "color_anchor_tether"):
            setattr(self, name, _unit(getattr(self, name)))
        self.video_downsample = max(1, int(self.video_downsample))
        self.audio_tokens = max(1, int(self.audio_tokens))
        self.color_proto_grid = max(1, int(self.color_proto_grid))
        self.identity_anchor_scale = max(0.0, float(self.identity_anchor_scale))
        self.drift_gate_temperature = max(0.0, float(self.drift_gate_temperature))
        self.color_max_correction = max(0.0, float(self.color_max_correction))
        self.color_enabled = bool(self.color_enabled or self.color_film_enabled)

    def reset(self) -> None:
        self.video = self.audio = self.video_anchor = self.audio_anchor = None
        self.color_stats = self.color_anchor_stats = None
        self.color_proto = self.color_anchor_proto = None
        self.color_last_drift = self.video_last_anchor_cosine = self.video_last_update_gate = None
        self.color_last_updated = False
        self.reference_initialized = False

    # ---- summaries of one chunk ----
    def _video_tokens(self, video_latent):
        return summarize_video_memory(video_latent, downsample=self.video_downsample, eps=self.eps)

    def _audio_tokens(self, audio_latent):
        return summarize_audio_memory(audio_latent, num_tokens=self.audio_tokens, eps=self.eps)

    def _color_of(self, video_latent):
        stats = tuple(t.detach().contiguous().clone() for t in _channel_stats(video_latent, self.eps))
        return stats, _lowfreq_proto(video_latent, self.color_proto_grid).detach().contiguous().clone()

    # ---- colour memory ----
    def color_snapshot(self) -> Optional[Dict[str, Any]]:
        if not self.color_enabled or self.color_stats is None or (
                self.color_alpha <= 0.0 and self.color_proto_alpha <= 0.0):
            return None
        return {"color_stats": tuple(t.detach() for t in self.color_stats),
                "color_proto": None if self.color_proto is None else self.color_proto.detach(),
                "color_alpha": self.color_alpha, "color_proto_alpha": self.color_proto_alpha,
                "color_max_correction": self.color_max_correction, "eps": self.eps}

    def apply_color_memory(self, video_latent: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        return apply_color_memory_snapshot(video_latent, self.color_snapshot())

    def _update_color_memory(self, video_latent: Optional[torch.Tensor], *, update_scale: float = 1.0) -> None:
        if not self.color_enabled or video_latent is None or video_latent.numel() == 0:
            return
        stats, proto = self._color_of(video_latent)
        if self.color_anchor_stats is None:
            self.color_anchor_stats, self.color_anchor_proto = stats, proto
            self.color_stats, self.color_proto = tuple(t.clone() for t in stats), proto.clone()
            self.color_last_drift, self.color_last_updated = 0.0, True
            return
        self.color_last_drift = _stats_drift(stats, self.color_anchor_stats, self.eps)
        beta = self.color_update_beta * _unit(update_scale)
        if (self.color_drift_threshold > 0.0 and self.color_last_drift > self.color_drift_threshold) or beta <= 0.0:
            self.color_last_updated = False
            return
        tether = self.color_anchor_tether
        prev = self.color_stats or stats
        mixed = [(1.0 - beta) * o.to(n.device) + beta * n for o, n in zip(prev, stats)]
        if tether > 0.0:
            mixed = [(1.0 - tether) * m + tether * a.to(m.device) for m, a in zip(mixed, self.color_anchor_stats)]
        self.color_stats = tuple(t.detach().contiguous() for t in mixed)
        p = (1.0 - beta) * (self.color_proto if self.color_proto is not None else proto).to(proto.device) \
            + beta * proto
        if tether > 0.0 and self.color_anchor_proto is not None:
            p = (1.0 - tether) * p + tether * self.color_anchor_proto.to(proto.device)
        self.color_proto = p.detach().contiguous()
        self.color_last_updated = True

    def _color_condition_vector(self) -> Optional[torch.Tensor]:
        """[B, 4C]: mean, log std, anchor mean, anchor log std."""
        if not self.color_film_enabled or self.color_stats is None:
            return None
        mu, sd = self.color_stats
        amu, asd = self.color_anchor_stats if self.color_anchor_stats is not None else (mu, sd)
        return torch.cat([mu.detach(), sd.detach().clamp_min(self.eps).log(), amu.detach().to(mu.device),
                          asd.detach().to(sd.device).clamp_min(self.eps).log()], dim=-1)

    # ---- anchor, update, conditioning ----
    def set_reference(self, video_latent: Optional[torch.Tensor], audio_latent: Optional[torch.Tensor] = None):
        """Freeze the first visible chunk as the anchor (once)."""
        if not (self.enabled and self.reference_anchor_enabled) or self.reference_initialized:
            return
        v = self._video_tokens(video_latent)
        if v is not None:
            self.video_anchor = v.detach().contiguous().clone()
            if self.video is None:
                self.video = self.video_anchor.clone()
            self.video_last_anchor_cosine = self.video_last_update_gate = 1.0
        a = self._audio_tokens(audio_latent)
        if a is not None:
            self.audio_anchor = a.detach().contiguous().clone()
            if self.audio is None:
                self.audio = self.audio_anchor.clone()
        if self.color_enabled and video_latent is not None and video_latent.numel() > 0:
            stats, proto = self._color_of(video_latent)
            self.color_anchor_stats, self.color_anchor_proto = stats, proto
            if self.color_stats is None:
                self.color_stats = tuple(t.clone() for t in stats)
            if self.color_proto is None:
                self.color_proto = proto.clone()
            self.color_last_drift, self.color_last_updated = 0.0, True
        if v is not None or a is not None:
            self.reference_initialized = True

    def _video_update_gate(self, tokens: torch.Tensor) -> float:
        if not self.drift_gate_enabled or self.video_anchor is None:
            self.video_last_anchor_cosine, self.video_last_update_gate = None, 1.0
            return 1.0
        score = _token_cosine(tokens, self.video_anchor, self.eps)
        g = _gate(score, self.drift_gate_threshold, self.drift_gate_temperature, self.drift_gate_min)
        self.video_last_anchor_cosine, self.video_last_update_gate = score, g
        return g

    def update(self, video_latent: Optional[torch.Tensor], audio_latent: Optional[torch.Tensor] = None) -> None:
        """Fold one generated chunk into the memory."""
        if not self.enabled:
            return
        gate = 1.0
        v = self._video_tokens(video_latent)
        if v is not None:
            if self.video_anchor is None:
                self.video_anchor = v.detach().contiguous().clone()
                self.video_last_anchor_cosine = self.video_last_update_gate = 1.0
            else:
                gate = self._video_update_gate(v)
            self.video = _blend(self.video, self.video_anchor, v, self.video_beta * gate, self.video_anchor_tether)
        a = self._audio_tokens(audio_latent)
        if a is not None:
            if self.audio_anchor is None:
                self.audio_anchor = a.detach().contiguous().clone()
            self.audio = _blend(self.audio, self.audio_anchor, a, self.audio_beta, self.audio_anchor_tether)
        self._update_color_memory(video_latent, update_scale=gate if self.drift_gate_apply_to_color else 1.0)

    def _video_condition_memory(self) -> Optional[torch.Tensor]:
        parts = []
        if self.identity_anchor_enabled and self.video_anchor is not None:
            anchor = self.video_anchor.detach()
            parts.append(anchor * self.identity_anchor_scale if self.identity_anchor_scale != 1.0 else anchor)
        if self.video is not None:
            parts.append(self.video)
        if not parts:
            return None
        return parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)

    def with_conditional_memory(self, conditional_dict: Dict[str, Any], *, device=None,
                                dtype=None) -> Dict[str, Any]:
        """``conditional_dict`` plus learned_memory_video / _audio / _color."""
        vm = self._video_condition_memory()
        if not self.enabled or (vm is None and self.audio is None):
            return conditional_dict
        move = (lambda t: t.to(device=device or t.device, dtype=dtype or t.dtype)) \
            if (device is not None or dtype is not None) else (lambda t: t)
        out = dict(conditional_dict)
        if vm is not None:
            out["learned_memory_video"] = move(vm)
        if self.audio is not None:
            out["learned_memory_audio"] = move(self.audio)
        color = self._color_condition_vector()
        if color is not None:
            out["learned_memory_color"] = move(color)
        return out


class StreamingMemory(LearnedMemoryState):
    """The production settings (taomate/inference/memory.py:4-29): identity
    anchor + EMA video tokens, drift gate, colour memory and FiLM."""

    def __init__(self) -> None:
        super().__init__(enabled=True, video_downsample=4, audio_tokens=64, video_beta=0.15, audio_beta=0.10,
                         video_anchor_tether=0.20, audio_anchor_tether=0.10, identity_anchor_enabled=True,
                         identity_anchor_scale=1.0, reference_anchor_enabled=True, drift_gate_enabled=True,
                         drift_gate_threshold=0.05, drift_gate_temperature=0.10, drift_gate_min=0.10,
                         drift_gate_apply_to_color=True, color_enabled=True, color_alpha=0.04,
                         color_proto_alpha=0.015, color_update_beta=0.03, color_anchor_tether=0.60,
                         color_proto_grid=4, color_drift_threshold=2.0, color_max_correction=0.35,
                         color_film_enabled=True)
