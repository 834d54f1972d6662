"""Learned long memory: detached summaries of the generated latents that
condition later chunks through the blocks' memory adapters (``taomate_amd.dit``).

Design.  The memory is a value: ``MemoryState``, a frozen record of three
tracks (video tokens, audio tokens, colour statistics), each an evolving
summary beside the frozen anchor it is tethered to.  Every operation is a pure
function from (settings, state, chunk) to a new state.  The decisions are
tensor arithmetic on the latents' device:
* the drift gate's sigmoid;
* the colour-drift threshold;
* the first-chunk initialisation.

Folding a chunk in therefore queues a few small kernels and never waits for
the GPU. The reference reads those values back as Python floats. Here they are
read only by the diagnostic properties. ``LearnedMemoryState`` is the mutable
handle the runtime holds. It carries the reference's class name, settings
fields and defaults, and methods (``set_reference``, ``update``,
``apply_color_memory``, ``with_conditional_memory``).

Behaviour follows taomate/runtime_support/learned_memory.py: token summaries
:192-229, EMA with an anchor tether :231-249, drift gate :120-166 and
:414-428, colour memory :35-103, :169-189, :430-487, the state's update order
:252-591, with the streaming settings of taomate/inference/memory.py:4-29.
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn.functional as F

__all__ = ["LearnedMemoryState", "StreamingMemory", "MemoryState", "summarize_video_memory",
           "summarize_audio_memory", "apply_color_memory_snapshot"]

Tensor = torch.Tensor


# ---------------------------------------------------------------------------
# summaries of one chunk
# ---------------------------------------------------------------------------

def _zscore(x: Tensor, dims: Tuple[int, ...], eps: float) -> Tensor:
    """Zero mean, unit population std over ``dims`` (std floored at eps)."""
    centred = x - x.mean(dim=dims, keepdim=True)
    return centred / x.std(dim=dims, keepdim=True, unbiased=False).clamp_min(eps)


def summarize_video_memory(video_latent: Optional[Tensor], *, downsample: int = 4,
                           eps: float = 1e-6) -> Optional[Tensor]:
    """[B, F, C, H, W] -> [B, (H/d)(W/d), C]: the chunk's mean frame, z-scored
    per channel over the spatial grid, average-pooled by d."""
    if video_latent is None or video_latent.numel() == 0:
        return None
    if video_latent.dim() != 5:
        raise ValueError(f"video_latent must be [B,F,C,H,W], got {tuple(video_latent.shape)}")
    frame = _zscore(video_latent.detach().float().mean(dim=1), (2, 3), eps)
    d = max(1, int(downsample))
    grid = (max(1, frame.shape[2] // d), max(1, frame.shape[3] // d))
    return F.adaptive_avg_pool2d(frame, grid).flatten(2).transpose(1, 2).contiguous()


def summarize_audio_memory(audio_latent: Optional[Tensor], *, num_tokens: int = 64,
                           eps: float = 1e-6) -> Optional[Tensor]:
    """[B, F, C] -> [B, num_tokens, C]: z-scored per channel over time,
    average-pooled to ``num_tokens`` steps."""
    if audio_latent is None or audio_latent.numel() == 0:
        return None
    if audio_latent.dim() != 3:
        raise ValueError(f"audio_latent must be [B,F,C], got {tuple(audio_latent.shape)}")
    seq = _zscore(audio_latent.detach().float().transpose(1, 2), (2,), eps)
    return F.adaptive_avg_pool1d(seq, max(1, int(num_tokens))).transpose(1, 2).contiguous()


def color_summary(video_latent: Tensor, grid: int, eps: float) -> Tuple[Tensor, Tensor, Tensor]:
    """(channel mean [B, C], channel population std [B, C], low-frequency
    prototype [B, C, g, g]) of a [B, F, C, H, W] chunk."""
    x = video_latent.detach().float()
    g = max(1, int(grid))
    return (x.mean(dim=(1, 3, 4)), x.std(dim=(1, 3, 4), unbiased=False).clamp_min(eps),
            F.adaptive_avg_pool2d(x.mean(dim=1), (g, g)))


# ---------------------------------------------------------------------------
# state
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class Track:
    """An evolving summary and the anchor it is tethered to."""
    value: Optional[Tensor] = None
    anchor: Optional[Tensor] = None


@dataclass(frozen=True)
class ColorTrack:
    """Evolving and anchor colour statistics and low-frequency prototypes,
    with the last chunk's drift score and whether it was folded in (0-dim
    device tensors)."""
    mean: Optional[Tensor] = None
    std: Optional[Tensor] = None
    proto: Optional[Tensor] = None
    anchor_mean: Optional[Tensor] = None
    anchor_std: Optional[Tensor] = None
    anchor_proto: Optional[Tensor] = None
    drift: Optional[Tensor] = None
    updated: Optional[Tensor] = None


@dataclass(frozen=True)
class MemoryState:
    video: Track = Track()
    audio: Track = Track()
    color: ColorTrack = ColorTrack()
    referenced: bool = False
    video_cosine: Optional[Tensor] = None    # last chunk's pooled cosine with the anchor
    video_gate: Optional[Tensor] = None      # last chunk's update gate


# ---------------------------------------------------------------------------
# pure operations
# ---------------------------------------------------------------------------

def _u(x):
    """Clamp to [0, 1] (floats and tensors)."""
    return x.clamp(0.0, 1.0) if torch.is_tensor(x) else min(1.0, max(0.0, float(x)))


def ema_toward(prev: Optional[Tensor], current: Tensor, beta, anchor: Optional[Tensor], tether: float) -> Tensor:
    """One EMA step of weight ``beta`` toward ``current`` then ``tether`` of
    the way back to ``anchor``; with no history the current value."""
    cur = current.detach()
    if prev is None:
        return cur.clone()
    b = _u(beta)
    out = prev.to(cur) * (1.0 - b) + cur * b
    t = _u(tether)
    if anchor is not None and t > 0.0:
        out = out * (1.0 - t) + anchor.to(cur) * t
    return out.contiguous()


def pooled_cosine(tokens: Tensor, anchor: Tensor, eps: float) -> Tensor:
    """Batch mean of the cosine between the flattened token grids (their
    common leading tokens), a 0-dim tensor on the tokens' device."""
    n = min(tokens.shape[1], anchor.shape[1])
    a = F.normalize(tokens[:, :n].float().flatten(1), dim=-1, eps=eps)
    b = F.normalize(anchor[:, :n].to(tokens).float().flatten(1), dim=-1, eps=eps)
    return (a * b).sum(-1).mean()


def soft_gate(score: Tensor, threshold: float, temperature: float, floor: float) -> Tensor:
    """floor + (1 - floor) sigmoid((score - threshold) / temperature), with
    the sigmoid taken as exactly 0 or 1 once its argument passes -50 / 50, and
    a step at the threshold for temperature 0."""
    lo = _u(floor)
    if temperature <= 0.0:
        return torch.where(score >= threshold, torch.ones_like(score), torch.full_like(score, lo))
    z = (score - threshold) / max(float(temperature), 1e-6)
    sig = torch.where(z >= 50.0, torch.ones_like(z), torch.where(z <= -50.0, torch.zeros_like(z), torch.sigmoid(z)))
    return lo + (1.0 - lo) * sig


def color_drift(mean: Tensor, std: Tensor, anchor_mean: Tensor, anchor_std: Tensor, eps: float) -> Tensor:
    """Mean |mean shift| in anchor stds plus 0.1 mean |log std ratio| (0-dim)."""
    asd = anchor_std.float().clamp_min(eps)
    shift = ((mean.float() - anchor_mean.float()).abs() / asd).mean()
    spread = (std.float().clamp_min(eps) / asd).log().abs().mean()
    return shift + 0.1 * spread


def _fold_color(s, col: ColorTrack, video: Tensor, scale) -> ColorTrack:
    """The chunk's colour statistics folded into the colour track: the first
    chunk becomes the anchor; later chunks move the statistics by
    color_update_beta * scale, unless their drift from the anchor passes the
    threshold, then the tether pulls back toward the anchor."""
    mean, std, proto = color_summary(video, s.color_proto_grid, s.eps)
    if col.anchor_mean is None:
        z = torch.zeros((), device=mean.device)
        return ColorTrack(mean.clone(), std.clone(), proto.clone(), mean, std, proto, z, torch.ones((), dtype=torch.bool,
                                                                                                      device=mean.device))
    drift = color_drift(mean, std, col.anchor_mean, col.anchor_std, s.eps)
    beta = s.color_update_beta * _u(scale)
    beta = beta if torch.is_tensor(beta) else torch.tensor(float(beta), device=mean.device)
    skip = beta <= 0.0
    if s.color_drift_threshold > 0.0:
        skip = skip | (drift > s.color_drift_threshold)
    t = s.color_anchor_tether

    def move(old, new, anc):
        mixed = old.to(new) * (1.0 - beta) + new * beta
        if t > 0.0:
            mixed = mixed * (1.0 - t) + anc.to(new) * t
        return torch.where(skip, old.to(new), mixed)

    prev_m = col.mean if col.mean is not None else mean
    prev_s = col.std if col.std is not None else std
    prev_p = col.proto if col.proto is not None else proto
    return dataclasses.replace(col, mean=move(prev_m, mean, col.anchor_mean), std=move(prev_s, std, col.anchor_std),
                               proto=move(prev_p, proto, col.anchor_proto), drift=drift, updated=~skip)


def anchored(s, st: MemoryState, video: Optional[Tensor], audio: Optional[Tensor]) -> MemoryState:
    """The first visible chunk frozen as the anchor of every track (once);
    an empty track also starts from it."""
    if not (s.enabled and s.reference_anchor_enabled) or st.referenced:
        return st
    v = summarize_video_memory(video, downsample=s.video_downsample, eps=s.eps)
    a = summarize_audio_memory(audio, num_tokens=s.audio_tokens, eps=s.eps)
    out = st
    if v is not None:
        one = torch.ones((), device=v.device)
        out = dataclasses.replace(out, video=Track(out.video.value if out.video.value is not None else v.clone(), v),
                                  video_cosine=one, video_gate=one)
    if a is not None:
        out = dataclasses.replace(out, audio=Track(out.audio.value if out.audio.value is not None else a.clone(), a))
    if s.color_enabled and video is not None and video.numel() > 0:
        m, sd, p = color_summary(video, s.color_proto_grid, s.eps)
        c = out.color
        out = dataclasses.replace(out, color=ColorTrack(
            c.mean if c.mean is not None else m.clone(), c.std if c.std is not None else sd.clone(),
            c.proto if c.proto is not None else p.clone(), m, sd, p, torch.zeros((), device=m.device),
            torch.ones((), dtype=torch.bool, device=m.device)))
    return dataclasses.replace(out, referenced=v is not None or a is not None)


def observe(s, st: MemoryState, video: Optional[Tensor], audio: Optional[Tensor]) -> MemoryState:
    """One generated chunk folded into the memory: video tokens (EMA gated by
    the drift from the anchor), audio tokens, then the colour statistics."""
    if not s.enabled:
        return st
    out = st
    gate = 1.0
    v = summarize_video_memory(video, downsample=s.video_downsample, eps=s.eps)
    if v is not None:
        if out.video.anchor is None:
            one = torch.ones((), device=v.device)
            out = dataclasses.replace(out, video=Track(out.video.value, v), video_cosine=one, video_gate=one)
        elif s.drift_gate_enabled:
            cos = pooled_cosine(v, out.video.anchor, s.eps)
            gate = soft_gate(cos, s.drift_gate_threshold, s.drift_gate_temperature, s.drift_gate_min)
            out = dataclasses.replace(out, video_cosine=cos, video_gate=gate)
        else:
            out = dataclasses.replace(out, video_cosine=None, video_gate=torch.ones((), device=v.device))
        out = dataclasses.replace(out, video=Track(
            ema_toward(out.video.value, v, s.video_beta * gate, out.video.anchor, s.video_anchor_tether),
            out.video.anchor))
    a = summarize_audio_memory(audio, num_tokens=s.audio_tokens, eps=s.eps)
    if a is not None:
        anchor = out.audio.anchor if out.audio.anchor is not None else a
        out = dataclasses.replace(out, audio=Track(
            ema_toward(out.audio.value, a, s.audio_beta, anchor, s.audio_anchor_tether), anchor))
    if s.color_enabled and video is not None and video.numel() > 0:
        out = dataclasses.replace(out, color=_fold_color(s, out.color, video,
                                                         gate if s.drift_gate_apply_to_color else 1.0))
    return out


def conditioning(s, st: MemoryState) -> Dict[str, Tensor]:
    """learned_memory_video ([identity anchor |] evolving tokens),
    learned_memory_audio and learned_memory_color ([mean, log std, anchor
    mean, anchor log std]) of the state; empty when there is nothing."""
    out: Dict[str, Tensor] = {}
    parts = []
    if s.identity_anchor_enabled and st.video.anchor is not None:
        parts.append(st.video.anchor * s.identity_anchor_scale if s.identity_anchor_scale != 1.0
                     else st.video.anchor)
    if st.video.value is not None:
        parts.append(st.video.value)
    if parts:
        out["learned_memory_video"] = torch.cat(parts, dim=1) if len(parts) > 1 else parts[0]
    if st.audio.value is not None:
        out["learned_memory_audio"] = st.audio.value
    c = st.color
    if s.color_film_enabled and c.mean is not None:
        am = c.anchor_mean if c.anchor_mean is not None else c.mean
        asd = c.anchor_std if c.anchor_std is not None else c.std
        out["learned_memory_color"] = torch.cat([c.mean, c.std.clamp_min(s.eps).log(), am.to(c.mean),
                                                 asd.to(c.std).clamp_min(s.eps).log()], dim=-1)
    return out


def _to_reference_stats(latent: Tensor, mean: Tensor, std: Tensor, alpha: float, eps: float) -> Tensor:
    """``alpha`` of the latents moved onto the given per-channel statistics."""
    cm, cs, _ = color_summary(latent, 1, eps)
    shape = (latent.shape[0], 1, latent.shape[2], 1, 1)
    x = latent.float()
    target = (x - cm.view(shape)) / cs.view(shape) * std.to(x).clamp_min(eps).view(shape) + mean.to(x).view(shape)
    return torch.lerp(x, target, alpha).to(latent.dtype)


def _toward_prototype(latent: Tensor, proto: Tensor, alpha: float, max_correction: float, eps: float) -> Tensor:
    """Add ``alpha`` of the prototype difference (clamped per channel to
    max_correction batch-mean stds, upsampled bilinearly) to every frame."""
    _, cs, own = color_summary(latent, proto.shape[-1], eps)
    delta = proto.to(own) - own
    if max_correction > 0.0:
        lim = (cs.mean(dim=0) * float(max_correction)).view(1, -1, 1, 1)
        delta = torch.clamp(delta, -lim, lim)
    delta = F.interpolate(delta, size=tuple(latent.shape[-2:]), mode="bilinear", align_corners=False)
    return (latent.float() + alpha * delta.unsqueeze(1)).to(latent.dtype)


def color_corrected(s, st: MemoryState, video: Optional[Tensor]) -> Optional[Tensor]:
    """The chunk's colours pulled toward the colour memory: channel
    statistics (color_alpha), then the low-frequency prototype
    (color_proto_alpha, limited by color_max_correction)."""
    c = st.color
    if video is None or not s.color_enabled or c.mean is None or (s.color_alpha <= 0.0 and s.color_proto_alpha <= 0.0):
        return video
    out = video
    if s.color_alpha > 0.0:
        out = _to_reference_stats(out, c.mean, c.std, s.color_alpha, s.eps)
    if s.color_proto_alpha > 0.0 and c.proto is not None:
        out = _toward_prototype(out, c.proto, s.color_proto_alpha, s.color_max_correction, s.eps)
    return out


def apply_color_memory_snapshot(video_latent: Optional[Tensor],
                                snapshot: Optional[Dict[str, Any]]) -> Optional[Tensor]:
    """Colour correction from a detached snapshot (``LearnedMemoryState.color_snapshot``)."""
    if video_latent is None or not snapshot:
        return video_latent
    eps = float(snapshot.get("eps", 1e-6))
    out = video_latent
    stats = snapshot.get("color_stats")
    if float(snapshot.get("color_alpha", 0.0)) > 0.0 and stats is not None:
        out = _to_reference_stats(out, stats[0], stats[1], _u(snapshot["color_alpha"]), eps)
    if float(snapshot.get("color_proto_alpha", 0.0)) > 0.0 and snapshot.get("color_proto") is not None:
        out = _toward_prototype(out, snapshot["color_proto"], _u(snapshot["color_proto_alpha"]),
                                float(snapshot.get("color_max_correction", 0.5)), eps)
    return out


# ---------------------------------------------------------------------------
# the mutable handle
# ---------------------------------------------------------------------------

def _state_attr(path: str, doc: str):
    """A read/write attribute of the handle that lives inside the frozen state."""
    head, _, tail = path.partition(".")

    def get(self):
        v = getattr(self.state, head)
        return getattr(v, tail) if tail else v

    def put(self, value):
        if tail:
            part = dataclasses.replace(getattr(self.state, head), **{tail: value})
            self.state = dataclasses.replace(self.state, **{head: part})
        else:
            self.state = dataclasses.replace(self.state, **{head: value})
    return property(get, put, doc=doc)


def _pair_attr(head: str, first: str, second: str, doc: str):
    def get(self):
        c = getattr(self.state, head)
        a, b = getattr(c, first), getattr(c, second)
        return None if a is None else (a, b)

    def put(self, value):
        a, b = (None, None) if value is None else value
        part = dataclasses.replace(getattr(self.state, head), **{first: a, second: b})
        self.state = dataclasses.replace(self.state, **{head: part})
    return property(get, put, doc=doc)


def _scalar_attr(path: str, as_bool: bool, doc: str):
    """A diagnostic scalar: the device tensor read back on access."""
    inner = _state_attr(path, doc)

    def get(self):
        v = inner.fget(self)
        if v is None:
            return None
        return bool(v) if as_bool else float(v)

    def put(self, value):
        if value is None:
            inner.fset(self, None)
        else:
            inner.fset(self, torch.tensor(bool(value) if as_bool else float(value)))
    return property(get, put, doc=doc)


@dataclass
class LearnedMemoryState:
    """The memory handle with the reference's settings fields and defaults
    (learned_memory.py:252-277); the state itself is ``state``, a
    ``MemoryState`` replaced by every update."""
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
    state: MemoryState = field(default_factory=MemoryState, init=False, repr=False)

    def __post_init__(self) -> None:
        for name in ("video_beta", "audio_beta", "video_anchor_tether", "audio_anchor_tether", "drift_gate_min",
                     "color_alpha", "color_proto_alpha", "color_update_beta", "color_anchor_tether"):
            setattr(self, name, _u(getattr(self, name)))
        self.video_downsample = max(1, int(self.video_downsample))
        self.audio_tokens = max(1, int(self.audio_tokens))
        self.color_proto_grid = max(1, int(self.color_proto_grid))
        self.identity_anchor_scale = max(0.0, float(self.identity_anchor_scale))
        self.drift_gate_temperature = max(0.0, float(self.drift_gate_temperature))
        self.color_max_correction = max(0.0, float(self.color_max_correction))
        self.color_enabled = bool(self.color_enabled or self.color_film_enabled)

    # the state under the reference's attribute names (the prefix-state file uses them)
    video = _state_attr("video.value", "evolving video tokens [B, N, C]")
    audio = _state_attr("audio.value", "evolving audio tokens [B, T, C]")
    video_anchor = _state_attr("video.anchor", "anchor video tokens")
    audio_anchor = _state_attr("audio.anchor", "anchor audio tokens")
    color_proto = _state_attr("color.proto", "evolving low-frequency prototype [B, C, g, g]")
    color_anchor_proto = _state_attr("color.anchor_proto", "anchor prototype")
    color_stats = _pair_attr("color", "mean", "std", "evolving (channel mean, channel std)")
    color_anchor_stats = _pair_attr("color", "anchor_mean", "anchor_std", "anchor (channel mean, channel std)")
    reference_initialized = _state_attr("referenced", "whether set_reference took effect")
    color_last_drift = _scalar_attr("color.drift", False, "last chunk's colour drift from the anchor")
    color_last_updated = _scalar_attr("color.updated", True, "whether the last chunk moved the colour memory")
    video_last_anchor_cosine = _scalar_attr("video_cosine", False, "last chunk's pooled cosine with the anchor")
    video_last_update_gate = _scalar_attr("video_gate", False, "last chunk's drift gate")

    def reset(self) -> None:
        self.state = MemoryState()

    def set_reference(self, video_latent: Optional[Tensor], audio_latent: Optional[Tensor] = None) -> None:
        self.state = anchored(self, self.state, video_latent, audio_latent)

    def update(self, video_latent: Optional[Tensor], audio_latent: Optional[Tensor] = None) -> None:
        self.state = observe(self, self.state, video_latent, audio_latent)

    def color_snapshot(self) -> Optional[Dict[str, Any]]:
        c = self.state.color
        if not self.color_enabled or c.mean is None or (self.color_alpha <= 0.0 and self.color_proto_alpha <= 0.0):
            return None
        return {"color_stats": (c.mean, c.std), "color_proto": c.proto, "color_alpha": self.color_alpha,
                "color_proto_alpha": self.color_proto_alpha, "color_max_correction": self.color_max_correction,
                "eps": self.eps}

    def apply_color_memory(self, video_latent: Optional[Tensor]) -> Optional[Tensor]:
        return color_corrected(self, self.state, video_latent)

    def with_conditional_memory(self, conditional_dict: Dict[str, Any], *, device=None,
                                dtype=None) -> Dict[str, Any]:
        """``conditional_dict`` plus the memory tensors (moved to ``device`` /
        ``dtype`` when given); unchanged when the memory is off or empty."""
        mem = conditioning(self, self.state) if self.enabled else {}
        if "learned_memory_video" not in mem and "learned_memory_audio" not in mem:
            return conditional_dict
        out = dict(conditional_dict)
        for k, v in mem.items():
            out[k] = v.to(device=device or v.device, dtype=dtype or v.dtype)
        return out


class StreamingMemory(LearnedMemoryState):
    """The streaming settings (taomate/inference/memory.py:4-29): identity
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
