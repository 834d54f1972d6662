"""float64 NumPy restatement of the learned long-memory state (oracle; test
infrastructure only).

Follows taomate/runtime_support/learned_memory.py:
  _normalize_spatial / _normalize_temporal      :23-32
  _channel_stats / _apply_channel_renorm        :35-65
  _lowfreq_proto / _apply_lowfreq_proto         :68-103
  _stats_drift_score / _pooled_cosine_score     :106-146
  _smooth_gate_from_score                       :149-166
  summarize_video_memory / _audio_memory        :192-229
  _ema_update                                   :231-249
  LearnedMemoryState.set_reference / update /
  _update_color_memory / with_conditional_memory  :356-591
Adaptive average pooling and bilinear resampling are written out from their
definitions (window [floor(i n / m), ceil((i + 1) n / m)); source coordinate
(i + 0.5) n / m - 0.5 clamped at 0, align_corners = False) rather than taken
from a library, so the product's PyTorch calls are checked against an
independent statement of the same arithmetic.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np


def _unit(x):
    return min(1.0, max(0.0, float(x)))


def adaptive_avg_pool_1d(x: np.ndarray, out: int) -> np.ndarray:
    """Last axis of length n pooled to ``out`` windows."""
    n = x.shape[-1]
    cols = []
    for i in range(out):
        a, b = (i * n) // out, -((-(i + 1) * n) // out)
        cols.append(x[..., a:b].mean(axis=-1))
    return np.stack(cols, axis=-1)


def adaptive_avg_pool_2d(x: np.ndarray, oh: int, ow: int) -> np.ndarray:
    return adaptive_avg_pool_1d(np.swapaxes(adaptive_avg_pool_1d(np.swapaxes(x, -1, -2), oh), -1, -2), ow)


def _bilinear_axis(x: np.ndarray, out: int) -> np.ndarray:
    """Resample the last axis (align_corners=False)."""
    n = x.shape[-1]
    res = np.empty(x.shape[:-1] + (out,))
    for i in range(out):
        src = max((i + 0.5) * n / out - 0.5, 0.0)
        i0 = min(int(math.floor(src)), n - 1)
        i1 = min(i0 + 1, n - 1)
        w = src - i0
        res[..., i] = x[..., i0] * (1.0 - w) + x[..., i1] * w
    return res


def bilinear(x: np.ndarray, oh: int, ow: int) -> np.ndarray:
    return _bilinear_axis(np.swapaxes(_bilinear_axis(np.swapaxes(x, -1, -2), oh), -1, -2), ow)


def _standardize(x: np.ndarray, axes, eps: float) -> np.ndarray:
    mu = x.mean(axis=axes, keepdims=True)
    sd = np.maximum(x.std(axis=axes, keepdims=True), eps)
    return (x - mu) / sd


def video_tokens(latent: np.ndarray, downsample: int = 4, eps: float = 1e-6) -> np.ndarray:
    """[B, F, C, H, W] -> [B, (H/d)(W/d), C]."""
    x = _standardize(latent.astype(np.float64).mean(axis=1), (-2, -1), eps)
    h, w = max(1, x.shape[-2] // downsample), max(1, x.shape[-1] // downsample)
    x = adaptive_avg_pool_2d(x, h, w)
    B, C = x.shape[:2]
    return x.reshape(B, C, h * w).transpose(0, 2, 1)


def audio_tokens(latent: np.ndarray, num_tokens: int = 64, eps: float = 1e-6) -> np.ndarray:
    """[B, F, C] -> [B, num_tokens, C]."""
    x = _standardize(latent.astype(np.float64).transpose(0, 2, 1), (-1,), eps)
    return adaptive_avg_pool_1d(x, num_tokens).transpose(0, 2, 1)


def channel_stats(latent: np.ndarray, eps: float) -> Tuple[np.ndarray, np.ndarray]:
    x = latent.astype(np.float64)
    return x.mean(axis=(1, 3, 4)), np.maximum(x.std(axis=(1, 3, 4)), eps)


def lowfreq_proto(latent: np.ndarray, grid: int) -> np.ndarray:
    return adaptive_avg_pool_2d(latent.astype(np.float64).mean(axis=1), grid, grid)


def apply_color(latent: np.ndarray, stats, proto, alpha: float, proto_alpha: float, max_corr: float,
                eps: float) -> np.ndarray:
    """_apply_channel_renorm then _apply_lowfreq_proto, in float64."""
    out = latent.astype(np.float64)
    if alpha > 0.0 and stats is not None:
        mu, sd = channel_stats(out, eps)
        rmu, rsd = stats[0], np.maximum(stats[1], eps)
        bc = lambda t: t[:, None, :, None, None]
        moved = (out - bc(mu)) / np.maximum(bc(sd), eps) * bc(rsd) + bc(rmu)
        out = out * (1.0 - alpha) + moved * alpha
    if proto_alpha > 0.0 and proto is not None:
        delta = proto - lowfreq_proto(out, proto.shape[-1])
        if max_corr > 0.0:
            lim = channel_stats(out, eps)[1].mean(axis=0).reshape(1, -1, 1, 1) * max_corr
            delta = np.maximum(np.minimum(delta, lim), -lim)
        delta = bilinear(delta, out.shape[-2], out.shape[-1])
        out = out + proto_alpha * delta[:, None]
    return out


def drift_score(stats, anchor, eps: float) -> float:
    mean_term = (np.abs(stats[0] - anchor[0]) / np.maximum(anchor[1], eps)).mean()
    std_term = np.abs(np.log(np.maximum(stats[1], eps) / np.maximum(anchor[1], eps))).mean()
    return float(mean_term + 0.1 * std_term)


def token_cosine(cur: np.ndarray, anc: np.ndarray, eps: float) -> float:
    n = min(cur.shape[1], anc.shape[1])
    a, b = cur[:, :n].reshape(cur.shape[0], -1), anc[:, :n].reshape(anc.shape[0], -1)
    a = a / np.maximum(np.linalg.norm(a, axis=-1, keepdims=True), eps)
    b = b / np.maximum(np.linalg.norm(b, axis=-1, keepdims=True), eps)
    return float((a * b).sum(-1).mean())


def gate(score: float, threshold: float, temperature: float, floor: float) -> float:
    if temperature <= 0.0:
        return 1.0 if score >= threshold else floor
    z = (score - threshold) / max(temperature, 1e-6)
    return floor + (1.0 - floor) / (1.0 + math.exp(-min(max(z, -50.0), 50.0)))


def ema(prev, anchor, cur, beta: float, tether: float):
    if prev is None:
        return cur.copy()
    out = prev * (1.0 - beta) + cur * beta
    if anchor is not None and tether > 0.0:
        out = out * (1.0 - tether) + anchor * tether
    return out


class MemoryOracle:
    """The state machine of LearnedMemoryState with the StreamingMemory
    settings by default (taomate/inference/memory.py:4-29)."""

    def __init__(self, **kw):
        cfg = dict(video_downsample=4, audio_tokens=64, video_beta=0.15, audio_beta=0.10, video_anchor_tether=0.20,
                   audio_anchor_tether=0.10, identity_anchor_enabled=True, identity_anchor_scale=1.0,
                   reference_anchor_enabled=True, drift_gate_enabled=True, drift_gate_threshold=0.05,
                   drift_gate_temperature=0.10, drift_gate_min=0.10, drift_gate_apply_to_color=True,
                   color_enabled=True, color_alpha=0.04, color_proto_alpha=0.015, color_update_beta=0.03,
                   color_anchor_tether=0.60, color_proto_grid=4, color_drift_threshold=2.0,
                   color_max_correction=0.35, color_film_enabled=True, eps=1e-6)
        cfg.update(kw)
        self.c = cfg
        self.video = self.audio = self.video_anchor = self.audio_anchor = None
        self.color_stats = self.color_anchor_stats = self.color_proto = self.color_anchor_proto = None
        self.reference_initialized = False
        self.last_gate = None

    def set_reference(self, video, audio):
        c = self.c
        if not c["reference_anchor_enabled"] or self.reference_initialized:
            return
        v = video_tokens(video, c["video_downsample"], c["eps"])
        self.video_anchor = v.copy()
        if self.video is None:
            self.video = v.copy()
        a = audio_tokens(audio, c["audio_tokens"], c["eps"])
        self.audio_anchor = a.copy()
        if self.audio is None:
            self.audio = a.copy()
        if c["color_enabled"]:
            st, pr = channel_stats(video, c["eps"]), lowfreq_proto(video, c["color_proto_grid"])
            self.color_anchor_stats, self.color_anchor_proto = st, pr
            if self.color_stats is None:
                self.color_stats = (st[0].copy(), st[1].copy())
            if self.color_proto is None:
                self.color_proto = pr.copy()
        self.reference_initialized = True

    def update(self, video, audio):
        c = self.c
        g = 1.0
        v = video_tokens(video, c["video_downsample"], c["eps"])
        if self.video_anchor is None:
            self.video_anchor = v.copy()
        elif c["drift_gate_enabled"]:
            g = gate(token_cosine(v, self.video_anchor, c["eps"]), c["drift_gate_threshold"],
                     c["drift_gate_temperature"], c["drift_gate_min"])
        self.last_gate = g
        self.video = ema(self.video, self.video_anchor, v, _unit(c["video_beta"] * g), c["video_anchor_tether"])
        a = audio_tokens(audio, c["audio_tokens"], c["eps"])
        if self.audio_anchor is None:
            self.audio_anchor = a.copy()
        self.audio = ema(self.audio, self.audio_anchor, a, c["audio_beta"], c["audio_anchor_tether"])
        if not c["color_enabled"]:
            return
        st, pr = channel_stats(video, c["eps"]), lowfreq_proto(video, c["color_proto_grid"])
        if self.color_anchor_stats is None:
            self.color_anchor_stats, self.color_anchor_proto = st, pr
            self.color_stats, self.color_proto = (st[0].copy(), st[1].copy()), pr.copy()
            return
        drift = drift_score(st, self.color_anchor_stats, c["eps"])
        beta = c["color_update_beta"] * (g if c["drift_gate_apply_to_color"] else 1.0)
        if (c["color_drift_threshold"] > 0.0 and drift > c["color_drift_threshold"]) or beta <= 0.0:
            return
        t = c["color_anchor_tether"]
        mixed = [(1 - beta) * o + beta * n for o, n in zip(self.color_stats, st)]
        if t > 0.0:
            mixed = [(1 - t) * m + t * a for m, a in zip(mixed, self.color_anchor_stats)]
        self.color_stats = tuple(mixed)
        p = (1 - beta) * self.color_proto + beta * pr
        if t > 0.0:
            p = (1 - t) * p + t * self.color_anchor_proto
        self.color_proto = p

    def conditioning(self) -> Dict[str, np.ndarray]:
        c = self.c
        out = {}
        parts = []
        if c["identity_anchor_enabled"] and self.video_anchor is not None:
            parts.append(self.video_anchor * c["identity_anchor_scale"])
        if self.video is not None:
            parts.append(self.video)
        if parts:
            out["learned_memory_video"] = np.concatenate(parts, axis=1)
        if self.audio is not None:
            out["learned_memory_audio"] = self.audio
        if c["color_film_enabled"] and self.color_stats is not None:
            mu, sd = self.color_stats
            amu, asd = self.color_anchor_stats
            e = c["eps"]
            out["learned_memory_color"] = np.concatenate(
                [mu, np.log(np.maximum(sd, e)), amu, np.log(np.maximum(asd, e))], axis=-1)
        return out

    def apply_color(self, video):
        c = self.c
        if not c["color_enabled"] or self.color_stats is None:
            return video.astype(np.float64)
        return apply_color(video, self.color_stats, self.color_proto, c["color_alpha"], c["color_proto_alpha"],
                           c["color_max_correction"], c["eps"])
