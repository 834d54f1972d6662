"""Interactive prefix state on disk: the clean prefix latents, the sink
latents, their prompts and the learned-memory state that let a session resume
without regenerating its prefix.

Fields follow _build_interactive_prefix_state_payload
(taomate/inference/streaming_runtime.py:1454-1500, version 2).  The reference
pickles the dict (``torch.save``, read back with ``weights_only=False``);
here the same content is one ``.safetensors`` file: every tensor (latents and
the memory's tokens, anchors and colour statistics) as a named tensor, every
scalar, string and memory setting in its JSON metadata, so loading runs no
code from the file.  Writes go to a temporary name and are renamed into place
(streaming_runtime.py:1440-1451); loads are cached per (path, mtime, size,
device, dtype) like _load_interactive_prefix_state (:1404-1437).
"""
from __future__ import annotations

import collections
import dataclasses
import json
import os
import time
from typing import Any, Dict, List, Optional

import torch

from .memory import LearnedMemoryState

__all__ = ["build_prefix_state_payload", "save_prefix_state", "load_prefix_state", "PREFIX_STATE_VERSION"]

PREFIX_STATE_VERSION = 2
BLOCKS_PER_WINDOW = 5   # streaming_runtime.py: block_count = window_count * 5 by default
_LATENTS = ("prefix_video_latent", "prefix_audio_latent", "decode_prefix_video_latent", "sink_video_latent",
            "sink_audio_latent")
_MEMORY_TENSORS = ("video", "audio", "video_anchor", "audio_anchor", "color_proto", "color_anchor_proto")
_MEMORY_PAIRS = ("color_stats", "color_anchor_stats")
_MEMORY_SCALARS = ("color_last_drift", "color_last_updated", "video_last_anchor_cosine", "video_last_update_gate",
                   "reference_initialized")
_CACHE: "collections.OrderedDict[tuple, Dict[str, Any]]" = collections.OrderedDict()
_CACHE_SIZE = 4


def build_prefix_state_payload(*, case_id: str, window_count: int, prefix_video_latent=None,
                               prefix_audio_latent=None, decode_prefix_video_latent=None,
                               prefix_source_prompts: Optional[List[str]] = None, sink_video_latent=None,
                               sink_audio_latent=None, sink_source_prompt: Optional[str] = None,
                               learned_memory_state: Optional[LearnedMemoryState] = None,
                               block_count: Optional[int] = None) -> Dict[str, Any]:
    """The version-2 payload (streaming_runtime.py:1454-1500)."""
    t = lambda v: v.detach().contiguous() if torch.is_tensor(v) else None
    return {"version": PREFIX_STATE_VERSION, "case_id": case_id, "updated_at": time.time(),
            "window_count": int(window_count),
            "block_count": int(block_count) if block_count is not None else int(window_count) * BLOCKS_PER_WINDOW,
            "prefix_video_latent": t(prefix_video_latent), "prefix_audio_latent": t(prefix_audio_latent),
            "decode_prefix_video_latent": t(decode_prefix_video_latent),
            "prefix_source_prompts": list(prefix_source_prompts) if prefix_source_prompts is not None else None,
            "sink_video_latent": t(sink_video_latent), "sink_audio_latent": t(sink_audio_latent),
            "sink_source_prompt": sink_source_prompt, "learned_memory_state": learned_memory_state}


def _memory_to_file(mem: Optional[LearnedMemoryState], tensors: Dict[str, torch.Tensor]):
    if mem is None:
        return None
    settings = {f.name: getattr(mem, f.name) for f in dataclasses.fields(mem) if f.init}
    for name in _MEMORY_TENSORS:
        v = getattr(mem, name)
        if v is not None:
            tensors[f"learned_memory.{name}"] = v.detach().to("cpu", copy=True).contiguous()
    for name in _MEMORY_PAIRS:
        v = getattr(mem, name)
        if v is not None:
            tensors[f"learned_memory.{name}.mean"] = v[0].detach().to("cpu", copy=True).contiguous()
            tensors[f"learned_memory.{name}.std"] = v[1].detach().to("cpu", copy=True).contiguous()
    return {"class": type(mem).__name__, "settings": settings,
            "state": {name: getattr(mem, name) for name in _MEMORY_SCALARS}}


def _memory_from_file(meta, tensors: Dict[str, torch.Tensor], device) -> Optional[LearnedMemoryState]:
    if meta is None:
        return None
    mem = LearnedMemoryState(**meta["settings"])
    for name in _MEMORY_TENSORS:
        v = tensors.get(f"learned_memory.{name}")
        setattr(mem, name, None if v is None else v.to(device).clone())
    for name in _MEMORY_PAIRS:
        mu, sd = tensors.get(f"learned_memory.{name}.mean"), tensors.get(f"learned_memory.{name}.std")
        setattr(mem, name, None if mu is None else (mu.to(device).clone(), sd.to(device).clone()))
    for name, v in meta["state"].items():
        if name in _MEMORY_SCALARS:
            setattr(mem, name, v)
    return mem


def _key(path: str, device, dtype) -> tuple:
    st = os.stat(path)
    return (os.path.abspath(path), st.st_mtime_ns, st.st_size, str(device), str(dtype))


def save_prefix_state(path: Optional[str], payload: Dict[str, Any]) -> bool:
    """Write ``payload`` to ``path`` (atomic rename); False without a path."""
    if not path:
        return False
    from safetensors.torch import save_file
    tensors: Dict[str, torch.Tensor] = {}
    meta: Dict[str, Any] = {}
    for k, v in payload.items():
        if k in _LATENTS:
            if v is not None:   # own copies: safetensors refuses tensors sharing storage
                tensors[k] = v.detach().to("cpu", copy=True).contiguous()
        elif k == "learned_memory_state":
            meta[k] = _memory_to_file(v, tensors)
        else:
            meta[k] = v
    os.makedirs(os.path.dirname(os.path.abspath(path)) or ".", exist_ok=True)
    tmp = f"{path}.tmp.{os.getpid()}.{time.time_ns()}"
    save_file(tensors, tmp, metadata={"prefix_state": json.dumps(meta)})
    os.replace(tmp, path)
    for key in [k for k in _CACHE if k[0] == os.path.abspath(path)]:
        _CACHE.pop(key, None)
    return True


def load_prefix_state(path: Optional[str], *, device="cuda", dtype: torch.dtype = torch.bfloat16
                      ) -> Optional[Dict[str, Any]]:
    """The payload with its latents on ``device`` in ``dtype`` and the memory
    state rebuilt there; None when there is no path or no file."""
    if not path or not os.path.exists(path):
        return None
    key = _key(path, device, dtype)
    hit = _CACHE.get(key)
    if hit is None:
        from safetensors import safe_open
        with safe_open(path, framework="pt", device="cpu") as f:
            meta = json.loads((f.metadata() or {}).get("prefix_state", "null"))
            if not isinstance(meta, dict) or meta.get("version") != PREFIX_STATE_VERSION:
                raise ValueError(f"{path}: not a version-{PREFIX_STATE_VERSION} prefix state")
            tensors = {k: f.get_tensor(k) for k in f.keys()}
        tensors = {k: (v.to(device=device, dtype=dtype) if k in _LATENTS else v.to(device)) for k, v in tensors.items()}
        hit = _CACHE[key] = (meta, tensors)
        while len(_CACHE) > _CACHE_SIZE:
            _CACHE.popitem(last=False)
    else:
        _CACHE.move_to_end(key)
    meta, tensors = hit
    out: Dict[str, Any] = {k: v for k, v in meta.items() if k != "learned_memory_state"}
    for k in _LATENTS:
        out[k] = tensors.get(k)
    # a fresh state object per load: callers update it in place
    out["learned_memory_state"] = _memory_from_file(meta.get("learned_memory_state"), tensors, device)
    return out
