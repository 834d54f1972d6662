"""TaoMate generator checkpoints in and out of ``taomate_amd.dit.AVModel``.

The checkpoint format is that of load_model_generator
(taomate/inference/model_runtime.py:182-425): a dict ``{"generator_ema":
state_dict}`` whose keys are the wrapper's ``model.<parameter>`` names, read
here with ``torch.load(..., weights_only=True, mmap=True)`` (no code runs
from the file) or from a ``.safetensors`` file of the same keys.  The block
configuration is read off the tensors the way the reference auto-detects it
(layer count, widths, gated attention, the LTX-2.3 text cross-attention
AdaLN, learned-memory adapters and FiLM); features this build does not run
(audio sink tokens, caption projection) are refused by name instead of being
dropped.
The model is built on the meta device and takes the checkpoint's tensors
with ``assign=True`` (no second copy of the weights), then moves to the
target device.
"""
from __future__ import annotations

import os
import re
from typing import Dict, Mapping, Optional, Tuple

import torch

from .dit import AVConfig, AVModel

__all__ = ["read_generator_state", "detect_config", "load_generator", "save_generator"]

_PREFIX = "model."


def read_generator_state(path: str) -> Dict[str, torch.Tensor]:
    """The generator's state dict, keys without the wrapper's ``model.`` prefix."""
    if path.endswith(".safetensors"):
        from safetensors.torch import load_file
        raw = load_file(path)
    else:
        ckpt = torch.load(path, map_location="cpu", mmap=True, weights_only=True)
        if not isinstance(ckpt, dict) or "generator_ema" not in ckpt:
            raise ValueError(f"{path}: expected a TaoMate EMA checkpoint {{'generator_ema': state_dict}}")
        raw = ckpt["generator_ema"]
    return {(k[len(_PREFIX):] if k.startswith(_PREFIX) else k): v for k, v in raw.items()}


def _shape(sd: Mapping[str, torch.Tensor], key: str) -> Tuple[int, ...]:
    if key not in sd:
        raise ValueError(f"checkpoint has no {key!r}")
    return tuple(sd[key].shape)


def detect_config(sd: Mapping[str, torch.Tensor], *, video_d_head: int = 128, audio_d_head: int = 64,
                  learned_memory_mode: str = "cross_attn_adapter", learned_memory_layer_interval: int = 4,
                  learned_memory_heads: int = 8) -> AVConfig:
    """AVConfig of a generator state dict (model_runtime.py:230-330).  Head
    sizes are not recoverable from the tensors: the defaults are the 22B
    model's (video 128, audio 64) and the head counts follow from the widths."""
    unsupported = {
        "audio sink tokens": any("audio_sink_tokens" in k or "sink_text_condition" in k for k in sd),
        "caption projection": any(k.startswith("caption_projection.") for k in sd),
    }
    vd, in_ch = _shape(sd, "patchify_proj.weight")
    # LTX-2.3 text cross-attention AdaLN: 9 modulation rows (model_runtime.py:256-261)
    coeff = _shape(sd, "adaln_single.linear.weight")[0] // vd
    if coeff not in (6, 9):
        unsupported[f"an AdaLN of {coeff} coefficients"] = True
    bad = [name for name, hit in unsupported.items() if hit]
    if bad:
        raise NotImplementedError(f"checkpoint uses features this build does not run: {', '.join(bad)}")
    ad = _shape(sd, "audio_patchify_proj.weight")[0]
    layers = 1 + max(int(m.group(1)) for k in sd for m in [re.match(r"transformer_blocks\.(\d+)\.", k)] if m)
    v_inner = _shape(sd, "transformer_blocks.0.attn1.to_q.weight")[0]
    a_inner = _shape(sd, "transformer_blocks.0.audio_attn1.to_q.weight")[0]
    if v_inner % video_d_head or a_inner % audio_d_head:
        raise ValueError(f"attention widths {v_inner} / {a_inner} are not multiples of the head sizes "
                         f"{video_d_head} / {audio_d_head}")
    memory = any("learned_memory" in k or "memory_attn" in k for k in sd)
    film = any("color_film" in k for k in sd)
    kw = {}
    if memory:
        kw.update(learned_memory_enabled=True, learned_memory_mode=learned_memory_mode,
                  learned_memory_layer_interval=learned_memory_layer_interval,
                  learned_memory_heads=learned_memory_heads,
                  learned_memory_video_dim=_shape(sd, "learned_memory_video_encoder.weight")[0],
                  learned_memory_audio_dim=_shape(sd, "learned_memory_audio_encoder.weight")[0])
    if film:
        key = next(k for k in sd if k.endswith("video_color_film.net.0.weight"))
        hidden, cond = _shape(sd, key)
        kw.update(learned_memory_color_film_enabled=True, learned_memory_color_condition_dim=cond,
                  learned_memory_color_film_hidden_dim=hidden)
    return AVConfig(num_layers=layers, video_dim=vd, audio_dim=ad, video_heads=v_inner // video_d_head,
                    audio_heads=a_inner // audio_d_head, video_d_head=video_d_head, audio_d_head=audio_d_head,
                    in_channels=in_ch, out_channels=_shape(sd, "proj_out.weight")[0],
                    apply_gated_attention=any("to_gate_logits" in k for k in sd), cross_attention_adaln=coeff == 9,
                    **kw)


def load_generator(model_ckpt_path: str, device="cuda", dtype: torch.dtype = torch.bfloat16,
                   cfg: Optional[AVConfig] = None, **detect_kw) -> AVModel:
    """Build the generator from a checkpoint: configuration detected from the
    tensors (or ``cfg``), weights assigned in ``dtype``; every parameter of the
    model must come from the checkpoint."""
    sd = read_generator_state(model_ckpt_path)
    cfg = cfg if cfg is not None else detect_config(sd, **detect_kw)
    with torch.device("meta"):
        model = AVModel(cfg)
    sd = {k: (v.to(dtype) if v.is_floating_point() and v.dtype != dtype else v) for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(sd, strict=False, assign=True)
    if missing:
        raise ValueError(f"checkpoint lacks {len(missing)} generator parameters, e.g. {missing[:5]}")
    if unexpected:
        raise ValueError(f"checkpoint has {len(unexpected)} tensors this model does not use, e.g. {unexpected[:5]}")
    return model.to(device=device).eval()


def save_generator(model: AVModel, path: str) -> None:
    """Write ``{"generator_ema": {"model.<name>": tensor}}`` (the layout
    load_model_generator reads), atomically."""
    # own copies: parameters may be views of one buffer (fuse_qkv_), which
    # safetensors refuses and torch.save would write whole
    sd = {_PREFIX + k: v.detach().to("cpu", copy=True).contiguous() for k, v in model.state_dict().items()}
    os.makedirs(os.path.dirname(os.path.abspath(path)) or ".", exist_ok=True)
    tmp = f"{path}.tmp.{os.getpid()}"
    if path.endswith(".safetensors"):
        from safetensors.torch import save_file
        save_file(sd, tmp)
    else:
        torch.save({"generator_ema": sd}, tmp)
    os.replace(tmp, path)
