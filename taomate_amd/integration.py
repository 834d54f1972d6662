"""Binding the gfx950 path into a running TaoMate process.

The reference is Python, so its "FFI" for this path is the set of module
attributes its code looks up at call time.  Most of those names are copied
into the calling module at import time with ``from ... import``:

  ltx_causal/attention/causal_attention.py:19-27   standard_attention_forward, apply_split_rotary_emb
  ltx_causal/transformer/causal_block.py:24        CausalLTXAttention
  ltx_causal/transformer/kv_cache.py:31-34         standard_attention_forward, CausalLTXAttention,
                                                    causal_precompute_freqs_cis
  taomate/inference/cache.py:5                     KVCache, LayerKVCache
  taomate/inference/model.py:8                     retain_streaming_context
  taomate/inference/runtime.py:16-20               retain_streaming_context

so rebinding only the defining module changes nothing for those callers.
``install`` rebinds every name in every module that holds it (the table
``BINDINGS``), including the functions kv_cache.py calls through its own
globals (``attention_with_cache`` from ``block_forward_with_cache``,
``_cat_cache`` and ``LayerKVCache`` in its cache update, kv_cache.py:2642-2656),
and replaces ``CausalLTX2DiffusionWrapper.init_kv_cache`` (wrapper.py:15-20) so
that the zero-argument call the runtime makes (model.py:101,
model_runtime.py:1101/1178) returns this package's cache types.  With an arena
plan, that call also gives each block's four cached attentions a KV arena (see
``kv_cache.attach_block_arenas``), so every cache field of the stream lives in
arena slots from its first append on.

Run it before the model is built (the blocks look ``CausalLTXAttention`` up
when they are constructed).  ``uninstall()`` on the returned handle restores
every original binding.
"""
from __future__ import annotations

import importlib
import sys
import types
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Mapping, Optional, Tuple

from . import attention as _attention
from . import cache as _cache
from . import kv_cache as _kv_cache
from . import rope as _rope

# (module, attribute, replacement): every place the reference's code finds a
# hot-path name, with the reference line that binds it there.
BINDINGS: Tuple[Tuple[str, str, Any], ...] = (
    # flex_attention_utils.py:225 (definition)
    ("ltx_causal.attention.flex_attention_utils", "standard_attention_forward", _attention.standard_attention_forward),
    # causal_attention.py:19-27 (imported), :61 (definition)
    ("ltx_causal.attention.causal_attention", "standard_attention_forward", _attention.standard_attention_forward),
    ("ltx_causal.attention.causal_attention", "apply_split_rotary_emb", _rope.apply_split_rotary_emb),
    ("ltx_causal.attention.causal_attention", "CausalLTXAttention", _attention.CausalLTXAttention),
    # causal_rope.py:102, :139 (definitions)
    ("ltx_causal.rope.causal_rope", "apply_split_rotary_emb", _rope.apply_split_rotary_emb),
    ("ltx_causal.rope.causal_rope", "causal_precompute_freqs_cis", _rope.causal_precompute_freqs_cis),
    # causal_block.py:24 (imported)
    ("ltx_causal.transformer.causal_block", "CausalLTXAttention", _attention.CausalLTXAttention),
    # kv_cache.py:31-34 (imported), :321-358, :394, :1148 (definitions)
    ("ltx_causal.transformer.kv_cache", "standard_attention_forward", _attention.standard_attention_forward),
    ("ltx_causal.transformer.kv_cache", "CausalLTXAttention", _attention.CausalLTXAttention),
    ("ltx_causal.transformer.kv_cache", "causal_precompute_freqs_cis", _rope.causal_precompute_freqs_cis),
    ("ltx_causal.transformer.kv_cache", "attention_with_cache", _attention.attention_with_cache),
    ("ltx_causal.transformer.kv_cache", "_cat_cache", _kv_cache._cat_cache),
    ("ltx_causal.transformer.kv_cache", "LayerKVCache", _kv_cache.LayerKVCache),
    ("ltx_causal.transformer.kv_cache", "KVCache", _kv_cache.KVCache),
    # taomate/inference/cache.py:5 (imported), :58 (definition)
    ("taomate.inference.cache", "KVCache", _kv_cache.KVCache),
    ("taomate.inference.cache", "LayerKVCache", _kv_cache.LayerKVCache),
    ("taomate.inference.cache", "retain_streaming_context", _cache.retain_streaming_context),
    # taomate/inference/model.py:8, runtime.py:16-20 (imported)
    ("taomate.inference.model", "retain_streaming_context", _cache.retain_streaming_context),
    ("taomate.inference.runtime", "retain_streaming_context", _cache.retain_streaming_context),
)

WRAPPER_MODULE = "ltx_causal.wrapper"
WRAPPER_CLASS = "CausalLTX2DiffusionWrapper"

_MISSING = object()


@dataclass(frozen=True)
class ArenaPlan:
    """KV arena capacity per cached attention of every block, in tokens:
    video-keyed kinds (video_self, v2a) and audio-keyed kinds (audio_self,
    a2v).  ``kv_dtype`` "fp8" applies to the video-keyed kinds, whose appends
    are whole latent frames of ``video_frame_tokens``."""
    video_tokens: int
    audio_tokens: int
    kv_dtype: str = "bf16"
    video_frame_tokens: int = 1

    @classmethod
    def for_stream(cls, video_hw: Tuple[int, int], max_video_frames: int = 32, max_audio_tokens: int = 512,
                   kv_dtype: str = "bf16") -> "ArenaPlan":
        """Capacities for a stream of ``video_hw`` latent frames.  A slot is
        busy while any cache view covers it, so the plan must hold everything
        the caller keeps alive at once.  The defaults cover the reference
        runtime at the start of the second window: the first window's 16
        frames (blocks of 4, 3, 3, 3, 3 frames appended without pruning,
        model_runtime.py:1257-1342) still referenced by the caller, the
        retained sink + 2 recent blocks of the new window, the block in flight
        and its commit (25 frames), with slack; audio blocks of 25-26 tokens
        each take 32 slots (appends start on 8-slot boundaries)."""
        hw = int(video_hw[0]) * int(video_hw[1])
        return cls(hw * int(max_video_frames), int(max_audio_tokens), kv_dtype, hw)


def init_kv_cache_for(model, plan: Optional[ArenaPlan] = None) -> _kv_cache.KVCache:
    """The zero-argument ``init_kv_cache()`` of the reference (wrapper.py:15-20)
    for ``model`` (anything with ``transformer_blocks``): one empty
    LayerKVCache per block.  With ``plan``, every block's cached attentions
    carry an arena plan first (kept across calls while the plan is unchanged,
    so a restarted stream reuses the arenas)."""
    blocks = model.transformer_blocks
    if plan is not None and model.__dict__.get("_ltx_arena_plan_applied") != plan:
        _kv_cache.attach_block_arenas(blocks, plan.video_tokens, plan.audio_tokens, plan.kv_dtype,
                                      plan.video_frame_tokens)
        model.__dict__["_ltx_arena_plan_applied"] = plan
    return _kv_cache.empty_kv_cache(len(blocks))


@dataclass
class Installation:
    """What ``install`` changed: (module, attribute, original) per binding, the
    modules that were absent, and the wrapper method it replaced."""
    bound: List[Tuple[types.ModuleType, str, Any]] = field(default_factory=list)
    skipped: List[str] = field(default_factory=list)
    wrapper: Optional[Tuple[type, Any]] = None

    def uninstall(self) -> None:
        for mod, attr, orig in reversed(self.bound):
            if orig is _MISSING:
                delattr(mod, attr)
            else:
                setattr(mod, attr, orig)
        self.bound.clear()
        if self.wrapper is not None:
            cls, orig = self.wrapper
            if orig is _MISSING:
                delattr(cls, "init_kv_cache")
            else:
                setattr(cls, "init_kv_cache", orig)
            self.wrapper = None


def _resolve(name: str, modules: Optional[Mapping[str, types.ModuleType]],
             importer: Callable[[str], types.ModuleType]) -> Optional[types.ModuleType]:
    if modules is not None:
        return modules.get(name)
    if name in sys.modules:
        return sys.modules[name]
    try:
        return importer(name)
    except ImportError:
        return None


def install(modules: Optional[Mapping[str, types.ModuleType]] = None, *, arena_plan: Optional[ArenaPlan] = None,
            require: bool = True, importer: Callable[[str], types.ModuleType] = importlib.import_module
            ) -> Installation:
    """Rebind the reference's hot-path names to this package's (``BINDINGS``)
    and replace ``CausalLTX2DiffusionWrapper.init_kv_cache``.

    ``modules`` maps module names to module objects; by default each is taken
    from ``sys.modules`` or imported (a TaoMate process).  With ``require``
    (the default) a module that is absent, or that lacks the attribute being
    replaced, is an error and nothing is changed; otherwise it is skipped and
    listed in ``Installation.skipped``."""
    inst = Installation()
    plan: List[Tuple[types.ModuleType, str, Any]] = []
    for modname, attr, repl in BINDINGS:
        mod = _resolve(modname, modules, importer)
        if mod is None or not hasattr(mod, attr):
            what = f"{modname}.{attr}" if mod is not None else modname
            if what not in inst.skipped:
                inst.skipped.append(what)
            continue
        plan.append((mod, attr, repl))
    wmod = _resolve(WRAPPER_MODULE, modules, importer)
    wcls = getattr(wmod, WRAPPER_CLASS, None) if wmod is not None else None
    if wcls is None:
        inst.skipped.append(f"{WRAPPER_MODULE}.{WRAPPER_CLASS}")
    if require and inst.skipped:
        raise ImportError(f"taomate_amd.install: not found: {', '.join(inst.skipped)} "
                          "(nothing was changed; pass require=False to skip them)")
    for mod, attr, repl in plan:
        inst.bound.append((mod, attr, mod.__dict__.get(attr, _MISSING)))
        setattr(mod, attr, repl)
    if wcls is not None:
        orig = wcls.__dict__.get("init_kv_cache", _MISSING)

        def init_kv_cache(self) -> _kv_cache.KVCache:
            """wrapper.py:15-20: this package's empty cache for the wrapped model."""
            return init_kv_cache_for(self.model, arena_plan)

        wcls.init_kv_cache = init_kv_cache
        inst.wrapper = (wcls, orig)
    return inst
