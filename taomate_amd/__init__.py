"""taomate_amd: TaoMate's chunked causal LTX attention path, native on MI355X (gfx950).

The public names mirror the reference's drop-in surface:

* ``attention_with_cache``, ``standard_attention_forward``, ``CausalLTXAttention``
  (ltx_causal/transformer/kv_cache.py:1148, ltx_causal/attention/flex_attention_utils.py:225,
  ltx_causal/attention/causal_attention.py:61)
* ``causal_precompute_freqs_cis``, ``apply_split_rotary_emb``, ``generate_freq_grid``
  (ltx_causal/rope/causal_rope.py:45-357)
* ``LayerKVCache``, ``KVCache``, ``init_kv_cache``, ``_cat_cache``
  (ltx_causal/transformer/kv_cache.py:321-398, ltx_causal/wrapper.py:15)
* ``install`` rebinds those names inside a running TaoMate process wherever its
  modules hold them, and replaces the wrapper's ``init_kv_cache()``
* ``retain_streaming_context``, ``cache_segments``, ``attach_segments``
  (taomate/inference/cache.py), ``compute_av_blocks`` (mask_builder.py:102)
* ``StreamingGenerator`` (the window and block loop of taomate/inference/model.py:33-248 and
  model_runtime.py:772-1342: 3-step denoise over the cached context, clean commit, memory
  update, retention)
* ``LearnedMemoryState``, ``StreamingMemory`` (taomate/runtime_support/learned_memory.py,
  taomate/inference/memory.py)
* ``load_generator`` / ``save_generator`` (taomate/inference/model_runtime.py:182-425) and the
  interactive prefix state (taomate/inference/streaming_runtime.py:1404-1500)

All device math goes through ``lib/libtaomate_ltx.so`` (C ABI in
``include/taomate_ltx.h``); importing works without it, the first kernel call
raises ``NativeLibraryError`` if it was not built.
"""
from ._native import NativeCallError, NativeLibraryError
from .attention import CausalLTXAttention, attention_with_cache, standard_attention_forward
from .blocks import AVBlock, compute_aligned_audio_frames, compute_av_blocks, global_block_at_index
from .cache import (attach_segments, cache_segments, prune_clean_kv_to_sink_recent,
                    retain_streaming_context)
from .kv_cache import (ArenaSpec, KVArena, KVArenaFull, KVCache, KVSpanView, LayerKVCache,
                       _cat_cache, attach_arena, attach_block_arenas, init_kv_cache)
from .integration import ArenaPlan, Installation, init_kv_cache_for, install
from .runtime import StreamingGenerator, denoising_sigmas
from .rope import CausalRopeType, apply_split_rotary_emb, causal_precompute_freqs_cis, generate_freq_grid
from .streaming import ChunkStream, retain_pinned_recent
from .memory import LearnedMemoryState, StreamingMemory
from . import dit
from .checkpoint import load_generator, save_generator
from .prefix_state import build_prefix_state_payload, load_prefix_state, save_prefix_state

__all__ = [
    "NativeCallError", "NativeLibraryError", "CausalLTXAttention", "attention_with_cache",
    "standard_attention_forward", "AVBlock", "compute_aligned_audio_frames", "compute_av_blocks",
    "global_block_at_index", "attach_segments", "cache_segments", "prune_clean_kv_to_sink_recent",
    "retain_streaming_context", "ArenaSpec", "KVArena", "KVArenaFull", "KVCache", "KVSpanView",
    "LayerKVCache", "_cat_cache", "init_kv_cache", "CausalRopeType", "apply_split_rotary_emb",
    "causal_precompute_freqs_cis", "generate_freq_grid", "ChunkStream", "retain_pinned_recent",
    "LearnedMemoryState", "StreamingMemory", "load_generator", "save_generator", "build_prefix_state_payload",
    "load_prefix_state", "save_prefix_state", "attach_arena", "attach_block_arenas", "ArenaPlan",
    "Installation", "init_kv_cache_for", "install", "StreamingGenerator", "denoising_sigmas",
]
