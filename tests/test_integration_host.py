"""install() against stand-in modules that carry the reference's module and
attribute names (no reference import): every binding site is rebound, the
wrapper's zero-argument init_kv_cache() returns this package's cache (with
arena plans on the blocks' cached attentions), and uninstall() restores
everything.  Also the module-attached arenas on the CPU."""
import types

import pytest
import torch
import torch.nn as nn

import taomate_amd as T
from taomate_amd import integration as I
from taomate_amd import kv_cache as KC


def _stand_ins():
    """One module object per reference module, each holding its own copy of
    the names it imports (what ``from x import y`` leaves behind)."""
    mods = {}
    for name, attr, _ in I.BINDINGS:
        mod = mods.setdefault(name, types.ModuleType(name))
        setattr(mod, attr, ("original", name, attr))
    wrapper = types.ModuleType(I.WRAPPER_MODULE)

    class Wrapper:
        def __init__(self, model):
            self.model = model

        def init_kv_cache(self):
            return "reference cache"

    wrapper.CausalLTX2DiffusionWrapper = Wrapper
    mods[I.WRAPPER_MODULE] = wrapper
    return mods


class _Attn:
    def __init__(self, heads, dim_head):
        self.heads, self.dim_head = heads, dim_head


class _Block:
    def __init__(self):
        self.attn1 = _Attn(32, 128)
        self.audio_attn1 = _Attn(32, 64)
        self.audio_to_video_attn = _Attn(32, 64)
        self.video_to_audio_attn = _Attn(32, 64)


class _Model:
    def __init__(self, n):
        self.transformer_blocks = [_Block() for _ in range(n)]


def test_install_rebinds_every_site_and_uninstall_restores():
    mods = _stand_ins()
    plan = T.ArenaPlan.for_stream((16, 24))
    inst = T.install(mods, arena_plan=plan)
    assert not inst.skipped
    assert len(inst.bound) == len(I.BINDINGS)
    for name, attr, repl in I.BINDINGS:
        assert getattr(mods[name], attr) is repl, (name, attr)
    # the names the reference's callers reach (kv_cache globals and the
    # modules that imported them by name) are this package's functions
    kvc = mods["ltx_causal.transformer.kv_cache"]
    assert kvc.attention_with_cache is T.attention_with_cache
    assert kvc._cat_cache is T._cat_cache and kvc.LayerKVCache is T.LayerKVCache
    assert mods["ltx_causal.transformer.causal_block"].CausalLTXAttention is T.CausalLTXAttention
    assert mods["taomate.inference.runtime"].retain_streaming_context is T.retain_streaming_context
    assert mods["taomate.inference.model"].retain_streaming_context is T.retain_streaming_context
    # the zero-argument init_kv_cache() of the wrapper
    model = _Model(3)
    cache = mods[I.WRAPPER_MODULE].CausalLTX2DiffusionWrapper(model).init_kv_cache()
    assert isinstance(cache, T.KVCache) and len(cache.layers) == 3
    assert all(isinstance(l, T.LayerKVCache) and l.video_self_k is None and l.a2v_v is None
               for l in cache.layers)
    blk = model.transformer_blocks[1]
    assert blk.attn1._ltx_arena_plan == T.ArenaSpec(12288, 32, 128, "bf16", 1)
    assert blk.video_to_audio_attn._ltx_arena_plan == T.ArenaSpec(12288, 32, 64, "bf16", 1)
    assert blk.audio_attn1._ltx_arena_plan == T.ArenaSpec(512, 32, 64, "bf16", 1)
    assert blk.audio_to_video_attn._ltx_arena_name == "layer1.a2v"
    inst.uninstall()
    for name, attr, _ in I.BINDINGS:
        assert getattr(mods[name], attr) == ("original", name, attr)
    assert mods[I.WRAPPER_MODULE].CausalLTX2DiffusionWrapper(model).init_kv_cache() == "reference cache"


def test_install_requires_every_site_unless_told_otherwise():
    mods = _stand_ins()
    del mods["taomate.inference.runtime"]
    delattr(mods["ltx_causal.transformer.kv_cache"], "_cat_cache")
    with pytest.raises(ImportError, match="taomate.inference.runtime"):
        T.install(mods)
    # nothing was changed by the refused call
    assert mods["ltx_causal.transformer.kv_cache"].attention_with_cache[0] == "original"
    inst = T.install(mods, require=False)
    assert set(inst.skipped) == {"taomate.inference.runtime", "ltx_causal.transformer.kv_cache._cat_cache"}
    assert mods["ltx_causal.transformer.kv_cache"].attention_with_cache is T.attention_with_cache
    inst.uninstall()
    assert mods["ltx_causal.transformer.kv_cache"].attention_with_cache[0] == "original"


def test_fp8_plan_applies_to_video_keyed_kinds_only():
    model = _Model(1)
    I.init_kv_cache_for(model, T.ArenaPlan.for_stream((16, 24), kv_dtype="fp8"))
    blk = model.transformer_blocks[0]
    assert blk.attn1._ltx_arena_plan.kv_dtype == "fp8" and blk.attn1._ltx_arena_plan.frame_tokens == 384
    assert blk.video_to_audio_attn._ltx_arena_plan.kv_dtype == "fp8"
    assert blk.audio_attn1._ltx_arena_plan.kv_dtype == "bf16"
    assert blk.audio_to_video_attn._ltx_arena_plan.kv_dtype == "bf16"


def test_module_arena_created_on_first_use_and_replaced_on_batch_change():
    attn = nn.Module()
    attn.heads, attn.dim_head = 2, 64
    assert KC.module_arena(attn, 1, "cpu") is None
    T.attach_arena(attn, 100, name="t")
    a = KC.module_arena(attn, 2, "cpu")
    assert a.B == 2 and a.cap == 104 and a.H == 2 and a.D == 64 and a.name == "t"
    assert KC.module_arena(attn, 2, "cpu") is a
    view = a.empty_view("k")
    b = KC.module_arena(attn, 1, "cpu")
    assert b is not a and b.B == 1
    assert view.arena is a          # a view keeps its own arena alive
    assert "_ltx_arena" not in dict(attn.named_buffers()) and not list(attn.parameters())
    KC.detach_arena(attn)
    assert KC.module_arena(attn, 1, "cpu") is None


def test_packed_qkv_lookup_accepts_reference_modules():
    """A module with only the reference's attributes (causal_attention.py:92-118)
    has no packed q/k/v: the three Linears are used."""
    from taomate_amd.attention import packed_qkv
    m = nn.Module()
    m.to_q, m.to_k, m.to_v = nn.Linear(8, 8), nn.Linear(8, 8), nn.Linear(8, 8)
    assert packed_qkv(m) is None
    ours = T.CausalLTXAttention(64, heads=1, dim_head=64).fuse_qkv_()
    assert packed_qkv(ours) is not None
