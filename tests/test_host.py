"""Host-side product logic on the CPU: block table, KV-arena allocation and
liveness, index-only eviction (bit-exact against the oracle's plan), and the
C ABI surface of the built library (symbols and argument checking only)."""
import ctypes
import gc
import os
import re

import pytest
import torch

import taomate_amd as T
from oracle import cache as OC
from taomate_amd import _native
from taomate_amd.kv_cache import KVArena, KVSpanView

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_blocks_match_oracle():
    for first in (0, 4):
        for n in (1, 4, 5, 9, 16, 40):
            if first and n < first:
                continue
            a = T.compute_av_blocks(n, num_frame_per_block_first=first)
            b = OC.compute_av_blocks(n, num_frame_per_block_first=first)
            assert [(x.block_idx, x.video_start, x.video_end, x.audio_start, x.audio_end) for x in a] == \
                   [(x.block_idx, x.video_start, x.video_end, x.audio_start, x.audio_end) for x in b]
    assert T.global_block_at_index(5).video_start == 4 + 4 * 3


def test_arena_alloc_first_fit_and_liveness():
    a = KVArena(1, 100, 1, 8, "cpu")
    assert a.cap == 104                   # whole 8-slot groups
    v1 = KVSpanView(a, "k", [(a.alloc(30), 30)])
    assert v1.spans == ((0, 30),)
    v2 = KVSpanView(a, "k", [(a.alloc(30), 30)])
    assert v2.spans == ((32, 30),)        # bf16 appends start on 8-slot boundaries
    del v1
    gc.collect()
    assert a.alloc(30) == 0               # freed slots are reused
    assert a.alloc(33) == 64
    v3 = KVSpanView(a, "k", [(64, 40)])
    with pytest.raises(T.KVArenaFull):
        a.alloc(33)
    assert a.alloc(30) == 0
    assert torch.count_nonzero(a.v_store) == 0   # key-major V starts zeroed
    assert a.v.shape == (1, 104, 1, 8) and a.v.stride(1) == 1
    del v2, v3


def test_fp8_arena_is_frame_aligned():
    a = KVArena(1, 96, 1, 8, "cpu", kv_dtype="fp8", frame_tokens=32)
    v = KVSpanView(a, "k", [(0, 32)])
    assert a.alloc(32) == 32
    with pytest.raises(ValueError):
        a.alloc(20)
    assert a.k_scales.shape == (1, 1, 3)
    del v


def test_span_view_slicing_and_cat_are_index_only():
    a = KVArena(2, 64, 3, 8, "cpu")
    v = KVSpanView(a, "k", [(10, 5), (40, 7), (20, 3)])
    assert v.shape == (2, 15, 3, 8)
    s = v[:, 3:9]
    assert s.spans == ((13, 2), (40, 4))
    c = T._cat_cache(v[:, 0:5], v[:, 12:15])
    assert c.spans == ((10, 5), (20, 3))
    adj = T._cat_cache(KVSpanView(a, "k", [(0, 4)]), KVSpanView(a, "k", [(4, 6)]))
    assert adj.spans == ((0, 10),)   # adjacent spans merge
    assert T._cat_cache(None, v) is v


def _put_ids(arena, start, ids):
    """Token id -> (id // 128, id % 128) in head-dim channels 0 and 1 (exact in bf16)."""
    n = ids.numel()
    arena.k[0, start:start + n, 0, 0] = (ids // 128).to(arena.k.dtype)
    arena.k[0, start:start + n, 0, 1] = (ids % 128).to(arena.k.dtype)


def _ids_of(view: KVSpanView):
    store = view.arena.k if view.which == "k" else view.arena.v
    return [int(store[0, s + i, 0, 0].item()) * 128 + int(store[0, s + i, 0, 1].item())
            for s, n in view.spans for i in range(n)]


@pytest.mark.parametrize("hw,n_blocks", [((2, 3), 12), ((16, 24), 8)])
def test_streaming_eviction_plan_bit_exact(hw, n_blocks):
    """Replays the reference's window loop (denoise steps that must not commit,
    the sigma=0 commit, segment append, retain_streaming_context) on arena
    views, writing each token's absolute id into its slot, and compares the
    logical token sequence after every commit with the oracle's plan."""
    plan = OC.streaming_plan(n_blocks, hw)
    per = hw[0] * hw[1]
    cap_v = 4 * per + 2 * 3 * per + 3 * 3 * per + 4 * 8   # + room for 8-slot alignment
    spec = {"video_self": T.ArenaSpec(cap_v, 1, 8), "audio_self": T.ArenaSpec(26 + 25 * 4 + 4 * 8, 1, 8)}
    cache = T.init_kv_cache(1, 1, spec, "cpu")
    blocks = T.compute_av_blocks(4 + (n_blocks - 1) * 3, num_frame_per_block_first=4)[:n_blocks]
    segments = []
    for bi, blk in enumerate(blocks):
        previous = list(cache.layers)
        lay = previous[0]
        nv, na = blk.video_frames * per, blk.audio_frames
        for _step in range(3):   # denoise steps: append into scratch slots, then discard
            sv = lay.video_self_k.arena.alloc(nv)
            sa = lay.audio_self_k.arena.alloc(na)
            step_v = T._cat_cache(lay.video_self_k, KVSpanView(lay.video_self_k.arena, "k", [(sv, nv)]))
            step_a = T._cat_cache(lay.audio_self_k, KVSpanView(lay.audio_self_k.arena, "k", [(sa, na)]))
            lay.video_self_k.arena.k[:, sv:sv + nv] = -1   # garbage that must never become visible
            lay.audio_self_k.arena.k[:, sa:sa + na] = -1
            del step_v, step_a
        cache.layers = list(previous)   # restore the snapshot (model_runtime.py:894-895)
        # sigma=0 commit: write the block's tokens, cat into the cache
        va, aa = lay.video_self_k.arena, lay.audio_self_k.arena
        sv, sa = va.alloc(nv), aa.alloc(na)
        _put_ids(va, sv, torch.arange(blk.video_start * per, blk.video_end * per))
        _put_ids(aa, sa, torch.arange(blk.audio_start, blk.audio_end))
        new = T.LayerKVCache(video_self_k=T._cat_cache(lay.video_self_k, KVSpanView(va, "k", [(sv, nv)])),
                             video_self_v=T._cat_cache(lay.video_self_v, KVSpanView(va, "v", [(sv, nv)])),
                             audio_self_k=T._cat_cache(lay.audio_self_k, KVSpanView(aa, "k", [(sa, na)])),
                             audio_self_v=T._cat_cache(lay.audio_self_v, KVSpanView(aa, "v", [(sa, na)])))
        cache.layers = [new]
        segments.append({"block_idx": blk.block_idx, "video_tokens": nv, "audio_tokens": na})
        T.attach_segments(cache, segments)
        cache = T.retain_streaming_context(cache)
        segments = T.cache_segments(cache)
        del previous, lay, new
        gc.collect()
        got_v = _ids_of(cache.layers[0].video_self_k)
        got_a = _ids_of(cache.layers[0].audio_self_k)
        assert got_v == plan[bi]["video_ids"], f"block {bi}"
        assert got_a == plan[bi]["audio_ids"], f"block {bi}"
        assert segments == plan[bi]["segments"]
        assert cache.layers[0].video_self_v.spans == cache.layers[0].video_self_k.spans


def test_plain_tensor_cache_path_matches_oracle():
    """Plain [B, L, H, D] tensors (no arena) slice/concatenate like the reference."""
    hw = (2, 3)
    plan = OC.streaming_plan(6, hw)
    blocks = T.compute_av_blocks(4 + 5 * 3, num_frame_per_block_first=4)[:6]
    cache = T.KVCache(layers=[T.LayerKVCache()])
    segs = []
    for bi, blk in enumerate(blocks):
        lay = cache.layers[0]
        v = torch.arange(blk.video_start * 6, blk.video_end * 6, dtype=torch.float32).view(1, -1, 1, 1)
        a = torch.arange(blk.audio_start, blk.audio_end, dtype=torch.float32).view(1, -1, 1, 1)
        cache.layers = [T.LayerKVCache(video_self_k=T._cat_cache(lay.video_self_k, v),
                                       audio_self_k=T._cat_cache(lay.audio_self_k, a))]
        segs.append({"block_idx": blk.block_idx, "video_tokens": blk.video_frames * 6,
                     "audio_tokens": blk.audio_frames})
        T.attach_segments(cache, segs)
        cache = T.retain_streaming_context(cache)
        segs = T.cache_segments(cache)
        assert cache.layers[0].video_self_k.flatten().long().tolist() == plan[bi]["video_ids"]
        assert cache.layers[0].audio_self_k.flatten().long().tolist() == plan[bi]["audio_ids"]


def test_prune_recent_blocks_variant():
    segs = [{"block_idx": i, "video_tokens": 10, "audio_tokens": 1} for i in range(5)]
    cache = T.attach_segments(T.KVCache(layers=[]), segs)
    out = T.prune_clean_kv_to_sink_recent(cache, recent_blocks=1)
    assert [s["block_idx"] for s in out.segments] == [0, 4]
    out = T.prune_clean_kv_to_sink_recent(cache, recent_blocks=0)
    assert [s["block_idx"] for s in out.segments] == [0]
    with pytest.raises(RuntimeError):
        T.retain_streaming_context(T.KVCache(layers=[]))


def _header_symbols():
    src = open(os.path.join(ROOT, "include", "taomate_ltx.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(ltx_\w+)\s*\(", src, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = _header_symbols()
    assert "ltx_flash_attn_fwd" in names and len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
        assert n in _native.SIGNATURES, n
    assert lib.ltx_abi_version() == _native.ABI_VERSION == 2


def test_abi_rejects_bad_arguments_without_a_gpu():
    lib = _native.load()
    rc = lib.ltx_rope_table(None, None, 1, None, 0, 3, 1, 1, 1, 0, 0, 20.0, 2048.0, 2048.0, 64, 1, 1, None)
    assert rc == -1 and b"null pointer" in lib.ltx_last_error()
    rc = lib.ltx_flash_attn_fwd(ctypes.c_void_p(16), 1, 1, 1, 96, 0, 0, 0, 0, None, None, None, 0, 0, 0,
                                0, 0, 0, 1, 1, None, None, 0, 0, 0, None, 0, None, ctypes.c_void_p(16), 0, 0,
                                0, None, 0.0, None, 0, None)
    assert rc == -1 and b"head dim" in lib.ltx_last_error()
    rc = lib.ltx_kv_gather(3, 1, 1, 8, None, 0, 0, 0, None, 0, 0, 0, 0, None, None, None)
    assert rc == -1
    p16 = ctypes.c_void_p(16)
    rc = lib.ltx_kv_append_fp8_pair(1, 100, 1, 128, 64, p16, 0, 128, 0, p16, p16, p16, 0, 128, 0, p16, p16,
                                    0, 128, 0, 0, 0, None)
    assert rc == -1 and b"multiple of frame_tokens" in lib.ltx_last_error()
    rc = lib.ltx_kv_append_fp8_pair(1, 128, 1, 128, 64, None, 0, 128, 0, p16, p16, p16, 0, 128, 0, p16, p16,
                                    0, 128, 0, 0, 0, None)
    assert rc == -1 and b"null pointer" in lib.ltx_last_error()
    with pytest.raises(_native.NativeCallError, match="n_segments"):
        _native.call("ltx_flash_attn_fwd", ctypes.c_void_p(16), 1, 1, 1, 128, 0, 0, 0, 17, None, None,
                     None, 0, 0, 0, 0, 0, 0, 1, 1, None, None, 0, 0, 0, None, 0, None, ctypes.c_void_p(16), 0,
                     0, 0, None, 0.0, None, 0, None)


def test_kernels_refuse_cpu_tensors():
    x = torch.zeros(1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensors"):
        T.kernels.qk_rmsnorm_rope(x, x.clone(), None, 1e-6, None, 1, 64)
