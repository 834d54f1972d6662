"""Bookkeeping of the anchor | memory | window | current chunk stream on the
CPU: ChunkStream's own span edits (commit, eviction, memory swap) with its
device work replaced by writes of absolute token ids into a slot map, checked
bit-exactly against the oracle's replay of the same policy and the committed
16x24 fixture; arena slots of evicted chunks and replaced memories are freed."""
import json
import os
import types

import numpy as np
import pytest
import torch

from oracle import cache as OC
from taomate_amd.kv_cache import KVSpanView
from taomate_amd.streaming import ChunkStream, retain_pinned_recent

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


class IdStream(ChunkStream):
    """ChunkStream whose prefill/attention write token ids instead of K/V."""

    def __init__(self, grid, kv_dtype, **kw):
        attn = types.SimpleNamespace(heads=1, dim_head=8, inner_dim=8)
        super().__init__(attn, grid, batch=1, device="cpu", kv_dtype=kv_dtype, **kw)
        self.ids = np.full(self.arena.cap, -1, np.int64)

    def _fill(self, f0, nf):
        n = nf * self.hw
        slot = self.arena.alloc(n)
        self.ids[slot:slot + n] = np.arange(f0 * self.hw, (f0 + nf) * self.hw)
        return KVSpanView(self.arena, "k", [(slot, n)]), KVSpanView(self.arena, "v", [(slot, n)])

    def _prefill_segment(self, x, f0, nf):
        return self._fill(f0, nf)

    def _attend(self, x, f0, nf):
        k, v = self._fill(f0, nf)
        return None, k, v

    def cache_ids(self):
        return np.concatenate([self.ids[s:s + n] for s, n in self.k.spans]).tolist()


def _run(grid, kv_dtype, n_chunks, **kw):
    st = IdStream(grid, kv_dtype, **kw)
    hw = grid[0] * grid[1]
    mf = kw.get("memory_frames", 2)
    z = lambda nf: torch.zeros(1, nf * hw, 1)
    st.prefill(z(kw.get("anchor_frames", 1)), z(mf) if mf else None)
    rows = []
    for _ in range(n_chunks):
        st.step(z(kw.get("chunk_frames", 3)))
        live = sum(b - a for a, b in st.arena.live_intervals())
        assert st.k.spans == st.v.spans
        assert live == st.k.shape[1], "arena holds slots no view references"
        rows.append({"segments": [dict(s) for s in st.segments], "video_ids": st.cache_ids(),
                     "memory_version": st.memory_version, "frames": st.cache_frames()})
    return rows


@pytest.mark.parametrize("kv_dtype,grid,window,memory,refresh", [
    ("bf16", (8, 12), 12, 2, 4), ("bf16", (16, 24), 12, 2, 4), ("fp8", (16, 24), 12, 2, 4),
    ("fp8", (8, 16), 12, 2, 4), ("fp8", (8, 12), 12, 2, 4), ("bf16", (4, 6), 6, 1, 2), ("fp8", (8, 8), 6, 1, 2),
    ("fp8", (5, 5), 6, 1, 2), ("bf16", (4, 6), 9, 0, 0)])
def test_chunk_stream_matches_oracle_plan(kv_dtype, grid, window, memory, refresh):
    kw = dict(memory_frames=memory, window_frames=window, refresh_every=refresh)
    rows = _run(grid, kv_dtype, 60, **kw)
    plan = OC.streaming_plan_window(60, grid, **kw) if memory else None
    hw = grid[0] * grid[1]
    for c, r in enumerate(rows):
        n_window = min(c + 1, window // 3)
        assert len(r["segments"]) == 1 + (1 if memory else 0) + n_window
        # cached frames: anchor, memory, then the newest window chunks in order
        exp = [("prefix", 0, 1)] + ([("memory", 1, memory)] if memory else [])
        exp += [("generated", 1 + memory + 3 * j, 3) for j in range(c + 1 - n_window, c + 1)]
        assert r["frames"] == exp
        ids = [i for _, f0, nf in exp for i in range(f0 * hw, (f0 + nf) * hw)]
        assert r["video_ids"] == ids
        if plan is not None:
            p = plan[c]
            assert r["segments"] == p["segments"] and r["video_ids"] == p["video_ids"]
            assert r["memory_version"] == p["memory_version"]


def test_chunk_stream_golden_16x24():
    with open(os.path.join(GOLDEN, "stream_plan_16x24_60.json")) as f:
        gold = json.load(f)
    rows = _run((16, 24), "fp8", 60)
    for r, g in zip(rows, gold):
        v = r["video_ids"]
        assert r["segments"] == g["segments"] and r["memory_version"] == g["memory_version"]
        assert (v[:3], v[-3:], len(v), sum(v)) == (g["video_head"], g["video_tail"], g["video_len"],
                                                   g["video_sum"])


def test_retain_pinned_recent_matches_oracle():
    kinds = ["prefix", "memory", "generated"]
    rng = np.random.default_rng(3)
    for _ in range(200):
        segs = [{"kind": kinds[int(k)]} for k in rng.integers(0, 3, int(rng.integers(0, 12)))]
        for recent in range(0, 5):
            assert retain_pinned_recent(segs, recent) == OC.retain_pinned_recent(segs, recent)


def test_stream_rejects_bad_window():
    with pytest.raises(ValueError):
        IdStream((4, 6), "bf16", window_frames=10)
    IdStream((8, 12), "fp8")            # 96-token frames: tiles are cut at frame boundaries
