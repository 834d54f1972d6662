"""Writes eviction_plan_16x24_60.json: the kept-token summary after each of 60
block commits (4-3-3-3 blocks, 16x24 latent grid, sink + 2 recent blocks),
produced by the oracle's replay of the commit/evict loop
(taomate/inference/model.py:202-246 with cache.py:58-67)."""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
from oracle import cache as OC  # noqa: E402

plan = OC.streaming_plan(60, (16, 24))
out = [{"block_idx": p["block_idx"], "segments": p["segments"], "video_head": p["video_ids"][:3],
        "video_len": len(p["video_ids"]), "video_sum": sum(p["video_ids"]),
        "audio_sum": sum(p["audio_ids"])} for p in plan]
path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "eviction_plan_16x24_60.json")
with open(path, "w") as f:
    json.dump(out, f, indent=0)
print(path)
