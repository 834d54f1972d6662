"""Writes the eviction-plan fixtures, produced by the oracle's replays of the
commit/evict loop (taomate/inference/model.py:202-246 with cache.py:58-67):

* eviction_plan_16x24_60.json: the kept-token summary after each of 60 block
  commits (4-3-3-3 blocks, 16x24 latent grid, sink + 2 recent blocks);
* stream_plan_16x24_60.json: the same after each of 60 chunk commits of the
  anchor (1 frame) | memory (2 frames, re-prefilled every 4 chunks) | window
  (12 frames) stream of 3-frame chunks on the 16x24 grid.
"""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
from oracle import cache as OC  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

plan = OC.streaming_plan(60, (16, 24))
out = [{"block_idx": p["block_idx"], "segments": p["segments"], "video_head": p["video_ids"][:3],
        "video_len": len(p["video_ids"]), "video_sum": sum(p["video_ids"]),
        "audio_sum": sum(p["audio_ids"])} for p in plan]
path = os.path.join(HERE, "eviction_plan_16x24_60.json")
with open(path, "w") as f:
    json.dump(out, f, indent=0)
print(path)

plan = OC.streaming_plan_window(60, (16, 24))
out = [{"chunk": p["chunk"], "segments": p["segments"], "memory_version": p["memory_version"],
        "video_head": p["video_ids"][:3], "video_tail": p["video_ids"][-3:], "video_len": len(p["video_ids"]),
        "video_sum": sum(p["video_ids"])} for p in plan]
path = os.path.join(HERE, "stream_plan_16x24_60.json")
with open(path, "w") as f:
    json.dump(out, f, indent=0)
print(path)
