"""CPU round trips of the disk formats: a generator checkpoint in the
load_model_generator layout (config detected from the tensors, every
parameter restored), the refusal of features this build does not run, and
the version-2 interactive prefix state with a learned-memory state."""
import json
import os

import pytest
import torch

from taomate_amd import checkpoint as C
from taomate_amd import dit as D
from taomate_amd.memory import StreamingMemory
from taomate_amd.prefix_state import build_prefix_state_payload, load_prefix_state, save_prefix_state

SMALL = dict(num_layers=4, video_dim=256, audio_dim=128, video_heads=2, audio_heads=2, video_d_head=128,
             audio_d_head=64)


@pytest.mark.parametrize("fmt", ["pt", "safetensors"])
@pytest.mark.parametrize("extras", [{}, dict(learned_memory_enabled=True, learned_memory_color_film_enabled=True,
                                              learned_memory_video_dim=512, learned_memory_audio_dim=256,
                                              apply_gated_attention=True)])
def test_generator_round_trip(tmp_path, fmt, extras):
    cfg = D.AVConfig(**SMALL, **extras)
    model = D.build_model(cfg, "cpu", seed=7, dtype=torch.float32)
    path = str(tmp_path / f"gen.{fmt}")
    C.save_generator(model, path)
    if fmt == "pt":   # the reference's layout: {"generator_ema": {"model.<name>": tensor}}
        raw = torch.load(path, weights_only=True)
        assert set(raw) == {"generator_ema"} and all(k.startswith("model.") for k in raw["generator_ema"])
    got = C.load_generator(path, device="cpu", dtype=torch.float32)
    for f in ("num_layers", "video_dim", "audio_dim", "video_heads", "audio_heads", "in_channels", "out_channels",
              "learned_memory_enabled", "learned_memory_color_film_enabled", "apply_gated_attention",
              "learned_memory_video_dim", "learned_memory_audio_dim"):
        assert getattr(got.cfg, f) == getattr(cfg, f), f
    ref = dict(model.state_dict())
    out = dict(got.state_dict())
    assert set(ref) == set(out)
    assert all(torch.equal(ref[k], out[k]) for k in ref)


def test_generator_refuses_unbuilt_features(tmp_path):
    model = D.build_model(D.AVConfig(**SMALL), "cpu", seed=1, dtype=torch.float32)
    sd = {"model." + k: v for k, v in model.state_dict().items()}
    sd["model.audio_sink_tokens"] = torch.zeros(16, 128)
    path = str(tmp_path / "sink.pt")
    torch.save({"generator_ema": sd}, path)
    with pytest.raises(NotImplementedError, match="audio sink tokens"):
        C.load_generator(path, device="cpu")
    torch.save({"other": sd}, path)
    with pytest.raises(ValueError, match="EMA checkpoint"):
        C.load_generator(path, device="cpu")
    # a missing parameter is an error, not a silent zero
    sd.pop("model.audio_sink_tokens")
    sd.pop("model.proj_out.bias")
    torch.save({"generator_ema": sd}, path)
    with pytest.raises(ValueError, match="lacks"):
        C.load_generator(path, device="cpu")


def test_prefix_state_round_trip(tmp_path):
    g = torch.Generator().manual_seed(5)
    mem = StreamingMemory()
    v = torch.randn(1, 4, 128, 16, 24, generator=g)
    a = torch.randn(1, 26, 128, generator=g)
    mem.set_reference(v, a)
    mem.update(v * 1.1, a)
    payload = build_prefix_state_payload(case_id="case-7", window_count=3, prefix_video_latent=v,
                                         prefix_audio_latent=a, prefix_source_prompts=["a cat", "a dog"],
                                         sink_video_latent=v[:, :1], sink_source_prompt="a cat",
                                         learned_memory_state=mem)
    path = str(tmp_path / "state" / "prefix.safetensors")
    assert save_prefix_state(path, payload) and not save_prefix_state(None, payload)
    assert [p for p in os.listdir(tmp_path / "state")] == ["prefix.safetensors"]   # no temporary left
    got = load_prefix_state(path, device="cpu", dtype=torch.float32)
    assert got["version"] == 2 and got["case_id"] == "case-7" and got["block_count"] == 15
    assert got["prefix_source_prompts"] == ["a cat", "a dog"] and got["sink_source_prompt"] == "a cat"
    assert torch.equal(got["prefix_video_latent"], v) and got["decode_prefix_video_latent"] is None
    m2 = got["learned_memory_state"]
    assert m2.color_film_enabled and m2.drift_gate_enabled and m2.reference_initialized
    for name in ("video", "audio", "video_anchor", "audio_anchor", "color_proto", "color_anchor_proto"):
        assert torch.equal(getattr(m2, name), getattr(mem, name)), name
    assert all(torch.equal(x, y) for x, y in zip(m2.color_stats, mem.color_stats))
    c1, c2 = mem.with_conditional_memory({}), m2.with_conditional_memory({})
    assert all(torch.equal(c1[k], c2[k]) for k in c1)
    # cached until the file changes
    assert load_prefix_state(path, device="cpu", dtype=torch.float32)["case_id"] == "case-7"
    payload["case_id"] = "case-8"
    save_prefix_state(path, payload)
    assert load_prefix_state(path, device="cpu", dtype=torch.float32)["case_id"] == "case-8"
    # the file is plain safetensors: tensors plus JSON metadata
    from safetensors import safe_open
    with safe_open(path, framework="pt") as f:
        assert json.loads(f.metadata()["prefix_state"])["window_count"] == 3
    assert load_prefix_state(str(tmp_path / "none.safetensors"), device="cpu") is None
