"""The generator's parameter names and shapes against the reference's, read
from its module definitions (the fixture tests/golden/reference_param_names.json,
written by tests/golden/make_param_names.py from ltx_causal/transformer/
causal_model.py:237-420, causal_block.py:108-376, compat.py and
ltx_causal/attention/causal_attention.py:92-118 with ``ast``).

* the product's AVModel at the 22B configuration has exactly the reference's
  parameters, with the same shapes, with and without the production options
  (gated attention, learned-memory adapters on every 4th block, colour FiLM);
* save_generator writes exactly those names under the wrapper's ``model.``
  prefix (taomate/inference/model_runtime.py:226-232), and detect_config reads
  the production configuration back from tensors of the reference's shapes.
"""
import json
import os

import pytest
import torch

from taomate_amd import checkpoint as C
from taomate_amd import dit as D

FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "reference_param_names.json")

PRODUCTION = dict(apply_gated_attention=True, learned_memory_enabled=True, learned_memory_mode="memory_kv_side_branch",
                  learned_memory_layer_interval=4, learned_memory_video_dim=512, learned_memory_audio_dim=256,
                  learned_memory_heads=8, learned_memory_color_film_enabled=True,
                  learned_memory_color_condition_dim=512, learned_memory_color_film_hidden_dim=256)


def _reference(name):
    with open(FIXTURE) as f:
        c = json.load(f)["configs"][name]
    out = {k: tuple(v) for k, v in c["top"].items()}
    for i in range(c["num_layers"]):
        kind = "adapter" if i in c["adapter_blocks"] else "plain"
        for k, v in c["block"][kind].items():
            out[f"transformer_blocks.{i}.{k}"] = tuple(v)
    assert len(out) == c["total"]
    return out


def _product(cfg):
    with torch.device("meta"):
        m = D.AVModel(cfg)
    return m, {k: tuple(v.shape) for k, v in m.state_dict().items()}


@pytest.mark.parametrize("name,extra", [("base", {}), ("production", PRODUCTION),
                                        ("ltx23", dict(PRODUCTION, cross_attention_adaln=True))])
def test_parameter_names_and_shapes_match_reference(name, extra):
    ref = _reference(name)
    _, got = _product(D.AVConfig(**extra))
    assert set(got) == set(ref), (sorted(set(got) - set(ref))[:5], sorted(set(ref) - set(got))[:5])
    bad = [k for k in ref if got[k] != ref[k]]
    assert not bad, [(k, got[k], ref[k]) for k in bad[:5]]


@pytest.mark.parametrize("name,adaln", [("production", False), ("ltx23", True)])
def test_detect_config_reads_reference_shapes(name, adaln):
    """A state dict with the reference's production names and shapes (meta
    tensors) detects to the production configuration and loads strictly; the
    LTX-2.3 layout (9-row modulation tables, prompt tables) detects with the
    text cross-attention AdaLN."""
    ref = _reference(name)
    sd = {k: torch.empty(v, device="meta") for k, v in ref.items()}
    cfg = C.detect_config(sd, learned_memory_mode="memory_kv_side_branch")
    want = D.AVConfig(**PRODUCTION, cross_attention_adaln=adaln)
    for f in ("num_layers", "video_dim", "audio_dim", "video_heads", "audio_heads", "video_d_head", "audio_d_head",
              "in_channels", "out_channels", "cross_attention_adaln") + tuple(PRODUCTION):
        assert getattr(cfg, f) == getattr(want, f), f
    m, _ = _product(cfg)
    missing, unexpected = m.load_state_dict(sd, strict=False, assign=True)
    assert not missing and not unexpected


def test_saved_keys_are_reference_names(tmp_path):
    """save_generator's keys: the wrapper's ``model.`` prefix plus the
    reference's names, on a reduced-width model of the production layout
    (the names do not depend on the widths)."""
    small = dict(num_layers=4, video_dim=256, audio_dim=128, video_heads=2, audio_heads=2, video_d_head=128,
                 audio_d_head=64)
    model = D.build_model(D.AVConfig(**small, **PRODUCTION), "cpu", seed=2, dtype=torch.float32)
    path = str(tmp_path / "gen.pt")
    C.save_generator(model, path)
    keys = set(torch.load(path, weights_only=True)["generator_ema"])
    ref = {k for k in _reference("production") if not k.startswith("transformer_blocks.")
           or int(k.split(".")[1]) < 4}
    assert keys == {"model." + k for k in ref}
