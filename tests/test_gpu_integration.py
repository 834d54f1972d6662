"""The drop-in path on a module built like the reference's: attention_with_cache
on a plain nn.Module that carries only the attributes of CausalLTXAttention
(causal_attention.py:92-118), starting from the reference's empty cache (every
field None, wrapper.py:15-20), against the fp32 oracle."""
import pytest
import torch
import torch.nn as nn

import taomate_amd as T

from .helpers import assert_bf16_close, cosine
from .test_gpu_layer import SEGS_SMALL, _layer_reference, gpu_pe, make_layer

pytestmark = pytest.mark.gpu


class ReferenceShapedAttention(nn.Module):
    """Exactly the attributes the reference module sets (causal_attention.py:92-118)."""

    def __init__(self, query_dim, context_dim=None, heads=8, dim_head=64, norm_eps=1e-6):
        super().__init__()
        self.rope_type = T.CausalRopeType.SPLIT
        self.heads = heads
        self.dim_head = dim_head
        self.inner_dim = heads * dim_head
        self.is_cross_attention = context_dim is not None
        context_dim = query_dim if context_dim is None else context_dim
        self.to_q = nn.Linear(query_dim, self.inner_dim, bias=True)
        self.to_k = nn.Linear(context_dim, self.inner_dim, bias=True)
        self.to_v = nn.Linear(context_dim, self.inner_dim, bias=True)
        self.q_norm = nn.RMSNorm(self.inner_dim, eps=norm_eps)
        self.k_norm = nn.RMSNorm(self.inner_dim, eps=norm_eps)
        self.to_gate_logits = None
        self.to_out = nn.Sequential(nn.Linear(self.inner_dim, query_dim, bias=True), nn.Identity())


def _reference_shaped(dev, d, H, Dh, seed):
    ours, w = make_layer(dev, d, H, Dh, seed)
    ref = ReferenceShapedAttention(d, heads=H, dim_head=Dh).to(dev, torch.bfloat16)
    ref.load_state_dict(ours.state_dict())
    assert not hasattr(ref, "_packed_qkv") and not hasattr(ref, "fuse_qkv_")
    return ref, w


@pytest.mark.parametrize("arena", [True, False], ids=["module_arena", "dense"])
def test_attention_with_cache_on_reference_shaped_module(dev, arena):
    """Prefill anchor | memory | window through attention_with_cache from an
    empty cache, then the 2-frame chunk over all of it (8x12 grid, 8 x 64
    heads, d = 512).  arena: the module carries an arena plan, so the first
    append of the None field already lands in arena slots; dense: no plan,
    the cache is plain [B, L, H, D] tensors as in the reference."""
    B, gh, gw, H, Dh, seed = 1, 8, 12, 8, 64, 0
    d, hw = H * Dh, gh * gw
    attn, w = _reference_shaped(dev, d, H, Dh, seed)
    if arena:
        T.attach_arena(attn, (6 + 2) * hw, name="video_self")
    xs, xc, ref, ref_k = _layer_reference(B, gh, gw, H, Dh, seed, w)
    cache = T.KVCache(layers=[T.LayerKVCache()])
    lay = cache.layers[0]
    kc, vc = lay.video_self_k, lay.video_self_v
    assert kc is None and vc is None
    with torch.no_grad():
        for (_, f0, nf), x in zip(SEGS_SMALL, xs):
            _, nk, nv = T.attention_with_cache(attn, x.to(dev, torch.bfloat16), None,
                                               gpu_pe(dev, (nf, gh, gw), d, H, f0, B), None, kc, vc)
            assert isinstance(nk, T.KVSpanView) == arena
            kc, vc = T._cat_cache(kc, nk), T._cat_cache(vc, nv)
        out, nk, nv = T.attention_with_cache(attn, xc.to(dev, torch.bfloat16), None,
                                             gpu_pe(dev, (2, gh, gw), d, H, 10, B), None, kc, vc)
    torch.cuda.synchronize()
    assert kc.shape == (B, 6 * hw, H, Dh) and nk.shape == (B, 2 * hw, H, Dh)
    assert_bf16_close(out, ref, f"reference-shaped module ({'arena' if arena else 'dense'})")
    new_k = nk.materialize() if arena else nk
    assert cosine(new_k, ref_k) >= 0.9999
    assert cosine(out, ref) >= 0.9999
