"""Pin the oracle against the golden fixtures written from transformers.

The fixtures (tests/golden/*.npz) come from transformers' Qwen3-MoE modules,
an implementation independent of the oracle.  A dropped term, a transposed
operand or a wrong index in the oracle fails one of these.
"""

import os

import numpy as np
import pytest
import torch

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


def test_rmsnorm_reference_recipe():
    # nki_custom_rmsnorm.py:182-214: seed 42, x (256,512) randn, w randn, eps 1e-6,
    # PASS if max|diff| < 1e-3.  We hold the oracle to 1e-5.
    g = _load("rmsnorm_seed42.npz")
    np.random.seed(42)
    x = np.random.randn(256, 512).astype(np.float32)
    w = np.random.randn(512).astype(np.float32)
    y = oracle.rmsnorm(torch.from_numpy(x), torch.from_numpy(w), float(g["eps"])).numpy()
    assert np.max(np.abs(y[:32] - g["y_head"])) < 1e-5
    y64 = y.astype(np.float64)
    assert abs(y64.sum() - float(g["y_sum"])) < 1e-2
    assert abs((y64 * y64).sum() / float(g["y_sumsq"]) - 1.0) < 1e-6
    # float64 closed form of the recipe (numpy_rmsnorm, nki_custom_rmsnorm.py:174-179)
    x64 = x.astype(np.float64)
    ref64 = x64 / np.sqrt(np.mean(x64 ** 2, axis=-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(y - ref64)) < 1e-3


def _moe_inputs():
    g = _load("moe_block_small.npz")
    x = torch.from_numpy(g["x"])
    router = torch.from_numpy(g["router"])
    gate_up_hf = torch.from_numpy(g["gate_up_hf"])  # (E, 2I, H)
    down_hf = torch.from_numpy(g["down_hf"])  # (E, H, I)
    # NxDI layout (qwen_with_nki.py:8928-8990): gate_up (E,H,2I), down (E,I,H)
    gate_up = gate_up_hf.transpose(1, 2).contiguous()
    down = down_hf.transpose(1, 2).contiguous()
    return g, x, router, gate_up, down


def test_router_matches_transformers():
    g, x, router, _, _ = _moe_inputs()
    k = int(g["k"])
    logits, top_w, top_i = oracle.router_topk(x, router, k)
    np.testing.assert_allclose(logits.numpy(), g["logits"], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(top_i.numpy(), g["top_i"])
    np.testing.assert_allclose(top_w.numpy(), g["top_w"], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("fn", ["moe_block_prefill", "moe_block_decode"])
def test_moe_block_matches_transformers(fn):
    g, x, router, gate_up, down = _moe_inputs()
    k = int(g["k"])
    out, top_i, _, _ = getattr(oracle, fn)(x, router, gate_up, down, k)
    np.testing.assert_array_equal(top_i.numpy(), g["top_i"])
    np.testing.assert_allclose(out.numpy(), g["y"], rtol=1e-4, atol=1e-6)


def _attn_weights(g, prefix=""):
    key = lambda n: (prefix + n).replace(".", "_")
    return {
        "q_proj": torch.from_numpy(g[key("q_proj.weight")]),
        "k_proj": torch.from_numpy(g[key("k_proj.weight")]),
        "v_proj": torch.from_numpy(g[key("v_proj.weight")]),
        "o_proj": torch.from_numpy(g[key("o_proj.weight")]),
        "q_norm": torch.from_numpy(g[key("q_norm.weight")]),
        "k_norm": torch.from_numpy(g[key("k_norm.weight")]),
    }


CFG_SMALL = dict(n_q=4, n_kv=2, head_dim=16, eps=1e-6, theta=1.0e6, top_k=2)


def test_rope_tables_match_transformers():
    g = _load("attention_small.npz")
    cos, sin = oracle.rope_tables(16, torch.from_numpy(g["pos"]), 1.0e6)
    np.testing.assert_allclose(cos.numpy(), g["cos"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(sin.numpy(), g["sin"], rtol=0, atol=1e-6)


def test_attention_matches_transformers():
    g = _load("attention_small.npz")
    w = _attn_weights(g)
    out, _ = oracle.attention_layer(torch.from_numpy(g["x"]), w, torch.from_numpy(g["pos"]), CFG_SMALL)
    np.testing.assert_allclose(out.numpy(), g["out"], rtol=1e-4, atol=1e-5)


def test_decoder_layer_matches_transformers():
    g = _load("decoder_layer_small.npz")
    w = _attn_weights(g, "self_attn.")
    w["input_layernorm"] = torch.from_numpy(g["input_layernorm_weight"])
    w["post_attention_layernorm"] = torch.from_numpy(g["post_attention_layernorm_weight"])
    w["router"] = torch.from_numpy(g["mlp_gate_weight"])
    w["gate_up_proj"] = torch.from_numpy(g["mlp_experts_gate_up_proj"]).transpose(1, 2).contiguous()
    w["down_proj"] = torch.from_numpy(g["mlp_experts_down_proj"]).transpose(1, 2).contiguous()
    out, _ = oracle.decoder_layer(torch.from_numpy(g["x"]), w, torch.from_numpy(g["pos"]), CFG_SMALL)
    np.testing.assert_allclose(out.numpy(), g["out"], rtol=1e-4, atol=1e-5)


def test_live_transformers_moe_block_if_available():
    """Same check as the fixture, regenerated live at a second shape."""
    tf = pytest.importorskip("transformers")
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe import modeling_qwen3_moe as tfm

    cfg = Qwen3MoeConfig(hidden_size=32, moe_intermediate_size=16, num_experts=6,
                         num_experts_per_tok=3, norm_topk_prob=True, num_hidden_layers=1)
    gen = torch.Generator().manual_seed(5)
    blk = tfm.Qwen3MoeSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(0.1 * torch.randn(p.shape, generator=gen))
        x = torch.randn(1, 9, 32, generator=gen)
        ref = blk(x).view(9, 32)
    with torch.no_grad():
        out, _, _, _ = oracle.moe_block_prefill(
            x.view(9, 32), blk.gate.weight, blk.experts.gate_up_proj.transpose(1, 2),
            blk.experts.down_proj.transpose(1, 2), 3)
    np.testing.assert_allclose(out.numpy(), ref.numpy(), rtol=1e-4, atol=1e-6)
    assert tf.__version__
