"""CPU tests of the model's host logic: the HF checkpoint converter (key
mapping, layouts, lm_head / tied embeddings, fp8 block dequantisation, lazy
safetensors shards), the attention-mask contract of the decoder layer, the
KV-cache (K, V) pair contract, and that the seams' early affinity modulation
schedule has no CPU fallback.  No GPU is touched.
"""

import pytest
import torch

from qmoe import model as qm
from qmoe import weights
from qmoe.attention import KVCache
from qmoe.moe import ExpertMLPs

L, H, E, I, NQ, NKV, D, V = 2, 64, 4, 32, 2, 1, 16, 50


def _config(**kw):
    nc = qm.MoENeuronConfig(batch_size=1, seq_len=16, max_length=16)
    base = dict(num_hidden_layers=L, hidden_size=H, num_experts=E, moe_intermediate_size=I,
                num_attention_heads=NQ, num_key_value_heads=NKV, head_dim=D, vocab_size=V,
                num_experts_per_tok=2, tie_word_embeddings=False)
    base.update(kw)
    return qm.Qwen3MoeInferenceConfig(nc, **base)


def _hf_state_dict(seed=0, prefix="model.", lm_head=True):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    sd = {f"{prefix}embed_tokens.weight": r(V, H), f"{prefix}norm.weight": r(H)}
    if lm_head:
        sd["lm_head.weight"] = r(V, H)
    for l in range(L):
        p = f"{prefix}layers.{l}."
        sd.update({
            f"{p}input_layernorm.weight": r(H), f"{p}post_attention_layernorm.weight": r(H),
            f"{p}self_attn.q_proj.weight": r(NQ * D, H), f"{p}self_attn.k_proj.weight": r(NKV * D, H),
            f"{p}self_attn.v_proj.weight": r(NKV * D, H), f"{p}self_attn.o_proj.weight": r(H, NQ * D),
            f"{p}self_attn.q_norm.weight": r(D), f"{p}self_attn.k_norm.weight": r(D),
            f"{p}mlp.gate.weight": r(E, H),
        })
        for e in range(E):
            sd[f"{p}mlp.experts.{e}.gate_proj.weight"] = r(I, H)
            sd[f"{p}mlp.experts.{e}.up_proj.weight"] = r(I, H)
            sd[f"{p}mlp.experts.{e}.down_proj.weight"] = r(H, I)
    return sd


def bf(t):
    return t.to(torch.bfloat16)


@pytest.mark.parametrize("prefix", ["model.", ""])
def test_converter_key_mapping_and_layouts(prefix):
    """qwen_with_nki.py:8883-8997: q/k/v concatenated in that order, norms and
    router renamed, experts packed so that unpacking gives back the NxDI
    (E, H, 2I) gate_up (gate columns first) and (E, I, H) down."""
    sd = _hf_state_dict(prefix=prefix)
    out = qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config())
    assert torch.equal(out["embed_tokens"], bf(sd[f"{prefix}embed_tokens.weight"]))
    assert torch.equal(out["norm"], bf(sd[f"{prefix}norm.weight"]))
    assert torch.equal(out["lm_head"], bf(sd["lm_head.weight"]))
    for l in range(L):
        p = f"{prefix}layers.{l}."
        lw = out["layers"][l]
        q, k, v = (sd[f"{p}self_attn.{n}_proj.weight"] for n in "qkv")
        assert lw["wqkv"].shape == ((NQ + 2 * NKV) * D, H)
        assert torch.equal(lw["wqkv"][: NQ * D], bf(q))
        assert torch.equal(lw["wqkv"][NQ * D: (NQ + NKV) * D], bf(k))
        assert torch.equal(lw["wqkv"][(NQ + NKV) * D:], bf(v))
        assert torch.equal(lw["wo"], bf(sd[f"{p}self_attn.o_proj.weight"]))
        assert torch.equal(lw["q_norm"], bf(sd[f"{p}self_attn.q_norm.weight"]))
        assert torch.equal(lw["k_norm"], bf(sd[f"{p}self_attn.k_norm.weight"]))
        assert torch.equal(lw["router"], bf(sd[f"{p}mlp.gate.weight"]))
        assert torch.equal(lw["input_layernorm"], bf(sd[f"{p}input_layernorm.weight"]))
        assert torch.equal(lw["post_attention_layernorm"], bf(sd[f"{p}post_attention_layernorm.weight"]))
        gate_up = weights.unpack_gate_up(lw["w13"])  # (E, H, 2I)
        down = weights.unpack_down(lw["w2"])  # (E, I, H)
        for e in range(E):
            ex = f"{p}mlp.experts.{e}."
            assert torch.equal(gate_up[e, :, :I], bf(sd[ex + "gate_proj.weight"]).t())
            assert torch.equal(gate_up[e, :, I:], bf(sd[ex + "up_proj.weight"]).t())
            assert torch.equal(down[e], bf(sd[ex + "down_proj.weight"]).t())


def test_converter_pads_intermediate_with_zero_units():
    """moe_intermediate_pad_size (qwen_with_nki.py:8959-8964): zero units are
    appended to every expert's gate, up and down; each expert's SwiGLU output
    is unchanged, and a padded width the kernels cannot take is refused."""
    import oracle

    sd = _hf_state_dict(seed=3)
    ref = qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config())
    out = qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config(moe_intermediate_pad_size=32))
    x = torch.randn(3, H, generator=torch.Generator().manual_seed(9))
    for l in range(L):
        gu, dn = weights.unpack_gate_up(out["layers"][l]["w13"]), weights.unpack_down(out["layers"][l]["w2"])
        gu0, dn0 = weights.unpack_gate_up(ref["layers"][l]["w13"]), weights.unpack_down(ref["layers"][l]["w2"])
        assert gu.shape == (E, H, 2 * (I + 32)) and dn.shape == (E, I + 32, H)
        assert torch.equal(gu[:, :, :I], gu0[:, :, :I]) and torch.equal(gu[:, :, I + 32: 2 * I + 32], gu0[:, :, I:])
        assert not gu[:, :, I: I + 32].any() and not gu[:, :, 2 * I + 32:].any()
        assert torch.equal(dn[:, :I], dn0) and not dn[:, I:].any()
        for e in range(E):
            a = oracle.expert_swiglu(x, gu[e].float(), dn[e].float())
            b = oracle.expert_swiglu(x, gu0[e].float(), dn0[e].float())
            assert torch.allclose(a, b, rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError, match="multiple of 32"):
        qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config(moe_intermediate_pad_size=16))


def test_converter_lm_head_tied_and_missing():
    sd = _hf_state_dict(lm_head=False)
    out = qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config(tie_word_embeddings=True))
    assert torch.equal(out["lm_head"], out["embed_tokens"])
    with pytest.raises(KeyError, match="lm_head"):
        qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config(tie_word_embeddings=False))
    del sd["model.layers.1.mlp.experts.3.up_proj.weight"]
    with pytest.raises(KeyError, match="up_proj"):
        qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config(tie_word_embeddings=True))


def test_converter_reads_safetensors_shards_lazily(tmp_path):
    """Two shards through SafetensorsDir convert exactly like the in-memory dict."""
    from safetensors.torch import save_file

    sd = {k: bf(v).contiguous() for k, v in _hf_state_dict(seed=5).items()}
    keys = sorted(sd)
    save_file({k: sd[k] for k in keys[::2]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({k: sd[k] for k in keys[1::2]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    lazy = qm.SafetensorsDir(str(tmp_path))
    assert sorted(lazy) == keys and len(lazy) == len(keys)
    a = qm.convert_qwen3_moe_hf_to_neuron_state_dict(lazy, _config())
    b = qm.convert_qwen3_moe_hf_to_neuron_state_dict(sd, _config())
    assert torch.equal(a["lm_head"], b["lm_head"]) and torch.equal(a["embed_tokens"], b["embed_tokens"])
    for la, lb in zip(a["layers"], b["layers"]):
        for name in la:
            assert torch.equal(la[name], lb[name]), name
    empty = tmp_path / "no_shards"
    empty.mkdir()
    with pytest.raises(ValueError, match="safetensors"):
        qm.SafetensorsDir(str(empty))


def _fp8_exact(rows, cols, block, seed):
    """A weight whose every value is an fp8 e4m3 number times a power-of-two
    block scale: dequantising its fp8 part with those scales is exact."""
    g = torch.Generator().manual_seed(seed)
    w8 = (torch.randn(rows, cols, generator=g) * 4).to(torch.float8_e4m3fn)
    nb0, nb1 = -(-rows // block[0]), -(-cols // block[1])
    scale = 2.0 ** torch.randint(-6, 3, (nb0, nb1), generator=g).float()
    full = torch.empty(rows, cols)
    for i in range(nb0):  # brute force, one block at a time
        for j in range(nb1):
            r0, c0 = i * block[0], j * block[1]
            full[r0:r0 + block[0], c0:c0 + block[1]] = w8[r0:r0 + block[0], c0:c0 + block[1]].float() * scale[i, j]
    return w8, scale, full


@pytest.mark.parametrize("rows,cols,block", [(256, 384, (128, 128)), (200, 130, (64, 32)), (7, 5, (4, 4))])
def test_fp8_block_dequant(rows, cols, block):
    """qwen_with_nki.py:8865-8880: every element scaled by its block's
    scale_inv; exact against a per-block brute force, partial blocks included."""
    w8, scale, full = _fp8_exact(rows, cols, block, rows + cols)
    got = qm.dequantize_fp8_block(w8, scale, list(block), dtype=torch.float32)
    assert torch.equal(got, full)
    assert torch.equal(qm.dequantize_fp8_block(w8, scale, block), full.to(torch.bfloat16))
    with pytest.raises(ValueError, match="tile"):
        qm.dequantize_fp8_block(w8, scale[:-1], block)
    with pytest.raises(ValueError, match="weight_block_size"):
        qm.dequantize_fp8_block(w8, scale, None)


def test_converter_dequantizes_fp8_weights():
    """A checkpoint whose expert and attention weights are fp8 with
    ``*_scale_inv`` partners converts to the dequantised values."""
    sd = _hf_state_dict(seed=9)
    block = [16, 16]
    expect = {}
    for name in ["model.layers.0.self_attn.q_proj.weight", "model.layers.1.mlp.experts.2.down_proj.weight",
                 "model.layers.0.mlp.experts.0.gate_proj.weight"]:
        r, c = sd[name].shape
        w8, scale, full = _fp8_exact(r, c, block, len(name))
        sd[name], sd[name + "_scale_inv"] = w8, scale
        expect[name] = full
    out = qm.convert_qwen3_moe_hf_to_neuron_state_dict(
        sd, _config(quantization_config={"weight_block_size": block}))
    assert torch.equal(out["layers"][0]["wqkv"][: NQ * D], bf(expect["model.layers.0.self_attn.q_proj.weight"]))
    assert torch.equal(weights.unpack_down(out["layers"][1]["w2"])[2],
                       bf(expect["model.layers.1.mlp.experts.2.down_proj.weight"]).t())
    assert torch.equal(weights.unpack_gate_up(out["layers"][0]["w13"])[0, :, :I],
                       bf(expect["model.layers.0.mlp.experts.0.gate_proj.weight"]).t())


def test_causal_mask_contract():
    pos = torch.zeros(2, 1, dtype=torch.int64)
    qm._check_causal_mask(None, pos)
    qm._check_causal_mask(torch.ones(2, 7), pos)
    qm._check_causal_mask(torch.tensor([[1, 1, 1, 0], [1, 1, 1, 1]]), pos)  # right padding
    with pytest.raises(ValueError, match="right-padded"):
        qm._check_causal_mask(torch.tensor([[0, 1, 1, 1], [1, 1, 1, 1]]), pos)  # left padding
    with pytest.raises(ValueError, match="right-padded"):
        qm._check_causal_mask(torch.tensor([[1, 0, 1, 1], [1, 1, 1, 1]]), pos)
    with pytest.raises(ValueError, match="0/1"):
        qm._check_causal_mask(torch.tensor([[1, 2], [1, 1]]), pos)
    with pytest.raises(ValueError, match="causal"):
        qm._check_causal_mask(torch.ones(2, 1, 4, 4), pos)
    with pytest.raises(ValueError, match="causal"):
        qm._check_causal_mask(torch.ones(3, 4), pos)


def test_kv_cache_pair_contract():
    with pytest.raises(ValueError, match="KVCache or a \\(K, V\\) pair"):
        KVCache.wrap((torch.zeros(1),))
    with pytest.raises(ValueError, match="GPU tensor"):
        KVCache.wrap((torch.zeros(1, 1, 4, 128, dtype=torch.bfloat16),) * 2)
    c = KVCache.__new__(KVCache)
    c.k, c.v = torch.zeros(1), torch.ones(1)
    k, v = c
    assert k is c.k and v is c.v and c[0] is c.k and c[1] is c.v and len(c) == 2
    assert KVCache.wrap(c) is c


def test_seams_early_affinity_modulation_has_no_cpu_fallback():
    """qwen_with_nki.py:5768-5775 (prefill) and 3449 (decode): the flag is off
    by default (Qwen3's setting); set, both seams take the early schedule,
    which runs on the HIP kernels only and so refuses host tensors."""
    ex = ExpertMLPs(torch.zeros(4, 64, 512, dtype=torch.bfloat16), torch.zeros(4, 4, 512, 8, dtype=torch.bfloat16), 2)
    assert ex.routed_experts_mlp_config.early_expert_affinity_modulation is False
    ex.routed_experts_mlp_config.early_expert_affinity_modulation = True
    x = torch.zeros(3, 512)
    masked = torch.zeros(3, 4)
    masked[:, :2] = 0.5
    tpid = torch.tensor([0, 1, 2, 3, 0, 1, 2, 3], dtype=torch.long)
    with pytest.raises(ValueError, match="must be on a GPU"):
        ex.torch_blockwise_matmul_inference(4, 2, x, masked, tpid, torch.tensor([0, 1], dtype=torch.long))
    with pytest.raises(ValueError, match="must be on a GPU"):
        ex.forward_selective_loading(x, torch.zeros(3, 4), torch.zeros(3, 2, dtype=torch.long))
