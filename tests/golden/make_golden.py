"""Write the golden fixtures in this folder from transformers' Qwen3-MoE modules.

transformers (``transformers.models.qwen3_moe.modeling_qwen3_moe``, version
printed into the fixture) is the third-party library the reference delegates
its CPU math to (qwen_with_nki.py:6, 40-42, 9048-9058).  It is an implementation
independent of the oracle, so these vectors pin the oracle's router, MoE block,
RMSNorm, RoPE, attention and decoder layer.  The reference itself is never
imported (it needs the absent Neuron SDK and downloads a model at import).

Run:  python tests/golden/make_golden.py   (CPU, a few seconds)
Shapes are tiny on purpose; fixtures are float32 .npz files of a few hundred KB.
"""

from __future__ import annotations

import os

import numpy as np
import torch
import transformers
from transformers import Qwen3MoeConfig
from transformers.models.qwen3_moe import modeling_qwen3_moe as tfm

HERE = os.path.dirname(os.path.abspath(__file__))


def _cfg():
    cfg = Qwen3MoeConfig(
        hidden_size=64,
        num_attention_heads=4,
        num_key_value_heads=2,
        head_dim=16,
        moe_intermediate_size=32,
        intermediate_size=64,
        num_experts=8,
        num_experts_per_tok=2,
        norm_topk_prob=True,
        num_hidden_layers=1,
        vocab_size=128,
        rope_theta=1.0e6,
        rms_norm_eps=1e-6,
        max_position_embeddings=16384,
    )
    cfg._attn_implementation = "eager"
    return cfg


def _init(module, gen, std=0.02):
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=gen))
            else:
                p.copy_(std * torch.randn(p.shape, generator=gen))


def _causal_mask(B, S):
    m = torch.full((S, S), float("-inf")).triu(1)
    return m.view(1, 1, S, S).expand(B, 1, S, S)


def rmsnorm_fixture():
    # The reference's known-answer recipe: nki_custom_rmsnorm.py:182-214.
    np.random.seed(42)
    x = np.random.randn(256, 512).astype(np.float32)
    w = np.random.randn(512).astype(np.float32)
    mod = tfm.Qwen3MoeRMSNorm(512, eps=1e-6)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w))
        y = mod(torch.from_numpy(x)).numpy()
    # x and w are regenerated from the seed by the test; keep 32 output rows
    # plus float64 checksums of the whole output.
    y64 = y.astype(np.float64)
    np.savez_compressed(
        os.path.join(HERE, "rmsnorm_seed42.npz"),
        y_head=y[:32], y_sum=y64.sum(), y_sumsq=(y64 * y64).sum(), eps=np.float32(1e-6),
    )


def router_moe_fixture():
    cfg = _cfg()
    gen = torch.Generator().manual_seed(1234)
    blk = tfm.Qwen3MoeSparseMoeBlock(cfg)
    _init(blk, gen, std=0.05)
    T = 24
    x = torch.randn(1, T, cfg.hidden_size, generator=gen)
    with torch.no_grad():
        logits, top_w, top_i = blk.gate(x.view(T, -1))
        y = blk(x).view(T, -1)
    np.savez_compressed(
        os.path.join(HERE, "moe_block_small.npz"),
        x=x.view(T, -1).numpy(),
        router=blk.gate.weight.detach().numpy(),
        gate_up_hf=blk.experts.gate_up_proj.detach().numpy(),  # (E, 2I, H)
        down_hf=blk.experts.down_proj.detach().numpy(),  # (E, H, I)
        logits=logits.numpy(),
        top_w=top_w.numpy(),
        top_i=top_i.numpy().astype(np.int64),
        y=y.numpy(),
        k=np.int64(cfg.num_experts_per_tok),
    )


def attention_fixture():
    cfg = _cfg()
    gen = torch.Generator().manual_seed(99)
    att = tfm.Qwen3MoeAttention(cfg, 0)
    _init(att, gen, std=0.1)
    rot = tfm.Qwen3MoeRotaryEmbedding(cfg)
    B, S = 2, 12
    x = torch.randn(B, S, cfg.hidden_size, generator=gen)
    # second batch row starts at a large position to exercise theta = 1e6
    pos = torch.stack([torch.arange(S), torch.arange(8000, 8000 + S)])
    with torch.no_grad():
        cos, sin = rot(x, pos)
        out, _ = att(x, (cos, sin), _causal_mask(B, S))
    sd = {n: p.detach().numpy() for n, p in att.named_parameters()}
    np.savez_compressed(
        os.path.join(HERE, "attention_small.npz"),
        x=x.numpy(), pos=pos.numpy(), cos=cos.numpy(), sin=sin.numpy(), out=out.numpy(),
        **{k.replace(".", "_"): v for k, v in sd.items()},
    )


def decoder_layer_fixture():
    cfg = _cfg()
    gen = torch.Generator().manual_seed(7)
    layer = tfm.Qwen3MoeDecoderLayer(cfg, 0)
    _init(layer, gen, std=0.05)
    rot = tfm.Qwen3MoeRotaryEmbedding(cfg)
    B, S = 1, 10
    x = torch.randn(B, S, cfg.hidden_size, generator=gen)
    pos = torch.arange(S).view(1, S)
    with torch.no_grad():
        cos, sin = rot(x, pos)
        out = layer(x, attention_mask=_causal_mask(B, S), position_ids=pos, position_embeddings=(cos, sin))
        if isinstance(out, tuple):
            out = out[0]
    sd = {n: p.detach().numpy() for n, p in layer.named_parameters()}
    np.savez_compressed(
        os.path.join(HERE, "decoder_layer_small.npz"),
        x=x.numpy(), pos=pos.numpy(), out=out.numpy(),
        **{k.replace(".", "_"): v for k, v in sd.items()},
    )


def main():
    torch.set_num_threads(1)
    rmsnorm_fixture()
    router_moe_fixture()
    attention_fixture()
    decoder_layer_fixture()
    with open(os.path.join(HERE, "SOURCE.txt"), "w") as f:
        f.write(
            "Fixtures written by tests/golden/make_golden.py from transformers "
            f"{transformers.__version__} (torch {torch.__version__}), float32 CPU.\n"
        )
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
