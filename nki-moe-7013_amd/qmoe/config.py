"""Model shape of Qwen3-30B-A3B (hot-path constants)."""

from __future__ import annotations

from dataclasses import dataclass, asdict


@dataclass
class Qwen3MoeShape:
    """Architecture constants.  Defaults are Qwen3-30B-A3B.

    Note: transformers' ``Qwen3MoeConfig`` defaults (24 layers,
    ``norm_topk_prob=False``) are not 30B-A3B; the reference forces top-k
    renormalisation regardless (qwen_with_nki.py:9894).
    """

    hidden_size: int = 2048
    num_hidden_layers: int = 48
    num_experts: int = 128
    num_experts_per_tok: int = 8
    moe_intermediate_size: int = 768
    num_attention_heads: int = 32
    num_key_value_heads: int = 4
    head_dim: int = 128
    vocab_size: int = 151936
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1.0e6
    max_position_embeddings: int = 40960
    norm_topk_prob: bool = True
    tie_word_embeddings: bool = False
    hidden_act: str = "silu"

    def to_dict(self):
        return asdict(self)


QWEN3_30B_A3B = Qwen3MoeShape()
