"""CPU oracle for the Qwen3-30B-A3B decoder-layer hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker / the timed CPU baseline.

The oracle restates, in fp32 PyTorch-on-CPU (and numpy for the integer
dispatch bookkeeping), the math that charleshong3/nki-moe-7013 delegates to
NxDI / neuronx_distributed / transformers.  Each function cites the reference
file:line it follows.  How each function is pinned (independent
implementation, closed form, invariant or brute force) is listed in
``PINNING`` below and exercised by ``tests/test_oracle_*.py``.
"""

from .qwen3_moe import (  # noqa: F401
    PINNING,
    rmsnorm,
    router_topk,
    moe_permute,
    expert_swiglu,
    moe_block_prefill,
    moe_block_decode,
    moe_experts_early,
    moe_block,
    rope_tables,
    apply_rope,
    qkv_norm_rope,
    gqa_attention,
    attention_layer,
    decoder_layer,
    pack_w13,
)
