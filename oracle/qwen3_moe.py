"""fp32 CPU restatement of the Qwen3-30B-A3B decoder-layer math.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the product path never
imports this module.

Weights are taken in the reference's own on-device layout, the one produced by
``convert_qwen3_moe_hf_to_neuron_state_dict`` (qwen_with_nki.py:8883-8997,
= qwen.py:119-233):

* ``gate_up_proj``  ``(E, H, 2I)``  gate columns ``[0, I)``, up ``[I, 2I)``
  (qwen_with_nki.py:8928-8966)
* ``down_proj``     ``(E, I, H)``   (qwen_with_nki.py:8968-8990)
* ``router``        ``(E, H)``      renamed from HF ``mlp.gate.weight``
  (qwen_with_nki.py:8915-8919)
* q/k/v/o projections in ``nn.Linear`` layout ``(out, in)``; ``q_norm`` /
  ``k_norm`` ``(D,)`` (renamed ``q_layernorm`` / ``k_layernorm``, 8903-8913).

Everything is computed in float32 (bf16 weights are upcast exactly), which is
the "fp32 reference" the tolerances are quoted against.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

# How each oracle function is pinned by something other than its own formula.
# Every entry is exercised by tests/test_oracle_*.py.
PINNING: Dict[str, str] = {
    "rmsnorm": (
        "transformers Qwen3MoeRMSNorm (independent implementation) via golden "
        "fixtures; the reference's known-answer recipe nki_custom_rmsnorm.py:182-214 "
        "(seed 42, (256,512), eps 1e-6) against a float64 closed form; scale "
        "invariance; unit output RMS for w=1"
    ),
    "router_topk": (
        "transformers Qwen3MoeTopKRouter golden fixtures; brute-force sort on "
        "tiny E; weights sum to 1; top-k of logits == top-k of probabilities"
    ),
    "moe_permute": (
        "brute-force Python loop on small inputs; counts sum to T*k; offsets "
        "are an exclusive scan; slot<->(token, j) bijection; stable by token"
    ),
    "moe_block_prefill": (
        "transformers Qwen3MoeSparseMoeBlock golden fixtures; float64 per-token "
        "brute force; k=1 with a single expert reduces to a dense SwiGLU MLP"
    ),
    "moe_block_decode": "equals moe_block_prefill and the float64 brute force",
    "moe_experts_early": (
        "k=1 (affinity 1) reduces to moe_block_prefill's output; the small-"
        "affinity limit silu(z) ~ z/2 fixes out/a^2 -> 0.5 ((x Wg)*(x Wu)) Wd in "
        "closed form (an affinity applied to the output would scale as a); "
        "the result is the sum of separate one-pair calls"
    ),
    "apply_rope": (
        "transformers apply_rotary_pos_emb / Qwen3MoeRotaryEmbedding golden "
        "fixtures; position 0 is the identity; per-pair norm preservation; "
        "R(a)R(b) = R(a+b)"
    ),
    "gqa_attention": (
        "transformers eager_attention_forward + repeat_kv golden fixtures; a "
        "single visible key returns its value row; uniform scores average V"
    ),
    "attention_layer": "transformers Qwen3MoeAttention golden fixtures",
    "decoder_layer": "transformers Qwen3MoeDecoderLayer golden fixtures",
}


# ----------------------------------------------------------------------------
# RMSNorm
# ----------------------------------------------------------------------------
def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``w * x * rsqrt(mean(x^2) + eps)`` in float32.

    Follows the device RMSNorm contract: fp32 upcast, normalise, multiply by
    the weight in fp32, one cast at the end (qwen_with_nki.py:1372-1384;
    numpy golden nki_custom_rmsnorm.py:174-179; CPU class
    qwen_with_nki.py:9048-9058 -> transformers Qwen3MoeRMSNorm).
    """
    x32 = x.float()
    var = x32.pow(2).mean(-1, keepdim=True)
    return w.float() * (x32 * torch.rsqrt(var + eps))


# ----------------------------------------------------------------------------
# Router
# ----------------------------------------------------------------------------
def router_topk(
    x: torch.Tensor,
    w_router: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
    normalize: bool = True,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Router: fp32 logits -> softmax over E -> top-k -> L1 renormalise.

    Router dtype fp32 and softmax activation: qwen_with_nki.py:9886-9888;
    ``normalize_top_k_affinities=True``: 9894; gather + ``F.normalize(p=1)``:
    2399-2405 (also 3460-3466).  Same math as transformers
    ``Qwen3MoeTopKRouter.forward``.  ``bias`` (per expert, added to the
    logits) is a benchmark device used to impose a skewed expert load; Qwen3
    itself has no router bias.

    Returns ``(logits[T,E] f32, top_w[T,k] f32, top_i[T,k] int64)``.
    """
    logits = x.float() @ w_router.float().t()
    if bias is not None:
        logits = logits + bias.float()
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    top_w, top_i = torch.topk(probs, k, dim=-1)
    if normalize:
        top_w = top_w / top_w.sum(dim=-1, keepdim=True)
    return logits, top_w, top_i


# ----------------------------------------------------------------------------
# Dispatch bookkeeping (histogram / exclusive scan / stable permutation)
# ----------------------------------------------------------------------------
def moe_permute(top_i: np.ndarray, num_experts: int, tile_m: int) -> Dict[str, np.ndarray]:
    """Expert-sorted dispatch metadata, restated in numpy.

    The reference consumes expert-sorted, per-expert blocks
    (``token_position_to_id`` / ``block_to_expert``, qwen_with_nki.py:5872-5881,
    5478-5479) that ``neuronx_distributed`` builds; its exact padded-block
    layout lives in that absent package.  The build uses the unpadded form of
    the same ordering: slot ``s`` enumerates (token, j) pairs sorted by expert
    and, within an expert, by token (stable), so a token never appears twice
    in one expert's rows and the reference's duplicate redirection
    (``_dedup_token_positions`` 5656-5667) is unnecessary.

    Returns counts[E], offsets[E+1], slot_token[T*k], token_slot[T*k] (slot of
    pair t*k+j), tiles[n_tiles, 3] = (expert, slot_begin, slot_end) in chunks
    of ``tile_m`` rows, and active[U] (experts with count > 0, ascending).
    """
    top_i = np.asarray(top_i, dtype=np.int64)
    T, k = top_i.shape
    flat = top_i.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    slot_token = (order // k).astype(np.int32)
    token_slot = np.empty(T * k, dtype=np.int32)
    token_slot[order] = np.arange(T * k, dtype=np.int32)
    tiles = []
    for e in range(num_experts):
        for r0 in range(int(offsets[e]), int(offsets[e + 1]), tile_m):
            tiles.append((e, r0, min(r0 + tile_m, int(offsets[e + 1]))))
    tiles_arr = np.asarray(tiles, dtype=np.int32).reshape(-1, 3)
    active = np.nonzero(counts)[0].astype(np.int32)
    return {
        "counts": counts,
        "offsets": offsets,
        "slot_token": slot_token,
        "token_slot": token_slot,
        "tiles": tiles_arr,
        "active": active,
    }


# ----------------------------------------------------------------------------
# Experts
# ----------------------------------------------------------------------------
def expert_swiglu(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor) -> torch.Tensor:
    """One expert's SwiGLU MLP on rows ``x[n,H]`` with NxDI-layout weights.

    ``gate_up (H, 2I)`` (gate columns first, qwen_with_nki.py:8928-8966),
    ``down (I, H)``.  ``silu(x Wg) * (x Wu)`` then ``. Wd`` -- the ``mlp_op``
    body the reference calls per block / per token (5765-5786, 3467-3478) and
    transformers ``Qwen3MoeExperts.forward``.
    """
    I = down.shape[0]
    gu = x.float() @ gate_up.float()
    act = F.silu(gu[:, :I]) * gu[:, I:]
    return act @ down.float()


def moe_block_prefill(
    x: torch.Tensor,
    w_router: torch.Tensor,
    gate_up: torch.Tensor,
    down: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
):
    """Sparse MoE block, prefill schedule.

    Follows ``_cte_moe_full_torch_passthrough`` (qwen_with_nki.py:5728-5789),
    the restatement of ``ExpertMLPsV2.torch_blockwise_matmul_inference``: per
    expert, gather its rows -> ``mlp_op`` -> multiply by the (masked,
    renormalised) affinity -> ``output[idx] += ...``.  Accumulates in fp32.

    Returns ``(out[T,H], top_i[T,k], top_w[T,k], logits[T,E])``.
    """
    T, H = x.shape
    E = gate_up.shape[0]
    logits, top_w, top_i = router_topk(x, w_router, k, bias)
    # expert_affinities_masked[T, E]: renormalised weight where selected, else 0
    aff = torch.zeros(T, E, dtype=torch.float32, device=x.device)
    aff.scatter_(1, top_i, top_w)
    out = torch.zeros(T, H, dtype=torch.float32, device=x.device)
    xf = x.float()
    for e in range(E):
        tok = torch.nonzero((top_i == e).any(dim=1), as_tuple=False).flatten()
        if tok.numel() == 0:
            continue
        y = expert_swiglu(xf[tok], gate_up[e], down[e])
        out.index_add_(0, tok, y * aff[tok, e].unsqueeze(1))
    return out, top_i, top_w, logits


def moe_block_decode(
    x: torch.Tensor,
    w_router: torch.Tensor,
    gate_up: torch.Tensor,
    down: torch.Tensor,
    k: int,
    bias: Optional[torch.Tensor] = None,
):
    """Sparse MoE block, decode (selective-loading) schedule.

    Follows the verbatim restatement of ``forward_selective_loading``
    (qwen_with_nki.py:3456-3478): gather the chosen affinities, L1-normalise,
    then per token run the k chosen experts and ``sum(out * aff, dim=0)``.
    """
    T, H = x.shape
    logits, top_w, top_i = router_topk(x, w_router, k, bias)
    xf = x.float()
    outs = []
    for t in range(T):
        per_e = torch.stack(
            [expert_swiglu(xf[t : t + 1], gate_up[int(e)], down[int(e)])[0] for e in top_i[t]]
        )
        outs.append(torch.sum(per_e * top_w[t].unsqueeze(1), dim=0))
    return torch.stack(outs), top_i, top_w, logits


def moe_experts_early(x: torch.Tensor, top_i: torch.Tensor, top_w: torch.Tensor, experts) -> torch.Tensor:
    """Routed experts with early affinity modulation: each selected (token,
    expert) pair's input row is multiplied by its affinity before the MLP,
    and the MLP outputs are added unscaled -- the
    ``early_expert_affinity_modulation`` branch of the blockwise loop
    (qwen_with_nki.py:5768-5775): per expert, gather its rows,
    ``x[tok] * aff[tok, e]`` -> ``mlp_op`` -> ``output[tok] += ...``.

    ``top_i``/``top_w`` ``[T,k]``; ``experts[e]`` gives ``(gate_up (H, 2I),
    down (I, H))``.  Returns ``out[T,H]`` in fp32.
    """
    T, H = x.shape
    out = torch.zeros(T, H, dtype=torch.float32)
    xf = x.float()
    for e in torch.unique(top_i).tolist():
        tok, j = torch.nonzero(top_i == e, as_tuple=True)
        rows = xf[tok] * top_w[tok, j].float().unsqueeze(1)
        out.index_add_(0, tok, expert_swiglu(rows, *experts[int(e)]))
    return out


def moe_block(x, w_router, gate_up, down, k, bias=None):
    """Dispatch like NxDI: decode (selective loading) for T == 1, else prefill."""
    if x.shape[0] == 1:
        return moe_block_decode(x, w_router, gate_up, down, k, bias)
    return moe_block_prefill(x, w_router, gate_up, down, k, bias)


# ----------------------------------------------------------------------------
# RoPE / attention
# ----------------------------------------------------------------------------
def rope_tables(head_dim: int, positions: torch.Tensor, theta: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 ``cos``/``sin`` of shape ``[..., head_dim]`` (halves duplicated).

    ``RotaryEmbedding(head_dim, base=rope_theta)`` (qwen_with_nki.py:10083-10087);
    inverse frequencies ``theta^(-2i/D)`` and the duplicated-half layout as in
    transformers ``Qwen3MoeRotaryEmbedding`` (default rope parameters).
    """
    inv_freq = 1.0 / (
        theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=positions.device).float() / head_dim)
    )
    freqs = positions.float().unsqueeze(-1) * inv_freq
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x*cos + rotate_half(x)*sin`` (pairs ``(i, i+D/2)``)."""
    return x * cos + _rotate_half(x) * sin


def qkv_norm_rope(x, wq, wk, wv, q_norm, k_norm, positions, n_q, n_kv, head_dim, eps, theta):
    """QKV projection -> per-head RMSNorm over head_dim -> RoPE.

    q/k RMSNorm(head_dim) (qwen_with_nki.py:10102-10103) applied before RoPE
    (``pre_rope_rmsnorm``, 10967; transformers Qwen3MoeAttention.forward).
    ``x[B,S,H]``, ``positions[B,S]``; returns q ``[B,n_q,S,D]``, k and v
    ``[B,n_kv,S,D]`` in fp32.
    """
    B, S, H = x.shape
    xf = x.float()
    q = (xf @ wq.float().t()).view(B, S, n_q, head_dim)
    k = (xf @ wk.float().t()).view(B, S, n_kv, head_dim)
    v = (xf @ wv.float().t()).view(B, S, n_kv, head_dim)
    q = rmsnorm(q, q_norm, eps).transpose(1, 2)
    k = rmsnorm(k, k_norm, eps).transpose(1, 2)
    v = v.transpose(1, 2)
    cos, sin = rope_tables(head_dim, positions, theta)  # [B,S,D]
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v


def gqa_attention(q, k, v, q_idx, k_len=None):
    """Causal grouped-query attention in fp32.

    ``q[B,Hq,S,D]``, ``k,v[B,Hkv,L,D]``; the query whose own key sits at cache
    index ``q_idx[b,s]`` sees cache entries ``[0, q_idx]`` (and ``< k_len[b]``
    if given).  RoPE positions do not enter here: they were applied to q/k.
    ``repeat_kv`` + ``softmax(q k^T / sqrt(D)) v`` as in transformers
    ``eager_attention_forward``; the reference's NxDI attention base applies
    the same math (qwen_with_nki.py:10089-10099).  Returns ``[B,S,Hq,D]``.
    """
    B, Hq, S, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    rep = Hq // Hkv
    kf = k.float().repeat_interleave(rep, dim=1)
    vf = v.float().repeat_interleave(rep, dim=1)
    scores = (q.float() @ kf.transpose(2, 3)) * (1.0 / math.sqrt(D))
    kpos = torch.arange(L, device=q.device).view(1, 1, 1, L)
    mask = kpos > torch.as_tensor(q_idx, device=q.device).view(B, 1, S, 1)
    if k_len is not None:
        mask = mask | (kpos >= torch.as_tensor(k_len, device=q.device).view(B, 1, 1, 1))
    scores = scores.masked_fill(mask, float("-inf"))
    p = torch.softmax(scores, dim=-1, dtype=torch.float32)
    return (p @ vf).transpose(1, 2).contiguous()


def attention_layer(x, w: Dict[str, torch.Tensor], positions, cfg, past_kv=None):
    """``NeuronQwen3MoEAttention`` forward (qwen_with_nki.py:10081-10109).

    ``x[B,S,H]`` (already input-normed), ``positions[B,S]`` are the RoPE
    positions.  With ``past_kv=(k[B,Hkv,P,D], v)`` the new keys are appended
    (contiguous cache) and causality is by cache index ``P + s``.
    Returns ``(out[B,S,H], (k_all, v_all))``.
    """
    B, S, H = x.shape
    q, k, v = qkv_norm_rope(
        x, w["q_proj"], w["k_proj"], w["v_proj"], w["q_norm"], w["k_norm"], positions,
        cfg["n_q"], cfg["n_kv"], cfg["head_dim"], cfg["eps"], cfg["theta"],
    )
    past = 0
    if past_kv is not None:
        past = past_kv[0].shape[2]
        k = torch.cat([past_kv[0].float(), k], dim=2)
        v = torch.cat([past_kv[1].float(), v], dim=2)
    q_idx = (past + torch.arange(S, device=x.device)).view(1, S).expand(B, S)
    o = gqa_attention(q, k, v, q_idx)
    o = o.reshape(B, S, -1) @ w["o_proj"].float().t()
    return o, (k, v)


def decoder_layer(h, w: Dict[str, torch.Tensor], positions, cfg, past_kv=None):
    """``NeuronQwen3MoeDecoderLayer.forward`` (qwen_with_nki.py:10155-10213).

    ``h1 = h + Attn(RMSNorm_in(h))``; ``out = h1 + MoE(RMSNorm_post(h1))``.
    Residual stream kept in fp32.  Returns ``(out, (k, v))``.
    """
    B, S, H = h.shape
    hf = h.float()
    a, kv = attention_layer(rmsnorm(hf, w["input_layernorm"], cfg["eps"]), w, positions, cfg, past_kv)
    h1 = hf + a
    y = rmsnorm(h1, w["post_attention_layernorm"], cfg["eps"]).reshape(B * S, H)
    m, _, _, _ = moe_block(y, w["router"], w["gate_up_proj"], w["down_proj"], cfg["top_k"])
    return h1 + m.view(B, S, H), kv


# ----------------------------------------------------------------------------
# Layout helpers used by tests to hand the same weights to other implementations
# ----------------------------------------------------------------------------
def pack_w13(gate_up: torch.Tensor, group: int = 32) -> torch.Tensor:
    """Reference re-layout used to check the product's packer.

    ``(E,H,2I)`` -> ``(E,2I,H)`` with gate/up rows interleaved every ``group``
    rows: packed rows ``[2g*j, 2g*j+g)`` are gate rows ``[g*j, g*j+g)`` and the
    next ``g`` rows are the matching up rows.
    """
    E, H, I2 = gate_up.shape
    I = I2 // 2
    t = gate_up.transpose(1, 2)  # (E, 2I, H)
    gate = t[:, :I].reshape(E, I // group, group, H)
    up = t[:, I:].reshape(E, I // group, group, H)
    return torch.stack([gate, up], dim=2).reshape(E, 2 * I, H).contiguous()
