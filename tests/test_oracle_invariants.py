"""Pin the oracle with closed forms, invariants and brute force.

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign, a transposed operand, an off-by-one in the scan) fails.
"""

import math

import numpy as np
import pytest
import torch
from hypothesis import given, settings, strategies as st

import oracle


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_scale_invariance_and_unit_rms():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 256, generator=g)
    w = torch.ones(256)
    y = oracle.rmsnorm(x, w, 0.0)
    # unit RMS with w = 1, eps = 0
    np.testing.assert_allclose(y.pow(2).mean(-1).numpy(), 1.0, rtol=1e-5)
    # scale invariance
    np.testing.assert_allclose(oracle.rmsnorm(3.5 * x, w, 0.0).numpy(), y.numpy(), rtol=1e-5, atol=1e-6)
    # the weight multiplies elementwise
    w2 = torch.randn(256, generator=g)
    np.testing.assert_allclose(oracle.rmsnorm(x, w2, 0.0).numpy(), (y * w2).numpy(), rtol=1e-5, atol=1e-6)
    # eps enters under the root: a zero row stays zero, a row of c gives c/sqrt(c^2+eps)
    c = 0.01
    z = oracle.rmsnorm(torch.full((1, 8), c), torch.ones(8), 1e-4)
    np.testing.assert_allclose(z.numpy(), c / math.sqrt(c * c + 1e-4), rtol=1e-6)


# ---------------------------------------------------------------- router
@settings(max_examples=25, deadline=None)
@given(T=st.integers(1, 12), E=st.integers(4, 24), seed=st.integers(0, 10_000))
def test_router_invariants(T, E, seed):
    k = min(4, E)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, 16, generator=g)
    w = torch.randn(E, 16, generator=g)
    logits, top_w, top_i = oracle.router_topk(x, w, k)
    np.testing.assert_allclose(top_w.sum(-1).numpy(), 1.0, rtol=1e-6)
    for t in range(T):
        li = logits[t].numpy().astype(np.float64)
        # brute force: indices of the k largest logits (softmax is monotone)
        order = sorted(range(E), key=lambda e: -li[e])
        assert set(top_i[t].tolist()) == set(order[:k])
        # weights = softmax restricted to the chosen k
        sel = li[top_i[t].numpy()]
        ref = np.exp(sel - sel.max()) / np.exp(sel - sel.max()).sum()
        np.testing.assert_allclose(top_w[t].numpy(), ref, rtol=1e-5)


def test_router_bias_shifts_selection():
    x = torch.zeros(3, 8)
    w = torch.zeros(5, 8)
    bias = torch.tensor([0.0, 5.0, 1.0, 4.0, 3.0])
    _, top_w, top_i = oracle.router_topk(x, w, 2, bias)
    assert top_i[0].tolist() == [1, 3]
    np.testing.assert_allclose(top_w[0].numpy(), [1 / (1 + math.exp(-1)), math.exp(-1) / (1 + math.exp(-1))], rtol=1e-6)


# ---------------------------------------------------------------- permute
def _permute_brute(top_i, E, tile_m):
    T, k = top_i.shape
    slots = []
    for e in range(E):
        for t in range(T):
            for j in range(k):
                if top_i[t, j] == e:
                    slots.append((t, j))
    counts = [sum(1 for t in range(T) for j in range(k) if top_i[t, j] == e) for e in range(E)]
    return slots, counts


@settings(max_examples=40, deadline=None)
@given(T=st.integers(1, 40), E=st.integers(2, 16), tile_m=st.sampled_from([1, 3, 8, 64]), seed=st.integers(0, 99999))
def test_permute_matches_brute_force(T, E, tile_m, seed):
    k = min(3, E)
    rng = np.random.default_rng(seed)
    top_i = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    r = oracle.moe_permute(top_i, E, tile_m)
    slots, counts = _permute_brute(top_i, E, tile_m)
    assert r["counts"].tolist() == counts
    assert r["offsets"][0] == 0 and r["offsets"][-1] == T * k
    assert np.all(np.diff(r["offsets"]) == r["counts"])
    assert [int(t) for t in r["slot_token"]] == [t for t, _ in slots]
    # token_slot is the inverse: slot of pair (t, j) holds token t and lies in expert top_i[t, j]
    for t in range(T):
        for j in range(k):
            s = r["token_slot"][t * k + j]
            assert r["slot_token"][s] == t
            e = top_i[t, j]
            assert r["offsets"][e] <= s < r["offsets"][e + 1]
    assert sorted(r["token_slot"].tolist()) == list(range(T * k))
    # tiles cover every slot once, never straddle experts, at most tile_m rows
    cover = np.zeros(T * k, dtype=int)
    for e, a, b in r["tiles"]:
        assert 0 < b - a <= tile_m
        assert r["offsets"][e] <= a and b <= r["offsets"][e + 1]
        cover[a:b] += 1
    assert np.all(cover == 1)
    assert r["active"].tolist() == [e for e in range(E) if counts[e] > 0]


# ---------------------------------------------------------------- experts
def _brute_moe_f64(x, router, gate_up, down, k):
    x = x.double().numpy()
    logits = x @ router.double().numpy().T
    T, H = x.shape
    I = down.shape[1]
    out = np.zeros((T, H))
    for t in range(T):
        p = np.exp(logits[t] - logits[t].max())
        p /= p.sum()
        idx = np.argsort(-p, kind="stable")[:k]
        w = p[idx] / p[idx].sum()
        for j, e in enumerate(idx):
            gu = x[t] @ gate_up[e].double().numpy()
            a = gu[:I] / (1 + np.exp(-gu[:I])) * gu[I:]
            out[t] += w[j] * (a @ down[e].double().numpy())
    return out


@pytest.mark.parametrize("T", [1, 5, 17])
def test_moe_block_vs_float64_brute_force(T):
    g = torch.Generator().manual_seed(T)
    E, H, I, k = 6, 24, 10, 2
    x = torch.randn(T, H, generator=g)
    router = torch.randn(E, H, generator=g)
    gate_up = 0.2 * torch.randn(E, H, 2 * I, generator=g)
    down = 0.2 * torch.randn(E, I, H, generator=g)
    ref = _brute_moe_f64(x, router, gate_up, down, k)
    for fn in (oracle.moe_block_prefill, oracle.moe_block_decode):
        out = fn(x, router, gate_up, down, k)[0].numpy()
        np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-6)


def test_moe_block_k1_single_expert_is_dense_swiglu():
    g = torch.Generator().manual_seed(3)
    H, I = 16, 8
    x = torch.randn(4, H, generator=g)
    wg, wu, wd = torch.randn(I, H, generator=g), torch.randn(I, H, generator=g), torch.randn(H, I, generator=g)
    gate_up = torch.cat([wg.t(), wu.t()], dim=1).unsqueeze(0)  # (1, H, 2I)
    down = wd.t().unsqueeze(0)  # (1, I, H)
    out = oracle.moe_block_prefill(x, torch.zeros(1, H), gate_up, down, 1)[0]
    dense = (torch.nn.functional.silu(x @ wg.t()) * (x @ wu.t())) @ wd.t()
    np.testing.assert_allclose(out.numpy(), dense.numpy(), rtol=1e-5, atol=1e-5)


def _early_case(seed, T=6, E=5, H=16, I=8, k=2):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    router = torch.randn(E, H, generator=g)
    gate_up = 0.3 * torch.randn(E, H, 2 * I, generator=g)
    down = 0.3 * torch.randn(E, I, H, generator=g)
    return x, router, gate_up, down, {e: (gate_up[e], down[e]) for e in range(E)}


def test_moe_experts_early_k1_is_the_late_block():
    """k = 1: the renormalised affinity is 1, so scaling the input or the
    output is the same; the result equals moe_block_prefill's."""
    x, router, gate_up, down, experts = _early_case(5)
    late, top_i, top_w, _ = oracle.moe_block_prefill(x, router, gate_up, down, 1)
    assert torch.all(top_w == 1.0)
    early = oracle.moe_experts_early(x, top_i, top_w, experts)
    np.testing.assert_allclose(early.numpy(), late.numpy(), rtol=1e-6, atol=1e-6)


def test_moe_experts_early_small_affinity_limit():
    """silu(z) = z / 2 + O(z^2): with every affinity a -> 0 the early output
    over a^2 tends to 0.5 * sum_j ((x Wg_j) * (x Wu_j)) Wd_j.  An affinity
    applied to the output instead would scale as a (ratio -> infinity), one
    read from the wrong pair would change the sum."""
    x, router, gate_up, down, experts = _early_case(9, k=3)
    _, top_i, _, _ = oracle.moe_block_prefill(x, router, gate_up, down, 3)
    I = down.shape[1]
    xd = x.double()
    limit = torch.zeros(x.shape, dtype=torch.float64)
    for t in range(x.shape[0]):
        for e in top_i[t].tolist():
            gu = xd[t] @ gate_up[e].double()
            limit[t] += 0.5 * (gu[:I] * gu[I:]) @ down[e].double()
    for a in (1e-2, 1e-3):
        out = oracle.moe_experts_early(x, top_i, torch.full(top_i.shape, a), experts).double() / a**2
        err = (out - limit).abs().max().item() / limit.abs().max().item()
        assert err < 30 * a, (a, err)


def test_moe_experts_early_is_a_sum_over_pairs():
    """The k pairs of a token are independent: the output is the sum of k
    one-pair calls, each with its own affinity."""
    x, router, gate_up, down, experts = _early_case(13, k=2)
    _, top_i, top_w, _ = oracle.moe_block_prefill(x, router, gate_up, down, 2)
    full = oracle.moe_experts_early(x, top_i, top_w, experts)
    parts = sum(oracle.moe_experts_early(x, top_i[:, j : j + 1], top_w[:, j : j + 1], experts) for j in range(2))
    np.testing.assert_allclose(full.numpy(), parts.numpy(), rtol=1e-5, atol=1e-6)
    late = oracle.moe_block_prefill(x, router, gate_up, down, 2)[0]
    assert (full - late).abs().max() > 1e-2  # a different schedule, not the late one


def test_pack_w13_interleave():
    E, H, I = 2, 4, 64
    gate_up = torch.arange(E * H * 2 * I, dtype=torch.float32).view(E, H, 2 * I)
    p = oracle.pack_w13(gate_up, 32)
    t = gate_up.transpose(1, 2)
    assert torch.equal(p[:, 0:32], t[:, 0:32])
    assert torch.equal(p[:, 32:64], t[:, I : I + 32])
    assert torch.equal(p[:, 64:96], t[:, 32:64])
    assert torch.equal(p[:, 96:128], t[:, I + 32 : I + 64])


# ---------------------------------------------------------------- RoPE / attention
def test_rope_position_zero_identity_and_rotation():
    D = 16
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, D, generator=g)
    cos, sin = oracle.rope_tables(D, torch.zeros(3, dtype=torch.long), 1e6)
    np.testing.assert_allclose(oracle.apply_rope(x, cos, sin).numpy(), x.numpy(), atol=0)
    pos = torch.tensor([5, 4000, 8191])
    cos, sin = oracle.rope_tables(D, pos, 1e6)
    y = oracle.apply_rope(x, cos, sin)
    # each (i, i+D/2) pair keeps its norm
    h = D // 2
    np.testing.assert_allclose((y[:, :h] ** 2 + y[:, h:] ** 2).numpy(), (x[:, :h] ** 2 + x[:, h:] ** 2).numpy(), rtol=1e-5)
    # R(a) R(b) = R(a + b)
    ca, sa = oracle.rope_tables(D, torch.tensor([7]), 1e6)
    cb, sb = oracle.rope_tables(D, torch.tensor([11]), 1e6)
    cab, sab = oracle.rope_tables(D, torch.tensor([18]), 1e6)
    two = oracle.apply_rope(oracle.apply_rope(x[:1], ca, sa), cb, sb)
    np.testing.assert_allclose(two.numpy(), oracle.apply_rope(x[:1], cab, sab).numpy(), atol=1e-5)
    # first pair rotates by exactly pos radians (inv_freq[0] = 1)
    np.testing.assert_allclose(cos[:, 0].numpy(), np.cos(pos.numpy().astype(np.float64)), atol=1e-3)


def test_attention_single_key_and_uniform():
    g = torch.Generator().manual_seed(2)
    B, Hq, Hkv, D = 1, 4, 2, 8
    q = torch.randn(B, Hq, 1, D, generator=g)
    k = torch.randn(B, Hkv, 5, D, generator=g)
    v = torch.randn(B, Hkv, 5, D, generator=g)
    # query at position 0 sees only key 0 -> returns v[0] of its kv head
    out = oracle.gqa_attention(q, k, v, torch.zeros(B, 1, dtype=torch.long))
    for h in range(Hq):
        np.testing.assert_allclose(out[0, 0, h].numpy(), v[0, h // 2, 0].numpy(), rtol=1e-6)
    # zero query -> uniform weights over the visible keys -> mean of v
    out = oracle.gqa_attention(torch.zeros_like(q), k, v, torch.full((B, 1), 4, dtype=torch.long))
    for h in range(Hq):
        np.testing.assert_allclose(out[0, 0, h].numpy(), v[0, h // 2].mean(0).numpy(), rtol=1e-5, atol=1e-6)


def test_attention_incremental_equals_full():
    g = torch.Generator().manual_seed(4)
    cfg = dict(n_q=4, n_kv=2, head_dim=8, eps=1e-6, theta=1e6, top_k=2)
    H = 16
    w = {n: 0.3 * torch.randn(s, generator=g) for n, s in [
        ("q_proj", (32, H)), ("k_proj", (16, H)), ("v_proj", (16, H)), ("o_proj", (H, 32))]}
    w["q_norm"] = torch.ones(8)
    w["k_norm"] = torch.ones(8)
    x = torch.randn(2, 6, H, generator=g)
    pos = torch.arange(6).repeat(2, 1)
    full, _ = oracle.attention_layer(x, w, pos, cfg)
    pre, kv = oracle.attention_layer(x[:, :5], w, pos[:, :5], cfg)
    last, _ = oracle.attention_layer(x[:, 5:], w, pos[:, 5:], cfg, past_kv=kv)
    np.testing.assert_allclose(pre.numpy(), full[:, :5].numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(last.numpy(), full[:, 5:].numpy(), rtol=1e-5, atol=1e-6)
