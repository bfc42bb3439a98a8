"""One tensor-parallel rank's share of a decoder layer, on one GPU.

Under TP = G the reference splits each expert's intermediate dimension and the
attention heads across ranks (moe_intermediate_size 768 / G per rank,
qwen_with_nki.py:1842; 32 query and 4 KV heads / G, KV heads replicated past
G = 4).  The kernels take those shapes unchanged:

  - experts: I = 192 (G = 4) and I = 96 (G = 8) through the prefill grouped
    GEMMs (the last gate_up weight panel is partly past 2I; at I = 96 the down
    pass has no 64-column cold pipeline) and the decode GEMVs;
  - attention: 8 query heads over 1 KV head (G = 4) and 4 over 1 (G = 8):
    QKV + q/k-norm + RoPE into the cache, causal prefill and split-KV decode.

Each against the oracle on the same seeded inputs, at the layer bars.
"""

import pytest
import torch

import oracle
from gpu_util import (ExpertCache, announce, assert_close_layer, bf16_randn, oracle_rows,
                      random_topk)

from qmoe import ops

pytestmark = pytest.mark.gpu

H, E, K_TOP, D = 2048, 128, 8, 128


@pytest.mark.parametrize("I", [192, 96])
def test_experts_rank_share(dev, I):
    announce(f"experts rank share I={I}: grouped T=1024 (Zipf), GEMV T=8")
    g = torch.Generator(device=dev).manual_seed(I)
    w13 = bf16_randn((E, 2 * I, H), g, dev, std=0.02)
    w2 = bf16_randn((E, I // 8, H, 8), g, dev, std=0.02)
    cache = ExpertCache(w13, w2)
    for T, seed in ((1024, 1), (8, 2)):
        x = bf16_randn((T, H), g, dev)
        top = torch.from_numpy(random_topk(T, K_TOP, E, seed + I, skew=1.1)).to(dev)
        tw = torch.rand(T, K_TOP, generator=g, device=dev)
        tw = tw / tw.sum(-1, keepdim=True)
        route = ops.moe_permute(top, E, 256)
        if T > 64:
            y = ops.moe_experts_grouped(x, w13, w2, route)
            counts = route.counts.cpu()
            assert int(counts.max()) > 256 and int(((counts > 0) & (counts <= 64)).sum()) > 0
        else:
            y = ops.moe_experts_gemv(x, w13, w2, route)
        out = ops.moe_combine(y, route, tw)
        torch.cuda.synchronize()
        # every row of the hottest expert's last tile and of a cold expert, plus a spread
        rows = sorted(set(range(0, T, max(1, T // 48))) | set(range(min(8, T))))
        ref = oracle_rows(x.cpu(), top.cpu(), tw.cpu(), cache, rows)
        tight = T <= 64  # fp32 activations on the GEMV path
        assert_close_layer(out.cpu()[rows], ref, f"experts I={I} T={T}",
                           max_abs_tol=2e-3 if tight else 2e-2, mean_rel_tol=1e-4 if tight else 5e-3)


@pytest.mark.parametrize("Hq,Hkv", [(8, 1), (4, 1)])
def test_attention_rank_share(dev, Hq, Hkv):
    announce(f"attention rank share Hq={Hq} Hkv={Hkv}: qkv B=2 S=300, prefill, decode ctx 300/8192")
    g = torch.Generator(device=dev).manual_seed(Hq * 10 + Hkv)
    wqkv = bf16_randn(((Hq + 2 * Hkv) * D, H), g, dev, std=0.02)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    B, S, S_max = 2, 300, 8192
    cos, sin = oracle.rope_tables(D, torch.arange(S_max), 1.0e6)
    cos, sin = cos[:, : D // 2].contiguous().to(dev), sin[:, : D // 2].contiguous().to(dev)
    x = bf16_randn((B * S, H), g, dev)
    pos = torch.arange(S, device=dev).repeat(B).to(torch.int32)
    kc = torch.zeros(B, Hkv, S_max, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = ops.qkv_norm_rope(x, wqkv, qn, kn, cos, sin, pos, B, S, Hq, Hkv, kc, vc, 1e-6)
    out = ops.attn_prefill(q.view(B * S, Hq, D), kc, vc, B, S, 0)
    torch.cuda.synchronize()
    wq, wk, wv = wqkv.float().cpu().split([Hq * D, Hkv * D, Hkv * D])
    rq, rk, rv = oracle.qkv_norm_rope(x.cpu().view(B, S, H), wq, wk, wv, qn.cpu(), kn.cpu(),
                                      pos.cpu().view(B, S).long(), Hq, Hkv, D, 1e-6, 1.0e6)
    for a, r, what in ((q.view(B, S, Hq, D).transpose(1, 2), rq, "q"), (kc[:, :, :S], rk, "k cache"),
                       (vc[:, :, :S], rv, "v cache")):
        err = (a.float().cpu() - r).abs() - r.abs() * 2 ** -8  # one bf16 rounding
        assert float(err.max()) <= 2e-4, what
    qi = torch.arange(S).view(1, S).expand(B, S)
    ref = oracle.gqa_attention(q.cpu().view(B, S, Hq, D).transpose(1, 2), kc.cpu()[:, :, :S],
                               vc.cpu()[:, :, :S], qi)
    assert_close_layer(out.cpu().view(B, S, Hq, D), ref, f"prefill Hq={Hq} Hkv={Hkv}")

    # decode: row 0 at context 300 (the prefilled rows), row 1 at 8192 (cache filled directly)
    kc[1] = bf16_randn((Hkv, S_max, D), g, dev)
    vc[1] = bf16_randn((Hkv, S_max, D), g, dev)
    qd = bf16_randn((B, Hq, D), g, dev)
    ctx = [S, S_max]
    od = ops.attn_decode(qd, kc, vc, torch.tensor(ctx, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    for b, L in enumerate(ctx):
        r = oracle.gqa_attention(qd.cpu()[b : b + 1].view(1, Hq, 1, D), kc.cpu()[b : b + 1, :, :L],
                                 vc.cpu()[b : b + 1, :, :L], torch.tensor([[L - 1]]))
        assert_close_layer(od.cpu()[b].view(Hq, D), r[0, 0], f"decode Hq={Hq} Hkv={Hkv} ctx={L}",
                           max_abs_tol=1e-2, mean_rel_tol=5e-3)
