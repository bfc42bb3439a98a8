"""Helpers shared by the GPU parity tests (seeded inputs, tolerance metrics)."""

import sys

import numpy as np
import torch

import oracle
from qmoe import weights

# Parity bars (from the hot path's accuracy contract):
#   layer / block outputs: max-abs <= 2e-2 and mean relative <= 5e-3 vs fp32
#   expert indices: bit-exact wherever the k-th / (k+1)-th router logit gap > 1e-3
MAX_ABS = 2e-2
MEAN_REL = 5e-3
GAP = 1e-3


def announce(msg: str) -> None:
    """Name the case before each GPU step (flushed, so a hard failure still shows it)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def mean_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).abs().mean() / b.abs().mean().clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double().cpu() - b.double().cpu()).abs().max())


def assert_close_layer(out: torch.Tensor, ref: torch.Tensor, what: str,
                       max_abs_tol: float = MAX_ABS, mean_rel_tol: float = MEAN_REL) -> None:
    ma, mr = max_abs(out, ref), mean_rel(out, ref)
    print(f"  {what}: max_abs={ma:.3e} mean_rel={mr:.3e}", flush=True)
    assert ma <= max_abs_tol, f"{what}: max abs {ma:.3e} > {max_abs_tol}"
    assert mr <= mean_rel_tol, f"{what}: mean rel {mr:.3e} > {mean_rel_tol}"


def bf16_randn(shape, gen, device, std=1.0):
    t = torch.empty(shape, dtype=torch.float32, device=device)
    t.normal_(0.0, std, generator=gen)
    return t.to(torch.bfloat16)


def gap_mask(logits: torch.Tensor, k: int) -> torch.Tensor:
    """Rows whose k-th and (k+1)-th largest logits differ by more than GAP."""
    top = torch.topk(logits.float(), k + 1, dim=-1).values
    return (top[:, k - 1] - top[:, k]) > GAP


def routing_agreement(y_ref: torch.Tensor, router: torch.Tensor, k: int, ours_idx: torch.Tensor):
    """Rows where the product and the fp32 reference chose the same experts,
    and the reference's k-th/(k+1)-th logit gap per row.  The product routes
    from the bf16 normed hidden state (as the reference's bf16 pipeline does),
    the reference from fp32, so near-tied rows may legitimately differ."""
    logits = y_ref.float() @ router.float().t()
    top = torch.topk(logits, k + 1, dim=-1)
    gap = top.values[:, k - 1] - top.values[:, k]
    same = (top.indices[:, :k].sort(-1).values == ours_idx.long().sort(-1).values).all(-1)
    return same, gap


def random_topk(T, k, E, seed, skew=None):
    """Seeded top-k expert ids [T, k] (int32, distinct per row); with ``skew``,
    expert popularity ~ rank^-skew over a random rank order."""
    rng = np.random.default_rng(seed)
    p = None
    if skew is not None:
        p = np.arange(1, E + 1, dtype=np.float64) ** (-skew)
        p = p[rng.permutation(E)]
        p /= p.sum()
    return np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)


class ExpertCache:
    """Unpacked (NxDI-layout) fp32 expert weights on the CPU, fetched lazily."""

    def __init__(self, w13, w2):
        self.w13, self.w2, self.c = w13, w2, {}

    def __getitem__(self, e):
        if e not in self.c:
            gu = weights.unpack_gate_up(self.w13[e : e + 1]).float().cpu()[0]  # (H, 2I)
            dn = weights.unpack_down(self.w2[e : e + 1]).float().cpu()[0]  # (I, H)
            self.c[e] = (gu, dn)
        return self.c[e]


def oracle_rows(x, top_i, top_w, cache, rows):
    """Oracle MoE output for selected token rows (decode schedule, 3456-3478)."""
    out = []
    for t in rows:
        xs = x[t : t + 1].float()
        acc = torch.stack([oracle.expert_swiglu(xs, *cache[int(e)])[0] for e in top_i[t]])
        out.append(torch.sum(acc * top_w[t].float().unsqueeze(1), dim=0))
    return torch.stack(out)


def check_layer_moe(out, base, y_ref, moe, top_k, what):
    """The MoE half of a decoder-layer step, held to the accuracy contract.

    ``out`` [N, H]: the product's layer output rows; ``base`` [N, H]: the fp32
    reference residual stream after attention; ``y_ref`` [N, H]: the fp32
    reference post-attention normed rows; ``moe``: the layer's MoEBlock (its
    last routing and the bf16 rows its router saw).
    1. The oracle routes from the product's own bf16 normed rows: expert ids
       exact wherever the k-th / (k+1)-th logit gap exceeds 1e-3.
    2. On every such row, the layer output within max-abs 2e-2 / mean
       relative 5e-3 of base + the oracle MoE of the fp32 normed row over
       those experts (weights: softmax of the fp32 row's logits over them;
       on rows where fp32 routing agrees this is the fp32 reference layer).
    3. Secondary, against fp32 routing: agreement on every row with a 1e-2
       gap and on at least 90% of rows."""
    router = moe.w_router
    idx = moe.last_routing[2].cpu().long()
    xhat = moe.last_input.cpu()
    rl, _, ri = oracle.router_topk(xhat, router.cpu(), top_k)
    ok = gap_mask(rl, top_k)
    assert torch.equal(idx[ok], ri[ok]), f"{what}: expert ids differ where the gap exceeds {GAP}"
    rows = [t for t in range(idx.shape[0]) if bool(ok[t])]
    assert rows, f"{what}: no row with a clear router gap"
    yl = y_ref.float().cpu() @ router.float().cpu().t()
    w = torch.softmax(yl.gather(1, ri), dim=1)
    ref = base.float().cpu()[rows] + oracle_rows(y_ref.cpu(), ri, w, ExpertCache(moe.experts.w13, moe.experts.w2),
                                                 rows)
    assert_close_layer(out.float().cpu()[rows], ref, what)
    same, gap = routing_agreement(y_ref.cpu(), router.cpu(), top_k, idx)
    assert bool(same[gap > 1e-2].all()), f"{what}: routing differs on a row with a clear fp32 router gap"
    assert same.float().mean() >= 0.9, f"{what}: fp32 routing agrees on {float(same.float().mean()):.2f} of rows"
