"""GPU parity tests: every libqmoe kernel against the oracle on the same
seeded inputs (bf16 inputs are handed to the oracle exactly, upcast to fp32).

Bars: bit-exact for integer / index work; expert indices exact where the
router-logit gap exceeds 1e-3; floating-point outputs within max-abs 2e-2 and
mean relative 5e-3 of the fp32 oracle (tighter where noted).
"""

import math

import numpy as np
import pytest
import torch

import oracle
from gpu_util import (GAP, announce, assert_close_layer, bf16_randn, gap_mask, max_abs, mean_rel)
from gpu_util import ExpertCache as _ExpertCache
from gpu_util import oracle_rows as _oracle_rows
from gpu_util import random_topk as _random_topk

from qmoe import _lib, ops, weights
from qmoe.moe import MoEBlock

pytestmark = pytest.mark.gpu

H, E, K_TOP, I = 2048, 128, 8, 768


@pytest.fixture(autouse=True)
def _fp32_reference_matmuls():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


# --------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(1, 256, 2048), (5, 4096, 2048), (16, 128, 2048), (8, 2048, 4096),
                                   (128, 256, 2048), (300, 384, 768), (77, 2048, 4096),
                                   # ragged N; 128x256 tiles; 256x256 tiles
                                   (300, 200, 128), (4096, 2048, 1024), (4096, 4096, 256),
                                   # the prefill router shape (64x64 tiles, four stages)
                                   (4096, 128, 2048),
                                   # from 224 tiles of 256x256: the 8-wave deep-staged pipeline
                                   # (ragged M and N; the B=8 x 1024 o_proj shape), and the
                                   # 256x256 two-stage one when N % 4 != 0
                                   (7000, 2052, 512), (8192, 2048, 4096), (7000, 2050, 512),
                                   # 2-8 rows, packed-A GEMV: 20 / 16 / 8 / 4 columns per workgroup,
                                   # 1-8 waves, ragged last workgroup
                                   (8, 5120, 2048), (2, 5123, 2048), (3, 4100, 1024), (7, 1000, 512),
                                   (6, 40000, 2048), (4, 2050, 4096)])
def test_gemm_vs_fp32(dev, M, N, K):
    announce(f"gemm M={M} N={N} K={K}")
    g = torch.Generator(device=dev).manual_seed(M * 7 + N)
    A = bf16_randn((M, K), g, dev)
    B = bf16_randn((N, K), g, dev, std=0.02)
    ref = A.float().cpu() @ B.float().cpu().t()
    c32 = ops.gemm(A, B, _lib.GEMM_STORE_F32)
    cbf = ops.gemm(A, B, _lib.GEMM_STORE_BF16)
    acc = torch.ones(M, N, device=dev)
    ops.gemm(A, B, _lib.GEMM_ADD_F32, out=acc)
    torch.cuda.synchronize()
    scale = float(ref.abs().max())
    assert max_abs(c32, ref) <= 1e-4 * scale
    assert max_abs(acc, ref + 1.0) <= 1e-4 * scale + 1e-6
    # bf16 output: within one bf16 rounding of the fp32 result
    assert float(((cbf.float().cpu() - ref).abs() - ref.abs() * 2 ** -8).max()) <= 1e-4 * scale


# 64 x 128 tiles (640 and 333 rows of the o_proj shape), 64 x 64 (the router
# shape, 300 x 200), 128 x 128 (1000 x 512)
@pytest.mark.parametrize("M,N,K", [(640, 2048, 4096), (333, 2048, 4096), (640, 128, 2048), (300, 200, 1024),
                                   (1000, 512, 2048)])
def test_gemm_splitk_vs_fp32(dev, M, N, K):
    """qmoe_gemm_ws: K split into slices through the workspace (the prefill
    o_proj and router shapes), each mode vs fp32; repeats are bit-identical
    (the slices are summed in a fixed order)."""
    announce(f"gemm split-K M={M} N={N} K={K}")
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    A = bf16_randn((M, K), g, dev)
    B = bf16_randn((N, K), g, dev, std=0.02)
    ws = ops.gemm_workspace(M, N, K, dev)
    assert ws is not None, "this shape should split K"
    ref = A.float().cpu() @ B.float().cpu().t()
    c32 = ops.gemm(A, B, _lib.GEMM_STORE_F32, workspace=ws)
    c32b = ops.gemm(A, B, _lib.GEMM_STORE_F32, workspace=ws)
    cbf = ops.gemm(A, B, _lib.GEMM_STORE_BF16, workspace=ws)
    acc = torch.ones(M, N, device=dev)
    ops.gemm(A, B, _lib.GEMM_ADD_F32, out=acc, workspace=ws)
    torch.cuda.synchronize()
    scale = float(ref.abs().max())
    assert torch.equal(c32, c32b)
    assert max_abs(c32, ref) <= 1e-4 * scale
    assert max_abs(acc, ref + 1.0) <= 1e-4 * scale + 1e-6
    assert float(((cbf.float().cpu() - ref).abs() - ref.abs() * 2 ** -8).max()) <= 1e-4 * scale


# --------------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("rows", [1, 37, 640])
def test_rmsnorm_residual(dev, rows):
    announce(f"rmsnorm rows={rows}")
    g = torch.Generator(device=dev).manual_seed(rows)
    x = torch.randn(rows, H, generator=g, device=dev)
    d = torch.randn(rows, H, generator=g, device=dev)
    w = bf16_randn((H,), g, dev)
    h = torch.empty_like(x)
    y = ops.rmsnorm_residual(x, w, 1e-6, delta=d, h_out=h)
    y2 = ops.rmsnorm_residual(x, w, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(h, x + d)  # the residual add is one fp32 add: bit-exact
    ref = oracle.rmsnorm((x + d).cpu(), w.cpu(), 1e-6)
    ref2 = oracle.rmsnorm(x.cpu(), w.cpu(), 1e-6)
    # one bf16 rounding of an fp32 value that may differ by a few ulp
    for out, r in ((y, ref), (y2, ref2)):
        err = (out.float().cpu() - r).abs() - r.abs() * 2 ** -8
        assert float(err.max()) <= 1e-5


@pytest.mark.parametrize("M,N,K", [(640, 2048, 4096), (300, 2048, 1024), (4096, 2048, 512), (33, 516, 256)])
def test_gemm_add_rmsnorm_bits(dev, M, N, K):
    """qmoe_gemm_ws_add_rmsnorm (o_proj into the residual + the post-attention
    norm) gives the bits of qmoe_gemm(ADD_F32) then qmoe_rmsnorm_residual:
    through the split-K reduction with the norm inside (640 x 2048 x 4096,
    300 x 2048 x 1024) and through the unsplit fallback (no workspace; a
    shape that does not split)."""
    announce(f"gemm_add_rmsnorm M={M} N={N} K={K}")
    g = torch.Generator(device=dev).manual_seed(M + 3 * N + K)
    A = bf16_randn((M, K), g, dev)
    B = bf16_randn((N, K), g, dev, std=0.02)
    w = bf16_randn((N,), g, dev)
    h0 = torch.randn(M, N, generator=g, device=dev)
    ws = ops.gemm_workspace(M, N, K, dev)
    for workspace in ([ws, None] if ws is not None else [None]):
        h_ref = h0.clone()
        ops.gemm(A, B, _lib.GEMM_ADD_F32, out=h_ref, workspace=workspace)
        x_ref = ops.rmsnorm_residual(h_ref, w, 1e-6)
        h = h0.clone()
        x = ops.gemm_add_rmsnorm(A, B, h, w, 1e-6, workspace=workspace)
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(x, x_ref), f"workspace={workspace is not None}"


# top-8 at H = 2048 (the one-pass row form), top-8 at H = 1024 and top-4
# (the per-chunk forms)
@pytest.mark.parametrize("T,y_bf16,Hh,kk", [(640, True, 2048, 8), (1000, False, 2048, 8), (9, True, 2048, 8),
                                            (50, True, 1024, 8), (30, False, 2048, 4)])
def test_moe_combine_norm_bits(dev, T, y_bf16, Hh, kk):
    """qmoe_moe_combine_norm (combine + residual, then the next layer's input
    norm) gives the bits of qmoe_moe_combine then qmoe_rmsnorm_residual, in
    place on the residual as the layers run it."""
    announce(f"moe_combine_norm T={T} bf16={y_bf16} H={Hh} k={kk}")
    g = torch.Generator(device=dev).manual_seed(T + 5)
    top = torch.from_numpy(_random_topk(T, kk, E, 13 + T)).to(dev)
    tw = torch.rand(T, kk, generator=g, device=dev)
    route = ops.moe_permute(top, E, 256)
    y = torch.randn(T * kk, Hh, generator=g, device=dev)
    y = y.to(torch.bfloat16) if y_bf16 else y
    w = bf16_randn((Hh,), g, dev)
    h0 = torch.randn(T, Hh, generator=g, device=dev)
    h_ref = h0.clone()
    ops.moe_combine(y, route, tw, residual=h_ref, out=h_ref)
    x_ref = ops.rmsnorm_residual(h_ref, w, 1e-6)
    h = h0.clone()
    out, x = ops.moe_combine(y, route, tw, residual=h, out=h, norm=(w, 1e-6))
    torch.cuda.synchronize()
    assert out is h
    assert torch.equal(h, h_ref) and torch.equal(x, x_ref)


def test_rmsnorm_reference_recipe_on_gpu(dev):
    """The reference's known-answer recipe (nki_custom_rmsnorm.py:182-214),
    at H=512: seed 42, x (256,512), w randn, eps 1e-6, max|diff| < 1e-3."""
    announce("rmsnorm seed-42 recipe")
    np.random.seed(42)
    x = np.random.randn(256, 512).astype(np.float32)
    w = np.random.randn(512).astype(np.float32)
    wb = torch.from_numpy(w).to(torch.bfloat16)
    y = ops.rmsnorm_residual(torch.from_numpy(x).to(dev), wb.to(dev), 1e-6)
    ref = oracle.rmsnorm(torch.from_numpy(x), wb.float(), 1e-6)
    torch.cuda.synchronize()
    assert float((y.float().cpu() - ref).abs().max()) < 3e-2  # bf16 output of |y| up to ~8
    assert float(((y.float().cpu() - ref).abs() - ref.abs() * 2 ** -8).max()) <= 1e-5


# --------------------------------------------------------------------------- router
@pytest.fixture(scope="module")
def router_w(dev):
    g = torch.Generator(device=dev).manual_seed(11)
    return bf16_randn((E, H), g, dev, std=0.02)


@pytest.mark.parametrize("T", [1, 8, 17, 64, 100, 128, 4096])
def test_router_topk(dev, router_w, T):
    announce(f"router T={T}")
    g = torch.Generator(device=dev).manual_seed(100 + T)
    x = bf16_randn((T, H), g, dev)
    logits, tw, ti = ops.router_topk(x, router_w, K_TOP)
    torch.cuda.synchronize()
    rl, rw, ri = oracle.router_topk(x.cpu(), router_w.cpu(), K_TOP)
    assert max_abs(logits, rl) <= 1e-4
    ok = gap_mask(rl, K_TOP)
    assert ok.float().mean() > 0.5
    assert torch.equal(ti.cpu().long()[ok], ri[ok])
    np.testing.assert_allclose(tw.cpu()[ok].numpy(), rw[ok].numpy(), rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(tw.sum(-1).cpu().numpy(), 1.0, rtol=1e-5)


def test_router_bias_zipf_selection(dev, router_w):
    announce("router with per-expert bias")
    T = 256
    g = torch.Generator(device=dev).manual_seed(3)
    x = bf16_randn((T, H), g, dev)
    bias = torch.linspace(2.0, -2.0, E, device=dev)
    logits, tw, ti = ops.router_topk(x, router_w, K_TOP, bias)
    torch.cuda.synchronize()
    rl, rw, ri = oracle.router_topk(x.cpu(), router_w.cpu(), K_TOP, bias.cpu())
    assert max_abs(logits, rl) <= 1e-4
    ok = gap_mask(rl, K_TOP)
    assert torch.equal(ti.cpu().long()[ok], ri[ok])


# Router at other expert counts, hidden sizes and k: the GEMV path (T <= 16)
# and the GEMM path (ragged T), with and without a bias.
@pytest.mark.parametrize("T,E_,H_,k,with_bias", [(12, 64, 512, 4, False), (300, 256, 1024, 8, True),
                                                 (1000, 128, 4096, 8, True), (77, 128, 192, 8, False)])
def test_router_topk_shapes(dev, T, E_, H_, k, with_bias):
    announce(f"router T={T} E={E_} H={H_} k={k} bias={with_bias}")
    g = torch.Generator(device=dev).manual_seed(7 * T + E_)
    w = bf16_randn((E_, H_), g, dev, std=0.02)
    x = bf16_randn((T, H_), g, dev)
    bias = torch.randn(E_, generator=g, device=dev) * 0.05 if with_bias else None
    logits, tw, ti = ops.router_topk(x, w, k, bias)
    torch.cuda.synchronize()
    rl, rw, ri = oracle.router_topk(x.cpu(), w.cpu(), k, None if bias is None else bias.cpu())
    assert max_abs(logits, rl) <= 1e-4
    ok = gap_mask(rl, k)
    assert ok.float().mean() > 0.5
    assert torch.equal(ti.cpu().long()[ok], ri[ok])
    np.testing.assert_allclose(tw.cpu()[ok].numpy(), rw[ok].numpy(), rtol=2e-5, atol=1e-7)


# Split-K router logits (T > 16 with the workspace, the default of
# ops.router_topk / moe_route) against the unsplit GEMM of qmoe_router_topk:
# the same selection away from near-ties, logits within fp32 rounding, and the
# same bits on a repeated call (the slices are summed in a fixed order).
@pytest.mark.parametrize("T,H_", [(17, 2048), (640, 2048), (1000, 4096), (1024, 2048)])
def test_router_split_k_matches_unsplit(dev, T, H_):
    announce(f"router split-K T={T} H={H_}")
    g = torch.Generator(device=dev).manual_seed(11 * T + H_)
    w = bf16_randn((E, H_), g, dev, std=0.02)
    x = bf16_randn((T, H_), g, dev)
    assert int(_lib.lib().qmoe_router_workspace(T, H_, E)) > 0
    l1, w1, i1 = ops.router_topk(x, w, K_TOP)
    l2, w2, i2 = ops.router_topk(x, w, K_TOP)
    lp = torch.empty(T, E, dtype=torch.float32, device=dev)
    ip = torch.empty(T, K_TOP, dtype=torch.int32, device=dev)
    wp = torch.empty(T, K_TOP, dtype=torch.float32, device=dev)
    assert _lib.lib().qmoe_router_topk(x.data_ptr(), w.data_ptr(), None, T, H_, E, K_TOP, ip.data_ptr(),
                                       wp.data_ptr(), lp.data_ptr(), ops._stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(l1, l2) and torch.equal(i1, i2) and torch.equal(w1, w2)
    assert float((l1 - lp).abs().max()) <= 1e-5
    ok = gap_mask(lp.cpu(), K_TOP)
    assert ok.float().mean() > 0.5
    assert torch.equal(i1.cpu()[ok], ip.cpu()[ok])
    np.testing.assert_allclose(w1.cpu()[ok].numpy(), wp.cpu()[ok].numpy(), rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------- permute
# T*k <= 4096 pairs: single-workgroup kernel; above: one workgroup per
# 1024-pair chunk (513: 5 chunks, the last ragged; 16384: 128 chunks; 40000:
# 313 chunks, ragged), or the single workgroup again when `tiles` holds only
# the tile table ("narrow").
@pytest.mark.parametrize("T,skew,tile_m,narrow", [
    (1, None, 128, False), (8, None, 128, False), (64, None, 128, False), (333, None, 128, False),
    (512, None, 128, False), (513, 1.1, 128, False), (4096, None, 128, False), (4096, 1.1, 128, False),
    (4096, 1.1, 256, False), (4096, 1.1, 256, True), (16384, 1.1, 128, False), (40000, 1.1, 256, False)])
def test_permute_bit_exact(dev, T, skew, tile_m, narrow):
    announce(f"permute T={T} skew={skew} tile_m={tile_m} narrow={narrow}")
    top = _random_topk(T, K_TOP, E, T, skew)
    route = ops.Route.alloc(T, K_TOP, E, tile_m, dev)
    if narrow:
        route.tiles = route.tiles[: route.max_tiles].clone()
    route = ops.moe_permute(torch.from_numpy(top).to(dev), E, tile_m, route=route)
    torch.cuda.synchronize()
    ref = oracle.moe_permute(top, E, tile_m)
    assert torch.equal(route.counts.cpu(), torch.from_numpy(ref["counts"]))
    assert torch.equal(route.offsets.cpu(), torch.from_numpy(ref["offsets"]))
    assert torch.equal(route.slot_token.cpu(), torch.from_numpy(ref["slot_token"]))
    assert torch.equal(route.token_slot.cpu(), torch.from_numpy(ref["token_slot"]))
    meta = route.meta.cpu()
    n_tiles, n_active = int(meta[0]), int(meta[1])
    assert int(meta[2]) == 0
    assert n_tiles == len(ref["tiles"]) and n_active == len(ref["active"])
    assert torch.equal(route.tiles.cpu()[:n_tiles, :3], torch.from_numpy(ref["tiles"]))
    assert torch.equal(route.active.cpu()[:n_active], torch.from_numpy(ref["active"]))


@pytest.mark.parametrize("T", [2, 1000])
def test_permute_rejects_out_of_range_ids(dev, T):
    announce(f"permute with an out-of-range expert id T={T}")
    top = torch.from_numpy(_random_topk(T, 8, 8, 5)).to(dev)
    top[T // 2, 3] = 200  # one bad id (in the last chunk's neighbourhood for T = 1000)
    route = ops.moe_permute(top, 8, 128)
    torch.cuda.synchronize()
    meta = route.meta.cpu()
    assert int(meta[2]) == 1 and int(meta[0]) == 0 and int(meta[1]) == 0
    assert torch.equal(route.token_slot.cpu(), torch.arange(T * 8, dtype=torch.int32))
    assert torch.equal(route.slot_token.cpu(), torch.arange(T * 8, dtype=torch.int32) // 8)


# --------------------------------------------------------------------------- experts
@pytest.fixture(scope="module")
def experts(dev):
    g = torch.Generator(device=dev).manual_seed(2024)
    w13 = bf16_randn((E, 2 * I, H), g, dev, std=0.02)
    w2 = bf16_randn((E, I // 8, H, 8), g, dev, std=0.02)  # blocked layout (random values)
    return w13, w2


@pytest.mark.parametrize("T", [1, 8, 64, 128, 512, 4096])
def test_experts_and_combine(dev, experts, T):
    """Permute -> experts (GEMV for T <= 64, MFMA grouped above) -> combine,
    with routing fixed to the same top-k for both sides."""
    announce(f"experts+combine T={T}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(7 + T)
    x = bf16_randn((T, H), g, dev)
    top = torch.from_numpy(_random_topk(T, K_TOP, E, 99 + T)).to(dev)
    tw = torch.rand(T, K_TOP, generator=g, device=dev)
    tw = tw / tw.sum(-1, keepdim=True)
    residual = torch.randn(T, H, generator=g, device=dev)
    route = ops.moe_permute(top, E, 256)
    y = ops.moe_experts_gemv(x, w13, w2, route) if T <= 64 else ops.moe_experts_grouped(x, w13, w2, route)
    out = ops.moe_combine(y, route, tw, residual=residual)
    torch.cuda.synchronize()
    rows = list(range(T)) if T <= 128 else sorted(np.random.default_rng(T).choice(T, 96, replace=False).tolist())
    cache = _ExpertCache(w13, w2)
    ref = _oracle_rows(x.cpu(), top.cpu(), tw.cpu(), cache, rows)
    got = (out.cpu() - residual.cpu())[rows]
    tight = T <= 64  # fp32 activations on the GEMV path
    assert_close_layer(got, ref, f"moe T={T}", max_abs_tol=2e-3 if tight else 2e-2,
                       mean_rel_tol=1e-4 if tight else 5e-3)


@pytest.mark.parametrize("T", [20, 64])
def test_experts_gemv_crowded_experts(dev, experts, T):
    """The T <= 64 expert GEMVs when a few experts take many tokens: every
    token routed to experts 0..7 (T rows each, so the gate/up token staging
    and the 16-row down passes both loop), plus a token order that is not
    the slot order."""
    announce(f"experts gemv crowded T={T}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(31 + T)
    x = bf16_randn((T, H), g, dev)
    top = torch.stack([torch.randperm(8, generator=torch.Generator().manual_seed(t)) for t in range(T)])
    top = top.to(torch.int32).to(dev)
    tw = torch.rand(T, K_TOP, generator=g, device=dev)
    tw = tw / tw.sum(-1, keepdim=True)
    route = ops.moe_permute(top, E, 256)
    y = ops.moe_experts_gemv(x, w13, w2, route)
    out = ops.moe_combine(y, route, tw)
    torch.cuda.synchronize()
    rows = list(range(T))
    ref = _oracle_rows(x.cpu(), top.cpu(), tw.cpu(), _ExpertCache(w13, w2), rows)
    assert_close_layer(out.cpu()[rows], ref, f"crowded moe T={T}", max_abs_tol=2e-3, mean_rel_tol=1e-4)


@pytest.mark.parametrize("tile_m", [32, 128])
def test_experts_grouped_small_tiles(dev, experts, tile_m):
    """Grouped experts take any tile table with runs of at most 256 rows: a
    32- or 128-row table gives the same bf16 y_slot bits as the 256-row one
    (each output element is one K-ordered MFMA chain either way)."""
    announce(f"grouped experts tile_m={tile_m} vs 256")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(3)
    T = 700
    x = bf16_randn((T, H), g, dev)
    top = torch.from_numpy(_random_topk(T, K_TOP, E, 3, skew=1.1)).to(dev)
    y_ref = ops.moe_experts_grouped(x, w13, w2, ops.moe_permute(top, E, 256))
    y = ops.moe_experts_grouped(x, w13, w2, ops.moe_permute(top, E, tile_m))
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)


def test_experts_deterministic(dev, experts):
    announce("experts repeat-run bitwise equality T=512")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(5)
    T = 512
    x = bf16_randn((T, H), g, dev)
    top = torch.from_numpy(_random_topk(T, K_TOP, E, 5, skew=1.1)).to(dev)
    tw = torch.full((T, K_TOP), 1.0 / K_TOP, device=dev)
    outs = []
    for _ in range(2):
        route = ops.moe_permute(top, E, 256)
        y = ops.moe_experts_grouped(x, w13, w2, route)
        outs.append(ops.moe_combine(y, route, tw))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_experts_grouped_route_reuse(dev, experts):
    """The grouped GEMMs hand out work through counters in the route's meta;
    the last workgroup of each launch puts them back to zero, so one route
    serves any number of calls: every call into NaN-filled outputs writes all
    of them, with the same bits as a call on a fresh route, and the counters
    read zero afterwards."""
    announce("grouped experts: one route, repeated calls")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(11)
    T = 700
    x1, x2 = bf16_randn((T, H), g, dev), bf16_randn((T, H), g, dev)
    top = torch.from_numpy(_random_topk(T, K_TOP, E, 11, skew=1.1)).to(dev)
    route = ops.moe_permute(top, E, 256)

    def run(x, r):
        act = torch.full((T * K_TOP, I), float("nan"), dtype=torch.bfloat16, device=dev)
        y = torch.full((T * K_TOP, H), float("nan"), dtype=torch.bfloat16, device=dev)
        return ops.moe_experts_grouped(x, w13, w2, r, act=act, y_slot=y)

    ys = [run(x, route) for x in (x1, x2, x1, x2)]
    fresh = [run(x, ops.moe_permute(top, E, 256)) for x in (x1, x2)]
    torch.cuda.synchronize()
    assert bool(torch.isfinite(ys[0]).all()) and bool(torch.isfinite(ys[1]).all())
    assert torch.equal(ys[0], fresh[0]) and torch.equal(ys[2], fresh[0])
    assert torch.equal(ys[1], fresh[1]) and torch.equal(ys[3], fresh[1])
    assert not torch.equal(ys[0], ys[1])
    assert int(route.meta[4:].abs().sum()) == 0 and int(route.meta[2]) == 0
    # the one-launch form's per-tile counters (word 3 of each tile row) are back at zero
    assert int(route.tiles[: int(route.meta[0]), 3].abs().sum()) == 0


@pytest.mark.parametrize("T,spread", [(700, "skew"), (640, "crowded"), (4096, "skew"), (96, "uniform")])
def test_experts_grouped_one_launch_vs_two(dev, experts, T, spread):
    """Both GEMMs in one launch (down items waiting on their tile's gate_up
    items) against the two-launch form, which the library takes when act is
    not 128-byte aligned: the same y_slot bits.  Routings: Zipf-skewed, a
    prompt whose tokens crowd onto 8 experts (the random-init model's deep
    layers: 3 tiles each for 8 experts, a few rows for the rest), uniform."""
    announce(f"grouped experts one launch vs two, T={T} {spread}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(13 + T)
    x = bf16_randn((T, H), g, dev)
    if spread == "crowded":
        rng = np.random.default_rng(T)
        top = np.stack([rng.permutation(E)[:K_TOP] for _ in range(T)])
        hot = rng.permutation(E)[:K_TOP]
        top[: T - 40] = np.stack([rng.permutation(hot) for _ in range(T - 40)])
        top = torch.from_numpy(top.astype(np.int32)).to(dev)
    else:
        top = torch.from_numpy(_random_topk(T, K_TOP, E, 17 + T, skew=1.1 if spread == "skew" else None)).to(dev)
    route = ops.moe_permute(top, E, 256)
    n = T * K_TOP * I
    flat = torch.empty(n + 64, dtype=torch.bfloat16, device=dev)
    assert flat.data_ptr() % 128 == 0
    y1 = ops.moe_experts_grouped(x, w13, w2, route, act=flat[:n].view(T * K_TOP, I))
    y2 = ops.moe_experts_grouped(x, w13, w2, route, act=flat[32:32 + n].view(T * K_TOP, I))  # 64 B off
    y3 = ops.moe_experts_grouped(x, w13, w2, route, act=flat[:n].view(T * K_TOP, I))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y1).all())
    assert torch.equal(y1, y2) and torch.equal(y1, y3)
    assert int(route.meta[2]) == 0 and int(route.tiles[: int(route.meta[0]), 3].abs().sum()) == 0


@pytest.mark.parametrize("T", [1, 8, 48, 49, 64, 128])
def test_moe_block_vs_oracle(dev, experts, router_w, T):
    """Full block, every path the bench times at the size it times it:
    T = 1 (one launch), 8 (three-launch decode block), 48 (dispatch + expert
    GEMVs, the last size on them), 49 and 64 (dispatch + grouped MFMA
    GEMMs), 128.  Expert ids exact wherever the gap exceeds 1e-3; every row
    vs the oracle (near-tied rows over the product's experts, weights from
    the oracle's logits)."""
    from qmoe import moe as qmoe_moe

    path = ("one launch" if T == 1 else "three-launch block" if T <= ops.DECODE_BLOCK_MAX_T else
            "expert GEMVs" if T <= qmoe_moe.GEMV_MAX_TOKENS else "grouped GEMMs")
    announce(f"moe block T={T} ({path})")
    assert qmoe_moe.GEMV_MAX_TOKENS == 48, "the T=48 / T=49 cases cover the GEMV / grouped switch"
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(1000 + T)
    x = bf16_randn((T, H), g, dev)
    blk = MoEBlock(router_w, w13, w2, K_TOP)
    out = blk(x)
    torch.cuda.synchronize()
    rl, rw, ri = oracle.router_topk(x.cpu(), router_w.cpu(), K_TOP)
    ok = gap_mask(rl, K_TOP)
    _, _, ti = blk.last_routing
    idx = ti.cpu().long()
    assert torch.equal(idx[ok], ri[ok])
    ri, rw = ri.clone(), rw.clone()
    ri[~ok] = idx[~ok]
    rw[~ok] = torch.softmax(rl[~ok].gather(1, idx[~ok]), dim=1)
    ref = _oracle_rows(x.cpu(), ri, rw, _ExpertCache(w13, w2), range(T))
    assert_close_layer(out.cpu(), ref, f"moe block T={T}")


def test_moe_block_prefill_zipf_T4096(dev, experts, router_w):
    """The prefill MoE block workload: T = 4096 tokens, H = 2048, 128 experts,
    top-8, I = 768, with the router bias fitted so that expert popularity
    follows Zipf(1.1) (the most popular expert takes every token: 16
    consecutive 256-row tiles; the coldest about 40 rows).  Routing: logits
    within 1e-4, expert ids exact wherever the gap exceeds 1e-3, histogram
    within 2% L1 of the Zipf targets.  Output: 160 sampled rows (including
    every row routed to the 8 coldest experts) vs oracle.moe_block_prefill."""
    import bench

    announce("moe block prefill T=4096, Zipf(1.1) routing")
    w13, w2 = experts
    T = 4096
    g = torch.Generator(device=dev).manual_seed(4096)
    x = bf16_randn((T, H), g, dev)
    bias, target = bench.zipf_router_bias(x, router_w, K_TOP)
    blk = MoEBlock(router_w, w13, w2, K_TOP, router_bias=bias)
    residual = torch.randn(T, H, generator=g, device=dev)
    out = blk(x, residual)
    torch.cuda.synchronize()
    logits, tw, ti = blk.last_routing
    rl, rw, ri = oracle.router_topk(x.cpu(), router_w.cpu(), K_TOP, bias.cpu())
    assert max_abs(logits, rl) <= 1e-4
    ok = gap_mask(rl, K_TOP)
    assert ok.float().mean() > 0.8
    assert torch.equal(ti.cpu().long()[ok], ri[ok])
    hist = bench.routing_histogram(ti, target, T)
    print(f"  routing vs Zipf(1.1): {hist}", flush=True)
    assert hist["achieved_rows_top8"][0] == T
    assert hist["l1_vs_target"] < 0.02 and hist["experts_below_32_rows"] == 0
    # sampled rows: every row of the 8 coldest experts, then random rows
    cold = torch.argsort(target)[:8].cpu()
    tic = ti.cpu().long()
    cold_rows = torch.nonzero(torch.isin(tic, cold).any(1)).flatten()
    cold_rows = cold_rows[ok[cold_rows]][:96]
    rng = np.random.default_rng(3)
    extra = torch.from_numpy(rng.choice(np.flatnonzero(ok.numpy()), 160 - len(cold_rows), replace=False))
    rows = torch.unique(torch.cat([cold_rows, extra]))
    gate_up = weights.unpack_gate_up(w13).float()  # (E, H, 2I), on the GPU
    down = weights.unpack_down(w2).float()  # (E, I, H)
    ref, r_i, _, _ = oracle.moe_block_prefill(x[rows.to(dev)], router_w, gate_up, down, K_TOP, bias)
    torch.cuda.synchronize()
    assert torch.equal(r_i.cpu().sort(1).values, ri[rows].sort(1).values)
    got = (out - residual)[rows.to(dev)]
    assert_close_layer(got.cpu(), ref.cpu(), "moe block T=4096 Zipf(1.1)")


def _blockwise_seam(ex, xf, ti, tw, B=16):
    """Call torch_blockwise_matmul_inference with the reference's block
    format for routing (ti, tw): blocks of B token rows per expert, padding
    rows pointing at the extra row T, affinities masked to the chosen experts."""
    T, dev = xf.shape[0], xf.device
    top = ti.long().cpu()
    blocks, b2e = [], []
    for e in range(E):
        toks = torch.nonzero((top == e).any(dim=1)).flatten().tolist()
        for s0 in range(0, len(toks), B):
            chunk = toks[s0 : s0 + B]
            blocks.append(chunk + [T] * (B - len(chunk)))
            b2e.append(e)
    masked = torch.zeros(T, E, device=dev)
    masked.scatter_(1, ti.long(), tw)
    tpid = torch.tensor(blocks, dtype=torch.long, device=dev).flatten()
    return ex.torch_blockwise_matmul_inference(B, len(blocks), xf, masked, tpid, torch.tensor(b2e, device=dev))


@pytest.mark.parametrize("T", [8, 96])
def test_expert_seams_match_block(dev, experts, router_w, T):
    """forward_selective_loading (qwen_with_nki.py:3456-3478) and
    torch_blockwise_matmul_inference (5872-5881, semantics 5728-5789) against
    the oracle MoE over the same routing: the selective seam with the
    L1-normalised softmax affinities of the chosen experts, the blockwise
    seam with the masked affinities of the reference's block format (blocks
    of 16 rows per expert, padding row id T).  The seams return the input
    dtype, so they get fp32 rows (bf16 values) and return fp32.  T = 8 runs
    the expert GEMVs (fp32 activations: 2e-3 / 1e-4), T = 96 the grouped MFMA
    GEMMs (bf16 activations: 2e-2 / 5e-3).  Both also match the block's own
    output at the layer bar."""
    announce(f"expert seams T={T}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(42 + T)
    x = bf16_randn((T, H), g, dev)
    blk = MoEBlock(router_w, w13, w2, K_TOP)
    ref_blk = blk(x)
    logits, tw, ti = blk.last_routing
    aff = torch.softmax(logits, dim=-1)
    xf = x.float()
    sel = blk.experts.forward_selective_loading(xf, aff, ti)
    top = ti.long().cpu()
    bw = _blockwise_seam(blk.experts, xf, ti, tw)
    torch.cuda.synchronize()
    assert sel.dtype == torch.float32 and bw.dtype == torch.float32
    chosen = torch.gather(aff.float().cpu(), 1, top)
    w_sel = chosen / chosen.sum(dim=1, keepdim=True)
    cache = _ExpertCache(w13, w2)
    ref_sel = _oracle_rows(x.cpu(), top, w_sel, cache, range(T))
    ref_bw = _oracle_rows(x.cpu(), top, tw.float().cpu(), cache, range(T))
    tol = (2e-3, 1e-4) if T <= 48 else (2e-2, 5e-3)
    assert_close_layer(sel.float().cpu(), ref_sel, "selective-loading seam vs oracle", *tol)
    assert_close_layer(bw.float().cpu(), ref_bw, "blockwise seam vs oracle", *tol)
    # the block runs other kernels (the decode block at T <= 8): the layer bar
    assert_close_layer(sel.float().cpu(), ref_blk.cpu(), "selective-loading seam vs block", 2e-2, 5e-3)
    assert_close_layer(bw.float().cpu(), ref_blk.cpu(), "blockwise seam vs block", 2e-2, 5e-3)


@pytest.mark.parametrize("T", [4, 96])
def test_expert_seams_early_affinity_modulation(dev, experts, router_w, T):
    """early_expert_affinity_modulation=True (qwen_with_nki.py:5768-5775,
    3449): both seams scale each (token, expert) pair's input row by its
    affinity and add the MLP outputs unscaled.  The scaled rows are rounded
    to bf16 (the experts read bf16), so the bar against the fp32 oracle of
    the same schedule is the layer bar, 2e-2 / 5e-3.  T = 4 runs the expert
    GEMVs on 32 pair rows, T = 96 the grouped GEMMs on 768.  The late
    (output-scaled) schedule is far from both: the flag took effect."""
    announce(f"expert seams, early affinity modulation, T={T}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(4242 + T)
    x = bf16_randn((T, H), g, dev)
    blk = MoEBlock(router_w, w13, w2, K_TOP)
    blk(x)
    logits, tw, ti = blk.last_routing
    ex = blk.experts
    ex.routed_experts_mlp_config.early_expert_affinity_modulation = True
    aff = torch.softmax(logits, dim=-1)
    xf = x.float()
    sel = ex.forward_selective_loading(xf, aff, ti)
    bw = _blockwise_seam(ex, xf, ti, tw)
    torch.cuda.synchronize()
    top = ti.long().cpu()
    chosen = torch.gather(aff.float().cpu(), 1, top)
    w_sel = chosen / chosen.sum(dim=1, keepdim=True)
    cache = _ExpertCache(w13, w2)
    ref_sel = oracle.moe_experts_early(x.cpu(), top, w_sel, cache)
    ref_bw = oracle.moe_experts_early(x.cpu(), top, tw.float().cpu(), cache)
    assert_close_layer(sel.float().cpu(), ref_sel, "early selective-loading seam vs oracle", 2e-2, 5e-3)
    assert_close_layer(bw.float().cpu(), ref_bw, "early blockwise seam vs oracle", 2e-2, 5e-3)
    late = _oracle_rows(x.cpu(), top, tw.float().cpu(), cache, range(T))
    assert max_abs(bw.float().cpu(), late) > 10 * max_abs(bw.float().cpu(), ref_bw)


# --------------------------------------------------------------------------- attention
HQ, HKV, D = 32, 4, 128


@pytest.fixture(scope="module")
def attn_w(dev):
    g = torch.Generator(device=dev).manual_seed(77)
    wqkv = bf16_randn(((HQ + 2 * HKV) * D, H), g, dev, std=0.02)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    return wqkv, qn, kn


def _rope(max_pos, dev):
    cos, sin = oracle.rope_tables(D, torch.arange(max_pos), 1.0e6)
    return cos[:, : D // 2].contiguous().to(dev), sin[:, : D // 2].contiguous().to(dev)


# B*S <= 16: GEMV + finish path (8, 16: batched decode steps); up to 255 rows:
# 128-row MFMA tiles; from 256 rows the direct-to-LDS pipelines: one
# workgroup per CU while the tiles fit one round, 64-row tiles (1 x 300, 2 x
# 180: ragged) or 128-row ones (1 x 640, 3 x 130: ragged), then 128-row
# tiles two per CU (3 x 257) and 256-row tiles (3 x 900, 8 x 1000: ragged)
@pytest.mark.parametrize("B,S,start", [(2, 100, 0), (1, 5, 8000), (3, 257, 0), (8, 1, 1279), (16, 1, 40),
                                       (1, 1, 0), (3, 900, 5), (2, 1024, 0), (1, 200, 3), (8, 1000, 3),
                                       (1, 640, 0), (3, 130, 11), (1, 300, 7), (2, 180, 0)])
def test_qkv_norm_rope(dev, attn_w, B, S, start):
    announce(f"qkv_norm_rope B={B} S={S} start={start}")
    wqkv, qn, kn = attn_w
    S_max = start + S + 3
    g = torch.Generator(device=dev).manual_seed(B * 1000 + S)
    x = bf16_randn((B * S, H), g, dev)
    pos = (start + torch.arange(S, device=dev)).repeat(B).to(torch.int32)
    cos, sin = _rope(S_max, dev)
    kc = torch.zeros(B, HKV, S_max, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = ops.qkv_norm_rope(x, wqkv, qn, kn, cos, sin, pos, B, S, HQ, HKV, kc, vc, 1e-6)
    torch.cuda.synchronize()
    wq, wk, wv = wqkv.float().cpu().split([HQ * D, HKV * D, HKV * D])
    rq, rk, rv = oracle.qkv_norm_rope(x.cpu().view(B, S, H), wq, wk, wv, qn.cpu(), kn.cpu(),
                                      pos.cpu().view(B, S).long(), HQ, HKV, D, 1e-6, 1.0e6)
    # bf16 outputs: one rounding of an fp32 value
    def chk(a, r, what):
        err = (a.float().cpu() - r).abs() - r.abs() * 2 ** -8
        assert float(err.max()) <= 2e-4, what
    chk(q.view(B, S, HQ, D).transpose(1, 2), rq, "q")
    chk(kc[:, :, start : start + S], rk, "k cache")
    chk(vc[:, :, start : start + S], rv, "v cache")
    assert float(kc[:, :, :start].abs().sum()) == 0.0 and float(kc[:, :, start + S :].abs().sum()) == 0.0


# (7, 7, 1, 5400): 21 heads on the one-head 256-row pipeline (215 wide tiles
# would not fill the GPU).  From 256 tiles of 128 tokens x 5 heads the wide
# kernel runs: the attention shape with a ragged last token block (T = 4400),
# 21 heads (five 640-row panels, the last holding one head) at T = 7800, and
# 4 q / 1 kv heads (6 heads: a second panel with one live head) at T = 16500.
@pytest.mark.parametrize("Hq_,Hkv_,B,S,start", [(7, 7, 1, 5400, 0), (32, 4, 4, 1100, 2), (7, 7, 2, 3900, 0),
                                                (4, 1, 1, 16500, 0)])
def test_qkv_norm_rope_wide_odd_heads(dev, Hq_, Hkv_, B, S, start):
    """Other head counts and ragged token blocks on the large-T QKV
    pipelines, vs the oracle."""
    announce(f"qkv_norm_rope wide Hq={Hq_} Hkv={Hkv_} T={B * S}")
    g = torch.Generator(device=dev).manual_seed(21 + Hq_ + S)
    wqkv = bf16_randn(((Hq_ + 2 * Hkv_) * D, H), g, dev, std=0.02)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    S_max = start + S + 3
    x = bf16_randn((B * S, H), g, dev)
    pos = (start + torch.arange(S, device=dev)).repeat(B).to(torch.int32)
    cos, sin = _rope(S_max, dev)
    kc = torch.zeros(B, Hkv_, S_max, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q = ops.qkv_norm_rope(x, wqkv, qn, kn, cos, sin, pos, B, S, Hq_, Hkv_, kc, vc, 1e-6)
    torch.cuda.synchronize()
    wq, wk, wv = wqkv.float().cpu().split([Hq_ * D, Hkv_ * D, Hkv_ * D])
    rq, rk, rv = oracle.qkv_norm_rope(x.cpu().view(B, S, H), wq, wk, wv, qn.cpu(), kn.cpu(),
                                      pos.cpu().view(B, S).long(), Hq_, Hkv_, D, 1e-6, 1.0e6)
    for a, r, what in ((q.view(B, S, Hq_, D).transpose(1, 2), rq, "q"), (kc[:, :, start : start + S], rk, "k"),
                       (vc[:, :, start : start + S], rv, "v")):
        err = (a.float().cpu() - r).abs() - r.abs() * 2 ** -8  # one bf16 rounding
        assert float(err.max()) <= 2e-4, what


@pytest.mark.parametrize("B,S,start", [(2, 200, 0), (1, 1024, 0), (2, 70, 130), (8, 64, 0)])
def test_attn_prefill(dev, B, S, start):
    announce(f"attn_prefill B={B} S={S} start={start}")
    S_max = start + S + 17
    g = torch.Generator(device=dev).manual_seed(S + start)
    q = bf16_randn((B * S, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    # poison the cache beyond the visible range: must not leak into outputs
    kc[:, :, start + S :] = float("nan")
    vc[:, :, start + S :] = float("nan")
    out = ops.attn_prefill(q, kc, vc, B, S, start)
    torch.cuda.synchronize()
    qi = (start + torch.arange(S)).view(1, S).expand(B, S)
    ref = oracle.gqa_attention(q.cpu().view(B, S, HQ, D).transpose(1, 2),
                               kc.cpu()[:, :, : start + S], vc.cpu()[:, :, : start + S], qi)
    assert_close_layer(out.cpu().view(B, S, HQ, D), ref, f"attn_prefill B={B} S={S}",
                       max_abs_tol=2e-2, mean_rel_tol=5e-3)


@pytest.mark.parametrize("B,S,start", [(1, 640, 0), (1, 512, 0), (1, 300, 0), (1, 440, 200), (2, 256, 0),
                                       (1, 1024, 0), (1, 64, 0)])
def test_attn_prefill_key_split(dev, B, S, start):
    """The workspace form: launches with fewer query tiles than CUs split
    their longer tiles' key ranges over two workgroups and merge the
    partials in the tile's last workgroup (640 and 512 tokens, and 440 at
    start 200, split; the others run unsplit).  Against the oracle, the same
    bits on a repeat call (split order, not arrival order), close to the
    unsplit launch, counters back at zero, NaN-poisoned rows unread."""
    announce(f"attn_prefill key split B={B} S={S} start={start}")
    S_max = start + S + 17
    g = torch.Generator(device=dev).manual_seed(3 * S + start + B)
    q = bf16_randn((B * S, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    kc[:, :, start + S :] = float("nan")
    vc[:, :, start + S :] = float("nan")
    ws = ops.attn_prefill_workspace(B, S, HQ, D, dev)
    out = ops.attn_prefill(q, kc, vc, B, S, start, workspace=ws)
    out2 = ops.attn_prefill(q, kc, vc, B, S, start, workspace=ws)
    plain = ops.attn_prefill(q, kc, vc, B, S, start)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    n_cnt = -(-S // 128) * HQ * B
    assert int(ws[:n_cnt].abs().sum()) == 0
    assert max_abs(out.float(), plain.float()) < 2e-2
    qi = (start + torch.arange(S)).view(1, S).expand(B, S)
    ref = oracle.gqa_attention(q.cpu().view(B, S, HQ, D).transpose(1, 2),
                               kc.cpu()[:, :, : start + S], vc.cpu()[:, :, : start + S], qi)
    assert_close_layer(out.cpu().view(B, S, HQ, D), ref, f"attn_prefill split B={B} S={S}",
                       max_abs_tol=2e-2, mean_rel_tol=5e-3)


def test_attention_layer_B8_prefill1024_decode_to_8192(dev, attn_w):
    """The attention-layer workload: batch 8, a 1024-token prefill into a
    cache of 8193 rows, decode steps right after it (positions 1024, 1025),
    then at context 1280 through the context-bucket launch (2048 rows) and at
    context 8192 (the cache rows between hold other tokens' K/V, written
    directly).  Each step through ``Attention.forward`` (QKV + q/k-norm +
    RoPE + cache append, causal GQA, o_proj into the residual) vs the
    oracle's attention layer over the same cache contents."""
    from qmoe.attention import Attention, KVCache

    announce("attention layer B=8 prefill 1024, decode at 1024, 1025, ctx 1280 and 8192")
    wqkv, qn, kn = attn_w
    B, S, S_max = 8, 1024, 8193
    g = torch.Generator(device=dev).manual_seed(8192)
    wo = bf16_randn((H, HQ * D), g, dev, std=0.02)
    att = Attention(wqkv, qn, kn, wo, HQ, HKV, D, 1e-6)
    cache = KVCache(B, HKV, S_max, D, dev)
    cos, sin = _rope(S_max, dev)
    wq, wk, wv = wqkv.float().split([HQ * D, HKV * D, HKV * D])
    w = {"q_proj": wq, "k_proj": wk, "v_proj": wv, "o_proj": wo.float(), "q_norm": qn.float(),
         "k_norm": kn.float()}
    c = dict(n_q=HQ, n_kv=HKV, head_dim=D, eps=1e-6, theta=1.0e6)
    # prefill
    x = bf16_randn((B * S, H), g, dev)
    pos = torch.arange(S, device=dev, dtype=torch.int32).repeat(B)
    res = torch.zeros(B * S, H, device=dev)
    att.forward(x, res, pos, B, S, cache, cos, sin, 0)
    torch.cuda.synchronize()
    ref, (rk, rv) = oracle.attention_layer(x.float().view(B, S, H), w, pos.view(B, S).long(), c)
    rows = torch.from_numpy(np.random.default_rng(0).choice(B * S, 256, replace=False)).to(dev)
    assert_close_layer(res[rows].cpu(), ref.reshape(B * S, H)[rows].cpu(), "attention prefill B=8 S=1024")
    # cache rows: one bf16 rounding of the fp32 value, plus the difference of
    # two fp32 summation orders over K = 2048 (the oracle's GEMM runs on the GPU here)
    for what, a, r in (("k", cache.k[:, :, :S], rk), ("v", cache.v[:, :, :S], rv)):
        err = (a.float() - r).abs() - r.abs() * 2 ** -8
        assert float(err.max()) <= 1e-3, f"{what} cache rows after prefill"

    def step(p, max_ctx=None, label=""):
        xd = bf16_randn((B, H), g, dev)
        pd = torch.full((B,), p, device=dev, dtype=torch.int32)
        out = torch.zeros(B, H, device=dev)
        past = (cache.k[:, :, :p].float().clone(), cache.v[:, :, :p].float().clone())
        att.forward(xd, out, pd, B, 1, cache, cos, sin, 0, max_ctx=max_ctx)
        torch.cuda.synchronize()
        r, _ = oracle.attention_layer(xd.float().view(B, 1, H), w, pd.view(B, 1).long(), c, past)
        assert_close_layer(out.cpu(), r.reshape(B, H).cpu(), f"attention decode {label}")

    step(1024, label="position 1024")
    step(1025, label="position 1025")
    cache.k[:, :, 1026:1279] = bf16_randn((B, HKV, 253, D), g, dev)
    cache.v[:, :, 1026:1279] = bf16_randn((B, HKV, 253, D), g, dev)
    step(1279, max_ctx=2048, label="ctx 1280 (2048-row bucket)")
    cache.k[:, :, 1280:8191] = bf16_randn((B, HKV, 6911, D), g, dev)
    cache.v[:, :, 1280:8191] = bf16_randn((B, HKV, 6911, D), g, dev)
    step(8191, label="ctx 8192")


@pytest.mark.parametrize("K,N", [(512, 100), (2048, 5120), (4096, 2048)])
def test_gemv_rmsnorm_fused(dev, K, N):
    """The input RMSNorm fused into the one-row GEMV gives the same bits as
    qmoe_rmsnorm_residual followed by qmoe_gemm, in every epilogue mode; and
    gemv_rmsnorm + qkv_finish equals qkv_norm_rope on the normed row."""
    announce(f"gemv_rmsnorm K={K} N={N}")
    g = torch.Generator(device=dev).manual_seed(K + N)
    h = torch.randn(1, K, generator=g, device=dev) * 3.0
    w = (1.0 + 0.2 * torch.randn(K, generator=g, device=dev)).to(torch.bfloat16)
    B = bf16_randn((N, K), g, dev, std=0.02)
    x = ops.rmsnorm_residual(h, w, 1e-6)
    for mode in (_lib.GEMM_STORE_BF16, _lib.GEMM_STORE_F32):
        ref = ops.gemm(x, B, mode)
        got = ops.gemv_rmsnorm(h, w, 1e-6, B, mode)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"mode {mode}"
    acc_ref = torch.randn(1, N, generator=g, device=dev)
    acc_got = acc_ref.clone()
    ops.gemm(x, B, _lib.GEMM_ADD_F32, out=acc_ref)
    ops.gemv_rmsnorm(h, w, 1e-6, B, _lib.GEMM_ADD_F32, out=acc_got)
    torch.cuda.synchronize()
    assert torch.equal(acc_got, acc_ref)


def test_qkv_finish_matches_qkv_norm_rope(dev, attn_w):
    announce("qkv_finish vs qkv_norm_rope, one token")
    wqkv, qn, kn = attn_w
    g = torch.Generator(device=dev).manual_seed(21)
    h = torch.randn(1, H, generator=g, device=dev)
    w = torch.ones(H, dtype=torch.bfloat16, device=dev)
    pos = torch.tensor([37], dtype=torch.int32, device=dev)
    cos, sin = _rope(64, dev)
    kc1 = torch.zeros(1, HKV, 64, D, dtype=torch.bfloat16, device=dev)
    vc1, kc2, vc2 = torch.zeros_like(kc1), torch.zeros_like(kc1), torch.zeros_like(kc1)
    q1 = ops.qkv_norm_rope(ops.rmsnorm_residual(h, w, 1e-6), wqkv, qn, kn, cos, sin, pos, 1, 1, HQ, HKV, kc1, vc1,
                           1e-6)
    raw = ops.gemv_rmsnorm(h, w, 1e-6, wqkv, _lib.GEMM_STORE_F32)
    q2 = ops.qkv_finish(raw, qn, kn, cos, sin, pos, 1, 1, HQ, HKV, kc2, vc2, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)


# (B, Hq, Hkv, S_max, positions, bucket): the new key first in the cache, last
# and first of a 64-key wave, G = 16 and G = 1, 8 rows at a capacity of 8193
# (four waves per split workgroup, keys up to the last cache row), and
# positions at or past the bucket (the row is written, not attended to).
@pytest.mark.parametrize("B,Hq_,Hkv_,S_max,pos,bucket", [
    (1, 32, 4, 2048, [0], None), (1, 32, 4, 2048, [63], 1024), (1, 32, 4, 2048, [64], 1024),
    (3, 32, 4, 2048, [700, 5, 1023], 1024), (2, 32, 2, 512, [100, 511], None), (2, 4, 4, 512, [10, 300], None),
    (8, 32, 4, 8193, [1279, 0, 255, 256, 4000, 8192, 63, 64], None),
    (3, 32, 4, 2048, [1024, 100, 2047], 1024), (1, 32, 4, 2048, [1500], 256),
    # batch 1 over a long cache (four waves per split workgroup), through a bucket too
    (1, 32, 4, 8193, [8000], None), (2, 32, 4, 8193, [100, 5000], 8192), (1, 32, 4, 8193, [700], 1024)])
def test_attn_decode_fused_matches_finish_then_decode(dev, B, Hq_, Hkv_, S_max, pos, bucket):
    """qmoe_attn_decode_fused gives the bits of qmoe_qkv_finish followed by the
    decode attention over ctx = position + 1: the same output and the same
    cache rows written.  The cache row at each position starts as NaN, so a
    fused launch that attended to the stale row instead of the new one fails."""
    announce(f"attn_decode_fused B={B} Hq={Hq_} Hkv={Hkv_} S_max={S_max} pos={pos} bucket={bucket}")
    g = torch.Generator(device=dev).manual_seed(S_max + sum(pos) + Hq_)
    raw = torch.randn(B, (Hq_ + 2 * Hkv_) * D, generator=g, device=dev)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = _rope(S_max, dev)
    kc = bf16_randn((B, Hkv_, S_max, D), g, dev)
    vc = bf16_randn((B, Hkv_, S_max, D), g, dev)
    for b, p in enumerate(pos):
        kc[b, :, p] = float("nan")
        vc[b, :, p] = float("nan")
    pt = torch.tensor(pos, dtype=torch.int32, device=dev)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    q1 = ops.qkv_finish(raw, qn, kn, cos, sin, pt, B, 1, Hq_, Hkv_, kc1, vc1, 1e-6)
    o1 = ops.attn_decode(q1, kc1, vc1, pt + 1, max_ctx=bucket)
    o2 = ops.attn_decode_fused(raw, qn, kn, cos, sin, pt, Hq_, Hkv_, kc2, vc2, 1e-6, max_ctx=bucket)
    o3 = ops.attn_decode_fused(raw, qn, kn, cos, sin, pt, Hq_, Hkv_, kc2, vc2, 1e-6, max_ctx=bucket)
    torch.cuda.synchronize()
    assert not torch.isnan(o1).any()
    assert torch.equal(o2, o1) and torch.equal(o3, o1)
    assert torch.equal(kc2, kc1) and torch.equal(vc2, vc1)


def test_attn_decode_fused_rejected_positions(dev):
    """A position outside [0, min(S_max, max_pos)) writes no cache row and its
    output row is zeros; the other rows are unaffected."""
    announce("attn_decode_fused rejected positions")
    B, S_max = 3, 256
    g = torch.Generator(device=dev).manual_seed(5)
    raw = torch.randn(B, (HQ + 2 * HKV) * D, generator=g, device=dev)
    qn = torch.ones(D, dtype=torch.bfloat16, device=dev)
    cos, sin = _rope(S_max, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    pt = torch.tensor([-1, 17, S_max], dtype=torch.int32, device=dev)
    kc1, vc1 = kc.clone(), vc.clone()
    o = ops.attn_decode_fused(raw, qn, qn, cos, sin, pt, HQ, HKV, kc1, vc1, 1e-6)
    kc2, vc2 = kc.clone(), vc.clone()
    q = ops.qkv_finish(raw[1:2].contiguous(), qn, qn, cos, sin, pt[1:2].contiguous(), 1, 1, HQ, HKV, kc2[1:2],
                       vc2[1:2], 1e-6)
    ref = ops.attn_decode(q, kc2[1:2], vc2[1:2], pt[1:2] + 1)
    torch.cuda.synchronize()
    assert torch.equal(o[0], torch.zeros_like(o[0])) and torch.equal(o[2], torch.zeros_like(o[2]))
    assert torch.equal(kc1[0], kc[0]) and torch.equal(kc1[2], kc[2]) and torch.equal(vc1[2], vc[2])
    assert torch.equal(o[1:2], ref) and torch.equal(kc1[1], kc2[1]) and torch.equal(vc1[1], vc2[1])


@pytest.mark.parametrize("ctx,bucket", [([1], 256), ([300, 1000, 17], 1024), ([256], 256),
                                        ([1000, 17, 640, 1024, 5, 900, 128, 129], 1024)])
def test_attn_decode_bucket(dev, ctx, bucket):
    """A launch sized for a context bucket gives the same bits as the one sized
    for the whole cache (S_max 2048): the live splits and the merge are the
    same work."""
    announce(f"attn_decode_bucket ctx={ctx} bucket={bucket}")
    B, S_max = len(ctx), 2048
    g = torch.Generator(device=dev).manual_seed(sum(ctx) + bucket)
    q = bf16_randn((B, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    cl = torch.tensor(ctx, dtype=torch.int32, device=dev)
    ref = ops.attn_decode(q, kc, vc, cl)
    got = ops.attn_decode(q, kc, vc, cl, max_ctx=bucket)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("B,S,start", [(1, 5, 0), (1, 5, 613), (2, 8, 130)])
def test_attn_prefill_device_start(dev, B, S, start):
    """The chunk start read from device memory (qmoe_attn_prefill_at) gives
    the same bits as the host-argument form, including replays of one
    captured launch at two positions."""
    announce(f"attn_prefill_at B={B} S={S} start={start}")
    S_max = start + S + 40
    g = torch.Generator(device=dev).manual_seed(S + start)
    q = bf16_randn((B * S, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    ref = ops.attn_prefill(q, kc, vc, B, S, start)
    st = torch.tensor([start], dtype=torch.int32, device=dev)
    got = ops.attn_prefill(q, kc, vc, B, S, st)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    out = torch.empty_like(ref)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.attn_prefill(q, kc, vc, B, S, st, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.attn_prefill(q, kc, vc, B, S, st, out=out)
    for p in (start + 17, start):
        st.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.attn_prefill(q, kc, vc, B, S, p))


@pytest.mark.parametrize("B,S,start", [(1, 5, 0), (1, 5, 700), (2, 3, 130), (1, 16, 63)])
def test_attn_decode_chunk(dev, B, S, start):
    """Few-token chunks at a device-held start as single-query decode problems
    (qmoe_attn_decode_chunk): against the oracle and the tiled prefill kernel,
    and in a captured graph replayed at two positions (including the clamp of
    a start past S_max - S)."""
    announce(f"attn_decode_chunk B={B} S={S} start={start}")
    S_max = start + S + 40
    g = torch.Generator(device=dev).manual_seed(3 * S + start)
    q = bf16_randn((B * S, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    st = torch.tensor([start], dtype=torch.int32, device=dev)
    got = ops.attn_decode_chunk(q, kc, vc, B, S, st)
    tiled = ops.attn_prefill(q, kc, vc, B, S, start)
    torch.cuda.synchronize()
    pos = torch.tensor([list(range(start, start + S))] * B)
    ref = oracle.gqa_attention(q.cpu().view(B, S, HQ, D).transpose(1, 2), kc.cpu()[:, :, : start + S],
                               vc.cpu()[:, :, : start + S], pos)
    assert_close_layer(got.cpu().view(B, S, HQ, D), ref, "attn_decode_chunk", max_abs_tol=1e-2,
                       mean_rel_tol=5e-3)
    assert float((got.float() - tiled.float()).abs().max()) <= 1e-2
    ws = ops.attn_decode_workspace(B * S, HQ, D, S_max, dev)
    out = torch.empty_like(got)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.attn_decode_chunk(q, kc, vc, B, S, st, workspace=ws, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.attn_decode_chunk(q, kc, vc, B, S, st, workspace=ws, out=out)
    for p, eff in ((start + 17, start + 17), (start, start), (S_max, S_max - S)):
        st.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        eager = ops.attn_decode_chunk(q, kc, vc, B, S, torch.tensor([eff], dtype=torch.int32, device=dev))
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# batch 8 with contexts that end on, just past and inside 64-key splits
@pytest.mark.parametrize("ctx", [[1], [300, 1000, 17], [8192] * 2, [1, 64, 65, 128, 129, 700, 1000, 2048]])
def test_attn_decode(dev, ctx):
    announce(f"attn_decode ctx={ctx}")
    B = len(ctx)
    S_max = max(max(ctx), 256)
    g = torch.Generator(device=dev).manual_seed(sum(ctx))
    q = bf16_randn((B, HQ, D), g, dev)
    kc = bf16_randn((B, HKV, S_max, D), g, dev)
    vc = bf16_randn((B, HKV, S_max, D), g, dev)
    cl = torch.tensor(ctx, dtype=torch.int32, device=dev)
    out = ops.attn_decode(q, kc, vc, cl)
    torch.cuda.synchronize()
    for b in range(B):
        L = ctx[b]
        ref = oracle.gqa_attention(q.cpu()[b : b + 1].view(1, HQ, 1, D), kc.cpu()[b : b + 1, :, :L],
                                   vc.cpu()[b : b + 1, :, :L], torch.tensor([[L - 1]]))
        assert_close_layer(out.cpu()[b].view(HQ, D), ref[0, 0], f"attn_decode ctx={L}",
                           max_abs_tol=1e-2, mean_rel_tol=5e-3)


# --------------------------------------------------------------------------- fused decode path
@pytest.mark.parametrize("T", [1, 3, 8, 17, 64, 65, 300, 640, 1024, 1025])
def test_moe_route_fused(dev, router_w, T):
    """qmoe_moe_route == router_topk + permute, on three calls in a row into
    the same buffers: the oracle's routing where the gap allows, the
    oracle's permutation of the ids it chose, the same bits as the two-step
    path, and the work counters back at zero."""
    announce(f"moe_route T={T}")
    g = torch.Generator(device=dev).manual_seed(500 + T)
    x = bf16_randn((T, H), g, dev)
    route = ops.Route.alloc(T, K_TOP, E, 128, dev, with_topk=True)
    for rep in range(3):
        ops.moe_route(x, router_w, K_TOP, None, 128, route=route)
        torch.cuda.synchronize()
        rl, rw, ri = oracle.router_topk(x.cpu(), router_w.cpu(), K_TOP)
        assert max_abs(route.logits, rl) <= 1e-4
        ok = gap_mask(rl, K_TOP)
        assert torch.equal(route.topk_idx.cpu().long()[ok], ri[ok])
        np.testing.assert_allclose(route.topk_w.cpu()[ok].numpy(), rw[ok].numpy(), rtol=2e-5, atol=1e-7)
        ref = oracle.moe_permute(route.topk_idx.cpu().numpy(), E, 128)
        assert torch.equal(route.slot_token.cpu(), torch.from_numpy(ref["slot_token"]))
        assert torch.equal(route.token_slot.cpu(), torch.from_numpy(ref["token_slot"]))
        assert torch.equal(route.offsets.cpu(), torch.from_numpy(ref["offsets"]))
        n_act = int(route.meta[1])
        assert torch.equal(route.active.cpu()[:n_act], torch.from_numpy(ref["active"]))
        assert int(route.meta[2]) == 0 and int(route.meta[4:].abs().sum()) == 0
    # the two-step path on the same logits: router_topk, then moe_permute
    logits, tw, ti = ops.router_topk(x, router_w, K_TOP)
    two = ops.moe_permute(ti, E, 128)
    torch.cuda.synchronize()
    assert torch.equal(route.logits, logits) and torch.equal(route.topk_idx, ti) and torch.equal(route.topk_w, tw)
    for f in ("counts", "offsets", "slot_token", "token_slot"):
        assert torch.equal(getattr(route, f), getattr(two, f)), f
    n_t, n_act = int(two.meta[0]), int(two.meta[1])
    assert torch.equal(route.meta[:3], two.meta[:3]) and torch.equal(route.tiles[:n_t], two.tiles[:n_t])
    assert torch.equal(route.active[:n_act], two.active[:n_act])


@pytest.mark.parametrize("T", [1, 2, 5, 8])
@pytest.mark.parametrize("normed", [False, True])
def test_moe_decode_block(dev, experts, router_w, T, normed):
    """Three-launch decode block: routing exact where the gap allows, output
    vs the oracle, repeat calls bitwise equal, in-place residual."""
    announce(f"moe_decode_block T={T} normed={normed}")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(900 + T)
    h = torch.randn(T, H, generator=g, device=dev)
    rms_w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    residual = torch.randn(T, H, generator=g, device=dev)
    bufs = ops.DecodeBlockBuffers.alloc(T, H, I, E, K_TOP, dev)
    if normed:
        x_ref = oracle.rmsnorm(h.cpu(), rms_w.cpu(), 1e-6).to(torch.bfloat16)
        run = lambda res, out: ops.moe_decode_block(router_w, w13, w2, K_TOP, h=h, rms_w=rms_w, eps=1e-6,
                                                    residual=res, out=out, bufs=bufs)
    else:
        x = h.to(torch.bfloat16)
        x_ref = x.cpu()
        run = lambda res, out: ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x, residual=res,
                                                    out=out, bufs=bufs)
    outs = [run(residual, None) for _ in range(3)]
    inplace = residual.clone()
    run(inplace, inplace)
    # a different input on the same workspace gives the fresh-workspace result
    x2 = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
    second = ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x2, residual=residual, bufs=bufs)
    fresh = ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x2, residual=residual,
                                 bufs=ops.DecodeBlockBuffers.alloc(T, H, I, E, K_TOP, dev))
    torch.cuda.synchronize()
    assert torch.equal(second, fresh)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert torch.equal(outs[0], inplace)
    outs[0] = run(residual, None)  # restore bufs (logits, top-k) for the checks below
    torch.cuda.synchronize()
    if normed:  # the fused RMSNorm output: one bf16 rounding of the fp32 value
        err = (bufs.x_out.float().cpu() - oracle.rmsnorm(h.cpu(), rms_w.cpu(), 1e-6)).abs()
        assert float((err - x_ref.float().abs() * 2 ** -8).max()) <= 1e-5
    xin = bufs.x_out.cpu() if normed else x_ref
    rl, rw, ri = oracle.router_topk(xin, router_w.cpu(), K_TOP)
    assert max_abs(bufs.logits, rl) <= 1e-4
    ok = gap_mask(rl, K_TOP)
    assert torch.equal(bufs.topk_idx.cpu().long()[ok], ri[ok])
    rows = [t for t in range(T) if bool(ok[t])]
    ref = _oracle_rows(xin, ri, rw, _ExpertCache(w13, w2), rows)
    assert_close_layer(outs[0].cpu()[rows] - residual.cpu()[rows], ref, f"decode block T={T}", 2e-3, 1e-4)


def _decode_status(bufs) -> int:
    """Status word of a decode-block workspace (nonzero once a wait gave up)."""
    off = _lib.DECODE_BLOCK_STATUS_OFFSET
    return int(bufs.workspace[off:off + 4].view(torch.int32).item())


def test_moe_decode_block_fused_state(dev, experts, router_w):
    """The single-launch T = 1 block carries call counters and tagged exchange
    slots in its workspace: 40 calls on one workspace with inputs changing
    from call to call each equal the same call on a fresh workspace (bitwise);
    three-launch T = 8 calls interleaved on the same workspace (their partials
    sit after the state) leave it intact; the status word stays 0."""
    announce("fused decode block: workspace state over 40 calls")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(77)
    bufs8 = ops.DecodeBlockBuffers.alloc(8, H, I, E, K_TOP, dev)
    bufs1 = ops.DecodeBlockBuffers(bufs8.logits[:1], bufs8.topk_idx[:1], bufs8.topk_w[:1], bufs8.workspace,
                                   bufs8.x_out[:1])
    xs = [bf16_randn((1, H), g, dev) for _ in range(5)]
    res = torch.randn(1, H, generator=g, device=dev)
    fresh = lambda T: ops.DecodeBlockBuffers.alloc(T, H, I, E, K_TOP, dev)
    refs = [ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x, residual=res, bufs=fresh(1)) for x in xs]
    x8 = bf16_randn((8, H), g, dev)
    res8 = torch.randn(8, H, generator=g, device=dev)
    ref8 = ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x8, residual=res8, bufs=fresh(8))
    for i in range(40):
        got = ops.moe_decode_block(router_w, w13, w2, K_TOP, x=xs[i % 5], residual=res, bufs=bufs1)
        assert torch.equal(got, refs[i % 5]), f"call {i}"
        if i % 7 == 3:
            assert torch.equal(ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x8, residual=res8, bufs=bufs8),
                               ref8), f"T=8 call after {i}"
    torch.cuda.synchronize()
    assert _decode_status(bufs8) == 0


def test_moe_decode_block_fused_graph_replays(dev, experts, router_w):
    """The single-launch block captured in a HIP graph: every replay (with
    eager calls on the same workspace between replays) equals eager."""
    announce("fused decode block: graph replays")
    w13, w2 = experts
    g = torch.Generator(device=dev).manual_seed(78)
    bufs = ops.DecodeBlockBuffers.alloc(1, H, I, E, K_TOP, dev)
    x = bf16_randn((1, H), g, dev)
    x_other = bf16_randn((1, H), g, dev)
    res = torch.randn(1, H, generator=g, device=dev)
    out = torch.empty(1, H, device=dev)
    ref = ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x, residual=res,
                               bufs=ops.DecodeBlockBuffers.alloc(1, H, I, E, K_TOP, dev))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x, residual=res, out=out, bufs=bufs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x, residual=res, out=out, bufs=bufs)
    for rep in range(6):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}"
        ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x_other, residual=res, bufs=bufs)
        torch.cuda.synchronize()
    assert _decode_status(bufs) == 0


@pytest.mark.parametrize("n_exp", [64, 256])
def test_moe_decode_block_fused_expert_counts(dev, n_exp):
    """The single-launch block at E = 64 (one key register per lane) and
    E = 256 (four), normed and not: routing exact where the gap allows, the
    output vs the oracle on the token's experts."""
    w_r = bf16_randn((n_exp, H), torch.Generator(device=dev).manual_seed(5 + n_exp), dev, std=0.02)
    g = torch.Generator(device=dev).manual_seed(600 + n_exp)
    w13 = bf16_randn((n_exp, 2 * I, H), g, dev, std=0.02)
    w2 = bf16_randn((n_exp, I // 8, H, 8), g, dev, std=0.02)
    rms_w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    for normed in (False, True):
        announce(f"fused decode block E={n_exp} normed={normed}")
        h = torch.randn(1, H, generator=g, device=dev)
        res = torch.randn(1, H, generator=g, device=dev)
        bufs = ops.DecodeBlockBuffers.alloc(1, H, I, n_exp, K_TOP, dev)
        if normed:
            out = ops.moe_decode_block(w_r, w13, w2, K_TOP, h=h, rms_w=rms_w, eps=1e-6, residual=res, bufs=bufs)
        else:
            out = ops.moe_decode_block(w_r, w13, w2, K_TOP, x=h.to(torch.bfloat16), residual=res, bufs=bufs)
        torch.cuda.synchronize()
        xin = bufs.x_out.cpu() if normed else h.to(torch.bfloat16).cpu()
        rl, rw, ri = oracle.router_topk(xin, w_r.cpu(), K_TOP)
        assert max_abs(bufs.logits, rl) <= 1e-4
        idx = bufs.topk_idx.cpu().long()
        if bool(gap_mask(rl, K_TOP)[0]):
            assert torch.equal(idx, ri)
            np.testing.assert_allclose(bufs.topk_w.cpu().numpy(), rw.numpy(), rtol=2e-5, atol=1e-7)
        else:  # near-tied k-th logit: the oracle takes the product's experts, weights from its own logits
            sel = rl.gather(1, idx)
            rw = torch.softmax(sel, dim=1)
            ri = idx
        ref = _oracle_rows(xin, ri, rw, _ExpertCache(w13, w2), [0])
        assert_close_layer(out.cpu() - res.cpu(), ref, f"fused block E={n_exp}", 2e-3, 1e-4)
        assert _decode_status(bufs) == 0


# --------------------------------------------------------------------------- embedding / greedy argmax
def test_embed_gather_and_bad_ids(dev):
    announce("embedding gather")
    g = torch.Generator(device=dev).manual_seed(3)
    V, Hh = 1000, 2048
    table = bf16_randn((V, Hh), g, dev)
    ids = torch.tensor([0, 999, 17, 17, 512], dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out = ops.embed(ids, table, err=err)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), table.cpu()[ids.cpu()].float())
    assert int(err.item()) == 0
    bad = torch.tensor([3, -1, V, 4], dtype=torch.int64, device=dev)
    out = ops.embed(bad, table, err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert float(out[1].abs().sum()) == 0.0 and float(out[2].abs().sum()) == 0.0
    assert torch.equal(out.cpu()[[0, 3]], table.cpu()[[3, 4]].float())


def test_argmax_rows_match_torch(dev):
    announce("argmax rows")
    g = torch.Generator(device=dev).manual_seed(4)
    n = 151936
    x = torch.randn(4, n, generator=g, device=dev)
    x[1, 777] = 50.0
    x[1, 99999] = 50.0  # tie: the lower index wins
    x[2, 1234] = float("nan")
    x[2, 5] = float("nan")  # first NaN wins
    x[3] = -float("inf")
    x[3, n - 1] = -1e30
    got = ops.argmax(x)
    torch.cuda.synchronize()
    assert got.cpu().tolist() == [int(x[0].cpu().argmax()), 777, 5, n - 1]
    y = torch.randn(7, 300, generator=g, device=dev)
    assert torch.equal(ops.argmax(y).cpu(), y.cpu().argmax(dim=-1))


def test_argmax_graph_replays(dev):
    """Captured argmax over a vocabulary-wide row, replayed with fresh data
    (written eagerly between replays): every replay equals torch.argmax."""
    announce("argmax in a HIP graph")
    g = torch.Generator(device=dev).manual_seed(5)
    n = 151936
    x = torch.empty(1, n, device=dev)
    out = torch.zeros(1, dtype=torch.int64, device=dev)
    ws = ops.argmax_workspace(1, dev)
    x.normal_(generator=g)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.argmax(x, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.argmax(x, out=out, workspace=ws)
    for i in range(6):
        x.normal_(generator=g)
        x[0, (i * 7919) % n] = 100.0 + i
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert int(out.item()) == (i * 7919) % n == int(x.cpu().argmax())


# --------------------------------------------------------------------------- empty batch
def test_empty_batch_through_every_op(dev, experts, router_w):
    """T = 0 is a valid batch: every op returns empty outputs and launches
    nothing, and the dispatch metadata says zero pairs (all counts 0, no
    tiles, no active experts, no error).  Torch hands the empty tensors over
    as address 0, which the library accepts for buffers of zero elements."""
    announce("empty batch T=0")
    w13, w2 = experts
    x0 = torch.empty(0, H, dtype=torch.bfloat16, device=dev)
    h0 = torch.empty(0, H, device=dev)
    nw = torch.ones(H, dtype=torch.bfloat16, device=dev)
    ti0 = torch.empty(0, K_TOP, dtype=torch.int32, device=dev)
    tw0 = torch.empty(0, K_TOP, device=dev)

    y = ops.rmsnorm_residual(h0, nw, 1e-6)
    assert y.shape == (0, H)
    logits, w, idx = ops.router_topk(x0, router_w, K_TOP)
    assert idx.shape == (0, K_TOP) and w.shape == (0, K_TOP) and logits.shape == (0, E)
    for tile_m in (128, 256):
        route = ops.moe_permute(ti0, E, tile_m)
        torch.cuda.synchronize()
        meta = route.meta.cpu()
        assert route.counts.cpu().eq(0).all() and route.offsets.cpu().eq(0).all()
        assert meta[:3].tolist() == [0, 0, 0]
        y_slot = ops.moe_experts_grouped(x0, w13, w2, route)
        assert y_slot.shape == (0, H)
        out = ops.moe_combine(y_slot, route, tw0)
        assert out.shape == (0, H)
        out, xn = ops.moe_combine(y_slot, route, tw0, residual=h0, out=h0, norm=(nw, 1e-6))
        assert out.shape == (0, H) and xn.shape == (0, H)
    route = ops.moe_route(x0, router_w, K_TOP, None, 256)
    torch.cuda.synchronize()
    assert route.meta.cpu()[:3].tolist() == [0, 0, 0]
    assert ops.moe_experts_gemv(x0, w13, w2, ops.moe_permute(ti0, E, 128)).shape == (0, H)
    assert ops.gemm(x0, router_w).shape == (0, E)
    assert ops.moe_decode_block(router_w, w13, w2, K_TOP, x=x0).shape == (0, H)
    assert MoEBlock(router_w, w13, w2, K_TOP)(x0).shape == (0, H)
    torch.cuda.synchronize()
