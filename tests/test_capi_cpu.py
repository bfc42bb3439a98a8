"""CPU-side checks of the C ABI: the library loads, exports every declared
entry point, and rejects bad arguments before launching anything.

No call here reaches a kernel launch: every call either fails host-side
validation inside the library (status QMOE_ERR_INVALID) or is rejected by the
Python wrapper (ValueError) before the library is called.
"""

import os
import re

import pytest
import torch

from conftest import ROOT

from qmoe import _lib, ops, weights

HEADER = os.path.join(ROOT, "include", "qmoe_capi.h")


def _declared_symbols():
    text = open(HEADER).read()
    decl = r"^(?:int|int64_t|const char\*)\s+(qmoe_[a-z0-9_]+)\("
    return sorted(set(re.findall(decl, text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_symbols()
    assert len(declared) >= 13
    for name in declared:
        assert hasattr(lib, name), f"libqmoe.so does not export {name}"
    assert set(declared) == set(_lib.PROTOTYPES), "ctypes prototypes out of sync with the header"


def test_header_constants_match_python_mirror():
    """Every numeric #define QMOE_X of the header that the Python side mirrors
    as _lib.X has the same value (buffer sizes such as the meta length)."""
    defs = dict(re.findall(r"^#define QMOE_(\w+) (\d+)", open(HEADER).read(), re.M))
    mirrored = {k: v for k, v in defs.items() if hasattr(_lib, k)}
    assert {"META_INTS", "GROUPED_MAX_TILE_M", "W2_BLOCK", "DECODE_BLOCK_WGS"} <= set(mirrored)
    for k, v in mirrored.items():
        assert getattr(_lib, k) == int(v), k


def test_version():
    assert _lib.lib().qmoe_version() == _lib.VERSION == 3


def test_route_meta_length_checked():
    """A dispatch meta shorter than QMOE_META_INTS is refused before any
    launch (the library writes and counts in all of its ints)."""
    import torch

    from qmoe import ops

    ops._need_meta(torch.zeros(_lib.META_INTS, dtype=torch.int32))
    with pytest.raises(ValueError, match="needs 24"):
        ops._need_meta(torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        ops._need_meta(torch.zeros(_lib.META_INTS, dtype=torch.int64))


@pytest.mark.parametrize(
    "call, msg",
    [
        (lambda l: l.qmoe_gemm(None, 64, None, 1, 128, 64, 0, None, 128, None), "null pointer"),
        (lambda l: l.qmoe_gemm(1, 64, 1, 1, 128, 64, 7, 1, 128, None), "bad mode"),
        (lambda l: l.qmoe_gemm(1, 104, 1, 40, 128, 100, 0, 1, 128, None), "K % 64"),
        (lambda l: l.qmoe_rmsnorm_residual(1, None, 1, 4, 6, 1e-6, None, 1, None), "multiple of 4"),
        (lambda l: l.qmoe_router_topk(1, 1, None, 1, 2048, 300, 8, 1, 1, 1, None), "E must be"),
        (lambda l: l.qmoe_router_topk(1, 1, None, 1, 2048, 128, 8, 1, 1, None, None), "null pointer"),
        (lambda l: l.qmoe_moe_permute(1, 4, 8, 128, 128, 10, 1, 1, 1, 1, 1, 1, 1, None), "max_tiles"),
        (lambda l: l.qmoe_moe_experts_gemv(1, 1, 1, 1, 1, 1, 1, 65, 2048, 768, 128, 8, 1, 1, None), "T must be"),
        (lambda l: l.qmoe_moe_experts_grouped(1, 1, 1, 1, 1, 1, 200, 4, 2048, 100, 128, 8, 1, 1, None), "I % 32"),
        (lambda l: l.qmoe_moe_experts_grouped(1, 1, 1, 1, 1, 1, 200, 4, 2176, 768, 128, 8, 1, 1, None), "H % 256"),
        (lambda l: l.qmoe_moe_combine(1, 0, 1, 1, None, 4, 8, 6, 1, None), "H % 4"),
        (lambda l: l.qmoe_embed(1, 100, 6, 1, 1, 1, 1, None), "H % 4 == 0"),
        (lambda l: l.qmoe_embed(None, 100, 8, 1, 1, 1, 1, None), "null pointer"),
        (lambda l: l.qmoe_argmax(1, 2, 100, 100, 1, 8, 1, None), "workspace too small"),
        (lambda l: l.qmoe_attn_decode_chunk(1, 1, 1, None, 1, 5, 32, 4, 128, 64, 0.1, 1, 1, None), "null pointer"),
        (lambda l: l.qmoe_attn_decode_chunk(1, 1, 1, 1, 1, 5, 32, 4, 128, 4, 0.1, 1, 1, None), "bad B/S/S_max"),
        (lambda l: l.qmoe_argmax(1, 2, 100, 50, 1, 1 << 20, 1, None), "bad rows/n/ldx"),
        # decode block: x, h, rms_w, eps, w_router, bias, w13, w2, residual, T, H, I, E, k,
        #   logits, topk_idx, topk_w, workspace, workspace_bytes, x_out, out, stream
        (lambda l: l.qmoe_moe_decode_block(1, None, None, 1e-6, 1, None, 1, 1, None, 1, 2048, 768, 128, 8,
                                           1, 1, 1, 1, 256 * 2048 * 4 - 4, None, 1, None), "workspace"),
        (lambda l: l.qmoe_moe_decode_block(1, None, None, 1e-6, 1, None, 1, 1, None, 9, 2048, 768, 128, 8,
                                           1, 1, 1, 1, 1 << 30, None, 1, None), "T must be"),
        (lambda l: l.qmoe_moe_decode_block(1, 1, None, 1e-6, 1, None, 1, 1, None, 1, 2048, 768, 128, 8,
                                           1, 1, 1, 1, 1 << 30, None, 1, None), "exactly one"),
        (lambda l: l.qmoe_moe_decode_block(1, None, None, 1e-6, 1, None, 1, 1, None, 1, 2048, 100, 128, 8,
                                           1, 1, 1, 1, 1 << 30, None, 1, None), "multiple of 32"),
        # allocation-free decode block: same arguments without workspace / workspace_bytes
        (lambda l: l.qmoe_moe_decode_block_noalloc(1, None, None, 1e-6, 1, None, 1, 1, None, 8, 4096, 768, 128, 8,
                                                   1, 1, 1, None, 1, None), "static scratch limit"),
        (lambda l: l.qmoe_moe_decode_block_noalloc(1, None, None, 1e-6, 1, None, 1, 1, None, 9, 1024, 768, 128, 8,
                                                   1, 1, 1, None, 1, None), "T must be"),
        (lambda l: l.qmoe_moe_decode_block_noalloc(1, None, None, 1e-6, None, None, 1, 1, None, 1, 2048, 768, 128, 8,
                                                   1, 1, 1, None, 1, None), "null pointer"),
        (lambda l: l.qmoe_qkv_norm_rope(1, 1, 1, 1, 1, 1, 10, 1, 1, 1, 2048, 32, 4, 64, 10, 1e-6, 1, 1, 1, 1, None), "head_dim"),
        (lambda l: l.qmoe_qkv_norm_rope(1, 1, 1, 1, 1, 1, 10, 1, 8, 1, 2048, 32, 4, 128, 10, 1e-6, 1, 1, 1, None, None),
         "needs the workspace"),
        (lambda l: l.qmoe_attn_prefill(1, 1, 1, 1, 10, 32, 4, 128, 8, 0, 0.1, 1, None), "S_max"),
        (lambda l: l.qmoe_attn_decode(1, 1, 1, 1, 1, 64, 2, 128, 16, 0.1, 1, 1, None), "Hq / Hkv <= 16"),
        (lambda l: l.qmoe_attn_decode_bucket(1, 1, 1, 1, 1, 32, 4, 128, 16, 32, 0.1, 1, 1, None), "max_ctx <= S_max"),
        (lambda l: l.qmoe_attn_prefill_at(1, 1, 1, 1, 8, 32, 4, 128, 4, 1, 0.1, 1, None), "S <= S_max"),
        (lambda l: l.qmoe_attn_prefill(1, 1, 1, 1, 10, 32, 4, 128, (1 << 22) + 1, 0, 0.1, 1, None),
         "S_max must be <="),
        (lambda l: l.qmoe_attn_prefill_at(1, 1, 1, 1, 8, 32, 4, 128, (1 << 22) + 1, 1, 0.1, 1, None),
         "S_max must be <="),
        (lambda l: l.qmoe_gemv_rmsnorm(1, 1, 1e-6, 1, 100, 1536, 0, 1, None), "K must be"),
        (lambda l: l.qmoe_qkv_finish(1, 1, 1, 1, 1, 10, 1, 4, 5, 32, 4, 128, 10, 1e-6, 1, 1, 1, None), "B*S <= 16"),
        # fused decode: qkv, q_norm_w, k_norm_w, cos, sin, max_pos, positions, B, Hq, Hkv, D, S_max, max_ctx,
        #   eps, scale, k_cache, v_cache, partial, out, stream
        (lambda l: l.qmoe_attn_decode_fused(1, 1, 1, 1, 1, 10, 1, 1, 32, 4, 64, 16, 16, 1e-6, 0.1, 1, 1, 1, 1, None),
         "head_dim"),
        (lambda l: l.qmoe_attn_decode_fused(1, 1, 1, 1, 1, 10, 1, 1, 32, 4, 128, 16, 32, 1e-6, 0.1, 1, 1, 1, 1, None),
         "max_ctx <= S_max"),
        (lambda l: l.qmoe_attn_decode_fused(1, 1, 1, 1, 1, 10, 1, 1, 64, 2, 128, 16, 16, 1e-6, 0.1, 1, 1, 1, 1, None),
         "Hq / Hkv <= 16"),
        (lambda l: l.qmoe_attn_decode_fused(None, 1, 1, 1, 1, 10, 1, 1, 32, 4, 128, 16, 16, 1e-6, 0.1, 1, 1, 1, 1,
                                            None), "null pointer"),
    ],
)
def test_invalid_arguments_rejected_before_launch(call, msg):
    # The pointers here are dummies: never let a case reach a real device.
    if torch.cuda.is_available():
        pytest.skip("host-side validation test; runs only where no GPU is visible")
    rc = call(_lib.lib())
    assert rc == _lib.QMOE_ERR_INVALID
    assert msg in _lib.last_error()


@pytest.mark.parametrize(
    "call",
    [
        # rows = 0: x, delta, h_out and y_out NULL; the norm weight still given
        lambda l: l.qmoe_rmsnorm_residual(None, None, 1, 0, 2048, 1e-6, None, None, None),
        lambda l: l.qmoe_router_topk(None, 1, None, 0, 2048, 128, 8, None, None, None, None),
        lambda l: l.qmoe_moe_combine(None, 1, None, None, None, 0, 8, 2048, None, None),
        lambda l: l.qmoe_moe_combine_norm(None, 1, None, None, None, 0, 8, 2048, None, 1, 1e-6, None, None),
        lambda l: l.qmoe_moe_experts_grouped(None, 1, 1, None, 1, 1, 128, 0, 2048, 768, 128, 8, None, None, None),
        lambda l: l.qmoe_moe_experts_gemv(None, 1, 1, 1, None, 1, 1, 0, 2048, 768, 128, 8, None, None, None),
        lambda l: l.qmoe_gemm(None, 2048, 1, 0, 128, 2048, 0, None, 128, None),
        lambda l: l.qmoe_gemm_ws_add_rmsnorm(None, 4096, 1, 0, 2048, 4096, None, 1, 1e-6, None, None, 0, None),
        lambda l: l.qmoe_qkv_norm_rope(None, 1, 1, 1, 1, 1, 10, None, 0, 1, 2048, 32, 4, 128, 10, 1e-6,
                                       None, 1, 1, None, None),
        lambda l: l.qmoe_attn_prefill(None, 1, 1, 0, 10, 32, 4, 128, 16, 0, 0.1, None, None),
        lambda l: l.qmoe_attn_prefill_at(None, 1, 1, 0, 10, 32, 4, 128, 16, None, 0.1, None, None),
        lambda l: l.qmoe_attn_decode(None, 1, 1, None, 0, 32, 4, 128, 16, 0.1, None, None, None),
        lambda l: l.qmoe_argmax(None, 0, 100, 100, None, 0, None, None),
        lambda l: l.qmoe_embed(1, 100, 8, None, 0, None, 1, None),
        lambda l: l.qmoe_moe_decode_block(None, None, None, 1e-6, 1, None, 1, 1, None, 0, 2048, 768, 128, 8,
                                          None, None, None, 1, 1 << 20, None, None, None),
    ],
)
def test_empty_batch_accepts_null_row_buffers(call):
    """A zero-row call launches nothing and returns 0, and the buffers sized
    by the row count may be NULL (torch hands an empty tensor over as
    address 0).  These calls return before any HIP call."""
    if torch.cuda.is_available():
        pytest.skip("host-side validation test; runs only where no GPU is visible")
    rc = call(_lib.lib())
    assert rc == _lib.QMOE_OK, _lib.last_error()


def test_empty_batch_still_requires_weights():
    """Weights are not sized by the batch: NULL stays an error at T = 0."""
    if torch.cuda.is_available():
        pytest.skip("host-side validation test; runs only where no GPU is visible")
    l = _lib.lib()
    assert l.qmoe_rmsnorm_residual(None, None, None, 0, 2048, 1e-6, None, None, None) == _lib.QMOE_ERR_INVALID
    assert "null pointer" in _lib.last_error()
    assert l.qmoe_moe_experts_grouped(None, None, 1, None, 1, 1, 128, 0, 2048, 768, 128, 8, None, None,
                                      None) == _lib.QMOE_ERR_INVALID
    assert l.qmoe_gemm(None, 2048, None, 0, 128, 2048, 0, None, 128, None) == _lib.QMOE_ERR_INVALID


def test_python_wrappers_reject_host_tensors():
    a = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.gemm(a, a)
    with pytest.raises(ValueError, match="GPU"):
        ops.rmsnorm_residual(torch.zeros(2, 8), torch.zeros(8, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="GPU|dtype"):
        ops.router_topk(torch.zeros(2, 8), torch.zeros(4, 8, dtype=torch.bfloat16), 2)


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.QMOE_ERR_INVALID, "x")
    with pytest.raises(_lib.QmoeError):
        _lib.check(_lib.QMOE_ERR_HIP, "x")
    _lib.check(_lib.QMOE_OK, "x")


def test_decode_block_workspace_size():
    lib = _lib.lib()
    st = _lib.DECODE_BLOCK_STATE_BYTES
    assert lib.qmoe_moe_decode_block_workspace(1, 2048) == st + _lib.DECODE_BLOCK_WGS * 2048 * 4
    assert lib.qmoe_moe_decode_block_workspace(8, 512) == st + _lib.DECODE_BLOCK_WGS * 8 * 512 * 4
    assert lib.qmoe_moe_decode_block_workspace(0, 2048) == st
    assert lib.qmoe_moe_decode_block_workspace(-1, 2048) == -1


def test_router_workspace_size():
    """Split-K router workspace: f32 [slices][T][E], slices from the split-K
    plan of the T x E x H logits GEMM (128 x 128 tiles once there are 16 of
    them, else 64 x 64; slices double while the grid stays within 512
    workgroups and each slice keeps >= 512 / 256 columns of H), none at
    T <= 16 or T > 1024, and never more than 16 slices."""
    l = _lib.lib()
    assert l.qmoe_router_workspace(8, 2048, 128) == 0  # GEMV path
    assert l.qmoe_router_workspace(64, 2048, 128) == 8 * 64 * 128 * 4  # 2 tiles x 8 slices
    assert l.qmoe_router_workspace(640, 2048, 128) == 8 * 640 * 128 * 4  # 20 tiles x 8
    assert l.qmoe_router_workspace(1024, 2048, 128) == 8 * 1024 * 128 * 4  # 32 tiles of 64 x 64 x 8
    assert l.qmoe_router_workspace(1025, 2048, 128) == 0  # unsplit above 1024 tokens
    assert l.qmoe_router_workspace(4096, 2048, 128) == 0
    assert l.qmoe_router_workspace(1000, 4096, 128) == 16 * 1000 * 128 * 4  # 32 tiles x 16
    assert l.qmoe_router_workspace(100, 192, 128) == 0  # K too short to split
    assert l.qmoe_router_workspace(-1, 2048, 128) == -1


def test_gemm_splitk_workspace_size():
    """Split-K workspace of qmoe_gemm_ws, f32 [slices][M][N]: 64 x 128 tiles
    when 40-127 tiles of 128 x 128 would cover the output (640 x 2048: 160
    tiles x 2 slices; 384 x 2048: 96 x 4), 128 x 128 from 16 such tiles
    otherwise (1024 x 2048: 128 x 4; 256 x 2048: 32 x 8), none from 256."""
    l = _lib.lib()
    assert l.qmoe_gemm_ws_workspace(640, 2048, 4096) == 2 * 640 * 2048 * 4
    assert l.qmoe_gemm_ws_workspace(384, 2048, 4096) == 4 * 384 * 2048 * 4
    assert l.qmoe_gemm_ws_workspace(1024, 2048, 4096) == 4 * 1024 * 2048 * 4
    assert l.qmoe_gemm_ws_workspace(256, 2048, 4096) == 8 * 256 * 2048 * 4
    assert l.qmoe_gemm_ws_workspace(4096, 2048, 4096) == 0
    assert l.qmoe_gemm_ws_workspace(-1, 2048, 4096) == -1


def test_permute_tiles_rows():
    """Rows of `tiles` for the per-chunk permutation: the tile-table bound
    ceil(T*k/tile_m) + E, then (E + 1) ints of scratch per 1024-pair chunk
    where that path runs (4096 < T*k <= 4096 chunks of 1024)."""
    l = _lib.lib()
    assert l.qmoe_moe_permute_tiles(4096, 8, 128, 256) == 128 + 128 + (32 * 129 + 3) // 4
    assert l.qmoe_moe_permute_tiles(513, 8, 128, 128) == 33 + 128 + (5 * 129 + 3) // 4
    assert l.qmoe_moe_permute_tiles(0, 8, 128, 128) == 128
    assert l.qmoe_moe_permute_tiles(512, 8, 128, 128) == 32 + 128  # one workgroup: no scratch
    assert l.qmoe_moe_permute_tiles(1 << 20, 8, 128, 256) == (1 << 15) + 128  # beyond 4096 chunks
    assert l.qmoe_moe_permute_tiles(4, 8, 128, 0) == -1


def test_blocked_down_layout():
    """w2[e, b, h, j] = down[e, 8b + j, h] (NxDI (E, I, H)) = W2[e, h, 8b + j];
    both conversions invert, and the HF path lands on the same bytes."""
    g = torch.Generator().manual_seed(3)
    E, I, H = 3, 40, 24
    down = torch.randn(E, I, H, generator=g)  # NxDI (E, I, H)
    b = weights.pack_down(down)
    assert tuple(b.shape) == (E, I // 8, H, 8)
    for e, blk, h, j in [(0, 0, 0, 0), (1, 2, 5, 7), (2, 4, 23, 3), (0, 3, 11, 1)]:
        assert b[e, blk, h, j] == down[e, 8 * blk + j, h]
    assert torch.equal(weights.unpack_down(b), down)
    w_ehi = down.transpose(1, 2).contiguous()  # (E, H, I)
    assert torch.equal(weights.block_down(w_ehi), b)
    assert torch.equal(weights.unblock_down(b), w_ehi)
    # one 8-unit slice of one expert is a contiguous H x 8 run
    flat = b.reshape(-1)
    s = 2
    assert torch.equal(flat[(1 * (I // 8) + s) * H * 8 : (1 * (I // 8) + s + 1) * H * 8].view(H, 8),
                       down[1, 8 * s : 8 * s + 8, :].t())
    with pytest.raises(ValueError):
        weights.block_down(torch.zeros(1, 4, 12))


def test_pack_gate_up_roundtrip_and_layout():
    import oracle

    g = torch.Generator().manual_seed(0)
    gu = torch.randn(3, 64, 2 * 96, generator=g)
    p = weights.pack_gate_up(gu)
    assert torch.equal(p, oracle.pack_w13(gu, 32))
    assert torch.equal(weights.unpack_gate_up(p), gu)
    # packed row 64j + 32 + r is the up row of unit 32j + r
    assert torch.equal(p[:, 64 + 32 + 5], gu.transpose(1, 2)[:, 96 + 32 + 5])


def test_from_hf_experts_matches_reference_conversion():
    # convert_qwen3_moe_hf_to_neuron_state_dict (qwen_with_nki.py:8928-8990):
    # gate_up[e] = cat(gate_proj.T, up_proj.T, dim=1); down[e] = down_proj.T
    g = torch.Generator().manual_seed(1)
    E, H, I = 2, 16, 64
    gp = [torch.randn(I, H, generator=g) for _ in range(E)]
    up = [torch.randn(I, H, generator=g) for _ in range(E)]
    dp = [torch.randn(H, I, generator=g) for _ in range(E)]
    w13, w2 = weights.from_hf_experts(gp, up, dp)
    nxdi_gu = torch.stack([torch.cat([gp[e].t(), up[e].t()], dim=1) for e in range(E)])
    nxdi_dn = torch.stack([dp[e].t() for e in range(E)])
    assert torch.equal(weights.unpack_gate_up(w13), nxdi_gu)
    assert torch.equal(w2, weights.pack_down(nxdi_dn))
