"""The allocation-free decode MoE block (qmoe_moe_decode_block_noalloc).

Called through the C ABI with ctypes and checked against the workspace entry
point qmoe_moe_decode_block on the same inputs: calls in a row on one GPU,
each later one with fewer tokens than the first, so they read a static
scratch array that still holds the first call's partials.  At I = 768 the
T = 1 calls take the single-launch path, whose call counters and exchange
slots live in the same static array (two T = 1 calls in a row).  Both entry points
run the same kernels in the same fixed summation order, so the bar is
bit-equality of the block output, the router logits, the top-k ids and the
top-k weights.
"""

import ctypes

import pytest
import torch

from gpu_util import announce, bf16_randn

from qmoe import _lib, ops

pytestmark = pytest.mark.gpu

H, E, K_TOP = 2048, 128, 8


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _noalloc(w_router, w13, w2, x, h, rms_w, residual, T):
    dev = w13.device
    I = w13.shape[1] // 2
    logits = torch.full((T, E), float("nan"), device=dev)
    idx = torch.full((T, K_TOP), -1, dtype=torch.int32, device=dev)
    w = torch.full((T, K_TOP), float("nan"), device=dev)
    x_out = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    out = torch.full((T, H), float("nan"), device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = _lib.lib().qmoe_moe_decode_block_noalloc(
        _ptr(x), _ptr(h), _ptr(rms_w), 1e-6, _ptr(w_router), None, _ptr(w13), _ptr(w2), _ptr(residual),
        T, H, I, E, K_TOP, _ptr(logits), _ptr(idx), _ptr(w), _ptr(x_out), _ptr(out), stream)
    _lib.check(rc, "qmoe_moe_decode_block_noalloc")
    return out, logits, idx, w, x_out


@pytest.mark.parametrize("I, Ts", [(256, (8, 3)), (768, (8, 1, 1))])
@pytest.mark.parametrize("normed", [False, True])
def test_noalloc_decode_block_matches_workspace_entry(dev, normed, I, Ts):
    g = torch.Generator(device=dev).manual_seed(4242 + int(normed) + I)
    w_router = bf16_randn((E, H), g, dev, 0.02)
    w13 = bf16_randn((E, 2 * I, H), g, dev, 0.02)
    w2 = bf16_randn((E, I // 8, H, 8), g, dev, 0.02)
    rms_w = (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    for T in Ts:  # the later calls are smaller than the first
        announce(f"noalloc decode block T={T} I={I} normed={normed}")
        h = torch.randn(T, H, generator=g, device=dev)
        residual = torch.randn(T, H, generator=g, device=dev)
        if normed:
            x, hh, rw = None, h, rms_w
        else:
            x, hh, rw = h.to(torch.bfloat16), None, None
        got, logits, idx, w, x_out = _noalloc(w_router, w13, w2, x, hh, rw, residual, T)
        bufs = ops.DecodeBlockBuffers.alloc(T, H, I, E, K_TOP, dev)
        ref = ops.moe_decode_block(w_router, w13, w2, K_TOP, x=x, h=hh, rms_w=rw, eps=1e-6,
                                   residual=residual, bufs=bufs)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), float((got - ref).abs().max())
        assert torch.equal(logits, bufs.logits)
        assert torch.equal(idx, bufs.topk_idx)
        assert torch.equal(w, bufs.topk_w)
        if normed:
            assert torch.equal(x_out, bufs.x_out)


def test_noalloc_decode_block_rejects_oversize(dev):
    announce("noalloc decode block size limit")
    T, Hb = 8, 4096  # T * H = 32768 > 16384: rejected before any launch
    z = torch.zeros(1, dtype=torch.bfloat16, device=dev)
    zf = torch.zeros(1, device=dev)
    zi = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = _lib.lib().qmoe_moe_decode_block_noalloc(
        _ptr(z), None, None, 1e-6, _ptr(z), None, _ptr(z), _ptr(z), None, T, Hb, 768, 128, 8,
        _ptr(zf), _ptr(zi), _ptr(zf), None, _ptr(zf), None)
    assert rc == _lib.QMOE_ERR_INVALID
    assert "static scratch limit" in _lib.last_error()
