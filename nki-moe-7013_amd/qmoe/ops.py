"""Validated torch-facing wrappers over the libqmoe C ABI.

Every wrapper checks device, dtype, contiguity and shape on the host and
raises ``ValueError`` before anything is launched; outputs and workspaces are
allocated here with torch (the library itself never allocates).  Work is
enqueued on torch's current HIP stream and never synchronises the host, so
every call can be captured into a ``torch.cuda.CUDAGraph``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, lib

BF16 = torch.bfloat16
F32 = torch.float32
I32 = torch.int32


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need(t: torch.Tensor, name: str, dtype, shape=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name}: expected a tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be on a GPU (got {t.device})")
    if t.dtype != dtype:
        raise ValueError(f"{name}: dtype must be {dtype} (got {t.dtype})")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape must be {tuple(shape)} (got {tuple(t.shape)})")


def _same_device(*ts) -> None:
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise ValueError(f"tensors are on different devices: {devs}")


# ----------------------------------------------------------------- RMSNorm
def rmsnorm_residual(
    x: torch.Tensor,
    w: torch.Tensor,
    eps: float,
    delta: Optional[torch.Tensor] = None,
    h_out: Optional[torch.Tensor] = None,
    y_out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``h = x (+ delta)`` (into ``h_out`` if given, may be ``x``); returns
    ``y = bf16(w * h * rsqrt(mean(h^2) + eps))``."""
    if x.dim() != 2:
        raise ValueError("x must be [rows, H]")
    R, H = x.shape
    _need(x, "x", F32)
    _need(w, "w", BF16, (H,))
    if delta is not None:
        _need(delta, "delta", F32, (R, H))
    if h_out is not None:
        _need(h_out, "h_out", F32, (R, H))
    if y_out is None:
        y_out = torch.empty(R, H, dtype=BF16, device=x.device)
    _need(y_out, "y_out", BF16, (R, H))
    _same_device(x, w, delta, h_out, y_out)
    check(
        lib().qmoe_rmsnorm_residual(
            _ptr(x), _ptr(delta), _ptr(w), R, H, float(eps), _ptr(h_out), _ptr(y_out), _stream()
        ),
        "qmoe_rmsnorm_residual",
    )
    return y_out


# ----------------------------------------------------------------- router
def router_topk(
    x: torch.Tensor, w_router: torch.Tensor, k: int, bias: Optional[torch.Tensor] = None,
    logits: Optional[torch.Tensor] = None, topk_idx: Optional[torch.Tensor] = None,
    topk_w: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Returns ``(logits[T,E] f32, topk_w[T,k] f32, topk_idx[T,k] i32)``."""
    T, H = x.shape
    E = w_router.shape[0]
    _need(x, "x", BF16)
    _need(w_router, "w_router", BF16, (E, H))
    if bias is not None:
        _need(bias, "bias", F32, (E,))
    dev = x.device
    logits = torch.empty(T, E, dtype=F32, device=dev) if logits is None else logits
    topk_idx = torch.empty(T, k, dtype=I32, device=dev) if topk_idx is None else topk_idx
    topk_w = torch.empty(T, k, dtype=F32, device=dev) if topk_w is None else topk_w
    _need(logits, "logits", F32, (T, E))
    _need(topk_idx, "topk_idx", I32, (T, k))
    _need(topk_w, "topk_w", F32, (T, k))
    _same_device(x, w_router, bias, logits, topk_idx, topk_w)
    ws = _router_workspace(T, H, E, dev)
    check(
        lib().qmoe_router_topk_ws(
            _ptr(x), _ptr(w_router), _ptr(bias), T, H, E, k, _ptr(topk_idx), _ptr(topk_w),
            _ptr(logits), _ptr(ws), _nbytes(ws), _stream(),
        ),
        "qmoe_router_topk_ws",
    )
    return logits, topk_w, topk_idx


def _router_workspace(T: int, H: int, E: int, dev) -> Optional[torch.Tensor]:
    """Split-K workspace of the router logits GEMM (None when T does not split)."""
    n = int(lib().qmoe_router_workspace(T, H, E))
    return torch.empty(max(n, 0) // 4, dtype=F32, device=dev) if n > 0 else None


def _nbytes(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.numel() * t.element_size()


# ----------------------------------------------------------------- dispatch
@dataclass
class Route:
    """Device-side dispatch metadata produced by :func:`moe_permute`."""

    T: int
    k: int
    E: int
    tile_m: int
    max_tiles: int
    counts: torch.Tensor  # [E]
    offsets: torch.Tensor  # [E+1]
    slot_token: torch.Tensor  # [T*k]
    token_slot: torch.Tensor  # [T*k]
    active: torch.Tensor  # [E]
    tiles: torch.Tensor  # [rows >= max_tiles, 4]: the tile table, then permutation scratch
    meta: torch.Tensor  # [META_INTS] = (n_tiles, n_active, error flag, unused, grouped GEMM work counters)
    logits: Optional[torch.Tensor] = None  # [T, E] f32 (filled by moe_route)
    topk_idx: Optional[torch.Tensor] = None  # [T, k] i32
    topk_w: Optional[torch.Tensor] = None  # [T, k] f32
    router_ws: Optional[torch.Tensor] = None  # split-K partials of the router logits (T > 16)

    @staticmethod
    def alloc(T: int, k: int, E: int, tile_m: int, device, with_topk: bool = False) -> "Route":
        max_tiles = -(-T * k // tile_m) + E  # bound on the number of tiles
        rows = int(lib().qmoe_moe_permute_tiles(T, k, E, tile_m))
        z = lambda *s: torch.empty(*s, dtype=I32, device=device)
        r = Route(T, k, E, tile_m, max_tiles, z(E), z(E + 1), z(T * k), z(T * k), z(E),
                  z(max(rows, max_tiles), 4), z(_lib.META_INTS))
        if with_topk:
            r.logits = torch.empty(T, E, dtype=F32, device=device)
            r.topk_idx = z(T, k)
            r.topk_w = torch.empty(T, k, dtype=F32, device=device)
        return r

    def ensure_router_ws(self, H: int, device) -> None:
        """Allocate the router's split-K workspace for hidden size H (once)."""
        need = int(lib().qmoe_router_workspace(self.T, H, self.E))
        if need > 0 and (self.router_ws is None or _nbytes(self.router_ws) < need):
            self.router_ws = torch.empty(need // 4, dtype=F32, device=device)


def _need_meta(meta: torch.Tensor) -> None:
    """The dispatch ``meta`` array must hold QMOE_META_INTS i32 (the library
    writes and counts in all of them: a shorter array would be overrun)."""
    if not isinstance(meta, torch.Tensor) or meta.dtype != I32 or not meta.is_contiguous():
        raise ValueError("route.meta: expected a contiguous int32 tensor")
    if meta.numel() < _lib.META_INTS:
        raise ValueError(f"route.meta: needs {_lib.META_INTS} int32 (got {meta.numel()})")


def moe_permute(topk_idx: torch.Tensor, E: int, tile_m: int = 128, route: Optional[Route] = None) -> Route:
    T, k = topk_idx.shape
    _need(topk_idx, "topk_idx", I32)
    if route is None:
        route = Route.alloc(T, k, E, tile_m, topk_idx.device)
    if (route.T, route.k, route.E, route.tile_m) != (T, k, E, tile_m):
        raise ValueError("route buffers were allocated for a different shape")
    _need_meta(route.meta)
    check(
        lib().qmoe_moe_permute(
            _ptr(topk_idx), T, k, E, tile_m, route.tiles.shape[0], _ptr(route.counts), _ptr(route.offsets),
            _ptr(route.slot_token), _ptr(route.token_slot), _ptr(route.active), _ptr(route.tiles),
            _ptr(route.meta), _stream(),
        ),
        "qmoe_moe_permute",
    )
    return route


def moe_route(x: torch.Tensor, w_router: torch.Tensor, k: int, bias: Optional[torch.Tensor] = None,
              tile_m: int = 128, route: Optional[Route] = None) -> Route:
    """Router + top-k + dispatch metadata (qmoe_moe_route_ws)."""
    T, H = x.shape
    E = w_router.shape[0]
    _need(x, "x", BF16)
    _need(w_router, "w_router", BF16, (E, H))
    if bias is not None:
        _need(bias, "bias", F32, (E,))
    if route is None:
        route = Route.alloc(T, k, E, tile_m, x.device, with_topk=True)
    if (route.T, route.k, route.E, route.tile_m) != (T, k, E, tile_m) or route.topk_idx is None:
        raise ValueError("route buffers were allocated for a different shape / without top-k buffers")
    _need_meta(route.meta)
    _same_device(x, w_router, bias, route.meta)
    route.ensure_router_ws(H, x.device)
    check(
        lib().qmoe_moe_route_ws(
            _ptr(x), _ptr(w_router), _ptr(bias), T, H, E, k, tile_m, route.tiles.shape[0], _ptr(route.logits),
            _ptr(route.topk_idx), _ptr(route.topk_w), _ptr(route.counts), _ptr(route.offsets),
            _ptr(route.slot_token), _ptr(route.token_slot), _ptr(route.active), _ptr(route.tiles),
            _ptr(route.meta), _ptr(route.router_ws), _nbytes(route.router_ws), _stream(),
        ),
        "qmoe_moe_route_ws",
    )
    return route


# ----------------------------------------------------------------- experts
def _check_experts(x, w13, w2):
    T, H = x.shape
    E, I2, H2 = w13.shape
    _need(x, "x", BF16)
    _need(w13, "w13", BF16)
    if H2 != H or I2 % 2:
        raise ValueError(f"w13 must be [E, 2I, H={H}] (got {tuple(w13.shape)})")
    I = I2 // 2
    _need_w2(w2, E, H, I)
    return T, H, I, E


def _need_w2(w2, E, H, I):
    if I % _lib.W2_BLOCK:
        raise ValueError(f"moe intermediate size {I} is not a multiple of {_lib.W2_BLOCK}")
    _need(w2, "w2 (blocked [E, I/8, H, 8])", BF16, (E, I // _lib.W2_BLOCK, H, _lib.W2_BLOCK))


def moe_experts_gemv(
    x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, route: Route,
    act: Optional[torch.Tensor] = None, y_slot: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Decode-shape experts; returns unweighted ``y_slot[T*k, H]`` (f32)."""
    T, H, I, E = _check_experts(x, w13, w2)
    if (route.T, route.E) != (T, E):
        raise ValueError("route does not match x / w13")
    _need_meta(route.meta)
    k = route.k
    dev = x.device
    act = torch.empty(T * k, I, dtype=F32, device=dev) if act is None else act
    y_slot = torch.empty(T * k, H, dtype=F32, device=dev) if y_slot is None else y_slot
    _need(act, "act", F32, (T * k, I))
    _need(y_slot, "y_slot", F32, (T * k, H))
    _same_device(x, w13, w2, route.offsets, act, y_slot)
    check(
        lib().qmoe_moe_experts_gemv(
            _ptr(x), _ptr(w13), _ptr(w2), _ptr(route.offsets), _ptr(route.slot_token),
            _ptr(route.active), _ptr(route.meta), T, H, I, E, k, _ptr(act), _ptr(y_slot), _stream(),
        ),
        "qmoe_moe_experts_gemv",
    )
    return y_slot


@dataclass
class DecodeBlockBuffers:
    """Outputs / workspace of :func:`moe_decode_block` (allocate once, reuse)."""

    logits: torch.Tensor  # [T, E] f32
    topk_idx: torch.Tensor  # [T, k] i32
    topk_w: torch.Tensor  # [T, k] f32
    workspace: torch.Tensor  # u8, qmoe_moe_decode_block_workspace(T, H) bytes
    x_out: torch.Tensor  # [T, H] bf16 (normalised input, when h is given)

    @staticmethod
    def alloc(T: int, H: int, I: int, E: int, k: int, device) -> "DecodeBlockBuffers":
        nbytes = int(lib().qmoe_moe_decode_block_workspace(T, H))
        return DecodeBlockBuffers(
            torch.empty(T, E, dtype=F32, device=device), torch.empty(T, k, dtype=I32, device=device),
            torch.empty(T, k, dtype=F32, device=device),
            torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device),
            torch.empty(T, H, dtype=BF16, device=device))


DECODE_BLOCK_MAX_T = 8


def moe_decode_block(
    w_router: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, k: int, *,
    x: Optional[torch.Tensor] = None, h: Optional[torch.Tensor] = None,
    rms_w: Optional[torch.Tensor] = None, eps: float = 1e-6, bias: Optional[torch.Tensor] = None,
    residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
    bufs: Optional[DecodeBlockBuffers] = None,
) -> torch.Tensor:
    """Whole decode MoE block (T <= 8): one launch at T = 1 and the
    Qwen3-30B-A3B shape, else three (router logits; top-k + fused
    gate/up/down work items with per-workgroup partial outputs; fixed-order
    reduction + residual):
    ``out = residual + MoE(x)`` with ``x`` given, or ``x = rmsnorm(h) * rms_w``.
    ``bufs.workspace`` carries state between calls (allocate it once, with
    :meth:`DecodeBlockBuffers.alloc`, which zeroes it)."""
    if (x is None) == (h is None):
        raise ValueError("pass exactly one of x (bf16) and h (f32)")
    src = x if x is not None else h
    T, H = src.shape
    E = w_router.shape[0]
    if x is not None:
        _need(x, "x", BF16)
    else:
        _need(h, "h", F32)
        if rms_w is None:
            raise ValueError("h needs rms_w")
        _need(rms_w, "rms_w", BF16, (H,))
    _need(w_router, "w_router", BF16, (E, H))
    _need(w13, "w13", BF16)
    if w13.shape[0] != E or w13.shape[2] != H:
        raise ValueError("w13 must be [E, 2I, H]")
    I = w13.shape[1] // 2
    _need_w2(w2, E, H, I)
    if bias is not None:
        _need(bias, "bias", F32, (E,))
    if residual is not None:
        _need(residual, "residual", F32, (T, H))
    dev = src.device
    bufs = DecodeBlockBuffers.alloc(T, H, I, E, k, dev) if bufs is None else bufs
    _need(bufs.logits, "logits", F32, (T, E))
    _need(bufs.topk_idx, "topk_idx", I32, (T, k))
    _need(bufs.topk_w, "topk_w", F32, (T, k))
    _need(bufs.workspace, "workspace", torch.uint8)
    _need(bufs.x_out, "x_out", BF16, (T, H))
    out = torch.empty(T, H, dtype=F32, device=dev) if out is None else out
    _need(out, "out", F32, (T, H))
    _same_device(src, w_router, w13, w2, bias, residual, out, bufs.workspace)
    check(
        lib().qmoe_moe_decode_block(
            _ptr(x), _ptr(h), _ptr(rms_w), float(eps), _ptr(w_router), _ptr(bias), _ptr(w13), _ptr(w2),
            _ptr(residual), T, H, I, E, k, _ptr(bufs.logits), _ptr(bufs.topk_idx), _ptr(bufs.topk_w),
            _ptr(bufs.workspace), bufs.workspace.numel(), _ptr(bufs.x_out), _ptr(out), _stream(),
        ),
        "qmoe_moe_decode_block",
    )
    return out


def moe_experts_grouped(
    x: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, route: Route,
    act: Optional[torch.Tensor] = None, y_slot: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Prefill-shape experts (MFMA); returns unweighted ``y_slot[T*k, H]`` (bf16)."""
    T, H, I, E = _check_experts(x, w13, w2)
    if (route.T, route.E) != (T, E) or not 0 < route.tile_m <= _lib.GROUPED_MAX_TILE_M:
        raise ValueError(f"route must match x / w13 and use tile_m <= {_lib.GROUPED_MAX_TILE_M}")
    _need_meta(route.meta)
    k = route.k
    dev = x.device
    act = torch.empty(T * k, I, dtype=BF16, device=dev) if act is None else act
    y_slot = torch.empty(T * k, H, dtype=BF16, device=dev) if y_slot is None else y_slot
    _need(act, "act", BF16, (T * k, I))
    _need(y_slot, "y_slot", BF16, (T * k, H))
    _same_device(x, w13, w2, route.tiles, act, y_slot)
    check(
        lib().qmoe_moe_experts_grouped(
            _ptr(x), _ptr(w13), _ptr(w2), _ptr(route.slot_token), _ptr(route.tiles), _ptr(route.meta),
            route.max_tiles, T, H, I, E, k, _ptr(act), _ptr(y_slot), _stream(),
        ),
        "qmoe_moe_experts_grouped",
    )
    return y_slot


def moe_combine(
    y_slot: torch.Tensor, route: Route, topk_w: torch.Tensor,
    residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
    norm: Optional[tuple] = None,
):
    """``out[t] = residual[t] + sum_j topk_w[t,j] * y_slot[token_slot[t*k+j]]`` (f32).
    ``norm = (rms_w, eps)``: also the RMSNorm of every ``out`` row (the bits
    of :func:`rmsnorm_residual` on ``out``), in the same launch; returns
    ``(out, x)`` with ``x`` bf16 ``[T, H]``."""
    T, k = route.T, route.k
    if y_slot.dim() != 2 or y_slot.shape[0] != T * k:
        raise ValueError("y_slot must be [T*k, H]")
    H = y_slot.shape[1]
    if y_slot.dtype not in (F32, BF16):
        raise ValueError("y_slot must be float32 or bfloat16")
    _need(y_slot, "y_slot", y_slot.dtype)
    _need(topk_w, "topk_w", F32, (T, k))
    if residual is not None:
        _need(residual, "residual", F32, (T, H))
    out = torch.empty(T, H, dtype=F32, device=y_slot.device) if out is None else out
    _need(out, "out", F32, (T, H))
    _same_device(y_slot, topk_w, residual, out, route.token_slot)
    if norm is not None:
        rms_w, eps = norm
        _need(rms_w, "rms_w", BF16, (H,))
        x = torch.empty(T, H, dtype=BF16, device=y_slot.device)
        _same_device(out, rms_w)
        check(
            lib().qmoe_moe_combine_norm(
                _ptr(y_slot), int(y_slot.dtype == BF16), _ptr(route.token_slot), _ptr(topk_w),
                _ptr(residual), T, k, H, _ptr(out), _ptr(rms_w), float(eps), _ptr(x), _stream(),
            ),
            "qmoe_moe_combine_norm",
        )
        return out, x
    check(
        lib().qmoe_moe_combine(
            _ptr(y_slot), int(y_slot.dtype == BF16), _ptr(route.token_slot), _ptr(topk_w),
            _ptr(residual), T, k, H, _ptr(out), _stream(),
        ),
        "qmoe_moe_combine",
    )
    return out


# ----------------------------------------------------------------- GEMM
def gemm_workspace(M: int, N: int, K: int, device) -> Optional[torch.Tensor]:
    """Workspace for :func:`gemm` with split-K (``None`` when the shape is
    not split: it already fills the GPU)."""
    n = int(lib().qmoe_gemm_ws_workspace(M, N, K))
    if n < 0:
        raise ValueError("negative GEMM size")
    return torch.empty(max(n // 4, 1), dtype=F32, device=device) if n > 0 else None


def gemm(A: torch.Tensor, B: torch.Tensor, mode: int = _lib.GEMM_STORE_BF16,
         out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``A[M,K] . B[N,K]^T`` with epilogue ``mode`` (store bf16 / store f32 / add f32).
    With ``workspace`` (from :func:`gemm_workspace`) a problem with few output
    tiles splits K over more workgroups (fixed-order, deterministic sum)."""
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise ValueError("A must be [M,K] and B [N,K]")
    M, K = A.shape
    N = B.shape[0]
    _need(A, "A", BF16)
    _need(B, "B", BF16)
    if out is None:
        if mode == _lib.GEMM_ADD_F32:
            raise ValueError("mode ADD_F32 needs out")
        out = torch.empty(M, N, dtype=BF16 if mode == _lib.GEMM_STORE_BF16 else F32, device=A.device)
    _need(out, "out", BF16 if mode == _lib.GEMM_STORE_BF16 else F32, (M, N))
    _same_device(A, B, out)
    if workspace is not None:
        _need(workspace, "workspace", F32)
        _same_device(A, workspace)
        check(lib().qmoe_gemm_ws(_ptr(A), K, _ptr(B), M, N, K, int(mode), _ptr(out), N, _ptr(workspace),
                                 workspace.numel() * 4, _stream()), "qmoe_gemm_ws")
        return out
    check(lib().qmoe_gemm(_ptr(A), K, _ptr(B), M, N, K, int(mode), _ptr(out), N, _stream()), "qmoe_gemm")
    return out


def gemm_add_rmsnorm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor, rms_w: torch.Tensor, eps: float,
                     workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``C += A . B^T`` (fp32 ``C[M, N]`` in place), then returns
    ``bf16(rmsnorm(C) * rms_w)``: the bits of :func:`gemm` (ADD_F32) then
    :func:`rmsnorm_residual`, with the norm inside the split-K reduction
    when ``workspace`` (from :func:`gemm_workspace`) enables one."""
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[1]:
        raise ValueError("A must be [M,K] and B [N,K]")
    M, K = A.shape
    N = B.shape[0]
    _need(A, "A", BF16)
    _need(B, "B", BF16)
    _need(C, "C", F32, (M, N))
    _need(rms_w, "rms_w", BF16, (N,))
    x = torch.empty(M, N, dtype=BF16, device=A.device)
    _same_device(A, B, C, rms_w)
    if workspace is not None:
        _need(workspace, "workspace", F32)
        _same_device(A, workspace)
    check(lib().qmoe_gemm_ws_add_rmsnorm(_ptr(A), K, _ptr(B), M, N, K, _ptr(C), _ptr(rms_w), float(eps), _ptr(x),
                                         _ptr(workspace), 0 if workspace is None else workspace.numel() * 4,
                                         _stream()), "qmoe_gemm_ws_add_rmsnorm")
    return x


def gemv_rmsnorm(h: torch.Tensor, rms_w: torch.Tensor, eps: float, B: torch.Tensor,
                 mode: int = _lib.GEMM_STORE_BF16, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``bf16(rmsnorm(h[1,K])) . B[N,K]^T`` in one launch (the same bits as
    :func:`rmsnorm_residual` then :func:`gemm`)."""
    if h.dim() != 2 or h.shape[0] != 1 or B.dim() != 2 or h.shape[1] != B.shape[1]:
        raise ValueError("h must be [1,K] and B [N,K]")
    K, N = h.shape[1], B.shape[0]
    _need(h, "h", F32)
    _need(rms_w, "rms_w", BF16, (K,))
    _need(B, "B", BF16)
    if out is None:
        if mode == _lib.GEMM_ADD_F32:
            raise ValueError("mode ADD_F32 needs out")
        out = torch.empty(1, N, dtype=BF16 if mode == _lib.GEMM_STORE_BF16 else F32, device=h.device)
    _need(out, "out", BF16 if mode == _lib.GEMM_STORE_BF16 else F32, (1, N))
    _same_device(h, rms_w, B, out)
    check(lib().qmoe_gemv_rmsnorm(_ptr(h), _ptr(rms_w), float(eps), _ptr(B), N, K, int(mode), _ptr(out), _stream()),
          "qmoe_gemv_rmsnorm")
    return out


def qkv_finish(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
               rope_cos: torch.Tensor, rope_sin: torch.Tensor, positions: torch.Tensor, B: int, S: int,
               Hq: int, Hkv: int, k_cache: torch.Tensor, v_cache: torch.Tensor, eps: float,
               q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-head q/k RMSNorm + RoPE from the raw projection ``qkv[B*S, (Hq+2Hkv)*D]``
    (f32), K/V rows into the cache; returns ``q[B*S, Hq, D]`` (bf16)."""
    T = B * S
    D = q_norm_w.shape[0]
    _need(qkv, "qkv", F32, (T, (Hq + 2 * Hkv) * D))
    _need(q_norm_w, "q_norm_w", BF16, (D,))
    _need(k_norm_w, "k_norm_w", BF16, (D,))
    max_pos = rope_cos.shape[0]
    _need(rope_cos, "rope_cos", F32, (max_pos, D // 2))
    _need(rope_sin, "rope_sin", F32, (max_pos, D // 2))
    _need(positions, "positions", I32, (T,))
    if k_cache.dim() != 4 or k_cache.shape[:2] != (B, Hkv) or k_cache.shape[3] != D:
        raise ValueError(f"k_cache must be [B={B}, Hkv={Hkv}, S_max, D={D}]")
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    q_out = torch.empty(T, Hq, D, dtype=BF16, device=qkv.device) if q_out is None else q_out
    _need(q_out, "q_out", BF16, (T, Hq, D))
    _same_device(qkv, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, k_cache, v_cache, q_out)
    check(
        lib().qmoe_qkv_finish(_ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_cos), _ptr(rope_sin), max_pos,
                              _ptr(positions), B, S, Hq, Hkv, D, k_cache.shape[2], float(eps), _ptr(q_out),
                              _ptr(k_cache), _ptr(v_cache), _stream()),
        "qmoe_qkv_finish",
    )
    return q_out


# ----------------------------------------------------------------- attention
def qkv_norm_rope(
    x: torch.Tensor, wqkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
    rope_cos: torch.Tensor, rope_sin: torch.Tensor, positions: torch.Tensor,
    B: int, S: int, Hq: int, Hkv: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
    eps: float, q_out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """QKV projection + per-head RMSNorm + RoPE; K/V written into the cache.
    Returns ``q[B*S, Hq, D]`` (bf16).  ``workspace`` (f32, at least
    :func:`qkv_norm_rope_workspace` bytes) is allocated here when not given."""
    T, H = x.shape
    D = q_norm_w.shape[0]
    if T != B * S:
        raise ValueError("x must be [B*S, H]")
    _need(x, "x", BF16)
    _need(wqkv, "wqkv", BF16, ((Hq + 2 * Hkv) * D, H))
    _need(q_norm_w, "q_norm_w", BF16, (D,))
    _need(k_norm_w, "k_norm_w", BF16, (D,))
    max_pos = rope_cos.shape[0]
    _need(rope_cos, "rope_cos", F32, (max_pos, D // 2))
    _need(rope_sin, "rope_sin", F32, (max_pos, D // 2))
    _need(positions, "positions", I32, (T,))
    if k_cache.dim() != 4 or k_cache.shape[:2] != (B, Hkv) or k_cache.shape[3] != D:
        raise ValueError(f"k_cache must be [B={B}, Hkv={Hkv}, S_max, D={D}]")
    S_max = k_cache.shape[2]
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    q_out = torch.empty(T, Hq, D, dtype=BF16, device=x.device) if q_out is None else q_out
    _need(q_out, "q_out", BF16, (T, Hq, D))
    ws_bytes = qkv_norm_rope_workspace(T, H, Hq, Hkv, D)
    if workspace is None and ws_bytes > 0:
        workspace = torch.empty(ws_bytes // 4, dtype=F32, device=x.device)
    if workspace is not None:
        _need(workspace, "workspace", F32)
        if workspace.numel() * 4 < ws_bytes:
            raise ValueError(f"workspace: need {ws_bytes} bytes, got {workspace.numel() * 4}")
    _same_device(x, wqkv, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, k_cache, v_cache, q_out,
                 workspace)
    check(
        lib().qmoe_qkv_norm_rope(
            _ptr(x), _ptr(wqkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_cos), _ptr(rope_sin),
            max_pos, _ptr(positions), B, S, H, Hq, Hkv, D, S_max, float(eps), _ptr(q_out),
            _ptr(k_cache), _ptr(v_cache), _ptr(workspace), _stream(),
        ),
        "qmoe_qkv_norm_rope",
    )
    return q_out


def qkv_norm_rope_workspace(T: int, H: int, Hq: int, Hkv: int, D: int) -> int:
    """Bytes of f32 workspace :func:`qkv_norm_rope` needs for ``T`` token rows."""
    return int(lib().qmoe_qkv_norm_rope_workspace(T, H, Hq, Hkv, D))


def attn_prefill_workspace(B: int, S: int, Hq: int, D: int, device) -> torch.Tensor:
    """Zeroed workspace for :func:`attn_prefill` (key-split launches)."""
    n = int(lib().qmoe_attn_prefill_workspace(B, S, Hq, D))
    if n < 0:
        raise ValueError("bad sizes for the prefill attention workspace")
    return torch.zeros(max(n, 4) // 4, dtype=I32, device=device)


def attn_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, B: int, S: int,
                 start=0, scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal GQA attention of ``q[B*S, Hq, D]`` against the cache; returns ``[B*S, Hq*D]``.
    ``start`` (cache index of the first query) is an int, or an int32 ``[1]``
    device tensor read by the kernel (clamped into ``[0, S_max - S]``), so a
    captured graph replays the call at any position.  ``workspace`` (from
    :func:`attn_prefill_workspace`, host ``start`` only) lets a small launch
    split its longer query tiles' key ranges over more workgroups."""
    T, Hq, D = q.shape
    if T != B * S:
        raise ValueError("q must be [B*S, Hq, D]")
    _need(q, "q", BF16)
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError("k_cache must be [B, Hkv, S_max, D]")
    Hkv, S_max = k_cache.shape[1], k_cache.shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = torch.empty(T, Hq * D, dtype=BF16, device=q.device) if out is None else out
    _need(out, "out", BF16, (T, Hq * D))
    if isinstance(start, torch.Tensor):
        _need(start, "start", I32, (1,))
        _same_device(q, k_cache, v_cache, out, start)
        check(
            lib().qmoe_attn_prefill_at(_ptr(q), _ptr(k_cache), _ptr(v_cache), B, S, Hq, Hkv, D, S_max,
                                       _ptr(start), float(scale), _ptr(out), _stream()),
            "qmoe_attn_prefill_at",
        )
        return out
    _same_device(q, k_cache, v_cache, out)
    if workspace is not None:
        _same_device(q, workspace)
        if not workspace.is_contiguous():
            raise ValueError("workspace must be contiguous")
        check(
            lib().qmoe_attn_prefill_ws(_ptr(q), _ptr(k_cache), _ptr(v_cache), B, S, Hq, Hkv, D, S_max,
                                       start, float(scale), _ptr(workspace), _nbytes(workspace), _ptr(out),
                                       _stream()),
            "qmoe_attn_prefill_ws",
        )
        return out
    check(
        lib().qmoe_attn_prefill(_ptr(q), _ptr(k_cache), _ptr(v_cache), B, S, Hq, Hkv, D, S_max,
                                start, float(scale), _ptr(out), _stream()),
        "qmoe_attn_prefill",
    )
    return out


def attn_decode_chunk(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, B: int, S: int,
                      start: torch.Tensor, scale: Optional[float] = None,
                      workspace: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention of a short chunk ``q[B*S, Hq, D]`` at cache positions
    ``start .. start+S-1`` (``start``: int32 ``[1]`` device tensor, clamped
    into ``[0, S_max - S]``) as ``B*S`` single-query decode problems; returns
    ``[B*S, Hq*D]``, the same values :func:`attn_prefill` computes (to
    rounding)."""
    T, Hq, D = q.shape
    if T != B * S:
        raise ValueError("q must be [B*S, Hq, D]")
    _need(q, "q", BF16)
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError("k_cache must be [B, Hkv, S_max, D]")
    Hkv, S_max = k_cache.shape[1], k_cache.shape[2]
    _need(start, "start", I32, (1,))
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    need = int(lib().qmoe_attn_decode_workspace(T, Hq, D, S_max))
    if workspace is None:
        workspace = torch.empty(need, dtype=F32, device=q.device)
    if workspace.dtype != F32 or workspace.numel() < need or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous float32 tensor of >= {need} elements")
    out = torch.empty(T, Hq * D, dtype=BF16, device=q.device) if out is None else out
    _need(out, "out", BF16, (T, Hq * D))
    _same_device(q, k_cache, v_cache, start, workspace, out)
    check(
        lib().qmoe_attn_decode_chunk(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(start), B, S, Hq, Hkv, D, S_max,
                                     float(scale), _ptr(workspace), _ptr(out), _stream()),
        "qmoe_attn_decode_chunk",
    )
    return out


def attn_decode_fused(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                      rope_cos: torch.Tensor, rope_sin: torch.Tensor, positions: torch.Tensor, Hq: int, Hkv: int,
                      k_cache: torch.Tensor, v_cache: torch.Tensor, eps: float, scale: Optional[float] = None,
                      workspace: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                      max_ctx: Optional[int] = None) -> torch.Tensor:
    """One decode step of the attention from the raw projection ``qkv[B, (Hq+2Hkv)*D]``
    (f32): the q/k norm + RoPE, the new K/V rows into the cache at ``positions[b]``,
    and attention over cache entries ``[0, positions[b]]`` in one split launch and
    the merge (``qkv_finish`` then ``attn_decode`` with ``ctx_len = positions + 1``,
    same bits).  Returns ``[B, Hq*D]`` bf16."""
    B = positions.shape[0]
    D = q_norm_w.shape[0]
    _need(qkv, "qkv", F32, (B, (Hq + 2 * Hkv) * D))
    _need(q_norm_w, "q_norm_w", BF16, (D,))
    _need(k_norm_w, "k_norm_w", BF16, (D,))
    max_pos = rope_cos.shape[0]
    _need(rope_cos, "rope_cos", F32, (max_pos, D // 2))
    _need(rope_sin, "rope_sin", F32, (max_pos, D // 2))
    _need(positions, "positions", I32, (B,))
    if k_cache.dim() != 4 or k_cache.shape[:2] != (B, Hkv) or k_cache.shape[3] != D:
        raise ValueError(f"k_cache must be [B={B}, Hkv={Hkv}, S_max, D={D}]")
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    S_max = k_cache.shape[2]
    max_ctx = S_max if max_ctx is None else int(max_ctx)
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    need = int(lib().qmoe_attn_decode_workspace(B, Hq, D, max_ctx))
    if workspace is None:
        workspace = torch.empty(need, dtype=F32, device=qkv.device)
    if workspace.dtype != F32 or workspace.numel() < need or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous float32 tensor of >= {need} elements")
    out = torch.empty(B, Hq * D, dtype=BF16, device=qkv.device) if out is None else out
    _need(out, "out", BF16, (B, Hq * D))
    _same_device(qkv, q_norm_w, k_norm_w, rope_cos, rope_sin, positions, k_cache, v_cache, workspace, out)
    check(
        lib().qmoe_attn_decode_fused(_ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_cos), _ptr(rope_sin),
                                     max_pos, _ptr(positions), B, Hq, Hkv, D, S_max, max_ctx, float(eps),
                                     float(scale), _ptr(k_cache), _ptr(v_cache), _ptr(workspace), _ptr(out),
                                     _stream()),
        "qmoe_attn_decode_fused",
    )
    return out


def attn_decode_workspace(B: int, Hq: int, D: int, S_max: int, device) -> torch.Tensor:
    n = int(lib().qmoe_attn_decode_workspace(B, Hq, D, S_max))
    return torch.empty(n, dtype=F32, device=device)


def attn_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, ctx_len: torch.Tensor,
                scale: Optional[float] = None, workspace: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, max_ctx: Optional[int] = None) -> torch.Tensor:
    """One query per batch row (``q[B, Hq, D]``) over cache entries ``[0, ctx_len[b])``;
    returns ``[B, Hq*D]``.  ``max_ctx`` (a context bucket, ``ctx_len <= max_ctx
    <= S_max``) sizes the launch for the bucket instead of the cache capacity."""
    B, Hq, D = q.shape
    _need(q, "q", BF16)
    _need(k_cache, "k_cache", BF16)
    _need(v_cache, "v_cache", BF16, tuple(k_cache.shape))
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError("k_cache must be [B, Hkv, S_max, D]")
    Hkv, S_max = k_cache.shape[1], k_cache.shape[2]
    _need(ctx_len, "ctx_len", I32, (B,))
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    if workspace is None:
        workspace = attn_decode_workspace(B, Hq, D, S_max, q.device)
    need = int(lib().qmoe_attn_decode_workspace(B, Hq, D, S_max))
    if workspace.dtype != F32 or workspace.numel() < need or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous float32 tensor of >= {need} elements")
    out = torch.empty(B, Hq * D, dtype=BF16, device=q.device) if out is None else out
    _need(out, "out", BF16, (B, Hq * D))
    _same_device(q, k_cache, v_cache, ctx_len, workspace, out)
    if max_ctx is not None and max_ctx < S_max:
        check(
            lib().qmoe_attn_decode_bucket(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(ctx_len), B, Hq, Hkv, D,
                                          S_max, int(max_ctx), float(scale), _ptr(workspace), _ptr(out),
                                          _stream()),
            "qmoe_attn_decode_bucket",
        )
        return out
    check(
        lib().qmoe_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(ctx_len), B, Hq, Hkv, D,
                               S_max, float(scale), _ptr(workspace), _ptr(out), _stream()),
        "qmoe_attn_decode",
    )
    return out


# ----------------------------------------------------------------- embedding / greedy argmax
def embed(ids: torch.Tensor, table: torch.Tensor, out: Optional[torch.Tensor] = None,
          err: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 rows ``table[ids]`` (``ids`` i64, any shape; returns ``[ids.numel(), H]``).
    Out-of-range ids give zero rows and set ``err[0] = 1`` (``err``: i32 [1],
    cleared by the caller) instead of trapping on the GPU."""
    if table.dim() != 2:
        raise ValueError("table must be [V, H]")
    V, H = table.shape
    _need(table, "table", BF16)
    flat = ids.reshape(-1)
    if flat.dtype != torch.int64:
        raise ValueError("ids must be int64")
    if not flat.is_contiguous():
        flat = flat.contiguous()
    n = flat.numel()
    out = torch.empty(n, H, dtype=F32, device=table.device) if out is None else out
    _need(out, "out", F32, (n, H))
    if err is None:
        err = torch.zeros(1, dtype=I32, device=table.device)
    _need(err, "err", I32, (1,))
    _same_device(flat, table, out, err)
    check(lib().qmoe_embed(_ptr(table), V, H, _ptr(flat), n, _ptr(out), _ptr(err), _stream()), "qmoe_embed")
    return out


def argmax_workspace(rows: int, device) -> torch.Tensor:
    n = int(lib().qmoe_argmax_workspace(rows))
    return torch.empty(max(n, 8), dtype=torch.uint8, device=device)


def argmax(x: torch.Tensor, out: Optional[torch.Tensor] = None,
           workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row-wise argmax of f32 ``x[rows, n]`` into i64 ``out[rows]`` (first max;
    NaN highest) -- graph-safe (no memset, no semaphores)."""
    if x.dim() != 2:
        raise ValueError("x must be [rows, n]")
    rows, n = x.shape
    _need(x, "x", F32)
    out = torch.empty(rows, dtype=torch.int64, device=x.device) if out is None else out
    _need(out, "out", torch.int64, (rows,))
    workspace = argmax_workspace(rows, x.device) if workspace is None else workspace
    _need(workspace, "workspace", torch.uint8)
    _same_device(x, out, workspace)
    check(lib().qmoe_argmax(_ptr(x), rows, n, n, _ptr(workspace), workspace.numel(), _ptr(out), _stream()),
          "qmoe_argmax")
    return out
