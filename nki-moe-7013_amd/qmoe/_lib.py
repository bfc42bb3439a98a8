"""ctypes binding of libqmoe.so (the C ABI declared in include/qmoe_capi.h).

Loading fails loudly: there is no fallback implementation of any kernel.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_void_p, c_char_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqmoe.so")

QMOE_OK = 0
QMOE_ERR_INVALID = 1
QMOE_ERR_HIP = 2

GEMM_STORE_BF16 = 0
GEMM_STORE_F32 = 1
GEMM_ADD_F32 = 2

W13_GROUP = 32
W2_BLOCK = 8
GROUPED_MAX_TILE_M = 256
VERSION = 3
META_INTS = 24
DECODE_BLOCK_WGS = 256
DECODE_BLOCK_NOALLOC_MAX_TH = 16384
DECODE_BLOCK_STATE_BYTES = 262144
DECODE_BLOCK_STATUS_OFFSET = 1024

P = c_void_p
I64 = c_int64

# name -> (restype, argtypes); mirrors include/qmoe_capi.h one to one.
PROTOTYPES = {
    "qmoe_version": (c_int, []),
    "qmoe_last_error": (c_char_p, []),
    "qmoe_rmsnorm_residual": (c_int, [P, P, P, I64, I64, c_float, P, P, P]),
    "qmoe_router_topk": (c_int, [P, P, P, I64, I64, I64, I64, P, P, P, P]),
    "qmoe_router_topk_ws": (c_int, [P, P, P, I64, I64, I64, I64, P, P, P, P, I64, P]),
    "qmoe_router_workspace": (c_int64, [I64, I64, I64]),
    "qmoe_moe_permute": (c_int, [P, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P]),
    "qmoe_moe_permute_tiles": (I64, [I64, I64, I64, I64]),
    "qmoe_moe_route": (c_int, [P, P, P, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, P]),
    "qmoe_moe_route_ws": (c_int, [P, P, P, I64, I64, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, P, I64,
                                  P]),
    "qmoe_moe_decode_block": (
        c_int, [P, P, P, c_float, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P, P, I64, P, P, P]),
    "qmoe_moe_decode_block_workspace": (c_int64, [I64, I64]),
    "qmoe_moe_decode_block_noalloc": (
        c_int, [P, P, P, c_float, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P, P, P, P]),
    "qmoe_moe_experts_gemv": (c_int, [P, P, P, P, P, P, P, I64, I64, I64, I64, I64, P, P, P]),
    "qmoe_moe_experts_grouped": (c_int, [P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, P, P, P]),
    "qmoe_moe_combine": (c_int, [P, c_int, P, P, P, I64, I64, I64, P, P]),
    "qmoe_moe_combine_norm": (c_int, [P, c_int, P, P, P, I64, I64, I64, P, P, c_float, P, P]),
    "qmoe_gemm": (c_int, [P, I64, P, I64, I64, I64, c_int, P, I64, P]),
    "qmoe_gemm_ws": (c_int, [P, I64, P, I64, I64, I64, c_int, P, I64, P, I64, P]),
    "qmoe_gemm_ws_add_rmsnorm": (c_int, [P, I64, P, I64, I64, I64, P, P, c_float, P, P, I64, P]),
    "qmoe_gemm_ws_workspace": (c_int64, [I64, I64, I64]),
    "qmoe_qkv_norm_rope": (
        c_int,
        [P, P, P, P, P, P, I64, P, I64, I64, I64, I64, I64, I64, I64, c_float, P, P, P, P, P],
    ),
    "qmoe_qkv_norm_rope_workspace": (c_int64, [I64, I64, I64, I64, I64]),
    "qmoe_attn_prefill": (c_int, [P, P, P, I64, I64, I64, I64, I64, I64, I64, c_float, P, P]),
    "qmoe_attn_prefill_at": (c_int, [P, P, P, I64, I64, I64, I64, I64, I64, P, c_float, P, P]),
    "qmoe_attn_prefill_ws": (c_int, [P, P, P, I64, I64, I64, I64, I64, I64, I64, c_float, P, I64, P, P]),
    "qmoe_attn_prefill_workspace": (c_int64, [I64, I64, I64, I64]),
    "qmoe_attn_decode_workspace": (c_int64, [I64, I64, I64, I64]),
    "qmoe_embed": (c_int, [P, I64, I64, P, I64, P, P, P]),
    "qmoe_argmax": (c_int, [P, I64, I64, I64, P, I64, P, P]),
    "qmoe_argmax_workspace": (c_int64, [I64]),
    "qmoe_attn_decode": (c_int, [P, P, P, P, I64, I64, I64, I64, I64, c_float, P, P, P]),
    "qmoe_gemv_rmsnorm": (c_int, [P, P, c_float, P, I64, I64, c_int, P, P]),
    "qmoe_qkv_finish": (c_int, [P, P, P, P, P, I64, P, I64, I64, I64, I64, I64, I64, c_float, P, P, P, P]),
    "qmoe_attn_decode_bucket": (c_int, [P, P, P, P, I64, I64, I64, I64, I64, I64, c_float, P, P, P]),
    "qmoe_attn_decode_fused": (c_int, [P, P, P, P, P, I64, P, I64, I64, I64, I64, I64, I64, c_float, c_float, P, P,
                                       P, P, P]),
    "qmoe_attn_decode_chunk": (c_int, [P, P, P, P, I64, I64, I64, I64, I64, I64, c_float, P, P, P]),
}


class QmoeError(RuntimeError):
    """A libqmoe entry point returned a non-zero status."""


_lib = None


def lib() -> ctypes.CDLL:
    """Load libqmoe.so once; raise ImportError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python nki-moe-7013_amd/build.py` "
            "(the HIP kernels have no fallback)"
        )
    l = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    _lib = l
    return l


def last_error() -> str:
    return (lib().qmoe_last_error() or b"").decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != QMOE_OK:
        kind = {QMOE_ERR_INVALID: "invalid argument", QMOE_ERR_HIP: "HIP error"}.get(rc, f"status {rc}")
        msg = f"{what}: {kind}: {last_error()}"
        if rc == QMOE_ERR_INVALID:
            raise ValueError(msg)
        raise QmoeError(msg)
