"""qmoe: MI355X-native (gfx950) kernels and host code for the Qwen3-30B-A3B
decoder-layer hot path (MoE block, GQA attention, residual RMSNorm).

The kernels live in ``libqmoe.so`` (HIP, C ABI in include/qmoe_capi.h) and are
reached through :mod:`qmoe.ops`; there is no fallback implementation.
"""

from ._lib import LIB_PATH, QmoeError, lib  # noqa: F401
from .config import QWEN3_30B_A3B, Qwen3MoeShape  # noqa: F401

__version__ = "0.1.0"
