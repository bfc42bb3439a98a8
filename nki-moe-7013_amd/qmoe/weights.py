"""Weight layouts and seeded random initialisation.

On-device layout of one MoE layer (both operands K-contiguous, so the decode
GEMV and the prefill MFMA GEMM read the same bytes along K):

* ``w13 [E, 2I, H]``: the reference's fused ``gate_up_proj (E, H, 2I)``
  (qwen_with_nki.py:8928-8966) transposed, with gate and up rows interleaved
  every 32 rows: packed rows ``[64j, 64j+32)`` are gate rows ``[32j, 32j+32)``
  and ``[64j+32, 64j+64)`` the matching up rows.  One 64-row block therefore
  yields 32 SwiGLU outputs without any cross-tile exchange.
* ``w2 [E, I/8, H, 8]``: the reference's ``down_proj (E, I, H)``
  (qwen_with_nki.py:8968-8990) in blocks of 8 intermediate units: element
  ``(e, b, h, j)`` is ``down[e, 8b + j, h]``.  One 8-unit slice of an expert is
  a contiguous ``H x 16``-byte run (the decode kernels stream exactly that per
  work item), and column ``h`` of a block is one 16-byte load.
* attention: ``wqkv [(Hq+2Hkv)*D, H]`` = q rows, k rows, v rows (the fused
  QKV concatenation of qwen_with_nki.py:8845-8862); ``wo [H, Hq*D]``.
"""

from __future__ import annotations

import torch

from ._lib import W13_GROUP, W2_BLOCK


def pack_gate_up(gate_up: torch.Tensor, group: int = W13_GROUP) -> torch.Tensor:
    """``(E, H, 2I)`` NxDI layout -> packed ``(E, 2I, H)`` (gate/up interleaved)."""
    E, H, I2 = gate_up.shape
    I = I2 // 2
    if I % group:
        raise ValueError(f"moe intermediate size {I} is not a multiple of {group}")
    t = gate_up.transpose(1, 2)
    gate = t[:, :I].reshape(E, I // group, group, H)
    up = t[:, I:].reshape(E, I // group, group, H)
    return torch.stack([gate, up], dim=2).reshape(E, 2 * I, H).contiguous()


def unpack_gate_up(w13: torch.Tensor, group: int = W13_GROUP) -> torch.Tensor:
    """Inverse of :func:`pack_gate_up`."""
    E, I2, H = w13.shape
    I = I2 // 2
    v = w13.reshape(E, I // group, 2, group, H)
    gate = v[:, :, 0].reshape(E, I, H)
    up = v[:, :, 1].reshape(E, I, H)
    return torch.cat([gate, up], dim=1).transpose(1, 2).contiguous()


def block_down(w2: torch.Tensor, block: int = W2_BLOCK) -> torch.Tensor:
    """Row-major down matrices ``(E, H, I)`` -> blocked ``(E, I/block, H, block)``."""
    E, H, I = w2.shape
    if I % block:
        raise ValueError(f"moe intermediate size {I} is not a multiple of {block}")
    return w2.reshape(E, H, I // block, block).permute(0, 2, 1, 3).contiguous()


def unblock_down(w2b: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`block_down`: ``(E, I/8, H, 8)`` -> ``(E, H, I)``."""
    E, NB, H, B = w2b.shape
    return w2b.permute(0, 2, 1, 3).reshape(E, H, NB * B).contiguous()


def pack_down(down: torch.Tensor) -> torch.Tensor:
    """``(E, I, H)`` NxDI layout -> blocked ``(E, I/8, H, 8)``."""
    E, I, H = down.shape
    return down.reshape(E, I // W2_BLOCK, W2_BLOCK, H).transpose(2, 3).contiguous()


def unpack_down(w2b: torch.Tensor) -> torch.Tensor:
    """Blocked ``(E, I/8, H, 8)`` -> NxDI ``(E, I, H)``."""
    E, NB, H, B = w2b.shape
    return w2b.transpose(2, 3).reshape(E, NB * B, H).contiguous()


def from_hf_experts(gate_proj, up_proj, down_proj):
    """Per-expert HF checkpoint tensors (``gate_proj/up_proj [I, H]``,
    ``down_proj [H, I]``, keys ``mlp.experts.{e}.*.weight``) -> ``(w13, w2)``."""
    gate = torch.stack(list(gate_proj))  # (E, I, H)
    up = torch.stack(list(up_proj))
    gate_up = torch.cat([gate, up], dim=1).transpose(1, 2)  # (E, H, 2I)
    w2 = torch.stack(list(down_proj))  # (E, H, I)
    return pack_gate_up(gate_up), block_down(w2)


def randn(shape, gen: torch.Generator, device, std: float = 0.02, dtype=torch.bfloat16) -> torch.Tensor:
    """N(0, std) in ``dtype``, generated on ``device`` from ``gen``."""
    t = torch.empty(shape, dtype=torch.float32, device=device)
    t.normal_(0.0, std, generator=gen)
    return t.to(dtype)
