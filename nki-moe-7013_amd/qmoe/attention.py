"""GQA attention with qk-RMSNorm + RoPE fused into the QKV epilogue and a
contiguous per-sequence KV cache, on libqmoe kernels.

Mirrors ``NeuronQwen3MoEAttention`` (qwen_with_nki.py:10081-10109): QKV
projection -> per-head RMSNorm over head_dim (q_layernorm / k_layernorm,
10102-10103) -> RoPE with base ``rope_theta`` (10083-10087) -> causal GQA
attention over the KV cache ``[B, Hkv, S, D]`` (9943-9946) -> o_proj.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib, ops


def rope_tables(head_dim: int, max_pos: int, theta: float, device) -> tuple:
    """fp32 ``cos``/``sin`` ``[max_pos, head_dim/2]`` with inverse frequencies
    ``theta^(-2i/D)`` (the first half of the duplicated-half layout)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=device).float() / head_dim))
    freqs = torch.arange(max_pos, device=device, dtype=torch.float32).unsqueeze(1) * inv_freq
    return freqs.cos().contiguous(), freqs.sin().contiguous()


# Chunks of up to this many query rows at a device-held start run as
# single-query decode problems (qmoe_attn_decode_chunk).
CHUNK_DECODE_MAX = 16


class KVCache:
    """Contiguous K/V cache of one layer: ``[B, Hkv, S_max, D]`` bf16 each.

    Unpacks like the reference's ``(K, V)`` present-key-value tuple
    (``k, v = cache``), and :meth:`wrap` takes such a tuple back without a copy."""

    def __init__(self, B: int, n_kv: int, S_max: int, head_dim: int, device):
        self.k = torch.zeros(B, n_kv, S_max, head_dim, dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)

    @classmethod
    def wrap(cls, kv) -> "KVCache":
        """A :class:`KVCache` as is, or a ``(K, V)`` pair of contiguous bf16
        ``[B, Hkv, S_max, D]`` device tensors viewed as one (no copy)."""
        if isinstance(kv, KVCache):
            return kv
        if not isinstance(kv, (tuple, list)) or len(kv) != 2:
            raise ValueError("past_key_value must be a KVCache or a (K, V) pair")
        k, v = kv
        for name, t in (("K", k), ("V", v)):
            if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.dim() != 4 \
                    or not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError(f"past_key_value {name} must be a contiguous bf16 [B, Hkv, S_max, D] GPU tensor")
        if k.shape != v.shape:
            raise ValueError("past_key_value K and V shapes differ")
        c = cls.__new__(cls)
        c.k, c.v = k, v
        return c

    @property
    def capacity(self) -> int:
        return self.k.shape[2]

    def __iter__(self):
        return iter((self.k, self.v))

    def __len__(self) -> int:
        return 2

    def __getitem__(self, i):
        return (self.k, self.v)[i]


class Attention:
    """One layer's attention.  ``forward`` adds ``o_proj(attn(x))`` to the fp32
    residual stream in place (the residual add of qwen_with_nki.py:10200 fused
    into the o_proj epilogue)."""

    def __init__(self, wqkv, q_norm, k_norm, wo, n_q: int, n_kv: int, head_dim: int, eps: float):
        self.wqkv, self.q_norm, self.k_norm, self.wo = wqkv, q_norm, k_norm, wo
        self.n_q, self.n_kv, self.head_dim, self.eps = n_q, n_kv, head_dim, eps
        self.scale = 1.0 / math.sqrt(head_dim)
        self._ws = {}

    def _decode_ws(self, B: int, cache: KVCache, device) -> torch.Tensor:
        ws = self._ws.get((B, cache.capacity))
        if ws is None:
            ws = ops.attn_decode_workspace(B, self.n_q, self.head_dim, cache.capacity, device)
            self._ws[(B, cache.capacity)] = ws
        return ws

    def forward(self, x: torch.Tensor, residual: torch.Tensor, positions: torch.Tensor, B: int, S: int,
                cache: KVCache, rope_cos: torch.Tensor, rope_sin: torch.Tensor, start=0,
                max_ctx: Optional[int] = None, norm: Optional[tuple] = None,
                post_norm: Optional[tuple] = None) -> torch.Tensor:
        """``x[B*S, H]`` bf16 (input-normed), ``residual[B*S, H]`` f32 (updated
        in place), ``positions[B*S]`` i32 (RoPE position == cache index).

        S > 1: causal prefill of a chunk starting at cache index ``start`` (an
        int, or an int32 ``[1]`` device tensor for graph replays at any position).
        S == 1: decode; row b sees cache entries ``[0, positions[b]]`` (at most
        the first ``max_ctx`` when a context bucket is given), on every path.
        On the GEMV path (B <= 16 decode rows) the finish runs inside the
        attention launch (``attn_decode_fused``).
        ``norm = (rms_w, eps)``: ``x`` is the fp32 residual row itself (B*S == 1)
        and the input RMSNorm is fused into the QKV GEMV.
        ``post_norm = (rms_w, eps)``: returns ``bf16(rmsnorm(residual) * rms_w)``
        of the updated residual, computed with the o_proj's residual add
        (instead of the residual itself).
        """
        n_ws = ops.qkv_norm_rope_workspace(B * S, x.shape[1], self.n_q, self.n_kv, self.head_dim)
        qws = self._ws.get(("qkv", B * S))
        if qws is None:
            qws = torch.empty(max(n_ws // 4, 1), dtype=torch.float32, device=x.device)
            self._ws[("qkv", B * S)] = qws
        if norm is not None and (B * S != 1 or n_ws == 0):
            raise ValueError("the fused input norm takes one fp32 row on the GEMV path")
        if S == 1 and n_ws > 0:
            # decode on the GEMV path: raw projection, then finish + attention in one launch
            raw = qws[: n_ws // 4].view(B, -1)
            if norm is not None:
                ops.gemv_rmsnorm(x, norm[0], norm[1], self.wqkv, _lib.GEMM_STORE_F32, out=raw)
            else:
                ops.gemm(x, self.wqkv, _lib.GEMM_STORE_F32, out=raw)
            o = ops.attn_decode_fused(raw, self.q_norm, self.k_norm, rope_cos, rope_sin, positions, self.n_q,
                                      self.n_kv, cache.k, cache.v, self.eps, self.scale,
                                      self._decode_ws(B, cache, x.device), max_ctx=max_ctx)
        else:
            q = ops.qkv_norm_rope(x, self.wqkv, self.q_norm, self.k_norm, rope_cos, rope_sin, positions, B, S,
                                  self.n_q, self.n_kv, cache.k, cache.v, self.eps, workspace=qws)
            if S > 1 and isinstance(start, torch.Tensor) and B * S <= CHUNK_DECODE_MAX:
                # a few-token chunk at a device-held position (speculative verification):
                # one decode problem per query spreads the K/V stream over many CUs
                ws = self._ws.get(("chunk", B * S, cache.capacity))
                if ws is None:
                    ws = ops.attn_decode_workspace(B * S, self.n_q, self.head_dim, cache.capacity, x.device)
                    self._ws[("chunk", B * S, cache.capacity)] = ws
                o = ops.attn_decode_chunk(q.view(B * S, self.n_q, self.head_dim), cache.k, cache.v, B, S, start,
                                          self.scale, ws)
            elif S > 1:
                aws = None
                if not isinstance(start, torch.Tensor):
                    aws = self._ws.get(("prefill", B, S))
                    if aws is None:
                        aws = ops.attn_prefill_workspace(B, S, self.n_q, self.head_dim, x.device)
                        self._ws[("prefill", B, S)] = aws
                o = ops.attn_prefill(q, cache.k, cache.v, B, S, start, self.scale, workspace=aws)
            else:
                o = ops.attn_decode(q.view(B, self.n_q, self.head_dim), cache.k, cache.v, positions + 1, self.scale,
                                    self._decode_ws(B, cache, x.device), max_ctx=max_ctx)
        key = ("oproj", o.shape[0])
        if key not in self._ws:  # split-K scratch for prefill-size token counts (None: not split)
            self._ws[key] = ops.gemm_workspace(o.shape[0], self.wo.shape[0], self.wo.shape[1], x.device)
        if post_norm is not None:
            return ops.gemm_add_rmsnorm(o, self.wo, residual, post_norm[0], post_norm[1], workspace=self._ws[key])
        ops.gemm(o, self.wo, _lib.GEMM_ADD_F32, out=residual, workspace=self._ws[key])
        return residual
