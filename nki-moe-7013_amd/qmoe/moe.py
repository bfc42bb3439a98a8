"""The sparse MoE block on libqmoe kernels.

Host-side mirror of the reference's MoE module surface:

* :class:`MoEBlock` -- router + experts + combine, the body of
  ``self.mlp(hidden_states, padding_mask)[0]`` in
  ``NeuronQwen3MoeDecoderLayer.forward`` (qwen_with_nki.py:10206), with the
  residual add of 10207 fused into the combine.
* :class:`ExpertMLPs` -- the two expert-dispatch seams the reference patches on
  NxDI's ``ExpertMLPsV2``: ``forward_selective_loading`` (decode,
  qwen_with_nki.py:2377, 3456-3478) and ``torch_blockwise_matmul_inference``
  (prefill, 5872-5881), with the same argument meaning.
"""

from __future__ import annotations

import dataclasses
from types import SimpleNamespace
from typing import Optional

import torch

from . import _lib, ops

# Token counts at or below this use the HBM-bound GEMV experts; above it the
# MFMA grouped GEMM.  (Each touched expert is streamed once either way; with
# 128 experts the two paths take the same time at T = 48 on MI355X: 242 us
# per block, against 212 / 233 us at T = 32 and 270 / 248 us at T = 64.)
GEMV_MAX_TOKENS = 48
# Row tile of the prefill dispatch table: one (up to) 256 x 256 MFMA tile per
# (tile, panel).
TILE_M = _lib.GROUPED_MAX_TILE_M
# Prompt sizes (up to this many routed (token, expert) pairs): 224-row tiles.
# There the one launch is bound by the crowded experts' full tiles (a 256-row
# gate_up item, then the tile's down items); 224 rows are 7 of the 8 32-row
# MFMA blocks, for about two more tiles per layer (640-token prompt, deep
# layers: 87.5 -> 82.8 and 88.2 -> 86.2 us, the same y_slot bits; 192 rows and
# 1024 tokens or more were slower).
SHORT_TILE_M, SHORT_TILE_MAX_PAIRS = 224, 6144


def tile_m_for(T: int, k: int) -> int:
    """Row tile of the dispatch table for T tokens routed to k experts each."""
    return SHORT_TILE_M if T * k <= SHORT_TILE_MAX_PAIRS else TILE_M


class ExpertMLPs:
    """Routed SwiGLU experts with packed weights ``w13 [E,2I,H]`` and blocked ``w2 [E,I/8,H,8]``."""

    def __init__(self, w13: torch.Tensor, w2: torch.Tensor, top_k: int,
                 normalize_top_k_affinities: bool = True):
        self.w13 = w13
        self.w2 = w2
        self.num_experts = w13.shape[0]
        self.hidden_size = w13.shape[2]
        self.intermediate_size = w13.shape[1] // 2
        self.top_k = top_k
        self.normalize_top_k_affinities = normalize_top_k_affinities
        # NxDI's RoutedExpertsMLPOpsConfig flag the seams read
        # (qwen_with_nki.py:5768, 3449): True scales each pair's input row by
        # its affinity before the MLP instead of the output after it (Qwen3
        # leaves it False).
        self.routed_experts_mlp_config = SimpleNamespace(early_expert_affinity_modulation=False)

    def run(self, x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor,
            residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Permute, run the experts, combine: ``residual + sum_j w_j * expert_j(x)`` (f32)."""
        T = x.shape[0]
        route = ops.moe_permute(topk_idx, self.num_experts, tile_m_for(T, topk_idx.shape[1]))
        if T <= GEMV_MAX_TOKENS:
            y = ops.moe_experts_gemv(x, self.w13, self.w2, route)
        else:
            y = ops.moe_experts_grouped(x, self.w13, self.w2, route)
        return ops.moe_combine(y, route, topk_w, residual, out)

    def run_early(self, x: torch.Tensor, topk_idx: torch.Tensor, topk_w: torch.Tensor) -> torch.Tensor:
        """``sum_j expert_j(w_j * x)`` (f32): early affinity modulation, the
        ``early_expert_affinity_modulation`` branch of qwen_with_nki.py:5768-5775.

        Every (token, expert) pair p = t*k + j becomes its own input row
        ``bf16(w_tj * x_t)`` (the experts read bf16) routed to its one expert;
        the combine kernel then sums each token's k outputs with unit weights
        in the fixed order j = 0..k-1, through the pair dispatch's own slot map."""
        T, k = topk_idx.shape
        if T == 0:
            return torch.zeros(0, x.shape[1], dtype=torch.float32, device=x.device)
        rows = (x.float().repeat_interleave(k, dim=0) * topk_w.reshape(T * k, 1).float()).to(torch.bfloat16)
        pair_idx = topk_idx.reshape(T * k, 1).contiguous()
        route = ops.moe_permute(pair_idx, self.num_experts, tile_m_for(T * k, 1))
        if T * k <= GEMV_MAX_TOKENS:
            y = ops.moe_experts_gemv(rows, self.w13, self.w2, route)
        else:
            y = ops.moe_experts_grouped(rows, self.w13, self.w2, route)
        # token_slot of the pair dispatch, read as [T, k]: entry (t, j) is the slot of pair t*k + j
        per_token = dataclasses.replace(route, T=T, k=k)
        return ops.moe_combine(y, per_token, torch.ones(T, k, dtype=torch.float32, device=x.device))

    # -- reference seams -------------------------------------------------------
    def forward_selective_loading(self, hidden_states: torch.Tensor, expert_affinities: torch.Tensor,
                                  expert_index: torch.Tensor) -> torch.Tensor:
        """Decode seam (qwen_with_nki.py:3456-3478): gather the chosen
        affinities from ``expert_affinities[T,E]``, L1-normalise them when
        ``normalize_top_k_affinities``, and return ``sum_j aff_j * mlp_j(x)``
        as ``[T,H]`` in the input dtype."""
        T = hidden_states.shape[0]
        idx = expert_index.to(torch.int32).contiguous()
        chosen = torch.gather(expert_affinities.float(), 1, expert_index.long())
        if self.normalize_top_k_affinities:
            chosen = torch.nn.functional.normalize(chosen, p=1.0, dim=1)
        x = hidden_states.to(torch.bfloat16).contiguous()
        if self._early():
            return self.run_early(x, idx, chosen.contiguous()).to(hidden_states.dtype).view(T, -1)
        out = self.run(x, idx, chosen.contiguous())
        return out.to(hidden_states.dtype).view(T, -1)

    def _early(self) -> bool:
        return bool(getattr(self.routed_experts_mlp_config, "early_expert_affinity_modulation", False))

    def torch_blockwise_matmul_inference(self, block_size, num_blocks, hidden_states,
                                         expert_affinities_masked, token_position_to_id,
                                         block_to_expert, pad_inputs_for_matmul=False) -> torch.Tensor:
        """Prefill seam (qwen_with_nki.py:5872-5881, semantics 5728-5789).

        The reference's blocks list, per expert, the token rows routed to it
        (padding rows point at the extra row ``T``); each selected (token,
        expert) pair contributes ``mlp_e(x_t) * expert_affinities_masked[t, e]``.
        The same pairs are recovered here as a top-k list and dispatched
        through the build's own permutation (a token never repeats within
        one expert, so the reference's duplicate redirection is not needed).
        """
        T, H = hidden_states.shape
        E = self.num_experts
        tok = token_position_to_id.view(int(num_blocks), int(block_size)).long()
        exp = block_to_expert.view(int(num_blocks), 1).long().expand_as(tok)
        valid = tok < T
        sel = torch.zeros(T + 1, E, dtype=torch.bool, device=hidden_states.device)
        sel[tok[valid], exp[valid]] = True
        sel = sel[:T]
        k = int(sel.sum(dim=1).max().item()) if T > 0 else 0
        if k == 0:
            return torch.zeros_like(hidden_states)
        # order each token's experts by affinity (descending), like top-k
        aff = torch.where(sel, expert_affinities_masked.float(), torch.full_like(expert_affinities_masked.float(), -1.0))
        top_w, top_i = torch.topk(aff, k, dim=1)
        if not bool((top_w >= 0).all()):
            raise ValueError("every token must be routed to the same number of experts")
        run = self.run_early if self._early() else self.run
        out = run(hidden_states.to(torch.bfloat16).contiguous(), top_i.to(torch.int32).contiguous(),
                  top_w.contiguous())
        return out.to(hidden_states.dtype)


class MoEBlock:
    """Router + experts + combine.  ``forward(x_bf16[T,H], residual_f32[T,H])``
    returns ``residual + MoE(x)`` in fp32."""

    def __init__(self, w_router: torch.Tensor, w13: torch.Tensor, w2: torch.Tensor, top_k: int,
                 router_bias: Optional[torch.Tensor] = None):
        self.w_router = w_router
        self.router_bias = router_bias
        self.experts = ExpertMLPs(w13, w2, top_k)
        self.top_k = top_k
        self.last_routing = None
        self.last_input = None  # the bf16 rows the router last saw (for checks)
        self._bufs = {}

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None, norm: Optional[tuple] = None):
        """``residual + MoE(x)`` (fp32) for bf16 ``x[T,H]``.  ``norm = (rms_w,
        eps)`` (above the decode-block size): the combine also normalises the
        finished rows, and the call returns ``(out, bf16 normed rows)``."""
        T = x.shape[0]
        ex = self.experts
        if norm is not None and T <= ops.DECODE_BLOCK_MAX_T:
            raise ValueError("the fused output norm is for T > DECODE_BLOCK_MAX_T")
        if T <= ops.DECODE_BLOCK_MAX_T:
            bufs = self._decode_bufs(T, x.device)
            out = ops.moe_decode_block(self.w_router, ex.w13, ex.w2, self.top_k, x=x, bias=self.router_bias,
                                       residual=residual, out=out, bufs=bufs)
            self.last_routing = (bufs.logits, bufs.topk_w, bufs.topk_idx)
            self.last_input = x
            return out
        route = ops.moe_route(x, self.w_router, self.top_k, self.router_bias, tile_m_for(T, self.top_k))
        self.last_routing = (route.logits, route.topk_w, route.topk_idx)
        self.last_input = x
        if T <= GEMV_MAX_TOKENS:
            y = ops.moe_experts_gemv(x, ex.w13, ex.w2, route)
        else:
            y = ops.moe_experts_grouped(x, ex.w13, ex.w2, route)
        return ops.moe_combine(y, route, route.topk_w, residual, out, norm=norm)

    def forward_normed(self, h: torch.Tensor, rms_w: torch.Tensor, eps: float,
                       residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None):
        """``residual + MoE(rmsnorm(h) * rms_w)``: the post-attention RMSNorm
        fused into the router launch when ``T <= 8``."""
        T = h.shape[0]
        if T <= ops.DECODE_BLOCK_MAX_T:
            ex = self.experts
            bufs = self._decode_bufs(T, h.device)
            out = ops.moe_decode_block(self.w_router, ex.w13, ex.w2, self.top_k, h=h, rms_w=rms_w, eps=eps,
                                       bias=self.router_bias, residual=residual, out=out, bufs=bufs)
            self.last_routing = (bufs.logits, bufs.topk_w, bufs.topk_idx)
            self.last_input = bufs.x_out
            return out
        x = ops.rmsnorm_residual(h, rms_w, eps)
        return self.forward(x, residual, out)

    def _decode_bufs(self, T: int, device) -> "ops.DecodeBlockBuffers":
        key = (T, str(device))
        b = self._bufs.get(key)
        if b is None:
            ex = self.experts
            b = ops.DecodeBlockBuffers.alloc(T, ex.hidden_size, ex.intermediate_size, ex.num_experts,
                                             self.top_k, device)
            self._bufs[key] = b
        return b

    __call__ = forward
