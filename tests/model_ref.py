"""fp32 reference of the Qwen3-MoE model, built from the oracle's functions.

Runs on whatever device the weights live on (the oracle's torch code is
device-agnostic), so the 48-layer model can be checked on the GPU.  It
reads the same bf16 weights as the product (upcast exactly to fp32) and
keeps every activation in fp32.
"""

import torch

import oracle
from qmoe import weights


def layer_weights_f32(lw, experts=True):
    """The product's packed layer weights -> oracle-format fp32 weights
    (expert tensors only when ``experts``)."""
    D = lw["q_norm"].shape[0]
    nkv_d = (lw["wqkv"].shape[0] - lw["wo"].shape[1]) // 2
    wq, wk, wv = lw["wqkv"].float().split([lw["wo"].shape[1], nkv_d, nkv_d])
    return {
        "input_layernorm": lw["input_layernorm"].float(),
        "post_attention_layernorm": lw["post_attention_layernorm"].float(),
        "q_proj": wq, "k_proj": wk, "v_proj": wv, "o_proj": lw["wo"].float(),
        "q_norm": lw["q_norm"].float(), "k_norm": lw["k_norm"].float(),
        "router": lw["router"].float(),
        "gate_up_proj": weights.unpack_gate_up(lw["w13"]).float() if experts else None,
        "down_proj": weights.unpack_down(lw["w2"]).float() if experts else None,
    }


def expert_f32(lw, e):
    """One expert's NxDI-layout fp32 weights: gate_up (H, 2I), down (I, H)."""
    return (weights.unpack_gate_up(lw["w13"][e : e + 1]).float()[0],
            weights.unpack_down(lw["w2"][e : e + 1]).float()[0])


def cfg_dict(config):
    return dict(n_q=config.num_attention_heads, n_kv=config.num_key_value_heads, head_dim=config.head_dim,
                eps=config.rms_norm_eps, theta=float(config.rope_theta), top_k=config.num_experts_per_tok)


class ReferenceModel:
    """Greedy fp32 reference over the product's parameter tree."""

    def __init__(self, params, config):
        self.p, self.config, self.cfg = params, config, cfg_dict(config)
        self.kv = [None] * len(params["layers"])
        self.min_gap = float("inf")  # smallest k-th/(k+1)-th router logit gap seen
        self.recording = False  # while set, _layer appends (input, output, router logits) to trace
        self.trace = []  # per layer, the prompt pass of greedy()
        self.step_trace = []  # per layer, greedy()'s first decode step

    def _layer(self, i, h, positions):
        lw = self.p["layers"][i]
        B, S, H = h.shape
        T = B * S
        w = layer_weights_f32(lw, experts=T > 8)
        a, kv = oracle.attention_layer(oracle.rmsnorm(h, w["input_layernorm"], self.cfg["eps"]), w,
                                       positions, self.cfg, self.kv[i])
        self.kv[i] = kv
        h1 = h + a
        y = oracle.rmsnorm(h1, w["post_attention_layernorm"], self.cfg["eps"]).reshape(T, H)
        k = self.cfg["top_k"]
        if T > 8:
            m, _, _, logits = oracle.moe_block_prefill(y, w["router"], w["gate_up_proj"], w["down_proj"], k)
        else:
            # decode schedule of oracle.moe_block_decode, fetching only the chosen experts
            logits, top_w, top_i = oracle.router_topk(y, w["router"], k)
            rows = []
            for t in range(T):
                per_e = torch.stack([oracle.expert_swiglu(y[t : t + 1], *expert_f32(lw, int(e)))[0]
                                     for e in top_i[t]])
                rows.append(torch.sum(per_e * top_w[t].unsqueeze(1), dim=0))
            m = torch.stack(rows)
        top = torch.topk(logits, k + 1, dim=-1).values
        gap = top[:, k - 1] - top[:, k]
        self.min_gap = min(self.min_gap, float(gap.min()))
        self._gaps = gap if self._gaps is None else torch.minimum(self._gaps, gap)
        out = h1 + m.view(B, S, H)
        if self.recording:
            self.trace.append((h.clone(), out.clone(), logits.clone()))
        return out

    def logits(self, input_ids, positions):
        h = torch.nn.functional.embedding(input_ids, self.p["embed_tokens"]).float()
        self._gaps = None
        for i in range(len(self.p["layers"])):
            h = self._layer(i, h, positions)
        self.last_hidden = h  # fp32 [B, S, H] after the last layer, before the final norm
        self.last_gaps = self._gaps  # per token: smallest k-th/(k+1)-th router gap over the layers
        last = oracle.rmsnorm(h[:, -1], self.p["norm"].float(), self.cfg["eps"])
        return last @ self.p["lm_head"].float().t()

    def greedy(self, prompt, n_new):
        B, S = prompt.shape
        dev = prompt.device
        pos = torch.arange(S, device=dev).expand(B, S)
        self.recording, self.trace = True, []
        lg = self.logits(prompt, pos)
        self.recording = False
        self.prompt_hidden, self.prompt_logits, self.prompt_gaps = self.last_hidden, lg, self.last_gaps
        toks, gaps = [lg.argmax(-1)], [_top2_gap(lg)]
        for t in range(1, n_new):
            p = torch.full((B, 1), S + t - 1, device=dev)
            if t == 1:  # record the first decode step apart from the prompt's trace
                prompt_trace, self.trace, self.recording = self.trace, [], True
                lg = self.logits(toks[-1].view(B, 1), p)
                self.step_trace, self.trace, self.recording = self.trace, prompt_trace, False
            else:
                lg = self.logits(toks[-1].view(B, 1), p)
            toks.append(lg.argmax(-1))
            gaps.append(_top2_gap(lg))
        return torch.stack(toks, 1), gaps


def _top2_gap(lg):
    t = torch.topk(lg.float(), 2, dim=-1).values
    return float((t[:, 0] - t[:, 1]).min())
