"""Qwen3-30B-A3B model-class surface on libqmoe kernels.

Host-side mirror of the reference's model module (``qwen_with_nki.py``, as
driven by ``main.py --mode generate``):

* :class:`MoENeuronConfig` / :class:`Qwen3MoeInferenceConfig` -- the two config
  objects ``prepare_inference`` builds (main.py:372-390; config semantics
  qwen_with_nki.py:9803-9894).
* :class:`NeuronQwen3MoeDecoderLayer` -- ``forward(hidden_states, ...)`` with
  the reference's 5-tuple return (qwen_with_nki.py:10155-10213).
* :class:`NeuronQwen3MoeModel` -- embedding, 48 layers, final norm, lm_head
  (qwen_with_nki.py:10231-10292).
* :class:`NeuronQwen3MoeForCausalLM` -- ``get_neuron_config_cls``,
  ``get_config_cls``, ``__init__(model_path, config)``, ``compile(path)``,
  ``load(path)``, ``reset()``, ``convert_hf_to_neuron_state_dict``
  (qwen_with_nki.py:10687-10971; main.py:386-410).
* :class:`HuggingFaceGenerationAdapter` -- ``generate(input_ids, ...)``
  (main.py:503, 557-569, 638-645).

The residual stream is fp32 between kernels; GEMM inputs are bf16.
Everything runs on one GPU; ``tp_degree`` other than 1 is rejected.
"""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Any, Callable, Dict, List, Optional

import torch

from . import _lib, ops, weights
from .attention import Attention, KVCache, rope_tables
from .config import Qwen3MoeShape
from .moe import MoEBlock


# ============================================================================ config
class MoENeuronConfig:
    """Run-time configuration (the subset of NxDI's ``MoENeuronConfig`` the
    generate path reads: main.py:377-386, 414, 454-495, 644)."""

    def __init__(self, **kwargs):
        self.batch_size = int(kwargs.pop("batch_size", 1))
        self.max_batch_size = int(kwargs.pop("max_batch_size", self.batch_size))
        self.seq_len = int(kwargs.pop("seq_len", 640))
        self.max_length = int(kwargs.pop("max_length", self.seq_len))
        self.max_context_length = int(kwargs.pop("max_context_length", self.seq_len))
        self.max_new_tokens = kwargs.pop("max_new_tokens", None)
        self.pad_token_id = kwargs.pop("pad_token_id", 0)
        dt = kwargs.pop("torch_dtype", torch.bfloat16)
        if isinstance(dt, str):
            dt = getattr(torch, dt.replace("torch.", ""))
        if dt != torch.bfloat16:
            raise ValueError("this build computes in bfloat16 (torch_dtype must be bfloat16)")
        self.torch_dtype = dt
        self.tp_degree = int(kwargs.pop("tp_degree", 1))
        if self.tp_degree != 1:
            raise ValueError("this build runs on one GPU: tp_degree must be 1")
        self.on_device_sampling_config = kwargs.pop("on_device_sampling_config", None)
        self.enable_fused_speculation = False
        # prompt-lookup speculation: candidates + 1 tokens verified per step
        # (the reference ships 5, qwen_with_nki.py:74); 0 or 1 = plain greedy
        self.speculation_length = int(kwargs.pop("speculation_length", 0))
        self.use_hip_graphs = bool(kwargs.pop("use_hip_graphs", True))
        self.seed = int(kwargs.pop("seed", 0))
        self.extra = kwargs  # every other generate-mode flag, accepted and ignored


class Qwen3MoeInferenceConfig:
    """Model config.  ``load_config`` is a callable that sets attributes on the
    config (``load_pretrained_config(path)``); without it the Qwen3-30B-A3B
    shape is used.  Applies the reference's fixed semantics:
    ``num_local_experts = num_experts``, no shared experts, fp32 softmax router,
    top-k renormalisation (qwen_with_nki.py:9803-9894)."""

    REQUIRED = [
        "head_dim", "hidden_act", "hidden_size", "max_position_embeddings", "moe_intermediate_size",
        "norm_topk_prob", "num_attention_heads", "num_experts", "num_experts_per_tok",
        "num_hidden_layers", "num_key_value_heads", "rms_norm_eps", "rope_theta",
        "tie_word_embeddings", "vocab_size",
    ]  # qwen.py:294-310

    def __init__(self, neuron_config: MoENeuronConfig, load_config: Optional[Callable] = None, **kw):
        self.neuron_config = neuron_config
        for k, v in Qwen3MoeShape().to_dict().items():
            setattr(self, k, v)
        if load_config is not None:
            load_config(self)
        for k, v in kw.items():
            setattr(self, k, v)
        missing = [a for a in self.REQUIRED if not hasattr(self, a)]
        if missing:
            raise ValueError(f"config is missing {missing}")
        if getattr(self, "hidden_act", "silu") != "silu":
            raise ValueError("only SwiGLU (silu) experts are supported")
        self.num_local_experts = self.num_experts
        self.n_shared_experts = 0
        self.intermediate_size = self.moe_intermediate_size
        self.router_dtype = torch.float32
        self.router_act_fn = "softmax"
        self.normalize_top_k_affinities = True

    def shape(self) -> Qwen3MoeShape:
        return Qwen3MoeShape(**{k: getattr(self, k) for k in Qwen3MoeShape().to_dict()})


def load_pretrained_config(model_path: str) -> Callable:
    """``config.json`` of a local HF checkpoint -> attribute setter (main.py:389)."""

    def _load(cfg):
        with open(os.path.join(model_path, "config.json")) as f:
            d = json.load(f)
        rp = d.get("rope_parameters") or {}
        if "rope_theta" not in d and "rope_theta" in rp:
            d["rope_theta"] = rp["rope_theta"]
        for k, v in d.items():
            setattr(cfg, k, v)

    return _load


# ============================================================================ layers
class RMSNormWeight:
    """Holds an RMSNorm weight; the normalisation itself runs in the kernels
    (fp32 upcast -> normalise -> x weight -> one cast, qwen_with_nki.py:1372-1384)."""

    def __init__(self, weight: torch.Tensor, eps: float):
        self.weight, self.eps = weight, eps


class NeuronQwen3MoeDecoderLayer:
    """``h = x + Attn(RMSNorm_in(x)); out = h + MoE(RMSNorm_post(h))``
    (qwen_with_nki.py:10155-10213).  The residual stream is fp32; both
    residual adds are fused into kernel epilogues."""

    def __init__(self, config: Qwen3MoeInferenceConfig, layer_idx: int, w: Dict[str, torch.Tensor]):
        c = config
        self.layer_idx = layer_idx
        self.input_layernorm = RMSNormWeight(w["input_layernorm"], c.rms_norm_eps)
        self.post_attention_layernorm = RMSNormWeight(w["post_attention_layernorm"], c.rms_norm_eps)
        self.self_attn = Attention(w["wqkv"], w["q_norm"], w["k_norm"], w["wo"], c.num_attention_heads,
                                   c.num_key_value_heads, c.head_dim, c.rms_norm_eps)
        self.mlp = MoEBlock(w["router"], w["w13"], w["w2"], c.num_experts_per_tok)
        self.cache: Optional[KVCache] = None

    def run(self, h: torch.Tensor, positions: torch.Tensor, B: int, S: int, rope, start=0,
            ctx_len: Optional[torch.Tensor] = None, max_ctx: Optional[int] = None) -> torch.Tensor:
        """In-place layer on the fp32 residual ``h[B*S, H]``."""
        eps = self.input_layernorm.eps
        if B * S == 1 and ops.qkv_norm_rope_workspace(1, h.shape[1], self.self_attn.n_q, self.self_attn.n_kv,
                                                      self.self_attn.head_dim) > 0:
            # one-token step: the input RMSNorm runs inside the QKV GEMV's staging
            self.self_attn.forward(h, h, positions, B, S, self.cache, rope[0], rope[1], start, ctx_len, max_ctx,
                                   norm=(self.input_layernorm.weight, eps))
        else:
            x = ops.rmsnorm_residual(h, self.input_layernorm.weight, eps)
            self.self_attn.forward(x, h, positions, B, S, self.cache, rope[0], rope[1], start, ctx_len, max_ctx)
        self.mlp.forward_normed(h, self.post_attention_layernorm.weight, eps, residual=h, out=h)
        return h

    def forward(self, hidden_states: torch.Tensor, attention_mask=None, position_ids=None,
                past_key_value=None, padding_mask=None, rope=None, **kwargs):
        """Reference layer contract: ``hidden_states[B,S,H]`` -> ``(hidden_states,
        present_key_value, cos_cache, sin_cache, None)``; the KV cache is the
        layer's contiguous cache (or ``past_key_value`` = a :class:`KVCache`)."""
        B, S, H = hidden_states.shape
        if past_key_value is not None:
            self.cache = past_key_value
        if position_ids is None:
            position_ids = torch.arange(S, device=hidden_states.device).expand(B, S)
        pos = position_ids.to(torch.int32).reshape(-1).contiguous()
        start = int(position_ids[0, 0])
        h = hidden_states.float().reshape(B * S, H).contiguous()
        self.run(h, pos, B, S, rope, start)
        out = h.view(B, S, H).to(hidden_states.dtype)
        return out, self.cache, rope[0], rope[1], None


class NeuronQwen3MoeModel:
    """Embedding -> layers -> final norm -> lm_head (qwen_with_nki.py:10246-10292)."""

    def __init__(self, config: Qwen3MoeInferenceConfig, params: Dict[str, Any]):
        self.config = config
        self.embed_tokens = params["embed_tokens"]
        self.layers = [NeuronQwen3MoeDecoderLayer(config, i, lw) for i, lw in enumerate(params["layers"])]
        self.norm = RMSNormWeight(params["norm"], config.rms_norm_eps)
        self.lm_head = params["lm_head"]
        dev = self.embed_tokens.device
        max_pos = min(int(config.max_position_embeddings), int(config.neuron_config.max_length) + 1)
        self.rope = rope_tables(config.head_dim, max_pos, float(config.rope_theta), dev)
        # set by the embedding gather when a token id is outside the vocabulary
        self.embed_err = torch.zeros(1, dtype=torch.int32, device=dev)

    def allocate_cache(self, B: int, S_max: int):
        c = self.config
        for l in self.layers:
            l.cache = KVCache(B, c.num_key_value_heads, S_max, c.head_dim, self.embed_tokens.device)

    def hidden(self, input_ids: torch.Tensor, positions: torch.Tensor, B: int, S: int, start,
               ctx_len: Optional[torch.Tensor] = None, h_buf: Optional[torch.Tensor] = None,
               max_ctx: Optional[int] = None) -> torch.Tensor:
        """fp32 final hidden states ``[B*S, H]`` (before the final norm)."""
        h = ops.embed(input_ids.reshape(-1).long(), self.embed_tokens, out=h_buf, err=self.embed_err)
        for layer in self.layers:
            layer.run(h, positions, B, S, self.rope, start, ctx_len, max_ctx)
        return h

    def check_embed(self) -> None:
        """Raise if any token id so far was outside the vocabulary (synchronises)."""
        if int(self.embed_err.item()):
            self.embed_err.zero_()
            raise ValueError("token id outside [0, vocab_size) reached the embedding")

    def logits(self, h_last: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Final RMSNorm + lm_head (fp32 accumulation) on rows ``h_last[n, H]``."""
        y = ops.rmsnorm_residual(h_last, self.norm.weight, self.norm.eps)
        return ops.gemm(y, self.lm_head, _lib.GEMM_STORE_F32, out=out)


def random_params(config: Qwen3MoeInferenceConfig, device, seed: int = 0, std: float = 0.02) -> Dict[str, Any]:
    """Random-init bf16 weights of the model, generated on the GPU from ``seed``
    (N(0, std) matrices; RMSNorm weights 1)."""
    c = config
    g = torch.Generator(device=device).manual_seed(seed)
    H, D, E, I = c.hidden_size, c.head_dim, c.num_experts, c.moe_intermediate_size
    nq, nkv = c.num_attention_heads, c.num_key_value_heads

    def rnd(*shape):
        return torch.empty(*shape, dtype=torch.bfloat16, device=device).normal_(0.0, std, generator=g)

    def ones(n):
        return torch.ones(n, dtype=torch.bfloat16, device=device)

    layers = []
    for _ in range(c.num_hidden_layers):
        layers.append({
            "input_layernorm": ones(H), "post_attention_layernorm": ones(H),
            "wqkv": rnd((nq + 2 * nkv) * D, H), "q_norm": ones(D), "k_norm": ones(D),
            "wo": rnd(H, nq * D), "router": rnd(E, H),
            "w13": rnd(E, 2 * I, H), "w2": rnd(E, I // 8, H, 8),
        })
    return {"embed_tokens": rnd(c.vocab_size, H), "layers": layers, "norm": ones(H),
            "lm_head": rnd(c.vocab_size, H)}


def convert_qwen3_moe_hf_to_neuron_state_dict(state_dict: Dict[str, torch.Tensor],
                                               config: Qwen3MoeInferenceConfig) -> Dict[str, Any]:
    """HF checkpoint tensors -> this build's parameter tree.

    Same key mapping as convert_qwen3_moe_hf_to_neuron_state_dict
    (qwen_with_nki.py:8883-8997): q/k/v concatenated (8845-8862), q_norm/k_norm,
    router from ``mlp.gate.weight`` (8915-8919), per-expert gate/up/down packed
    (8928-8990) -- here into the gate/up-interleaved ``w13 [E,2I,H]`` and
    blocked ``w2 [E,I/8,H,8]`` layouts.  Accepts keys with or without the ``model.`` prefix.
    """
    sd = {k[len("model."):] if k.startswith("model.") else k: v for k, v in state_dict.items()}
    bf = lambda t: t.to(torch.bfloat16).contiguous()
    layers = []
    for l in range(config.num_hidden_layers):
        p = f"layers.{l}."
        E = config.num_experts
        w13, w2 = weights.from_hf_experts(
            [sd[f"{p}mlp.experts.{e}.gate_proj.weight"].float() for e in range(E)],
            [sd[f"{p}mlp.experts.{e}.up_proj.weight"].float() for e in range(E)],
            [sd[f"{p}mlp.experts.{e}.down_proj.weight"].float() for e in range(E)],
        )
        layers.append({
            "input_layernorm": bf(sd[f"{p}input_layernorm.weight"]),
            "post_attention_layernorm": bf(sd[f"{p}post_attention_layernorm.weight"]),
            "wqkv": bf(torch.cat([sd[f"{p}self_attn.q_proj.weight"], sd[f"{p}self_attn.k_proj.weight"],
                                  sd[f"{p}self_attn.v_proj.weight"]])),
            "q_norm": bf(sd[f"{p}self_attn.q_norm.weight"]), "k_norm": bf(sd[f"{p}self_attn.k_norm.weight"]),
            "wo": bf(sd[f"{p}self_attn.o_proj.weight"]), "router": bf(sd[f"{p}mlp.gate.weight"]),
            "w13": bf(w13), "w2": bf(w2),
        })
    lm = sd.get("lm_head.weight", state_dict.get("lm_head.weight"))
    if lm is None and getattr(config, "tie_word_embeddings", False):
        lm = sd["embed_tokens.weight"]
    return {"embed_tokens": bf(sd["embed_tokens.weight"]), "layers": layers, "norm": bf(sd["norm.weight"]),
            "lm_head": bf(lm)}


# ============================================================================ causal LM
@dataclass
class CausalLMOutput:
    logits: torch.Tensor  # [B, V] fp32 (last position)


class NeuronQwen3MoeForCausalLM:
    """Drop-in for the reference's model class (qwen_with_nki.py:10687-10971)."""

    _model_cls = NeuronQwen3MoeModel

    def __init__(self, model_path: Optional[str], config: Optional[Qwen3MoeInferenceConfig] = None):
        if config is None:
            config = Qwen3MoeInferenceConfig(MoENeuronConfig(), load_pretrained_config(model_path))
        self.model_path = model_path
        self.config = config
        self.neuron_config = config.neuron_config
        self.on_device_sampling = config.neuron_config.on_device_sampling_config is not None
        self.model: Optional[NeuronQwen3MoeModel] = None
        self.device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else None
        self._graphs: Dict[Any, Any] = {}
        self.position = 0

    # -- class surface --------------------------------------------------------
    @classmethod
    def get_neuron_config_cls(cls):
        return MoENeuronConfig

    @classmethod
    def get_config_cls(cls):
        return Qwen3MoeInferenceConfig

    @staticmethod
    def load_hf_model(model_path, **kwargs):
        raise RuntimeError("load_hf_model needs the transformers reference model; use load() with a local "
                           "checkpoint directory instead (no downloads are made)")

    @staticmethod
    def convert_hf_to_neuron_state_dict(state_dict, config):
        return convert_qwen3_moe_hf_to_neuron_state_dict(state_dict, config)

    def compile(self, compiled_model_path: Optional[str] = None, debug: bool = False):
        """No graph compiler here: record the resolved config next to the
        artefacts (kernels are prebuilt; decode steps are captured into HIP
        graphs on first use)."""
        _lib.lib()
        if compiled_model_path:
            os.makedirs(compiled_model_path, exist_ok=True)
            d = {k: v for k, v in vars(self.config).items() if isinstance(v, (int, float, str, bool))}
            with open(os.path.join(compiled_model_path, "qmoe_config.json"), "w") as f:
                json.dump(d, f, indent=1)

    def load(self, compiled_model_path: Optional[str] = None, params: Optional[Dict[str, Any]] = None):
        """Materialise the weights on the GPU and allocate the KV cache.  Uses
        ``params`` if given, else safetensors shards under ``model_path``, else
        seeded random-init weights (``neuron_config.seed``)."""
        if self.device is None:
            raise RuntimeError("no GPU visible: this model runs only on an MI355X")
        if params is None:
            params = self._load_params()
        self.model = self._model_cls(self.config, params)
        self.model.allocate_cache(self.neuron_config.max_batch_size, int(self.neuron_config.max_length) + 1)
        self.reset()

    def _load_params(self):
        path = self.model_path
        if path and os.path.isdir(path) and any(f.endswith(".safetensors") for f in os.listdir(path)):
            from safetensors.torch import load_file

            sd = {}
            for f in sorted(os.listdir(path)):
                if f.endswith(".safetensors"):
                    sd.update(load_file(os.path.join(path, f), device="cpu"))
            params = convert_qwen3_moe_hf_to_neuron_state_dict(sd, self.config)
            return _to_device(params, self.device)
        return random_params(self.config, self.device, seed=self.neuron_config.seed)

    def reset(self):
        """Start a new sequence (the KV cache is overwritten from position 0)."""
        self.position = 0

    # -- forward ---------------------------------------------------------------
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Context encoding of ``input_ids[B,S]`` at positions 0..S-1; returns
        last-position logits ``[B, V]`` (fp32)."""
        B, S = input_ids.shape
        dev = self.device
        pos = torch.arange(S, device=dev, dtype=torch.int32).repeat(B)
        h = self.model.hidden(input_ids.to(dev), pos, B, S, 0)
        last = h.view(B, S, -1)[:, -1].contiguous()
        self.position = S
        return self.model.logits(last)

    def decode_step(self, token_ids: torch.Tensor) -> torch.Tensor:
        """One token per sequence at the current position; returns ``[B, V]`` logits."""
        B = token_ids.shape[0]
        dev = self.device
        pos = torch.full((B,), self.position, device=dev, dtype=torch.int32)
        h = self.model.hidden(token_ids.to(dev).view(B, 1), pos, B, 1, self.position)
        self.position += 1
        return self.model.logits(h)

    def forward(self, input_ids: torch.Tensor, attention_mask=None, position_ids=None, **kw) -> CausalLMOutput:
        if input_ids.shape[1] > 1 or self.position == 0:
            return CausalLMOutput(self.prefill(input_ids))
        return CausalLMOutput(self.decode_step(input_ids[:, -1]))

    __call__ = forward

    # -- greedy decode with a captured step --------------------------------------
    def greedy_decode(self, first_token: torch.Tensor, n_steps: int, use_graph: Optional[bool] = None) -> torch.Tensor:
        """``n_steps`` greedy tokens after ``first_token[B]``; with a HIP graph
        the whole step (embedding, 48 layers, lm_head, argmax, position += 1)
        is one replay.  Returns ``[B, n_steps]`` token ids."""
        use_graph = self.neuron_config.use_hip_graphs if use_graph is None else use_graph
        B = first_token.shape[0]
        if not use_graph:
            toks, cur = [], first_token.to(self.device)
            for _ in range(n_steps):
                cur = ops.argmax(self.decode_step(cur))
                toks.append(cur)
            self.model.check_embed()
            return torch.stack(toks, dim=1)
        st = self._decode_state(B)
        st["tok"].copy_(first_token.to(self.device).view(B).long())
        st["pos"].fill_(self.position)
        out = torch.empty(B, n_steps, dtype=torch.long, device=self.device)
        for i in range(n_steps):
            self._decode_graph(B, self._bucket(self.position + i + 1)).replay()
            out[:, i].copy_(st["tok"])
        self.position += n_steps
        self.model.check_embed()
        return out

    # Decode graphs, one per (batch, context bucket): the attention launch of a
    # bucket covers cache rows [0, bucket) only.  Buckets double from 256 up to
    # the cache capacity.
    DECODE_BUCKET_MIN = 256

    def _bucket(self, ctx: int) -> int:
        cap = self.model.layers[0].cache.capacity
        b = self.DECODE_BUCKET_MIN
        while b < ctx and b < cap:
            b *= 2
        return min(b, cap)

    def _decode_state(self, B: int):
        """Step buffers shared by every bucket's graph of batch ``B``."""
        st = self._graphs.get(("state", B))
        if st is None:
            dev = self.device
            st = {"tok": torch.zeros(B, dtype=torch.long, device=dev),
                  "pos": torch.zeros(B, dtype=torch.int32, device=dev),
                  "h": torch.empty(B, self.config.hidden_size, device=dev),
                  "logits": torch.empty(B, self.config.vocab_size, device=dev),
                  "am_ws": ops.argmax_workspace(B, dev)}
            self._graphs[("state", B)] = st
        return st

    def _decode_graph(self, B: int, bucket: int):
        key = ("decode", B, bucket)
        g = self._graphs.get(key)
        if g is not None:
            return g
        m, st = self.model, self._decode_state(B)

        # Every op of the step is a library kernel or an elementwise torch op:
        # no reduction that records a memset into the graph (torch's argmax
        # over a 151,936-wide row would), so replays stay correct.
        def step():
            ctx = st["pos"] + 1
            h = m.hidden(st["tok"].view(B, 1), st["pos"], B, 1, 0, ctx_len=ctx, h_buf=st["h"], max_ctx=bucket)
            m.logits(h, out=st["logits"])
            ops.argmax(st["logits"], out=st["tok"], workspace=st["am_ws"])
            st["pos"].add_(1)

        # Warm-up on a side stream (allocations, lazily created workspaces), then
        # capture.  The warm-up writes one K/V cache slot: the slot at the
        # current step position, which the next real step overwrites.
        saved = (st["tok"].clone(), st["pos"].clone())
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        st["tok"].copy_(saved[0])
        st["pos"].copy_(saved[1])
        torch.cuda.synchronize()
        self._graphs[key] = g
        return g

    # -- prompt-lookup speculative decoding ---------------------------------------
    def spec_generate(self, prompt: torch.Tensor, max_new_tokens: int, spec_len: int = 5,
                      ngram: int = 4, ngram_min: int = 1, strategy: str = "majority1"):
        """Greedy generation with prompt-lookup speculation (batch 1): each
        step proposes up to ``spec_len - 1`` tokens from n-gram matches in the
        tokens so far, verifies ``[last, candidates]`` in one ``spec_len``-token
        pass (a captured graph) and keeps the candidates that agree with the
        model's greedy choice plus the model's next token; with no match it
        runs the one-token decode step.  Restates ``_spec_generate``
        (qwen_with_nki.py:575-1211) without its adaptive gating and tracing.
        Returns (tokens ``[1, T0 + max_new_tokens]``, stats dict)."""
        from . import speculative

        if prompt.dim() != 2 or prompt.shape[0] != 1:
            raise ValueError("spec_generate takes one prompt [1, T0]")
        if spec_len < 2:
            raise ValueError("spec_len must be at least 2")
        T0 = prompt.shape[1]
        cap = self.model.layers[0].cache.capacity
        if T0 + max_new_tokens > cap:
            raise ValueError(f"prompt + new tokens ({T0}+{max_new_tokens}) exceed the cache ({cap})")
        self.reset()
        seq = prompt[0].tolist()
        if max_new_tokens <= 0:
            return prompt.clone(), {"steps": 0, "verify_steps": 0, "accepted": 0}
        first = int(self.prefill(prompt).argmax(-1)[0])
        seq.append(first)
        stats = {"steps": 0, "verify_steps": 0, "accepted": 0}
        k = spec_len - 1
        while len(seq) - T0 < max_new_tokens:
            last = seq[-1]
            cand, _ = speculative.prompt_lookup(seq, k, ngram, ngram_min, strategy)
            room = max_new_tokens - (len(seq) - T0)
            cand = cand[: max(0, room - 1)]
            stats["steps"] += 1
            if cand and self.position + spec_len <= cap:
                st = self._verify_graph(spec_len)
                toks = [last] + speculative.pad_candidates(cand, k)
                st["tok"].copy_(torch.tensor(toks, dtype=torch.long))
                st["pos"].copy_(torch.arange(self.position, self.position + spec_len, dtype=torch.int32))
                st["start"].fill_(self.position)
                st["graph"].replay()
                target = st["out"].tolist()
                m, emitted = speculative.accept(cand, target)
                stats["verify_steps"] += 1
                stats["accepted"] += m
                self.position += m + 1  # cache rows of last and the accepted candidates are final
                seq.extend(emitted)
            else:
                nxt = self.greedy_decode(torch.tensor([last], device=self.device), 1)
                seq.append(int(nxt[0, 0]))
        self.model.check_embed()
        out = torch.tensor(seq[: T0 + max_new_tokens], dtype=torch.long).view(1, -1)
        return out, stats

    def _verify_graph(self, S: int):
        """Captured ``S``-token pass at a device-resident position (batch 1):
        embedding, 48 layers (attention over the cache with the chunk start read
        on the device), final norm + lm_head for all S rows, per-row argmax."""
        key = ("verify", S)
        st = self._graphs.get(key)
        if st is not None:
            return st
        dev, m = self.device, self.model
        st = {"tok": torch.zeros(S, dtype=torch.long, device=dev),
              "pos": torch.zeros(S, dtype=torch.int32, device=dev),
              "start": torch.zeros(1, dtype=torch.int32, device=dev),
              "h": torch.empty(S, self.config.hidden_size, device=dev),
              "logits": torch.empty(S, self.config.vocab_size, device=dev),
              "out": torch.zeros(S, dtype=torch.long, device=dev),
              "am_ws": ops.argmax_workspace(S, dev)}

        def step():
            h = m.hidden(st["tok"].view(1, S), st["pos"], 1, S, st["start"], h_buf=st["h"])
            m.logits(h, out=st["logits"])
            ops.argmax(st["logits"], out=st["out"], workspace=st["am_ws"])

        # warm-up and capture write cache rows [position, position + S): rows the
        # first real verification at this position overwrites
        st["pos"].copy_(torch.arange(self.position, self.position + S, dtype=torch.int32))
        st["start"].fill_(self.position)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
        st["graph"] = g
        self._graphs[key] = st
        return st



def _to_device(params, device):
    if isinstance(params, torch.Tensor):
        return params.to(device)
    if isinstance(params, dict):
        return {k: _to_device(v, device) for k, v in params.items()}
    if isinstance(params, list):
        return [_to_device(v, device) for v in params]
    return params


# ============================================================================ generation
class HuggingFaceGenerationAdapter:
    """``generate`` for :class:`NeuronQwen3MoeForCausalLM` (main.py:503,
    557-569, 638-645).  Greedy decoding (``do_sample`` must be false; the
    reference's sampling defaults are a decoding policy outside this path)."""

    def __init__(self, model: NeuronQwen3MoeForCausalLM):
        self.model = model

    def generate(self, input_ids: torch.Tensor, attention_mask=None, generation_config=None,
                 max_length: Optional[int] = None, max_new_tokens: Optional[int] = None,
                 **kw) -> torch.Tensor:
        m = self.model
        if generation_config is not None and getattr(generation_config, "do_sample", False):
            raise ValueError("only greedy decoding is implemented (set do_sample=False)")
        B, S = input_ids.shape
        if max_new_tokens is None:
            limit = max_length if max_length is not None else m.neuron_config.max_length
            max_new_tokens = max(0, int(limit) - S)
        if S + max_new_tokens > m.neuron_config.max_length + 1:
            raise ValueError(f"prompt + new tokens ({S}+{max_new_tokens}) exceed max_length "
                             f"{m.neuron_config.max_length}")
        spec = int(getattr(m.neuron_config, "speculation_length", 0))
        if spec >= 2 and B == 1 and max_new_tokens > 1:
            out, _ = m.spec_generate(input_ids, max_new_tokens, spec_len=spec)
            return out.to(m.device)
        m.reset()
        logits = m.prefill(input_ids)
        first = logits.argmax(dim=-1)
        if max_new_tokens <= 1:
            new = first.view(B, -1)[:, :max_new_tokens]
        else:
            rest = m.greedy_decode(first, max_new_tokens - 1)
            new = torch.cat([first.view(B, 1), rest], dim=1)
        return torch.cat([input_ids.to(new.device), new], dim=1)
