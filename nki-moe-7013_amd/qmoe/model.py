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
from collections.abc import Mapping
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
            raise ValueError("qmoe computes in bfloat16 (torch_dtype must be bfloat16)")
        self.torch_dtype = dt
        self.tp_degree = int(kwargs.pop("tp_degree", 1))
        if self.tp_degree != 1:
            raise ValueError("qmoe runs on one GPU: tp_degree must be 1")
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
    residual adds are fused into kernel epilogues.

    ``NeuronQwen3MoeDecoderLayer(config, layer_idx)`` builds the layer with
    seeded random-init weights on the current GPU, as the reference's
    constructor (10113-10153) creates its own parameters; pass ``w`` (one
    layer of :func:`random_params` or of the checkpoint converter) to use
    given weights."""

    def __init__(self, config: Qwen3MoeInferenceConfig, layer_idx: int,
                 w: Optional[Dict[str, torch.Tensor]] = None):
        c = config
        if w is None:
            if not torch.cuda.is_available():
                raise RuntimeError("no GPU visible: this layer runs only on an MI355X")
            dev = torch.device("cuda", torch.cuda.current_device())
            seed = int(getattr(c.neuron_config, "seed", 0)) * 1000003 + int(layer_idx)
            w = random_layer_params(c, dev, torch.Generator(device=dev).manual_seed(seed))
        self.config = c
        self.layer_idx = layer_idx
        self.hidden_size = c.hidden_size
        self.input_layernorm = RMSNormWeight(w["input_layernorm"], c.rms_norm_eps)
        self.post_attention_layernorm = RMSNormWeight(w["post_attention_layernorm"], c.rms_norm_eps)
        self.self_attn = Attention(w["wqkv"], w["q_norm"], w["k_norm"], w["wo"], c.num_attention_heads,
                                   c.num_key_value_heads, c.head_dim, c.rms_norm_eps)
        self.mlp = MoEBlock(w["router"], w["w13"], w["w2"], c.num_experts_per_tok)
        self.cache: Optional[KVCache] = None
        self._rope = None  # (cos, sin) built from head_dim / rope_theta on first use

    def run(self, h: torch.Tensor, positions: torch.Tensor, B: int, S: int, rope, start=0,
            max_ctx: Optional[int] = None, x_in: Optional[torch.Tensor] = None,
            next_norm: Optional[tuple] = None) -> Optional[torch.Tensor]:
        """In-place layer on the fp32 residual ``h[B*S, H]``.

        Above the decode-block size the RMSNorms ride on the launches that
        finish their input rows: the post-attention norm on the o_proj's
        residual add, and, with ``next_norm = (rms_w, eps)`` (the next layer's
        input norm), that norm on the MoE combine; the latter's bf16 rows are
        returned for the next layer's ``x_in`` (the bits of a separate
        ``rmsnorm_residual``).  Otherwise returns None."""
        eps = self.input_layernorm.eps
        if B * S == 1 and ops.qkv_norm_rope_workspace(1, h.shape[1], self.self_attn.n_q, self.self_attn.n_kv,
                                                      self.self_attn.head_dim) > 0:
            # one-token step: the input RMSNorm runs inside the QKV GEMV's staging
            self.self_attn.forward(h, h, positions, B, S, self.cache, rope[0], rope[1], start, max_ctx,
                                   norm=(self.input_layernorm.weight, eps))
            self.mlp.forward_normed(h, self.post_attention_layernorm.weight, eps, residual=h, out=h)
            return None
        x = x_in if x_in is not None else ops.rmsnorm_residual(h, self.input_layernorm.weight, eps)
        if B * S <= ops.DECODE_BLOCK_MAX_T:
            self.self_attn.forward(x, h, positions, B, S, self.cache, rope[0], rope[1], start, max_ctx)
            self.mlp.forward_normed(h, self.post_attention_layernorm.weight, eps, residual=h, out=h)
            return None
        x2 = self.self_attn.forward(x, h, positions, B, S, self.cache, rope[0], rope[1], start, max_ctx,
                                    post_norm=(self.post_attention_layernorm.weight, eps))
        if next_norm is None:
            self.mlp.forward(x2, residual=h, out=h)
            return None
        return self.mlp.forward(x2, residual=h, out=h, norm=next_norm)[1]

    def rope_tables(self, n_pos: int, device):
        """cos/sin tables covering positions ``[0, n_pos)`` from the config's
        head_dim and rope_theta (the reference's ``RotaryEmbedding``,
        qwen_with_nki.py:10083-10087); grown in powers of two when needed."""
        c = self.config
        limit = int(getattr(c, "max_position_embeddings", n_pos))
        if n_pos > limit:
            raise ValueError(f"position {n_pos - 1} is beyond max_position_embeddings={limit}")
        if self._rope is None or self._rope[0].shape[0] < n_pos or self._rope[0].device != device:
            size = min(limit, max(256, 1 << (int(n_pos) - 1).bit_length()))
            self._rope = rope_tables(c.head_dim, size, float(c.rope_theta), device)
        return self._rope

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                position_ids: Optional[torch.Tensor] = None, past_key_value=None, padding_mask=None,
                rope=None, **kwargs):
        """The reference layer contract (qwen_with_nki.py:10155-10213):
        ``hidden_states[B, S, H]`` -> ``(hidden_states, present_key_value,
        cos_cache, sin_cache, None)``.

        * ``position_ids[B, S]`` (default ``0..S-1``): row b holds consecutive
          positions; a chunk with S > 1 starts at the same position in every
          row; position == cache index.
        * ``past_key_value``: a :class:`KVCache` or a ``(K, V)`` pair of bf16
          ``[B, Hkv, S_max, D]`` tensors, updated in place.  Without it the
          layer keeps its own cache, allocated on first use with room for
          ``neuron_config.max_length + 1`` positions (reallocated by a chunk
          that starts at position 0 and does not fit).
        * ``attention_mask``: attention is causal over cache rows
          ``[0, position]``; a mask is accepted when it says exactly that or
          marks right padding (``[B, L]`` of 1s then 0s: rows past a
          sequence's end only affect those rows' own outputs).  Any other mask
          is rejected.
        * ``rope``: optional ``(cos, sin)`` tables; by default the layer builds
          them from ``head_dim`` and ``rope_theta``.

        Returns ``hidden_states`` in the input dtype; ``present_key_value`` is
        the cache, which unpacks as ``(K, V)``."""
        if hidden_states.dim() != 3 or hidden_states.shape[2] != self.hidden_size:
            raise ValueError(f"hidden_states must be [B, S, {self.hidden_size}]")
        if not hidden_states.is_cuda:
            raise ValueError("hidden_states must be on the GPU")
        B, S, H = hidden_states.shape
        dev = hidden_states.device
        if position_ids is None:
            position_ids = torch.arange(S, device=dev).expand(B, S)
        if position_ids.shape != (B, S):
            raise ValueError(f"position_ids must be [{B}, {S}]")
        pos_cpu = position_ids.detach().to("cpu", torch.int64)
        if bool((pos_cpu < 0).any()):
            raise ValueError("position_ids must be non-negative")
        if S > 1 and not torch.equal(pos_cpu, pos_cpu[:1, :1] + torch.arange(S).expand(B, S)):
            raise ValueError("a chunk of S > 1 tokens needs positions start..start+S-1, the same in every row")
        starts = pos_cpu[:, 0]
        _check_causal_mask(attention_mask, pos_cpu)
        end = int(pos_cpu.max()) + 1
        if past_key_value is not None:
            self.cache = KVCache.wrap(past_key_value)
        elif (self.cache is None or self.cache.k.shape[0] != B or self.cache.capacity < end) and int(starts.min()) == 0:
            cap = max(end, int(self.config.neuron_config.max_length) + 1)
            self.cache = KVCache(B, self.config.num_key_value_heads, cap, self.config.head_dim, dev)
        if self.cache is None or self.cache.k.shape[0] != B:
            raise ValueError("no KV cache for this batch: start at position 0 or pass past_key_value")
        if self.cache.capacity < end:
            raise ValueError(f"position {end - 1} is beyond the KV cache capacity {self.cache.capacity}")
        if rope is None:
            rope = self.rope_tables(end, dev)
        pos = position_ids.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
        # the layer runs in place on its fp32 residual stream: always a copy,
        # never the caller's tensor (an fp32 input would otherwise be overwritten)
        h = hidden_states.reshape(B * S, H).to(torch.float32, copy=True).contiguous()
        if S > 1:
            self.run(h, pos, B, S, rope, int(starts[0]))
        else:
            self.run(h, pos, B, 1, rope, 0)
        out = h.view(B, S, H).to(hidden_states.dtype)
        return out, self.cache, rope[0], rope[1], None


def _check_causal_mask(mask: Optional[torch.Tensor], pos: torch.Tensor) -> None:
    """Accept ``None`` or a 2-D 0/1 mask ``[B, L]`` that is 1 up to a
    sequence's length and 0 after it (right padding, main.py:366) and that
    covers every query position; anything else would ask for attention the
    causal cache kernels do not compute."""
    if mask is None:
        return
    m = mask.detach().to("cpu")
    B = pos.shape[0]
    if m.dim() != 2 or m.shape[0] != B:
        raise ValueError("attention_mask must be None or [B, L] (right padding); "
                         "attention here is causal over the contiguous KV cache")
    m = m.to(torch.int64)
    if not bool(((m == 0) | (m == 1)).all()):
        raise ValueError("attention_mask must hold 0/1")
    lengths = m.sum(1)
    prefix = torch.arange(m.shape[1]).expand_as(m) < lengths.unsqueeze(1)
    if not torch.equal(m.bool(), prefix):
        raise ValueError("attention_mask must be right-padded (1s then 0s); "
                         "other masks are not supported by the causal cache kernels")


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
               h_buf: Optional[torch.Tensor] = None, max_ctx: Optional[int] = None) -> torch.Tensor:
        """fp32 final hidden states ``[B*S, H]`` (before the final norm)."""
        h = ops.embed(input_ids.reshape(-1).long(), self.embed_tokens, out=h_buf, err=self.embed_err)
        x = None  # the next layer's normed input rows, when the previous layer produced them
        for i, layer in enumerate(self.layers):
            nxt = self.layers[i + 1].input_layernorm if i + 1 < len(self.layers) else None
            x = layer.run(h, positions, B, S, self.rope, start, max_ctx, x_in=x,
                          next_norm=None if nxt is None else (nxt.weight, nxt.eps))
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


def random_layer_params(config: Qwen3MoeInferenceConfig, device, g: torch.Generator,
                        std: float = 0.02) -> Dict[str, torch.Tensor]:
    """One decoder layer of random-init bf16 weights drawn from ``g`` on the
    GPU (N(0, std) matrices; RMSNorm weights 1)."""
    c = config
    H, D, E, I = c.hidden_size, c.head_dim, c.num_experts, c.moe_intermediate_size
    nq, nkv = c.num_attention_heads, c.num_key_value_heads

    def rnd(*shape):
        return torch.empty(*shape, dtype=torch.bfloat16, device=device).normal_(0.0, std, generator=g)

    def ones(n):
        return torch.ones(n, dtype=torch.bfloat16, device=device)

    return {
        "input_layernorm": ones(H), "post_attention_layernorm": ones(H),
        "wqkv": rnd((nq + 2 * nkv) * D, H), "q_norm": ones(D), "k_norm": ones(D),
        "wo": rnd(H, nq * D), "router": rnd(E, H),
        "w13": rnd(E, 2 * I, H), "w2": rnd(E, I // 8, H, 8),
    }


def random_params(config: Qwen3MoeInferenceConfig, device, seed: int = 0, std: float = 0.02) -> Dict[str, Any]:
    """Random-init bf16 weights of the model, generated on the GPU from ``seed``
    (N(0, std) matrices; RMSNorm weights 1)."""
    c = config
    g = torch.Generator(device=device).manual_seed(seed)
    H = c.hidden_size

    def rnd(*shape):
        return torch.empty(*shape, dtype=torch.bfloat16, device=device).normal_(0.0, std, generator=g)

    layers = [random_layer_params(c, device, g, std) for _ in range(c.num_hidden_layers)]
    return {"embed_tokens": rnd(c.vocab_size, H), "layers": layers,
            "norm": torch.ones(H, dtype=torch.bfloat16, device=device), "lm_head": rnd(c.vocab_size, H)}


def dequantize_fp8_block(weight: torch.Tensor, scale_inv: torch.Tensor, block_size,
                         dtype=torch.bfloat16) -> torch.Tensor:
    """Block-scaled fp8 weight -> ``dtype``: element ``(r, c)`` is
    ``fp32(weight[r, c]) * scale_inv[r // b0, c // b1]`` with ``block_size =
    (b0, b1)`` (``maybe_dequantize_layer``, qwen_with_nki.py:8865-8880; the
    checkpoint's ``*_scale_inv`` tensors multiply).  A partial last block
    uses its block's scale."""
    if not block_size or len(block_size) != 2:
        raise ValueError("fp8 weights need config.quantization_config['weight_block_size'] = [b0, b1]")
    b0, b1 = int(block_size[0]), int(block_size[1])
    if weight.dim() != 2 or scale_inv.dim() != 2:
        raise ValueError("block dequantisation takes 2-D weights and scales")
    R, C = weight.shape
    if scale_inv.shape != (-(-R // b0), -(-C // b1)):
        raise ValueError(f"scale_inv {tuple(scale_inv.shape)} does not tile a {R}x{C} weight in {b0}x{b1} blocks")
    s = scale_inv.float().repeat_interleave(b0, dim=0).repeat_interleave(b1, dim=1)[:R, :C]
    return (weight.float() * s).to(dtype)


class SafetensorsDir(Mapping):
    """Lazy ``key -> tensor`` view of the ``*.safetensors`` shards of a local
    checkpoint directory: a tensor is read (memory-mapped) when it is asked
    for, so a converter can go one layer at a time."""

    def __init__(self, path: str):
        from safetensors import safe_open

        self._handles, self._where = {}, {}
        for f in sorted(os.listdir(path)):
            if f.endswith(".safetensors"):
                h = safe_open(os.path.join(path, f), framework="pt", device="cpu")
                self._handles[f] = h
                for k in h.keys():
                    self._where[k] = f
        if not self._where:
            raise ValueError(f"no *.safetensors tensors under {path}")

    def __getitem__(self, key):
        return self._handles[self._where[key]].get_tensor(key)

    def __iter__(self):
        return iter(self._where)

    def __len__(self):
        return len(self._where)


def convert_qwen3_moe_hf_to_neuron_state_dict(state_dict, config: Qwen3MoeInferenceConfig,
                                               device=None) -> Dict[str, Any]:
    """HF checkpoint tensors -> the qmoe parameter tree.

    Same key mapping as convert_qwen3_moe_hf_to_neuron_state_dict
    (qwen_with_nki.py:8883-8997): fp8 block dequantisation of every weight
    that has a ``*_scale_inv`` partner (8865-8880), q/k/v concatenated
    (8845-8862), q_norm/k_norm, router from ``mlp.gate.weight`` (8915-8919),
    per-expert gate/up/down packed (8928-8990) -- here into the
    gate/up-interleaved ``w13 [E,2I,H]`` and blocked ``w2 [E,I/8,H,8]``
    layouts.  lm_head from ``lm_head.weight``, or the embedding when
    ``tie_word_embeddings``.  Keys may carry the ``model.`` prefix.

    ``state_dict`` is any mapping (a dict, or a lazy :class:`SafetensorsDir`).
    With ``device`` each converted tensor is moved there as soon as it is
    built, so host memory holds about one layer at a time."""
    keys = {(k[len("model."):] if k.startswith("model.") else k): k for k in state_dict.keys()}
    qcfg = getattr(config, "quantization_config", None) or {}
    block = qcfg.get("weight_block_size") if isinstance(qcfg, dict) else getattr(qcfg, "weight_block_size", None)

    def get(name):
        if name not in keys:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        t = state_dict[keys[name]]
        if name + "_scale_inv" in keys:
            t = dequantize_fp8_block(t, state_dict[keys[name + "_scale_inv"]], block)
        return t

    def put(t):
        t = t.to(torch.bfloat16).contiguous()
        return t.to(device) if device is not None else t

    layers = []
    E = config.num_experts
    # Intermediate padding (qwen_with_nki.py:8959-8964, 8975-8985): zero units
    # appended to every expert.  A zero gate/up row gives a zero SwiGLU
    # output and a zero down column adds nothing, so the block output is the
    # unpadded one; the padded width must still suit the kernels.
    pad = int(getattr(config, "moe_intermediate_pad_size", 0) or 0)
    if pad < 0:
        raise ValueError(f"moe_intermediate_pad_size must be >= 0 (got {pad})")
    if pad and (config.moe_intermediate_size + pad) % _lib.W13_GROUP:
        raise ValueError(f"moe_intermediate_size + moe_intermediate_pad_size = "
                         f"{config.moe_intermediate_size + pad} is not a multiple of {_lib.W13_GROUP}")
    pad_rows = (lambda t: torch.nn.functional.pad(t, (0, 0, 0, pad))) if pad else (lambda t: t)
    pad_cols = (lambda t: torch.nn.functional.pad(t, (0, pad))) if pad else (lambda t: t)
    for l in range(config.num_hidden_layers):
        p = f"layers.{l}."
        w13, w2 = weights.from_hf_experts(
            [pad_rows(get(f"{p}mlp.experts.{e}.gate_proj.weight").float()) for e in range(E)],
            [pad_rows(get(f"{p}mlp.experts.{e}.up_proj.weight").float()) for e in range(E)],
            [pad_cols(get(f"{p}mlp.experts.{e}.down_proj.weight").float()) for e in range(E)],
        )
        layers.append({
            "input_layernorm": put(get(f"{p}input_layernorm.weight")),
            "post_attention_layernorm": put(get(f"{p}post_attention_layernorm.weight")),
            "wqkv": put(torch.cat([get(f"{p}self_attn.q_proj.weight"), get(f"{p}self_attn.k_proj.weight"),
                                   get(f"{p}self_attn.v_proj.weight")])),
            "q_norm": put(get(f"{p}self_attn.q_norm.weight")), "k_norm": put(get(f"{p}self_attn.k_norm.weight")),
            "wo": put(get(f"{p}self_attn.o_proj.weight")), "router": put(get(f"{p}mlp.gate.weight")),
            "w13": put(w13), "w2": put(w2),
        })
        del w13, w2
    if "lm_head.weight" in keys:
        lm = get("lm_head.weight")
    elif getattr(config, "tie_word_embeddings", False):
        lm = get("embed_tokens.weight")
    else:
        raise KeyError("checkpoint has no lm_head.weight and tie_word_embeddings is false")
    return {"embed_tokens": put(get("embed_tokens.weight")), "layers": layers, "norm": put(get("norm.weight")),
            "lm_head": put(lm)}


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
            return convert_qwen3_moe_hf_to_neuron_state_dict(SafetensorsDir(path), self.config, device=self.device)
        return random_params(self.config, self.device, seed=self.neuron_config.seed)

    def reset(self):
        """Start a new sequence (the KV cache is overwritten from position 0)."""
        self.position = 0

    # -- forward ---------------------------------------------------------------
    def prefill(self, input_ids: torch.Tensor, lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Context encoding of ``input_ids[B,S]`` at positions 0..S-1; returns
        the logits ``[B, V]`` (fp32) of each row's last token: position S-1, or
        ``lengths[b] - 1`` for right-padded rows (pad tokens sit after a row's
        end, so causal attention keeps them out of its real positions)."""
        B, S = input_ids.shape
        dev = self.device
        pos = torch.arange(S, device=dev, dtype=torch.int32).repeat(B)
        h = self.model.hidden(input_ids.to(dev), pos, B, S, 0)
        if lengths is None:
            last = h.view(B, S, -1)[:, -1].contiguous()
        else:
            rows = torch.arange(B, device=dev) * S + lengths.to(dev).long() - 1
            last = h.index_select(0, rows).contiguous()
        self.position = S
        return self.model.logits(last)

    def decode_step(self, token_ids: torch.Tensor, positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        """One token per sequence, at ``positions[b]`` (default: the current
        position for every row); returns ``[B, V]`` logits."""
        B = token_ids.shape[0]
        dev = self.device
        if positions is None:
            pos = torch.full((B,), self.position, device=dev, dtype=torch.int32)
            self.position += 1
        else:
            pos = positions.to(device=dev, dtype=torch.int32).contiguous()
            self.position = int(pos.max()) + 1
        h = self.model.hidden(token_ids.to(dev).view(B, 1), pos, B, 1, 0)
        return self.model.logits(h)

    def forward(self, input_ids: torch.Tensor, attention_mask=None, position_ids=None, **kw) -> CausalLMOutput:
        if input_ids.shape[1] > 1 or self.position == 0:
            return CausalLMOutput(self.prefill(input_ids))
        return CausalLMOutput(self.decode_step(input_ids[:, -1]))

    __call__ = forward

    # -- greedy decode with a captured step --------------------------------------
    def greedy_decode(self, first_token: torch.Tensor, n_steps: int, use_graph: Optional[bool] = None,
                      positions: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``n_steps`` greedy tokens after ``first_token[B]``, row b starting at
        ``positions[b]`` (default: the current position for every row); with a
        HIP graph the whole step (embedding, 48 layers, lm_head, argmax,
        position += 1) is one replay.  Returns ``[B, n_steps]`` token ids."""
        use_graph = self.neuron_config.use_hip_graphs if use_graph is None else use_graph
        B = first_token.shape[0]
        if positions is None:
            positions = torch.full((B,), self.position, dtype=torch.int32)
        pos0 = positions.to(device=self.device, dtype=torch.int32).view(B)
        top = int(pos0.max())
        if not use_graph:
            toks, cur = [], first_token.to(self.device)
            for i in range(n_steps):
                cur = ops.argmax(self.decode_step(cur, pos0 + i))
                toks.append(cur)
            self.position = top + n_steps
            self.model.check_embed()
            return torch.stack(toks, dim=1)
        st = self._decode_state(B)
        st["tok"].copy_(first_token.to(self.device).view(B).long())
        st["pos"].copy_(pos0)
        out = torch.empty(B, n_steps, dtype=torch.long, device=self.device)
        for i in range(n_steps):
            self._decode_graph(B, self._bucket(top + i + 1)).replay()
            out[:, i].copy_(st["tok"])
        self.position = top + n_steps
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
            h = m.hidden(st["tok"].view(B, 1), st["pos"], B, 1, 0, h_buf=st["h"], max_ctx=bucket)
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
        # right-padded prompts (main.py:366, 480-486): row b has lengths[b]
        # real tokens; its new tokens continue from position lengths[b] and,
        # as in HF generate, are appended after the padded prompt row
        lengths = None
        if attention_mask is not None:
            _check_causal_mask(attention_mask, torch.zeros(B, 1, dtype=torch.int64))
            am = attention_mask.detach().to("cpu", torch.int64)
            if am.shape != (B, S):
                raise ValueError(f"attention_mask must be [{B}, {S}] like input_ids")
            lengths = am.sum(1)
            if bool((lengths < 1).any()):
                raise ValueError("every prompt row needs at least one real token")
            if bool((lengths == S).all()):
                lengths = None
        spec = int(getattr(m.neuron_config, "speculation_length", 0))
        if spec >= 2 and B == 1 and max_new_tokens > 1:
            prompt = input_ids if lengths is None else input_ids[:, : int(lengths[0])]
            out, _ = m.spec_generate(prompt, max_new_tokens, spec_len=spec)
            return torch.cat([input_ids.to(m.device), out[:, prompt.shape[1]:].to(m.device)], dim=1)
        m.reset()
        logits = m.prefill(input_ids, lengths)
        first = logits.argmax(dim=-1)
        if max_new_tokens <= 1:
            new = first.view(B, -1)[:, :max_new_tokens]
        else:
            rest = m.greedy_decode(first, max_new_tokens - 1,
                                   positions=None if lengths is None else lengths.to(torch.int32))
            new = torch.cat([first.view(B, 1), rest], dim=1)
        return torch.cat([input_ids.to(new.device), new], dim=1)
