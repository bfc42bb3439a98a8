"""Generate-mode driver: the call sequence of ``main.py --mode generate``.

``prepare_inference`` mirrors main.py:372-433 (config objects -> model ->
compile -> load -> tokenizer -> generation config) and ``run_generation``
mirrors main.py:634-649, on the MI355X model class.  Decoding is greedy,
optionally with prompt-lookup speculation (``--speculation-length 5``: the
reference's shipped setting).  With no local checkpoint the model is
random-init (seeded) and prompts are token ids.

    python -m qmoe.driver --model-path random --prompt-ids 1,2,3 --seq-len 64
"""

from __future__ import annotations

import argparse
import copy
import os
import time
from types import SimpleNamespace
from typing import List, Optional

import torch

from .model import (HuggingFaceGenerationAdapter, NeuronQwen3MoeForCausalLM, load_pretrained_config)


def parse_args(argv=None):
    p = argparse.ArgumentParser(description="Qwen3-30B-A3B on MI355X (generate mode)")
    p.add_argument("--mode", default="generate", choices=["generate"])
    p.add_argument("--model-path", default="random",
                   help="local HF checkpoint directory, or 'random' for seeded random-init weights")
    p.add_argument("--compiled-model-path", default=None)
    p.add_argument("--prompt", dest="prompts", action="append", default=None)
    p.add_argument("--prompt-ids", default=None, help="comma-separated token ids (no tokenizer needed)")
    p.add_argument("--random-prompt-len", type=int, default=None)
    p.add_argument("--seq-len", type=int, default=640)
    p.add_argument("--batch-size", type=int, default=1)
    p.add_argument("--max-new-tokens", type=int, default=None)
    p.add_argument("--torch-dtype", default="bfloat16")
    p.add_argument("--tp-degree", type=int, default=1)
    p.add_argument("--num-layers", type=int, default=None, help="override num_hidden_layers")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--enable-nki", action="store_true", help="accepted for main.py compatibility")
    p.add_argument("--skip-compile", action="store_true")
    p.add_argument("--do-sample", action="store_true")
    p.add_argument("--speculation-length", type=int, default=0,
                   help="prompt-lookup speculation: tokens verified per step (the reference ships 5); 0 = off")
    return p.parse_args(argv)


def prepare_inference(model_cls, args):
    """main.py:372-433: build the configs, the model, compile, load."""
    kw = copy.deepcopy({k: v for k, v in vars(args).items() if v is not None})
    neuron_config = model_cls.get_neuron_config_cls()(
        batch_size=kw.get("batch_size", 1), seq_len=kw.get("seq_len", 640),
        max_length=kw.get("seq_len", 640), torch_dtype=kw.get("torch_dtype", "bfloat16"),
        tp_degree=kw.get("tp_degree", 1), seed=kw.get("seed", 0),
        speculation_length=kw.get("speculation_length", 0))
    path = args.model_path
    load_config = None
    if path and os.path.isfile(os.path.join(path, "config.json")):
        load_config = load_pretrained_config(path)
    config = model_cls.get_config_cls()(neuron_config, load_config=load_config)
    if args.num_layers is not None:
        config.num_hidden_layers = args.num_layers
    model = model_cls(path, config)
    if not getattr(args, "skip_compile", False):
        model.compile(args.compiled_model_path)
    model.load(args.compiled_model_path)
    tokenizer = None
    if path and os.path.isdir(path):
        try:
            from transformers import AutoTokenizer

            tokenizer = AutoTokenizer.from_pretrained(path, padding_side="right")
            tokenizer.pad_token = tokenizer.eos_token
            neuron_config.pad_token_id = tokenizer.pad_token_id
        except Exception:
            tokenizer = None
    generation_config = SimpleNamespace(do_sample=bool(args.do_sample))
    return model, tokenizer, generation_config


def run_generation(model, tokenizer, prompts, generation_config, prompt_ids: Optional[torch.Tensor] = None):
    """main.py:634-649.  Text prompts are right-padded to the longest
    (main.py:366) and their attention mask goes to ``generate``, so each row
    continues from its own last real token."""
    attention_mask = None
    if prompt_ids is None:
        if tokenizer is None:
            raise ValueError("text prompts need a tokenizer (local --model-path); use --prompt-ids")
        enc = tokenizer(prompts, padding=True, return_tensors="pt")
        prompt_ids, attention_mask = enc.input_ids, enc.attention_mask
    adapter = HuggingFaceGenerationAdapter(model)
    t0 = time.perf_counter()
    out = adapter.generate(prompt_ids, attention_mask=attention_mask, generation_config=generation_config,
                           max_length=model.neuron_config.max_length)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"Generated {out.shape[1] - prompt_ids.shape[1]} tokens x {out.shape[0]} in {dt:.3f} s")
    if tokenizer is not None:
        for i, s in enumerate(tokenizer.batch_decode(out, skip_special_tokens=True)):
            print(f"Output {i}: {s}")
    else:
        for i, row in enumerate(out.tolist()):
            print(f"Output {i}: {row}")
    return out


def main(argv=None):
    args = parse_args(argv)
    model, tok, gen = prepare_inference(NeuronQwen3MoeForCausalLM, args)
    ids = None
    if args.prompt_ids:
        ids = torch.tensor([[int(t) for t in args.prompt_ids.split(",")]] * args.batch_size)
    elif args.random_prompt_len:
        g = torch.Generator().manual_seed(args.seed)
        ids = torch.randint(0, model.config.vocab_size, (args.batch_size, args.random_prompt_len), generator=g)
    return run_generation(model, tok, args.prompts, gen, ids)


if __name__ == "__main__":
    main()
