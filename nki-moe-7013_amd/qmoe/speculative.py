"""Prompt-lookup speculation: the candidate search of the reference's
speculative decoding driver.

``prompt_lookup`` restates ``_prompt_lookup_with_meta``
(qwen_with_nki.py:351-453) with its shipped defaults: n-gram sizes from
``n = 4`` down to ``n_min = 1`` (lines 74-79) and the ``majority1`` strategy
(line 307): for the largest n-gram size whose last ``n`` tokens occur earlier
in the sequence, the continuation of the most recent occurrence is proposed;
for single-token matches (n = 1) each of the ``k`` candidate slots takes the
most frequent token that followed any occurrence (ties to the smallest id).
The verification of the candidates runs on the GPU
(:meth:`qmoe.model.NeuronQwen3MoeForCausalLM.spec_generate`).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np

STRATEGIES = ("last", "first", "majority", "majority1")


def _strategy_for(strategy: str, ngram: int) -> str:
    if strategy == "majority1":
        return "majority" if ngram == 1 else "last"
    return strategy


def prompt_lookup(seq: Sequence[int], k: int, n: int = 4, n_min: int = 1,
                  strategy: str = "majority1") -> Tuple[List[int], int]:
    """Up to ``k`` candidate tokens continuing ``seq`` and the n-gram size that
    produced them (``([], 0)`` when nothing matches)."""
    if strategy not in STRATEGIES:
        raise ValueError(f"strategy must be one of {STRATEGIES}")
    a = np.asarray(seq, dtype=np.int64)
    T = a.shape[0]
    for size in range(n, n_min - 1, -1):
        if T < size + 1:
            continue
        head = a[: T - size]  # windows never include the tail itself
        if head.shape[0] < size:
            continue
        windows = np.lib.stride_tricks.sliding_window_view(head, size)
        hits = np.nonzero((windows == a[T - size:]).all(axis=1))[0]
        if hits.size == 0:
            continue
        how = _strategy_for(strategy, size)
        if how == "majority" and hits.size > 1:
            cont: List[int] = []
            for j in range(k):
                p = hits + size + j
                p = p[p < T]
                if p.size == 0:
                    break
                vals, counts = np.unique(a[p], return_counts=True)  # sorted: ties -> smallest id
                cont.append(int(vals[np.argmax(counts)]))
        else:
            pick = int(hits[0] if how == "first" else hits[-1])
            cont = a[pick + size: min(pick + size + k, T)].tolist()
        if cont:
            return cont, size
    return [], 0


def accept(candidates: Sequence[int], target: Sequence[int]) -> Tuple[int, List[int]]:
    """Greedy verification: ``target[i]`` is the model's token after the
    verified prefix of length i.  Returns the number of accepted candidates m
    and the emitted tokens ``candidates[:m] + [target[m]]``."""
    m = 0
    while m < len(candidates) and int(candidates[m]) == int(target[m]):
        m += 1
    return m, [int(t) for t in candidates[:m]] + [int(target[m])]


def pad_candidates(candidates: Sequence[int], k: int, fill: Optional[int] = None) -> List[int]:
    """``candidates`` padded to ``k`` tokens (repeating the last one) for a
    fixed-shape verification step; the padding is never accepted past the
    real candidates."""
    c = [int(t) for t in candidates[:k]]
    if not c:
        c = [int(fill if fill is not None else 0)]
    return c + [c[-1]] * (k - len(c))
