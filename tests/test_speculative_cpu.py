"""Prompt-lookup candidate search and greedy acceptance (host logic of the
speculative decoding driver, qwen_with_nki.py:351-453, 575-1211): known
answers worked by hand, and a brute-force restatement with explicit loops on
random small-alphabet sequences (many matches, ties in the majority vote)."""

import random

import pytest

from qmoe import speculative as sp


def _brute(seq, k, n, n_min, strategy):
    T = len(seq)
    for size in range(n, n_min - 1, -1):
        if T < size + 1 or T - size < size:
            continue
        tail = seq[T - size:]
        hits = [i for i in range(0, T - 2 * size + 1) if seq[i:i + size] == tail]
        if not hits:
            continue
        how = strategy
        if strategy == "majority1":
            how = "majority" if size == 1 else "last"
        if how == "majority" and len(hits) > 1:
            cont = []
            for j in range(k):
                vals = [seq[i + size + j] for i in hits if i + size + j < T]
                if not vals:
                    break
                counts = {}
                for v in vals:
                    counts[v] = counts.get(v, 0) + 1
                top = max(counts.values())
                cont.append(min(v for v, c in counts.items() if c == top))
        else:
            pick = hits[0] if how == "first" else hits[-1]
            cont = seq[pick + size: min(pick + size + k, T)]
        if cont:
            return cont, size
    return [], 0


def test_known_answers():
    # 3-gram [1,2,3] seen at 0 -> continuation of that occurrence
    assert sp.prompt_lookup([1, 2, 3, 4, 1, 2, 3], 3) == ([4, 1, 2], 3)
    # only single-token matches: slot-wise majority, ties to the smallest id
    assert sp.prompt_lookup([9, 1, 2, 1, 3, 1, 4, 1], 2) == ([2, 1], 1)
    # the same sequence with "last": the continuation of the latest match only
    assert sp.prompt_lookup([9, 1, 2, 1, 3, 1, 4, 1], 2, strategy="last") == ([4, 1], 1)
    assert sp.prompt_lookup([9, 1, 2, 1, 3, 1, 4, 1], 2, strategy="first") == ([2, 1], 1)
    # nothing repeats
    assert sp.prompt_lookup([1, 2, 3, 4, 5], 4) == ([], 0)
    # continuation cut at the end of the sequence
    assert sp.prompt_lookup([7, 8, 7], 4) == ([8, 7], 1)


@pytest.mark.parametrize("strategy", sp.STRATEGIES)
@pytest.mark.parametrize("seed", range(40))
def test_matches_brute_force(strategy, seed):
    rng = random.Random(seed * 7 + len(strategy))
    T = rng.randint(1, 60)
    alpha = rng.choice([2, 3, 5, 50])
    seq = [rng.randrange(alpha) for _ in range(T)]
    k = rng.randint(1, 6)
    n = rng.randint(1, 5)
    n_min = rng.randint(1, n)
    assert sp.prompt_lookup(seq, k, n, n_min, strategy) == _brute(seq, k, n, n_min, strategy)


def test_accept_and_pad():
    assert sp.accept([5, 6, 7], [5, 6, 9, 1]) == (2, [5, 6, 9])
    assert sp.accept([5, 6, 7], [4, 6, 7, 1]) == (0, [4])
    assert sp.accept([5, 6, 7], [5, 6, 7, 8]) == (3, [5, 6, 7, 8])
    assert sp.accept([], [3]) == (0, [3])
    assert sp.pad_candidates([4, 5], 4) == [4, 5, 5, 5]
    assert sp.pad_candidates([1, 2, 3, 4, 5], 4) == [1, 2, 3, 4]
