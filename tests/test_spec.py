"""Host side of speculative decoding (no GPU): the n-gram drafter and the draft
length rule exported by libminfer (mega.cu:557-589, cuda_infer.cu:1212-1225).

The drafter is checked against an independent brute force over every (n, start)
pair, plus known answers that pin the reference's choices: the longest n-gram
wins over a later shorter one, the latest earlier start wins among equal n, and
the draft is capped by the tokens available after the match and by kmax.
"""
import ctypes as C
import math

import numpy as np

import minfer


def draft(h, ngmax, kmax):
    arr = (C.c_int32 * max(len(h), 1))(*h)
    out = (C.c_int32 * 16)()
    k = minfer.lib().mi_ngram_draft(arr, len(h), ngmax, kmax, out)
    return list(out[:k])


def brute(h, ngmax, kmax):
    L = len(h)
    if kmax <= 0:
        return []
    for n in range(ngmax, 0, -1):
        starts = [j for j in range(0, L - n) if h[j:j + n] == h[L - n:]]
        if starts:
            j = max(starts)
            return h[j + n:j + n + min(kmax, L - (j + n))]
    return []


def test_known_answers():
    # longest n first: [1,2,3] recurs at 0 (followed by 7), the 1-gram [3] recurs later at 5
    assert draft([1, 2, 3, 7, 8, 3, 9, 1, 2, 3], 3, 4) == [7, 8, 3, 9]
    assert draft([1, 2, 3, 7, 8, 3, 9, 1, 2, 3], 1, 4) == [9, 1, 2, 3]
    # latest earlier start among equal n
    assert draft([5, 6, 1, 5, 6, 2, 5, 6], 2, 3) == [2, 5, 6]
    # capped by kmax and by what follows the match
    assert draft([4, 4, 4], 2, 8) == [4]
    assert draft([1, 2, 3, 4, 1], 3, 2) == [2, 3]
    # nothing to match
    assert draft([1, 2, 3], 3, 4) == []
    assert draft([7], 3, 4) == []
    assert draft([1, 1], 3, 0) == []


def test_matches_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(3000):
        L = int(rng.integers(1, 40))
        h = [int(v) for v in rng.integers(0, int(rng.integers(2, 6)), L)]
        ng = int(rng.integers(1, 5))
        k = int(rng.integers(0, 8))
        assert draft(h, ng, k) == brute(h, ng, k), (h, ng, k)


def test_best_draft_len():
    f = minfer.lib().mi_best_draft_len
    slope = 0.074                     # SPEC_SLOPE default (mega.cu:1022)
    ks = [f(a, slope, 8) for a in np.linspace(0.01, 0.99, 99)]
    assert ks[0] == 0 and ks[-1] == 7
    assert all(b >= a for a, b in zip(ks, ks[1:]))          # longer drafts as acceptance grows
    for a in (0.2, 0.5, 0.7, 0.9):
        v = [1.0] + [(1 - a ** (K + 1)) / (1 - a) / (1 + slope * K) for K in range(1, 8)]
        best = max(range(8), key=lambda K: (v[K], -K))
        assert f(a, slope, 8) == best
    assert f(0.9, 0.0, 8) == 7 and f(0.9, 10.0, 8) == 0     # free / very costly extra tokens
    assert all(math.isfinite(f(a, slope, 1)) and f(a, slope, 1) == 0 for a in (0.1, 0.9))
