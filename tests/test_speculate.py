"""The n-gram draft of speculative decoding (speculate.rs:122-150), host code
in the engine library, checked on the CPU.

The reference ships no tests for this module; the cases below are worked by
hand from the function's stated rules (longest n-gram first, most recent
occurrence first, at most `want` tokens, never past the end of the history),
and a brute force that enumerates every match and keeps the latest one
cross-checks random histories.
"""
import numpy as np
import pytest

from whetstone_amd import engine as E


@pytest.mark.parametrize("hist,kw,want", [
    # the 3-gram tail [1,2,3] occurred at 0: what followed it
    ([1, 2, 3, 9, 1, 2, 3], dict(want=3), [9, 1, 2]),
    # no 3-gram match; the 2-gram [5,6] occurred at 0 and 3: the latest wins
    ([5, 6, 7, 5, 6, 8, 5, 6], dict(want=3), [8, 5, 6]),
    # a 3-gram match (older) beats a 2-gram match (more recent)
    ([1, 2, 3, 4, 9, 2, 3, 7, 1, 2, 3], dict(want=3), [4, 9, 2]),
    # clipped at the end of the history
    ([1, 2, 1, 2], dict(want=3), [1, 2]),
    ([1, 2, 1, 2], dict(want=1), [1]),
    # nothing matches
    ([1, 2, 3, 4, 5], dict(want=3), []),
    # want 0 proposes nothing
    ([1, 2, 1, 2], dict(want=0), []),
    # too short for the minimum n-gram: n_max = min(3, len-1) = 1 < 2
    ([7, 7], dict(want=3), []),
    # ngram_min 1: a single repeated token is a match
    ([4, 8, 4], dict(want=2, ngram_min=1), [8, 4]),
    # ngram_max 2 ignores the longer (older) match
    ([1, 2, 3, 4, 9, 2, 3, 7, 1, 2, 3], dict(want=2, ngram_max=2), [7, 1]),
])
def test_propose_hand_cases(hist, kw, want):
    args = dict(ngram_max=3, ngram_min=2)
    args.update(kw)
    assert E.spec_propose(hist, **args) == want


def _brute(hist, ngram_max, ngram_min, want):
    if want == 0:
        return []
    L = len(hist)
    for n in range(min(ngram_max, max(L - 1, 0)), ngram_min - 1, -1):
        if L <= n:
            continue
        tail = hist[L - n:]
        starts = [s for s in range(L - n) if hist[s:s + n] == tail]
        for s in sorted(starts, reverse=True):
            got = hist[s + n:s + n + want]
            if got:
                return got
    return []


def test_propose_matches_brute_force_on_random_histories():
    rng = np.random.default_rng(3)
    for trial in range(400):
        L = int(rng.integers(1, 40))
        hist = [int(v) for v in rng.integers(0, int(rng.integers(2, 6)), L)]
        nmax, nmin = int(rng.integers(0, 5)), int(rng.integers(1, 4))
        want = int(rng.integers(0, 8))
        got = E.spec_propose(hist, ngram_max=nmax, ngram_min=nmin, want=want)
        assert got == _brute(hist, nmax, nmin, want), (trial, hist, nmax, nmin, want)


def test_spec_stats_ratios():
    s = E.SpecStats(rounds=4, empty_rounds=1, proposed=9, accepted=6)
    assert s.acceptance() == pytest.approx(6 / 9)
    assert s.tokens_per_round() == pytest.approx(10 / 4)
    assert E.SpecStats().acceptance() == 0.0 and E.SpecStats().tokens_per_round() == 0.0
    c = E.SpecConfig()
    assert (c.draft, c.ngram_max, c.ngram_min) == (4, 3, 2)  # SpecConfig::default
