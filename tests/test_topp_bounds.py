"""The bound the one-wave kernel's top-p certification puts on the float
normaliser psum (main.cpp:758-760: psum += probs[i] over the sorted exp terms,
in binary32), checked on the mathematics it rests on: each of the n - 1
inexact adds of non-negative terms is off by at most half an ulp of its
result, whose binade is at most that of the float sum, itself at most
S (1 + gam_t) with gam_t = n 2^-24 (1 + 2^-10) (the recursive-sum bound,
Higham, Accuracy and Stability of Numerical Algorithms, §4.2).  So
|psum - S| <= (n - 1) 2^(E - 24) with 2^E the binade of S (1 + gam_t), never
more than gam_t S.  Sequences: random sorted exp terms, and adds that each
round up by almost half an ulp (where half that bound fails)."""
import math

import numpy as np


def _fsum32(e):
    s = np.float32(0.0)
    for x in e:
        s = np.float32(s + x)
    return float(s)


def _bound(e):
    n = len(e)
    S = math.fsum(float(x) for x in e)
    gam_t = n * 2.0**-24 * (1 + 2.0**-10)
    es = math.frexp(S * (1 + gam_t))[1] - 1
    return S, (n - 1) * 2.0**(es - 24), gam_t * S


def test_psum_bound_random_sorted_terms():
    rng = np.random.default_rng(0x75)
    worst = 0.0
    for trial in range(300):
        n = int(rng.integers(2, 1200))
        spread = float(rng.uniform(1.0, 40.0))
        x = np.sort(rng.uniform(0.0, spread, n))  # max - v >= 0, ascending
        x[0] = 0.0
        e = np.exp(-x).astype(np.float32)           # e_0 = 1, descending
        S, D, T = _bound(e)
        err = abs(_fsum32(e) - S)
        assert err <= D, (trial, n, err, D)
        assert D <= T
        worst = max(worst, err / D)
    assert worst > 0.0


def test_psum_bound_is_reached_by_round_up_adds():
    # 1 then terms just above half an ulp of [1, 2): every add rounds up by
    # nearly half an ulp, so the error nears (n - 1) 2^-24 and half the
    # bound (a binade too low) would fail
    n = 4000
    e = np.full(n, np.float32(2.0**-24 * (1 + 2.0**-12)), dtype=np.float32)
    e[0] = np.float32(1.0)
    S, D, T = _bound(e)
    err = abs(_fsum32(e) - S)
    assert err <= D
    assert err > D / 2
    # crossing into [2, 4): the bound takes the higher binade's half ulp
    e2 = np.concatenate([np.float32([1.0, 0.999]), np.full(3000, np.float32(2.0**-23 * 1.001))])
    S2, D2, _ = _bound(e2)
    assert abs(_fsum32(e2) - S2) <= D2
