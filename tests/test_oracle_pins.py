"""Pins the CPU oracle (oracle/cbx_oracle.cpp) before anything is checked
against it.

The reference holds no golden vectors for its sampler, so each stage of
sample_next_token_ex (src/main.cpp:726-801) is pinned by something the oracle's
own code does not restate: the C++ standard's known answers, libstdc++'s
routines called directly, numpy's independent MT19937, exact values where the
arithmetic is exact, float64 recomputation with margins, and brute force on
tiny vocabularies.  Each case names the plausible mistake it catches.
"""
import math

import numpy as np
import pytest

import oracle_lib as O

F32 = np.float32
NEG_INF = float("-inf")


def plain(**kw):
    """Parameters with every filter off unless given."""
    base = dict(top_k=0, top_p=1.0, temp=1.0, repeat_penalty=1.0, min_p=0.0, cfg_weight=0.0)
    base.update(kw)
    return O.OParams(base["top_k"], base["top_p"], base["temp"], base["repeat_penalty"],
                     base["min_p"], base["cfg_weight"])


def kept_set(logits, p, history=(), **kw):
    _, _, probs, kept = O.sample_row(logits, history, p, 0.5, want_probs=True, **kw)
    return set(np.nonzero(probs)[0].tolist()), probs


# --------------------------------------------------------------------------
# RNG front end: std::mt19937 and generate_canonical (random.tcc:3348-3375)
# --------------------------------------------------------------------------

def test_mt19937_standard_check_value():
    # [rand.predef]: the 10000th invocation of a default-constructed mt19937
    # produces 4123659995.
    assert O.lib().cbx_oracle_mt_10000th() == 4123659995


def test_generate_canonical_closed_form_against_numpy_mt19937():
    # numpy's legacy RandomState(seed) seeds MT19937 with init_genrand(seed),
    # an implementation independent of libstdc++.  generate_canonical<double,53>
    # takes two 32-bit outputs: u = RN64(x0 + x1*2^32) / 2^64 (clamped below 1).
    for seed in (0, 42, 5489, 123456789):
        us = O.mt_canonical(seed, 4000)
        raw = np.random.RandomState(seed).randint(0, 2**32, size=8000, dtype=np.uint64)
        raw = [int(v) for v in raw]
        exp = [float(raw[2 * i] + raw[2 * i + 1] * 2**32) / 2.0**64 for i in range(4000)]
        exp = [min(v, math.nextafter(1.0, 0.0)) for v in exp]
        assert np.array_equal(us, np.array(exp)), seed
    # the 10000th-output check value through numpy too (ties numpy to the KAT)
    raw = np.random.RandomState(5489).randint(0, 2**32, size=10000, dtype=np.uint64)
    assert int(raw[-1]) == 4123659995


# --------------------------------------------------------------------------
# Draw stage: std::discrete_distribution (random.tcc:2657-2712)
# --------------------------------------------------------------------------

def _words_for(u):
    """Two 32-bit words whose generate_canonical value is exactly u (u*2^64 an
    integer below 2^64)."""
    n = int(u * 2.0**64)
    assert n / 2.0**64 == u
    return n & 0xFFFFFFFF, n >> 32


@pytest.mark.parametrize("probs", [
    [0.25, 0.25, 0.25, 0.25],
    [0.0, 0.5, 0.5, 0.0],
    [1.0 / 3, 1.0 / 3, 1.0 / 3, 0.0],
    [0.0, 0.0, 1.0],
    [0.1, 0.2, 0.3, 0.4],
    [1e-30, 0.5, 1e-30, 0.5, 0.0, 0.0],
])
def test_cdf_draw_matches_libstdcxx_at_boundaries(probs):
    # The restated CDF + lower_bound against libstdc++'s own distribution at
    # exact boundary values.  Catches: upper_bound instead of lower_bound, a
    # CDF in sorted rather than index order, a missing forced 1.0 on the last
    # entry, float instead of double accumulation.
    p = np.array(probs, dtype=F32)
    w = p.astype(np.float64)
    cdf = np.cumsum(w / w.sum())
    cand = {0.0, math.nextafter(1.0, 0.0), 0.5, 0.25, 0.75}
    for c in cdf[:-1]:
        for v in (c, math.nextafter(c, 0.0), math.nextafter(c, 1.0)):
            if 0.0 <= v < 1.0:
                cand.add(v)
    for u in sorted(cand):
        # round to a value representable as k / 2^64 so the engine can make it
        k = int(u * 2.0**64)
        uu = k / 2.0**64
        if uu >= 1.0:
            continue
        x0, x1 = k & 0xFFFFFFFF, k >> 32
        assert O.cdf_draw(p, uu) == O.stdlib_draw(p, x0, x1), (probs, uu)


def test_cdf_draw_matches_libstdcxx_random():
    rng = np.random.default_rng(7)
    for trial in range(3000):
        n = int(rng.integers(2, 40))
        p = rng.random(n).astype(F32)
        p[rng.random(n) < 0.3] = 0.0
        if p.sum() == 0:
            p[0] = 1.0
        p = (p / p.sum()).astype(F32)
        x0, x1 = (int(v) for v in rng.integers(0, 2**32, size=2))
        u = float(x0 + x1 * 2**32) / 2.0**64
        if u >= 1.0:
            continue
        assert O.cdf_draw(p, u) == O.stdlib_draw(p, x0, x1)


def test_draw_quirks():
    # u == 0 selects index 0 even when its probability is 0 (lower_bound on a
    # CDF whose leading entries are 0).
    assert O.cdf_draw(np.array([0, 0.5, 0.5, 0], F32), 0.0) == 0
    # A zero-probability last id is returned when u lies above the last
    # computed cumulative value: that entry is forced to exactly 1.0.
    p = np.array([1 / 3, 1 / 3, 1 / 3, 0.0], F32)
    w = p.astype(np.float64)
    s = w[0] + w[1] + w[2]
    c2 = (w[0] / s + w[1] / s) + w[2] / s
    if c2 < 1.0:
        u = math.nextafter(1.0, 0.0)
        x0, x1 = _words_for(u)
        assert O.stdlib_draw(p, x0, x1) == 3
        assert O.cdf_draw(p, u) == 3
    # fewer than two weights: no CDF, index 0
    assert O.cdf_draw(np.array([1.0], F32), 0.7) == 0


def test_engine_driven_run_equals_injected_uniforms():
    # The engine loop (std::discrete_distribution on a live mt19937, history
    # growing, chatterbox_engine.cpp:338-353) must equal the u-injected path fed
    # the generate_canonical values that loop consumed.
    rng = np.random.default_rng(11)
    V, steps = 300, 200
    logits = (rng.standard_normal((steps, V)) * 3).astype(F32)
    p = O.params(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.3)
    toks, us = O.run_mt19937(logits, np.array([], np.int32), p, seed=42, grow_history=True)
    hist = []
    draws = O.mt_canonical(42, 2 * steps)
    di = 0
    for t in range(steps):
        assert us[t] == draws[di]
        tok, info = O.sample_row(logits[t], hist, p, draws[di])
        assert info & O.INFO_DREW
        di += 1
        assert tok == toks[t], t
        hist.append(tok)


# --------------------------------------------------------------------------
# Stage 1: temperature (main.cpp:735-738)
# --------------------------------------------------------------------------

def test_temperature_multiplies_by_float_reciprocal():
    # s * (1.0f/T) and s / T differ in the last bit for some s.  The penalty is
    # off and only two ids survive, so p0 = 1 / (1 + exp(s1' - s0')) exposes
    # the scaled value through the float division in the softmax.
    T = F32(0.7)
    inv = F32(1.0) / T
    rng = np.random.default_rng(3)
    found = None
    for s in (rng.standard_normal(20000) * 4).astype(F32):
        if F32(s * inv) != F32(s / T):
            found = s
            break
    assert found is not None
    logits = np.array([found, F32(0.0)], F32)
    _, _, probs, _ = O.sample_row(logits, [], plain(temp=0.7), 0.5, want_probs=True)
    mul = F32(found * inv)
    div = F32(found / T)

    def probs_for(scaled):
        mx = max(scaled, F32(0.0))
        a = O.libm_expf(np.array([F32(scaled - mx)], F32))[0]
        b = O.libm_expf(np.array([F32(F32(0.0) - mx)], F32))[0]
        s = F32(a + b)
        return np.array([F32(a / s), F32(b / s)], F32)

    assert np.array_equal(probs, probs_for(mul))
    assert not np.array_equal(probs_for(mul), probs_for(div))


# --------------------------------------------------------------------------
# Stage 2: top-k (main.cpp:740-748)
# --------------------------------------------------------------------------

def test_top_k_distinct_values_brute_force():
    rng = np.random.default_rng(5)
    for _ in range(200):
        V = int(rng.integers(2, 30))
        k = int(rng.integers(1, V))
        x = rng.permutation(V).astype(F32) - F32(V / 2)  # distinct
        ks, _ = kept_set(x, plain(top_k=k))
        assert ks == set(np.argsort(-x)[:k].tolist())


def test_top_k_tie_at_threshold_large_magnitude():
    # k=2 over [5,4,4,4,1]: the 3rd largest is 4; only one value is above it,
    # so the threshold is nudged by 1e-10f -- a no-op at 4.0 -- and every 4 is
    # dropped: ONE survivor.  (Keeping ties, or ">=", would keep four.)
    ks, _ = kept_set(np.array([5, 4, 4, 4, 1], F32), plain(top_k=2))
    assert ks == {0}


def test_top_k_tie_at_threshold_small_magnitude():
    # Same shape near 1e-4, where 1e-10 is about 14 ulps: the nudge moves the
    # threshold below the tied values and all of them survive.
    x = np.array([0.5, 1e-4, 1e-4, 1e-4, -1.0], F32)
    assert F32(x[1] - F32(1e-10)) < x[1]
    ks, _ = kept_set(x, plain(top_k=2))
    assert ks == {0, 1, 2, 3}


@pytest.mark.parametrize("k", [0, -3, 5, 6])
def test_top_k_inactive_outside_open_range(k):
    ks, _ = kept_set(np.arange(5, dtype=F32), plain(top_k=k))
    assert ks == {0, 1, 2, 3, 4}


# --------------------------------------------------------------------------
# Stage 3: top-p (main.cpp:750-772)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("top_p,n_kept", [(0.25, 1), (0.5, 2), (0.5000001, 3), (0.75, 3),
                                          (0.9999999, 4), (0.0, 1), (-1.0, 1)])
def test_top_p_exact_quarters(top_p, n_kept):
    # Four equal scores: exp(0) = 1 each, psum = 4, probabilities exactly 0.25
    # and every running sum exact.  The crossing item is kept and the test is
    # ">=" (">" would keep one more at 0.5, 0.25 and 0.75).
    x = np.full(4, 2.5, F32)
    _, info, probs, kept = O.sample_row(x, [], plain(top_p=top_p), 0.5, want_probs=True)
    assert kept == n_kept
    if n_kept < 4:
        assert info & O.INFO_TOPP_TIE


def test_top_p_float64_with_margin():
    # Distinct scores; a top_p chosen at least 1e-4 away from every float64
    # cumulative boundary has an unambiguous answer: the shortest prefix of
    # the descending order whose mass reaches top_p.
    rng = np.random.default_rng(9)
    checked = 0
    for _ in range(400):
        V = int(rng.integers(3, 25))
        x = (rng.standard_normal(V) * 2).astype(F32)
        order = np.argsort(-x.astype(np.float64), kind="stable")
        e = np.exp(x.astype(np.float64) - x.max())
        cum = np.cumsum(e[order] / e.sum())
        tp = float(rng.uniform(0.05, 0.99))
        if np.min(np.abs(cum - tp)) < 1e-4:
            continue
        n = int(np.searchsorted(cum, tp) + 1)
        ks, _ = kept_set(x, plain(top_p=tp))
        assert ks == set(order[:n].tolist())
        checked += 1
    assert checked > 300


def test_top_p_inactive_at_one():
    ks, _ = kept_set(np.arange(6, dtype=F32), plain(top_p=1.0))
    assert len(ks) == 6


# --------------------------------------------------------------------------
# Stage 3b: min-p (extension; ratio to the best survivor)
# --------------------------------------------------------------------------

def test_min_p_ratio_form():
    # Ratios exp(-d) for gaps d = 0..3: 1, .368, .135, .0498.  min_p = 0.1
    # drops only the last; min_p = 0.2 also drops the third.
    x = np.array([0, -1, -2, -3], F32)
    assert kept_set(x, plain(min_p=0.1))[0] == {0, 1, 2}
    assert kept_set(x, plain(min_p=0.2))[0] == {0, 1}
    assert kept_set(x, plain(min_p=1.0))[0] == {0}


# --------------------------------------------------------------------------
# Stage 4: repetition penalty (main.cpp:774-781)
# --------------------------------------------------------------------------

def test_repetition_penalty_direction_and_uniqueness():
    # pen=2 on history {0, 1, 1, 7 (out of range), -3}: s0 = 2/2 = 1,
    # s1 = -2*2 = -4 (once, not twice), s2 and s3 unchanged.
    x = np.array([2.0, -2.0, 1.0, 0.5], F32)
    _, probs = kept_set(x, plain(repeat_penalty=2.0), history=[0, 1, 1, 7, -3])
    s = np.array([1.0, -4.0, 1.0, 0.5])
    e = np.exp(s - s.max())
    assert np.allclose(probs, e / e.sum(), rtol=1e-6, atol=0)


def test_repetition_penalty_after_top_p():
    # [2, 1.9, -10, -10]: id 0 alone has mass 0.525 >= 0.5, so top-p keeps only
    # it; the penalty then lowers it but it is the only survivor.  Applying
    # the penalty before top-p would make id 1 the top choice.
    x = np.array([2.0, 1.9, -10, -10], F32)
    for u in (0.01, 0.5, 0.99):
        tok, _ = O.sample_row(x, [0], plain(top_p=0.5, repeat_penalty=2.0), u)
        assert tok == 0


def test_repetition_penalty_skips_filtered_ids():
    # id 2 is removed by top-k; history naming it must not resurrect it.
    x = np.array([3.0, 2.0, 1.0, 0.0], F32)
    ks, _ = kept_set(x, plain(top_k=2, repeat_penalty=0.5), history=[2, 3])
    assert ks == {0, 1}


# --------------------------------------------------------------------------
# Stage 5-6: softmax, greedy, empty rows (main.cpp:783-800)
# --------------------------------------------------------------------------

def test_softmax_matches_float64():
    rng = np.random.default_rng(13)
    for _ in range(50):
        x = (rng.standard_normal(500) * 3).astype(F32)
        _, probs = kept_set(x, plain())
        e = np.exp(x.astype(np.float64) - x.max())
        assert np.allclose(probs, e / e.sum(), rtol=2e-6, atol=1e-12)
        assert abs(float(probs.astype(np.float64).sum()) - 1.0) < 1e-5


def test_greedy_first_argmax():
    tok, info = O.sample_row(np.array([1, 3, 3, 2], F32), [], plain(temp=0.0), 0.99)
    assert tok == 1 and info & O.INFO_GREEDY and not info & O.INFO_DREW


def test_all_filtered_returns_zero():
    x = np.full(8, NEG_INF, F32)
    tok, info = O.sample_row(x, [], O.params(), 0.7)
    assert tok == 0 and info & O.INFO_EMPTY and not info & O.INFO_DREW


# --------------------------------------------------------------------------
# Extensions: CFG, allowed mask, forced stop
# --------------------------------------------------------------------------

def test_cfg_combine_exact():
    # c + 0.5*(c - u) with u = 0 is 1.5*c exactly for these values.
    c = np.array([1.0, 2.0, -4.0, 0.5], F32)
    u = np.zeros(4, F32)
    _, probs_cfg = kept_set(c, plain(cfg_weight=0.5), uncond=u)
    _, probs_ref = kept_set(c * F32(1.5), plain())
    assert np.array_equal(probs_cfg, probs_ref)
    # w = 0 is the cond row itself
    _, probs_w0 = kept_set(c, plain(cfg_weight=0.0), uncond=np.full(4, 9.0, F32))
    _, probs_c = kept_set(c, plain())
    assert np.array_equal(probs_w0, probs_c)


def test_allowed_mask_and_forced_stop():
    x = np.arange(40, dtype=F32)
    allowed = np.zeros(2, np.uint32)
    allowed[0] = (1 << 3) | (1 << 17)
    allowed[1] = 1 << (33 - 32)
    ks, _ = kept_set(x, plain(), allowed=allowed)
    assert ks == {3, 17, 33}
    for u in (1e-9, 0.3, 0.999):
        tok, _ = O.sample_row(x, [], O.params(), u, force_stop=True, stop_token=21)
        assert tok == 21
    # the lower_bound quirk survives the mask: u == 0 picks id 0
    tok, _ = O.sample_row(x, [], O.params(), 0.0, force_stop=True, stop_token=21)
    assert tok == 0
    tok, info = O.sample_row(x, [], O.params(), 0.5, allowed=np.zeros(2, np.uint32))
    assert tok == 0 and info & O.INFO_EMPTY


# --------------------------------------------------------------------------
# Whole sampler: brute force over u on tiny vocabularies
# --------------------------------------------------------------------------

def _f64_pipeline(x, hist, top_k, top_p, temp, pen):
    """Reference stage order in float64 (independent of the oracle's code)."""
    s = x.astype(np.float64)
    if temp > 0 and temp != 1:
        s = s * (1.0 / temp)
    n = len(s)
    alive = np.ones(n, bool)
    if 0 < top_k < n:
        thr = np.sort(s)[::-1][top_k]
        alive &= s > thr
    if top_p < 1:
        idx = [i for i in np.argsort(-s, kind="stable") if alive[i]]
        e = np.exp(s[idx] - s[idx[0]])
        cum = np.cumsum(e / e.sum())
        n_keep = int(np.searchsorted(cum, top_p) + 1)
        keep = np.zeros(n, bool)
        keep[idx[:n_keep]] = True
        alive &= keep
        margin = np.min(np.abs(cum - top_p))
    else:
        margin = 1.0
    if pen != 1:
        for t in set(hist):
            if 0 <= t < n and alive[t]:
                s[t] = s[t] / pen if s[t] > 0 else s[t] * pen
    e = np.where(alive, np.exp(s - s[alive].max()), 0.0)
    return e / e.sum(), margin


def test_brute_force_distribution_over_u():
    rng = np.random.default_rng(17)
    grid = (np.arange(4000) + 0.5) / 4000
    done = 0
    for _ in range(40):
        V = int(rng.integers(3, 9))
        x = (rng.standard_normal(V) * 2).astype(F32)
        hist = rng.integers(0, V, size=3).tolist()
        top_k = int(rng.integers(0, V + 1))
        top_p = float(rng.uniform(0.5, 1.0))
        temp = float(rng.uniform(0.5, 1.5))
        pen = 1.3
        p64, margin = _f64_pipeline(x, hist, top_k, F32(top_p), F32(temp), F32(pen))
        if margin < 1e-4:
            continue
        p = O.OParams(top_k, top_p, temp, pen, 0.0, 0.0)
        counts = np.zeros(V)
        for u in grid:
            counts[O.sample_row(x, hist, p, u)[0]] += 1
        assert np.allclose(counts / len(grid), p64, atol=1.5 / len(grid) + 1e-6)
        done += 1
    assert done > 20
