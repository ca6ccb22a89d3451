"""Pins for the oracle's sampler (slm/sampling.rs:96-210), CPU only.

Known-answer and behavioural tests are the reference's own (cited).  The
mathematical pins check what the algorithm fixes independently of its code:
the inverse-CDF property over an exhaustive grid of draws, the exact top-k
support, the minimal top-p prefix, and the penalty's per-occurrence effect.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest


def P(orc, **kw):
    return orc.SamplingParams(**kw)


def draws_for(r_values):
    """u64 draws whose next_f32 is exactly r (r on the 2^-24 grid)."""
    return [int(round(r * (1 << 24))) << 40 for r in r_values]


# ---- the reference's tests ---------------------------------------------------

def test_argmax_first_known_answers(orc):
    # sampling.rs:392-405
    a = orc.argmax_first
    assert a([]) == 0 and a([1.0]) == 0 and a([0.1, 2.0, 2.0, 1.0]) == 1
    assert a([3.0, 3.0, 3.0]) == 0 and a([-1.0, -0.5, -0.5]) == 1
    assert a([float("-inf"), float("-inf")]) == 0
    tok, _ = orc.sample([1.0, 5.0, 5.0], P(orc, temperature=0.0))
    assert tok == 1


def test_pick_by_mass_known_answers(orc):
    # sampling.rs:408-422
    pb = orc.pick_by_mass
    assert pb([0.5, 0.4, 0.0, 0.0], 0.95) == 1
    assert pb([0.0, 0.0, 0.0], 0.5) == 0
    assert pb([0.2, 0.3, 0.5], 0.0) == 0 and pb([0.2, 0.3, 0.5], 0.2) == 0
    assert pb([0.2, 0.3, 0.5], 0.21) == 1 and pb([0.2, 0.3, 0.5], 1.0) == 2
    assert pb([0.0, 1.0], 0.0) == 1


def test_out_of_vocabulary_recent_tokens_are_ignored(orc):
    # sampling.rs:219-232
    p = P(orc, temperature=0.0, repetition_penalty=1.5)
    assert orc.sample([0.5, -1.2, 2.3], p, [99])[0] == orc.sample([0.5, -1.2, 2.3], p, [])[0]


def test_top_p_one_equals_disabled(orc):
    # sampling.rs:251-264
    logits = [0.5, -1.2, 2.3, 0.0, 1.1]
    a, b = orc.Rng(5), orc.Rng(5)
    for _ in range(100):
        assert orc.sample_with_params(logits, P(orc), [], a) == orc.sample_with_params(logits, P(orc, top_p=1.0), [], b)


def test_temperature_only_matches_legacy_sampler(orc):
    # sampling.rs:266-297; the legacy draw uses the platform expf like the reference
    m = ctypes.CDLL(ctypes.util.find_library("m"))
    m.expf.argtypes = [ctypes.c_float]
    m.expf.restype = ctypes.c_float
    logits = np.array([0.5, -1.2, 2.3, 0.0, 1.1, -0.4], np.float32)
    temp = np.float32(0.8)

    def legacy(rng):
        mx = logits.max()
        p = np.array([m.expf(float(np.float32(np.float32(l - mx) / temp))) for l in logits], np.float32)
        s = np.cumsum(p, dtype=np.float32)[-1]
        p = (p / s).astype(np.float32)
        r = rng.next_f32()
        c = np.float32(0.0)
        for i, pi in enumerate(p):
            c = np.float32(c + pi)
            if r <= c:
                return i
        return len(p) - 1

    r1, r2 = orc.Rng(42), orc.Rng(42)
    for _ in range(200):
        assert legacy(r1) == orc.sample_with_params(logits, P(orc, temperature=0.8), [], r2)


def test_top_k_restricts_support(orc):
    # sampling.rs:300-318
    p = P(orc, temperature=1.0, top_k=2)
    rng = orc.Rng(7)
    for _ in range(500):
        assert orc.sample_with_params([5.0, 4.0, -2.0, -3.0, -5.0], p, [], rng) in (0, 1)


def test_top_p_nucleus_keeps_minimal_set(orc):
    # sampling.rs:321-336
    p = P(orc, temperature=1.0, top_p=0.5)
    rng = orc.Rng(3)
    for _ in range(500):
        assert orc.sample_with_params([10.0, 1.0, 0.5, 0.0], p, [], rng) == 0


def test_repetition_penalty_suppresses(orc):
    # sampling.rs:339-362
    p = P(orc, temperature=1.0, repetition_penalty=100.0)
    rng = orc.Rng(11)
    ones = sum(orc.sample_with_params([4.0, 3.0, -2.0], p, [0], rng) == 1 for _ in range(1000))
    assert ones > 800


def test_zero_temperature_is_argmax_and_draws_nothing(orc):
    # sampling.rs:365-389
    logits = [0.1, 2.0, 1.9, -1.0]
    for t in (0.0, -1.0):
        for s in range(20):
            assert orc.sample_with_params(logits, P(orc, temperature=t), [], orc.Rng(s)) == 1
    assert orc.sample_with_params(logits, P(orc, temperature=0.0, repetition_penalty=2.0), [1], orc.Rng(0)) == 2
    r = orc.Rng(3)
    before = r.next_u64()
    r2 = orc.Rng(3)
    orc.sample_with_params(logits, P(orc, temperature=0.0), [], r2)
    assert r2.next_u64() == before


# ---- mathematical pins ---------------------------------------------------------

def softmax64(l, t):
    z = (np.asarray(l, np.float64) - np.max(l)) / t
    e = np.exp(z)
    return e / e.sum()


def test_inverse_cdf_over_exhaustive_draw_grid(orc):
    """Token frequencies over an even grid of draws equal the softmax mass."""
    logits = np.array([0.3, -1.0, 2.0, 0.7, -0.2, 1.4, -3.0, 0.0], np.float32)
    t = 0.7
    G = 1 << 14
    draws = draws_for(np.arange(G) / G)
    counts = np.zeros(8)
    for d in draws:
        counts[orc.sample(logits, P(orc, temperature=t), [], d)[0]] += 1
    assert np.abs(counts / G - softmax64(logits, t)).max() < 2.0 / G + 1e-5


def test_top_k_support_is_the_k_largest(orc):
    rng = np.random.default_rng(4)
    for trial in range(40):
        n = int(rng.integers(5, 400))
        logits = (rng.standard_normal(n) * 3).astype(np.float32)
        k = int(rng.integers(1, n))
        top = set(np.argsort(-logits.astype(np.float64), kind="stable")[:k].tolist())
        seen = set()
        for r in np.linspace(0, 1, 257):
            tok, info = orc.sample(logits, P(orc, temperature=1.3, top_k=k), [], draws_for([r])[0])
            seen.add(tok)
        assert seen <= top


def test_top_p_support_is_the_minimal_prefix(orc):
    rng = np.random.default_rng(5)
    for trial in range(40):
        n = int(rng.integers(3, 300))
        logits = (rng.standard_normal(n) * 2).astype(np.float32)
        tp = float(rng.uniform(0.05, 0.99))
        p = softmax64(logits, 0.9)
        order = np.argsort(-p, kind="stable")
        cum = np.cumsum(p[order])
        c = int(np.searchsorted(cum, tp))  # first position with cum >= tp
        if min(abs(cum[c] - tp), abs(cum[c - 1] - tp) if c else 1.0) < 1e-5:
            continue  # decision margin too small for a float64 restatement
        nucleus = set(order[: c + 1].tolist())
        mass = p[list(nucleus)].sum()
        G = 512
        counts = {}
        for r in (np.arange(G) + 0.5) / G:
            tok, info = orc.sample(logits, P(orc, temperature=0.9, top_p=tp), [], draws_for([r])[0])
            counts[tok] = counts.get(tok, 0) + 1
        assert set(counts) <= nucleus
        for tok, cnt in counts.items():
            assert abs(cnt / G - p[tok] / mass) < 2.0 / G + 1e-4


def test_penalty_applies_once_per_occurrence(orc):
    """Two occurrences divide a positive logit twice; negatives are multiplied."""
    logits = np.array([2.0, -1.0, 0.5, 0.0], np.float32)
    pen = np.float32(1.7)
    pen_l = logits.copy()
    pen_l[0] = np.float32(np.float32(logits[0] / pen) / pen)
    pen_l[1] = np.float32(logits[1] * pen)
    G = 1 << 13
    counts = np.zeros(4)
    for d in draws_for(np.arange(G) / G):
        counts[orc.sample(logits, P(orc, temperature=1.0, repetition_penalty=1.7), [0, 1, 0, 9], d)[0]] += 1
    assert np.abs(counts / G - softmax64(pen_l, 1.0)).max() < 2.0 / G + 1e-5
    # zero logit: l > 0 is false, so it is multiplied (stays zero)
    assert orc.sample([0.0, -5.0], P(orc, temperature=0.0, repetition_penalty=3.0), [0])[0] == 0


def test_fallback_draws_u64_mod_n(orc):
    # sampling.rs:158-168: a NaN or vanishing softmax mass falls back to next_u64 % n
    for logits in ([float("nan")] * 5, [float("-inf")] * 5, [float("inf"), 0.0, 1.0, 2.0, 3.0]):
        for d in (0, 7, 123456789012345):
            tok, info = orc.sample(logits, P(orc, temperature=1.0), [], d)
            assert info.path == orc.PATH_FALLBACK and tok == d % 5


def test_margins_are_reported(orc):
    tok, info = orc.sample([1.0, 1.0 + 1e-7, 0.0], P(orc, temperature=0.0))
    assert info.path == orc.PATH_GREEDY and info.greedy_gap < 1e-6
    tok, info = orc.sample([0.0, 0.0, 0.0, 0.0], P(orc, temperature=1.0, top_p=0.6), [], draws_for([0.3])[0])
    assert info.topp_tie == 1 and info.margin == 0.0
