"""Pins the sampling oracle (oracle/cpu_sample.c) to published values, numpy
restatements built a different way (sorting and cumulative sums instead of the
key-space search) and the properties that define the filters. CPU only.
"""
from __future__ import annotations

import numpy as np
import pytest

import synth
from synth import SAMPLE_CASES, from_order_key_np, order_key_np, sample_logits

F32_MAX = float(np.finfo(np.float32).max)

# SplitMix64 seeded with 0: its first five outputs as published with the
# generator (Vigna's splitmix64.c reference values).
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC,
                    0x1B39896A51A8749B]
GAMMA = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def test_split_mix64_published_outputs(ora):
    # output c of the stream seeded with 0 mixes the state c * gamma
    for c, want in enumerate(SPLITMIX64_SEED0):
        assert ora.split_mix64((c * GAMMA) & M64) == want
        assert ora.counter_rng(0, c) == want  # CounterRng(seed, c) is output c of the stream at `seed`
    # the numpy restatement used for the synthetic logits agrees
    got = synth.split_mix64_np(np.array([(c * GAMMA) & M64 for c in range(5)], dtype=np.uint64))
    assert [int(v) for v in got] == SPLITMIX64_SEED0


def test_counter_uniform_grid_and_range(ora):
    us = np.array([ora.counter_uniform(7, c) for c in range(20000)], dtype=np.float64)
    assert np.all((us >= 0.0) & (us < 1.0))
    assert np.all(np.floor(us * 2 ** 24) == us * 2 ** 24)  # on the 2^-24 grid
    assert abs(us.mean() - 0.5) < 0.01 and abs(us.var() - 1.0 / 12.0) < 0.005
    assert ora.counter_uniform(0, 0) == (0xE220A8397B1DCDAF >> 40) / 2 ** 24


def test_argmax_first_maximum_and_floors(ora):
    rng = np.random.default_rng(1)
    for n in (1, 5, 1000, 4097):
        x = rng.normal(size=n).astype(np.float32)
        assert ora.argmax(x, -F32_MAX) == int(np.argmax(x))
        x = np.round(x)  # many ties
        assert ora.argmax(x, -np.inf) == int(np.argmax(x))
    x = np.full(10, -np.inf, np.float32)
    assert ora.argmax(x, -F32_MAX) == 0 and ora.argmax(x, -np.inf) == 0
    x[7] = -F32_MAX  # only values above the floor count
    assert ora.argmax(x, -F32_MAX) == 0 and ora.argmax(x, -np.inf) == 7
    x[3] = np.nan
    assert ora.argmax(x, -np.inf) == 7  # NaN never wins


def np_filter(logits: np.ndarray, t: float, k: int, p: float) -> np.ndarray:
    """The filter written from its definition with sorting, independently of the oracle."""
    n = logits.size
    if not t > 0:
        out = np.zeros(n, np.float32)
        out[int(np.argmax(logits))] = 1.0
        return out
    v = logits.astype(np.float32)
    if t != 1.0:
        v = v * (np.float32(1.0) / np.float32(t))
    if 1 < k < n:
        kth = from_order_key_np(np.sort(order_key_np(v))[::-1][k - 1])
        v = np.where(v < kth, np.float32(-np.inf), v).astype(np.float32)
    e = np.exp(v - v.max()).astype(np.float32)
    prob = e * np.float32(1.0 / e.astype(np.float64).sum())
    if 0 < p < 1:
        thr = 1.0 - float(np.float32(p))
        srt = np.sort(prob)
        cum = np.cumsum(srt.astype(np.float64))
        # mass at or below each distinct value = cum at its last occurrence
        last = np.r_[srt[1:] != srt[:-1], True]
        vals, mass = srt[last], cum[last]
        over = np.nonzero(mass > thr)[0]
        if over.size:
            prob = np.where(prob < vals[over[0]], np.float32(0.0), prob).astype(np.float32)
        if prob.max() == 0:
            prob[int(np.argmax(prob))] = 1.0
        prob = prob * np.float32(1.0 / prob.astype(np.float64).sum())
    return prob.astype(np.float32)


@pytest.mark.parametrize("case", SAMPLE_CASES, ids=[c[5] for c in SAMPLE_CASES])
@pytest.mark.parametrize("n", [4096, 151936])
def test_filter_matches_sorting_restatement(ora, case, n):
    t, k, p, seed, tie, _ = case
    logits = sample_logits(seed, tie, n)
    got, margin = ora.filter_to_probs(logits, t, k, p)
    want = np_filter(logits, t, k, p)
    assert margin > 1e-9, "top_p decision too close to call for two implementations"
    assert np.array_equal(got > 0, want > 0), "kept sets differ"
    # expf (glibc) and numpy's float32 exp may differ by an ulp or two
    assert np.all(np.abs(got.astype(np.float64) - want) <= 4 * 2.0 ** -23 * np.abs(want) + 1e-37)
    assert abs(got.astype(np.float64).sum() - 1.0) < 1e-5


def test_filter_properties(ora):
    logits = sample_logits(16, False, 4096)
    base, _ = ora.filter_to_probs(logits, 1.0, 0, 1.0)
    assert np.all(base > 0)
    # top_k keeps exactly the k largest (no ties in this data)
    probs, _ = ora.filter_to_probs(logits, 1.0, 40, 1.0)
    kept = np.nonzero(probs)[0]
    assert set(kept) == set(np.argsort(-logits, kind="stable")[:40])
    # ties at the threshold are all kept
    tl = sample_logits(21, True, 4096)
    probs, _ = ora.filter_to_probs(tl, 1.0, 8, 1.0)
    kth = np.sort(tl)[::-1][7]
    assert set(np.nonzero(probs)[0]) == set(np.nonzero(tl >= kth)[0]) and np.count_nonzero(probs) >= 8
    # top_p: dropped mass <= 1 - p, and dropping the smallest kept value too would exceed it
    for p in (0.05, 0.5, 0.9, 0.95):
        probs, _ = ora.filter_to_probs(logits, 1.0, 0, p)
        dropped = base[probs == 0].astype(np.float64).sum()
        smallest = base[probs > 0].min()
        assert dropped <= 1 - p + 1e-12
        assert dropped + base[base == smallest].astype(np.float64).sum() > 1 - p
    # temperature -> 0 approaches the one-hot; greedy is exactly the one-hot
    g, _ = ora.filter_to_probs(logits, 0.0, 0, 1.0)
    assert g[int(np.argmax(logits))] == 1.0 and g.sum() == 1.0
    cold, _ = ora.filter_to_probs(logits, 0.001, 0, 1.0)
    assert int(np.argmax(cold)) == int(np.argmax(logits)) and cold.max() > 0.5
    # a single surviving token gets probability 1
    one, _ = ora.filter_to_probs(logits, 1.0, 0, 1e-6)
    assert np.count_nonzero(one) == 1 and abs(float(one.max()) - 1.0) <= 2.0 ** -23


def np_inverse(probs: np.ndarray, u: float) -> int:
    cum = np.cumsum(probs.astype(np.float64))  # sequential, as the serial loop
    i = int(np.searchsorted(cum, float(np.float32(u)), side="right"))
    return i if i < probs.size else int(np.argmax(probs))


def test_inverse_sample_matches_cumsum(ora):
    rng = np.random.default_rng(3)
    for n in (1, 3, 1000, 151936):
        probs = rng.random(n).astype(np.float32)
        probs /= probs.sum()
        for u in list(rng.random(50).astype(np.float32)) + [0.0, np.float32(0.99999994)]:
            assert ora.inverse_sample(probs, float(u)) == np_inverse(probs, float(u))


def test_inverse_sample_exact_boundaries_and_fallback(ora):
    # dyadic probabilities: the running sums are exact, u on a boundary goes past it
    probs = np.array([0.25, 0.0, 0.125, 0.5, 0.125], np.float32)
    for u, want in [(0.0, 0), (0.25, 2), (0.2499999, 0), (0.375, 3), (0.875, 4), (0.9999, 4)]:
        assert ora.inverse_sample(probs, u) == want == np_inverse(probs, u)
    # total below u: the first maximum
    half = np.array([0.1, 0.2, 0.2, 0.0], np.float32)
    assert ora.inverse_sample(half, 0.75) == 1


def test_sample_token_greedy_draws_nothing(ora):
    logits = sample_logits(11, False, 4096)
    toks = {ora.sample_token(logits, 0.0, 0, 1.0, 11, c) for c in range(16)}
    assert toks == {int(np.argmax(logits))}
    # a sampled case draws several distinct tokens over 16 counters
    logits = sample_logits(13, False, 4096)
    toks = {ora.sample_token(logits, 1.0, 0, 1.0, 13, c) for c in range(16)}
    assert len(toks) > 1


def test_top_p_decision_rules_at_a_boundary(ora):
    """Where the three ways of comparing the top_p mass S(t) with 1 - top_p part.

    probs 2^-60, 0.25, 0.75 (exact in fp32) with top_p = 0.75, so 1 - top_p =
    0.25 exactly. Dropping {2^-60, 0.25} removes a mass of
    0.25 + 2^-60, just above 0.25: the exact rule (the oracle's) and the device
    kernel's 2^-62 grid both refuse that cut and drop only 2^-60, while the
    reference's double sums round 0.25 + 2^-60 to 0.25 (an ulp of 0.25 is 2^-54)
    and drop 0.25 as well. This build decides on the exact mass (a recorded
    deviation); the two differ only when S(t) lies within ~n * 2^-53 of
    1 - top_p."""
    tiny = 2.0 ** -60
    probs = np.array([tiny, 0.25, 0.75], np.float32)
    assert float(probs[0]) == tiny
    assert float(probs[0]) + 0.25 == 0.25  # the double sum loses the tiny mass

    def kept(top_p, rule):
        return (probs > np.float32(ora.top_p_cut(probs, top_p, rule))).tolist()

    assert kept(0.75, ora.TOPP_EXACT) == [False, True, True]
    assert kept(0.75, ora.TOPP_GRID62) == [False, True, True]
    assert kept(0.75, ora.TOPP_DOUBLE) == [False, False, True]
    # away from the boundary the rules agree: with 1 - top_p = 0.5 the mass
    # 2^-60 + 0.25 is well below it, and adding 0.75 well above
    for rule in (ora.TOPP_EXACT, ora.TOPP_GRID62, ora.TOPP_DOUBLE):
        assert kept(0.5, rule) == [False, False, True]


def test_top_p_rules_agree_on_random_distributions(ora):
    rng = np.random.default_rng(31)
    for trial in range(40):
        logits = rng.normal(0, 2, 4096).astype(np.float32)
        e = np.exp(logits - logits.max())
        probs = (e / e.sum()).astype(np.float32)
        top_p = float(rng.uniform(0.5, 0.99))
        kept = {tuple(np.flatnonzero(probs > np.float32(ora.top_p_cut(probs, top_p, r))))
                for r in (ora.TOPP_EXACT, ora.TOPP_GRID62, ora.TOPP_DOUBLE)}
        assert len(kept) == 1, trial
