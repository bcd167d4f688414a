"""The CPU restatement of bc-infer's sampler (oracle/bc_sample.c, crates/bc-infer/src/sample.rs),
pinned without running the reference: its own test (greedy_and_nucleus, sample.rs:78-89), the
published splitmix64 sequence behind uniform (sample.rs:74-81), and draws whose answers follow
from the algorithm's definition in closed form or in distribution."""
import ctypes
import ctypes.util
import math

import numpy as np
import pytest

import oracle as O

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


def test_reference_greedy_and_nucleus():
    """sample.rs:78-89, word for word."""
    scores = [0.1, 3.0, 2.9, -5.0]
    assert O.sample(scores, 0.0, 1.0, 0, 0) == 1
    assert all(O.sample(scores, 1.0, 0.01, 7, i) == 1 for i in range(20))
    picks = [O.sample(scores, 1.0, 0.95, 7, i) for i in range(200)]
    assert 1 in picks and 2 in picks and 3 not in picks
    assert picks == [O.sample(scores, 1.0, 0.95, 7, i) for i in range(200)], "seeded"


def test_uniform_is_the_first_splitmix64_output():
    """uniform(seed) = (splitmix64's first output from seed) >> 40 over 2^24; the generator is
    pinned by its published sequence in test_oracle.py."""
    for seed in (0, 1, 7, 1234567, GOLDEN, M64, 0xDEADBEEF12345678):
        z = O.splitmix64(seed, 1)[0]
        assert O.uniform(seed) == (z >> 40) / float(1 << 24)


def test_argmax_takes_the_first_highest():
    rng = np.random.default_rng(1)
    for n in (1, 2, 7, 1000):
        s = rng.integers(-3, 4, size=n).astype(np.float32)  # many ties
        assert O.argmax(s) == int(np.argmax(s))
    s = np.array([1.0, np.nan, 1.0, 0.5], np.float32)
    assert O.argmax(s) == 0, "NaN never wins, ties go to the first"
    s = np.array([np.nan, 2.0, 3.0], np.float32)
    assert O.argmax(s) == 0, "a NaN at index 0 is never passed (every comparison with it is false)"
    assert O.argmax(np.full(5, -np.inf, np.float32)) == 0


def draw_index(seed, step):
    return O.uniform(seed ^ ((step * GOLDEN) & M64))


def test_draw_in_closed_form():
    """p = [1, 1/2, 1/2] exactly (scores 0, -ln 2, -ln 2 at T = 1), top_p = 1: the nucleus is all
    three (masses 0.5, 0.75, 1), kept = 2, r = 2u; token 0 when u <= 1/2, token 1 (the first of
    the equal pair) when u <= 3/4, else token 2."""
    ln2 = float(np.float32(math.log(2.0)))
    scores = [0.0, -ln2, -ln2]
    assert O.sample(scores, 1.0, 1.0, 0, 0) in (0, 1, 2)
    for seed in (3, 99):
        for step in range(300):
            u = draw_index(seed, step)
            want = 0 if u <= 0.5 else (1 if u <= 0.75 else 2)
            assert O.sample(scores, 1.0, 1.0, seed, step) == want, (seed, step, u)


def test_nucleus_cut():
    """p = [1, 1/2, 1/4, 1/8] (total 15/8): running masses 8/15, 12/15, 14/15, 1. top_p 0.7 keeps
    two tokens, 0.85 three, 0.95 all four; a kept token's frequency is its share of the kept
    mass."""
    ln2 = math.log(2.0)
    scores = [0.0, -ln2, -2 * ln2, -3 * ln2]
    for top_p, n in ((0.7, 2), (0.85, 3), (0.95, 4)):
        picks = np.array([O.sample(scores, 1.0, top_p, 5, i) for i in range(4000)])
        assert set(picks.tolist()) == set(range(n)), top_p
        share = np.array([1, 0.5, 0.25, 0.125][:n]) / sum([1, 0.5, 0.25, 0.125][:n])
        freq = np.bincount(picks, minlength=n) / len(picks)
        assert np.abs(freq - share).max() < 0.03, (top_p, freq, share)


def test_frequencies_follow_the_tempered_softmax():
    """top_p = 1: token i is drawn with probability softmax(s / T)_i (chi-square, 20000 draws);
    a wrong temperature, sign or normalisation fails by far."""
    rng = np.random.default_rng(2)
    s = rng.standard_normal(6).astype(np.float32)
    T = 0.7
    p = np.exp((s - s.max()) / T)
    p /= p.sum()
    n = 20000
    picks = np.array([O.sample(s, T, 1.0, 11, i) for i in range(n)])
    obs = np.bincount(picks, minlength=6)
    chi2 = float(((obs - n * p) ** 2 / (n * p)).sum())
    assert chi2 < 30.0, (chi2, obs, n * p)  # 5 degrees of freedom: p < 1e-5 for a correct sampler


def test_exp_is_libm_expf_but_at_midpoints():
    """The restatement's exp (correctly rounded) against the C library's expf, the one the
    reference's f32::exp calls: equal but for rare arguments near a rounding midpoint, and then
    by one ulp."""
    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    libm.expf.argtypes = [ctypes.c_float]
    libm.expf.restype = ctypes.c_float
    xs = np.random.default_rng(3).uniform(-80.0, 0.0, 20000).astype(np.float32)
    ours = np.array([O.lib().bcs_exp(float(x)) for x in xs], np.float32)
    theirs = np.array([libm.expf(float(x)) for x in xs], np.float32)
    diff = ours.view(np.int32).astype(np.int64) - theirs.view(np.int32).astype(np.int64)
    assert np.abs(diff).max() <= 1
    assert np.count_nonzero(diff) <= 20, np.count_nonzero(diff)


@pytest.mark.parametrize("mistake", ["step", "shift"])
def test_a_planted_mistake_in_the_draw_is_caught(mistake):
    """The closed-form draw fails for a draw seeded without the step's golden-ratio mix, or
    with another bit window of the generator."""
    ln2 = float(np.float32(math.log(2.0)))
    scores = [0.0, -ln2, -ln2]
    bad = 0
    for step in range(200):
        if mistake == "step":
            u = O.uniform(5 ^ step)
        else:
            u = (O.splitmix64(5 ^ ((step * GOLDEN) & M64), 1)[0] >> 39 & 0xFFFFFF) / float(1 << 24)
        want = 0 if u <= 0.5 else (1 if u <= 0.75 else 2)
        bad += O.sample(scores, 1.0, 1.0, 5, step) != want
    assert bad > 20
