"""The oracle against the reference's own known-answer tests
(tests/sampling.spec.ts:13-146) and against closed forms the mathematics fixes."""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle.oracle import Decoding

DEFAULT = Decoding()


def d(**kw):
    c = Decoding()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_temperature_zero_is_greedy(oracle):  # sampling.spec.ts:13-15
    assert oracle.sample_token([0.2, 4, 1], [], d(temperature=0), 0.5)[0] == 1


def test_top_k_one_is_deterministic(oracle):  # sampling.spec.ts:17-19
    assert oracle.sample_token([0.2, 4, 1], [], d(topK=1), 0.99)[0] == 1


def test_seeded_sampling_is_reproducible(oracle):  # sampling.spec.ts:21-28
    cfg = d(topK=0, topP=1)
    a = [oracle.sample_token([1, 1, 1], [], cfg, oracle.draw(71, i))[0] for i in range(20)]
    b = [oracle.sample_token([1, 1, 1], [], cfg, oracle.draw(71, i))[0] for i in range(20)]
    assert a == b
    # three equal logits: token = floor(3u) up to the cursor walk's rounding
    for i in range(20):
        u = oracle.draw(71, i)
        assert a[i] == min(2, int(u * 3)) or abs(u * 3 - round(u * 3)) < 1e-12


def test_repetition_penalty_moves_selection(oracle):  # sampling.spec.ts:30-32
    assert oracle.sample_token([2, 1.5], [0], d(temperature=0, repetitionPenalty=2), 0)[0] == 1


def test_zero_window_disables_penalties(oracle):  # sampling.spec.ts:34-46
    assert oracle.sample_token([2, 1.5], [0], d(temperature=0, repetitionPenalty=2, repetitionWindow=0), 0)[0] == 0


def test_presence_and_frequency_penalties(oracle):  # sampling.spec.ts:86-103
    cfg = d(temperature=0, repetitionPenalty=1, repetitionWindow=2, presencePenalty=0.1, frequencyPenalty=0.3)
    assert oracle.sample_token([2, 1.5], [0, 0], cfg, 0)[0] == 1
    cfg2 = d(temperature=0, repetitionPenalty=1, repetitionWindow=1, presencePenalty=0.5, frequencyPenalty=0)
    assert oracle.sample_token([2, 2.1], [0, 1], cfg2, 0)[0] == 0


def test_min_p(oracle):  # sampling.spec.ts:105-115
    cfg = d(temperature=1, topK=0, topP=1, typicalP=1, minP=0.6)
    assert oracle.sample_token([math.log(0.6), math.log(0.3), math.log(0.1)], [], cfg, 0.99)[0] == 0


def test_top_p(oracle):  # sampling.spec.ts:117-127
    cfg = d(temperature=1, topK=0, topP=0.5, minP=0, typicalP=1)
    assert oracle.sample_token([math.log(0.6), math.log(0.3), math.log(0.1)], [], cfg, 0.99)[0] == 0


def test_typical_p(oracle):  # sampling.spec.ts:129-139
    cfg = d(temperature=1, topK=0, topP=1, minP=0, typicalP=0.3)
    assert oracle.sample_token([math.log(0.45), math.log(0.4), math.log(0.15)], [], cfg, 0.5)[0] == 1


def test_token_log_probability(oracle):  # sampling.spec.ts:141-146
    logits = [math.log(0.6), math.log(0.3), math.log(0.1)]
    assert oracle.token_log_probability(logits, 0) == pytest.approx(math.log(0.6), abs=5e-3)
    assert oracle.token_log_probability(logits, 2) == pytest.approx(math.log(0.1), abs=5e-3)
    assert math.isnan(oracle.token_log_probability(logits, 3))


# ---------------------------------------------------------------- closed forms


def test_uniform_categorical_is_inverse_cdf(oracle):
    """T=1, K=0, P=1 over logits log(w): the draw is the inverse CDF of w."""
    w = [Fraction(1, 10), Fraction(2, 10), Fraction(3, 10), Fraction(4, 10)]
    logits = [math.log(float(x)) for x in w]
    cfg = d(temperature=1, topK=0, topP=1, minP=0, typicalP=1, repetitionWindow=0)
    # sorted desc: ids 3,2,1,0 with mass .4 .3 .2 .1
    order = [3, 2, 1, 0]
    cum = [Fraction(4, 10), Fraction(7, 10), Fraction(9, 10), Fraction(1)]
    for k in range(1, 1000):
        u = k / 1000
        t, tr = oracle.sample_token(logits, [], cfg, u)
        idx = next(i for i, c in enumerate(cum) if Fraction(u) <= c)
        # the walk's rounding can move exact breakpoints by an ulp; skip those u
        if any(abs(Fraction(u) - c) < Fraction(1, 10 ** 12) for c in cum):
            continue
        assert t == order[idx], (u, t)
        assert tr.probability == pytest.approx(float(w[order[idx]]), rel=1e-15)


def test_softmax_probability_closed_form(oracle):
    """probability = exp(l_i/T - max) / sum_j exp(l_j/T - max) for the chosen id."""
    rng = np.random.default_rng(3)
    for _ in range(20):
        x = rng.normal(0, 3, 50).astype(np.float32)
        T = float(rng.uniform(0.3, 2))
        cfg = d(temperature=T, topK=5, topP=1, minP=0, typicalP=1, repetitionWindow=0)
        t, tr = oracle.sample_token(x, [], cfg, float(rng.random()))
        v = x.astype(np.float64) / T
        p = np.exp(v - v.max()) / np.exp(v - v.max()).sum()
        assert tr.probability == pytest.approx(p[t], rel=1e-13)
        assert t in np.argsort(-v, kind="stable")[:5]


def test_ties_resolve_by_ascending_id(oracle):
    x = np.array([1, 3, 3, 3, 2], dtype=np.float32)
    assert oracle.sample_token(x, [], d(temperature=0), 0)[0] == 1
    cfg = d(temperature=1, topK=2, topP=1, repetitionWindow=0)
    # top-2 of the stable order are ids 1 and 2, each half the mass
    assert oracle.sample_token(x, [], cfg, 0.25)[0] == 1
    assert oracle.sample_token(x, [], cfg, 0.75)[0] == 2


def test_top_k_one_equals_greedy_for_any_u(oracle):
    rng = np.random.default_rng(5)
    for _ in range(30):
        x = rng.normal(0, 2, 64).astype(np.float32)
        hist = rng.integers(0, 64, 10).tolist()
        g = oracle.sample_token(x, hist, d(temperature=0, repetitionPenalty=1.3, presencePenalty=0.2), 0)[0]
        k1 = oracle.sample_token(x, hist, d(temperature=0.9, topK=1, repetitionPenalty=1.3, presencePenalty=0.2),
                                 float(rng.random()))[0]
        assert g == k1


def test_penalty_formula_closed_form(oracle):
    """l' = (l<0 ? l*rp : l/rp) - (pp + count*fp) for every id of the window."""
    x = np.array([2.0, -1.0, 0.5, 3.0], dtype=np.float32)
    cfg = d(temperature=0, repetitionPenalty=2.0, presencePenalty=0.25, frequencyPenalty=0.5, repetitionWindow=3)
    # window = last 3 ids of [3, 0, 1, 1] = [0, 1, 1]: id0 count1, id1 count2
    # id0: 2/2 - (0.25+0.5) = 0.25 ; id1: -1*2 - (0.25+1.0) = -3.25 ; id2 0.5 ; id3 3.0
    assert oracle.sample_token(x, [3, 0, 1, 1], cfg, 0)[0] == 3
    x2 = np.array([2.0, -1.0, 0.5, 0.1], dtype=np.float32)
    assert oracle.sample_token(x2, [3, 0, 1, 1], cfg, 0)[0] == 2  # 0.5 > 0.25 > 0.1


def test_out_of_range_history_ids_are_skipped(oracle):
    x = np.array([1.0, 0.9], dtype=np.float32)
    cfg = d(temperature=0, repetitionPenalty=5, repetitionWindow=4)
    assert oracle.sample_token(x, [-1, 7, 262144, 99], cfg, 0)[0] == 0


def test_softcap_closed_form(oracle):
    """The final-logit softcap cap*tanh(x/cap) (no reference vectors: the
    reference declares the cap but never applies it) against the binary64
    closed form: within one binary32 ulp of the correctly rounded value, odd,
    saturating at +-cap, the identity to first order near 0, NaN kept."""
    rng = np.random.default_rng(21)
    x = np.concatenate([rng.normal(0, 25, 200000), rng.normal(0, 1e-3, 20000), rng.uniform(-400, 400, 20000)])
    x = x.astype(np.float32)
    for cap in (30.0, 50.0):
        got = oracle.softcap(x, cap).astype(np.float64)
        ref = cap * np.tanh(x.astype(np.float64) / cap)
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs(got - ref) <= ulp), cap
        assert np.array_equal(oracle.softcap(-x, cap), -oracle.softcap(x, cap))
    big = np.array([1e6, -1e6, np.inf, -np.inf], np.float32)
    assert oracle.softcap(big, 30.0).tolist() == [30.0, -30.0, 30.0, -30.0]
    tiny = np.array([1e-20, -3e-10], np.float32)
    assert np.array_equal(oracle.softcap(tiny, 30.0), tiny)
    assert np.isnan(oracle.softcap(np.array([np.nan], np.float32), 30.0)[0])
