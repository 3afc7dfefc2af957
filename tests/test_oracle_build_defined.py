"""Pins for the oracle's build-defined stages (penalties, logit bias, min-p,
grammar mask with nucleus), which have no reference function to compare
with: closed forms on exactly representable values, IEEE f32 arithmetic done
independently by numpy, identity parameters that must reduce the row sampler
to the reference's own nucleus_mask + sample_categorical (pinned by the
reference goldens in test_oracle_golden.py), and the single-legal-token and
min_p in {0, 1} limits."""
import math

import numpy as np
import pytest


def row(seed, n=64, scale=2.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * scale).astype(np.float32), rng


def test_identity_parameters_reduce_to_reference_composition(orc):
    for seed in range(40):
        x, rng = row(seed, n=200)
        T = float(rng.uniform(0.3, 1.5))
        top_p = float(rng.uniform(0.3, 1.0))
        top_k = int(rng.choice([0, 5, 20, 199, 200, 500]))
        u = float(rng.random())
        r = orc.sample_row(x, temperature=T, top_p=top_p, top_k=top_k, uniform=u)
        assert r["status"] == 0
        assert np.array_equal(r["adjusted"].view(np.uint32), x.view(np.uint32))
        st, mask = orc.nucleus_mask(x, T, top_p, top_k)
        assert st == 0
        assert np.array_equal(r["kept"], mask)
        st, tok, lp = orc.sample_categorical(x, mask.astype(np.uint8), T, u)
        assert st == 0 and r["token"] == tok and r["sampling_logprob"] == lp


def test_penalty_closed_forms(orc):
    x = np.array([4.0, -3.0, 1.0, 1.0, 8.0, 1.0, 5.0, 2.5], dtype=np.float32)
    r = orc.sample_row(x, temperature=1.0, uniform=0.5, repetition=2.0, presence=0.5, frequency=0.25,
                       history=[0, 1, 1, 4, 4, 4, 3, 5], bias_ids=[2, 3], bias_values=[0.5, 1.0])
    a = r["adjusted"]
    assert a[0] == 4.0 / 2 - 1 * 0.25 - 0.5            # 1.25: divide (l > 0), once per distinct token
    assert a[1] == -3.0 * 2 - 2 * 0.25 - 0.5           # -7.0: multiply (l < 0), count 2
    assert a[2] == 1.5                                 # bias only
    assert a[3] == (1.0 + 1.0) / 2 - 0.25 - 0.5        # 0.25: bias before the penalty
    assert a[4] == 8.0 / 2 - 3 * 0.25 - 0.5            # 2.75: count 3, repetition applied once
    assert a[5] == 1.0 / 2 - 0.25 - 0.5                # -0.25
    assert a[6] == 5.0 and a[7] == 2.5                 # untouched
    # a quotient that rounds: l / rep correctly rounded in f32 (IEEE, numpy)
    y = np.array([1.0, 0.7, -0.3], dtype=np.float32)
    r = orc.sample_row(y, temperature=1.0, uniform=0.1, repetition=3.0, history=[0, 1, 2])
    want = np.array([np.float32(1.0) / np.float32(3.0), np.float32(0.7) / np.float32(3.0),
                     np.float32(-0.3) * np.float32(3.0)], dtype=np.float32)
    assert np.array_equal(r["adjusted"].view(np.uint32), want.view(np.uint32))
    # frequency term rounds as (float)count * frequency, then two subtractions
    z = np.array([10.0], dtype=np.float32)
    r = orc.sample_row(z, temperature=1.0, uniform=0.1, frequency=0.1, presence=0.3, history=[0] * 7)
    step = np.float32(np.float32(10.0) - np.float32(7.0) * np.float32(0.1))
    assert r["adjusted"][0] == np.float32(step - np.float32(0.3))


def test_min_p_limits(orc):
    x = np.array([3.0, 1.0, 3.0, -2.0, 3.0, 0.5, 2.9], dtype=np.float32)
    for u in (0.0, 0.2, 0.5, 0.9, 0.999):
        r = orc.sample_row(x, temperature=0.7, min_p=1.0, uniform=u)
        # min_p = 1 keeps exactly the tokens tied at the maximum
        assert r["status"] == 0
        assert np.array_equal(np.nonzero(r["kept"])[0], [0, 2, 4])
        assert r["token"] in (0, 2, 4)
        assert math.isclose(r["sampling_logprob"], -math.log(3.0), rel_tol=1e-12)
        # min_p = 0 is no filter at all
        a = orc.sample_row(x, temperature=0.7, min_p=0.0, uniform=u)
        b = orc.sample_row(x, temperature=0.7, uniform=u)
        assert a["token"] == b["token"] and np.array_equal(a["kept"], b["kept"])


def test_min_p_threshold_and_order(orc):
    for seed in range(20):
        x, rng = row(100 + seed, n=300, scale=3.0)
        T = float(rng.uniform(0.4, 1.6))
        mp = float(rng.uniform(0.01, 0.5))
        r = orc.sample_row(x, temperature=T, top_p=1.0, min_p=mp, uniform=float(rng.random()))
        M = float(x.max())
        # p_i >= min_p * p_max  <=>  (l_i - M) / T >= ln(min_p), in f64
        want = ((x.astype(np.float64) - M) / T) >= math.log(mp)
        assert np.array_equal(r["kept"], want)
        # applied after the nucleus: a nucleus of one token stays one token
        top = orc.sample_row(x, temperature=T, top_p=1e-9, min_p=mp, uniform=0.3)
        assert top["kept"].sum() == 1 and top["token"] == int(np.argmax(x))


def test_mask_with_nucleus_is_the_nucleus_of_the_legal_row(orc):
    for seed in range(30):
        x, rng = row(200 + seed, n=160)
        legal = rng.random(160) < 0.3
        legal[int(rng.integers(160))] = True
        words = np.zeros(5, dtype=np.uint32)
        for i in np.nonzero(legal)[0]:
            words[i // 32] |= np.uint32(1 << (i % 32))
        T = float(rng.uniform(0.3, 1.5))
        top_p = float(rng.uniform(0.3, 1.0))
        k = int(rng.choice([0, 3, int(legal.sum()), 1000]))
        u = float(rng.random())
        r = orc.sample_row(x, temperature=T, top_p=top_p, top_k=k, uniform=u, mask_words=words)
        ids = np.nonzero(legal)[0]
        compact = x[ids]
        st, m = orc.nucleus_mask(compact, T, top_p, k)
        st2, pick, lp = orc.sample_categorical(compact, m.astype(np.uint8), T, u)
        assert r["status"] == 0 and st == 0 and st2 == 0
        assert r["token"] == ids[pick] and r["sampling_logprob"] == lp
        kept = np.zeros(160, dtype=bool)
        kept[ids[m]] = True
        assert np.array_equal(r["kept"], kept)


def test_single_legal_token_wins_for_every_uniform(orc):
    x, rng = row(300, n=96)
    words = np.zeros(3, dtype=np.uint32)
    words[1] = np.uint32(1 << 7)    # token 39 only
    for u in (0.0, 0.25, 0.5, 0.999999):
        for T, p, k in ((0.3, 0.1, 0), (1.0, 1.0, 5), (1.7, 0.95, 0)):
            r = orc.sample_row(x, temperature=T, top_p=p, top_k=k, uniform=u, mask_words=words)
            assert r["status"] == 0 and r["token"] == 39 and r["kept_count"] == 1
            assert r["sampling_logprob"] == 0.0


def test_build_defined_error_precedence(orc):
    x, _ = row(400, n=16)
    s = lambda **kw: orc.sample_row(x, **{"temperature": 1.0, "uniform": 0.5, **kw})["status"]
    assert s(temperature=-1.0, top_p=2.0) == -4            # temperature first
    assert s(top_p=0.0, min_p=2.0) == -8                   # then top_p
    assert s(min_p=1.5, repetition=0.0) == -9              # then min_p
    assert s(repetition=0.0, history=[99]) == -10          # then penalties
    assert s(presence=float("inf")) == -10
    assert s(history=[3, 16]) == -11                       # history id outside the row
    assert s(bias_ids=[4, 4], bias_values=[1.0, 1.0]) == -12   # not strictly increasing
    assert s(bias_ids=[2], bias_values=[float("nan")]) == -12
    assert s(history=[16], bias_ids=[3, 2], bias_values=[1.0, 1.0]) == -11
    assert s(uniform=1.0, bias_ids=[3, 2], bias_values=[1.0, 1.0]) == -12
    y = x.copy()
    y[5] = 3e38
    assert orc.sample_row(y, temperature=1.0, uniform=0.5, bias_ids=[5], bias_values=[3e38])["status"] == -6
    assert s(uniform=1.0) == -5


def test_suppression_is_the_reference_f32_min_write(orc):
    """A bias entry of -inf (suppression) must give what the reference's
    ChatFormat::suppress gives: the logit written as f32::MIN before the
    pick (crates/core/chat-format/src/lib.rs:771-780), here checked on rows
    without other bias or penalties against the oracle run on the rewritten
    row, for sampling, greedy and top-k/top-p rules; with penalties and a
    bias on the same row, the suppressed tokens still read f32::MIN."""
    fmin = np.float32(-3.4028234663852886e38)
    for seed in range(30):
        x, rng = row(300 + seed, n=96)
        sup = np.unique(rng.integers(0, 96, int(rng.integers(1, 12))))
        if seed % 3 == 0:
            sup = np.unique(np.concatenate([sup, [int(np.argmax(x))]]))   # the argmax is suppressed
        y = x.copy()
        y[sup] = fmin
        T = [0.0, 0.7, 1.3][seed % 3]
        kw = dict(temperature=T, top_p=float(rng.uniform(0.5, 1.0)), top_k=int(rng.choice([0, 5, 40])),
                  uniform=float(rng.random()))
        a = orc.sample_row(x, bias_ids=sup, bias_values=np.full(sup.size, -np.inf, np.float32), **kw)
        b = orc.sample_row(y, **kw)
        for k in ("status", "token", "sampling_logprob", "kept_count"):
            assert a[k] == b[k], (seed, k, a[k], b[k])
        assert np.array_equal(a["adjusted"].view(np.uint32), y.view(np.uint32))
        assert np.array_equal(a["kept"], b["kept"])
    # every token suppressed: all logits equal f32::MIN; greedy takes ID 0
    x, rng = row(7, n=50)
    allids = np.arange(50)
    g = orc.sample_row(x, temperature=0.0, bias_ids=allids, bias_values=np.full(50, -np.inf, np.float32))
    assert g["status"] == 0 and g["token"] == 0
    # with penalties and a bias elsewhere: suppressed ids read f32::MIN, the rest as before
    r = orc.sample_row(x, temperature=1.0, uniform=0.3, repetition=1.3, presence=0.2, frequency=0.1,
                       history=[3, 3, 4, 9], bias_ids=[3, 4, 20], bias_values=[-np.inf, 0.5, -np.inf])
    q = orc.sample_row(x, temperature=1.0, uniform=0.3, repetition=1.3, presence=0.2, frequency=0.1,
                       history=[3, 3, 4, 9], bias_ids=[4], bias_values=[0.5])
    assert r["status"] == 0
    assert r["adjusted"][3] == fmin and r["adjusted"][20] == fmin
    other = np.setdiff1d(np.arange(50), [3, 20])
    assert np.array_equal(r["adjusted"][other].view(np.uint32), q["adjusted"][other].view(np.uint32))
    # +inf and NaN bias values stay invalid
    for bad in (np.inf, np.nan):
        z = orc.sample_row(x, temperature=1.0, uniform=0.3, bias_ids=[1], bias_values=[bad])
        assert z["status"] == -12   # ORC_INVALID_BIAS
