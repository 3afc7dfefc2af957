"""Pins the CPU oracle to the reference's own known answers (CPU only).

Every expected value below is transcribed from the arclabs561/metallix test
suites (tests/golden/reference_vectors.json cites file:line), or fixed by
mathematics independent of the oracle's code (closed forms, brute force on
tiny inputs, exact laws).
"""
import itertools
import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
F32_MAX = float(np.finfo(np.float32).max)
ONE_MINUS_ULP = float.fromhex("0x1.fffffffffffffp-1")


def bits(x: float) -> str:
    return "0x%016x" % np.array(x, dtype=np.float64).view(np.uint64)


# ---- entropy ---------------------------------------------------------------
def test_icdf_v1_golden_tokens(orc):
    g = GOLD["icdf_v1"]
    rng = orc.ChaChaStream(g["seed"])
    toks = []
    for d in range(24):
        u = orc.unit_uniform(rng.next_u64())
        st, tok, _ = orc.sample_categorical(g["rows"][d % 3], None, g["temperature"], u)
        assert st == 0
        toks.append(tok)
    assert toks == g["tokens"]


def test_unit_uniform_bits(orc):
    for word, expect in GOLD["unit_uniform"]["cases"]:
        assert bits(orc.unit_uniform(word)) == expect
    for bit in range(64):
        expect = 0.0 if bit < 11 else 2.0 ** (bit - 64)
        assert bits(orc.unit_uniform(1 << bit)) == bits(expect)


# ---- sample_categorical (sampling.rs:160-379) -------------------------------
def enumerate_policy(logits, legal, t):
    w = [math.exp(float(np.float32(l)) / t) if ok else 0.0 for l, ok in zip(logits, legal)]
    s = sum(w)
    return [x / s for x in w]


def oracle_token(probs, u):
    cum = 0.0
    last = None
    for i, p in enumerate(probs):
        cum += p
        if p > 0:
            last = i
        if u < cum:
            return i
    return last


def test_hand_computed_distribution(orc):
    ln2 = GOLD["sample_categorical"]["ln2_f32"]
    ratio = math.exp(ln2)
    st, tok, lp = orc.sample_categorical([0.0, ln2], [1, 1], 1.0, 0.2)
    assert (st, tok) == (0, 0) and abs(lp - math.log(1 / (1 + ratio))) < 1e-12
    st, tok, lp = orc.sample_categorical([0.0, ln2], [1, 1], 1.0, 0.4)
    assert (st, tok) == (0, 1) and abs(lp - math.log(ratio / (1 + ratio))) < 1e-12
    st, tok, lp = orc.sample_categorical([0.0, ln2], [1, 1], 2.0, 0.5)
    r2 = math.exp(ln2 / 2)
    assert tok == 1 and abs(lp - math.log(r2 / (1 + r2))) < 1e-12


def test_uniform_boundaries_and_masking(orc):
    assert orc.sample_categorical([0.0, 0.0], [1, 1], 1.0, 0.0)[1] == 0
    assert orc.sample_categorical([0.0, 0.0], [1, 1], 1.0, 0.5)[1] == 1
    assert orc.sample_categorical([0.0, 0.0], [1, 1], 1.0, ONE_MINUS_ULP)[1] == 1
    st, tok, lp = orc.sample_categorical([0.0, 100.0, 2.0, 1000.0], [1, 0, 1, 0], 1.0, 0.2)
    assert tok == 2 and abs(lp + math.log(1 + math.exp(-2.0))) < 1e-12
    st, tok, lp = orc.sample_categorical([-F32_MAX, F32_MAX], [1, 1], 1.0, 0.5)
    assert tok == 1 and abs(lp) < 1e-12


def test_independent_f64_definition(orc):
    ln2 = GOLD["sample_categorical"]["ln2_f32"]
    cases = [([0.0, 0.0, 100.0, -100.0], [1, 1, 0, 0], 1.0, [0.0, 0.5, ONE_MINUS_ULP]),
             ([0.0, ln2, 2 * ln2], [1, 1, 1], 0.5, [0.0, 0.1, 0.5, 0.99]),
             ([0.0, -20.0], [1, 1], 1.0, [0.0, 1.0 - 1e-10])]
    for logits, legal, t, us in cases:
        probs = enumerate_policy(logits, legal, t)
        for u in us:
            st, tok, lp = orc.sample_categorical(logits, legal, t, u)
            exp = oracle_token(probs, u)
            assert st == 0 and tok == exp
            assert abs(lp - math.log(probs[exp])) < 1e-12


def test_error_matrix(orc):
    assert orc.sample_categorical([0.0], [0], 1.0, 0.0)[0] == -3
    for t in (0.0, -1.0, math.nan, math.inf):
        assert orc.sample_categorical([0.0], [1], t, 0.0)[0] == -4
    for u in (-1.0, 1.0, math.nan, math.inf):
        assert orc.sample_categorical([0.0], [1], 1.0, u)[0] == -5
    for l in (math.nan, math.inf, -math.inf):
        assert orc.sample_categorical([l], [1], 1.0, 0.0)[0] == -6
        assert orc.sample_categorical([0.0, l], [1, 0], 1.0, 0.0)[0] == -6
    assert orc.sample_categorical([0.0, F32_MAX], [1, 1], 2.2250738585072014e-308, 0.0)[0] == -4


def test_seeded_stream_matches_independent_enumeration(orc):
    # qwen_forward.rs:2204-2238: seed 41, T 0.7, logits [0, 1, -2]
    rng = orc.ChaChaStream(41)
    expect_rng = orc.ChaChaStream(41)
    logits = [0.0, 1.0, -2.0]
    for _ in range(8):
        word = expect_rng.next_u64()
        high, low = word >> 32, (word >> 11) & ((1 << 21) - 1)
        u = (high * 2097152.0 + low) / 9007199254740992.0
        w = [math.exp(l / 0.7) for l in logits]
        n = sum(w)
        target, cum, exp = u * n, 0.0, None
        for i, x in enumerate(w):
            cum += x
            if target < cum:
                exp = i
                break
        st, tok, lp = orc.sample_categorical(logits, None, 0.7, orc.unit_uniform(rng.next_u64()))
        assert tok == exp and abs(lp - math.log(w[exp] / n)) < 1e-12


# ---- nucleus_mask (qwen_forward.rs:2491-2552) --------------------------------
def test_nucleus_kept_set_table(orc):
    g = GOLD["nucleus_table"]
    for case in g["cases"]:
        st, kept = orc.nucleus_mask(g["logits"], case["temperature"], case["top_p"], case["top_k"])
        assert st == 0 and list(kept) == case["kept"], case
    assert orc.nucleus_mask(g["logits"], 1.0, g["invalid_top_p"])[0] != 0


def test_seeded_nucleus_stays_in_nucleus(orc):
    logits = [(i * 37 % 17) / 4.0 for i in range(64)]
    st, nucleus = orc.nucleus_mask(logits, 0.8, 0.6, 0)
    assert nucleus.sum() > 1
    rng = orc.ChaChaStream(11)
    for _ in range(200):
        st, tok, _ = orc.sample_categorical(logits, nucleus, 0.8, orc.unit_uniform(rng.next_u64()))
        assert nucleus[tok]


def _by_logit(logits):
    keys = [np.array(l, dtype=np.float32).view(np.int32).item() for l in logits]
    keys = [k ^ ((k >> 31) & 0x7FFFFFFF) for k in keys]
    return sorted(range(len(logits)), key=lambda i: (-keys[i], i))


def test_top_k_candidates_sample_what_the_whole_row_samples(orc):
    # qwen_forward.rs:2572-2605: the compact, ID-sorted candidate row draws the
    # same token as the whole row whenever the candidates settle the head.
    logits = np.array([(i * 7919 % 997) / 90.0 for i in range(3000)], dtype=np.float32)
    order = _by_logit(logits)
    for t, p, k in [(0.6, 0.95, 20), (1.0, 0.3, 5), (1.7, 1.0, 64)]:
        count = next(c for c in range(k + 1, 3000) if logits[order[k - 1]] > logits[order[c - 1]])
        ids = sorted(order[:count])
        compact = logits[ids]
        whole_rng, comp_rng = orc.ChaChaStream(5), orc.ChaChaStream(5)
        st, whole_mask = orc.nucleus_mask(logits, t, p, k)
        st, comp_mask = orc.nucleus_mask(compact, t, p, k)
        for _ in range(300):
            _, a, _ = orc.sample_categorical(logits, whole_mask, t, orc.unit_uniform(whole_rng.next_u64()))
            _, b, _ = orc.sample_categorical(compact, comp_mask, t, orc.unit_uniform(comp_rng.next_u64()))
            assert a == ids[b]


def nucleus_definition(logits, t, top_p, top_k):
    """nucleus_mask restated from its documentation (tokens in descending
    logit order, ID order on ties, the first top_k, until their mass reaches
    top_p of the kept mass), summed with Python floats in that order."""
    n = len(logits)
    x = [float(np.float32(v)) for v in logits]
    if top_p >= 1.0 and not (0 < top_k < n):
        return [True] * n
    m = max(x)
    w = [math.exp((v - m) / t) for v in x]
    order = _by_logit(logits)
    if 0 < top_k < n:
        head = order[:top_k]
        target = top_p * sum(w[i] for i in head)
    else:
        head = order
        target = top_p * sum(w)
    mask, cov = [False] * n, 0.0
    for i in head:
        mask[i] = True
        cov += w[i]
        if cov >= target:
            break
    return mask


def test_nucleus_brute_force_tiny_rows(orc):
    rng = np.random.default_rng(5)
    for trial in range(400):
        n = int(rng.integers(1, 9))
        vals = rng.choice([-1.0, -0.0, 0.0, 0.5, 1.0, 2.0, 3.0], size=n).astype(np.float32)
        t = float(rng.choice([0.3, 1.0, 2.5]))
        p = float(rng.choice([0.2, 0.5, 0.9, 1.0]))
        k = int(rng.integers(0, n + 2))
        st, kept = orc.nucleus_mask(vals, t, p, k)
        assert st == 0
        assert list(kept) == nucleus_definition(vals, t, p, k), (vals, t, p, k)


# ---- greedy / masked argmax / mask layout ------------------------------------
def test_greedy_ties_and_finiteness(orc):
    assert orc.greedy_token([3.0, 3.0]) == (0, 0)
    assert orc.greedy_token([-0.0, 0.0, -1.0]) == (0, 0)
    assert orc.greedy_token([0.0, math.nan])[0] == -6
    st, lp = orc.selected_model_logprob([3.0, 3.0], 0)
    assert abs(lp + math.log(2)) < 1e-12
    st, lp = orc.selected_model_logprob([-F32_MAX, F32_MAX], 1)
    assert abs(lp) < 2.3e-16


def test_masked_argmax_matches_row_scan(orc):
    rng = np.random.default_rng(7)
    for _ in range(300):
        width = int(rng.integers(1, 200))
        dense = rng.random(7) < 0.3
        sparse = rng.random(224) < 0.5
        vals = rng.integers(-3, 4, size=224)
        logits = np.array([(-0.0 if (v == 0 and i % 2 == 0) else float(v)) for i, v in enumerate(vals)], dtype=np.float32)
        words = np.zeros(7, dtype=np.uint32)
        for i in range(224):
            if sparse[i] or dense[i // 32]:
                words[i // 32] |= np.uint32(1 << (i % 32))
        expect = None
        for i in range(width):
            if (words[i // 32] >> (i % 32)) & 1 and (expect is None or logits[i] > logits[expect]):
                expect = i
        got = orc.masked_argmax(words, logits, width)
        assert got == (-1 if expect is None else expect)


def test_fill_legal_mask_layout(orc):
    words = np.array([0b1011, 0x80000001, 0xFFFFFFFF], dtype=np.uint32)
    legal = orc.fill_legal_mask(words, 70, 96)
    expect = np.zeros(96, dtype=bool)
    expect[[0, 1, 3, 32, 63]] = True
    expect[64:70] = True
    assert (legal == expect).all()


def test_token_logprob_top_matches_sort(orc):
    rng = np.random.default_rng(3)
    x = rng.integers(-5, 6, size=500).astype(np.float32)
    st, ids, lps, m, ln = orc.token_logprob_top(x, 28)
    order = _by_logit(x)[:28]
    assert list(ids) == order
    lse = math.log(sum(math.exp(float(v) - 5.0) for v in x))
    for i, lp in zip(ids, lps):
        assert abs(lp - (float(x[i]) - 5.0 - lse)) < 1e-12
    eq = np.zeros(1000, dtype=np.float32)
    st, ids, lps, m, ln = orc.token_logprob_top(eq, 3)
    assert list(ids) == [0, 1, 2] and abs(lps[0] + math.log(1000)) < 1e-12


# ---- race-v2 (race.rs:221-374) -------------------------------------------------
def test_philox_known_answers(orc):
    for c, k, e in GOLD["philox_kat"]["cases"]:
        assert orc.philox4x32_10(c, k) == e


def test_race_noise_vectors(orc):
    g = GOLD["race_noise"]
    for row, b, noise in g["cases"]:
        got = orc.race_bits(g["seed"], g["choice"], g["position"], row)
        assert got == int(b, 16)
        expect = float(np.array(int(noise, 16), dtype=np.uint64).view(np.float64))
        assert abs(orc.gumbel_from_bits(got) - expect) < 1e-15
    for b in (0, 1, (1 << 63) - 1, 1 << 63, (1 << 64) - 2, (1 << 64) - 1):
        assert -3.81 <= orc.gumbel_from_bits(b) < 45.06


def test_race_golden_tokens(orc):
    g = GOLD["race_golden"]
    toks = [orc.sample_race(g["logits"], g["legal"], g["temperature"], g["seed"], g["choice"], pos)[1]
            for pos in range(24)]
    assert toks == g["tokens"]


def test_race_temperature_law(orc):
    logits = [0.3, -0.6, 1.1, 0.0, 0.7, 2.0]
    legal = [1, 1, 1, 1, 1, 0]
    counts = [0] * 6
    for pos in range(30000):
        counts[orc.sample_race(logits, legal, 0.6, 11, 0, pos)[1]] += 1
    assert counts[5] == 0
    w = [math.exp(l / 0.6) for l in logits[:5]]
    tot = sum(w)
    chi = sum((c - x / tot * 30000) ** 2 / (x / tot * 30000) for c, x in zip(counts, w))
    assert chi < 40.0


# ---- accept_or_resample (speculative.rs:369-444) --------------------------------
def test_accept_or_resample_units(orc):
    g = GOLD["accept_or_resample"]
    assert orc.accept_or_resample(g["target"], g["draft"], 0, 0.999, 0.0) == (0, "accepted")
    for u in (0.0, 0.3, 0.6, 0.999):
        st, v = orc.accept_or_resample(g["target"], g["draft"], 2, 0.0, u)
        assert st == 0 and v[0] == "resampled" and v[1] in (0, 1)
    assert orc.accept_or_resample(g["target"], g["draft"], 3, 0.0, 0.0)[0] == -13
    assert orc.accept_or_resample(g["target"], g["draft"][:2], 0, 0.0, 0.0)[0] == -14
    assert orc.accept_or_resample(g["target"], g["draft"], 0, 1.0, 0.0)[0] == -5


class SplitMix:
    def __init__(self, s):
        self.s = s

    def next_u64(self):
        self.s = (self.s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def uniform(self):
        return (self.next_u64() >> 11) / float(1 << 53)


def toy_logits(context):
    last = context[-1]
    before = context[-2] if len(context) >= 2 else 0
    length = len(context)
    out = []
    for tok in range(3):
        mix = (last * 7 + before * 3 + tok * 5 + length) % 11
        out.append(float(np.float32(np.float32(mix) * np.float32(0.37))) - (0.8 if tok == last else 0.0))
    return [float(np.float32(v)) for v in out]


def test_stochastic_draft_rule_matches_exact_sequence_law(orc):
    # speculative/tests.rs:512-566 with a reduced sample count and a bound
    # scaled to it: drafts from a wrong q, verified by accept_or_resample,
    # must reproduce the target's exact 4-token sequence law.
    T, VOCAB, PROMPT, LENGTH, SAMPLES = 0.8, 3, [0, 2, 1], 4, 12000
    probs = lambda ctx: [w / s for w, s in ((x, sum(math.exp(v / T) for v in toy_logits(ctx))) for x in (math.exp(v / T) for v in toy_logits(ctx)))]

    def qdist(ctx):
        q = [0.15] * VOCAB
        q[(ctx[-1] + 1) % VOCAB] = 0.7
        return q

    def cat(p, u):
        cum = 0.0
        for i, x in enumerate(p):
            cum += x
            if u < cum:
                return i
        return len(p) - 1

    rng = SplitMix(21)
    counts = {}
    for _ in range(SAMPLES):
        ctx = list(PROMPT)
        while len(ctx) < len(PROMPT) + LENGTH:
            drafts, dctx = [], list(ctx)
            for _ in range(min(3, len(PROMPT) + LENGTH - len(ctx))):
                q = qdist(dctx)
                t = cat(q, rng.uniform())
                drafts.append((t, q))
                dctx.append(t)
            all_ok = True
            for t, q in drafts:
                p = probs(ctx)
                st, v = orc.accept_or_resample(p, q, t, rng.uniform(), rng.uniform())
                assert st == 0
                if v == "accepted":
                    ctx.append(t)
                else:
                    ctx.append(v[1])
                    all_ok = False
                    break
            if all_ok and len(ctx) < len(PROMPT) + LENGTH:
                ctx.append(cat(probs(ctx), rng.uniform()))
        key = tuple(ctx[len(PROMPT):])
        counts[key] = counts.get(key, 0) + 1
    chi = 0.0
    for seq in itertools.product(range(VOCAB), repeat=LENGTH):
        ctx, pr = list(PROMPT), 1.0
        for tok in seq:
            pr *= probs(ctx)[tok]
            ctx.append(tok)
        e = pr * SAMPLES
        chi += (counts.get(seq, 0) - e) ** 2 / e
    assert chi < 160.0, chi
