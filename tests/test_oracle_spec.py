"""Pins the oracle's speculative-verify row (orc_spec_verify_row) on the CPU.

orc_spec_verify_row composes the reference's accept_or_resample
(crates/core/engine/src/speculative.rs:369-444) position by position over
temperature weights of two logit rows, stops at the first rejection and
takes the bonus token from target row K with sample_categorical
(crates/core/engine/src/sampling.rs:56-103) when every draft is accepted.
Every GPU test of mxs_spec_verify compares against this function, so each
part of the composition is fixed here by something other than a restatement
of its formula:

- identical target and draft rows give p/q == 1 exactly, so every draft is
  accepted, and the bonus is the independently pinned sample_categorical
  over target row K (not any other row);
- weights chosen so that p/q and the residual are exact binary fractions fix
  which accept and resample uniform each position consumes;
- a one-hot residual fixes the resampled id whatever the uniform;
- the error order follows accept_or_resample's checks, and positions after
  the first rejection are never examined;
- the exact-sequence law of speculative/tests.rs:448-566, with drafts from a
  wrong q, is reproduced through this function on a three-token vocabulary.
"""
import itertools
import math

import numpy as np

V8 = 8


def f32(a):
    return np.asarray(a, dtype=np.float32)


def test_identical_rows_accept_every_draft_and_bonus_is_row_k(orc):
    rng = np.random.default_rng(5)
    for K in (1, 2, 4, 7):
        for T in (0.35, 1.0, 2.5):
            tgt = f32(rng.standard_normal((K + 1, 50)) * 3.0)
            drf = tgt[:K].copy()
            toks = rng.integers(0, 50, size=K).astype(np.int32)
            ua = rng.random(K) * 0.999999
            ur = rng.random(K)
            ub = float(rng.random())
            st, out, cnt, acc = orc.spec_verify_row(tgt, drf, toks, T, ua, ur, ub)
            assert st == 0 and cnt == K + 1 and acc == K
            assert list(out[:K]) == list(toks)
            st_b, tok_b, _ = orc.sample_categorical(tgt[K], None, T, ub)
            assert st_b == 0 and out[K] == tok_b


def test_bonus_comes_from_target_row_k_not_another_row(orc):
    # rows 0..K-1 put all mass on token 0, row K on token 5: the bonus is 5
    K = 3
    tgt = np.zeros((K + 1, V8), np.float32)
    tgt[:K, 0] = 60.0
    tgt[K, 5] = 60.0
    drf = tgt[:K].copy()
    st, out, cnt, acc = orc.spec_verify_row(tgt, drf, [0, 0, 0], 1.0, [0.5] * K, [0.5] * K, 0.5)
    assert st == 0 and list(out) == [0, 0, 0, 5] and cnt == 4 and acc == 3


def test_forced_rejection_with_one_hot_residual(orc):
    # Position j: target mass on B, draft mass on A, draft token A.  p(A) is
    # about e^-50 so any accept uniform >= 1e-20 rejects; the residual
    # max(0, p - q) is exactly one-hot on B (every other token has p == q).
    A, B = 2, 6
    for K in (1, 3, 5):
        for j in range(K):
            tgt = np.zeros((K + 1, V8), np.float32)
            drf = np.zeros((K, V8), np.float32)
            toks = np.full(K, 1, np.int32)
            for i in range(K):
                tgt[i, 1] = 50.0
                drf[i, 1] = 50.0            # identical rows before j: accepted
            tgt[j] = 0.0
            drf[j] = 0.0
            tgt[j, B] = 50.0
            drf[j, A] = 50.0
            toks[j] = A
            for ur in (0.0, 0.37, 0.999999):
                st, out, cnt, acc = orc.spec_verify_row(tgt, drf, toks, 1.0, [0.5] * K, [ur] * K, 0.25)
                assert st == 0, st
                assert cnt == j + 1 and acc == j
                assert list(out[:j]) == [1] * j and out[j] == B


def test_accept_uniform_of_each_position(orc):
    # target [0, 0] -> p = (1/2, 1/2); draft [0, -1000] -> q = (1, 0):
    # drafting token 0 gives p/q == 1/2 exactly, so position j accepts iff
    # accept_u[j] < 1/2; the residual (0, 1/2) resamples token 1.
    K = 4
    tgt = np.zeros((K + 1, 2), np.float32)
    drf = np.tile(f32([0.0, -1000.0]), (K, 1))
    toks = np.zeros(K, np.int32)
    for reject_at in range(K):
        ua = np.full(K, 0.4)
        ua[reject_at] = 0.5                 # exactly p/q: not accepted (strict <)
        ua[reject_at + 1:] = 0.0            # would accept, but are never reached
        st, out, cnt, acc = orc.spec_verify_row(tgt, drf, toks, 1.0, ua, np.full(K, 0.3), 0.5)
        assert st == 0 and cnt == reject_at + 1 and acc == reject_at
        assert list(out[:reject_at]) == [0] * reject_at and out[reject_at] == 1


def test_resample_uniform_of_each_position(orc):
    # target [0, 0, 0] -> p = 1/3 each; draft [0, -1000, -1000] -> q = (1, 0, 0);
    # residual (0, 1/3, 1/3): resample_u[j] < 1/2 picks 1, else 2.
    K = 3
    tgt = np.zeros((K + 1, 3), np.float32)
    drf = np.tile(f32([0.0, -1000.0, -1000.0]), (K, 1))
    toks = np.zeros(K, np.int32)
    for j in range(K):
        ua = np.zeros(K)                    # p/q = 1/3 > 0: accepted
        ua[j] = 0.9                         # rejected here
        for low in (True, False):
            ur = np.full(K, 0.9 if low else 0.1)
            ur[j] = 0.1 if low else 0.9
            st, out, cnt, acc = orc.spec_verify_row(tgt, drf, toks, 1.0, ua, ur, 0.5)
            assert st == 0 and cnt == j + 1 and acc == j
            assert out[j] == (1 if low else 2)


def test_error_order(orc):
    K = 3
    tgt = np.zeros((K + 1, 4), np.float32)
    drf = np.zeros((K, 4), np.float32)
    toks = np.zeros(K, np.int32)
    ok = dict(ua=[0.5] * K, ur=[0.5] * K, ub=0.5)

    def run(t=tgt, d=drf, tk=toks, T=1.0, ua=ok["ua"], ur=ok["ur"], ub=ok["ub"]):
        return orc.spec_verify_row(t, d, tk, T, ua, ur, ub)[0]

    assert run(T=0.0) == -4
    assert run(T=-1.0) == -4
    assert run(T=math.inf) == -4
    bad = tgt.copy(); bad[0, 2] = math.nan
    assert run(t=bad) == -6
    bad = drf.copy(); bad[0, 1] = math.inf
    assert run(d=bad) == -6
    assert run(T=math.nan, t=bad) == -4      # temperature first
    assert run(tk=np.array([0, -1, 0], np.int32)) == -13
    assert run(tk=np.array([0, 4, 0], np.int32)) == -13
    assert run(ua=[0.5, 1.0, 0.5]) == -5     # uniforms before the token range
    assert run(ua=[0.5, 1.0, 0.5], tk=np.array([0, 9, 0], np.int32)) == -5
    assert run(ur=[0.5, -0.1, 0.5]) == -5
    assert run(ub=1.0) == -5                 # the bonus draw's own check
    # position 0 rejects: later positions' errors are never reached
    t2 = np.zeros((K + 1, 2), np.float32)
    d2 = np.tile(f32([0.0, -1000.0]), (K, 1))
    st, out, cnt, acc = orc.spec_verify_row(t2, d2, np.array([0, 7, 7], np.int32), 1.0, [0.9, 1.5, 1.5],
                                            [0.2, 0.2, 0.2], 2.0)
    assert st == 0 and cnt == 1 and acc == 0 and out[0] == 1


def test_large_offset_between_target_and_draft_rows(orc):
    # each row is weighted against its own maximum: a target row near 800
    # and a draft row near 0 would overflow exp with a shared maximum
    K = 2
    rng = np.random.default_rng(9)
    base = f32(rng.standard_normal((K + 1, 16)))
    tgt = base + np.float32(800.0)
    drf = base[:K].copy()
    toks = np.array([3, 7], np.int32)
    st, out, cnt, acc = orc.spec_verify_row(tgt, drf, toks, 1.0, [0.3, 0.3], [0.5, 0.5], 0.5)
    assert st == 0
    # rows that differ only by a constant have equal temperature weights up
    # to rounding: p/q within 1e-12 of 1, so u = 0.3 accepts both
    assert cnt == 3 and acc == 2 and list(out[:2]) == [3, 7]


class SplitMix:
    """SplitMix64 (speculative/tests.rs:128-149)."""

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


# The toy model both the exact-sequence-law check and the point-mass walk use.
TOY_VOCAB, TOY_PROMPT = 3, [0, 2, 1]   # speculative/tests.rs:14-15


def toy_logits(context):
    """speculative/tests.rs:37-52: the toy model's next-token row."""
    last = context[-1] if context else 0
    before = context[-2] if len(context) >= 2 else 0
    n = len(context)
    return np.array([np.float32(np.float32((last * 7 + before * 3 + t * 5 + n) % 11) * np.float32(0.37))
                     - (np.float32(0.8) if t == last else np.float32(0.0)) for t in range(TOY_VOCAB)],
                    dtype=np.float32)


def weights(logits, T):
    x = np.asarray(logits, dtype=np.float64)
    w = np.exp((x - x.max()) / T)
    return w / w.sum()


def law_chi(orc, samples, seed, bonus_row=None):
    """Drafts from a wrong q, verified by orc_spec_verify_row (K drafts per
    round, bonus from row K), over every 4-token continuation of the toy
    model; returns the chi-square against the target's exact law (80
    degrees of freedom).  `bonus_row` plants a mistake in the inputs: target
    row K replaced by row `bonus_row`."""
    T, VOCAB, PROMPT, LENGTH = 0.8, 3, [0, 2, 1], 4

    def draft_logits(ctx):
        q = np.full(VOCAB, 0.15)
        q[(ctx[-1] + 1) % VOCAB] = 0.7
        return f32(np.log(q) * T)

    def cat(p, u):
        cum = 0.0
        for i, x in enumerate(p):
            cum += x
            if u < cum:
                return i
        return len(p) - 1

    rng = SplitMix(seed)
    counts = {}
    for _ in range(samples):
        ctx = list(PROMPT)
        while len(ctx) < len(PROMPT) + LENGTH:
            K = min(3, len(PROMPT) + LENGTH - len(ctx))
            dctx, toks, drows = list(ctx), [], []
            for _ in range(K):
                dl = draft_logits(dctx)
                t = cat(weights(dl, T), rng.uniform())
                toks.append(t)
                drows.append(dl)
                dctx.append(t)
            trows = [toy_logits(list(ctx) + toks[:j]) for j in range(K + 1)]
            if bonus_row is not None:
                trows[K] = trows[bonus_row]
            ua = [rng.uniform() for _ in range(K)]
            ur = [rng.uniform() for _ in range(K)]
            ub = rng.uniform()
            st, out, cnt, acc = orc.spec_verify_row(np.stack(trows), np.stack(drows), toks, T, ua, ur, ub)
            assert st == 0
            ctx += [int(v) for v in out[:cnt]]
        key = tuple(ctx[len(PROMPT):len(PROMPT) + LENGTH])
        counts[key] = counts.get(key, 0) + 1
    chi = 0.0
    for seq in itertools.product(range(VOCAB), repeat=LENGTH):
        ctx, pr = list(PROMPT), 1.0
        for tok in seq:
            pr *= weights(toy_logits(ctx), T)[tok]
            ctx.append(tok)
        e = pr * samples
        chi += (counts.get(seq, 0) - e) ** 2 / e
    return chi


def test_exact_sequence_law_through_spec_verify_row(orc):
    """speculative/tests.rs:512-566 driven through orc_spec_verify_row, with
    fewer samples and a bound scaled to them."""
    chi = law_chi(orc, 6000, 21)
    assert chi < 160.0, chi


def test_law_check_sees_a_wrong_bonus_row(orc):
    """The law check is strong enough to catch a misread composition: with
    the bonus drawn from target row 0 instead of row K it fails."""
    chi = law_chi(orc, 6000, 21, bonus_row=0)
    assert chi > 160.0, chi


# ---- A9: the point-mass verify walk (accept_and_roll_back) --------------------
def toy_sample(orc, row, uniform):
    st, tok, _ = orc.sample_categorical(row, None, 0.9, uniform)
    assert st == 0
    return tok


def test_walk_stops_at_a_stop_token(orc):
    """speculative/tests.rs:608-631: picks 1, 2, 0 over draft [1, 2, 2] with
    token 2 stopping: emitted [1, 2], 2 accepted, stopped, and the third row
    is never settled."""
    picks = iter([1, 2, 0])
    settled = []

    def pick_at(i):
        settled.append(i)
        t = next(picks)
        return t, t == 2

    emitted, accepted, stopped = orc.accept_and_roll_back([1, 2, 2], pick_at)
    assert (emitted, accepted, stopped) == ([1, 2], 2, True)
    assert settled == [0, 1]


def test_walk_rejection_positions_and_bonus(orc):
    for k in range(0, 5):
        draft = list(range(10, 10 + k))
        for diverge in range(k + 1):   # diverge == k: every draft accepted, the bonus row ends it
            def pick_at(i, diverge=diverge, draft=draft):
                return (draft[i] if i < diverge else 99), False
            emitted, accepted, stopped = orc.accept_and_roll_back(draft, pick_at)
            assert accepted == diverge and not stopped
            assert emitted == draft[:diverge] + [99]


def test_pre_drawn_row_uniforms_reproduce_plain_sampling(orc):
    """speculative/tests.rs:271-321 on the oracle: speculative decoding of the
    toy model whose rows carry pre-drawn uniforms (row i reads i draws ahead,
    one draw committed per settled row) emits exactly what plain sampling
    emits, for random drafts that reject at every position."""
    Rng = orc.SplitMix64

    def decode_plain(seed, length=24):
        rng = Rng(seed)
        ctx = list(TOY_PROMPT)
        out = []
        while len(out) < length:
            t = toy_sample(orc, toy_logits(ctx), rng.uniform())
            out.append(t)
            ctx.append(t)
        return out

    for seed in range(20):
        expected = decode_plain(seed)
        stream = Rng(seed)
        draft_rng = Rng(seed ^ 0xABCD)
        out = [toy_sample(orc, toy_logits(TOY_PROMPT), stream.uniform())]
        rejected = 0
        while len(out) < 24:
            limit = 24 - len(out) - 1
            k = min(draft_rng.next_u64() % 4, limit)
            proposal = [int((draft_rng.next_u64() % 1024) % TOY_VOCAB) for _ in range(k)]
            ctx = TOY_PROMPT + out
            rows = [toy_logits(ctx + proposal[:i]) for i in range(k + 1)]
            peek = Rng(stream.state)
            ahead = [peek.uniform() for _ in range(k + 1)]
            emitted, accepted, stopped, _ = orc.point_mass_verify(rows, proposal, ahead, temperature=0.9)
            for _ in emitted:
                stream.uniform()   # one committed draw per settled row
            rejected += int(0 < accepted < k)
            out.extend(emitted)
        assert out == expected, f"seed {seed}"
        if seed == 0:
            assert rejected > 0
