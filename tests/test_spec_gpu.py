"""GPU parity of mxs_spec_verify against the oracle's position walk over
accept_or_resample (crates/core/engine/src/speculative.rs:369-444) with the
bonus draw by sample_categorical: statuses, emitted tokens, counts and
accepted counts identical; no row may come back uncertified on these
inputs."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def sampler(torch_mod):
    from metallix_amd import Sampler

    s = Sampler(max_rows=64, max_vocab=262144)
    yield s
    s.close()


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run(torch, sampler, orc, d, name):
    tgt, drf = d["target"], d["draft"]
    rows, k1, V = tgt.shape
    K = k1 - 1
    say(f"case {name}: rows {rows} K {K} vocab {V}")
    dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=dt))).to("cuda")
    out, cnt, acc, st = sampler.spec_verify(
        dev(tgt, np.float32), dev(drf, np.float32) if K else None, dev(d["draft_tokens"], np.int32) if K else None,
        dev(d["temperature"], np.float64), dev(d["accept_u"], np.float64) if K else None,
        dev(d["resample_u"], np.float64) if K else None, dev(d["bonus_u"], np.float64))
    torch.cuda.synchronize()
    out, cnt, acc, st = (a.cpu().numpy() for a in (out, cnt, acc, st))
    problems = []
    for r in range(rows):
        rs, rout, rcnt, racc = orc.spec_verify_row(
            tgt[r], drf[r] if K else np.zeros((0, V), np.float32), d["draft_tokens"][r] if K else np.zeros(0, np.int32),
            float(d["temperature"][r]), d["accept_u"][r] if K else np.zeros(0), d["resample_u"][r] if K else np.zeros(0),
            float(d["bonus_u"][r]))
        if st[r] != rs:
            problems.append(f"row {r}: status gpu {st[r]} ref {rs}")
            continue
        if rs != 0:
            continue
        if cnt[r] != rcnt or acc[r] != racc or not np.array_equal(out[r, :rcnt], rout[:rcnt]):
            problems.append(f"row {r}: gpu {out[r, :cnt[r]]} ({cnt[r]}, {acc[r]}) ref {rout[:rcnt]} ({rcnt}, {racc})")
    assert not problems, "\n".join(problems[:20])
    return st, cnt, acc


def make(rows, K, V, seed, T=1.0, noise=0.5, peaks=True):
    rng = np.random.default_rng(seed)
    tgt = (rng.standard_normal((rows, K + 1, V)) * 2.0).astype(np.float32)
    if peaks:
        for r in range(rows):
            for j in range(K + 1):
                idx = rng.integers(0, V, 1 + int(rng.integers(0, 10)))
                tgt[r, j, idx] += rng.uniform(4, 10, idx.size).astype(np.float32)
    drf = (tgt[:, :K].astype(np.float64) + noise * rng.standard_normal((rows, K, V))).astype(np.float32)
    toks = np.zeros((rows, K), dtype=np.int32)
    for r in range(rows):
        for j in range(K):
            q = np.exp((drf[r, j].astype(np.float64) - drf[r, j].max()) / T)
            cdf = np.cumsum(q)
            toks[r, j] = min(int(np.searchsorted(cdf, rng.random() * cdf[-1], side="right")), V - 1)
    return dict(target=tgt, draft=drf, draft_tokens=toks, temperature=np.full(rows, T),
                accept_u=rng.random((rows, K)), resample_u=rng.random((rows, K)), bonus_u=rng.random(rows))


def test_config5(torch_mod, sampler, orc):
    from metallix_amd import synth

    run(torch_mod, sampler, orc, synth.config5(), "cfg5")


@pytest.mark.parametrize("T", [0.5, 1.5])
def test_rejections_at_every_position(torch_mod, sampler, orc, T):
    d = make(16, 4, 151936, 31 + int(T * 10), T=T, noise=1.5)
    # force the first rejection onto position r % 4 (accept before it)
    for r in range(16):
        d["accept_u"][r, :] = 0.0
        d["accept_u"][r, r % 4] = 0.999999
    st, cnt, acc = run(torch_mod, sampler, orc, d, f"rejections T={T}")
    assert (acc < 4).sum() >= 8


def test_all_accepted_bonus_and_identical(torch_mod, sampler, orc):
    d = make(8, 4, 151936, 41)
    d["accept_u"][:] = 0.0                       # every draft accepted: the bonus draw
    d["draft"][4:] = d["target"][4:, :4]         # p == q: always accepted
    d["accept_u"][4:] = 0.999
    st, cnt, acc = run(torch_mod, sampler, orc, d, "bonus")
    assert (cnt == 5).all()


@pytest.mark.parametrize("rows,K,V", [(4, 0, 151936), (4, 8, 4096), (6, 3, 1001), (4, 2, 7), (2, 4, 262144)])
def test_shapes(torch_mod, sampler, orc, rows, K, V):
    run(torch_mod, sampler, orc, make(rows, K, V, 51 + K + V, noise=1.0), f"shape {K}x{V}")


def test_error_matrix(torch_mod, sampler, orc):
    d = make(8, 3, 4096, 61)
    d["temperature"][0] = 0.0                    # invalid temperature
    d["accept_u"][1, 0] = 1.0                    # invalid uniform at position 0
    d["draft_tokens"][2, 0] = -1                 # token out of range (negative)
    d["draft_tokens"][3, 1] = 4096               # token out of range, position 1
    d["accept_u"][3, 0] = 0.0
    d["target"][4, 0, 9] = np.nan                # non-finite at position 0
    d["accept_u"][5, :] = 0.0
    d["target"][5, 3, 17] = np.inf               # non-finite at the bonus position
    d["draft"][6, 0, d["draft_tokens"][6, 0]] = -1e30   # q = 0: Probabilities
    d["bonus_u"][7] = -0.5                       # invalid bonus uniform
    d["accept_u"][7, :] = 0.0
    run(torch_mod, sampler, orc, d, "errors")


# ---- A9: point-mass verify on device picks -------------------------------------
def test_point_mass_verify_toy_model_reproduces_plain_sampling(torch_mod, sampler, orc):
    """speculative/tests.rs:271-321 with device picks: the toy model's rows
    (V = 3) are verified by one mxs_sample call per step (row i carries the
    uniform i draws ahead), and the emitted sequence equals plain sampling of
    the oracle with the same stream, for random drafts."""
    import test_oracle_spec as toy

    torch = torch_mod
    Rng = orc.SplitMix64
    for seed in range(6):
        rng = Rng(seed)
        ctx, expected = list(toy.TOY_PROMPT), []
        while len(expected) < 24:
            t = toy.toy_sample(orc, toy.toy_logits(ctx), rng.uniform())
            expected.append(t)
            ctx.append(t)
        stream = Rng(seed)
        draft_rng = Rng(seed ^ 0xABCD)
        out = [toy.toy_sample(orc, toy.toy_logits(toy.TOY_PROMPT), stream.uniform())]
        while len(out) < 24:
            limit = 24 - len(out) - 1
            k = int(min(draft_rng.next_u64() % 4, limit))
            proposal = [int((draft_rng.next_u64() % 1024) % toy.TOY_VOCAB) for _ in range(k)]
            rows = np.stack([toy.toy_logits(toy.TOY_PROMPT + out + proposal[:i]) for i in range(k + 1)])
            peek = Rng(stream.state)
            ahead = np.array([peek.uniform() for _ in range(k + 1)])
            logits = torch.zeros((k + 1, 4), dtype=torch.float32, device="cuda")
            logits[:, :3] = torch.from_numpy(rows).to("cuda")
            res = sampler.verify_point_mass(
                logits, np.array([proposal], dtype=np.int64).reshape(1, k),
                torch.full((k + 1,), 0.9, dtype=torch.float64, device="cuda"),
                torch.from_numpy(ahead).to("cuda"), vocab=3)[0]
            assert res["status"] == 0
            for _ in res["emitted"]:
                stream.uniform()
            out.extend(res["emitted"])
        assert out == expected, f"seed {seed}"


def test_point_mass_verify_matches_the_oracle_walk(torch_mod, sampler, orc):
    """Sequences of 5 scored positions at V = 151936 under config 2's rules:
    drafts follow the oracle's picks for a random number of positions and
    then leave them (or not at all: the bonus row), some with a stop token
    inside the draft; the device walk's emitted tokens, acceptance count and
    stop flag equal the oracle walk's."""
    from metallix_amd import synth

    torch = torch_mod
    S, K = 12, 4
    b = synth.config2(rows=S * (K + 1))
    rng = np.random.default_rng(347)
    ref_tok = orc.sample_batch(b)["token"].reshape(S, K + 1)
    draft = np.zeros((S, K), dtype=np.int64)
    stop_ids = set()
    for s in range(S):
        d = int(rng.integers(0, K + 1))      # positions that follow the picks
        draft[s, :d] = ref_tok[s, :d]
        if d < K:
            draft[s, d:] = (ref_tok[s, d:K] + 1 + rng.integers(0, 100, K - d)) % b.vocab
        if s % 4 == 3 and d > 1:
            stop_ids.add(int(ref_tok[s, 1]))
    from helpers import to_device

    logits, kw = to_device(torch, b)
    temp, uni = kw.pop("temperature"), kw.pop("uniform")
    got = sampler.verify_point_mass(logits, draft, temp, uni, stop_ids=stop_ids, **kw)
    for s in range(S):
        # the oracle walk over the oracle's per-row picks (same rows, rules and uniforms)
        picks = ref_tok[s]
        e_ref, a_ref, st_ref = orc.accept_and_roll_back(draft[s], lambda i: (picks[i], int(picks[i]) in stop_ids))
        assert got[s]["status"] == 0, (s, got[s])
        assert got[s]["emitted"] == e_ref, (s, got[s], e_ref)
        assert got[s]["accepted"] == a_ref and got[s]["stopped"] == st_ref
