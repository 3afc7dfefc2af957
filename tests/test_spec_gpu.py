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
