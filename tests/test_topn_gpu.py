"""GPU parity of mxs_logsoftmax_topn against the oracle's token_logprob
(crates/app/cli/src/chat_turn.rs:506-563): top-N IDs bit-exact (total order,
lowest ID on ties), maximum exact, log-normalizer and logprobs within 1e-5
relative (1e-12 absolute near zero)."""
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

    s = Sampler(max_rows=256, max_vocab=262144)
    yield s
    s.close()


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def upload(torch, x, bf16_bits=None):
    R, V = x.shape
    stride = (V + 3) // 4 * 4
    if bf16_bits is not None:
        host = np.zeros((R, stride), dtype=np.uint16)
        host[:, :V] = bf16_bits
        return torch.from_numpy(host.view(np.int16)).to("cuda").view(torch.bfloat16)
    host = np.zeros((R, stride), dtype=np.float32)
    host[:, :V] = x
    return torch.from_numpy(host).to("cuda")


def close(g, e, rel=1e-5, abs_=1e-12):
    return abs(g - e) <= max(rel * abs(e), abs_)


def check(torch, sampler, orc, x, n, bf16_bits=None, name=""):
    say(f"case {name}: rows {x.shape[0]} vocab {x.shape[1]} n {n}")
    t = upload(torch, x, bf16_bits)
    ids, lps, mx, ln, st = sampler.logsoftmax_topn(t, n, vocab=x.shape[1])
    torch.cuda.synchronize()
    ids, lps, mx, ln, st = (a.cpu().numpy() for a in (ids, lps, mx, ln, st))
    problems = []
    for r in range(x.shape[0]):
        rs, rids, rlps, rmx, rln = orc.token_logprob_top(x[r], n)
        if not np.all(np.isfinite(x[r])):
            if st[r] != -6:
                problems.append(f"row {r}: status {st[r]}, want -6 (non-finite)")
            continue
        if st[r] != 0:
            problems.append(f"row {r}: status {st[r]}")
            continue
        k = len(rids)
        if not np.array_equal(ids[r, :k], rids):
            problems.append(f"row {r}: ids {ids[r, :k][:8]} ref {rids[:8]}")
            continue
        if k < n and not np.all(ids[r, k:] == -1):
            problems.append(f"row {r}: padding ids {ids[r, k:]}")
        if mx[r] != rmx:
            problems.append(f"row {r}: maximum {mx[r]!r} ref {rmx!r}")
        # every weight but the maximum's is within 2^-22 of exact, so ln S is
        # within 2^-22 (S - 1) / S of the reference's
        if not abs(ln[r] - rln) <= 2.0 ** -22 + 1e-13:
            problems.append(f"row {r}: log_normalizer {ln[r]!r} ref {rln!r}")
        for j in range(k):
            if not close(lps[r, j], rlps[j]):
                problems.append(f"row {r}: logprob[{j}] {lps[r, j]!r} ref {rlps[j]!r}")
                break
    assert not problems, "\n".join(problems[:20])


def test_config4_top20_plus_8(torch_mod, sampler, orc):
    from metallix_amd import synth

    b = synth.config4()
    assert b.rows == 256 and b.vocab == 262144
    check(torch_mod, sampler, orc, b.logits, 28, name="cfg4")


@pytest.mark.parametrize("rows,V,n", [(4, 1, 1), (4, 3, 5), (8, 100, 28), (8, 4097, 64), (8, 20481, 20),
                                      (8, 40961, 28), (16, 151936, 28), (4, 151936, 64), (4, 151936, 1)])
def test_random_shapes(torch_mod, sampler, orc, rows, V, n):
    rng = np.random.default_rng(1000 + V + n)
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    check(torch_mod, sampler, orc, x, n, name=f"random {V}")


def test_ties_and_constant_rows(torch_mod, sampler, orc):
    rng = np.random.default_rng(7)
    V = 151936
    x = np.zeros((6, V), dtype=np.float32)
    x[1] = rng.integers(-3, 4, V).astype(np.float32)          # few distinct values, many ties
    x[2] = np.where(rng.random(V) < 0.01, 5.0, -1.0).astype(np.float32)
    x[3, ::7] = -0.0                                           # -0.0 ranks below +0.0
    x[4] = rng.standard_normal(V).astype(np.float32)
    x[4, 1000:1100] = x[4].max() + 1.0                         # 100 tied maxima
    x[5] = -1e30
    check(torch_mod, sampler, orc, x, 64, name="ties")


def test_bf16_and_nonfinite(torch_mod, sampler, orc):
    from metallix_amd import synth

    rng = np.random.default_rng(11)
    V = 151936
    x = (rng.standard_normal((6, V)) * 2.5).astype(np.float32)
    bits = synth.to_bf16_bits(x)
    bits[2, 77] = 0x7fc0      # NaN
    bits[4, 5] = 0x7f80       # +inf
    x = synth.bf16_bits_to_f32(bits)
    check(torch_mod, sampler, orc, x, 28, bf16_bits=bits, name="bf16")
