"""GPU parity of race-v2 picks (mxs_sample_race) against the CPU oracle.

The oracle builds each row's kept set and adjusted logits (the same
build-defined stages mxs_sample uses, checked bit-exact by compare()), then
runs its restatement of sample_race (crates/core/engine/src/sampling/race.rs:
114-147) over that set with the row's key.  Bar: statuses and tokens
identical, sampling logprobs within 1e-5 relative, no uncertified row.
"""
import sys

import numpy as np
import pytest

from helpers import compare, to_device, unpack_bits

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


def race_keys(rows, salt):
    from metallix_amd import synth

    s = synth.Stream(0x72616365 + salt)
    seed = s.u64(rows)
    choice = (s.u64(rows) % np.uint64(4)).astype(np.uint32)
    position = (s.u64(rows) % np.uint64(1 << 20)).astype(np.uint32)
    return seed, choice, position


def run_race(torch, sampler, b, keys):
    logits, kw = to_device(torch, b)
    seed, choice, position = keys
    dev = logits.device
    race = (torch.from_numpy(seed.view(np.int64)).to(dev),
            torch.from_numpy(choice.view(np.int32)).to(dev),
            torch.from_numpy(position.view(np.int32)).to(dev))
    out = sampler.sample(logits, debug=True, race=race, **kw)
    torch.cuda.synchronize()
    return dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
                sampling_logprob=out.sampling_logprob.cpu().numpy(),
                adjusted=out.adjusted.cpu().numpy(), kept=unpack_bits(out.kept_bits.cpu().numpy(), b.vocab))


def oracle_race(orc, b, keys):
    ref = orc.sample_batch(b, debug=True)
    seed, choice, position = keys
    for r in range(b.rows):
        if ref["status"][r] != 0 or b.temperature[r] == 0.0:
            continue
        st, tok, lp = orc.sample_race(ref["adjusted"][r], ref["kept"][r], float(b.temperature[r]),
                                      int(seed[r]), int(choice[r]), int(position[r]))
        ref["status"][r] = st
        ref["token"][r] = tok if st == 0 else -1
        ref["sampling_logprob"][r] = lp
    return ref


def check(torch_mod, sampler, orc, b, salt):
    print(f"race case {b.name}: rows {b.rows} vocab {b.vocab} salt {salt}", flush=True)
    sys.stdout.flush()
    keys = race_keys(b.rows, salt)
    gpu = run_race(torch_mod, sampler, b, keys)
    ref = oracle_race(orc, b, keys)
    # tokens must match exactly: a race pick has no CDF boundary to excuse
    mism = [r for r in range(b.rows) if gpu["status"][r] == 0 and gpu["token"][r] != ref["token"][r]]
    assert not mism, f"race tokens differ on rows {mism[:10]}"
    compare(b, gpu, ref)
    return gpu, ref


def mixed(rows, vocab):
    """config 2's rows with every rule the kept set can come from: top-k,
    top-p, min-p, keep-all (whole-row race), greedy, and logit bias."""
    from metallix_amd import synth

    b = synth.config2(rows=rows, vocab=vocab)
    b.name = "race-mixed"
    s = synth.Stream(0x5eed)
    for r in range(rows):
        kind = r % 6
        if kind == 4:                       # keep-all: the whole-row race
            b.top_k[r] = 0
            b.top_p[r] = 1.0
            b.min_p[r] = 0.0
        elif kind == 5 and r % 12 == 5:     # greedy rows keep the finisher's pick
            b.temperature[r] = 0.0
    nb = 8
    ids = np.sort(np.stack([np.sort(s.u64(nb) % np.uint64(vocab)) for _ in range(rows)]), axis=1)
    bias_ids, offs = [], [0]
    for r in range(rows):
        u = np.unique(ids[r]).astype(np.uint32)
        bias_ids.append(u)
        offs.append(offs[-1] + len(u))
    b.bias_ids = np.concatenate(bias_ids)
    b.bias_offsets = np.array(offs, dtype=np.uint32)
    b.bias_values = (4.0 * (s.uniform(len(b.bias_ids)) - 0.25)).astype(np.float32)
    return b


@pytest.mark.parametrize("vocab,salt", [(4096, 1), (50000, 2), (151936, 3)])
def test_race_mixed_rules(torch_mod, sampler, orc, vocab, salt):
    gpu, ref = check(torch_mod, sampler, orc, mixed(24, vocab), salt)
    assert (gpu["status"] == 0).sum() == 24


def test_race_past_64_rows(torch_mod, sampler, orc):
    """96 rows: race row groups and race scratch past row 64."""
    gpu, ref = check(torch_mod, sampler, orc, mixed(96, 20000), 5)
    assert (gpu["status"] == 0).sum() == 96


def test_race_masked_bf16(torch_mod, sampler, orc):
    from metallix_amd import synth

    b = synth.config3(rows=8)
    check(torch_mod, sampler, orc, b, 7)


def test_race_config2_full(torch_mod, sampler, orc):
    from metallix_amd import synth

    check(torch_mod, sampler, orc, synth.config2(), 9)


def test_race_keys_move_the_pick(torch_mod, sampler, orc):
    """Keep-all rows at T = 1 over flat logits: the winner follows the noise,
    so different positions give different tokens (and each is the oracle's)."""
    from metallix_amd import synth

    V, R = 8192, 16
    x = np.zeros((R, V), dtype=np.float32)
    b = synth.Batch(name="race-flat", logits=x, temperature=np.ones(R), uniform=np.zeros(R))
    gpu, _ = check(torch_mod, sampler, orc, b, 11)
    assert len(set(gpu["token"].tolist())) > R // 2


@pytest.mark.parametrize("T", [0.01, 0.3, 20.0])
def test_race_whole_row_temperature_extremes(torch_mod, sampler, orc, T):
    """Whole-row races at extreme temperatures: at T = 0.01 the f32
    screening scores reach magnitudes near 1e3 (the error bound's relative
    term matters), at T = 20 the noise dominates and many tokens lie close
    to the winner."""
    from metallix_amd import synth

    b = synth.config2(rows=8, vocab=151936)
    b.name = f"race-whole-T{T}"
    b.top_k[:] = 0
    b.top_p[:] = 1.0
    b.min_p[:] = 0.0
    b.temperature[:] = T
    gpu, _ = check(torch_mod, sampler, orc, b, 13)
    assert (gpu["status"] == 0).all()


def test_race_heavy_histories(torch_mod, sampler, orc):
    """Penalty histories with counts past the race kernel's 16-bit count
    pairs: 70000 entries with one token repeated 66000 times (saturating
    counts, recounted from the history), 65535 entries that are all one
    token, and 40000 entries split between the two tokens of one count
    word.  Those tokens lead their rows by enough that a wrong count moves
    the winner or its log probability."""
    from metallix_amd import synth

    R, V = 8, 20000
    s = synth.Stream(0x4857)
    x = s.normal(R * V).reshape(R, V).astype(np.float32)
    hists = []
    for r in range(R):
        if r == 0:
            h = np.concatenate([np.full(66000, 7), np.full(3000, 8), s.u64(1000) % np.uint64(V)])
        elif r == 1:
            h = np.full(65535, 9)
        elif r == 2:
            h = np.concatenate([np.full(39000, 10), np.full(1000, 11)])
        else:
            h = s.u64(200 * r) % np.uint64(V)
        hists.append(np.asarray(h, dtype=np.uint32))
    for r, toks in enumerate(([7, 8], [8, 9], [10, 11])):
        x[r, toks] = 12.0
    b = synth.Batch(name="race-heavy-hist", logits=x, temperature=np.ones(R), uniform=np.zeros(R))
    b.top_k = np.array([0, 0, 0, 0, 50, 0, 1000, 0], dtype=np.uint32)
    b.top_p = np.array([1.0, 1.0, 1.0, 1.0, 0.9, 1.0, 0.95, 1.0])
    b.min_p = np.zeros(R)
    b.repetition = np.full(R, 1.1, dtype=np.float32)
    b.presence = np.full(R, 0.05, dtype=np.float32)
    b.frequency = np.full(R, 1.0e-4, dtype=np.float32)
    b.history_offsets = np.concatenate([[0], np.cumsum([len(h) for h in hists])]).astype(np.uint32)
    b.history_ids = np.concatenate(hists)
    gpu, _ = check(torch_mod, sampler, orc, b, 17)
    assert (gpu["status"] == 0).all(), gpu["status"]
