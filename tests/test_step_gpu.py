"""GPU parity of one engine step (mxs_step): every row's pick and, for the
rows that ask, the log-probability receipt over the suppressed logits
(TurnLoop::pick, crates/app/cli/src/chat_turn.rs:290-303; token_logprob,
:506-563; ChatFormat::suppress, crates/core/chat-format/src/lib.rs:761-780).
Picks are held to compare() (statuses, adjusted logits, kept sets and tokens
bit-exact, logprobs within 1e-5); receipts to the oracle's
orc_token_logprob_top on the same suppressed row: IDs bit-exact, logprobs
and the picked token's log probability within 1e-5 relative."""
import sys

import numpy as np
import pytest

from helpers import compare, to_device, u32, unpack_bits

pytestmark = pytest.mark.gpu

F32_MIN = float(np.finfo(np.float32).min)
NONE = 0xFFFFFFFF   # MXS_RECEIPT_NONE: no receipt for the row


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def sampler(torch_mod):
    from metallix_amd import Sampler

    s = Sampler(max_rows=64, max_vocab=151936)
    yield s
    s.close()


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def suppressed(b, sup):
    """b with the checkpoint's suppressed IDs merged into its bias CSR."""
    from metallix_amd.sampler import with_suppression

    b.bias_offsets, b.bias_ids, b.bias_values = with_suppression(b.rows, sup, b.bias_offsets, b.bias_ids,
                                                                 b.bias_values, vocab=b.vocab)
    return b


def check_step(torch, sampler, orc, b, sup, tops, n, allow_uncertified=0):
    say(f"case step {b.name}: rows {b.rows} vocab {b.vocab} n {n} suppressed {len(sup)}")
    logits, kw = to_device(torch, b)
    top_t = torch.from_numpy(u32(tops)).to(logits.device)
    out, rec = sampler.step(logits, receipt_top=top_t, n=n, debug=True, **kw)
    torch.cuda.synchronize()
    gpu = dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
               sampling_logprob=out.sampling_logprob.cpu().numpy(), adjusted=out.adjusted.cpu().numpy(),
               kept=unpack_bits(out.kept_bits.cpu().numpy(), b.vocab))
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref, allow_uncertified=allow_uncertified)
    ids, lps = rec.ids.cpu().numpy(), rec.logprobs.cpu().numpy()
    tlp, rst = rec.token_logprob.cpu().numpy(), rec.status.cpu().numpy()
    problems = []
    for r in range(b.rows):
        if tops[r] == NONE:
            if not (np.all(ids[r] == -1) and np.isnan(tlp[r])):
                problems.append(f"row {r}: no receipt asked, outputs written")
            continue
        x = np.asarray(b.logits[r], dtype=np.float32).copy()
        x[np.asarray([i for i in sup if i < b.vocab], dtype=np.int64)] = F32_MIN   # (IDs past the row: skipped)
        if not np.all(np.isfinite(x)):
            # A non-finite logit fails the row's pick (the reference's turn
            # stops there and scores no receipt): the receipt reports the
            # same status, with no entries and NaN log probabilities.
            if not (rst[r] == ref["status"][r] == -6 and np.all(ids[r] == -1) and np.all(np.isnan(lps[r]))
                    and np.isnan(tlp[r])):
                problems.append(f"row {r}: non-finite receipt {rst[r]} {ids[r, :3]} {lps[r, :3]} {tlp[r]}")
            continue
        st, rids, rlps, rmx, rln = orc.token_logprob_top(x, n)
        if rst[r] != 0 or st != 0:
            problems.append(f"row {r}: receipt status {rst[r]} ref {st}")
            continue
        k = len(rids)
        if not np.array_equal(ids[r, :k], rids):
            problems.append(f"row {r}: ids {ids[r, :6]} ref {rids[:6]}")
            continue
        if k < n and not (np.all(ids[r, k:] == -1) and np.all(np.isneginf(lps[r, k:]))):
            problems.append(f"row {r}: entries past the vocabulary {ids[r, k:k + 3]} {lps[r, k:k + 3]}")
        if not np.allclose(lps[r, :k], rlps, rtol=1e-5, atol=0.0):
            problems.append(f"row {r}: logprobs {lps[r, :4]} ref {rlps[:4]}")
        t = int(gpu["token"][r])
        if t >= 0:
            want = (float(x[t]) - rmx) - rln
            if not abs(tlp[r] - want) <= 1e-5 * abs(want) + 1e-12:
                problems.append(f"row {r}: token logprob {tlp[r]!r} ref {want!r}")
        elif not np.isnan(tlp[r]):
            problems.append(f"row {r}: no token, logprob {tlp[r]!r}")
    assert not problems, "\n".join(problems[:20])
    return gpu, rec


def test_step_config2_rules_with_suppression(torch_mod, sampler, orc):
    """24 rows of config 2's rules; the suppressed set holds row 0's largest
    logit (its receipt's maximum moves), IDs near the row's end and two past
    it, which ChatFormat::suppress skips (chat-format/src/lib.rs:771-778)."""
    from metallix_amd import synth

    b = synth.config2(rows=24)
    b.name = "step-cfg2"
    sup = sorted({int(np.argmax(b.logits[0])), 151643, 151935, 17, 90000, 151936, 200000})
    b = suppressed(b, sup)
    # (0: the picked token's log probability with no top entries)
    tops = np.array([[NONE, 0, 1, 5, 20][r % 5] for r in range(b.rows)], dtype=np.uint32)
    gpu, _ = check_step(torch_mod, sampler, orc, b, sup, tops, 28)
    assert int(gpu["token"][0]) not in sup


def test_step_bf16_masked_rows(torch_mod, sampler, orc):
    """Config 3's bf16 grammar rows (the receipt reads bf16 logits; the mask
    does not enter the receipt, as token_logprob scores the raw row)."""
    from metallix_amd import synth

    b = synth.config3(rows=8)
    b.name = "step-cfg3"
    sup = [3, 100, 151000]
    b = suppressed(b, sup)
    tops = np.array([3, NONE, 1, 20, 0, 5, 56, NONE], dtype=np.uint32)
    check_step(torch_mod, sampler, orc, b, sup, tops, 64)


def test_step_receipt_ties_flat_and_nonfinite(torch_mod, sampler, orc):
    """Receipt edge cases of the one-pass step: a constant row and a top
    plateau of 3000 equal logits (ties past the chunks' candidate capacity:
    the exact path, ties in token-ID order), a NaN (non-finite status, no
    entries), a suppressed row maximum, a masked row (the general chunk
    body: the receipt reads the chunk again) and ordinary rows; n = 64."""
    from metallix_amd.synth import Batch

    V, R = 50000, 8
    rng = np.random.default_rng(91)
    x = (rng.standard_normal((R, V)) * 2.0).astype(np.float32)
    x[0, :] = 0.5                                   # constant row
    x[1, rng.choice(V // 4, 3000, replace=False)] = 9.0   # a plateau inside chunk 0
    x[2, 777] = np.nan                              # non-finite
    x[3, 4242] = 12.0                               # the row maximum, suppressed below
    x[4, :] = np.round(x[4, :])                     # many ties at every integer
    words = (V + 31) // 32
    mask = np.zeros((R, words), dtype=np.uint32)
    mask[:] = 0xFFFFFFFF
    mask[5, : words // 2] = 0x55555555              # a masked row: every other token in the first half
    b = Batch(name="step-edges", logits=x, temperature=np.array([0.7, 1.0, 1.0, 0.0, 1.2, 0.9, 1.0, 0.5]),
              uniform=rng.random(R), top_k=np.array([20, 0, 5, 0, 50, 0, 1000, 0], dtype=np.uint32),
              top_p=np.array([0.9, 1.0, 0.9, 1.0, 0.8, 0.95, 0.7, 1.0]),
              min_p=np.array([0.0, 0.05, 0.0, 0.0, 0.0, 0.1, 0.05, 0.0]), mask_words=mask, tokenizer_vocab=V)
    sup = [4242, 11, 49999]
    b = suppressed(b, sup)
    tops = np.array([56, 56, 56, 56, 56, 56, NONE, 0], dtype=np.uint32)
    # (the constant row's pick: a nucleus cut among equal weights may come
    # back uncertified, with the oracle's token or a boundary draw)
    gpu, _ = check_step(torch_mod, sampler, orc, b, sup, tops, 64, allow_uncertified=1)
    assert set(np.nonzero(gpu["status"] == 1)[0]) <= {0}


def test_step_receipt_small_vocab(torch_mod, sampler, orc):
    """A vocabulary of 40 under n = 64: 40 entries, the rest -1 / -inf."""
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 40)) * 3.0).astype(np.float32)
    x[1, :] = 1.0
    b = Batch(name="step-small", logits=x, temperature=np.array([1.0, 0.5, 0.0]), uniform=rng.random(3),
              top_k=np.array([0, 5, 0], dtype=np.uint32), top_p=np.array([0.9, 1.0, 1.0]),
              min_p=np.array([0.0, 0.0, 0.0]))
    b = suppressed(b, [7])
    check_step(torch_mod, sampler, orc, b, [7], np.array([56, 3, 0], dtype=np.uint32), 64)


def test_step_race_rows(torch_mod, sampler, orc):
    """mxs_step with race keys: race-v2 picks, and receipts for the winner."""
    from metallix_amd import synth
    from test_race_gpu import oracle_race, race_keys

    torch = torch_mod
    b = synth.config2(rows=8, vocab=50000)
    b.name = "step-race"
    sup = [11, 4000]
    b = suppressed(b, sup)
    say(f"case step-race: rows {b.rows} vocab {b.vocab}")
    keys = race_keys(b.rows, 21)
    logits, kw = to_device(torch, b)
    dev = logits.device
    race = (torch.from_numpy(keys[0].view(np.int64)).to(dev), torch.from_numpy(keys[1].view(np.int32)).to(dev),
            torch.from_numpy(keys[2].view(np.int32)).to(dev))
    tops = np.full(b.rows, 5, dtype=np.uint32)
    out, rec = sampler.step(logits, receipt_top=torch.from_numpy(u32(tops)).to(dev), n=13, race=race, **kw)
    torch.cuda.synchronize()
    tok, st = out.token.cpu().numpy(), out.status.cpu().numpy()
    ref = oracle_race(orc, b, keys)
    tlp = rec.token_logprob.cpu().numpy()
    # a race row is uncertified only when two f64 scores lie within the
    # device's error bound: at most one here, and it still carries the
    # oracle's winner
    assert int((st == 1).sum()) <= 1, st
    for r in range(b.rows):
        assert st[r] in (0, 1), (r, st[r])
        assert tok[r] == ref["token"][r], (r, st[r], tok[r], ref["token"][r])
        x = np.asarray(b.logits[r], dtype=np.float32).copy()
        x[sup] = F32_MIN
        _, _, _, rmx, rln = orc.token_logprob_top(x, 13)
        want = (float(x[tok[r]]) - rmx) - rln
        assert abs(tlp[r] - want) <= 1e-5 * abs(want), (r, tlp[r], want)


def test_engine_step_host_loop(torch_mod, sampler, orc):
    """EngineStep over RowRequests equals the reference's per-row loop:
    suppress, pick, then a receipt for non-stop tokens with the unspellable
    IDs past the tokenizer's vocabulary dropped from the top + 8 head."""
    from metallix_amd.engine import EngineStep, RowRequest

    torch = torch_mod
    V, TV = 50000, 49990
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((12, V)) * 2.0).astype(np.float32)
    x[:, TV:] += 6.0   # padded rows past the tokenizer: likely, unspellable
    for r in range(12):
        x[r, rng.choice(TV, 10, replace=False)] += 7.0
    sup = [int(np.argmax(x[2])), 123]
    x5 = x[5].copy()
    x5[sup] = F32_MIN
    stop = int(np.argmax(x5))   # row 5's greedy pick (every token legal) is a stop token
    words = (V + 31) // 32
    mask = np.zeros(words, dtype=np.uint32)
    legal = rng.choice(TV, 300, replace=False)
    np.bitwise_or.at(mask, legal // 32, np.uint32(1) << (legal % 32).astype(np.uint32))
    reqs = []
    for r in range(12):
        q = RowRequest(temperature=[0.0, 0.7, 1.0, 1.3][r % 4], top_k=[0, 20, 0, 50][r % 4],
                       top_p=[1.0, 0.9, 0.8, 1.0][r % 4], min_p=0.05 if r % 3 == 0 else 0.0,
                       uniform=float(rng.random()), top_logprobs=[None, 3, 10, 0][r % 4] if r != 5 else 4)
        if r % 5 == 1:
            q.history = rng.integers(0, V, 40).tolist()
            q.repetition, q.presence, q.frequency = 1.1, 0.3, 0.2
        if r % 6 == 4:
            q.bias = {int(i): float(v) for i, v in zip(rng.choice(V, 5, replace=False), rng.normal(0, 2, 5))}
        if r in (3, 8):
            q.mask = mask
        if r == 5:
            q.temperature = 0.0
            q.mask = None
        reqs.append(q)
    say("case engine-step: rows 12 vocab 50000")
    logits = torch.from_numpy(x).cuda()
    res = EngineStep(sampler, suppress_ids=sup, stop_ids=[stop], tokenizer_vocab=TV).run(logits, reqs)
    for r, (q, got) in enumerate(zip(reqs, res)):
        bias = dict(q.bias)
        for s_ in sup:
            bias[s_] = -np.inf
        bi = sorted(bias)
        ref = orc.sample_row(x[r], temperature=q.temperature, top_p=q.top_p, min_p=q.min_p, uniform=q.uniform,
                             top_k=q.top_k, repetition=q.repetition, presence=q.presence, frequency=q.frequency,
                             history=q.history if q.history else None, bias_ids=bi if bi else None,
                             bias_values=[bias[i] for i in bi] if bi else None,
                             mask_words=q.mask if q.mask is not None else None)
        assert got.status in (0, 1) and ref["status"] == 0, (r, got.status, ref["status"])
        # an uncertified row still carries the oracle's token (no boundary
        # draw among these rows)
        assert got.token == ref["token"], (r, got.status, got.token, ref["token"])
        if q.top_logprobs is None or got.token == stop:
            assert got.receipt is None, r
            continue
        assert got.receipt.token == got.token, r
        xs = x[r].copy()
        xs[sup] = F32_MIN
        _, rids, rlps, rmx, rln = orc.token_logprob_top(xs, q.top_logprobs + 8)
        head = [(int(i), float(l)) for i, l in zip(rids, rlps) if i < TV][: q.top_logprobs]
        assert [i for i, _ in got.receipt.top] == [i for i, _ in head], r
        assert np.allclose([l for _, l in got.receipt.top], [l for _, l in head], rtol=1e-5, atol=0)
        want = (float(xs[got.token]) - rmx) - rln
        assert abs(got.receipt.logprob - want) <= 1e-5 * abs(want), (r, got.receipt.logprob, want)
    assert sum(g.status == 1 for g in res) <= 1, [g.status for g in res]
    assert res[5].token == stop and res[5].receipt is None
    assert res[3].receipt is not None and res[3].receipt.top == []   # top_logprobs 0: the logprob alone
