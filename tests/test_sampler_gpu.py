"""GPU parity: the HIP sampler against the CPU oracle on identical inputs.

Bar: statuses, adjusted logits, kept sets and tokens bit-exact; sampling
logprobs within 1e-5 relative; the only tolerated token difference is a draw
whose uniform lies within 1e-6 of a CDF boundary (checked per row), and the
device must flag no row uncertified on these inputs.
"""
import math
import sys

import numpy as np
import pytest

from helpers import compare, run_gpu

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


def check(torch_mod, sampler, orc, b, **kw):
    say(f"case {b.name}: rows {b.rows} vocab {b.vocab}")
    ref = orc.sample_batch(b, debug=True)
    gpu = run_gpu(torch_mod, sampler, b)
    compare(b, gpu, ref, **kw)
    return gpu, ref


def test_config1_sampled_and_greedy(torch_mod, sampler, orc):
    from metallix_amd import synth

    gpu, ref = check(torch_mod, sampler, orc, synth.config1())
    assert gpu["token"][0] == ref["token"][0]
    gpu, ref = check(torch_mod, sampler, orc, synth.config1(greedy=True))
    assert gpu["token"][0] == ref["token"][0]


def test_config2_batched_mixed(torch_mod, sampler, orc):
    from metallix_amd import synth

    check(torch_mod, sampler, orc, synth.config2())


def test_config3_bf16_grammar_masks(torch_mod, sampler, orc):
    from metallix_amd import synth

    gpu, ref = check(torch_mod, sampler, orc, synth.config3())
    single = [0, 9, 18, 27]
    assert all(gpu["kept_count"][r] == 1 for r in single)


def test_config4_large_vocab(torch_mod, sampler, orc):
    """BASELINE config 4 at its stated size, 256 x 262144."""
    from metallix_amd import synth

    b = synth.config4()
    assert b.rows == 256 and b.vocab == 262144
    check(torch_mod, sampler, orc, b)


# ---- randomized small and ragged shapes ----------------------------------------
def random_batch(seed, rows, V, *, mask=False, penalties=False, bias=False, ties=False):
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(seed)
    if ties:
        x = rng.integers(-4, 5, size=(rows, V)).astype(np.float32) * np.float32(0.5)
        x[rng.random((rows, V)) < 0.05] = -0.0
    else:
        x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    T = rng.choice([0.0, 0.25, 0.7, 1.0, 1.8], size=rows)
    topk = rng.choice([0, 1, 2, 5, 40, max(V - 1, 1), V, V + 3], size=rows).astype(np.uint32)
    topp = rng.choice([1.0, 0.95, 0.6, 0.2, 1e-9], size=rows)
    minp = rng.choice([0.0, 0.0, 0.05, 0.5, 1.0], size=rows)
    b = Batch(name=f"random-{seed}", logits=x, temperature=T, uniform=rng.random(rows), top_k=topk,
              top_p=topp, min_p=minp)
    if penalties:
        b.repetition = rng.choice([1.0, 1.1, 1.5], size=rows).astype(np.float32)
        b.presence = rng.choice([0.0, 0.5], size=rows).astype(np.float32)
        b.frequency = rng.choice([0.0, 0.3, -0.25], size=rows).astype(np.float32)
        lens = rng.integers(0, 3 * V // 2 + 2, size=rows)
        b.history_offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
        b.history_ids = rng.integers(0, V, size=int(lens.sum())).astype(np.uint32)
    if bias:
        ids, offs = [], [0]
        for r in range(rows):
            k = int(rng.integers(0, min(V, 12) + 1))
            ids.append(np.sort(rng.choice(V, size=k, replace=False)))
            offs.append(offs[-1] + k)
        b.bias_offsets = np.array(offs, dtype=np.uint32)
        b.bias_ids = np.concatenate(ids).astype(np.uint32) if offs[-1] else np.zeros(0, np.uint32)
        b.bias_values = rng.choice([-100.0, -1.5, 0.0, 2.0, 25.0], size=offs[-1]).astype(np.float32)
    if mask:
        words = (V + 31) // 32
        legal = rng.random((rows, V)) < rng.choice([0.02, 0.3, 1.0], size=(rows, 1))
        legal[np.arange(rows), rng.integers(0, V, size=rows)] = True
        m = np.zeros((rows, words), dtype=np.uint32)
        for r in range(rows):
            idx = np.nonzero(legal[r])[0]
            np.bitwise_or.at(m[r], idx // 32, (np.uint32(1) << (idx % 32).astype(np.uint32)))
        b.mask_words = m
        b.tokenizer_vocab = V
    return b


SHAPES = [(8, 1), (8, 3), (8, 5), (8, 31), (8, 33), (8, 100), (8, 4096), (8, 5003), (4, 40962), (4, 90001)]


@pytest.mark.parametrize("rows,V", SHAPES)
def test_random_plain(torch_mod, sampler, orc, rows, V):
    check(torch_mod, sampler, orc, random_batch(1000 + V, rows, V))


@pytest.mark.parametrize("rows,V", SHAPES)
def test_random_ties_penalties_bias(torch_mod, sampler, orc, rows, V):
    check(torch_mod, sampler, orc, random_batch(2000 + V, rows, V, ties=True, penalties=True, bias=True))


@pytest.mark.parametrize("rows,V", SHAPES)
def test_random_masked(torch_mod, sampler, orc, rows, V):
    check(torch_mod, sampler, orc, random_batch(3000 + V, rows, V, mask=True, penalties=True))


def test_random_batch_past_128_rows(torch_mod, sampler, orc):
    """160 rows: grid row groups past 16 and every per-row scratch region
    past row 128 (counters, exchange words, chunk statistics, candidates)."""
    b = random_batch(4160, 160, 20003, penalties=True, bias=True)
    check(torch_mod, sampler, orc, b)
    b = random_batch(4161, 160, 20003, mask=True)
    check(torch_mod, sampler, orc, b)


def test_error_matrix(torch_mod, sampler, orc):
    from metallix_amd.synth import Batch

    V = 64
    base = np.linspace(-3, 3, V, dtype=np.float32)
    cases = []
    def add(**kw):
        x = kw.pop("x", base.copy())
        cases.append((x, kw))
    add(temperature=-1.0)
    add(temperature=math.nan)
    add(temperature=math.inf)
    add(temperature=1.0, top_p=0.0)
    add(temperature=1.0, top_p=1.5)
    add(temperature=1.0, min_p=-0.1)
    add(temperature=1.0, min_p=2.0)
    add(temperature=1.0, repetition=0.0)
    add(temperature=1.0, presence=math.inf)
    add(temperature=1.0, uniform=1.0)
    add(temperature=1.0, uniform=-0.5)
    add(temperature=0.0, uniform=7.0)          # greedy ignores the uniform
    xn = base.copy(); xn[5] = math.nan
    add(x=xn, temperature=1.0)
    xi = base.copy(); xi[63] = -math.inf
    add(x=xi, temperature=0.0)
    add(temperature=1e-300, x=np.array([0.0] * 62 + [3.0e38, -3.0e38], dtype=np.float32))
    rows = len(cases)
    x = np.stack([c[0] for c in cases])
    g = lambda k, d: np.array([c[1].get(k, d) for c in cases])
    b = Batch(name="errors", logits=x, temperature=g("temperature", 1.0).astype(np.float64),
              uniform=g("uniform", 0.3).astype(np.float64), top_p=g("top_p", 1.0).astype(np.float64),
              min_p=g("min_p", 0.0).astype(np.float64), repetition=g("repetition", 1.0).astype(np.float32),
              presence=g("presence", 0.0).astype(np.float32), top_k=np.zeros(rows, np.uint32))
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert list(gpu["status"]) == list(ref["status"])


def test_history_and_bias_validation(torch_mod, sampler, orc):
    from metallix_amd.synth import Batch

    V = 100
    x = np.tile(np.linspace(-2, 2, V, dtype=np.float32), (4, 1))
    b = Batch(name="ids", logits=x, temperature=np.ones(4), uniform=np.full(4, 0.5),
              history_offsets=np.array([0, 1, 2, 2, 2], np.uint32), history_ids=np.array([3, V], np.uint32),
              bias_offsets=np.array([0, 0, 0, 2, 3], np.uint32), bias_ids=np.array([5, 5, 7], np.uint32),
              bias_values=np.array([1.0, 2.0, math.nan], np.float32))
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert list(ref["status"]) == [0, -11, -12, -12]


def selection_batch(seed, rows, V):
    """Peaked rows (noise plus a few high logits) over the parameter ranges
    the register-slot finisher decides: top-k from 1 to 4096, top-p and
    min-p on and off, low and high temperatures, and rows whose top logits
    tie exactly (the crossing-bin ranking and the general paths)."""
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    for r in range(rows):
        npk = int(rng.integers(1, 60))
        ids = rng.choice(V, size=npk, replace=False)
        x[r, ids] += rng.uniform(3.0, 10.0, size=npk).astype(np.float32)
        if r % 7 == 3:   # a tied plateau at the top
            ids = rng.choice(V, size=int(rng.integers(2, 200)), replace=False)
            x[r, ids] = np.float32(x[r].max() + 0.5)
    T = rng.choice([0.3, 0.8, 1.5, 3.0], size=rows)
    topk = rng.choice([0, 1, 20, 64, 500, 1000, 2000, 4096], size=rows).astype(np.uint32)
    topp = rng.choice([1.0, 0.95, 0.7, 0.5], size=rows)
    minp = rng.choice([0.0, 0.001, 0.05, 0.3], size=rows)
    return Batch(name=f"selection-{seed}", logits=x, temperature=T, uniform=rng.random(rows), top_k=topk,
                 top_p=topp, min_p=minp)


@pytest.mark.parametrize("seed", [1, 2])
def test_selection_finisher_mix(torch_mod, sampler, orc, seed):
    """Parity over the selection finisher's range, every row certified.
    Rows whose nucleus holds more than 8192 tokens (min_p 0.001 at high
    temperature) take the large-set path; their nucleus cut rests on the
    row mass, which the chunks sum from f64 weights once a chunk holds more
    than 2048 min-p candidates (an f32 mass's bound, about 5e-6 of the
    total, is coarser than one token's share there)."""
    b = selection_batch(seed, 64, 151936)
    say(f"case {b.name}: rows {b.rows} vocab {b.vocab}")
    ref = orc.sample_batch(b, debug=True)
    gpu = run_gpu(torch_mod, sampler, b)
    wide = np.asarray(ref["kept"]).sum(axis=1) > 8192
    unc = np.asarray(gpu["status"]) == 1
    say(f"wide rows {int(wide.sum())}, uncertified {int(unc.sum())}")
    assert wide.any()
    compare(b, gpu, ref)


def test_wide_min_p_nuclei_certified(torch_mod, sampler, orc):
    """Rows whose min-p set is most of the vocabulary (min_p 0.001 at
    temperatures 2 to 4, with and without penalties) and whose top-p
    nucleus holds tens of thousands of tokens: each token carries about
    1e-5 of the row mass, and every row's cut and draw must still be
    certified and match the reference."""
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(4242)
    rows, V = 24, 151936
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    for r in range(rows):
        ids = rng.choice(V, size=int(rng.integers(1, 30)), replace=False)
        x[r, ids] += rng.uniform(2.0, 6.0, size=len(ids)).astype(np.float32)
    hist = rng.integers(0, V, size=rows * 512).astype(np.uint32)
    pen = np.arange(rows) % 2 == 0
    b = Batch(name="wide-min-p", logits=x, temperature=rng.choice([2.0, 3.0, 4.0], size=rows),
              uniform=rng.random(rows), top_k=np.zeros(rows, np.uint32), top_p=rng.choice([0.5, 0.7, 0.9], size=rows),
              min_p=np.full(rows, 0.001), repetition=np.where(pen, 1.2, 1.0).astype(np.float32),
              presence=np.where(pen, 0.4, 0.0).astype(np.float32), frequency=np.where(pen, 0.2, 0.0).astype(np.float32),
              history_offsets=(np.arange(rows + 1, dtype=np.uint32) * 512), history_ids=hist)
    say(f"case {b.name}: rows {b.rows} vocab {b.vocab}")
    ref = orc.sample_batch(b, debug=True)
    gpu = run_gpu(torch_mod, sampler, b)
    kept = np.asarray(ref["kept"]).sum(axis=1)
    say(f"kept sizes {int(kept.min())}..{int(kept.max())}")
    assert (kept > 8192).all()
    compare(b, gpu, ref)


def test_min_p_near_one_over_log_softmax(torch_mod, sampler, orc):
    """min_p 0.999 (and neighbours) over rows whose maximum is exactly 0
    with a few hundred tokens within 0.01 of it, so T ln(min_p) (about -1e-3)
    cuts among them: an f32 logarithm of min_p, whose error is absolute
    (T 2^-24), would misplace that cut when the logits give no relative
    margin."""
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(999)
    rows, V = 16, 151936
    x = rng.standard_normal((rows, V)) * 0.5 - 12.0
    x[:, :400] = rng.standard_normal((rows, 400)) * 0.002    # near-maximal tokens
    x = (x - x.max(axis=1, keepdims=True)).astype(np.float32)  # maximum exactly 0
    b = Batch(name="minp-near-one", logits=x, temperature=rng.choice([0.5, 1.0, 2.0], size=rows),
              uniform=rng.random(rows), top_k=np.zeros(rows, np.uint32),
              top_p=rng.choice([1.0, 0.9], size=rows), min_p=rng.choice([0.999, 0.9999, 0.99], size=rows))
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert (np.asarray(ref["kept"]).sum(axis=1) > 1).any()


def test_keepall_rows_with_history_and_bias(torch_mod, sampler, orc):
    """Keep-all rows (top_k 0, top_p 1, min_p 0) over config 2's 2048-id
    histories plus a logit bias: the inverse-CDF draw over the whole row
    re-derives its segment's penalised logits (history counts, bias lookup)."""
    from metallix_amd import synth

    b = synth.config2(rows=16)
    b.name = "keepall-history"
    b.top_k[:] = 0
    b.top_p[:] = 1.0
    b.min_p[:] = 0.0
    s = synth.Stream(0xb1a5)
    ids, offs = [], [0]
    for r in range(b.rows):
        u = np.unique(s.u64(64) % np.uint64(b.vocab)).astype(np.uint32)
        ids.append(u)
        offs.append(offs[-1] + len(u))
    b.bias_ids = np.concatenate(ids)
    b.bias_offsets = np.array(offs, dtype=np.uint32)
    b.bias_values = (3.0 * (s.uniform(len(b.bias_ids)) - 0.5)).astype(np.float32)
    check(torch_mod, sampler, orc, b)


def test_nonpositive_bias_rows(torch_mod, sampler, orc):
    """Config 2's rows with logit-bias lists whose values are all at most 0
    (-inf suppressions, negative and zero biases), of 1 to 1025 entries, on
    tokens that are also in the row's history or are its argmax: the lean
    chunk body takes lists of up to 1024 such entries, the general body the
    rest; both are held to the oracle.  Then the lean body's validation:
    repeated or out-of-range bias ids with non-positive values."""
    from metallix_amd import synth
    from metallix_amd.synth import Batch

    b = synth.config2(rows=24)
    b.name = "nonpositive-bias"
    rng = np.random.default_rng(4242)
    b.temperature[::7] = 0.0
    sizes = [1, 8, 300, 1000, 1024, 1025] * 4
    ids_l, vals_l, offs = [], [], [0]
    for r in range(b.rows):
        h = b.history_ids[b.history_offsets[r]:b.history_offsets[r + 1]]
        pool = np.concatenate([rng.integers(0, b.vocab, sizes[r]), h[:sizes[r] // 3], [np.argmax(b.logits[r])]])
        ids = np.unique(pool.astype(np.uint32))[: sizes[r]]
        kind = rng.integers(0, 3, ids.size)
        vals = np.where(kind == 0, -np.inf, np.where(kind == 1, -np.abs(rng.standard_normal(ids.size)) * 3.0, 0.0))
        ids_l.append(ids)
        vals_l.append(vals.astype(np.float32))
        offs.append(offs[-1] + ids.size)
    b.bias_offsets = np.array(offs, dtype=np.uint32)
    b.bias_ids = np.concatenate(ids_l)
    b.bias_values = np.concatenate(vals_l)
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert (gpu["status"] == 0).all()

    V = 100
    x = np.tile(np.linspace(-2, 2, V, dtype=np.float32), (4, 1))
    c = Batch(name="bias-ids", logits=x, temperature=np.ones(4), uniform=np.full(4, 0.5),
              bias_offsets=np.array([0, 2, 4, 5, 7], np.uint32), bias_ids=np.array([3, 9, 5, 5, V, 1, 99], np.uint32),
              bias_values=np.array([-1.0, -np.inf, -2.0, 0.0, -1.0, -np.inf, -0.5], np.float32))
    gpu, ref = check(torch_mod, sampler, orc, c)
    assert list(ref["status"]) == [0, -12, -12, 0]


def test_nonpositive_bias_default_layout(torch_mod, sampler, orc):
    """All of config 2 (64 rows: four chunks per row, the layout of the
    benchmark) with the checkpoint's suppressed IDs and a non-positive bias
    list per row: every row takes the lean chunk body with bias owners."""
    from metallix_amd import synth
    from metallix_amd.sampler import with_suppression

    b = synth.config2()
    b.name = "nonpositive-bias-64"
    rng = np.random.default_rng(991)
    own_ids = [np.unique(rng.integers(0, b.vocab, 40)).astype(np.uint32) for _ in range(b.rows)]
    for r in range(0, b.rows, 3):   # some rows bias their own argmax and history tokens down
        h = b.history_ids[b.history_offsets[r]:b.history_offsets[r + 1]]
        own_ids[r] = np.unique(np.concatenate([own_ids[r], h[:20], [np.argmax(b.logits[r])]]).astype(np.uint32))
    own_off = np.concatenate([[0], np.cumsum([len(i) for i in own_ids])]).astype(np.uint32)
    own_val = (-np.abs(rng.standard_normal(int(own_off[-1]))) * 2.0).astype(np.float32)
    sup = [151643, 151645, int(np.argmax(b.logits[1]))]
    b.bias_offsets, b.bias_ids, b.bias_values = with_suppression(b.rows, sup, own_off, np.concatenate(own_ids),
                                                                 own_val)
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert (gpu["status"] == 0).all()


def test_suppressed_tokens(torch_mod, sampler, orc):
    """A7: the checkpoint's suppress list (ChatFormat::suppress,
    crates/core/chat-format/src/lib.rs:761-780), given to the device as -inf
    bias entries merged with the row's own bias (with_suppression): the
    suppressed tokens' adjusted logits are f32::MIN and the picks match the
    oracle's.  Rows cover greedy with its argmax suppressed, top-k / top-p /
    min-p rules, penalties, a row whose peaks are all suppressed, and
    config-3-style masked bf16 rows."""
    from metallix_amd import synth
    from metallix_amd.sampler import with_suppression

    b = synth.config2(rows=24)
    b.name = "suppress-cfg2"
    rng = np.random.default_rng(761)
    sup = np.unique(np.concatenate([rng.integers(0, b.vocab, 40), np.argmax(b.logits, axis=1)[:6]]))
    b.temperature[::5] = 0.0                      # greedy rows: several argmaxes are suppressed
    own_ids = [np.unique(rng.integers(0, b.vocab, 8)).astype(np.uint32) for _ in range(b.rows)]
    own_off = np.concatenate([[0], np.cumsum([len(i) for i in own_ids])]).astype(np.uint32)
    own_val = (rng.standard_normal(int(own_off[-1])) * 2.0).astype(np.float32)
    b.bias_offsets, b.bias_ids, b.bias_values = with_suppression(b.rows, sup, own_off, np.concatenate(own_ids),
                                                                 own_val)
    gpu, ref = check(torch_mod, sampler, orc, b)
    assert (gpu["status"] == 0).all()
    assert (gpu["adjusted"][:, sup] == np.float32(-3.4028234663852886e38)).all()
    assert not np.isin(gpu["token"], sup).any()

    # every peak of one row suppressed, at T 1 over a small vocabulary
    x = np.full((4, 512), -2.0, dtype=np.float32)
    x[:, 100:110] = 9.0
    c = synth.Batch(name="suppress-peaks", logits=x, temperature=np.ones(4), uniform=rng.random(4),
                    top_k=np.array([0, 5, 0, 1], dtype=np.uint32), top_p=np.array([0.9, 1.0, 1.0, 1.0]))
    c.bias_offsets, c.bias_ids, c.bias_values = with_suppression(4, np.arange(100, 110))
    gpu, ref = check(torch_mod, sampler, orc, c)
    assert not np.isin(gpu["token"], np.arange(100, 110)).any()

    # masked bf16 rows (the grammar path) with suppression
    d = synth.config3(rows=8)
    d.name = "suppress-masked"
    d.bias_offsets, d.bias_ids, d.bias_values = with_suppression(d.rows, rng.integers(0, d.vocab, 300))
    check(torch_mod, sampler, orc, d)
