"""Every finisher path of mxs_sample, reached at V = 151936 and checked
against the oracle.  mxs_debug_set_paths records the path each row took
(MXS_PATH_* of include/mx_sampler.h); one batch holds a row built for each
path, and the test asserts both the path and parity (statuses, adjusted
logits, kept sets and tokens bit-exact, logprobs within 1e-5).  The
reference's counterparts are the row-level rules the paths implement:
greedy_token (chat_generation.rs:2213-2231), nucleus_mask
(qwen_forward.rs:474-549) and sample_categorical (sampling.rs:56-158)."""
import sys

import numpy as np
import pytest

from helpers import compare, run_gpu, to_device

pytestmark = pytest.mark.gpu

V = 151936
PATHS = {"ERROR": 1, "GREEDY": 2, "KEEPALL": 3, "KEEPALL_RACE": 4, "SELECT": 5, "WAVE": 6, "FAST": 7,
         "EXACT": 8, "EXACT_SORTED": 9, "EXACT_REPLAY": 10, "LARGE": 11, "SHORT": 12,
         "LARGE_K": 11}


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def sampler(torch_mod):
    from metallix_amd import Sampler

    s = Sampler(max_rows=64, max_vocab=V)
    yield s
    s.close()


def path_batch(pad=0):
    """One row per path: (expected path, logits, T, top_k, top_p, min_p),
    then `pad` top-k rows named PAD (no expected path) that bring the batch
    to the row count where each row streams in the default chunk layout."""
    from metallix_amd.synth import Batch

    rng = np.random.default_rng(2365)
    rows = []

    def noise(scale=1.0, shift=0.0):
        return (rng.standard_normal(V) * scale + shift).astype(np.float32)

    def crowd(n, base=5.0, step=1e-6, floor=-40.0):
        """n near-equal logits base - i step at random ids, the rest at floor."""
        x = np.full(V, floor, dtype=np.float32)
        ids = rng.choice(V, n, replace=False)
        x[ids] = (base - step * np.arange(n)).astype(np.float32)
        return x

    peaked = noise(2.0)
    peaked[rng.choice(V, 20, replace=False)] += 8.0
    rows.append(("ERROR", peaked.copy(), -1.0, 20, 0.9, 0.0))          # invalid temperature
    rows.append(("GREEDY", peaked.copy(), 0.0, 0, 1.0, 0.0))
    rows.append(("KEEPALL", noise(2.0), 0.9, 0, 1.0, 0.0))
    rows.append(("SHORT", peaked.copy(), 0.7, 20, 0.8, 0.0))
    rows.append(("SELECT", peaked.copy(), 0.7, 100, 0.8, 0.0))     # k above the one-wave finisher's 64
    # a grammar-masked row (mask below) with 60 legal tokens, top-p only
    rows.append(("WAVE", noise(1.0), 1.0, 0, 0.9, 0.0))
    rows.append(("FAST", crowd(3000, step=1e-3), 1.0, 0, 1.0, 0.01))   # a min-p set of 3000
    def groups(*spec, floor=-40.0):
        """(count, value) groups of equal logits at random ids, the rest at floor."""
        x = np.full(V, floor, dtype=np.float32)
        ids = rng.choice(V, sum(n for n, _ in spec), replace=False)
        at = 0
        for n, v in spec:
            x[ids[at:at + n]] = np.float32(v)
            at += n
        return x

    # 300 logits at 5.0 over 7000 at 4.9, k 500: every chunk emits more
    # candidates than its register slots, and the k-th key is one of 7000
    # equal keys (the LDS select gives up; the radix select finds the head)
    two = groups((300, 5.0), (7000, 4.9))
    rows.append(("EXACT", two.copy(), 1.0, 500, 1.0, 0.0))
    rows.append(("EXACT_SORTED", two.copy(), 1.0, 500, 0.5, 0.0))
    # 7000 equal logits, a head of 1200 and top_p 0.5: the nucleus ends
    # exactly on a token boundary, which only the reference's own
    # sequential sums settle
    rows.append(("EXACT_REPLAY", groups((7000, 5.0)), 1.0, 1200, 0.5, 0.0))
    rows.append(("LARGE", crowd(10000, step=1e-4), 1.0, 0, 0.7, 0.0))
    # 9000 equal logits, a head of 1200 and top_p 0.5: the head's value bin
    # holds more tokens than the finisher's LDS cache, so the row stays on
    # the candidate-list finisher, which has no replay: the exact boundary
    # comes back uncertified (and settles from the exported candidates)
    rows.append(("LARGE_K", groups((9000, 5.0)), 1.0, 1200, 0.5, 0.0))
    for _ in range(pad):
        rows.append(("PAD", noise(2.0), 0.8, 50, 0.9, 0.05))
    names = [r[0] for r in rows]
    words = (V + 31) // 32
    mask = np.full((len(rows), words), 0xFFFFFFFF, dtype=np.uint32)
    w = names.index("WAVE")
    mask[w] = 0
    legal = rng.choice(V, 60, replace=False)
    np.bitwise_or.at(mask[w], legal // 32, (np.uint32(1) << (legal % 32).astype(np.uint32)))
    b = Batch(name="finisher-paths", logits=np.stack([r[1] for r in rows]),
              temperature=np.array([r[2] for r in rows]), uniform=rng.random(len(rows)),
              top_k=np.array([r[3] for r in rows], dtype=np.uint32), top_p=np.array([r[4] for r in rows]),
              min_p=np.array([r[5] for r in rows]), mask_words=mask, tokenizer_vocab=V)
    return names, b


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_every_finisher_path(torch_mod, sampler, orc):
    torch = torch_mod
    names, b = path_batch(pad=64 - 12)
    say(f"case finisher-paths: rows {b.rows} vocab {b.vocab}")
    buf = torch.zeros(b.rows, dtype=torch.int32, device="cuda")
    sampler.lib.mxs_debug_set_paths(sampler.ctx, buf.data_ptr())
    try:
        gpu = run_gpu(torch, sampler, b)
    finally:
        sampler.lib.mxs_debug_set_paths(sampler.ctx, None)
    got = buf.cpu().numpy()
    inv = {v: k for k, v in PATHS.items()}
    wrong = [(n, inv.get(int(p), int(p))) for n, p in zip(names, got) if n != "PAD" and PATHS[n] != int(p)]
    assert not wrong, f"rows took other paths: {wrong}"
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref, allow_uncertified=2)
    # an uncertified row may only be the large-set row (f32 chunk masses) or
    # the exact boundary of a head too large for the LDS cache
    unc = [names[r] for r in np.nonzero(gpu["status"] == 1)[0]]
    assert set(unc) <= {"LARGE", "LARGE_K"}, unc

    # the keep-all row under race-v2: the finisher keeps every token, no draw
    from test_race_gpu import oracle_race, race_keys

    keys = race_keys(b.rows, 3)
    logits, kw = to_device(torch, b)
    dev = logits.device
    race = (torch.from_numpy(keys[0].view(np.int64)).to(dev), torch.from_numpy(keys[1].view(np.int32)).to(dev),
            torch.from_numpy(keys[2].view(np.int32)).to(dev))
    sampler.lib.mxs_debug_set_paths(sampler.ctx, buf.data_ptr())
    try:
        out = sampler.sample(logits, race=race, **kw)
        torch.cuda.synchronize()
    finally:
        sampler.lib.mxs_debug_set_paths(sampler.ctx, None)
    got = buf.cpu().numpy()
    assert got[names.index("KEEPALL")] == PATHS["KEEPALL_RACE"]
    rref = oracle_race(orc, b, keys)
    tok = out.token.cpu().numpy()
    st = out.status.cpu().numpy()
    # only the large-set row may come back uncertified (its kept set rests on
    # the f32 chunk masses); every other row carries the oracle's winner
    assert set(names[r] for r in np.nonzero(st == 1)[0]) <= {"LARGE", "LARGE_K"}, st
    for r in range(b.rows):
        if names[r] == "ERROR":    # invalid temperature: the first pass's error, as without the race
            assert st[r] == gpu["status"][r] and st[r] < 0, st[r]
            continue
        assert st[r] in (0, 1), (names[r], st[r])
        if names[r] not in ("LARGE", "LARGE_K"):
            assert tok[r] == rref["token"][r], (names[r], st[r], tok[r], rref["token"][r])


def test_path_rows_small_batch(torch_mod, sampler, orc):
    """The same rows as one 12-row batch: fewer chunks than CUs, so each
    row streams in twice as many chunks (and its candidates reach the
    finishers from eight chunk lists instead of four).  Parity only: the
    paths follow from the layout.  The replay row's 7000 equal logits
    split into eight chunks of about 875, fewer than its k = 1200, so every
    chunk also emits its 19000 floor logits (ties at its k-th value): its
    lists outgrow the finisher's LDS cache, the head's value bin (the 7000)
    is compacted into it, and the replay settles the exact boundary.  The
    9000 of LARGE_K do not fit: that row stays uncertified."""
    names, b = path_batch()
    say(f"case finisher-paths-small: rows {b.rows} vocab {b.vocab}")
    gpu = run_gpu(torch_mod, sampler, b)
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref, allow_uncertified=2)
    unc = [names[r] for r in np.nonzero(gpu["status"] == 1)[0]]
    assert set(unc) <= {"LARGE", "LARGE_K"}, unc


def test_settle_uncertified_rows_from_exported_candidates(torch_mod, sampler, orc):
    """Candidate export (mxs_export_candidates; the reference's
    wait_with_candidates and pick_from_candidates, picks.rs:429-466,
    chat_generation.rs:2088-2131).  After the small-batch pick of the path
    rows, every status-1 row is a top-k row whose exported list settles on
    the host to the oracle's token without reading the row back; every
    certified top-k row's list settles to the device's token; the greedy,
    keep-all and error rows have no list (-1)."""
    from helpers import settle_from_candidates

    torch = torch_mod
    names, b = path_batch()
    say(f"case export-candidates: rows {b.rows} vocab {b.vocab}")
    gpu = run_gpu(torch, sampler, b, debug=False)
    ref = orc.sample_batch(b)
    W = 2048
    cnt, ids, lg = sampler.export_candidates(b.rows, W)
    torch.cuda.synchronize()
    cnt, ids, lg = cnt.cpu().numpy(), ids.cpu().numpy(), lg.cpu().numpy()
    unc = [r for r in range(b.rows) if gpu["status"][r] == 1]
    assert unc, "the path rows in the small-batch layout leave the replay row uncertified"
    settled = []
    for r in range(b.rows):
        if names[r] in ("ERROR", "GREEDY", "KEEPALL"):
            assert cnt[r] == -1, (names[r], cnt[r])
            continue
        k = int(b.top_k[r])
        if not 0 < k <= W:
            assert gpu["status"][r] != 1, f"uncertified row {names[r]} is not a top-k row the export settles"
            continue
        assert k <= cnt[r] <= W, (names[r], cnt[r])
        n = int(cnt[r])
        assert np.all(np.diff(ids[r, :n]) > 0), "token-ID order"
        tok = settle_from_candidates(orc, b, r, ids[r, :n], lg[r, :n])
        assert tok == ref["token"][r], (names[r], tok, ref["token"][r])
        if gpu["status"][r] == 0:
            assert tok == gpu["token"][r], (names[r], tok, gpu["token"][r])
        settled.append(names[r])
    assert all(names[r] in settled for r in unc), (unc, settled)


def test_large_heads_reduce_into_the_lds_cache(torch_mod, sampler, orc):
    """Heads of 1100 to 4096 over the full vocabulary: the chunks' lists
    outgrow the finisher's LDS cache (for k above 2048 every token is a
    candidate), the finisher histograms them below the row maximum and
    compacts the head's bins into the cache (finisher stamps 12-14).  Parity
    with the oracle on kept sets, adjusted logits, tokens and logprobs, with
    and without top_p / min_p, and with a penalised history on two rows."""
    from metallix_amd.synth import Batch

    torch = torch_mod
    rng = np.random.default_rng(4096)
    R = 16
    x = (rng.standard_normal((R, V)) * 2.0).astype(np.float32)
    x[3, rng.choice(V, 40, replace=False)] += 6.0
    k = np.array([1100, 2000, 3000, 4096] * 4, dtype=np.uint32)
    T = rng.uniform(0.5, 1.5, R)
    top_p = np.where(np.arange(R) % 2 == 0, 1.0, rng.uniform(0.5, 0.99, R))
    min_p = np.where(np.arange(R) % 4 == 3, 0.01, 0.0)
    u = rng.random(R)
    offs = np.zeros(R + 1, dtype=np.uint32)
    hist = [rng.choice(V, 300, replace=False).astype(np.uint32) if r in (5, 10) else np.zeros(0, np.uint32)
            for r in range(R)]
    offs[1:] = np.cumsum([len(h) for h in hist])
    b = Batch(name="large-heads", logits=x, temperature=T, uniform=u, top_k=k, top_p=top_p, min_p=min_p,
              repetition=np.full(R, 1.1, np.float32), presence=np.full(R, 0.5, np.float32),
              frequency=np.full(R, 0.3, np.float32), history_offsets=offs, history_ids=np.concatenate(hist))
    say(f"case large-heads: rows {R} vocab {V}")
    tb = torch.zeros(R * 65 * 16, dtype=torch.int64, device="cuda")
    sampler.lib.mxs_debug_set_timing(sampler.ctx, tb.data_ptr())
    try:
        gpu = run_gpu(torch, sampler, b)
    finally:
        sampler.lib.mxs_debug_set_timing(sampler.ctx, None)
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref)
    # the rows with k >= 2000 (chunk bounds from 2048 thread maxima or none)
    # went through the reduction (stamp 14 set)
    t = tb.view(R, 65, 16).cpu().numpy()
    big = k >= 2000
    assert (t[big, 64, 14] > 0).all(), t[:, 64, 12:15]


@pytest.mark.parametrize("seed", [21, 22])
def test_large_heads_random_plateaus(torch_mod, sampler, orc, seed):
    """Large heads over rows whose logits sit on a coarse grid (many equal
    values, so the head's value bin can hold more than the finisher's LDS
    cache and the list finisher keeps the row), with random k, T, top_p and
    min_p: parity with the oracle (status-1 rows only at exact boundaries,
    each still the oracle's token or a boundary draw)."""
    from metallix_amd.synth import Batch

    torch = torch_mod
    rng = np.random.default_rng(seed)
    R = 12
    x = (rng.standard_normal((R, V)) * 2.0).astype(np.float32)
    grid = rng.choice([0.25, 0.5, 1.0], R)
    coarse = rng.random(R) < 0.6
    x[coarse] = (np.round(x[coarse] / grid[coarse, None]) * grid[coarse, None]).astype(np.float32)
    k = rng.integers(1000, 4097, R).astype(np.uint32)
    T = rng.uniform(0.4, 1.5, R)
    top_p = np.where(rng.random(R) < 0.5, 1.0, rng.uniform(0.5, 0.99, R))
    min_p = np.where(rng.random(R) < 0.3, 0.01, 0.0)
    b = Batch(name="large-heads-plateaus", logits=x, temperature=T, uniform=rng.random(R), top_k=k,
              top_p=top_p, min_p=min_p)
    say(f"case large-heads-plateaus seed {seed}: rows {R} vocab {V}")
    gpu = run_gpu(torch, sampler, b)
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref, allow_uncertified=R)
