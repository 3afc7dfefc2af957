"""The lm_head epilogue fusion: a bf16 lm_head GEMM for gfx950
(mxs_lmhead_bf16) whose epilogue writes per-tile statistics
(metallix_amd/csrc/mxs_epilogue.h), and the finish-only pick over them
(mxs_finish_tiles), which reads only the logits tiles a top-k head can
reach.  Qwen3-0.6B-shaped head: hidden 1024, V 151936, 64 rows.  The
producer being fused is the reference's lm_head ahead of its device picks
(crates/models/qwen/src/forward.rs:1745-1761, Qwen3TokenPicks::start_with,
picks.rs:279-381).  The picks are checked against the oracle over the GEMM's
own f32 logits, read back, and against mxs_sample over the same logits."""
import numpy as np
import pytest

from helpers import compare, u32

pytestmark = pytest.mark.gpu

HID, V, R = 1024, 151936, 64


@pytest.fixture(scope="module")
def torch_mod():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="module")
def sampler(torch_mod):
    from metallix_amd import Sampler

    s = Sampler(max_rows=R, max_vocab=V)
    yield s
    s.close()


@pytest.fixture(scope="module")
def head(torch_mod):
    """Seeded bf16 hidden states and weights: logits of about N(0, 2^2),
    with a few rows' peaks from hidden states aligned to weight rows."""
    torch = torch_mod
    g = torch.Generator(device="cuda").manual_seed(1234)
    w = (torch.randn((V, HID), generator=g, device="cuda") * (2.0 / HID ** 0.5)).to(torch.bfloat16)
    h = torch.randn((R, HID), generator=g, device="cuda").to(torch.bfloat16)
    # rows 0..15 lean toward a few vocabulary rows (sharper distributions)
    for r in range(16):
        ids = torch.randint(0, V, (1 + r % 5,), generator=g, device="cuda")
        h[r] = (h[r].float() + 1.5 * w[ids].float().sum(0) * HID ** 0.5 / 2.0).to(torch.bfloat16)
    torch.cuda.synchronize()
    return h.contiguous(), w.contiguous()


def say(msg):
    import sys

    print(msg, flush=True)
    sys.stdout.flush()


def test_gemm_matches_fp32(torch_mod, sampler, head):
    """The MFMA GEMM against torch's f32 product of the same bf16 inputs,
    within the f32 summation bound 2 K 2^-24 sum |h| |w| per entry."""
    torch = torch_mod
    h, w = head
    say(f"case lmhead-gemm: rows {R} hidden {HID} vocab {V}")
    logits, _ = sampler.lmhead(h, w)
    torch.cuda.synchronize()
    hf, wf = h.float(), w.float()
    ref = torch.matmul(hf, wf.t().contiguous())
    bound = torch.matmul(hf.abs(), wf.abs().t().contiguous()) * (2.0 * HID * 2.0 ** -24) + 1e-30
    err = (logits - ref).abs()
    assert bool((err <= bound).all()), f"max err {err.max().item()} vs bound {bound.max().item()}"
    assert float(ref.std()) > 1.0   # the logits have a sampling-relevant scale


def rules(rng):
    """Greedy rows, top-k rows over k in {1, 20, 50, 100, 1000, 4096} with
    temperatures, top_p and some min_p, and three rows with a rule the
    finish-only pick does not serve (T > 0 without k)."""
    T = rng.uniform(0.3, 1.5, R)
    k = np.array([[1, 20, 50, 100, 1000, 4096][i % 6] for i in range(R)], dtype=np.uint32)
    top_p = rng.uniform(0.5, 1.0, R)
    top_p[::7] = 1.0
    min_p = np.where(np.arange(R) % 5 == 3, 0.05, 0.0)
    T[::8] = 0.0                        # greedy
    k[[5, 29, 47]] = 0                  # T > 0 without k: unsupported here
    T[[5, 29, 47]] = 0.8
    u = rng.random(R)
    return T, k, top_p, min_p, u


def test_finish_tiles_matches_oracle_and_sample(torch_mod, sampler, head, orc):
    """GEMM + epilogue statistics + finish-only pick: statuses, tokens, kept
    counts and logprobs as the oracle over the read-back logits (at most a
    boundary draw's worth of status-1 rows, each still the oracle's token),
    and the same tokens as mxs_sample over the same logits; unsupported
    rules report MXS_ROW_UNSUPPORTED_RULE."""
    from metallix_amd.synth import Batch

    torch = torch_mod
    h, w = head
    rng = np.random.default_rng(77)
    T, k, top_p, min_p, u = rules(rng)
    say(f"case lmhead-finish: rows {R} vocab {V}")
    logits, st = sampler.lmhead(h, w, stats=True)
    dev = logits.device
    D = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    kw = dict(top_k=D(u32(k)), top_p=D(top_p), min_p=D(min_p), uniform=D(u))
    out = sampler.finish_tiles(logits, st, D(T), **kw)
    torch.cuda.synchronize()
    gpu = dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
               sampling_logprob=out.sampling_logprob.cpu().numpy(), kept_count=out.kept_count.cpu().numpy())
    unsupported = [5, 29, 47]
    assert all(gpu["status"][r] == -15 for r in unsupported), gpu["status"][unsupported]
    keep = [r for r in range(R) if r not in unsupported]
    x = logits.cpu().numpy()
    b = Batch(name="lmhead", logits=x[keep], temperature=T[keep], uniform=u[keep], top_k=k[keep],
              top_p=top_p[keep], min_p=min_p[keep], tokenizer_vocab=V)
    ref = orc.sample_batch(b, debug=True)
    sub = {key: val[keep] for key, val in gpu.items()}
    compare(b, sub, ref, allow_uncertified=2, check_kept=False)
    # the same picks as mxs_sample over the same logits
    full = sampler.sample(logits, D(T), **kw)
    torch.cuda.synchronize()
    ft, fs = full.token.cpu().numpy(), full.status.cpu().numpy()
    for r in keep:
        if gpu["status"][r] == 0 and fs[r] == 0:
            assert gpu["token"][r] == ft[r], (r, gpu["token"][r], ft[r])


def test_finish_tiles_nonfinite_and_greedy_ties(torch_mod, sampler, orc):
    """A weight row that overflows to +inf makes every row's logits
    non-finite (MXS_ROW_NON_FINITE_LOGIT, as greedy_token and the nucleus
    path refuse them); and a head of equal logits across tiles keeps the
    lowest ID (greedy) and the lowest-ID ties of a top-k head."""
    torch = torch_mod
    K2, V2, R2 = 128, 4096, 4
    hid = torch.ones((R2, K2), dtype=torch.bfloat16, device="cuda")
    wt = torch.zeros((V2, K2), dtype=torch.bfloat16, device="cuda")
    wt[1000, 0] = 3e38
    wt[1000, 1] = 3e38
    lg, st = sampler.lmhead(hid, wt, stats=True)
    T = torch.tensor([0.0, 1.0, 0.0, 0.7], dtype=torch.float64, device="cuda")
    kk = torch.from_numpy(u32(np.array([0, 20, 0, 3], dtype=np.uint32))).to("cuda")
    out = sampler.finish_tiles(lg, st, T, top_k=kk, uniform=torch.full((R2,), 0.5, dtype=torch.float64, device="cuda"))
    torch.cuda.synchronize()
    assert (out.status.cpu().numpy() == -6).all(), out.status.cpu().numpy()
    # equal logits: rows of hidden 1 against weight rows with a 1.0 at every 500th token
    wt2 = torch.zeros((V2, K2), dtype=torch.bfloat16, device="cuda")
    wt2[::500, 0] = 1.0
    lg2, st2 = sampler.lmhead(hid, wt2, stats=True)
    out2 = sampler.finish_tiles(lg2, st2, T, top_k=kk, uniform=torch.full((R2,), 0.5, dtype=torch.float64, device="cuda"))
    torch.cuda.synchronize()
    from metallix_amd.synth import Batch

    x = lg2.cpu().numpy()
    b = Batch(name="ties", logits=x, temperature=T.cpu().numpy(), uniform=np.full(R2, 0.5),
              top_k=np.array([0, 20, 0, 3], dtype=np.uint32), tokenizer_vocab=V2)
    ref = orc.sample_batch(b, debug=True)
    gpu = dict(token=out2.token.cpu().numpy(), status=out2.status.cpu().numpy(),
               sampling_logprob=out2.sampling_logprob.cpu().numpy(), kept_count=out2.kept_count.cpu().numpy())
    compare(b, gpu, ref, check_kept=False)
    assert gpu["token"][0] == 0 and gpu["token"][2] == 0


def test_entry_points_reject_what_they_do_not_serve(torch_mod, sampler):
    """mxs_lmhead_bf16 refuses more than 64 rows, a hidden size that is not
    a multiple of 128, a vocabulary that is not a multiple of 4 and
    misaligned pointers; mxs_finish_tiles refuses bf16 logits, penalties and
    too small a statistics buffer (the Python side) before any launch."""
    import ctypes

    from metallix_amd.sampler import SamplerError

    torch = torch_mod
    lib, ctx = sampler.lib, sampler.ctx
    h = torch.zeros((65, 128), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((256, 128), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((65, 256), dtype=torch.float32, device="cuda")
    EINVAL = -1
    call = lambda rows, K, V, hp=h.data_ptr(), wp=w.data_ptr(), lp=lg.data_ptr(), ld=256: lib.mxs_lmhead_bf16(
        ctx, hp, wp, rows, K, V, lp, ld, None)
    assert call(65, 128, 256) == EINVAL                  # more than 64 rows
    assert call(4, 96, 256) == EINVAL                    # hidden_dim not a multiple of 128
    assert call(4, 128, 254) == EINVAL                   # vocab not a multiple of 4
    assert call(4, 128, 256, hp=h.data_ptr() + 2) == EINVAL   # misaligned hidden
    assert call(4, 128, 256, ld=255) == EINVAL           # stride below vocab / not a multiple of 4
    assert call(0, 128, 256) == 0                        # nothing to do
    assert b"128" in lib.mxs_last_error(ctx) or b"stride" in lib.mxs_last_error(ctx)
    torch.cuda.synchronize()

    logits, st = sampler.lmhead(h[:4], w, stats=True)
    T = torch.full((4,), 0.7, dtype=torch.float64, device="cuda")
    kk = torch.full((4,), 20, dtype=torch.int32, device="cuda")
    with pytest.raises(SamplerError):                    # bf16 logits
        sampler.finish_tiles(logits.to(torch.bfloat16), st, T, top_k=kk)
    with pytest.raises(ValueError):                      # statistics buffer too small
        sampler.finish_tiles(logits, st[:, :4], T, top_k=kk)
    with pytest.raises(SamplerError):                    # penalties are not served
        b, o, _, _ = sampler._structs(logits, T, top_k=kk,
                                      repetition=torch.full((4,), 1.1, dtype=torch.float32, device="cuda"))
        o.adjusted = None
        sampler._check(lib.mxs_finish_tiles(ctx, ctypes.byref(b), st.data_ptr(), ctypes.byref(o)), "mxs_finish_tiles")
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_finish_tiles_random_shapes(torch_mod, sampler, orc, seed):
    """Random shapes and rules through the GEMM + finish-only pick: vocab
    from 1000 to 40000 (some below the 256-token tile count of a head, so
    the value-grid histogram path runs), 1 to 64 rows, k from 1 to 4096,
    logits with plateaus (rounded to 1/8) on some rows; picks as the oracle
    over the read-back logits and as mxs_sample over the same logits."""
    from metallix_amd.synth import Batch

    torch = torch_mod
    rng = np.random.default_rng(seed)
    K2 = 128 * int(rng.integers(1, 4))
    V2 = 4 * int(rng.integers(250, 10000))
    R2 = int(rng.integers(1, 65))
    say(f"case finish-tiles-random seed {seed}: rows {R2} hidden {K2} vocab {V2}")
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn((V2, K2), generator=g, device="cuda") * (2.5 / K2 ** 0.5)).to(torch.bfloat16)
    h = torch.randn((R2, K2), generator=g, device="cuda").to(torch.bfloat16)
    if seed % 2:   # plateaus: many equal weights rows, so equal logits
        w[: V2 // 3] = torch.round(w[: V2 // 3].float() * 8).to(torch.bfloat16) / 8
    logits, st = sampler.lmhead(h.contiguous(), w.contiguous(), stats=True)
    T = rng.uniform(0.3, 1.5, R2)
    T[rng.random(R2) < 0.25] = 0.0
    k = rng.choice([1, 2, 7, 20, 64, 300, 1000, 4096], R2).astype(np.uint32)
    k = np.minimum(k, V2 - 1).astype(np.uint32)
    top_p = np.where(rng.random(R2) < 0.5, 1.0, rng.uniform(0.3, 0.99, R2))
    min_p = np.where(rng.random(R2) < 0.3, 0.02, 0.0)
    u = rng.random(R2)
    D = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    kw = dict(top_k=D(u32(k)), top_p=D(top_p), min_p=D(min_p), uniform=D(u))
    out = sampler.finish_tiles(logits, st, D(T), **kw)
    full = sampler.sample(logits, D(T), **kw)
    torch.cuda.synchronize()
    gpu = dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
               sampling_logprob=out.sampling_logprob.cpu().numpy(), kept_count=out.kept_count.cpu().numpy())
    b = Batch(name="finish-random", logits=logits.cpu().numpy(), temperature=T, uniform=u, top_k=k,
              top_p=top_p, min_p=min_p, tokenizer_vocab=V2)
    ref = orc.sample_batch(b, debug=True)
    compare(b, gpu, ref, allow_uncertified=max(2, R2 // 8), check_kept=False)
    ft, fs = full.token.cpu().numpy(), full.status.cpu().numpy()
    both = (gpu["status"] == 0) & (fs == 0)
    assert (gpu["token"][both] == ft[both]).all()
