"""GPU test of mxs_logsoftmax_topn_noalloc, the context-free entry point
whose scratch is a static device array of the library (no counterpart in the
reference).  Through the C ABI, two calls in a row on one stream (the second
with a smaller input) must give exactly what mxs_logsoftmax_topn gives on the
same inputs (the same kernels), and the second also matches the oracle's
token_logprob (crates/app/cli/src/chat_turn.rs:506-563) under the top-N
test's bar.  Sizes past MXS_TOPN_STATIC_BYTES are rejected before launch."""
import ctypes
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


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def outputs(torch, rows, n):
    return (torch.full((rows, max(n, 1)), -7, dtype=torch.int32, device="cuda"),
            torch.full((rows, max(n, 1)), 7.0, dtype=torch.float64, device="cuda"),
            torch.zeros(rows, dtype=torch.float64, device="cuda"),
            torch.zeros(rows, dtype=torch.float64, device="cuda"),
            torch.full((rows,), 99, dtype=torch.int32, device="cuda"))


def call_noalloc(torch, lib, logits, V, n):
    rows = logits.shape[0]
    ids, lps, mx, ln, st = outputs(torch, rows, n)
    stream = torch.cuda.current_stream()
    rc = lib.mxs_logsoftmax_topn_noalloc(ctypes.c_void_p(stream.cuda_stream), logits.data_ptr(), 0, rows, V,
                                         logits.stride(0), n, ids.data_ptr(), lps.data_ptr(), mx.data_ptr(),
                                         ln.data_ptr(), st.data_ptr())
    assert rc == 0, lib.mxs_last_error(None)
    return ids[:, :n], lps[:, :n], mx, ln, st


def upload(torch, x):
    R, V = x.shape
    stride = (V + 3) // 4 * 4
    host = np.zeros((R, stride), dtype=np.float32)
    host[:, :V] = x
    return torch.from_numpy(host).to("cuda")


def test_noalloc_matches_context_entry_point_twice(torch_mod, orc):
    torch = torch_mod
    from metallix_amd import Sampler
    from metallix_amd.sampler import load_library

    lib = load_library()
    s = Sampler(max_rows=64, max_vocab=151936, stream=torch.cuda.current_stream())
    try:
        rng = np.random.default_rng(2024)
        cases = [(64, 151936, 28), (8, 40961, 20)]   # the second call is smaller
        got = []
        for rows, V, n in cases:
            say(f"noalloc case: rows {rows} vocab {V} n {n}")
            x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
            x[:, rng.integers(0, V, 16)] += 6.0
            t = upload(torch, x)
            a = call_noalloc(torch, lib, t, V, n)
            b = s.logsoftmax_topn(t, n, vocab=V)
            torch.cuda.synchronize()
            a = [v.cpu().numpy() for v in a]
            b = [v.cpu().numpy() for v in b]
            for name, u, w in zip(("ids", "logprobs", "maximum", "log_normalizer", "status"), a, b):
                assert np.array_equal(u, w), f"{name} differs from mxs_logsoftmax_topn (rows {rows}, V {V})"
            assert (a[4] == 0).all()
            got.append((x, n, a))
        # the second (smaller) call against the oracle
        x, n, (ids, lps, mx, ln, st) = got[1]
        for r in range(x.shape[0]):
            rs, rids, rlps, rmx, rln = orc.token_logprob_top(x[r], n)
            assert np.array_equal(ids[r, :len(rids)], rids), f"row {r}"
            assert mx[r] == rmx
            assert abs(ln[r] - rln) <= 2.0 ** -22 + 1e-13   # weights within 2^-22 of exact
            assert np.allclose(lps[r, :len(rids)], rlps, rtol=1e-5, atol=1e-12)
    finally:
        s.close()


def test_noalloc_rejects_sizes_past_the_static_array(torch_mod):
    from metallix_amd.sampler import load_library

    lib = load_library()
    dummy = torch_mod.zeros(64, dtype=torch_mod.float32, device="cuda")
    p = dummy.data_ptr()
    # 4096 rows x 32 chunks x (24 + 8 * 64) bytes is far past 8 MiB
    rc = lib.mxs_logsoftmax_topn_noalloc(None, p, 0, 4096, 262144, 262144, 64, p, p, p, p, p)
    assert rc == -1
    assert b"MXS_TOPN_STATIC_BYTES" in lib.mxs_last_error(None)
