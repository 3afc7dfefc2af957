"""GPU tests of the grammar-mask staging (mxs_mask_host / mxs_mask_upload):
the SimpleVob words a constraint computes on the host each step
(crates/core/engine/src/constraint.rs:777-806) reach the device bit for bit,
and double-buffered steps, each queued without a host wait on the picks,
sample under their own step's masks: every step is held to compare()
against the oracle given that step's words."""
import copy
import ctypes
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


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def device_to_host(ptr, nbytes):
    """hipMemcpy (device to host) of raw device memory the sampler owns."""
    hip = ctypes.CDLL("libamdhip64.so")
    out = np.zeros(nbytes // 4, dtype=np.uint32)
    rc = hip.hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(ptr), ctypes.c_size_t(nbytes),
                       ctypes.c_int(2))
    assert rc == 0, rc
    return out


def test_upload_round_trip(torch_mod):
    from metallix_amd import Sampler

    say("case mask-round-trip: rows 32 vocab 151936")
    s = Sampler(max_rows=32, max_vocab=151936)
    try:
        words = (151936 + 31) // 32
        rng = np.random.default_rng(5)
        got = []
        for slot in (0, 1):
            host = s.mask_host(slot)
            assert host.shape[0] == 32 and host.shape[1] >= words and host.shape[1] % 4 == 0
            host[:] = rng.integers(0, 2**32, size=host.shape, dtype=np.uint64).astype(np.uint32)
            want = host.copy()
            dev = s.mask_upload(slot, 32)
            s.sync()
            back = device_to_host(dev.data_ptr(), want.size * 4).reshape(want.shape)
            got.append(np.array_equal(back, want))
            # a partial upload copies its rows only
            host[:4] = 0
            dev = s.mask_upload(slot, 4)
            s.sync()
            back = device_to_host(dev.data_ptr(), want.size * 4).reshape(want.shape)
            got.append(np.array_equal(back[:4], np.zeros_like(want[:4])) and np.array_equal(back[4:], want[4:]))
        assert all(got), got
    finally:
        s.close()


def test_double_buffered_steps(torch_mod, orc):
    """Eight steps over slots 0 1 0 1 0 0 1 1 (a slot reused back to back
    too), each with its own masks (config 3's rows rolled by the step), all
    queued before one synchronisation."""
    from metallix_amd import Sampler, synth

    torch = torch_mod
    base = synth.config3(rows=16)
    words = base.mask_words.shape[1]
    s = Sampler(max_rows=16, max_vocab=base.vocab)
    try:
        logits, kw = to_device(torch, base)
        slots = [0, 1, 0, 1, 0, 0, 1, 1]
        outs, batches = [], []
        for i, slot in enumerate(slots):
            b = copy.copy(base)
            b.mask_words = np.roll(base.mask_words, i, axis=0)
            b.uniform = np.roll(base.uniform, 3 * i)
            say(f"case mask-step {i}: slot {slot} rows {b.rows}")
            host = s.mask_host(slot)
            host[:, :] = 0
            host[:b.rows, :words] = b.mask_words
            dev = s.mask_upload(slot, b.rows)
            skw = dict(kw)
            skw["uniform"] = torch.from_numpy(b.uniform.astype(np.float64)).cuda()
            skw["mask"] = dev
            outs.append(s.sample(logits, debug=True, **skw))
            batches.append(b)
        s.sync()
        for i, (b, out) in enumerate(zip(batches, outs)):
            gpu = dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
                       sampling_logprob=out.sampling_logprob.cpu().numpy(), adjusted=out.adjusted.cpu().numpy(),
                       kept=unpack_bits(out.kept_bits.cpu().numpy(), b.vocab))
            compare(b, gpu, orc.sample_batch(b, debug=True))
            say(f"mask-step {i} matches")
    finally:
        s.close()


def test_upload_requires_staging_and_bounds(torch_mod):
    from metallix_amd import Sampler, SamplerError

    s = Sampler(max_rows=4, max_vocab=1000)
    try:
        with pytest.raises(SamplerError):
            s.mask_upload(0, 4)        # nothing staged yet
        s.mask_host(1)
        with pytest.raises(SamplerError):
            s.mask_upload(1, 5)        # more rows than the context holds
        with pytest.raises(SamplerError):
            s.mask_host(2)             # two slots only
    finally:
        s.close()
