"""Shared test helpers: upload synthetic batches, compare with the oracle."""
from __future__ import annotations

import numpy as np


def u32(t):
    """numpy u32 -> int32 view (torch has no general uint32 tensors)."""
    return np.ascontiguousarray(np.asarray(t, dtype=np.uint32)).view(np.int32)


def to_device(torch, b, dev="cuda"):
    """Uploads a synth.Batch; returns (logits tensor, kwargs for Sampler.sample)."""
    R, V = b.rows, b.vocab
    stride = (V + 3) // 4 * 4
    if b.bf16_bits is not None:
        host = np.zeros((R, stride), dtype=np.uint16)
        host[:, :V] = b.bf16_bits
        logits = torch.from_numpy(host.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        host = np.zeros((R, stride), dtype=np.float32)
        host[:, :V] = b.logits
        logits = torch.from_numpy(host).to(dev)
    T = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=dt))).to(dev)
    kw = dict(
        temperature=T(b.temperature, np.float64), uniform=T(b.uniform, np.float64),
        top_k=None if b.top_k is None else T(u32(b.top_k), np.int32),
        top_p=T(b.top_p, np.float64), min_p=T(b.min_p, np.float64),
        repetition=T(b.repetition, np.float32), presence=T(b.presence, np.float32),
        frequency=T(b.frequency, np.float32), vocab=V,
    )
    if b.history_offsets is not None:
        kw["history"] = (T(u32(b.history_offsets), np.int32), T(u32(b.history_ids), np.int32))
    if b.bias_offsets is not None:
        kw["bias"] = (T(u32(b.bias_offsets), np.int32), T(u32(b.bias_ids), np.int32), T(b.bias_values, np.float32))
    if b.mask_words is not None:
        kw["mask"] = T(u32(b.mask_words), np.int32)
        kw["tokenizer_vocab"] = b.tokenizer_vocab or V
    return logits, kw


def unpack_bits(words, V):
    w = np.asarray(words).view(np.uint32)
    out = np.zeros((w.shape[0], w.shape[1] * 32), dtype=bool)
    for b in range(32):
        out[:, b::32] = (w >> np.uint32(b)) & 1
    return out[:, :V]


def cdf_gap(b, row, kept, adjusted):
    """Distance in u-space from row `row`'s uniform to the nearest boundary of
    the inverse CDF over `kept` (that row's kept flags, ID order) with weights
    from `adjusted` (that row's adjusted logits), in f64 (used to recognise a
    documented boundary draw)."""
    x = np.asarray(adjusted).astype(np.float64)
    k = np.nonzero(kept)[0]
    if len(k) == 0:
        return 1.0
    m = x[k].max()
    w = np.exp((x[k] - m) / b.temperature[row])
    cum = np.cumsum(w) / w.sum()
    return float(np.min(np.abs(cum - b.uniform[row])))


def run_gpu(torch, sampler, b, debug=True):
    logits, kw = to_device(torch, b)
    out = sampler.sample(logits, debug=debug, **kw)
    torch.cuda.synchronize()
    res = dict(token=out.token.cpu().numpy(), status=out.status.cpu().numpy(),
               sampling_logprob=out.sampling_logprob.cpu().numpy(), kept_count=out.kept_count.cpu().numpy())
    if debug:
        res["adjusted"] = out.adjusted.cpu().numpy()
        res["kept"] = unpack_bits(out.kept_bits.cpu().numpy(), b.vocab)
    return res


def compare(b, gpu, ref, *, allow_uncertified=0, check_kept=True, rel=1e-5):
    """Asserts parity: statuses, tokens, kept sets and adjusted logits
    bit-exact; logprobs within `rel`; a token mismatch is allowed only on a
    row whose uniform lies within 1e-6 of a CDF boundary of the oracle's
    kept set.  At most `allow_uncertified` rows may carry status 1, and
    those too must match the oracle's token (or be such a boundary draw)."""
    R = b.rows
    problems = []
    unc = int((gpu["status"] == 1).sum())
    assert unc <= allow_uncertified, f"{unc} uncertified rows: {np.nonzero(gpu['status'] == 1)[0][:10]}"
    for r in range(R):
        gs, rs = int(gpu["status"][r]), int(ref["status"][r])
        if gs == 1:
            # Uncertified: the kept set rests on a decision inside the device's
            # error bound, so only the adjusted logits and the token are held:
            # the token must be the oracle's, or the row's uniform must lie
            # within 1e-6 of a CDF boundary of the oracle's kept set.
            if rs != 0:
                problems.append(f"row {r}: gpu uncertified, ref status {rs}")
                continue
            if "adjusted" in ref and "adjusted" in gpu and not np.array_equal(
                    gpu["adjusted"][r].view(np.uint32), ref["adjusted"][r].view(np.uint32)):
                problems.append(f"row {r}: adjusted logits differ (uncertified row)")
            if gpu["token"][r] != ref["token"][r]:
                gap = cdf_gap(b, r, ref["kept"][r], ref["adjusted"][r]) if "kept" in ref else 0.0
                if gap > 1e-6:
                    problems.append(f"row {r}: uncertified token gpu {gpu['token'][r]} ref {ref['token'][r]} "
                                    f"(cdf gap {gap:.3g})")
            continue
        if gs != rs:
            problems.append(f"row {r}: status gpu {gs} ref {rs}")
            continue
        if rs != 0:
            continue
        if "adjusted" in ref and "adjusted" in gpu:
            a, e = gpu["adjusted"][r], ref["adjusted"][r]
            if not np.array_equal(a.view(np.uint32), e.view(np.uint32)):
                bad = np.nonzero(a.view(np.uint32) != e.view(np.uint32))[0]
                problems.append(f"row {r}: adjusted logits differ at {bad[:5]}")
        if check_kept and "kept" in ref and "kept" in gpu:
            if not np.array_equal(gpu["kept"][r], ref["kept"][r]):
                d = np.nonzero(gpu["kept"][r] != ref["kept"][r])[0]
                problems.append(f"row {r}: kept sets differ at {d[:5]} (gpu {gpu['kept'][r].sum()} ref {ref['kept'][r].sum()})")
        if gpu["token"][r] != ref["token"][r]:
            gap = cdf_gap(b, r, ref["kept"][r], ref["adjusted"][r]) if "kept" in ref else 0.0
            if gap > 1e-6:
                problems.append(f"row {r}: token gpu {gpu['token'][r]} ref {ref['token'][r]} (cdf gap {gap:.3g})")
            continue
        g, e = gpu["sampling_logprob"][r], ref["sampling_logprob"][r]
        if abs(g - e) > rel * max(abs(e), 1e-300) and abs(g - e) > 1e-12:
            problems.append(f"row {r}: logprob gpu {g!r} ref {e!r}")
    assert not problems, "\n".join(problems[:20])


def settle_from_candidates(orc, b, r, ids, logits):
    """The host settle of row r from its exported candidates
    (mxs_export_candidates), as pick_from_candidates does for a top-k rule
    (crates/app/cli/src/chat_generation.rs:2088-2131): the row's rule (T,
    top_k, top_p, min_p and its uniform) applied by the oracle to the list
    alone, every other token at f32::MIN (weight 0, below any head); the
    list's logits already carry the penalties, bias and mask."""
    from metallix_amd.synth import Batch

    x = np.full(b.vocab, np.finfo(np.float32).min, dtype=np.float32)
    x[np.asarray(ids, dtype=np.int64)] = np.asarray(logits, dtype=np.float32)
    pick = lambda a, dflt: (np.asarray(a)[r:r + 1] if a is not None else dflt)
    one = Batch(name="settle", logits=x[None, :], temperature=b.temperature[r:r + 1],
                uniform=b.uniform[r:r + 1], top_k=pick(b.top_k, np.zeros(1, np.uint32)),
                top_p=pick(b.top_p, np.ones(1)), min_p=pick(b.min_p, np.zeros(1)),
                tokenizer_vocab=b.tokenizer_vocab)
    return int(orc.sample_batch(one)["token"][0])
