"""ctypes binding of the CPU oracle (oracle/mx_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP sampler and the
timed CPU baseline of bench.py.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libmx_oracle.so"

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_dbl = ctypes.c_double


class RowParams(ctypes.Structure):
    _fields_ = [
        ("temperature", _dbl), ("top_p", _dbl), ("min_p", _dbl), ("uniform", _dbl),
        ("top_k", ctypes.c_uint32), ("repetition", ctypes.c_float), ("presence", ctypes.c_float),
        ("frequency", ctypes.c_float),
        ("history", _vp), ("history_len", _sz),
        ("bias_ids", _vp), ("bias_values", _vp), ("bias_len", _sz),
        ("mask_words", _vp), ("mask_nwords", _sz), ("tokenizer_vocab", _sz),
    ]


class RowResult(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int32), ("token", ctypes.c_int32),
                ("sampling_logprob", _dbl), ("kept_count", ctypes.c_uint32)]


class BatchC(ctypes.Structure):
    _fields_ = [
        ("logits", _vp), ("rows", _sz), ("vocab", _sz),
        ("temperature", _vp), ("top_p", _vp), ("min_p", _vp), ("uniform", _vp),
        ("top_k", _vp), ("repetition", _vp), ("presence", _vp), ("frequency", _vp),
        ("history_offsets", _vp), ("history_ids", _vp),
        ("bias_offsets", _vp), ("bias_ids", _vp), ("bias_values", _vp),
        ("mask_words", _vp), ("mask_nwords", _sz), ("tokenizer_vocab", _sz),
    ]


class ChaCha8(ctypes.Structure):
    _fields_ = [("key", ctypes.c_uint32 * 8), ("counter", ctypes.c_uint64),
                ("buf", ctypes.c_uint32 * 64), ("index", ctypes.c_uint32)]


def build() -> Path:
    res = subprocess.run(["make", "-C", str(HERE)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_unit_uniform.restype = _dbl
        L.orc_unit_uniform.argtypes = [ctypes.c_uint64]
        L.orc_chacha8_next_u64.restype = ctypes.c_uint64
        L.orc_gumbel_from_bits.restype = _dbl
        L.orc_gumbel_from_bits.argtypes = [ctypes.c_uint64]
        L.orc_race_bits.restype = ctypes.c_uint64
        L.orc_race_bits.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_race_score.restype = _dbl
        L.orc_race_score.argtypes = [ctypes.c_float, _dbl, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        for name in ("orc_sample_categorical", "orc_nucleus_mask", "orc_greedy_token", "orc_masked_argmax",
                     "orc_selected_model_logprob", "orc_token_logprob_top", "orc_accept_or_resample",
                     "orc_sample_race", "orc_sample_row", "orc_adjust_logits", "orc_spec_verify_row",
                     "orc_sample_batch", "orc_sample_batch_threads"):
            getattr(L, name).restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(_vp)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---- reference primitives --------------------------------------------------
def unit_uniform(word: int) -> float:
    return lib().orc_unit_uniform(ctypes.c_uint64(word))


class ChaChaStream:
    """ChaCha8Rng::seed_from_u64(seed) (rand_chacha 0.9.0 / rand_core 0.9.3)."""

    def __init__(self, seed: int):
        self.s = ChaCha8()
        lib().orc_chacha8_seed_from_u64(ctypes.byref(self.s), ctypes.c_uint64(seed))

    def next_u64(self) -> int:
        return lib().orc_chacha8_next_u64(ctypes.byref(self.s))


def sample_categorical(logits, legal, temperature: float, uniform: float):
    x = f32(logits)
    lg = None if legal is None else np.ascontiguousarray(np.asarray(legal, dtype=np.uint8))
    tok = ctypes.c_uint32()
    lp = _dbl()
    st = lib().orc_sample_categorical(_p(x), _p(lg), _sz(x.size), _dbl(temperature), _dbl(uniform),
                                      ctypes.byref(tok), ctypes.byref(lp))
    return st, tok.value, lp.value


def nucleus_mask(logits, temperature: float, top_p: float, top_k: int = 0):
    x = f32(logits)
    m = np.zeros(x.size, dtype=np.uint8)
    st = lib().orc_nucleus_mask(_p(x), _sz(x.size), _dbl(temperature), _dbl(top_p), _sz(top_k), _p(m))
    return st, m.astype(bool)


def greedy_token(logits):
    x = f32(logits)
    t = ctypes.c_int32()
    st = lib().orc_greedy_token(_p(x), _sz(x.size), ctypes.byref(t))
    return st, t.value


def masked_argmax(words, logits, width: int):
    w = np.ascontiguousarray(np.asarray(words, dtype=np.uint32))
    x = f32(logits)
    idx = ctypes.c_int64()
    lib().orc_masked_argmax(_p(w), _sz(w.size), _p(x), _sz(width), ctypes.byref(idx))
    return idx.value


def fill_legal_mask(words, tokenizer_vocab: int, n: int):
    w = np.ascontiguousarray(np.asarray(words, dtype=np.uint32))
    out = np.zeros(n, dtype=np.uint8)
    lib().orc_fill_legal_mask(_p(w), _sz(w.size), _sz(tokenizer_vocab), _p(out), _sz(n))
    return out.astype(bool)


def selected_model_logprob(logits, token: int):
    x = f32(logits)
    lp = _dbl()
    st = lib().orc_selected_model_logprob(_p(x), _sz(x.size), ctypes.c_uint32(token), ctypes.byref(lp))
    return st, lp.value


def token_logprob_top(logits, top: int):
    x = f32(logits)
    n = min(top, x.size)
    ids = np.zeros(n, dtype=np.int32)
    lps = np.zeros(n, dtype=np.float64)
    mx, ln = _dbl(), _dbl()
    st = lib().orc_token_logprob_top(_p(x), _sz(x.size), _sz(top), _p(ids), _p(lps), ctypes.byref(mx), ctypes.byref(ln))
    return st, ids, lps, mx.value, ln.value


def accept_or_resample(target, draft, drafted: int, accept_uniform: float, resample_uniform: float):
    t = np.ascontiguousarray(np.asarray(target, dtype=np.float64))
    d = np.ascontiguousarray(np.asarray(draft, dtype=np.float64))
    acc = ctypes.c_int()
    res = _sz()
    st = lib().orc_accept_or_resample(_p(t), _p(d), _sz(min(t.size, d.size) if t.size != d.size else t.size),
                                      _sz(drafted), _dbl(accept_uniform), _dbl(resample_uniform),
                                      ctypes.byref(acc), ctypes.byref(res))
    if t.size != d.size:
        return -14, None
    if st:
        return st, None
    return 0, ("accepted" if acc.value else ("resampled", res.value))


def philox4x32_10(counter, key):
    out = (ctypes.c_uint32 * 4)()
    lib().orc_philox4x32_10((ctypes.c_uint32 * 4)(*counter), (ctypes.c_uint32 * 2)(*key), out)
    return list(out)


def race_bits(seed: int, choice: int, position: int, row: int) -> int:
    return lib().orc_race_bits(seed, choice, position, row)


def gumbel_from_bits(bits: int) -> float:
    return lib().orc_gumbel_from_bits(bits)


def sample_race(logits, legal, temperature: float, seed: int, choice: int, position: int):
    x = f32(logits)
    lg = None if legal is None else np.ascontiguousarray(np.asarray(legal, dtype=np.uint8))
    tok = ctypes.c_uint32()
    lp = _dbl()
    st = lib().orc_sample_race(_p(x), _p(lg), _sz(x.size), _dbl(temperature), ctypes.c_uint64(seed),
                               ctypes.c_uint32(choice), ctypes.c_uint32(position), ctypes.byref(tok), ctypes.byref(lp))
    return st, tok.value, lp.value


# ---- composed row / batch sampler (build-defined stages) ---------------------
def sample_row(logits, *, temperature, top_p=1.0, min_p=0.0, uniform=0.0, top_k=0, repetition=1.0,
               presence=0.0, frequency=0.0, history=None, bias_ids=None, bias_values=None,
               mask_words=None, tokenizer_vocab=None):
    x = f32(logits)
    n = x.size
    keep = []
    p = RowParams()
    p.temperature, p.top_p, p.min_p, p.uniform = temperature, top_p, min_p, uniform
    p.top_k, p.repetition, p.presence, p.frequency = top_k, repetition, presence, frequency
    if history is not None and len(history):
        h = np.ascontiguousarray(np.asarray(history, dtype=np.uint32)); keep.append(h)
        p.history, p.history_len = h.ctypes.data, h.size
    if bias_ids is not None and len(bias_ids):
        bi = np.ascontiguousarray(np.asarray(bias_ids, dtype=np.uint32))
        bv = f32(bias_values); keep += [bi, bv]
        p.bias_ids, p.bias_values, p.bias_len = bi.ctypes.data, bv.ctypes.data, bi.size
    if mask_words is not None:
        mw = np.ascontiguousarray(np.asarray(mask_words, dtype=np.uint32)); keep.append(mw)
        p.mask_words, p.mask_nwords = mw.ctypes.data, mw.size
        p.tokenizer_vocab = n if tokenizer_vocab is None else tokenizer_vocab
    adj = np.zeros(n, dtype=np.float32)
    kept = np.zeros(n, dtype=np.uint8)
    r = RowResult()
    lib().orc_sample_row(_p(x), _sz(n), ctypes.byref(p), _p(adj), _p(kept), ctypes.byref(r))
    return dict(status=r.status, token=r.token, sampling_logprob=r.sampling_logprob,
                kept_count=r.kept_count, adjusted=adj, kept=kept.astype(bool))


def _batch_struct(b, keep):
    s = BatchC()

    def arr(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(np.asarray(a, dtype=dt))
        keep.append(a)
        return a.ctypes.data

    s.logits = arr(b.logits, np.float32)
    s.rows, s.vocab = b.rows, b.vocab
    s.temperature = arr(b.temperature, np.float64)
    s.top_p = arr(b.top_p, np.float64)
    s.min_p = arr(b.min_p, np.float64)
    s.uniform = arr(b.uniform, np.float64)
    s.top_k = arr(b.top_k, np.uint32)
    s.repetition = arr(b.repetition, np.float32)
    s.presence = arr(b.presence, np.float32)
    s.frequency = arr(b.frequency, np.float32)
    s.history_offsets = arr(b.history_offsets, np.uint32)
    s.history_ids = arr(b.history_ids, np.uint32)
    s.bias_offsets = arr(b.bias_offsets, np.uint32)
    s.bias_ids = arr(b.bias_ids, np.uint32)
    s.bias_values = arr(b.bias_values, np.float32)
    if b.mask_words is not None:
        s.mask_words = arr(b.mask_words, np.uint32)
        s.mask_nwords = b.mask_words.shape[1]
        s.tokenizer_vocab = b.tokenizer_vocab or b.vocab
    return s


def sample_batch(b, rows: Optional[range] = None, debug: bool = False):
    """Oracle over a synth.Batch; returns dict of numpy arrays."""
    keep = []
    s = _batch_struct(b, keep)
    R, V = b.rows, b.vocab
    tok = np.zeros(R, dtype=np.int32)
    lp = np.zeros(R, dtype=np.float64)
    st = np.zeros(R, dtype=np.int32)
    lo, hi = (0, R) if rows is None else (rows.start, rows.stop)
    adj = np.zeros((R, V), dtype=np.float32) if debug else None
    kept = np.zeros((R, V), dtype=np.uint8) if debug else None
    lib().orc_sample_batch(ctypes.byref(s), _sz(lo), _sz(hi), _p(tok), _p(lp), _p(st), _p(adj), _p(kept))
    out = dict(token=tok, sampling_logprob=lp, status=st)
    if debug:
        out["adjusted"] = adj
        out["kept"] = kept.astype(bool)
    return out


def sample_batch_threads(b, threads: int):
    keep = []
    s = _batch_struct(b, keep)
    R = b.rows
    tok = np.zeros(R, dtype=np.int32)
    lp = np.zeros(R, dtype=np.float64)
    st = np.zeros(R, dtype=np.int32)
    lib().orc_sample_batch_threads(ctypes.byref(s), ctypes.c_int(threads), _p(tok), _p(lp), _p(st))
    return dict(token=tok, sampling_logprob=lp, status=st)


def spec_verify_row(target, draft, draft_tokens, temperature, accept_u, resample_u, bonus_u):
    t = f32(target)
    d = f32(draft)
    k, V = d.shape
    toks = np.ascontiguousarray(np.asarray(draft_tokens, dtype=np.int32))
    ua = np.ascontiguousarray(np.asarray(accept_u, dtype=np.float64))
    ur = np.ascontiguousarray(np.asarray(resample_u, dtype=np.float64))
    out = np.full(k + 1, -1, dtype=np.int32)
    cnt = ctypes.c_int32()
    acc = ctypes.c_int32()
    st = lib().orc_spec_verify_row(_p(t), _p(d), _sz(V), _sz(k), _p(toks), _dbl(temperature), _p(ua), _p(ur),
                                   _dbl(bonus_u), _p(out), ctypes.byref(cnt), ctypes.byref(acc))
    return st, out, cnt.value, acc.value


# ---- point-mass verify walk (A9) ---------------------------------------------
def accept_and_roll_back(draft, pick_at):
    """The acceptance walk of speculative decoding
    (crates/core/engine/src/speculative.rs:318-347): rows 0..=len(draft) are
    settled in order by pick_at(i) -> (token, stop); a row's token is
    emitted, counts as accepted when it equals draft[i], and the walk ends
    after a stop token, after the first row that leaves the draft, or after
    the bonus row (index len(draft)).  Returns (emitted, accepted, stopped);
    rows after the end are never settled."""
    emitted, accepted, stopped = [], 0, False
    for index in range(len(draft) + 1):
        token, stop = pick_at(index)
        emitted.append(int(token))
        matches = index < len(draft) and int(draft[index]) == int(token)
        if matches:
            accepted += 1
        if stop:
            stopped = True
            break
        if not matches:
            break
    return emitted, accepted, stopped


def point_mass_verify(rows_logits, draft, uniforms, stop_ids=(), **rule):
    """The walk over rows settled by the row sampler (sample_row with the
    row's uniform: uniform_ahead(i), crates/app/cli/src/qwen_forward.rs:
    283-292, as the device verify reads it).  Returns (emitted, accepted,
    stopped, statuses of the settled rows)."""
    stops = set(int(t) for t in stop_ids)
    statuses = []

    def pick_at(i):
        r = sample_row(rows_logits[i], uniform=float(uniforms[i]), **rule)
        statuses.append(r["status"])
        return r["token"], r["token"] in stops

    emitted, accepted, stopped = accept_and_roll_back(draft, pick_at)
    return emitted, accepted, stopped, statuses


class SplitMix64:
    """SplitMix64 (the reference tests' Rng, speculative/tests.rs:128-149)."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFFFFFFFFFF

    def next_u64(self) -> int:
        m = 0xFFFFFFFFFFFFFFFF
        self.state = (self.state + 0x9E3779B97F4A7C15) & m
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)

    def uniform(self) -> float:
        return (self.next_u64() >> 11) / float(1 << 53)
