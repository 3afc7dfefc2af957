"""Deterministic synthetic sampler inputs for the five benchmark configurations.

Every random quantity comes from SplitMix64 (the constants of the reference's
test RNG, crates/core/engine/src/speculative/tests.rs:128-149) with master
seed 0x6D780000 + config and row stream seed master ^ (row * 0x9E3779B97F4A7C15).
Uniforms are (x >> 11) * 2^-53; normals are Box-Muller in f64 rounded to f32
(bf16 by round-to-nearest-even for config 3).  The same bytes feed the GPU
sampler and the CPU oracle.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
QWEN3_VOCAB = 151936
GEMMA_VOCAB = 262144


class Stream:
    """SplitMix64 stream: vectorised draws of consecutive outputs."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            steps = (np.arange(1, n + 1, dtype=np.uint64) * GOLDEN) + self.state
            self.state = steps[-1] if n else self.state
            z = steps
            z = (z ^ (z >> np.uint64(30))) * M1
            z = (z ^ (z >> np.uint64(27))) * M2
            return z ^ (z >> np.uint64(31))

    def uniform(self, n: int) -> np.ndarray:
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, n: int) -> np.ndarray:
        m = (n + 1) // 2
        u1 = self.uniform(m)
        u2 = self.uniform(m)
        r = np.sqrt(-2.0 * np.log1p(-u1))
        t = 2.0 * np.pi * u2
        return np.concatenate([r * np.cos(t), r * np.sin(t)])[:n] if n else np.zeros(0)

    def ints(self, n: int, hi: int) -> np.ndarray:
        return np.minimum((self.uniform(n) * hi).astype(np.int64), hi - 1)


def row_stream(cfg: int, row: int, salt: int = 0) -> Stream:
    master = (0x6D780000 + cfg + (salt << 32)) & 0xFFFFFFFFFFFFFFFF
    with np.errstate(over="ignore"):
        seed = int(np.uint64(master) ^ (np.uint64(row) * GOLDEN))
    return Stream(seed)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounding = np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))
    return ((b + rounding) >> np.uint64(16)).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << np.uint32(16)).view(np.float32)


@dataclass
class Batch:
    """One batch of sampler inputs (host numpy arrays)."""

    name: str
    logits: np.ndarray                     # f32 [rows, vocab] (bf16 configs: the widened values)
    temperature: np.ndarray                # f64 [rows]
    uniform: np.ndarray                    # f64 [rows]
    top_k: Optional[np.ndarray] = None     # u32
    top_p: Optional[np.ndarray] = None     # f64
    min_p: Optional[np.ndarray] = None     # f64
    repetition: Optional[np.ndarray] = None
    presence: Optional[np.ndarray] = None
    frequency: Optional[np.ndarray] = None
    history_offsets: Optional[np.ndarray] = None
    history_ids: Optional[np.ndarray] = None
    bias_offsets: Optional[np.ndarray] = None
    bias_ids: Optional[np.ndarray] = None
    bias_values: Optional[np.ndarray] = None
    mask_words: Optional[np.ndarray] = None  # u32 [rows, ceil(vocab/32)]
    tokenizer_vocab: int = 0
    bf16_bits: Optional[np.ndarray] = None   # u16 [rows, vocab] when the device input is bf16
    extra: Dict[str, np.ndarray] = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def input_bytes(self) -> int:
        """Compulsory bytes read by one sampling pass over this batch."""
        n = (self.bf16_bits.nbytes if self.bf16_bits is not None else self.logits.nbytes)
        for a in (self.history_ids, self.bias_ids, self.bias_values, self.mask_words):
            if a is not None:
                n += a.nbytes
        n += self.rows * (8 * 4 + 4 * 4)  # per-row parameters
        return n

    def output_bytes(self) -> int:
        return self.rows * (4 + 8 + 4)


def _peaks(s: Stream, logits_row: np.ndarray, count: int, lo: float, hi: float) -> None:
    ids = s.ints(count, logits_row.shape[0])
    amps = lo + (hi - lo) * s.uniform(count)
    for i, a in zip(ids, amps):
        logits_row[i] = np.float32(np.float64(logits_row[i]) + a)


def _zipf_table(V: int, s: float) -> np.ndarray:
    w = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    c = np.cumsum(w)
    return c / c[-1]


def _permutation(cfg: int, V: int) -> np.ndarray:
    keys = row_stream(cfg, 0, salt=7).u64(V)
    return np.argsort(keys, kind="stable").astype(np.uint32)


def config1(vocab: int = QWEN3_VOCAB, greedy: bool = False) -> Batch:
    """1 x V f32 N(0, 2^2) + 20 peaks +8.0; T 0.7, top_k 20, top_p 0.8,
    repetition 1.05 over 512 uniform history ids (or greedy)."""
    s = row_stream(1, 0)
    x = (2.0 * s.normal(vocab)).astype(np.float32)
    ids = s.ints(20, vocab)
    for i in ids:
        x[i] = np.float32(np.float64(x[i]) + 8.0)
    hist = s.ints(512, vocab).astype(np.uint32)
    u = s.uniform(1)
    return Batch(
        name="cfg1-greedy" if greedy else "cfg1", logits=x[None, :],
        temperature=np.array([0.0 if greedy else 0.7]), uniform=u,
        top_k=np.array([20], dtype=np.uint32), top_p=np.array([0.8]),
        repetition=np.array([1.05], dtype=np.float32),
        history_offsets=np.array([0, 512], dtype=np.uint32), history_ids=hist,
    )


def config2(rows: int = 64, vocab: int = QWEN3_VOCAB) -> Batch:
    """64 x V f32 N(0, 2^2) + 1..50 peaks of +4..+10 per row; T ~ U[0.3, 1.5],
    top_k {0, 20, 50, 1000}[row % 4], top_p ~ U[0.5, 1), min_p 0.05,
    presence 0.5 / frequency 0.3 / repetition 1.1 over 2048-id Zipf(1.1)
    histories (rank -> id by a seeded permutation)."""
    x = np.empty((rows, vocab), dtype=np.float32)
    T = np.empty(rows)
    tp = np.empty(rows)
    u = np.empty(rows)
    hist = np.empty((rows, 2048), dtype=np.uint32)
    zt = _zipf_table(vocab, 1.1)
    perm = _permutation(2, vocab)
    for r in range(rows):
        s = row_stream(2, r)
        x[r] = (2.0 * s.normal(vocab)).astype(np.float32)
        npk = 1 + int(s.ints(1, 50)[0])
        _peaks(s, x[r], npk, 4.0, 10.0)
        T[r] = 0.3 + 1.2 * s.uniform(1)[0]
        tp[r] = 0.5 + 0.5 * s.uniform(1)[0]
        ranks = np.searchsorted(zt, s.uniform(2048), side="right")
        hist[r] = perm[np.minimum(ranks, vocab - 1)]
        u[r] = s.uniform(1)[0]
    topk = np.array([[0, 20, 50, 1000][r % 4] for r in range(rows)], dtype=np.uint32)
    return Batch(
        name="cfg2", logits=x, temperature=T, uniform=u, top_k=topk, top_p=tp,
        min_p=np.full(rows, 0.05), repetition=np.full(rows, 1.1, dtype=np.float32),
        presence=np.full(rows, 0.5, dtype=np.float32), frequency=np.full(rows, 0.3, dtype=np.float32),
        history_offsets=(np.arange(rows + 1, dtype=np.uint32) * 2048), history_ids=hist.reshape(-1),
    )


def config3(rows: int = 32, vocab: int = QWEN3_VOCAB) -> Batch:
    """32 x V bf16 N(0, 2.5^2); per-row packed u32 mask allowing 0.5-5% of the
    vocabulary as runs of 1..64 tokens at random offsets (rows 0, 9, 18, 27:
    exactly one token); T 1.0, top_p 0.95, categorical draw."""
    words = (vocab + 31) // 32
    bits = np.empty((rows, vocab), dtype=np.uint16)
    mask = np.zeros((rows, words), dtype=np.uint32)
    u = np.empty(rows)
    for r in range(rows):
        s = row_stream(3, r)
        bits[r] = to_bf16_bits((2.5 * s.normal(vocab)).astype(np.float32))
        legal = np.zeros(vocab, dtype=bool)
        if r in (0, 9, 18, 27):
            legal[int(s.ints(1, vocab)[0])] = True
        else:
            frac = 0.005 + 0.045 * s.uniform(1)[0]
            target = int(frac * vocab)
            while legal.sum() < target:
                run = 1 + int(s.ints(1, 64)[0])
                start = int(s.ints(1, vocab)[0])
                legal[start:start + run] = True
        u[r] = s.uniform(1)[0]
        idx = np.nonzero(legal)[0]
        np.bitwise_or.at(mask[r], idx // 32, (np.uint32(1) << (idx % 32).astype(np.uint32)))
    return Batch(
        name="cfg3", logits=bf16_bits_to_f32(bits), temperature=np.ones(rows), uniform=u,
        top_p=np.full(rows, 0.95), mask_words=mask, tokenizer_vocab=vocab, bf16_bits=bits,
    )


def config4(rows: int = 256, vocab: int = GEMMA_VOCAB) -> Batch:
    """256 x 262144 f32 N(0, 3^2) + 100 peaks (+4..+10) per row; T 1.0,
    top_k 64, top_p 0.95; the top-20 logprobs are a separate call."""
    x = np.empty((rows, vocab), dtype=np.float32)
    u = np.empty(rows)
    for r in range(rows):
        s = row_stream(4, r)
        x[r] = (3.0 * s.normal(vocab)).astype(np.float32)
        _peaks(s, x[r], 100, 4.0, 10.0)
        u[r] = s.uniform(1)[0]
    return Batch(
        name="cfg4", logits=x, temperature=np.ones(rows), uniform=u,
        top_k=np.full(rows, 64, dtype=np.uint32), top_p=np.full(rows, 0.95),
    )


def config5(rows: int = 16, draft_len: int = 4, vocab: int = QWEN3_VOCAB) -> Dict[str, np.ndarray]:
    """Speculative verify: target [rows, draft_len+1, V] ~ N(0, 2^2) + 1..10
    peaks per position; draft = target[:, :draft_len] + N(0, 0.5^2); draft
    tokens drawn from softmax(draft) (T 1) with seeded uniforms; accept,
    resample and bonus uniforms."""
    tgt = np.empty((rows, draft_len + 1, vocab), dtype=np.float32)
    drf = np.empty((rows, draft_len, vocab), dtype=np.float32)
    toks = np.empty((rows, draft_len), dtype=np.int32)
    ua = np.empty((rows, draft_len))
    ur = np.empty((rows, draft_len))
    ub = np.empty(rows)
    for r in range(rows):
        s = row_stream(5, r)
        for j in range(draft_len + 1):
            tgt[r, j] = (2.0 * s.normal(vocab)).astype(np.float32)
            _peaks(s, tgt[r, j], 1 + int(s.ints(1, 10)[0]), 4.0, 10.0)
        for j in range(draft_len):
            drf[r, j] = (tgt[r, j].astype(np.float64) + 0.5 * s.normal(vocab)).astype(np.float32)
            q = np.exp(drf[r, j].astype(np.float64) - drf[r, j].max())
            cdf = np.cumsum(q)
            toks[r, j] = int(min(np.searchsorted(cdf, s.uniform(1)[0] * cdf[-1], side="right"), vocab - 1))
        ua[r] = s.uniform(draft_len)
        ur[r] = s.uniform(draft_len)
        ub[r] = s.uniform(1)[0]
    return dict(target=tgt, draft=drf, draft_tokens=toks, temperature=np.ones(rows),
                accept_u=ua, resample_u=ur, bonus_u=ub)
