"""One decode step of a batch of sequences on one device call.

The reference's engine picks each sequence's next token in a host loop over
the batch (EngineLoop::decode_now, crates/app/cli/src/engine_loop.rs:
1080-1134): for every row, TurnLoop::pick (crates/app/cli/src/chat_turn.rs:
290-303) applies the checkpoint's suppression (ChatFormat::suppress,
crates/core/chat-format/src/lib.rs:761-780), picks under the sequence's
rule, and, when the turn asked for top_logprobs and the token is not a stop
token (receipt_wanted, chat_turn.rs:413-418), scores a receipt with
token_logprob (chat_turn.rs:506-563).  `EngineStep.run` does the same for
the whole batch with one `mxs_step`: the picks and the receipts are queued
together, read back once, and only the per-row bookkeeping (stop tokens,
the drop of unspellable IDs from the over-selected head) stays on the host.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping, Optional, Sequence

import numpy as np

from .sampler import RECEIPT_NONE, with_suppression

RECEIPT_OVERSELECT = 8   # token_logprob ranks top + 8 before dropping unspellable IDs (chat_turn.rs:527-530)


@dataclass
class RowRequest:
    """One sequence's rule for this step (SamplingPolicy plus the stages
    this sampler defines, and the turn's top_logprobs)."""
    temperature: float = 0.0            # 0: greedy
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    repetition: float = 1.0
    presence: float = 0.0
    frequency: float = 0.0
    history: Sequence[int] = ()
    bias: Mapping[int, float] = field(default_factory=dict)
    uniform: float = 0.0                # the draw's variate (unit_uniform of the turn's next u64)
    top_logprobs: Optional[int] = None  # receipt size; None: no receipt, 0: the token's logprob only
    mask: Optional[np.ndarray] = None   # u32 words over the logit row (SimpleVob layout), None: all legal


@dataclass
class Receipt:
    logprob: float                      # log probability of `token`
    top: list                           # [(id, logprob)], most likely first
    token: int = -1                     # the token `logprob` scores: the device's pick


@dataclass
class RowResult:
    """One row's pick.  A row with status 1 (uncertified) carries the
    device's token, which the caller may settle again on the host
    (chat_turn.rs:348-358); its receipt then still scores the device's token
    (`receipt.token`): the top list and the normalizer do not depend on the
    pick, so a caller that settles another token rescores only its logprob."""
    token: int
    status: int
    sampling_logprob: float
    receipt: Optional[Receipt]


def pack_rows(requests: Sequence[RowRequest], vocab: int, suppress_ids=(),
              tokenizer_vocab: Optional[int] = None) -> dict:
    """Host arrays of one step's batch: per-row rule arrays, the history
    and bias CSRs (the suppressed IDs merged in as -inf bias entries, which
    the sampler writes as f32::MIN; IDs past the row are skipped, as
    ChatFormat::suppress skips them), the receipt sizes (RECEIPT_NONE for
    rows without one), and the mask words when any row has one: all ones
    for rows without a mask, and in masked rows every ID at or past
    `tokenizer_vocab` cleared, as fill_legal_mask never marks them legal
    (crates/core/engine/src/constraint.rs:793-806)."""
    R = len(requests)
    f = lambda name, dt: np.array([getattr(q, name) for q in requests], dtype=dt)
    out = dict(temperature=f("temperature", np.float64), top_k=f("top_k", np.uint32),
               top_p=f("top_p", np.float64), min_p=f("min_p", np.float64),
               repetition=f("repetition", np.float32), presence=f("presence", np.float32),
               frequency=f("frequency", np.float32), uniform=f("uniform", np.float64))
    hoff = np.zeros(R + 1, dtype=np.uint32)
    for r, q in enumerate(requests):
        hoff[r + 1] = hoff[r] + len(q.history)
    hids = np.concatenate([np.asarray(q.history, dtype=np.uint32) for q in requests]) if hoff[-1] else None
    out["history"] = (hoff, hids) if hids is not None else None
    boff = np.zeros(R + 1, dtype=np.uint32)
    bids, bvals = [], []
    for r, q in enumerate(requests):
        items = sorted((int(k), float(v)) for k, v in q.bias.items())
        bids.append(np.array([k for k, _ in items], dtype=np.uint32))
        bvals.append(np.array([v for _, v in items], dtype=np.float32))
        boff[r + 1] = boff[r] + len(items)
    ids = np.concatenate(bids) if boff[-1] else np.zeros(0, np.uint32)
    vals = np.concatenate(bvals) if boff[-1] else np.zeros(0, np.float32)
    if len(suppress_ids):
        out["bias"] = with_suppression(R, suppress_ids, boff, ids, vals, vocab=vocab)
    elif boff[-1]:
        out["bias"] = (boff, ids, vals)
    else:
        out["bias"] = None
    out["receipt_top"] = np.array([RECEIPT_NONE if q.top_logprobs is None else int(q.top_logprobs)
                                   for q in requests], dtype=np.uint32)
    if any(q.mask is not None for q in requests):
        words = (vocab + 31) // 32
        m = np.full((R, words), 0xFFFFFFFF, dtype=np.uint32)
        for r, q in enumerate(requests):
            if q.mask is not None:
                w = np.asarray(q.mask, dtype=np.uint32)
                assert w.size == words, "a mask covers the logit row: ceil(vocab / 32) words"
                m[r] = w
                if tokenizer_vocab is not None and tokenizer_vocab < 32 * words:
                    tv = int(tokenizer_vocab)
                    m[r, tv // 32 + 1:] = 0
                    if tv % 32:
                        m[r, tv // 32] &= np.uint32((1 << (tv % 32)) - 1)
                    else:
                        m[r, tv // 32] = 0
        out["mask"] = m
    else:
        out["mask"] = None
    return out


def settle_receipt(token: int, ids, logprobs, token_logprob: float, top: Optional[int], stop_ids=(),
                   spellable=None) -> Optional[Receipt]:
    """The receipt the turn records for `token` (TurnLoop::accept,
    chat_turn.rs:420-433): none when the turn asked for none or the token
    is a stop token (receipt_wanted, :413-418); otherwise the over-selected
    head with IDs that have no spelling dropped (token_bytes fails past the
    tokenizer's vocabulary, :543-554), its first `top` entries (none for a
    top of 0: the token's log probability alone)."""
    if top is None or token in set(int(t) for t in stop_ids):
        return None
    head = []
    for i, lp in zip(np.asarray(ids)[: top + RECEIPT_OVERSELECT], np.asarray(logprobs)[: top + RECEIPT_OVERSELECT]):
        i = int(i)
        if i < 0 or (spellable is not None and not spellable(i)):
            continue
        head.append((i, float(lp)))
    return Receipt(logprob=float(token_logprob), top=head[:top], token=int(token))


class EngineStep:
    """Batched decode step over a Sampler: one mxs_step per call."""

    def __init__(self, sampler, *, suppress_ids=(), stop_ids=(), tokenizer_vocab: Optional[int] = None):
        self.sampler = sampler
        self.suppress_ids = tuple(int(t) for t in suppress_ids)
        self.stop_ids = tuple(int(t) for t in stop_ids)
        self.tokenizer_vocab = tokenizer_vocab

    def run(self, logits, requests: Sequence[RowRequest]) -> list:
        """Picks every row of `logits` (a device tensor [rows, >= vocab])
        under its request; returns one RowResult per row."""
        s = self.sampler
        torch = s.torch
        R, V = logits.shape[0], logits.shape[1]
        assert len(requests) == R
        h = pack_rows(requests, V, self.suppress_ids, self.tokenizer_vocab)
        dev = logits.device
        T = lambda a, dt: torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=dt))).to(dev)
        i32 = lambda a: T(np.asarray(a, dtype=np.uint32).view(np.int32), np.int32)
        kw = dict(temperature=T(h["temperature"], np.float64), uniform=T(h["uniform"], np.float64),
                  top_k=i32(h["top_k"]), top_p=T(h["top_p"], np.float64), min_p=T(h["min_p"], np.float64),
                  repetition=T(h["repetition"], np.float32), presence=T(h["presence"], np.float32),
                  frequency=T(h["frequency"], np.float32), vocab=V)
        if h["history"] is not None:
            kw["history"] = (i32(h["history"][0]), i32(h["history"][1]))
        if h["bias"] is not None:
            kw["bias"] = (i32(h["bias"][0]), i32(h["bias"][1]), T(h["bias"][2], np.float32))
        if h["mask"] is not None:
            kw["mask"] = i32(h["mask"])
            kw["tokenizer_vocab"] = V
        tops = h["receipt_top"]
        wanted = tops[tops != RECEIPT_NONE]
        n = int(min(64, max(1, (int(wanted.max()) if wanted.size else 0) + RECEIPT_OVERSELECT)))
        out, rec = s.step(logits, receipt_top=i32(tops), n=n, **kw)
        s.sync()
        tok, st = out.token.cpu().numpy(), out.status.cpu().numpy()
        slp = out.sampling_logprob.cpu().numpy()
        ids, lps, tlp = rec.ids.cpu().numpy(), rec.logprobs.cpu().numpy(), rec.token_logprob.cpu().numpy()
        tv = self.tokenizer_vocab
        spell = (lambda i: i < tv) if tv is not None else None
        res = []
        for r, q in enumerate(requests):
            receipt = None
            if st[r] >= 0 and q.top_logprobs is not None:
                receipt = settle_receipt(int(tok[r]), ids[r], lps[r], float(tlp[r]), q.top_logprobs, self.stop_ids,
                                         spell)
            res.append(RowResult(token=int(tok[r]), status=int(st[r]), sampling_logprob=float(slp[r]),
                                 receipt=receipt))
        return res
