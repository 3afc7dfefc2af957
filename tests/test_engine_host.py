"""Host side of the batched engine step (metallix_amd.engine), no GPU: the
batch packing and the receipt bookkeeping the reference keeps per row
(TurnLoop::receipt_wanted and token_logprob's spelling filter,
crates/app/cli/src/chat_turn.rs:413-418, 506-563)."""
import numpy as np

from metallix_amd.engine import RowRequest, pack_rows, settle_receipt
from metallix_amd.sampler import RECEIPT_NONE, with_suppression


def test_pack_rows_csr_and_suppression():
    reqs = [RowRequest(temperature=0.7, top_k=20, history=[5, 9, 5], bias={7: 1.5, 3: -2.0}, top_logprobs=5),
            RowRequest(),
            RowRequest(temperature=1.0, top_p=0.9, history=[1], bias={11: 0.25}, uniform=0.5)]
    h = pack_rows(reqs, vocab=100, suppress_ids=[11, 50, 100, 4000])   # IDs past the row are skipped
    assert h["temperature"].tolist() == [0.7, 0.0, 1.0]
    assert h["top_k"].tolist() == [20, 0, 0]
    hoff, hids = h["history"]
    assert hoff.tolist() == [0, 3, 3, 4] and hids.tolist() == [5, 9, 5, 1]
    boff, bids, bvals = h["bias"]
    # per row: ids strictly increasing; suppressed ids as -inf, replacing a row's own bias
    assert boff.tolist() == [0, 4, 6, 8]
    assert bids[0:4].tolist() == [3, 7, 11, 50] and bvals[0:4].tolist() == [-2.0, 1.5, -np.inf, -np.inf]
    assert bids[4:6].tolist() == [11, 50] and np.all(np.isneginf(bvals[4:6]))
    assert bids[6:8].tolist() == [11, 50] and np.all(np.isneginf(bvals[6:8]))
    assert h["receipt_top"].tolist() == [5, RECEIPT_NONE, RECEIPT_NONE]
    assert h["mask"] is None


def test_pack_rows_mask_rows_default_to_all_legal():
    words = (70 + 31) // 32
    m = np.zeros(words, dtype=np.uint32)
    m[0] = 0b1010
    h = pack_rows([RowRequest(mask=m), RowRequest()], vocab=70)
    assert h["mask"].shape == (2, words)
    assert h["mask"][0].tolist() == m.tolist()
    assert np.all(h["mask"][1] == 0xFFFFFFFF)
    assert h["history"] is None and h["bias"] is None


def test_receipt_sizes_none_and_zero():
    # None: no receipt; 0: a receipt of the token's log probability alone
    # (logprobs: true without top_logprobs is Some(0), chat_completions.rs:241-243)
    h = pack_rows([RowRequest(top_logprobs=None), RowRequest(top_logprobs=0), RowRequest(top_logprobs=3)], vocab=10)
    assert h["receipt_top"].tolist() == [RECEIPT_NONE, 0, 3]
    ids = np.array([4, 2, 7], dtype=np.int32)
    r = settle_receipt(2, ids, np.array([-0.1, -2.0, -3.0]), -2.0, 0)
    assert r is not None and r.top == [] and r.logprob == -2.0 and r.token == 2


def test_suppression_skips_ids_past_the_row():
    # ChatFormat::suppress writes only the IDs inside the row
    # (logits.get_mut(index) is None past it, chat-format/src/lib.rs:771-778)
    offs, ids, vals = with_suppression(2, [3, 9, 10, 70000], vocab=10)
    assert offs.tolist() == [0, 2, 4] and ids.tolist() == [3, 9, 3, 9] and np.all(np.isneginf(vals))
    offs, ids, _ = with_suppression(1, [3, 10])   # no vocabulary given: every ID kept (the sampler rejects 10)
    assert ids.tolist() == [3, 10]


def test_pack_rows_masks_stop_at_the_tokenizer_vocabulary():
    # fill_legal_mask never marks an ID at or past the tokenizer's vocabulary
    # legal (constraint.rs:793-806); rows without a mask keep every ID
    V, words = 100, 4
    m = np.full(words, 0xFFFFFFFF, dtype=np.uint32)
    h = pack_rows([RowRequest(mask=m), RowRequest()], vocab=V, tokenizer_vocab=70)
    assert h["mask"][0].tolist() == [0xFFFFFFFF, 0xFFFFFFFF, 0x3F, 0]
    assert np.all(h["mask"][1] == 0xFFFFFFFF)
    h = pack_rows([RowRequest(mask=m)], vocab=V, tokenizer_vocab=64)
    assert h["mask"][0].tolist() == [0xFFFFFFFF, 0xFFFFFFFF, 0, 0]


def test_settle_receipt_follows_the_reference_bookkeeping():
    ids = np.array([9, 120, 4, 130, 7, 1, 2, 3, 5, 6, 8, 10, 11], dtype=np.int32)
    lps = -np.arange(ids.size, dtype=np.float64) - 0.5
    # no receipt asked, or a stop token: none (receipt_wanted)
    assert settle_receipt(9, ids, lps, -0.5, None) is None
    assert settle_receipt(9, ids, lps, -0.5, 3, stop_ids=[9]) is None
    # the over-selected head (top + 8) minus unspellable IDs, first `top` kept
    r = settle_receipt(4, ids, lps, -2.5, 3, spellable=lambda i: i < 100)
    assert r.logprob == -2.5
    assert r.top == [(9, -0.5), (4, -2.5), (7, -4.5)]
    # the head is top + 8 long: entries past it never fill in for dropped ones
    r = settle_receipt(4, ids, lps, -2.5, 3, spellable=lambda i: i in (9, 11))
    assert r.top == [(9, -0.5)]
