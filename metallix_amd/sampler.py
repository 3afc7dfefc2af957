"""ctypes binding of libmx_sampler.so (include/mx_sampler.h).

`Sampler` mirrors the reference's device-pick plugin: one handle owns the
kernels and scratch (mlx_kernels::MetalKernel, crates/metal/mlx-kernels/src/
lib.rs:203-215); `sample` queues a batched pick on the stream like
Qwen3TokenPicks::start_with (crates/models/qwen/src/forward/picks.rs:279-381)
and returns device tensors the caller reads back after synchronising, the
Qwen3TokenPicks::wait step (picks.rs:390-401).  Per-row statuses mirror
engine::sampling::SamplingError (crates/core/engine/src/sampling.rs:19-43).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libmx_sampler.so"

MXS_F32 = 0
MXS_BF16 = 1

ROW_STATUS = {
    0: "ok",
    1: "uncertified",
    -1: "EmptyLogits",
    -2: "MaskLengthMismatch",
    -3: "EmptySupport",
    -4: "InvalidTemperature",
    -5: "InvalidUniform",
    -6: "NonFiniteLogit",
    -7: "VocabularyTooLarge",
    -8: "InvalidTopP",
    -9: "InvalidMinP",
    -10: "InvalidPenalty",
    -11: "InvalidHistory",
    -12: "InvalidBias",
    -13: "TokenOutOfRange",
    -14: "Probabilities",
    -15: "UnsupportedRule",   # mxs_finish_tiles: a rule other than greedy or top-k
}

_vp = ctypes.c_void_p


class MxsBatch(ctypes.Structure):
    _fields_ = [
        ("logits", _vp), ("dtype", ctypes.c_int32), ("rows", ctypes.c_uint32),
        ("vocab", ctypes.c_uint32), ("row_stride", ctypes.c_uint64),
        ("temperature", _vp), ("top_k", _vp), ("top_p", _vp), ("min_p", _vp),
        ("repetition", _vp), ("presence", _vp), ("frequency", _vp), ("uniform", _vp),
        ("history_offsets", _vp), ("history_ids", _vp),
        ("bias_offsets", _vp), ("bias_ids", _vp), ("bias_values", _vp),
        ("mask_words", _vp), ("mask_stride", ctypes.c_uint64),
        ("tokenizer_vocab", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
    ]


class MxsOut(ctypes.Structure):
    _fields_ = [
        ("token", _vp), ("sampling_logprob", _vp), ("status", _vp),
        ("kept_count", _vp), ("adjusted", _vp), ("kept_bits", _vp),
    ]


class MxsRace(ctypes.Structure):
    _fields_ = [("seed", _vp), ("choice", _vp), ("position", _vp)]


class MxsReceipts(ctypes.Structure):
    _fields_ = [
        ("top", _vp), ("n", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
        ("ids", _vp), ("logprobs", _vp), ("token_logprob", _vp), ("status", _vp),
    ]


# Exported symbols and their prototypes, as declared in include/mx_sampler.h.
PROTOTYPES = {
    "mxs_abi_version": (ctypes.c_int, []),
    "mxs_status_string": (ctypes.c_char_p, [ctypes.c_int32]),
    "mxs_create": (ctypes.c_int, [ctypes.c_int, _vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(_vp)]),
    "mxs_destroy": (ctypes.c_int, [_vp]),
    "mxs_set_stream": (ctypes.c_int, [_vp, _vp]),
    "mxs_sample": (ctypes.c_int, [_vp, ctypes.POINTER(MxsBatch), ctypes.POINTER(MxsOut)]),
    "mxs_sample_race": (ctypes.c_int, [_vp, ctypes.POINTER(MxsBatch), ctypes.POINTER(MxsRace),
                                       ctypes.POINTER(MxsOut)]),
    "mxs_logsoftmax_topn": (ctypes.c_int, [_vp, _vp, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                           ctypes.c_uint64, ctypes.c_uint32, _vp, _vp, _vp, _vp, _vp]),
    "mxs_logsoftmax_topn_noalloc": (ctypes.c_int, [_vp, _vp, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                                   ctypes.c_uint64, ctypes.c_uint32, _vp, _vp, _vp, _vp, _vp]),
    "mxs_spec_verify": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "mxs_step": (ctypes.c_int, [_vp, ctypes.POINTER(MxsBatch), ctypes.POINTER(MxsRace), ctypes.POINTER(MxsOut),
                                ctypes.POINTER(MxsReceipts)]),
    "mxs_mask_host": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_uint64)]),
    "mxs_mask_upload": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(_vp)]),
    "mxs_sync": (ctypes.c_int, [_vp]),
    "mxs_export_candidates": (ctypes.c_int, [_vp, ctypes.c_uint32, ctypes.c_uint32, _vp, _vp, _vp]),
    "mxs_lmhead_bf16": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _vp,
                                       ctypes.c_uint64, _vp]),
    "mxs_finish_tiles": (ctypes.c_int, [_vp, ctypes.POINTER(MxsBatch), _vp, ctypes.POINTER(MxsOut)]),
    "mxs_debug_set_timing": (ctypes.c_int, [_vp, _vp]),
    "mxs_debug_floor": (ctypes.c_int, [_vp, _vp, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                       ctypes.c_uint32, _vp, _vp]),
    "mxs_debug_set_paths": (ctypes.c_int, [_vp, _vp]),
    "mxs_last_error": (ctypes.c_char_p, [_vp]),
}

_LIB = None


class SamplerError(RuntimeError):
    pass


ABI_VERSION = 2                 # MXS_ABI_VERSION of include/mx_sampler.h
RECEIPT_NONE = 0xFFFFFFFF       # MXS_RECEIPT_NONE: a receipt_top entry for "no receipt"
TILE_TOKENS = 256               # MXS_TILE_TOKENS: vocabulary entries per epilogue-statistics tile
TILE_STAT_BYTES = 8             # MXS_TILE_STAT_BYTES: bytes per (row, tile)


def load_library(path: Optional[Path] = None):
    """Loads the built library; raises when it is missing (no fallback)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise SamplerError(f"{p} is not built: run `python -m metallix_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mxs_abi_version() != ABI_VERSION:
        raise SamplerError(f"{p} implements ABI {lib.mxs_abi_version()}, these bindings ABI {ABI_VERSION}: rebuild")
    if path is None:
        _LIB = lib
    return lib


def with_suppression(rows: int, suppress_ids, bias_offsets=None, bias_ids=None, bias_values=None, *,
                     vocab: Optional[int] = None):
    """Host-side CSR for the sampler's bias stage with the checkpoint's
    suppressed tokens merged in (ChatFormat::suppress,
    crates/core/chat-format/src/lib.rs:761-780): every row gets a -inf entry
    for each id of `suppress_ids` (ids are per checkpoint, the same for every
    row), which the sampler turns into an adjusted logit of f32::MIN.  A
    suppressed id keeps no bias of its own.  An id at or past `vocab` (the
    logit row's length) is skipped, as the reference's `logits.get_mut`
    returns None for it (:771-778); without `vocab` every id is kept, and the
    sampler reports one past the row as an invalid bias entry.  Returns
    numpy (offsets u32[rows + 1], ids u32, values f32), ids strictly
    increasing within a row."""
    import numpy as np

    sup = np.unique(np.asarray(suppress_ids, dtype=np.int64))
    if vocab is not None:
        sup = sup[(sup >= 0) & (sup < int(vocab))]
    sup = sup.astype(np.uint32)
    offs, ids, vals = [0], [], []
    for r in range(rows):
        if bias_offsets is not None:
            b0, b1 = int(bias_offsets[r]), int(bias_offsets[r + 1])
            bi = np.asarray(bias_ids[b0:b1], dtype=np.uint32)
            bv = np.asarray(bias_values[b0:b1], dtype=np.float32)
            keep = ~np.isin(bi, sup)
            bi, bv = bi[keep], bv[keep]
        else:
            bi, bv = np.zeros(0, np.uint32), np.zeros(0, np.float32)
        ri = np.concatenate([bi, sup])
        rv = np.concatenate([bv, np.full(sup.size, -np.inf, dtype=np.float32)])
        order = np.argsort(ri, kind="stable")
        ids.append(ri[order])
        vals.append(rv[order])
        offs.append(offs[-1] + ri.size)
    return (np.asarray(offs, dtype=np.uint32), np.concatenate(ids).astype(np.uint32),
            np.concatenate(vals).astype(np.float32))


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


class DeviceWords:
    """A staging slot's device mask words, as `Sampler.sample(mask=...)`
    takes them (a data pointer and a row stride in words)."""

    def __init__(self, ptr: int, stride: int, rows: int):
        self.ptr, self.stride_words, self.rows = ptr, stride, rows

    def data_ptr(self) -> int:
        return self.ptr

    def stride(self, dim: int) -> int:
        assert dim == 0
        return self.stride_words


@dataclass
class ReceiptResult:
    """Device tensors of one step's receipts (mxs_receipts)."""
    ids: "object"
    logprobs: "object"
    token_logprob: "object"
    status: "object"


@dataclass
class SampleResult:
    token: "object"
    sampling_logprob: "object"
    status: "object"
    kept_count: "object"
    adjusted: "object" = None
    kept_bits: "object" = None


class Sampler:
    """One sampler context on one GPU and stream (not thread-safe)."""

    def __init__(self, max_rows: int, max_vocab: int, device: int = 0, stream=None):
        import torch

        if not torch.cuda.is_available():
            raise SamplerError("no GPU visible: the HIP sampler has no CPU path")
        self.torch = torch
        self.lib = load_library()
        self.device = device
        self.stream = stream if stream is not None else torch.cuda.current_stream(device)
        ctx = _vp()
        rc = self.lib.mxs_create(device, _vp(self.stream.cuda_stream), max_rows, max_vocab, ctypes.byref(ctx))
        if rc != 0:
            raise SamplerError(f"mxs_create failed: {rc}")
        self.ctx = ctx
        self.max_rows = max_rows
        self.max_vocab = max_vocab

    def close(self):
        if getattr(self, "ctx", None):
            self.lib.mxs_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str):
        if rc != 0:
            msg = self.lib.mxs_last_error(self.ctx)
            raise SamplerError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")

    def sample(self, logits, temperature, *, top_k=None, top_p=None, min_p=None, repetition=None,
               presence=None, frequency=None, uniform=None, history=None, bias=None, mask=None,
               tokenizer_vocab=None, debug: bool = False, out: Optional[SampleResult] = None,
               vocab: Optional[int] = None, race=None) -> SampleResult:
        """Queues one batched pick.  All tensor arguments live on the GPU.

        history: (offsets u32[rows+1], ids u32) CSR; bias: (offsets, ids, values f32);
        mask: u32[rows, mask_stride].
        race: (seed u64 as int64[rows], choice u32[rows] or None, position u32[rows])
        selects race-v2 (Qwen3Selection::Race, picks.rs:40-66) instead of the
        inverse-CDF draw; `uniform` is then unused.
        """
        b, o, r, out = self._structs(logits, temperature, top_k=top_k, top_p=top_p, min_p=min_p,
                                     repetition=repetition, presence=presence, frequency=frequency, uniform=uniform,
                                     history=history, bias=bias, mask=mask, tokenizer_vocab=tokenizer_vocab,
                                     debug=debug, out=out, vocab=vocab, race=race)
        if r is not None:
            self._check(self.lib.mxs_sample_race(self.ctx, ctypes.byref(b), ctypes.byref(r), ctypes.byref(o)),
                        "mxs_sample_race")
            self._keep = (b, o, r)
            return out
        self._check(self.lib.mxs_sample(self.ctx, ctypes.byref(b), ctypes.byref(o)), "mxs_sample")
        self._keep = (b, o)
        return out

    def lmhead(self, hidden, weight, *, stats: bool = False, logits=None):
        """Queues the bf16 lm_head GEMM (mxs_lmhead_bf16): hidden bf16[rows,
        hidden_dim], weight bf16[vocab, hidden_dim] on the device; returns
        (logits f32[rows, vocab], tile statistics u8[rows, ceil(vocab/256)
        * TILE_STAT_BYTES] or None).  With stats the epilogue also writes the statistics
        finish_tiles reads."""
        torch = self.torch
        rows, K = hidden.shape
        V = weight.shape[0]
        dev = hidden.device
        with torch.cuda.stream(self.stream):
            if logits is None:
                logits = torch.empty((rows, V), dtype=torch.float32, device=dev)
            st = (torch.empty((rows, -(-V // TILE_TOKENS) * TILE_STAT_BYTES), dtype=torch.uint8, device=dev)
                  if stats else None)
        self._check(self.lib.mxs_lmhead_bf16(self.ctx, hidden.data_ptr(), weight.data_ptr(), rows, K, V,
                                             logits.data_ptr(), logits.stride(0), _ptr(st)), "mxs_lmhead_bf16")
        return logits, st

    def finish_tiles(self, logits, tile_stats, temperature, *, top_k=None, top_p=None, min_p=None, uniform=None,
                     debug: bool = False, out: Optional[SampleResult] = None) -> SampleResult:
        """Queues the finish-only pick (mxs_finish_tiles) over the lm_head's
        logits and tile statistics: greedy and top-k rows, as `sample`
        picks them (no penalties, bias or mask)."""
        rows, V = logits.shape
        need = rows * -(-V // TILE_TOKENS) * TILE_STAT_BYTES
        if tile_stats.device != logits.device or tile_stats.numel() * tile_stats.element_size() < need:
            raise ValueError(f"tile_stats must hold {need} bytes on the logits' device")
        b, o, _, out = self._structs(logits, temperature, top_k=top_k, top_p=top_p, min_p=min_p, uniform=uniform,
                                     debug=debug, out=out)
        o.adjusted = None
        out.adjusted = None
        self._check(self.lib.mxs_finish_tiles(self.ctx, ctypes.byref(b), tile_stats.data_ptr(), ctypes.byref(o)),
                    "mxs_finish_tiles")
        self._keep = (b, o)
        return out

    def lmhead_launcher(self, hidden, weight, logits, tile_stats=None):
        """Pre-built lmhead for repeated calls into the same logits (and tile
        statistics): returns f() that re-issues mxs_lmhead_bf16."""
        rows, K = hidden.shape
        V = weight.shape[0]
        fn = self.lib.mxs_lmhead_bf16
        args = (self.ctx, hidden.data_ptr(), weight.data_ptr(), rows, K, V, logits.data_ptr(), logits.stride(0),
                _ptr(tile_stats))

        def launch():
            rc = fn(*args)
            if rc != 0:
                self._check(rc, "mxs_lmhead_bf16")

        return launch

    def finish_launcher(self, logits, tile_stats, temperature, **rule):
        """Pre-built finish_tiles for repeated calls over the same logits and
        tile statistics with the same rules and outputs: returns f() that
        re-issues mxs_finish_tiles (f.out holds the outputs)."""
        out = self.finish_tiles(logits, tile_stats, temperature, **rule)
        b, o = self._keep
        bp, op, sp = ctypes.byref(b), ctypes.byref(o), tile_stats.data_ptr()
        fn, ctx = self.lib.mxs_finish_tiles, self.ctx

        def launch():
            rc = fn(ctx, bp, sp, op)
            if rc != 0:
                self._check(rc, "mxs_finish_tiles")

        launch.out = out
        launch.keep = (b, o)
        return launch

    def step(self, logits, temperature, *, receipt_top=None, n: int = 28, race=None, **kw):
        """Queues one engine step (mxs_step): every row's pick as `sample`
        does, then the receipts over the suppressed logits (the bias
        entries of -inf) of the rows whose receipt_top entry (u32[rows] on
        the device; None: every row) is not RECEIPT_NONE, with n IDs per
        row (an entry of 0 still gets the picked token's log probability).
        Returns (SampleResult, ReceiptResult) of device tensors."""
        torch = self.torch
        b, o, r, out = self._structs(logits, temperature, race=race, **kw)
        rows, dev = logits.shape[0], logits.device
        with torch.cuda.stream(self.stream):   # the fills run before the step on its stream
            rec = ReceiptResult(
                ids=torch.full((rows, n), -1, dtype=torch.int32, device=dev),
                logprobs=torch.full((rows, n), float("nan"), dtype=torch.float64, device=dev),
                token_logprob=torch.full((rows,), float("nan"), dtype=torch.float64, device=dev),
                status=torch.zeros(rows, dtype=torch.int32, device=dev),
            )
        R = MxsReceipts()
        R.top = _ptr(receipt_top)
        R.n = n
        R.ids, R.logprobs = rec.ids.data_ptr(), rec.logprobs.data_ptr()
        R.token_logprob, R.status = rec.token_logprob.data_ptr(), rec.status.data_ptr()
        rp = ctypes.byref(r) if r is not None else None
        self._check(self.lib.mxs_step(self.ctx, ctypes.byref(b), rp, ctypes.byref(o), ctypes.byref(R)), "mxs_step")
        self._keep = (b, o, r, R)
        return out, rec

    def step_launcher(self, logits, *, receipt_top=None, n: int = 28, **kw):
        """Pre-built mxs_step for repeated steps with the same rules and
        outputs: returns f(logits) that only swaps the logits pointer (its
        .out and .receipts hold the device outputs)."""
        out, rec = self.step(logits, receipt_top=receipt_top, n=n, **kw)
        b, o, r, R = self._keep
        bp, op, Rp = ctypes.byref(b), ctypes.byref(o), ctypes.byref(R)
        rp = ctypes.byref(r) if r is not None else None
        ctx, fs = self.ctx, self.lib.mxs_step

        def launch(t):
            b.logits = t.data_ptr()
            rc = fs(ctx, bp, rp, op, Rp)
            if rc != 0:
                self._check(rc, "mxs_step")

        launch.out, launch.receipts = out, rec
        return launch

    def _structs(self, logits, temperature, *, top_k=None, top_p=None, min_p=None, repetition=None,
                 presence=None, frequency=None, uniform=None, history=None, bias=None, mask=None,
                 tokenizer_vocab=None, debug: bool = False, out: Optional[SampleResult] = None,
                 vocab: Optional[int] = None, race=None):
        torch = self.torch
        rows = logits.shape[0]
        V = vocab if vocab is not None else logits.shape[1]
        dev = logits.device
        if out is None:
            out = SampleResult(
                token=torch.empty(rows, dtype=torch.int32, device=dev),
                sampling_logprob=torch.empty(rows, dtype=torch.float64, device=dev),
                status=torch.empty(rows, dtype=torch.int32, device=dev),
                kept_count=torch.empty(rows, dtype=torch.int32, device=dev),
            )
            if debug:
                out.adjusted = torch.empty((rows, V), dtype=torch.float32, device=dev)
                out.kept_bits = torch.empty((rows, (V + 31) // 32), dtype=torch.int32, device=dev)
        b = MxsBatch()
        b.logits = logits.data_ptr()
        b.dtype = MXS_BF16 if logits.dtype == torch.bfloat16 else MXS_F32
        b.rows = rows
        b.vocab = V
        b.row_stride = logits.stride(0)
        b.temperature = _ptr(temperature)
        b.top_k = _ptr(top_k)
        b.top_p = _ptr(top_p)
        b.min_p = _ptr(min_p)
        b.repetition = _ptr(repetition)
        b.presence = _ptr(presence)
        b.frequency = _ptr(frequency)
        b.uniform = _ptr(uniform)
        if history is not None:
            b.history_offsets, b.history_ids = _ptr(history[0]), _ptr(history[1])
        if bias is not None:
            b.bias_offsets, b.bias_ids, b.bias_values = _ptr(bias[0]), _ptr(bias[1]), _ptr(bias[2])
        if mask is not None:
            b.mask_words = mask.data_ptr()
            b.mask_stride = mask.stride(0)
            b.tokenizer_vocab = V if tokenizer_vocab is None else tokenizer_vocab
        o = MxsOut()
        o.token = out.token.data_ptr()
        o.sampling_logprob = _ptr(out.sampling_logprob)
        o.status = out.status.data_ptr()
        o.kept_count = _ptr(out.kept_count)
        o.adjusted = _ptr(out.adjusted)
        o.kept_bits = _ptr(out.kept_bits)
        r = None
        if race is not None:
            r = MxsRace()
            r.seed, r.choice, r.position = _ptr(race[0]), _ptr(race[1]), _ptr(race[2])
        return b, o, r, out

    def launcher(self, logits, **kw):
        """Pre-built launch for repeated picks with the same parameters and
        outputs: returns f(logits) that only swaps the logits pointer."""
        out = self.sample(logits, **kw)
        keep = self._keep
        b, o = keep[:2]
        bp, op = ctypes.byref(b), ctypes.byref(o)
        ctx = self.ctx
        if len(keep) == 3:   # race-v2
            rp, fr = ctypes.byref(keep[2]), self.lib.mxs_sample_race
            fn, what = (lambda: fr(ctx, bp, rp, op)), "mxs_sample_race"
        else:
            fs = self.lib.mxs_sample
            fn, what = (lambda: fs(ctx, bp, op)), "mxs_sample"

        def launch(t):
            b.logits = t.data_ptr()
            rc = fn()
            if rc != 0:
                self._check(rc, what)

        launch.out = out
        return launch

    def verify_point_mass(self, logits, draft, temperature, uniform, *, stop_ids=(), **rule):
        """Point-mass speculative verification on device picks (A9): the
        walk of accept_and_roll_back (crates/core/engine/src/speculative.rs:
        318-347, as accept_verified exposes it for device picks) over S
        sequences of K + 1 scored positions.  `logits` [S * (K + 1), V] on
        the device, sequence-major; `draft` host ints [S, K]; `temperature`,
        `uniform` and the other rule tensors of `sample` are per row (row i
        of a sequence carries uniform_ahead(i), crates/app/cli/src/
        qwen_forward.rs:283-292).  Every row is picked in one mxs_sample
        call; on the host each sequence keeps picks in order until one
        leaves the draft, is a stop token, or is the bonus row.  Returns, per
        sequence, dict(emitted, accepted, stopped, status): status is 0, or
        the first non-zero row status among the settled rows (1: the host
        settles that row, as TokenPicker does, chat_turn.rs:348-358)."""
        import numpy as np

        draft = np.asarray(draft)
        S, K = draft.shape
        assert logits.shape[0] == S * (K + 1), "logits rows must be S * (K + 1)"
        out = self.sample(logits, temperature, uniform=uniform, **rule)
        self.sync()
        tok = out.token.cpu().numpy().reshape(S, K + 1)
        st = out.status.cpu().numpy().reshape(S, K + 1)
        stops = set(int(t) for t in stop_ids)
        res = []
        for s_ in range(S):
            emitted, accepted, stopped, status = [], 0, False, 0
            for i in range(K + 1):
                if status == 0 and st[s_, i] != 0:
                    status = int(st[s_, i])
                t = int(tok[s_, i])
                emitted.append(t)
                matches = i < K and int(draft[s_, i]) == t
                accepted += int(matches)
                if t in stops:
                    stopped = True
                    break
                if not matches:
                    break
            res.append(dict(emitted=emitted, accepted=accepted, stopped=stopped, status=status))
        return res

    def logsoftmax_topn(self, logits, n: int, *, vocab: Optional[int] = None):
        """Queues the T=1 log-softmax of every row with its n most likely IDs
        (token_logprob, crates/app/cli/src/chat_turn.rs:506-563).  Returns
        device tensors (ids i32[rows, n], logprobs f64[rows, n], maximum
        f64[rows], log_normalizer f64[rows], status i32[rows])."""
        torch = self.torch
        rows = logits.shape[0]
        V = vocab if vocab is not None else logits.shape[1]
        dev = logits.device
        ids = torch.empty((rows, max(n, 1)), dtype=torch.int32, device=dev)
        lps = torch.empty((rows, max(n, 1)), dtype=torch.float64, device=dev)
        mx = torch.empty(rows, dtype=torch.float64, device=dev)
        ln = torch.empty(rows, dtype=torch.float64, device=dev)
        st = torch.empty(rows, dtype=torch.int32, device=dev)
        dtype = MXS_BF16 if logits.dtype == torch.bfloat16 else MXS_F32
        rc = self.lib.mxs_logsoftmax_topn(self.ctx, logits.data_ptr(), dtype, rows, V, logits.stride(0), n,
                                          ids.data_ptr(), lps.data_ptr(), mx.data_ptr(), ln.data_ptr(),
                                          st.data_ptr())
        self._check(rc, "mxs_logsoftmax_topn")
        return ids[:, :n], lps[:, :n], mx, ln, st

    def spec_verify(self, target, draft, draft_tokens, temperature, accept_uniform, resample_uniform,
                    bonus_uniform):
        """Queues speculative verification (accept_or_resample position by
        position, crates/core/engine/src/speculative.rs:369-444; the bonus
        draw past an accepted draft).  target f32[rows, K+1, V], draft
        f32[rows, K, V], draft_tokens i32[rows, K], temperature f64[rows],
        accept/resample f64[rows, K], bonus f64[rows].  Returns device tensors
        (out_tokens i32[rows, K+1], count, accepted, status i32[rows])."""
        torch = self.torch
        rows, k1, V = target.shape
        K = k1 - 1
        dev = target.device
        out = torch.empty((rows, k1), dtype=torch.int32, device=dev)
        cnt = torch.empty(rows, dtype=torch.int32, device=dev)
        acc = torch.empty(rows, dtype=torch.int32, device=dev)
        st = torch.empty(rows, dtype=torch.int32, device=dev)
        rc = self.lib.mxs_spec_verify(self.ctx, target.data_ptr(), _ptr(draft) if K else None, rows, K, V,
                                      _ptr(draft_tokens) if K else None, temperature.data_ptr(),
                                      _ptr(accept_uniform) if K else None, _ptr(resample_uniform) if K else None,
                                      bonus_uniform.data_ptr(), out.data_ptr(), cnt.data_ptr(), acc.data_ptr(),
                                      st.data_ptr())
        self._check(rc, "mxs_spec_verify")
        return out, cnt, acc, st

    def export_candidates(self, rows: int, width: int):
        """Queues mxs_export_candidates for the first `rows` rows of the last
        pick on this context: returns device tensors (count i32[rows], ids
        i32[rows, width], logits f32[rows, width]); count -1 marks a row with
        no candidate list, otherwise the first count entries are the row's
        candidates (its top `width` when it had more) in token-ID order."""
        torch = self.torch
        dev = torch.device("cuda", self.device)
        count = torch.empty(rows, dtype=torch.int32, device=dev)
        ids = torch.empty((rows, width), dtype=torch.int32, device=dev)
        logits = torch.empty((rows, width), dtype=torch.float32, device=dev)
        self._check(self.lib.mxs_export_candidates(self.ctx, rows, width, count.data_ptr(), ids.data_ptr(),
                                                   logits.data_ptr()), "mxs_export_candidates")
        return count, ids, logits

    def spec_launcher(self, target, draft, draft_tokens, temperature, accept_uniform, resample_uniform,
                      bonus_uniform):
        """Pre-built spec_verify for repeated calls with the same per-row
        inputs and outputs: returns f(target, draft) that only swaps the two
        logits pointers (f.out holds spec_verify's output tensors)."""
        out = self.spec_verify(target, draft, draft_tokens, temperature, accept_uniform, resample_uniform,
                               bonus_uniform)
        rows, k1, V = target.shape
        K = k1 - 1
        fn, ctx = self.lib.mxs_spec_verify, self.ctx
        rest = (_ptr(draft_tokens) if K else None, temperature.data_ptr(),
                _ptr(accept_uniform) if K else None, _ptr(resample_uniform) if K else None,
                bonus_uniform.data_ptr(), *(t.data_ptr() for t in out))

        def launch(tgt, drf):
            rc = fn(ctx, tgt.data_ptr(), drf.data_ptr() if K else None, rows, K, V, *rest)
            if rc != 0:
                self._check(rc, "mxs_spec_verify")

        launch.out = out
        return launch

    def mask_host(self, slot: int):
        """The pinned host words of staging slot `slot` as a numpy u32 array
        [max_rows, stride] (mxs_mask_host: returns once the slot's previous
        upload has read them, so the caller may overwrite them)."""
        import numpy as np

        ptr, stride = _vp(), ctypes.c_uint64()
        self._check(self.lib.mxs_mask_host(self.ctx, slot, ctypes.byref(ptr), ctypes.byref(stride)), "mxs_mask_host")
        self._mask_stride = stride.value
        n = self.max_rows * stride.value
        buf = (ctypes.c_uint32 * n).from_address(ptr.value)
        return np.frombuffer(buf, dtype=np.uint32).reshape(self.max_rows, stride.value)

    def mask_upload(self, slot: int, rows: int) -> DeviceWords:
        """Queues the upload of the slot's first `rows` rows (mxs_mask_upload);
        returns the device words for `sample(mask=...)`."""
        ptr = _vp()
        self._check(self.lib.mxs_mask_upload(self.ctx, slot, rows, ctypes.byref(ptr)), "mxs_mask_upload")
        return DeviceWords(ptr.value, self._mask_stride, rows)

    def sync(self):
        self._check(self.lib.mxs_sync(self.ctx), "mxs_sync")
