"""Benchmark: sampled rows/s of the HIP token sampler on one MI355X.

Default workload (the metric's configuration):
B=64 rows x V=151936 f32 logits drawn N(0, 2^2) with 1-50 peaks per row,
per-row temperature U[0.3, 1.5], top_k in {0, 20, 50, 1000}, top_p U[0.5, 1),
min_p 0.05, presence 0.5 / frequency 0.3 / repetition 1.1 over 2048-token
Zipf(1.1) histories, one seeded uniform per row.  One step = one full
pipeline pass (penalties + top-k + top-p + min-p + draw) over the batch: one
mxs_sample call, which is one kernel launch (sample_kernel).

`--config N` times the other configurations of BASELINE.json instead
(1: one Qwen3 row, stochastic; 3: 32 bf16 rows under grammar masks; 4:
256 x 262144 f32 rows, a pick plus the top-20 log-softmax per row; 5:
speculative verification of 16 rows with 4 drafted tokens each).

Inputs are resident in HBM before timing starts.  The logits rotate over
enough copies (at least 300 MB, more than the 256 MB Infinity Cache) that
every step streams its logits from HBM rather than from the cache.  The CPU
baseline is the C restatement of the reference sampler (oracle/) timed on
this host on a bounded sample of the same rows.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sampled rows/s at B=64,V=151936 fp32; achieved HBM GB/s vs MI355X peak"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 300 << 20
OUT_BYTES_PER_ROW = 4 + 8 + 4 + 4       # token, sampling_logprob, status, kept_count
TOPN = 28                               # the top 20 logprobs plus the reference's 8 spares (chat_turn.rs:506-563)


def nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def sample_bytes(logits, kw) -> int:
    """Compulsory bytes of one mxs_sample call: the V logits of every row
    and every per-row input read once, the outputs written once."""
    rows, V = logits.shape[0], kw["vocab"]
    n = rows * V * logits.element_size()
    for k, v in kw.items():
        if isinstance(v, tuple):
            n += sum(nbytes(t) for t in v)
        elif hasattr(v, "element_size"):
            n += nbytes(v)
    return n + rows * OUT_BYTES_PER_ROW


def topn_bytes(logits, V, n) -> int:
    """mxs_logsoftmax_topn: the logits once; ids i32 + logprobs f64 for n
    per row, maximum and log-normaliser f64, status i32."""
    rows = logits.shape[0]
    return rows * V * logits.element_size() + rows * (n * 12 + 8 + 8 + 4)


def spec_bytes(d) -> int:
    """mxs_spec_verify: target and draft logits once, the per-row inputs,
    the outputs (tokens [rows, K+1], count, accepted, status)."""
    rows, k1, _ = d["target"].shape
    n = nbytes(d["target"]) + nbytes(d["draft"]) + nbytes(d["draft_tokens"]) + nbytes(d["temperature"])
    n += nbytes(d["accept_u"]) + nbytes(d["resample_u"]) + nbytes(d["bonus_u"])
    return n + rows * k1 * 4 + rows * 12


def rotation(per_copy: int) -> int:
    return max(2, min(1024, -(-ROTATE_BYTES // max(per_copy, 1))))


class Call:
    """One API call of a step: `fn(i)` queues it on the sampler's stream
    against input copy i; `bytes_` are its algorithmic bytes."""

    def __init__(self, name, kernels, fn, bytes_):
        self.name, self.kernels, self.fn, self.bytes_ = name, kernels, fn, bytes_


def build_workload(cfg, torch, Sampler, synth, to_device):
    """Returns (description, rows per step, sampler, [Call], check(), batch
    or dict for the CPU baseline)."""
    if cfg == 5:
        d = synth.config5()
        rows, k1, V = d["target"].shape
        dev = "cuda"
        T = lambda a, dt=None: torch.from_numpy(a if dt is None else a.astype(dt)).to(dev)
        tgt0, drf0 = T(d["target"]), T(d["draft"])
        per = nbytes(tgt0) + nbytes(drf0)
        nb = rotation(per)
        tgts = [tgt0] + [tgt0.clone() for _ in range(nb - 1)]
        drfs = [drf0] + [drf0.clone() for _ in range(nb - 1)]
        dt = T(d["draft_tokens"])
        temp, ua, ur, ub = T(d["temperature"]), T(d["accept_u"]), T(d["resample_u"]), T(d["bonus_u"])
        stream = torch.cuda.Stream()
        s = Sampler(max_rows=rows, max_vocab=V, stream=stream)
        with torch.cuda.stream(stream):
            launch = s.spec_launcher(tgt0, drf0, dt, temp, ua, ur, ub)
        res = {"out": launch.out}

        def spec(i):
            launch(tgts[i % nb], drfs[i % nb])

        dd = dict(target=tgt0, draft=drf0, draft_tokens=dt, temperature=temp, accept_u=ua,
                  resample_u=ur, bonus_u=ub)
        calls = [Call("mxs_spec_verify", "spec_pass1<true> + spec_pass2<true>", spec, spec_bytes(dd))]

        def check():
            st = res["out"][3].cpu().numpy()
            assert (st >= 0).all(), f"row errors in the benchmark batch: {st}"
            return int((st == 1).sum())

        desc = (f"cfg5: speculative verify, {rows} rows x draft {k1 - 1} x V={V} f32 target + draft, "
                f"accept min(1,p/q), residual resample, bonus draw; inputs rotated over {nb} HBM copies")
        return desc, rows, s, calls, check, d, stream

    b = {1: synth.config1, 2: synth.config2, 3: synth.config3, 4: synth.config4}[cfg]()
    logits, kw = to_device(torch, b)
    nb = rotation(nbytes(logits))
    bufs = [logits] + [logits.clone() for _ in range(nb - 1)]
    stream = torch.cuda.Stream()
    s = Sampler(max_rows=b.rows, max_vocab=b.vocab, stream=stream)
    with torch.cuda.stream(stream):
        launch = s.launcher(bufs[0], **kw)
    calls = [Call("mxs_sample", "sample_kernel", lambda i: launch(bufs[i % nb]), sample_bytes(logits, kw))]
    res = {}
    if cfg == 1:   # config 1 also runs greedy (temperature 0) on the same logits
        gkw = dict(kw)
        gkw["temperature"] = torch.zeros_like(kw["temperature"])
        with torch.cuda.stream(stream):
            glaunch = s.launcher(bufs[0], **gkw)
        calls.append(Call("mxs_sample greedy", "sample_kernel", lambda i: glaunch(bufs[i % nb]),
                          sample_bytes(logits, gkw)))
        res["greedy"] = glaunch
    if cfg == 4:
        def topn(i):
            res["topn"] = s.logsoftmax_topn(bufs[i % nb], TOPN, vocab=b.vocab)

        calls.append(Call("mxs_logsoftmax_topn", "topn_kernel + topn_merge_kernel", topn,
                          topn_bytes(logits, b.vocab, TOPN)))

    def check():
        st = launch.out.status.cpu().numpy()
        assert (st >= 0).all(), f"row errors in the benchmark batch: {st}"
        unc = int((st == 1).sum())
        if "greedy" in res:
            g = res["greedy"].out.status.cpu().numpy()
            assert (g == 0).all(), f"greedy row errors: {g}"
        if "topn" in res:
            t = res["topn"][4].cpu().numpy()
            assert (t >= 0).all(), f"row errors in the top-n batch: {t}"
        return unc

    descs = {
        1: "cfg1: 1 x V=151936 f32, T 0.7, top_k 20, top_p 0.8, repetition 1.05 over 512 ids, inverse-CDF draw",
        2: "cfg2: B=64 x V=151936 f32, penalties + top-k {0,20,50,1000} + top-p U[.5,1) + min-p .05 + "
           "inverse-CDF draw",
        3: "cfg3: 32 x V=151936 bf16, packed u32 grammar masks (0.5-5% legal), T 1, top_p .95, draw",
        4: "cfg4: 256 x V=262144 f32, T 1, top_k 64, top_p .95, draw; plus log-softmax top-20 per row",
    }
    desc = descs[cfg] + f"; logits rotated over {nb} HBM copies"
    return desc, b.rows, s, calls, check, b, stream


def cpu_baseline(cfg, data, seconds: float):
    """Times the oracle (the reference sampler restated in C) on this host."""
    import numpy as np
    from oracle import oracle

    oracle.lib()

    if cfg == 5:
        def one_pass():
            d = data
            for r in range(d["target"].shape[0]):
                oracle.spec_verify_row(d["target"][r], d["draft"][r], d["draft_tokens"][r], float(d["temperature"][r]),
                                       d["accept_u"][r], d["resample_u"][r], float(d["bonus_u"][r]))
            return d["target"].shape[0]
    elif cfg == 4:
        def one_pass():
            b = data
            rows = range(0, 8)
            oracle.sample_batch(b, rows=rows)
            for r in rows:
                oracle.token_logprob_top(b.logits[r], TOPN)
            return len(rows)
    else:
        def one_pass():
            oracle.sample_batch(data)
            return data.rows

    rows_done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        rows_done += one_pass()
    single = rows_done / (time.perf_counter() - t0)
    out = {
        "value": round(single, 2), "unit": "rows/s", "cores": 1, "kind": "port",
        "sample": f"{rows_done} rows of the same cfg{cfg} inputs (1 thread, rows serial, {seconds:.0f} s)",
    }
    if cfg in (2, 3):
        # Rows partitioned over host threads.  The GPU box gives one GPU's
        # job a 16-core share of the host, whatever nproc reports, so the
        # pool stops at 16; nproc is reported beside it.
        nproc = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
        threads = max(1, min(16, nproc))
        rows_mt, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < seconds / 2:
            oracle.sample_batch_threads(data, threads)
            rows_mt += data.rows
        out["multi_thread"] = {"value": round(rows_mt / (time.perf_counter() - t0), 2), "cores": threads,
                               "nproc": nproc, "sample": f"{rows_mt} rows"}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                out["cpu"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return out


def committed_traffic(cfg):
    """HBM bytes per dispatch from the committed counter summary (FETCH_SIZE
    and WRITE_SIZE passes scaled by a plain copy's readings)."""
    p = ROOT / "profiles" / "hbm_traffic.json"
    try:
        return json.loads(p.read_text()).get(f"cfg{cfg}", {})
    except Exception:
        return {}


def time_steps(torch, stream, calls, steps, warmup):
    """Back-to-back steps bracketed by events on the sampler's stream; then,
    for each call of the step, K back-to-back calls of that call alone, also
    bracketed by events on that stream (its mean launch duration: with one
    kernel per call the GPU runs that kernel back to back)."""
    def timed(fns):
        t_begin = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            t_begin.record(stream)
            for i in range(steps):
                for f in fns:
                    f(i)
            t_end.record(stream)
        torch.cuda.synchronize()
        return t_begin.elapsed_time(t_end) / steps

    with torch.cuda.stream(stream):
        for i in range(warmup):
            for c in calls:
                c.fn(i)
    ms_per_step = timed([c.fn for c in calls])
    per_call = [ms_per_step] if len(calls) == 1 else [timed([c.fn]) for c in calls]
    return ms_per_step, per_call


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=(1, 2, 3, 4, 5),
                    help="BASELINE.json configuration to time (2 = the metric's)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--race", action="store_true", help="also time race-v2 picks (mxs_sample_race, config 2)")
    ap.add_argument("--masks", action="store_true",
                    help="also time config-3 steps whose masks are uploaded from pinned staging each step")
    ap.add_argument("--receipts", action="store_true",
                    help="also time engine steps with top-20 receipts for every row (mxs_step, config 2)")
    ap.add_argument("--stream-floor", action="store_true",
                    help="also time mxs_sample's launch floor and stream floor (its grid, workgroup size and LDS; "
                         "configs 1-4) and account for one call's time from the workgroups' entry and exit stamps")
    ap.add_argument("--lmhead", action="store_true",
                    help="also time the lm_head GEMM + mxs_sample against the GEMM with tile statistics + "
                         "mxs_finish_tiles (config 2)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain 256 MiB device copies (scales the FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = 256 << 20
        src = torch.empty(n // 4, dtype=torch.float32, device="cuda").uniform_()
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n, "bytes_written": n, "launches": 10}), flush=True)
        return

    from metallix_amd import Sampler, synth

    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import to_device

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    cfg = args.config
    desc, rows, s, calls, check, data, stream = build_workload(cfg, torch, Sampler, synth, to_device)
    ms_per_step, per_call = time_steps(torch, stream, calls, args.steps, args.warmup)
    uncertified = check()

    traffic = committed_traffic(cfg)
    kernels = []
    for c, mean_ms in zip(calls, per_call):
        gbs = c.bytes_ / (mean_ms / 1e3) / 1e9
        kernels.append({
            "call": c.name, "kernels": c.kernels, "algorithmic_bytes": c.bytes_,
            "ms_mean": round(mean_ms, 6),
            "achieved_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic.get(c.name),
        })
    dom = max(kernels, key=lambda k: k["ms_mean"])
    step_bytes = sum(c.bytes_ for c in calls)
    props = torch.cuda.get_device_properties(0)
    res = {
        "metric": METRIC if cfg == 2 else f"sampled rows/s, config {cfg}; achieved HBM GB/s vs MI355X peak",
        "value": round(rows / (ms_per_step / 1e3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16" if cfg == 3 else "f32") + " logits, f64 sampling math",
        "data": f"synthetic (seeded SplitMix64, BASELINE config {cfg})",
        "config": {"workload": desc, "rows": rows},
        "roofline": {
            "bound": "hbm",
            "achieved": dom["achieved_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": dom["frac"],
            "traffic": dom["traffic"],
            "kernel": dom["kernels"],
            "algorithmic_bytes": dom["algorithmic_bytes"],
            "kernel_ms_mean": dom["ms_mean"],
            "step_gbs": round(step_bytes / (ms_per_step / 1e3) / 1e9, 1),
            "step_frac": round(step_bytes / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "device": props.name,
        },
        "calls": kernels,
        "uncertified_rows": uncertified,
    }
    if args.race and cfg == 2:
        res["race"] = race_bench(torch, s, stream, data, args.steps, args.warmup)
    if args.masks and cfg == 3:
        res["mask_upload"] = mask_bench(torch, s, stream, data, args.steps, args.warmup)
    if args.receipts and cfg == 2:
        res["engine_step"] = step_bench(torch, s, stream, data, args.steps, args.warmup,
                                        None if args.no_cpu else args.cpu_seconds)
    if args.lmhead and cfg == 2:
        res["lmhead"] = lmhead_bench(torch, s, stream, args.steps, args.warmup)
    if args.stream_floor and cfg in (1, 2, 3, 4):
        res["floors"] = floor_bench(torch, s, stream, data, args.steps, args.warmup)
    res["cpu_baseline"] = None if args.no_cpu else cpu_baseline(cfg, data, args.cpu_seconds)
    print(json.dumps(res), flush=True)


def floor_bench(torch, s, stream, b, steps, warmup):
    """What bounds one mxs_sample call, on resident logits rotated as in the
    main timing:
    - launch_floor: a kernel of mxs_sample's grid, workgroup size and LDS per
      workgroup whose workgroups exit at once;
    - stream_floor: the same launch, each workgroup reading its chunk of the
      logits once (all loads issued up front) and writing the maximum;
    - sample: mxs_sample itself;
    each back to back, from events on the stream.  Then `accounting`: single
    calls (the queue kept busy before each, so the events bracket the kernel
    alone), medians over 12 calls of the event-timed duration and of the
    workgroups' wall-clock stamps (100 MHz, relative to the first
    workgroup's first instruction): the last workgroup's entry, the last
    chunk body's start, the last exit of a chunk workgroup that does not
    finish its row, the last finisher's end and the last exit.
    The difference between the event time and the last exit is the launch's
    dispatch and completion overhead."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import to_device

    logits, kw = to_device(torch, b)
    nb = rotation(nbytes(logits))
    bufs = [logits] + [logits.clone() for _ in range(nb - 1)]
    dev = logits.device
    rows, V = logits.shape
    dt = 0 if logits.dtype == torch.float32 else 1     # MXS_F32, MXS_BF16
    out = torch.empty(rows * 64, dtype=torch.float32, device=dev)
    fst = torch.zeros(rows * 64 * 2, dtype=torch.int64, device=dev)

    def floor(mode):
        def f(i):
            rc = s.lib.mxs_debug_floor(s.ctx, bufs[i % nb].data_ptr(), dt, rows, V, V, mode, out.data_ptr(),
                                       fst.data_ptr() if mode == 2 else None)
            assert rc == 0, s.lib.mxs_last_error(s.ctx)
        return f

    with torch.cuda.stream(stream):
        launch = s.launcher(bufs[0], **kw)
    res = {}
    for name, fn in (("launch_floor", floor(0)), ("stream_floor", floor(1)), ("sample", lambda i: launch(bufs[i % nb]))):
        with torch.cuda.stream(stream):
            for i in range(warmup):
                fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for i in range(steps):
                fn(i)
            e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        res[name] = {"us_per_launch": round(ms * 1e3, 3), "logits_gbs": round(nbytes(logits) / (ms / 1e3) / 1e9, 1)}
    # the stream floor read every logit: its chunk maxima make the row maxima
    floor(1)(0)
    torch.cuda.synchronize()
    C = int(out.view(rows, 64).isfinite().sum(dim=1).max().item())
    got = out.view(rows, 64)[:, :C].max(dim=1).values
    assert torch.equal(got, bufs[0].float().max(dim=1).values), "stream floor maxima differ from torch.max"

    # the stream floor's own span: first entry to last exit, one call at a time
    spans = []
    for it in range(12):
        fst.zero_()
        floor(1)(it + 1)
        floor(2)(it)
        torch.cuda.synchronize()
        f = fst.view(rows, 64, 2).cpu().numpy().astype(np.float64)
        ok = f[..., 0] > 0
        spans.append([(f[..., 1][ok].max() - f[..., 0][ok].min()) / 100.0,
                      (f[..., 0][ok].max() - f[..., 0][ok].min()) / 100.0])
    sp = np.median(np.array(spans), axis=0)
    res["stream_floor"]["span_us"] = round(sp[0], 2)
    res["stream_floor"]["last_entry_us"] = round(sp[1], 2)

    SL, TS = 65, 16
    tb = torch.zeros(rows * SL * TS, dtype=torch.int64, device=dev)
    s.lib.mxs_debug_set_timing(s.ctx, tb.data_ptr())
    acc = []
    try:
        for it in range(12):
            tb.zero_()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                for j in range(8):      # keeps the queue busy while the host queues the timed call
                    floor(1)(j + 1)
                e0.record(stream)
                launch(bufs[0])
                e1.record(stream)
            torch.cuda.synchronize()
            t = tb.view(rows, SL, TS).cpu().numpy().astype(np.float64)
            ent = t[:, :SL - 1, 8]
            t0 = ent[ent > 0].min()
            rel = lambda a: (a[a > 0] - t0) / 100.0     # µs
            ce, fe = rel(t[:, :SL - 1, 9]), rel(t[:, SL - 1, 9])
            acc.append([e0.elapsed_time(e1) * 1e3, rel(ent).max(), rel(t[:, :SL - 1, 0]).max(),
                        ce.max() if ce.size else 0.0, rel(t[:, SL - 1, 7]).max(), max(ce.max() if ce.size else 0.0,
                                                                                      fe.max())])
    finally:
        s.lib.mxs_debug_set_timing(s.ctx, None)
    m = np.median(np.array(acc), axis=0)
    res["accounting_us"] = {
        "event_duration": round(m[0], 2), "last_workgroup_entry": round(m[1], 2),
        "last_chunk_body_start": round(m[2], 2), "last_chunk_exit": round(m[3], 2),
        "last_finisher_end": round(m[4], 2), "last_exit": round(m[5], 2),
        "dispatch_and_completion": round(m[0] - m[5], 2),
    }
    return res


def step_bench(torch, s, stream, b, steps, warmup, cpu_seconds):
    """Engine steps (mxs_step) on resident config-2 logits: every row's pick
    plus a top-20 receipt (28 ranked IDs, the reference's top + 8) for every
    row, over the logits with two suppressed IDs.  Time per step, back to
    back, from events on the stream; beside it the reference's per-row host
    loop (the oracle's pick and token_logprob per row) on a bounded sample."""
    import numpy as np

    from metallix_amd.sampler import with_suppression

    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import to_device, u32

    sup = [151643, 151645]
    saved = (b.bias_offsets, b.bias_ids, b.bias_values)
    b.bias_offsets, b.bias_ids, b.bias_values = with_suppression(b.rows, sup, *saved, vocab=b.vocab)
    logits, kw = to_device(torch, b)
    b.bias_offsets, b.bias_ids, b.bias_values = saved
    nb = rotation(nbytes(logits))
    bufs = [logits] + [logits.clone() for _ in range(nb - 1)]
    tops = torch.from_numpy(u32(np.full(b.rows, 20, dtype=np.uint32))).to(logits.device)
    with torch.cuda.stream(stream):
        launch = s.step_launcher(bufs[0], receipt_top=tops, n=TOPN, **kw)
        for i in range(warmup):
            launch(bufs[i % nb])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for i in range(steps):
            launch(bufs[i % nb])
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    st = launch.out.status.cpu().numpy()
    rst = launch.receipts.status.cpu().numpy()
    assert (st >= 0).all() and (rst == 0).all(), f"row errors in the step benchmark: {st} {rst}"
    res = {"ms_per_step": round(ms, 6), "rows_per_s": round(b.rows / (ms / 1e3), 1),
           "receipt_top": 20, "ranked_ids": TOPN, "suppressed_ids": sup,
           # one read of the logits (the receipts come from the pick's pass) and
           # the receipts' outputs
           "algorithmic_bytes": sample_bytes(logits, kw) + b.rows * (TOPN * (4 + 8) + 8 + 4)}
    if cpu_seconds:
        from oracle import oracle

        x = np.asarray(b.logits, dtype=np.float32)
        rows_done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds / 2:
            for r in range(0, 8):
                oracle.sample_row(x[r], temperature=float(b.temperature[r]), top_p=float(b.top_p[r]),
                                  min_p=float(b.min_p[r]), uniform=float(b.uniform[r]), top_k=int(b.top_k[r]),
                                  repetition=float(b.repetition[r]), presence=float(b.presence[r]),
                                  frequency=float(b.frequency[r]),
                                  history=b.history_ids[b.history_offsets[r]:b.history_offsets[r + 1]],
                                  bias_ids=sup, bias_values=[-np.inf] * len(sup))
                xs = x[r].copy()
                xs[sup] = np.finfo(np.float32).min
                oracle.token_logprob_top(xs, TOPN)
                rows_done += 1
        res["cpu_per_row_loop"] = {"value": round(rows_done / (time.perf_counter() - t0), 2), "unit": "rows/s",
                                   "cores": 1, "kind": "port",
                                   "sample": f"{rows_done} rows (rows 0-7 of cfg2, pick + token_logprob each)"}
    return res


def mask_bench(torch, s, stream, b, steps, warmup):
    """Config-3 steps whose grammar masks come from the host each step: the
    rows' words sit in the two pinned staging slots (where a constraint
    engine would write them), and every step re-stages its slot
    (mxs_mask_host, which waits for that slot's previous upload), uploads it
    on the copy stream (mxs_mask_upload) and picks under it; slots
    alternate, so step n + 1's upload overlaps step n's pick.  Time per
    step, back to back, from events on the sampler's stream, beside the
    same picks over device-resident masks."""
    import ctypes

    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import to_device

    from metallix_amd.sampler import DeviceWords

    logits, kw = to_device(torch, b)
    nb = rotation(nbytes(logits))
    bufs = [logits] + [logits.clone() for _ in range(nb - 1)]
    words = b.mask_words.shape[1]
    launches = []
    with torch.cuda.stream(stream):
        for slot in (0, 1):
            host = s.mask_host(slot)
            host[:] = 0
            host[:b.rows, :words] = b.mask_words
            dev = s.mask_upload(slot, b.rows)
            kws = dict(kw)
            kws["mask"] = DeviceWords(dev.data_ptr(), dev.stride(0), b.rows)
            launches.append(s.launcher(bufs[0], **kws))
    lib, ctx = s.lib, s.ctx
    hp, hs, dp = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_void_p()

    def step(i):
        slot = i & 1
        if lib.mxs_mask_host(ctx, slot, ctypes.byref(hp), ctypes.byref(hs)) != 0:
            raise RuntimeError("mxs_mask_host failed")
        if lib.mxs_mask_upload(ctx, slot, b.rows, ctypes.byref(dp)) != 0:
            raise RuntimeError("mxs_mask_upload failed")
        launches[slot](bufs[i % nb])

    with torch.cuda.stream(stream):
        for i in range(warmup):
            step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        e0.record(stream)
        for i in range(steps):
            step(i)
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    st = launches[(steps - 1) & 1].out.status.cpu().numpy()
    assert (st >= 0).all(), f"row errors in the mask benchmark: {st}"
    mbytes = b.rows * hs.value * 4
    return {"ms_per_step": round(ms, 6), "rows_per_s": round(b.rows / (ms / 1e3), 1),
            "upload_bytes_per_step": mbytes, "upload_gbs": round(mbytes / (ms / 1e3) / 1e9, 2)}


def lmhead_bench(torch, s, stream, steps, warmup):
    """The lm_head epilogue fusion on a Qwen3-0.6B-shaped head (hidden 1024,
    V 151936, 64 rows; bf16 hidden states and weights, seeded, the 311 MB of
    weights larger than the 256 MB Infinity Cache so every GEMM streams them
    from HBM): the GEMM writing f32 logits, then mxs_sample over them, beside
    the GEMM whose epilogue also writes tile statistics, then
    mxs_finish_tiles.  Rules: the greedy and top-k rows the finish-only
    pick serves, with a head small enough that the tile maxima prune the
    read (a quarter greedy, the rest top_k in {20, 50, 100} at T U[0.3,
    1.5], top_p U[0.5, 1), min_p 0.05 on a quarter of the rows), one seeded
    uniform per row.  Time per step and per call, back to back, from events
    on the stream."""
    import numpy as np

    from metallix_amd.sampler import TILE_STAT_BYTES, TILE_TOKENS

    R, K, V = 64, 1024, 151936
    g = torch.Generator(device="cuda").manual_seed(20261202)
    with torch.cuda.stream(stream):
        w = (torch.randn((V, K), generator=g, device="cuda") * (2.0 / K ** 0.5)).to(torch.bfloat16)
        h = torch.randn((R, K), generator=g, device="cuda").to(torch.bfloat16)
        logits = torch.empty((R, V), dtype=torch.float32, device="cuda")
        stats = torch.empty((R, -(-V // TILE_TOKENS) * TILE_STAT_BYTES), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    rng = np.random.default_rng(20261202)
    T = rng.uniform(0.3, 1.5, R)
    kk = np.array([(0, 20, 50, 100)[i % 4] for i in range(R)], dtype=np.uint32)
    T[kk == 0] = 0.0
    D = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    rule = dict(top_k=D(kk.view(np.int32)), top_p=D(rng.uniform(0.5, 1.0, R)),
                min_p=D(np.where(np.arange(R) % 4 == 1, 0.05, 0.0)), uniform=D(rng.random(R)))
    gemm = s.lmhead_launcher(h, w, logits)
    gemm_st = s.lmhead_launcher(h, w, logits, stats)
    with torch.cuda.stream(stream):
        gemm_st()
        fin = s.finish_launcher(logits, stats, D(T), **rule)
        samp = s.launcher(logits, temperature=D(T), **rule)
    torch.cuda.synchronize()

    def timed(fns):
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                for f in fns:
                    f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for _ in range(steps):
                for f in fns:
                    f()
            e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    sample_path = timed([gemm, lambda: samp(logits)])
    t_sample = samp.out.token.cpu().numpy().copy()
    s_sample = samp.out.status.cpu().numpy().copy()
    fused_path = timed([gemm_st, fin])
    t_fin, s_fin = fin.out.token.cpu().numpy(), fin.out.status.cpu().numpy()
    assert (s_fin >= 0).all() and (s_sample >= 0).all(), (s_fin, s_sample)
    both = (s_fin == 0) & (s_sample == 0)
    assert (t_fin[both] == t_sample[both]).all(), "the two paths picked different tokens"
    ms = {"gemm": timed([gemm]), "gemm_stats": timed([gemm_st]), "mxs_sample": timed([lambda: samp(logits)]),
          "mxs_finish_tiles": timed([fin])}
    gemm_bytes = V * K * 2 + R * K * 2 + R * V * 4
    stat_bytes = stats.numel()
    gbs = gemm_bytes / (ms["gemm"] / 1e3) / 1e9
    return {
        "workload": f"lm_head bf16 [{R} x {K}] x [{V} x {K}]^T -> f32 logits, then the pick",
        "gemm_plus_sample_ms": round(sample_path, 6),
        "gemm_plus_finish_ms": round(fused_path, 6),
        "rows_per_s_sample_path": round(R / (sample_path / 1e3), 1),
        "rows_per_s_fused_path": round(R / (fused_path / 1e3), 1),
        "call_ms": {k: round(v, 6) for k, v in ms.items()},
        "gemm_algorithmic_bytes": gemm_bytes,
        "gemm_achieved_gbs": round(gbs, 1),
        "gemm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "tile_stat_bytes": stat_bytes,
        "uncertified_rows": {"sample": int((s_sample == 1).sum()), "finish": int((s_fin == 1).sum())},
        "same_tokens_rows": int(both.sum()),
    }


def race_bench(torch, s, stream, b, steps, warmup):
    """race-v2 picks (mxs_sample_race) on resident config-2 logits: the
    batch's own rules (a kept set of 1 to ~600 tokens per row), and every row
    a whole-row race (top_k 0, top_p 1, min_p 0: the race kernel scores all V
    tokens).  Time per call, back to back, from events on the stream."""
    import numpy as np

    from metallix_amd import synth

    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import to_device

    logits, kw = to_device(torch, b)
    nb = rotation(nbytes(logits))
    bufs = [logits] + [logits.clone() for _ in range(nb - 1)]
    st = synth.Stream(0x72616365)
    dev = logits.device
    race = (torch.from_numpy(st.u64(b.rows).view(np.int64)).to(dev),
            None, torch.from_numpy(np.arange(b.rows, dtype=np.int32)).to(dev))
    whole = dict(kw)
    whole["top_k"] = torch.zeros_like(kw["top_k"])
    whole["top_p"] = torch.ones_like(kw["top_p"])
    whole["min_p"] = torch.zeros_like(kw["min_p"])
    res = {}
    for name, args_ in (("cfg2_rules", kw), ("whole_row", whole)):
        with torch.cuda.stream(stream):
            launch = s.launcher(bufs[0], race=race, **args_)
            for i in range(warmup):
                launch(bufs[i % nb])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for i in range(steps):
                launch(bufs[i % nb])
            e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        stat = launch.out.status.cpu().numpy()
        assert (stat >= 0).all(), f"row errors in the race benchmark: {stat}"
        res[name] = {"ms_per_step": round(ms, 6), "rows_per_s": round(b.rows / (ms / 1e3), 1),
                     "uncertified_rows": int((stat == 1).sum())}
    return res


if __name__ == "__main__":
    main()
