"""Benchmark: sampled rows/s of the HIP token sampler on one MI355X.

Workload (the metric's configuration): B=64 rows x
V=151936 f32 logits drawn N(0, 2^2) with 1-50 peaks per row, per-row
temperature U[0.3, 1.5], top_k in {0, 20, 50, 1000}, top_p U[0.5, 1),
min_p 0.05, presence 0.5 / frequency 0.3 / repetition 1.1 over 2048-token
Zipf(1.1) histories, one seeded uniform per row.  One step = one full
pipeline pass (penalties + top-k + top-p + min-p + draw) over the batch.

Inputs are resident in HBM before timing starts.  The logits rotate over 8
copies (311 MB, more than the 256 MB Infinity Cache) so every step streams
its logits from HBM rather than from the cache.  The CPU baseline is the C
restatement of the reference sampler (oracle/) timed on this host on a
bounded sample of the same rows.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sampled rows/s at B=64,V=151936 fp32; achieved HBM GB/s vs MI355X peak"
HBM_PEAK_GBS = 8000.0
NBUF = 8


def algorithmic_bytes(b) -> int:
    """Compulsory bytes of one pass: inputs read once, required outputs written once."""
    n = b.logits.nbytes                                  # 38,895,616
    n += b.history_ids.nbytes + b.history_offsets.nbytes  # 524,288 + 260
    n += b.rows * (8 + 4 + 8 + 8 + 4 + 4 + 4 + 8)        # T, top_k, top_p, min_p, rep, pres, freq, u
    n += b.rows * (4 + 8 + 4)                            # token, sampling_logprob, status
    return n


def cpu_baseline(b, seconds: float):
    """Times the oracle (the reference sampler restated in C) on this host."""
    import numpy as np
    from oracle import oracle

    oracle.lib()
    rows_done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.sample_batch(b)
        rows_done += b.rows
    single = rows_done / (time.perf_counter() - t0)
    threads = max(1, min(16, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()))
    rows_mt, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        oracle.sample_batch_threads(b, threads)
        rows_mt += b.rows
    multi = rows_mt / (time.perf_counter() - t0)
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(single, 2), "unit": "rows/s", "cores": 1, "kind": "port",
        "sample": f"{rows_done} rows of the same cfg2 batch (1 thread, rows serial, {seconds:.0f} s)",
        "multi_thread": {"value": round(multi, 2), "cores": threads, "sample": f"{rows_mt} rows"},
        "cpu": cpu,
    }


def committed_traffic():
    p = ROOT / "profiles" / "sample_kernel_cfg2_traffic.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--race", action="store_true", help="also time race-v2 picks (mxs_sample_race)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain 256 MiB device copies (scales the FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
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
    b = synth.config2()
    logits, kw = to_device(torch, b)
    bufs = [logits] + [logits.clone() for _ in range(NBUF - 1)]
    stream = torch.cuda.Stream()
    s = Sampler(max_rows=b.rows, max_vocab=b.vocab, stream=stream)
    with torch.cuda.stream(stream):
        launch = s.launcher(bufs[0], **kw)
        out = launch.out
        for i in range(args.warmup):
            launch(bufs[i % NBUF])
    torch.cuda.synchronize()
    # Timed region: K back-to-back steps on the sampler's stream, bracketed by
    # events on that stream; a second pair per launch gives kernel durations.
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    t_begin = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        t_begin.record(stream)
        for i in range(args.steps):
            launch(bufs[i % NBUF])
        t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_begin.elapsed_time(t_end)
    # Kernel durations: a separate pass with events around each launch and
    # one the library records between its two kernels (the chunk pass,
    # sample_kernel, and the row finisher, finish_kernel).
    mids = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    with torch.cuda.stream(stream):
        for i in range(args.steps):
            mids[i].record(stream)   # creates the underlying hipEvent_t
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(args.steps):
            starts[i].record(stream)
            s.lib.mxs_debug_set_split_event(s.ctx, ctypes.c_void_p(mids[i].cuda_event))
            launch(bufs[i % NBUF])
            ends[i].record(stream)
    s.lib.mxs_debug_set_split_event(s.ctx, None)
    torch.cuda.synchronize()
    chunk = sorted(st.elapsed_time(md) for st, md in zip(starts, mids))
    fin = sorted(md.elapsed_time(en) for md, en in zip(mids, ends))
    per = sorted(st.elapsed_time(en) for st, en in zip(starts, ends))
    kern_ms = float(np.mean(chunk))
    status = out.status.cpu().numpy()
    assert (status >= 0).all(), f"row errors in the benchmark batch: {status}"

    ms_per_step = total_ms / args.steps
    rows_per_s = b.rows / (ms_per_step / 1e3)
    bytes_ = algorithmic_bytes(b)
    # the chunk pass streams every input byte: its rate against HBM peak
    achieved = bytes_ / (kern_ms / 1e3) / 1e9
    step_gbs = bytes_ / (ms_per_step / 1e3) / 1e9
    props = torch.cuda.get_device_properties(0)
    res = {
        "metric": METRIC,
        "value": round(rows_per_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 logits, f64 sampling math",
        "data": "synthetic (seeded SplitMix64, BASELINE config 2)",
        "config": {
            "workload": "cfg2: B=64 x V=151936 f32, penalties + top-k {0,20,50,1000} + top-p U[.5,1) + "
                        "min-p .05 + inverse-CDF draw; logits rotated over 8 HBM copies",
            "rows": b.rows, "vocab": b.vocab, "history": 2048,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": committed_traffic(),
            "kernel": "sample_kernel<float>",
            "algorithmic_bytes": bytes_,
            "kernel_ms_mean": round(kern_ms, 6),
            "kernel_ms_median": round(chunk[len(chunk) // 2], 6),
            "finish_kernel_ms_mean": round(float(np.mean(fin)), 6),
            "pipeline_ms_mean": round(float(np.mean(per)), 6),
            "pipeline_gbs": round(bytes_ / (float(np.mean(per)) / 1e3) / 1e9, 1),
            "step_gbs": round(step_gbs, 1),
            "device": props.name,
        },
    }
    if args.race:
        res["race"] = race_bench(torch, s, stream, bufs, kw, b, args.steps, args.warmup)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(b, args.cpu_seconds)
    else:
        res["cpu_baseline"] = None
    print(json.dumps(res), flush=True)


def race_bench(torch, s, stream, bufs, kw, b, steps, warmup):
    """race-v2 picks (mxs_sample_race) on the same resident config-2 logits:
    the batch's own rules (a kept set of 1 to ~600 tokens per row), and every
    row a whole-row race (top_k 0, top_p 1, min_p 0: the race kernel scores
    all V tokens).  Time per call, back to back, from events on the stream."""
    import numpy as np

    from metallix_amd import synth

    st = synth.Stream(0x72616365)
    dev = bufs[0].device
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
                launch(bufs[i % NBUF])
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for i in range(steps):
                launch(bufs[i % NBUF])
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
