"""Benchmark of the gfx950 sampling stage.

A step is one nerve_sampler_step over one batch of synthetic logits already
resident in HBM. The default workload is C5, the configuration the headline
metric is quoted on: B=256 rows x V=151936 bf16 logits (Student-t(4) * 2), a
2048-id history per row with repetition 1.1 / frequency 0.5 / presence 0.3,
top-k 50, top-p 0.9, per-row temperature in [0.5, 1.2] and a Philox draw.
Consecutive steps advance each row's stream tick on the device (reference
stream-control semantics), so K timed steps are K different draws with no host
work in between. Steps rotate over --buffers copies of the logits (4 x 78 MB
by default, more than the 256 MB memory-side cache), so every step reads its
logits from HBM.

Prints one JSON line: rows/s (whole job), us/step, the HBM roofline of the
sampling kernel (algorithmic bytes / device time per step from HIP events on
the launch stream, against 8 TB/s), the HBM traffic per launch measured by
rocprofv3 counters when a summary of them is present under profiles/, and the
CPU oracle timed on the host cores of the same machine on a bounded sample of
the same workload.

After the timed steps the last one is recomputed with the CPU oracle at the
same tick (same logits, history, seeds, Philox stream) and the bench fails on
any mismatch, so the path timed is the path checked. HBM traffic counters are
collected separately (llmoop_amd/traffic.py).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec + µs/step at B=256×V=151936; % of HBM roofline"
KERNEL = "sample_rows_kernel"
PROFILE_FILE = os.path.join(ROOT, "profiles", "sample_rows_kernel_{}_profile.md")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C5", help="C1..C5, C5P (C5 is the headline workload)")
    ap.add_argument("--buffers", type=int, default=4, help="logits copies the steps rotate over")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0, help="host threads of the CPU baseline (0: up to 16)")
    ap.add_argument("--slices", type=int, default=0, help="workgroups per row (0 = automatic)")
    ap.add_argument("--no-check", action="store_true", help="skip the oracle check of the last timed step")
    return ap.parse_args()


def cpu_baseline(w, budget_s: float, threads: int = 0) -> dict:
    """The oracle (a C restatement of the reference semantics, -O3, OpenMP
    over rows) on the host cores: as many full-batch steps as fit the budget."""
    from oracle import oracle

    threads = threads or min(os.cpu_count() or 1, 16)
    kw = dict(history=w.history, history_len=w.history_len, allowed=w.allowed, seeds=w.seeds)
    done_rows = 0
    t0 = time.perf_counter()
    step = 0
    while True:
        oracle.sample(w.logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, threads=threads,
                      steps=np.full(w.batch, step, np.uint64), **kw)
        done_rows += w.batch
        step += 1
        el = time.perf_counter() - t0
        if el >= budget_s or step >= 200:
            break
    return {
        "value": done_rows / el,
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{step} full {w.name} steps ({w.batch} rows x V={w.vocab}) in {el:.1f} s, "
                  f"OpenMP over rows, {threads} threads",
        "us_per_step": el / step * 1e6,
    }


def measured_traffic(workload: str):
    """Calibrated HBM bytes per launch from the committed counter summary of
    this workload, or None."""
    try:
        text = open(PROFILE_FILE.format(workload)).read()
    except OSError:
        return None
    if f"workload: {workload}" not in text:
        return None
    m = re.search(r"traffic_bytes_per_launch = (\d+)", text)
    return int(m.group(1)) if m else None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(rows are independent: B rows shard over GPUs with no exchange)", file=sys.stderr)
        sys.exit(2)
    import torch

    from llmoop_amd import sampler as S
    from llmoop_amd import workloads

    dev = torch.device("cuda:0")
    w = workloads.make(args.config, seed=2024, step=0)
    B, V = w.batch, w.vocab
    sampler = S.Sampler(V, B, dtype=w.dtype, top_k_capacity=w.top_k_capacity,
                        history_capacity=0 if w.history is None else w.history.shape[1],
                        slices_per_row=args.slices)

    def dev_arr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a)
        view = {np.uint32: np.int32, np.uint16: np.int16, np.uint64: np.int64}.get(a.dtype.type, a.dtype.type)
        return torch.from_numpy(a.view(view).copy()).to(dev)

    nbuf = max(1, args.buffers)
    logits0 = dev_arr(w.logits)
    logits = [logits0] + [logits0.clone() for _ in range(nbuf - 1)]
    params = S.params_tensor(w.params, dev)
    history = dev_arr(w.history)
    history_len = dev_arr(w.history_len)
    allowed = dev_arr(w.allowed)
    seeds = dev_arr(w.seeds)
    stream_control = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)

    def step(i):
        sampler.step(logits[i % nbuf], params, out, history=history, history_len=history_len, allowed=allowed,
                     seeds=seeds, rng=w.rng, eos_token_id=w.eos_token_id, stream_control=stream_control)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # K steps: wall clock on the host, device time from HIP events on the
    # launch stream (torch's current stream) around the same K launches
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        step(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    device_s = start.elapsed_time(end) / 1e3 / args.steps

    tick = stream_control[:, 1].cpu().numpy().view(np.uint32)
    if not (tick == args.warmup + args.steps).all():
        sys.exit("bench.py: stream ticks did not advance once per step")
    parity = None
    if not args.no_check:
        # the last timed step (tick warmup + steps - 1) recomputed by the oracle
        from oracle import oracle

        last = args.warmup + args.steps - 1
        ref = oracle.sample(w.logits, w.params, top_k_capacity=w.top_k_capacity, history=w.history,
                            history_len=w.history_len, allowed=w.allowed, seeds=w.seeds,
                            steps=np.full(B, last, np.uint64), rng=w.rng, eos_token_id=w.eos_token_id,
                            threads=min(os.cpu_count() or 1, 16))
        got = out.cpu().numpy().view(np.uint32)
        bad = int((got != ref["out"]).any(axis=1).sum())
        parity = {"rows_checked": B, "rows_mismatched": bad, "tick": last, "checker": "oracle (CPU)"}
        if bad:
            print(json.dumps({"parity": parity}), flush=True)
            sys.exit(f"bench.py: {bad} of {B} rows of the last timed step differ from the oracle")

    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / device_s / 1e9
    traffic = measured_traffic(w.name) if args.slices == 0 else None
    res = {
        "metric": METRIC,
        "value": B * args.steps / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "us_per_step": wall / args.steps * 1e6,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.dtype == "f32" else "bf16 logits, f32 arithmetic",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.description}",
            "batch": B,
            "vocab": V,
            "logits_dtype": w.dtype,
            "top_k": 50 if w.name in ("C3", "C4", "C5", "C5P") else int(w.params["top_k"][0]),
            "history": 0 if w.history is None else int(w.history.shape[1]),
            "slices_per_row": sampler.slices_per_row,
            "logits_buffers": nbuf,
            "parallelism": "single GPU; one workgroup per (row, vocab slice)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "kernel": KERNEL,
            "device_us_per_step": device_s * 1e6,
            "algorithmic_bytes": alg_bytes,
        },
        "parity": parity,
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds, args.cpu_threads)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
