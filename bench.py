"""Benchmark of the gfx950 sampling stage.

A step is one nerve_sampler_step over one batch of synthetic logits already
resident in HBM (one fused launch). The default workload is C5, the
configuration the headline metric is quoted on: B=256 rows x V=151936 bf16
logits (Student-t(4) * 2), a 2048-id history per row with repetition 1.1 /
frequency 0.5 / presence 0.3, top-k 50, top-p 0.9, per-row temperature in
[0.5, 1.2] and a Philox draw. Consecutive steps advance each row's stream
tick on the device (reference stream-control semantics), so K timed steps are
K different draws with no host work in between.

Prints one JSON line: rows/s (whole job), us/step, the HBM roofline of the
sampling kernel (algorithmic bytes / average kernel time from HIP events on
the launch stream, against 8 TB/s) and the CPU oracle timed on the host cores
of the same machine on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec + µs/step at B=256×V=151936; % of HBM roofline"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C5", help="C1..C5 (C5 is the headline workload)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--slices", type=int, default=0, help="workgroups per row (0 = automatic)")
    ap.add_argument("--variant", default="", help="diagnostics: no-history | greedy | no-penalty")
    return ap.parse_args()


def cpu_baseline(w, budget_s: float) -> dict:
    """The oracle (a C restatement of the reference semantics, -O3, OpenMP
    over rows) on the host cores: as many full-batch steps as fit the budget."""
    from oracle import oracle

    threads = min(os.cpu_count() or 1, 16)
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
    if args.variant == "no-history":
        w.history = w.history_len = None
    elif args.variant == "greedy":
        w.params["method"] = 0
    elif args.variant == "no-penalty":
        w.params["repetition_penalty"] = 1.0
        w.params["frequency_penalty"] = 0.0
        w.params["presence_penalty"] = 0.0
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

    logits = dev_arr(w.logits)
    params = S.params_tensor(w.params, dev)
    history = dev_arr(w.history)
    history_len = dev_arr(w.history_len)
    allowed = dev_arr(w.allowed)
    seeds = dev_arr(w.seeds)
    stream_control = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)

    def step():
        sampler.step(logits, params, out, history=history, history_len=history_len, allowed=allowed,
                     seeds=seeds, rng=w.rng, eos_token_id=w.eos_token_id, stream_control=stream_control)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # whole-step wall clock over K steps
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # kernel time from HIP events on the launch stream (torch's current stream)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        starts[i].record()
        step()
        ends[i].record()
    torch.cuda.synchronize()
    kern_ms = np.array([s.elapsed_time(e) for s, e in zip(starts, ends)])
    kern_avg_s = float(np.mean(kern_ms)) / 1e3

    tick = stream_control[:, 1].cpu().numpy().view(np.uint32)
    assert (tick == args.warmup + 2 * args.steps).all(), "stream ticks did not advance once per step"

    alg_bytes = w.algorithmic_bytes()
    achieved = alg_bytes / kern_avg_s / 1e9
    us_per_step = wall / args.steps * 1e6
    res = {
        "metric": METRIC,
        "value": B * args.steps / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "us_per_step": us_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.description}",
            "batch": B,
            "vocab": V,
            "logits_dtype": w.dtype,
            "top_k": 50 if w.name in ("C3", "C4", "C5") else int(w.params["top_k"][0]),
            "history": 0 if w.history is None else int(w.history.shape[1]),
            "slices_per_row": sampler.slices_per_row,
            "parallelism": "single GPU; one workgroup per (row, vocab slice)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
            "kernel": "sample_rows_kernel",
            "kernel_us": kern_avg_s * 1e6,
            "algorithmic_bytes": alg_bytes,
        },
    }
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
