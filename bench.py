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

--config L5 times the decode tail instead: the LM-head projection (bf16
frames x bf16 tied weight -> f32 logits, with the tile-record epilogue) and the
step over the tile records, next to the projection followed by the dense step
and each kernel alone; the last fused step is checked against the oracle.
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
    ap.add_argument("--config", default="C5",
                    help="C1..C5, C5P (C5 is the headline workload); L5: LM-head projection + step")
    ap.add_argument("--input-size", type=int, default=4096, help="L5: width of the projected frames")
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


def main_l5(args):
    """L5: one decode tail = the LM-head projection (bf16 frames x bf16 weight
    -> f32 logits, with the tile-record epilogue) then the step that samples
    from the records. The same step through the projection without records
    and the dense step, and each kernel alone, are timed beside it."""
    import torch

    from llmoop_amd import sampler as S
    from llmoop_amd import workloads

    dev = torch.device("cuda:0")
    w = workloads.make("L5", seed=2024, step=0, input_size=args.input_size)
    B, V, D = w.batch, w.vocab, args.input_size
    frames, weight = workloads.lm_head_inputs(w, dev)
    sampler = S.Sampler(V, B, dtype="f32", top_k_capacity=w.top_k_capacity, history_capacity=w.history.shape[1])

    def dev_arr(a):
        a = np.ascontiguousarray(a)
        view = {np.uint32: np.int32, np.uint16: np.int16, np.uint64: np.int64}.get(a.dtype.type, a.dtype.type)
        return torch.from_numpy(a.view(view).copy()).to(dev)

    logits = torch.empty((B, V), dtype=torch.float32, device=dev)
    records = torch.empty((B, 2 * S.tile_count(V)), dtype=torch.int32, device=dev)
    params = S.params_tensor(w.params, dev)
    kw = dict(history=dev_arr(w.history), history_len=dev_arr(w.history_len), seeds=dev_arr(w.seeds), rng=w.rng)
    sc = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    scale = float(w.extra["scale"])

    def project(rec=True):
        S.lm_head_project(frames, weight, logits, output_scale=scale, tile_records=records if rec else None)

    def fused():
        project()
        sampler.step(logits, params, out, stream_control=sc, tile_records=records, **kw)

    def unfused():
        project(False)
        sampler.step(logits, params, out, stream_control=sc, **kw)

    def timed(fn, n):
        for _ in range(min(args.warmup, 10)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n, e0.elapsed_time(e1) / 1e3 / n

    n = max(1, args.steps)
    sc.zero_()
    wall, dev_s = timed(fused, n)
    ticks_done = int(sc[0, 1].item())
    parity = None
    if not args.no_check:
        from oracle import oracle

        ref = oracle.sample(logits.cpu().numpy(), w.params, top_k_capacity=w.top_k_capacity, history=w.history,
                            history_len=w.history_len, seeds=w.seeds, steps=np.full(B, ticks_done - 1, np.uint64),
                            rng=w.rng, threads=min(os.cpu_count() or 1, 16))
        bad = int((out.cpu().numpy().view(np.uint32) != ref["out"]).any(axis=1).sum())
        parity = {"rows_checked": B, "rows_mismatched": bad, "tick": ticks_done - 1, "checker": "oracle (CPU)"}
        if bad:
            print(json.dumps({"parity": parity}), flush=True)
            sys.exit(f"bench.py: {bad} of {B} rows of the last fused step differ from the oracle")
    _, unfused_s = timed(unfused, n)
    _, proj_s = timed(project, n)
    _, proj_norec_s = timed(lambda: project(False), n)
    _, tiles_s = timed(lambda: sampler.step(logits, params, out, stream_control=sc, tile_records=records, **kw), n)
    _, dense_s = timed(lambda: sampler.step(logits, params, out, stream_control=sc, **kw), n)
    # the projection's once-through bytes: weight and frames read, logits and records written
    proj_bytes = V * D * 2 + B * D * 2 + B * V * 4 + B * S.tile_count(V) * 8
    flops = 2.0 * B * V * D
    achieved = proj_bytes / proj_s / 1e9
    res = {
        "metric": "sampled rows/sec of LM head + sampling step (B=256, V=151936)",
        "value": B / wall,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "us_per_step": wall * 1e6,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x bf16 -> f32 projection, f32 sampling",
        "data": "synthetic (random bf16 frames and weight made on the device)",
        "config": {"workload": f"L5: {w.description}", "batch": B, "vocab": V, "input_size": D,
                   "parallelism": "single GPU"},
        "device_us": {"fused_step": dev_s * 1e6, "unfused_step": unfused_s * 1e6,
                      "projection_with_records": proj_s * 1e6, "projection": proj_norec_s * 1e6,
                      "tile_step": tiles_s * 1e6, "dense_step": dense_s * 1e6},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "lm_head_kernel",
                     "algorithmic_bytes": proj_bytes, "mfma_tflops": flops / proj_s / 1e12,
                     "mfma_frac_of_2500": flops / proj_s / 1e12 / 2500.0},
        "parity": parity,
    }
    print(json.dumps(res), flush=True)


def main():
    args = parse()
    if args.config.upper() == "L5" and args.gpus == 1:
        return main_l5(args)
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
