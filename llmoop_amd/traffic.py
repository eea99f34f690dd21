"""HBM traffic of the sampling kernel from rocprofv3 byte counters.

FETCH_SIZE and WRITE_SIZE count bytes at the memory side in their own units;
a kernel that reads and writes a known number of bytes, measured in the same
rocprofv3 run, gives the factor that turns them into bytes.

  python llmoop_amd/traffic.py run --config C5 --steps 50 --calibrate-mib 256
      runs `steps` sampling steps of the workload (L5: projection with tile
      records + tile step), then 20 elementwise
      negations of MIB MiB of float32 (each reads and writes exactly MIB MiB);
      meant to run under `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE)
  python llmoop_amd/traffic.py summary DIR [DIR ...] --calibrate-mib 256
      reads the counter_collection.csv files under the DIRs and prints the
      per-kernel averages and the calibrated bytes per sampling launch
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

KERNEL = "sample_rows_kernel"
COPY_KERNEL = "neg_kernel"


def run_l5(steps: int) -> None:
    """The fused decode tail of L5: projection with tile records, then the tile step."""
    import torch

    from llmoop_amd import sampler as S
    from llmoop_amd import workloads

    dev = torch.device("cuda:0")
    w = workloads.make("L5", seed=2024, step=0)
    frames, weight = workloads.lm_head_inputs(w, dev)
    B, V = w.batch, w.vocab
    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=w.top_k_capacity, history_capacity=w.history.shape[1])
    lg = torch.empty((B, V), dtype=torch.float32, device=dev)
    rec = torch.empty((B, 2 * S.tile_count(V)), dtype=torch.int32, device=dev)

    def dev_arr(a):
        a = np.ascontiguousarray(a)
        view = {np.uint32: np.int32, np.uint64: np.int64}.get(a.dtype.type, a.dtype.type)
        return torch.from_numpy(a.view(view).copy()).to(dev)

    params = S.params_tensor(w.params, dev)
    kw = dict(history=dev_arr(w.history), history_len=dev_arr(w.history_len), seeds=dev_arr(w.seeds), rng=w.rng)
    sc = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    for _ in range(steps):
        S.lm_head_project(frames, weight, lg, output_scale=float(w.extra["scale"]), tile_records=rec)
        smp.step(lg, params, out, stream_control=sc, tile_records=rec, **kw)
    torch.cuda.synchronize()


def run(config: str, steps: int, calibrate_mib: int) -> None:
    import torch

    from llmoop_amd import workloads

    dev = torch.device("cuda:0")
    if config.upper() == "L5":
        run_l5(steps)
        w = None
    else:
        w = workloads.make(config, seed=2024, step=0)

    def dev_arr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a)
        view = {np.uint32: np.int32, np.uint16: np.int16, np.uint64: np.int64}.get(a.dtype.type, a.dtype.type)
        return torch.from_numpy(a.view(view).copy()).to(dev)

    if w is not None:
        _run_steps(w, steps, dev, dev_arr)
    if calibrate_mib:
        n = calibrate_mib * 2**20 // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()


def _run_steps(w, steps, dev, dev_arr) -> None:
    import torch

    from llmoop_amd import sampler as S

    smp = S.Sampler(w.vocab, w.batch, dtype=w.dtype, top_k_capacity=w.top_k_capacity,
                    history_capacity=0 if w.history is None else w.history.shape[1])
    lg, params = dev_arr(w.logits), S.params_tensor(w.params, dev)
    kw = dict(history=dev_arr(w.history), history_len=dev_arr(w.history_len), allowed=dev_arr(w.allowed),
              seeds=dev_arr(w.seeds), rng=w.rng, eos_token_id=w.eos_token_id)
    sc = torch.zeros((w.batch, 5), dtype=torch.int32, device=dev)
    out = torch.zeros((w.batch, 4), dtype=torch.int32, device=dev)
    for _ in range(steps):
        smp.step(lg, params, out, stream_control=sc, **kw)
    torch.cuda.synchronize()


def read_counters(directories) -> dict:
    """{kernel name: {counter: [per-dispatch values]}} from rocprofv3 CSVs."""
    out: dict = {}
    for d in directories:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for r in csv.DictReader(f):
                    per = out.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], {})
                    key = (path, r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(per)))
                    per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    return {k: {c: list(v.values()) for c, v in d.items()} for k, d in out.items()}


def summary(directories, calibrate_mib: int, kernel: str = KERNEL) -> int | None:
    counters = read_counters(directories)
    rows = []
    for name, d in counters.items():
        for c, v in d.items():
            rows.append((name, c, float(np.mean(v)), len(v)))
    for name, c, mean, n in sorted(rows):
        print(f"{c:10s} {mean:14.1f}  n={n:4d}  {name[:100]}")

    def pick(pattern, counter):
        vals = [m for name, c, m, _ in rows if c == counter and re.search(pattern, name)]
        return max(vals) if vals else None

    fetch, write = pick(kernel, "FETCH_SIZE"), pick(kernel, "WRITE_SIZE")
    cfetch, cwrite = pick(COPY_KERNEL, "FETCH_SIZE"), pick(COPY_KERNEL, "WRITE_SIZE")
    if fetch is None or cfetch is None:
        print("missing sampling-kernel or calibration-kernel counters")
        return None
    copy_bytes = calibrate_mib * 2**20
    fr = copy_bytes / (cfetch * 1024.0)
    wr = copy_bytes / (cwrite * 1024.0) if cwrite else 1.0
    traffic = fetch * 1024.0 * fr + (write or 0.0) * 1024.0 * wr
    print(f"calibration kernel: {copy_bytes} B read and written; FETCH_SIZE {cfetch:.1f} KiB -> factor {fr:.4f}; "
          f"WRITE_SIZE {cwrite} KiB -> factor {wr:.4f}")
    print(f"traffic_bytes_per_launch = {traffic:.0f}")
    return int(traffic)


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--config", default="C5")
    r.add_argument("--steps", type=int, default=50)
    r.add_argument("--calibrate-mib", type=int, default=256)
    s = sub.add_parser("summary")
    s.add_argument("dirs", nargs="+")
    s.add_argument("--calibrate-mib", type=int, default=256)
    s.add_argument("--kernel", default=KERNEL, help="kernel name pattern of the per-launch traffic")
    a = ap.parse_args()
    if a.cmd == "run":
        run(a.config, a.steps, a.calibrate_mib)
    else:
        summary(a.dirs, a.calibrate_mib, a.kernel)


if __name__ == "__main__":
    main()
