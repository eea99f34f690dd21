"""The LM-head projection with its tile-record epilogue, and the step that
samples from the tile records (nerve_lm_head_project, nerve_tile_records,
nerve_sampler_step_tiles).

- The projection is a floating-point GEMM: it is checked against a float64
  product of the same bf16 inputs, within a bound on f32 summation-order error
  (1e-4 of the sum of |products|); its tile records are checked bit-exactly
  against records computed in numpy from the logits it wrote.
- The tile step must return exactly what the dense step returns on the same
  logits (token ids, output records, survivor ids and logits, probabilities
  bit for bit), and what the oracle returns.
"""
import zlib

import numpy as np
import pytest

from llmoop_amd import sampler as S
from tests.gpu_util import assert_parity, run_gpu, to_dev

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def order_keys(bits: np.ndarray) -> np.ndarray:
    """The unsigned order key of binary32 bit patterns (NaN -> 0, +-0 -> 0x80000000)."""
    b = bits.astype(np.uint32)
    mag = b & np.uint32(0x7FFFFFFF)
    b = np.where(mag == 0, np.uint32(0), b)
    key = np.where(b & np.uint32(0x80000000), ~b, b | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(mag > np.uint32(0x7F800000), np.uint32(0), key)


def records_of(logits_f32: np.ndarray, vocab: int) -> np.ndarray:
    bits = np.ascontiguousarray(logits_f32[:, :vocab], dtype=np.float32).view(np.uint32)
    B = bits.shape[0]
    T = (vocab + 63) // 64
    pad = np.zeros((B, T * 64), np.uint32)
    keys = order_keys(bits)
    pad[:, :vocab] = keys
    nan = np.zeros((B, T * 64), np.uint32)
    nan[:, :vocab] = ((bits & 0x7FFFFFFF) > 0x7F800000).astype(np.uint32)
    out = np.zeros((B, T, 2), np.uint32)
    out[:, :, 0] = pad.reshape(B, T, 64).max(axis=2)
    out[:, :, 1] = nan.reshape(B, T, 64).sum(axis=2)
    return out


def bf16_bits(x):
    from llmoop_amd.workloads import to_bf16_bits

    return to_bf16_bits(x)


def bf16_value(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


# 70000 and 140000 columns need more 256-column blocks than the GPU has CUs:
# the last, partial round uses 128-column blocks
@pytest.mark.parametrize("B,D,V", [(1, 64, 1000), (37, 512, 4099), (256, 256, 8192), (300, 128, 1031),
                                   (40, 64, 70000), (9, 128, 140000)])
def test_lm_head_projection(B, D, V):
    import torch

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(B * 1000 + V)
    fr = bf16_bits(rng.standard_normal((B, D)).astype(np.float32))
    w = bf16_bits((rng.standard_normal((V, D)) * 0.05).astype(np.float32))
    if B > 3:
        fr[3, 5] = 0x7FC0  # a NaN frame: its row of logits is NaN
    scale = 0.75
    ls = V + 5
    _say(f"lm_head B={B} D={D} V={V}")
    lg = torch.full((B, ls), 7.0, dtype=torch.float32, device=dev)
    T = S.tile_count(V)
    rec = torch.full((B, 2 * T), -1, dtype=torch.int32, device=dev)
    S.lm_head_project(to_dev(fr, dev, torch), to_dev(w, dev, torch), lg, output_scale=scale, tile_records=rec)
    torch.cuda.synchronize()
    got = lg.cpu().numpy()
    assert (got[:, V:] == 7.0).all(), "columns past the vocabulary were written"
    a = bf16_value(fr).astype(np.float64)
    b = bf16_value(w).astype(np.float64)
    ref = (a @ b.T) * scale
    bound = 1e-4 * (np.abs(a) @ np.abs(b).T) * abs(scale) + 1e-30
    fin = np.isfinite(ref)
    assert np.all(np.abs(got[:, :V][fin] - ref[fin]) <= bound[fin])
    assert np.all(np.isnan(got[:, :V][~fin]))
    want = records_of(got, V)
    np.testing.assert_array_equal(rec.cpu().numpy().view(np.uint32).reshape(B, T, 2), want)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_tile_records_of_existing_logits(dtype):
    import torch

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(11)
    B, V, ls = 5, 3000, 3008
    x = (rng.standard_normal((B, ls)) * 3).astype(np.float32)
    x[0, 10] = np.nan
    x[1, :] = -np.inf
    x[2, 64:128] = 0.0
    x[2, 70] = -0.0
    x[3, 2999] = np.inf
    x[4, 3000:] = 1e30  # past the vocabulary: ignored
    arr = bf16_bits(x) if dtype == "bf16" else x
    vals = bf16_value(arr) if dtype == "bf16" else x
    _say(f"tile records {dtype}")
    T = S.tile_count(V)
    rec = torch.zeros((B, 2 * T), dtype=torch.int32, device=dev)
    S.tile_records(to_dev(arr, dev, torch), rec, vocab=V)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(rec.cpu().numpy().view(np.uint32).reshape(B, T, 2), records_of(vals, V))


def _params(rng, B, kcap, method=None):
    p = np.zeros(B, dtype=S.ROW_PARAMS)
    p["method"] = rng.integers(0, 2, B) if method is None else method
    p["temperature"] = rng.uniform(0.3, 1.5, B)
    p["top_k"] = rng.integers(1, kcap + 1, B)
    p["top_p"] = rng.uniform(0.2, 1.0, B)
    p["min_p"] = np.where(rng.random(B) < 0.5, 0.0, rng.uniform(0, 0.3, B))
    p["repetition_penalty"] = rng.uniform(1.0, 1.5, B)
    p["frequency_penalty"] = rng.uniform(0, 0.6, B)
    p["presence_penalty"] = rng.uniform(0, 0.6, B)
    return p


def _pack(bits: np.ndarray) -> np.ndarray:
    B, n = bits.shape
    W = (n + 31) // 32
    pad = np.zeros((B, W * 32), bool)
    pad[:, :n] = bits
    weights = np.uint64(1) << np.arange(32, dtype=np.uint64)
    return (pad.reshape(B, W, 32).astype(np.uint64) * weights).sum(axis=2).astype(np.uint32)


TILE_CASES = [
    # label, dtype, V, kcap, penalty state, mask, value kind, params tweak
    ("decode-bf16", "bf16", 151936, 64, "history", False, "student", None),
    ("decode-f32-mask", "f32", 128256, 64, "history", True, "normal", None),
    ("penalised-top-bf16", "bf16", 100000, 64, "history-top", False, "student", None),
    ("seen-f32", "f32", 50000, 64, "seen", False, "normal", None),
    ("seen-top-mask-bf16", "bf16", 60000, 64, "seen-top", True, "student", None),
    ("raising-penalties", "f32", 40000, 64, "history-top", False, "normal", "raising"),
    ("greedy-nan", "f32", 30000, 16, "history", False, "nan", "greedy"),
    ("constant", "bf16", 20000, 64, "none", False, "constant", None),
    ("ties", "f32", 20000, 64, "history", True, "ties", None),
    ("kcap-1024", "bf16", 65536, 1024, "history", False, "normal", "bigk"),
    ("small-vocab", "f32", 200, 16, "seen", True, "normal", None),
    ("odd-vocab", "f32", 32003, 64, "none", True, "normal", None),
]


def _tile_case(label, dtype, V, kcap, pen, mask, kind, tweak):
    rng = np.random.default_rng(zlib.crc32(label.encode()) & 0xFFFF)
    B = 12
    if kind == "student":
        x = (rng.standard_t(4, size=(B, V)) * 2).astype(np.float32)
    elif kind == "constant":
        x = np.full((B, V), 1.5, np.float32)
    elif kind == "ties":
        x = rng.integers(-3, 3, size=(B, V)).astype(np.float32)
    else:
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    if kind == "nan":
        x[1, 77] = np.nan
        x[4, 5000] = np.nan
    params = _params(rng, B, kcap)
    if tweak == "raising":
        params["repetition_penalty"] = rng.uniform(0.5, 0.9, B)
        params["presence_penalty"] = rng.uniform(-1.0, 0.0, B)
    if tweak == "greedy":
        params["method"] = 0
    if tweak == "bigk":
        params["top_k"] = rng.integers(500, kcap + 1, B)
    kw = dict(seeds=rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    top = np.argsort(-x, axis=1)[:, :150]
    if pen.startswith("history"):
        H = 512
        hist = rng.integers(0, V, (B, H)).astype(np.uint32)
        if pen == "history-top":
            hist = np.take_along_axis(top, rng.integers(0, 150, (B, H)), axis=1).astype(np.uint32)
        kw["history"] = hist
        kw["history_len"] = rng.integers(H // 2, H + 1, B).astype(np.uint32)
    elif pen.startswith("seen"):
        bits = rng.random((B, V)) < 0.01
        if pen == "seen-top":
            np.put_along_axis(bits, top, True, axis=1)
        kw["seen"] = _pack(bits)
    if mask:
        allow = rng.random((B, V)) < 0.8
        allow[0] = False  # EOS fallback row
        kw["allowed"] = _pack(allow)
    logits = bf16_bits(x) if dtype == "bf16" else x
    return logits, params, kw


@pytest.mark.parametrize("case", TILE_CASES, ids=[c[0] for c in TILE_CASES])
def test_tile_step_matches_dense_and_oracle(oracle, case):
    label, dtype, V, kcap = case[:4]
    logits, params, kw = _tile_case(*case)
    _say(f"tile step {label}")
    dense = run_gpu(logits, params, top_k_capacity=kcap, rng=S.RNG_PHILOX, **kw)
    tiles = run_gpu(logits, params, top_k_capacity=kcap, rng=S.RNG_PHILOX, tiles=True, **kw)
    for key in ("out", "topk_ids", "topk_logits", "topk_probs"):
        np.testing.assert_array_equal(tiles[key].view(np.uint32), dense[key].view(np.uint32), err_msg=f"{label}: {key}")
    ref = oracle.sample(logits, params, top_k_capacity=kcap, rng=S.RNG_PHILOX, threads=8, **kw)
    assert_parity(tiles, ref, params, label=label, prob_rtol=1e-5 if dtype == "f32" else 2e-3)


def test_tile_step_with_lane_prefixes():
    """Per-lane prefixes over a shared seen bitmap (sample_batch): tiles == dense."""
    rng = np.random.default_rng(5)
    B, V = 10, 50000
    x = (rng.standard_t(4, size=(B, V)) * 2).astype(np.float32)
    seen = _pack(rng.random((B, V)) < 0.01)
    top = np.argsort(-x, axis=1)[:, :40]
    pre = top[:, :20].astype(np.uint32)
    counts = rng.integers(0, 21, B).astype(np.uint32)
    params = _params(rng, B, 64)
    kw = dict(seen=seen, prefix_ids=pre, prefix_counts=counts, seeds=rng.integers(0, 2**32, B).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    _say("tile step prefixes")
    dense = run_gpu(x, params, top_k_capacity=64, rng=S.RNG_PHILOX, **kw)
    tiles = run_gpu(x, params, top_k_capacity=64, rng=S.RNG_PHILOX, tiles=True, **kw)
    for key in ("out", "topk_ids", "topk_logits", "topk_probs"):
        np.testing.assert_array_equal(tiles[key].view(np.uint32), dense[key].view(np.uint32), err_msg=key)


def test_fused_projection_and_step(oracle):
    """B=256 x V=151936 from a D=1024 projection: the fused path (projection
    with records, tile step) against the projection's logits through the dense
    step and through the oracle."""
    import torch

    from llmoop_amd import workloads

    dev = torch.device("cuda:0")
    w = workloads.make("L5", seed=3, step=0, input_size=1024)
    _say("fused L5 D=1024")
    fr, wt = workloads.lm_head_inputs(w, dev)
    B, V = w.batch, w.vocab
    lg = torch.empty((B, V), dtype=torch.float32, device=dev)
    rec = torch.empty((B, 2 * S.tile_count(V)), dtype=torch.int32, device=dev)
    S.lm_head_project(fr, wt, lg, output_scale=w.extra["scale"], tile_records=rec)
    torch.cuda.synchronize()
    logits = lg.cpu().numpy()
    np.testing.assert_array_equal(rec.cpu().numpy().view(np.uint32).reshape(B, -1, 2), records_of(logits, V))
    kw = dict(history=w.history, history_len=w.history_len, seeds=w.seeds, steps=w.steps)
    dense = run_gpu(logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, **kw)
    tiles = run_gpu(logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, tiles=True, **kw)
    for key in ("out", "topk_ids", "topk_logits", "topk_probs"):
        np.testing.assert_array_equal(tiles[key].view(np.uint32), dense[key].view(np.uint32), err_msg=key)
    ref = oracle.sample(logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, threads=16, **kw)
    assert_parity(tiles, ref, w.params, label="fused-L5")
