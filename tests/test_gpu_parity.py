"""GPU parity: the HIP sampler through the C ABI against the CPU oracle on the
same seeded inputs. Token ids, output records and survivor sets are compared
bit-exactly; post-filter probabilities within 1e-5 relative (they are computed
with the same binary32 operation sequence, so they match exactly in practice).
"""
import zlib

import numpy as np
import pytest

from tests.gpu_util import assert_parity, run_gpu

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _random_params(rng, B, kcap, method=None):
    from llmoop_amd.sampler import ROW_PARAMS

    p = np.zeros(B, dtype=ROW_PARAMS)
    p["method"] = rng.integers(0, 2, B) if method is None else method
    p["temperature"] = rng.uniform(0.3, 1.5, B)
    p["top_k"] = rng.integers(1, kcap + 1, B)
    p["top_p"] = rng.uniform(0.2, 1.0, B)
    p["min_p"] = np.where(rng.random(B) < 0.5, 0.0, rng.uniform(0, 0.3, B))
    p["repetition_penalty"] = rng.uniform(0.8, 1.5, B)
    p["frequency_penalty"] = rng.uniform(0, 0.6, B)
    p["presence_penalty"] = rng.uniform(-0.5, 0.6, B)
    return p


CASES = [
    # (label, B, V, dtype, kcap, penalty mode, mask, value kind)
    ("small-f32", 8, 97, "f32", 16, "history", False, "normal"),
    ("small-bf16", 8, 200, "bf16", 16, "seen", True, "normal"),
    ("ties-f32", 6, 3000, "f32", 32, "none", False, "ties"),
    ("ties-bf16", 6, 5000, "bf16", 64, "history", True, "ties"),
    ("mid-f32", 16, 32000, "f32", 64, "history", True, "normal"),
    ("mid-bf16", 16, 50257, "bf16", 64, "seen", False, "normal"),
    ("big-bf16", 12, 151936, "bf16", 64, "history", False, "student"),
    ("big-f32-mask", 12, 128256, "f32", 64, "history", True, "normal"),
    ("odd-vocab", 10, 32003, "f32", 64, "none", True, "normal"),
    ("odd-vocab-bf16", 10, 151939, "bf16", 64, "history", False, "normal"),
    ("kcap-256", 8, 65536, "f32", 256, "history", False, "normal"),
    ("kcap-1024", 4, 65536, "bf16", 1024, "none", False, "normal"),
    ("sorted-desc", 4, 40000, "f32", 64, "none", False, "sorted"),
    ("constant", 4, 40000, "bf16", 64, "none", False, "constant"),
]


def _make_case(seed, B, V, dtype, kcap, pen, mask, kind):
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(seed)
    if kind == "ties":
        x = rng.integers(-4, 4, size=(B, V)).astype(np.float32)
    elif kind == "student":
        x = (rng.standard_t(4, size=(B, V)) * 2).astype(np.float32)
    elif kind == "sorted":
        x = np.sort(rng.standard_normal((B, V)).astype(np.float32), axis=1)[:, ::-1].copy()
    elif kind == "constant":
        x = np.zeros((B, V), np.float32)
    else:
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    logits = to_bf16_bits(x) if dtype == "bf16" else x
    params = _random_params(rng, B, kcap)
    kw = {
        "seeds": rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
        "steps": rng.integers(0, 2**40, B, dtype=np.uint64),
    }
    W = (V + 31) // 32
    if pen == "history":
        H = 48
        kw["history"] = rng.integers(0, V + 5, size=(B, H)).astype(np.uint32)
        kw["history"][:, :8] = kw["history"][:, 8:16]  # duplicates -> counts > 1
        kw["history_len"] = rng.integers(0, H + 1, B).astype(np.uint32)
    elif pen == "seen":
        kw["seen"] = (rng.random((B, W)) < 0.02).astype(np.uint32) * rng.integers(0, 2**32, (B, W), dtype=np.uint64).astype(np.uint32)
    if mask:
        a = rng.integers(0, 2**32, size=(B, W), dtype=np.uint64).astype(np.uint32)
        a &= rng.integers(0, 2**32, size=(B, W), dtype=np.uint64).astype(np.uint32)
        a[0] = 0
        kw["allowed"] = a
    return logits, params, kw


@pytest.mark.parametrize("label,B,V,dtype,kcap,pen,mask,kind", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("rng_mode", [0, 1])
def test_random_parity(oracle, label, B, V, dtype, kcap, pen, mask, kind, rng_mode):
    logits, params, kw = _make_case(zlib.crc32(f"{label}/{rng_mode}".encode()) & 0xFFFF, B, V, dtype, kcap, pen, mask, kind)
    _say(f"{label} rng={rng_mode} B={B} V={V} {dtype} kcap={kcap}")
    ref = oracle.sample(logits, params, top_k_capacity=kcap, rng=rng_mode, threads=8, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=kcap, rng=rng_mode, **kw)
    assert_parity(gpu, ref, params, label=label)


@pytest.mark.parametrize("slices", [1, 2, 3, 7, 16])
def test_slice_count_does_not_change_results(oracle, slices):
    logits, params, kw = _make_case(77, 8, 20000, "f32", 64, "history", True, "normal")
    _say(f"slices={slices}")
    ref = oracle.sample(logits, params, top_k_capacity=64, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=64, slices_per_row=slices, **kw)
    assert_parity(gpu, ref, params, label=f"slices={slices}")


@pytest.mark.parametrize("slices", [1, 3])
def test_greedy_nan_replay_with_history(oracle, slices):
    """Greedy rows holding a NaN replay the reference lane structure with the
    penalties: from the step's own bitmap and repeat table (one slice), or
    from the history's counts rebuilt after the merge (several slices)."""
    logits, params, kw = _make_case(91, 8, 40000, "f32", 64, "history", False, "normal")
    params["method"] = 0
    params["repetition_penalty"] = 1.3
    logits[1, 700] = np.nan
    logits[5, 39999] = np.nan
    logits[6, 3] = np.nan  # in the first stride of the replay's lanes
    _say(f"greedy nan replay slices={slices}")
    ref = oracle.sample(logits, params, top_k_capacity=64, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=64, slices_per_row=slices, **kw)
    assert_parity(gpu, ref, params, label=f"greedy-nan-{slices}")


def test_unaligned_row_stride_uses_scalar_loads(oracle):
    rng = np.random.default_rng(5)
    B, V, stride = 6, 5001, 5003
    x = (rng.standard_normal((B, stride)) * 2).astype(np.float32)
    params = _random_params(rng, B, 32)
    _say("unaligned stride")
    ref = oracle.sample(x, params, top_k_capacity=32, vocab_size=V)
    from llmoop_amd import sampler as S

    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=32)
    gpu = run_gpu(x, params, top_k_capacity=32, vocab=V, sampler=smp)
    assert_parity(gpu, ref, params, label="unaligned")
    # the count the step used: one element per load, 512 x 16 tokens per slice
    assert smp.slices_per_row == 1
    smp.close()


def test_large_vocab_with_kcap_1024(oracle):
    """V = 201088 bf16 with top_k_capacity 1024: the handle is sized for the
    16-byte-load kernels (2 slices per row, 3 by the automatic split of long
    rows in short batches; the lists then exceed the in-kernel merge area and
    the finish kernel merges them), and an unaligned row that would
    need more slices than it holds is rejected with a message, not a fault."""
    import torch

    from llmoop_amd import sampler as S
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(8)
    B, V = 4, 201088
    x = to_bf16_bits((rng.standard_normal((B, V)) * 2).astype(np.float32))
    params = _random_params(rng, B, 1024, method=1)
    _say("V=201088 kcap=1024")
    smp = S.Sampler(V, B, dtype="bf16", top_k_capacity=1024)
    ref = oracle.sample(x, params, top_k_capacity=1024)
    gpu = run_gpu(x, params, top_k_capacity=1024, sampler=smp)
    assert_parity(gpu, ref, params, label="V=201088", prob_rtol=2e-3)
    assert smp.slices_per_row == 3
    dev = torch.device("cuda:0")
    odd = torch.zeros((B, V + 1), dtype=torch.int16, device=dev)[:, 1:]  # 2-byte aligned rows only
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    with pytest.raises(S.SamplerError, match="slices"):
        smp.step(odd, S.params_tensor(params, dev), out)
    smp.close()


def test_special_values(oracle):
    B, V = 10, 4096
    rng = np.random.default_rng(11)
    x = rng.standard_normal((B, V)).astype(np.float32)
    x[0, 0] = np.nan            # greedy: lane 0 keeps NaN
    x[1, 1029] = np.nan         # greedy: a later NaN never wins
    x[2, :] = -np.inf           # all -inf
    x[3, 100:200] = np.inf      # +inf survivors -> NaN weights, reference falls to the last index
    x[4, :] = 0.0
    x[4, 7] = -0.0              # signed zero ties with +0.0
    x[4, 3] = -0.0
    x[5, ::3] = np.nan          # sampled rows skip NaN
    x[6, :] = -3.4028235e38     # -FLT_MAX everywhere: real tokens beat padding
    x[7, 10] = 1e-40            # subnormals
    x[7, 11] = -1e-40
    x[8, :] = np.nan
    x[9, :4000] = -np.inf
    params = _random_params(rng, B, 16)
    params["method"][[0, 1, 2, 4, 6, 8]] = 0
    params["method"][[3, 5, 7, 9]] = 1
    _say("special values")
    ref = oracle.sample(x, params, top_k_capacity=16)
    gpu = run_gpu(x, params, top_k_capacity=16)
    assert_parity(gpu, ref, params, label="special")


def test_greedy_small_vocab_all_neg_inf_pads_with_vocab_id(oracle):
    x = np.full((2, 10), -np.inf, np.float32)
    x[1, 4] = -3.4028235e38
    from llmoop_amd.sampler import make_params

    params = make_params(2, method=0)
    _say("greedy small vocab")
    ref = oracle.sample(x, params, top_k_capacity=1)
    gpu = run_gpu(x, params, top_k_capacity=1)
    assert_parity(gpu, ref, params, label="small-vocab-greedy")
    assert list(gpu["token_id"]) == [10, 4]


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5", "C5P"])
def test_benchmark_configs_full_size(oracle, name):
    from llmoop_amd import workloads

    w = workloads.make(name, seed=99, step=5)
    _say(f"config {name}")
    kw = dict(history=w.history, history_len=w.history_len, allowed=w.allowed, seeds=w.seeds, steps=w.steps)
    ref = oracle.sample(w.logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, threads=16, **kw)
    gpu = run_gpu(w.logits, w.params, top_k_capacity=w.top_k_capacity, rng=w.rng, **kw)
    assert_parity(gpu, ref, w.params, label=name, prob_rtol=1e-5 if w.dtype == "f32" else 2e-3)
    if name == "C4":
        empty = w.extra["empty_rows"]
        assert (gpu["token_id"][empty] == 2).all()
        assert (gpu["flags"][empty] == 3).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_penalised_top_tokens_take_the_exact_path(oracle, dtype):
    """The top raw logits of each row are all in its history with a large
    repetition penalty: the lane reports (raw values) point at tokens whose
    configured values fall far below, so fewer than k candidates reach the
    report threshold and the slice must fall back to the exact selection."""
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(31)
    B, V, H = 8, 40000, 256
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    hist = np.zeros((B, H), np.uint32)
    for r in range(B):
        top = np.argsort(-x[r])[:150]
        hist[r, :150] = top
        hist[r, 150:] = rng.integers(0, V, H - 150)
    logits = to_bf16_bits(x) if dtype == "bf16" else x
    params = _random_params(rng, B, 64, method=1)
    params["top_k"] = 50
    params["repetition_penalty"] = 50.0
    params["frequency_penalty"] = 0.0
    params["presence_penalty"] = 0.0
    params["min_p"] = 0.0
    kw = dict(history=hist, history_len=np.full(B, H, np.uint32),
              seeds=rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    _say(f"penalised top tokens {dtype}")
    ref = oracle.sample(logits, params, top_k_capacity=64, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=64, **kw)
    assert_parity(gpu, ref, params, label="penalised-top", prob_rtol=1e-5 if dtype == "f32" else 2e-3)
    # no survivor is one of the penalised top tokens
    for r in range(B):
        assert not set(gpu["topk_ids"][r][:50]) & set(hist[r, :150].tolist())


PENALISED_TOP_CASES = [
    # (label, dtype, V, row stride, slices, penalty state, mask, greedy rows)
    ("mask-greedy-bf16", "bf16", 60000, 60000, 0, "history", True, True),
    ("seen-f32", "f32", 50000, 50000, 0, "seen", False, False),
    ("seen-mask-bf16", "bf16", 151936, 151936, 0, "seen", True, True),
    ("unaligned-f32", "f32", 30001, 30003, 0, "history", False, True),
    ("slices3-bf16", "bf16", 100000, 100000, 3, "history", True, False),
    ("counts-f32", "f32", 128256, 128256, 0, "history", False, False),
]


@pytest.mark.parametrize("label,dtype,V,stride,slices,pen,mask,greedy", PENALISED_TOP_CASES,
                         ids=[c[0] for c in PENALISED_TOP_CASES])
def test_penalised_top_tokens_variants(oracle, label, dtype, V, stride, slices, pen, mask, greedy):
    """Rows whose largest raw logits are all penalised (history drawn from the
    row's own top tokens), across the kernel variants: masked rows with
    greedy rows among them, seen bitmaps, unaligned rows (one element per
    load), several slices per row, and repeat counts that drive the
    frequency penalty."""
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(zlib.crc32(label.encode()) & 0xFFFF)
    B, H = 8, 512
    x = (rng.standard_t(4, size=(B, stride)) * 2.0).astype(np.float32)
    top = np.argsort(-x[:, :V], axis=1)[:, :160]
    params = _random_params(rng, B, 64, method=1)
    params["top_k"] = rng.integers(20, 65, B)
    params["repetition_penalty"] = rng.uniform(1.05, 3.0, B)
    params["frequency_penalty"] = rng.uniform(0.0, 0.8, B)
    params["presence_penalty"] = rng.uniform(0.0, 0.8, B)
    if greedy:
        params["method"][::3] = 0
    kw = dict(seeds=rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    W = (V + 31) // 32
    if pen == "history":
        kw["history"] = np.take_along_axis(top, rng.integers(0, top.shape[1], (B, H)), axis=1).astype(np.uint32)
        kw["history_len"] = np.full(B, H, np.uint32)
    else:
        bits = np.zeros((B, W * 32), bool)
        np.put_along_axis(bits, top, True, axis=1)
        weights = np.uint64(1) << np.arange(32, dtype=np.uint64)
        kw["seen"] = (bits.reshape(B, W, 32).astype(np.uint64) * weights).sum(axis=2).astype(np.uint32)
    if mask:
        allow = rng.random((B, W * 32)) < 0.7
        allow[:, V:] = False
        weights = np.uint64(1) << np.arange(32, dtype=np.uint64)
        kw["allowed"] = (allow.reshape(B, W, 32).astype(np.uint64) * weights).sum(axis=2).astype(np.uint32)
    logits = to_bf16_bits(x) if dtype == "bf16" else x
    _say(f"penalised top {label}")
    ref = oracle.sample(logits, params, top_k_capacity=64, vocab_size=V, threads=8, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=64, vocab=V, slices_per_row=slices, **kw)
    assert_parity(gpu, ref, params, label=label, prob_rtol=1e-5 if dtype == "f32" else 2e-3)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_many_repeated_history_ids(oracle, dtype):
    """Each row's history repeats its top raw tokens many times (hundreds of
    occurrences beyond the first), so the repeat counts go through the table
    rather than the short scan, and the frequency penalty separates tokens by
    their counts."""
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(57)
    B, V, H = 6, 30000, 512
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    hist = np.zeros((B, H), np.uint32)
    for r in range(B):
        top = np.argsort(-x[r])[:40]
        reps = np.repeat(top, rng.integers(1, 12, top.size))[:H]
        hist[r, :reps.size] = reps
        hist[r, reps.size:] = rng.integers(0, V, H - reps.size)
        rng.shuffle(hist[r])
    logits = to_bf16_bits(x) if dtype == "bf16" else x
    params = _random_params(rng, B, 64, method=1)
    params["top_k"] = 40
    params["repetition_penalty"] = 1.05
    params["frequency_penalty"] = 0.15
    params["presence_penalty"] = 0.1
    kw = dict(history=hist, history_len=np.full(B, H, np.uint32),
              seeds=rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    _say(f"many repeated history ids {dtype}")
    ref = oracle.sample(logits, params, top_k_capacity=64, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=64, **kw)
    assert_parity(gpu, ref, params, label="many-repeats", prob_rtol=1e-5 if dtype == "f32" else 2e-3)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kcap", [64, 1024])
def test_exact_path_with_ties_beyond_the_candidate_list(oracle, dtype, kcap):
    """The 150 top raw logits of each row sit far above the rest and are all
    penalised out of reach, so the slice falls back to the exact selection;
    the remaining values are small integers, so thousands of tokens tie at
    the k-th value and only the lowest ids among them may survive."""
    from llmoop_amd.workloads import to_bf16_bits

    rng = np.random.default_rng(73 + kcap)
    B, V, H = 8, 40000, 256
    x = rng.integers(-4, 4, size=(B, V)).astype(np.float32)
    hist = np.zeros((B, H), np.uint32)
    for r in range(B):
        top = rng.choice(V, 150, replace=False)
        x[r, top] = 10.0
        hist[r, :150] = top
        hist[r, 150:] = top[rng.integers(0, 150, H - 150)]
    logits = to_bf16_bits(x) if dtype == "bf16" else x
    params = _random_params(rng, B, kcap, method=1)
    params["top_k"] = rng.integers(1, kcap + 1, B)
    params["repetition_penalty"] = 50.0
    params["frequency_penalty"] = 0.0
    params["presence_penalty"] = 0.0
    kw = dict(history=hist, history_len=np.full(B, H, np.uint32),
              seeds=rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32),
              steps=rng.integers(0, 2**40, B, dtype=np.uint64))
    _say(f"exact path with ties {dtype} kcap={kcap}")
    ref = oracle.sample(logits, params, top_k_capacity=kcap, **kw)
    gpu = run_gpu(logits, params, top_k_capacity=kcap, **kw)
    assert_parity(gpu, ref, params, label="exact-ties", prob_rtol=1e-5 if dtype == "f32" else 2e-3)
