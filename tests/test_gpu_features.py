"""GPU tests of the decode-loop features around the step: the feedback-control
commit (greedy_sampler_f32.comp.template:35-50), the device-side append of the
sampled token to the penalty state (multi_stream_batch_runner.rs:235-240), the
per-lane seen-state prefixes of sample_lanes / sample_batch
(batched_output_projection.rs:277-371), and consecutive steps driven by stream
control at the full C5 shape. Every step goes through the C ABI; sampled rows
are checked bit-exactly against the CPU oracle fed the same state, feedback
words against hand-computed values.
"""
import numpy as np
import pytest

from llmoop_amd import sampler as S
from llmoop_amd import workloads
from oracle import oracle
from tests.gpu_util import to_dev

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _torch():
    import torch

    return torch, torch.device("cuda:0")


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


# ---- feedback control ---------------------------------------------------------


def _greedy_case(B, V, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    winners = rng.integers(0, V, B)
    x[np.arange(B), winners] = 20.0
    return x, winners


@pytest.mark.parametrize("case", ["enabled-no-stop", "eos", "cancel", "disabled", "already-stopped", "eos-and-cancel"])
def test_feedback_control_commit(case):
    torch, dev = _torch()
    _say(f"feedback {case}")
    V = 4096
    x, winners = _greedy_case(1, V, 11)
    tok = int(winners[0])
    fc = np.zeros(S.FEEDBACK_HEADER_WORDS, np.uint32)
    stop = np.zeros((V + 31) // 32, np.uint32)
    stop[5] = 1 << 3  # an unrelated stop token
    if case != "disabled":
        fc[0] = S.FEEDBACK_ENABLED
    if case in ("eos", "eos-and-cancel"):
        stop[tok >> 5] |= 1 << (tok & 31)
    if case in ("cancel", "eos-and-cancel"):
        fc[0] |= S.FEEDBACK_CANCEL_REQUESTED
    if case == "already-stopped":
        fc[2] = S.STOP_REASON_EOS
        stop[tok >> 5] |= 1 << (tok & 31)
    fc[9] = 7
    smp = S.Sampler(V, 1, dtype="f32", top_k_capacity=8)
    params = S.params_tensor(S.make_params(1, method=S.METHOD_GREEDY), dev)
    out = torch.zeros((1, 4), dtype=torch.int32, device=dev)
    fcd = to_dev(fc, dev, torch)
    smp.step(to_dev(x, dev, torch), params, out, feedback_control=fcd, stop_tokens=to_dev(stop, dev, torch))
    torch.cuda.synchronize()
    got = _u32(fcd)
    assert _u32(out)[0, 0] == tok
    want = fc.copy()
    if case != "disabled":
        want[9] = 8
        if case == "eos":
            want[2], want[8] = S.STOP_REASON_EOS, 2
        elif case in ("cancel", "eos-and-cancel"):
            want[2], want[8] = S.STOP_REASON_CANCELLED, 2
    np.testing.assert_array_equal(got, want)
    smp.close()


def test_feedback_control_per_row_blocks():
    """B rows with their own blocks and masks; one shared block counts every row."""
    torch, dev = _torch()
    _say("feedback per-row blocks")
    B, V = 6, 2000
    x, winners = _greedy_case(B, V, 12)
    fc = np.zeros((B, 16), np.uint32)
    fc[:, 0] = S.FEEDBACK_ENABLED
    fc[1, 0] |= S.FEEDBACK_CANCEL_REQUESTED
    fc[4, 0] = 0
    W = (V + 31) // 32
    stop = np.zeros((B, W), np.uint32)
    for r in (2, 4, 5):
        t = int(winners[r])
        stop[r, t >> 5] |= 1 << (t & 31)
    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=8)
    params = S.params_tensor(S.make_params(B, method=S.METHOD_GREEDY), dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    fcd = to_dev(fc, dev, torch)
    smp.step(to_dev(x, dev, torch), params, out, feedback_control=fcd, stop_tokens=to_dev(stop, dev, torch))
    shared = torch.zeros(12, dtype=torch.int32, device=dev)
    shared[0] = S.FEEDBACK_ENABLED
    smp.step(to_dev(x, dev, torch), params, out, feedback_control=shared)
    torch.cuda.synchronize()
    got = _u32(fcd)
    want = fc.copy()
    for r in range(B):
        if r == 4:
            continue
        want[r, 9] = 1
    want[1, 2], want[1, 8] = S.STOP_REASON_CANCELLED, 2
    want[2, 2], want[2, 8] = S.STOP_REASON_EOS, 2
    want[5, 2], want[5, 8] = S.STOP_REASON_EOS, 2
    np.testing.assert_array_equal(got, want)
    sh = _u32(shared)
    assert sh[9] == B and sh[2] == 0 and sh[8] == 0
    smp.close()


# ---- device-side history append -------------------------------------------------


def _ring_append(hist, hlen, tokens, V):
    for r, t in enumerate(tokens):
        if t < V:
            hist[r, hlen[r] % hist.shape[1]] = t
            hlen[r] += 1


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_history_append_across_steps(dtype):
    """K consecutive steps with NERVE_BATCH_APPEND_HISTORY and stream control:
    each step against the oracle fed the history with every earlier token
    appended (the lists wrap, so the rows read the last H ids)."""
    torch, dev = _torch()
    _say(f"history append {dtype}")
    B, V, H, K = 8, 32000, 24, 5
    rng = np.random.default_rng(21)
    x = rng.normal(0, 2.5, size=(B, V)).astype(np.float32)
    x[:, :64] += 6.0  # a small hot set, so appended tokens come back as candidates
    logits = workloads.to_bf16_bits(x) if dtype == "bf16" else x
    params = S.make_params(B, temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.3,
                           frequency_penalty=0.7, presence_penalty=0.4)
    params["method"][0] = S.METHOD_GREEDY
    hist = rng.integers(0, 64, size=(B, H)).astype(np.uint32)
    hlen = np.array([0, 3, 10, 20, 23, 24, 30, 47], np.uint32)
    seeds = rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32)
    smp = S.Sampler(V, B, dtype=dtype, top_k_capacity=64, history_capacity=H)
    hd, hld = to_dev(hist, dev, torch), to_dev(hlen, dev, torch)
    sc = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    sc[:, 1] = 100
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    pd = S.params_tensor(params, dev)
    lg = to_dev(logits, dev, torch)
    for k in range(K):
        ref = oracle.sample(logits, params, top_k_capacity=64, history=hist, history_len=hlen, seeds=seeds,
                            steps=np.full(B, 100 + k, np.uint64), rng=S.RNG_PHILOX, threads=8)
        smp.step(lg, pd, out, history=hd, history_len=hld, seeds=to_dev(seeds, dev, torch), rng=S.RNG_PHILOX,
                 stream_control=sc, flags=S.BATCH_APPEND_HISTORY)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_u32(out), ref["out"], err_msg=f"step {k}")
        _ring_append(hist, hlen, ref["token_id"], V)
        np.testing.assert_array_equal(_u32(hld), hlen, err_msg=f"history_len after step {k}")
        np.testing.assert_array_equal(_u32(hd), hist, err_msg=f"history after step {k}")
    assert (_u32(sc)[:, 1] == 100 + K).all()
    smp.close()


def test_seen_append_across_steps():
    """Set semantics: the sampled token's seen bit is set for the next step."""
    torch, dev = _torch()
    _say("seen append")
    B, V, K = 6, 5000, 4
    rng = np.random.default_rng(22)
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    x[:, :16] += 5.0
    params = S.make_params(B, temperature=1.0, top_k=8, repetition_penalty=1.5, presence_penalty=0.8)
    W = (V + 31) // 32
    seen = np.zeros((B, W), np.uint32)
    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=16)
    sd = to_dev(seen, dev, torch)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    pd, lg = S.params_tensor(params, dev), to_dev(x, dev, torch)
    for k in range(K):
        steps = np.full(B, k, np.uint64)
        ref = oracle.sample(x, params, top_k_capacity=16, seen=seen, steps=steps)
        smp.step(lg, pd, out, seen=sd, steps=to_dev(steps, dev, torch), flags=S.BATCH_APPEND_HISTORY)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_u32(out), ref["out"], err_msg=f"step {k}")
        for r, t in enumerate(ref["token_id"]):
            seen[r, t >> 5] |= np.uint32(1 << (int(t) & 31))
        np.testing.assert_array_equal(_u32(sd), seen, err_msg=f"seen after step {k}")
    smp.close()


# ---- per-lane prefixes (sample_lanes / sample_batch) ------------------------------


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_lane_prefixes_against_oracle(dtype):
    """Each row samples with the shared base bitmap plus its own prefix; the
    base bitmap is not modified."""
    torch, dev = _torch()
    _say(f"lane prefixes {dtype}")
    B, V = 12, 50257
    rng = np.random.default_rng(23)
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    x[:, :200] += 5.0
    logits = workloads.to_bf16_bits(x) if dtype == "bf16" else x
    W = (V + 31) // 32
    base = np.zeros(W, np.uint32)
    oracle.record_tokens(base, V, rng.integers(0, 200, 30))
    counts = np.array([0, 1, 2, 5, 9, 17, 33, 64, 64, 3, 0, 12], np.int32)
    P = 64
    ids = rng.integers(0, 200, size=(B, P)).astype(np.uint32)
    ids[7, 5] = V + 10  # out of range: ignored, like record_seen_tokens_batch64
    per_row = np.tile(base, (B, 1))
    for r in range(B):
        oracle.record_tokens(per_row[r], V, ids[r, : counts[r]])
    params = S.make_params(B, temperature=0.8, top_k=50, top_p=0.95, repetition_penalty=1.4, presence_penalty=0.6)
    steps = rng.integers(0, 2**40, B).astype(np.uint64)
    ref = oracle.sample(logits, params, top_k_capacity=64, seen=per_row, steps=steps, threads=8)
    smp = S.Sampler(V, B, dtype=dtype, top_k_capacity=64)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    based = to_dev(base[None], dev, torch)
    smp.step(to_dev(logits, dev, torch), S.params_tensor(params, dev), out, seen=based, seen_shared=True,
             prefix_ids=to_dev(ids, dev, torch), prefix_counts=to_dev(counts, dev, torch),
             steps=to_dev(steps, dev, torch))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u32(out), ref["out"])
    np.testing.assert_array_equal(_u32(based)[0], base)
    smp.close()


def test_sample_batch_convention():
    """prefix_counts null and stride 0: row r takes ids[..=r]; consecutive
    ticks from tick_base (sample_batch, batched_output_projection.rs:277-298)."""
    torch, dev = _torch()
    _say("sample_batch convention")
    B, V = 16, 32000
    rng = np.random.default_rng(24)
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    x[:, :100] += 4.0
    W = (V + 31) // 32
    base = np.zeros(W, np.uint32)
    oracle.record_tokens(base, V, [3, 7, 50])
    window = rng.integers(0, 100, B).astype(np.uint32)
    per_row = np.tile(base, (B, 1))
    for r in range(B):
        oracle.record_tokens(per_row[r], V, window[: r + 1])
    params = S.make_params(B, temperature=0.7, top_k=20, top_p=0.9, repetition_penalty=1.2, presence_penalty=0.5)
    tick0 = (1 << 32) - 5  # the carry into the high word happens inside the window
    steps = np.arange(B, dtype=np.uint64) + np.uint64(tick0)
    seeds = np.full(B, 0x9E3779B9, np.uint32)
    ref = oracle.sample(x, params, top_k_capacity=32, seen=per_row, steps=steps, seeds=seeds, threads=8)
    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=32)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    sc = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    smp.step(to_dev(x, dev, torch), S.params_tensor(params, dev), out, seen=to_dev(base[None], dev, torch),
             seen_shared=True, prefix_ids=to_dev(window, dev, torch), seeds=to_dev(seeds, dev, torch),
             stream_control=sc, flags=S.BATCH_CONSECUTIVE_TICKS, tick_base=tick0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u32(out), ref["out"])
    nxt = steps + np.uint64(1)
    scw = _u32(sc)
    np.testing.assert_array_equal(scw[:, 1], (nxt & np.uint64(0xFFFFFFFF)).astype(np.uint32))
    np.testing.assert_array_equal(scw[:, 0], ref["token_id"])
    smp.close()


def test_runner_sample_batch_matches_lanes():
    """SamplerRunner.sample_batch writes the runner's ring slots and returns the
    lane records; the reference's two-lane isolation is covered elsewhere."""
    torch, dev = _torch()
    _say("runner sample_batch")
    V = 4096
    spec = S.SamplerSpec(sampler_id="sampler", method="temperature_top_k_top_p", temperature=1.0, top_k=16,
                         top_p=1.0, repetition_penalty=2.0, top_k_capacity=16, logits_byte_capacity=V * 4,
                         scratch_byte_capacity=16 * 8)
    runner = S.SamplerRunner(spec, history_capacity_activations=8, random_seed=5, max_lanes=4)
    rng = np.random.default_rng(25)
    x = rng.normal(0, 1.0, size=(4, V)).astype(np.float32)
    x[:, :4] += 6.0
    runs = runner.sample_batch(torch.from_numpy(x).to(dev), [0, 1, 2, 3], start_stream_tick=10)
    W = (V + 31) // 32
    per_row = np.zeros((4, W), np.uint32)
    for r in range(4):
        oracle.record_tokens(per_row[r], V, list(range(r + 1)))
    params = oracle.make_params(4, temperature=1.0, top_k=16, top_p=1.0, repetition_penalty=2.0)
    ref = oracle.sample(x, params, top_k_capacity=16, seen=per_row, seeds=np.full(4, 5, np.uint32),
                        steps=np.arange(10, 14, dtype=np.uint64))
    assert [r.token_id for r in runs] == [int(t) for t in ref["token_id"]]
    for i, t in enumerate(range(10, 14)):
        assert runner.completed_run_at(t).token_id == runs[i].token_id
    runner.sampler.close()


# ---- consecutive full-size steps (the path the bench times) -------------------------


def test_c5_consecutive_steps_stream_control():
    """Three consecutive C5 steps at full size with Philox ticks taken from
    stream control (as bench.py runs them), each against the oracle."""
    torch, dev = _torch()
    _say("C5 consecutive steps")
    w = workloads.make("C5", seed=2024, step=0)
    B, V = w.batch, w.vocab
    smp = S.Sampler(V, B, dtype=w.dtype, top_k_capacity=w.top_k_capacity, history_capacity=w.history.shape[1])
    sc = torch.zeros((B, 5), dtype=torch.int32, device=dev)
    t0 = 977
    sc[:, 1] = t0
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    lg, pd = to_dev(w.logits, dev, torch), S.params_tensor(w.params, dev)
    hd, hld, sd = to_dev(w.history, dev, torch), to_dev(w.history_len, dev, torch), to_dev(w.seeds, dev, torch)
    for k in range(3):
        smp.step(lg, pd, out, history=hd, history_len=hld, seeds=sd, rng=w.rng, stream_control=sc)
        torch.cuda.synchronize()
        ref = oracle.sample(w.logits, w.params, top_k_capacity=w.top_k_capacity, history=w.history,
                            history_len=w.history_len, seeds=w.seeds, steps=np.full(B, t0 + k, np.uint64),
                            rng=w.rng, threads=16)
        bad = np.nonzero((_u32(out) != ref["out"]).any(axis=1))[0]
        assert bad.size == 0, f"step {k}: {bad.size} rows differ, first {bad[0]}"
    assert (_u32(sc)[:, 1] == t0 + 3).all()
    smp.close()


def test_batch_argument_errors():
    """The new batch fields are checked before any launch."""
    torch, dev = _torch()
    _say("batch argument errors")
    B, V = 70, 1000
    smp = S.Sampler(V, B, dtype="f32", top_k_capacity=8)
    x = torch.zeros((B, V), dtype=torch.float32, device=dev)
    params = S.params_tensor(S.make_params(B), dev)
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    ids = torch.zeros(B, dtype=torch.int32, device=dev)
    seen = torch.zeros((1, (V + 31) // 32), dtype=torch.int32, device=dev)
    fc = torch.zeros(12, dtype=torch.int32, device=dev)
    cases = [
        (dict(prefix_ids=ids), S.ERR_INVALID_ARGUMENT),                                   # prefix without seen
        (dict(seen=seen, seen_shared=True, prefix_ids=ids), S.ERR_TOKEN_BATCH_CAPACITY_EXCEEDED),  # [..=r] past 64
        (dict(flags=1 << 7), S.ERR_INVALID_ARGUMENT),                                    # unknown flag
        (dict(flags=S.BATCH_APPEND_HISTORY), S.ERR_INVALID_ARGUMENT),                    # nothing to append to
        (dict(stop_tokens=fc), S.ERR_INVALID_ARGUMENT),                                  # stop mask without a block
    ]
    for kw, code in cases:
        with pytest.raises(S.SamplerError) as e:
            smp.step(x, params, out, **kw)
        assert e.value.code == code, kw
    smp.close()
