"""GPU test of nerve_sampler_step_static_scratch, the entry point that
allocates nothing: its outputs equal nerve_sampler_step's on two calls in a
row (the second with a smaller batch), with rows split over several slices so
the static scratch array is the one used; larger needs are rejected, and a
handle created with NERVE_DESC_NO_SCRATCH (no device memory of its own) steps
through it."""
import numpy as np
import pytest

from llmoop_amd import sampler as S
from llmoop_amd import workloads
from tests.gpu_util import to_dev

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _case(B, V, seed, dtype):
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(4, size=(B, V)) * 2.0).astype(np.float32)
    logits = workloads.to_bf16_bits(x) if dtype == "bf16" else x
    params = S.make_params(B, temperature=rng.uniform(0.5, 1.2, B).astype(np.float32), top_k=50, top_p=0.9,
                           repetition_penalty=1.1, frequency_penalty=0.5, presence_penalty=0.3)
    params["method"][: B // 4] = S.METHOD_GREEDY
    H = 256
    hist = rng.integers(0, V, size=(B, H)).astype(np.uint32)
    seeds = rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32)
    steps = rng.integers(0, 2**40, B).astype(np.uint64)
    return logits, params, hist, seeds, steps


def _run(smp, entry, logits, params, hist, seeds, steps, kcap, torch, dev):
    B = logits.shape[0]
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    tid = torch.zeros((B, kcap), dtype=torch.int32, device=dev)
    tpr = torch.zeros((B, kcap), dtype=torch.float32, device=dev)
    hlen = np.full(B, hist.shape[1], np.uint32)
    smp.step(to_dev(logits, dev, torch), S.params_tensor(params, dev), out, history=to_dev(hist, dev, torch),
             history_len=to_dev(hlen, dev, torch), seeds=to_dev(seeds, dev, torch), steps=to_dev(steps, dev, torch),
             rng=S.RNG_PHILOX, topk_ids=tid, topk_probs=tpr, entry=entry)
    torch.cuda.synchronize()
    return out.cpu().numpy(), tid.cpu().numpy(), tpr.cpu().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_static_scratch_entry_matches_step(dtype):
    import torch

    dev = torch.device("cuda:0")
    V, kcap = 151936, 64
    smp = S.Sampler(V, 64, dtype=dtype, top_k_capacity=kcap, history_capacity=256, slices_per_row=3)
    assert smp.slices_per_row >= 3
    for call, B in enumerate((64, 23)):
        _say(f"static scratch {dtype} call {call} B={B}")
        args = _case(B, V, 100 + call, dtype)
        a = _run(smp, "nerve_sampler_step", *args, kcap, torch, dev)
        b = _run(smp, "nerve_sampler_step_static_scratch", *args, kcap, torch, dev)
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)
    smp.close()


def test_static_scratch_limits_and_no_scratch_handle():
    import torch

    dev = torch.device("cuda:0")
    V, kcap = 65536, 1024
    _say("static scratch limits")
    # 256 rows x 4 slices x 1024 entries x 8 bytes = 8 MiB > 4 MiB
    big = S.Sampler(V, 256, dtype="f32", top_k_capacity=kcap, slices_per_row=4)
    x = torch.zeros((256, V), dtype=torch.float32, device=dev)
    params = S.params_tensor(S.make_params(256, top_k=8), dev)
    out = torch.zeros((256, 4), dtype=torch.int32, device=dev)
    with pytest.raises(S.SamplerError) as e:
        big.step(x, params, out, entry="nerve_sampler_step_static_scratch")
    assert e.value.code == S.ERR_INVALID_ARGUMENT and "static array" in str(e.value)
    big.close()
    _say("no-scratch handle")
    B, V = 16, 100000
    ns = S.Sampler(V, B, dtype="f32", top_k_capacity=64, slices_per_row=2, flags=S.DESC_NO_SCRATCH)
    ref = S.Sampler(V, B, dtype="f32", top_k_capacity=64, slices_per_row=2)
    rng = np.random.default_rng(7)
    xs = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    params = S.params_tensor(S.make_params(B, top_k=40, top_p=0.9, temperature=0.8), dev)
    outs = []
    for smp, entry in ((ref, "nerve_sampler_step"), (ns, "nerve_sampler_step_static_scratch")):
        out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
        smp.step(torch.from_numpy(xs).to(dev), params, out, entry=entry)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    np.testing.assert_array_equal(outs[0], outs[1])
    with pytest.raises(S.SamplerError) as e:
        ns.step(torch.from_numpy(xs).to(dev), params, torch.zeros((B, 4), dtype=torch.int32, device=dev))
    assert "NERVE_DESC_NO_SCRATCH" in str(e.value)
    ns.close()
    ref.close()
