"""Shared helpers of the GPU parity tests: run one batch through the C ABI
(libnerve_sampler.so via llmoop_amd.sampler) and through the CPU oracle on
the same numpy inputs, and compare."""
from __future__ import annotations

import numpy as np

from llmoop_amd import sampler as S


def to_dev(a, dev, torch):
    if a is None:
        return None
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a.copy()).to(dev)


def run_gpu(logits, params, *, top_k_capacity, history=None, history_len=None, seen=None, allowed=None,
            seeds=None, steps=None, rng=S.RNG_REFERENCE_HASH, eos_token_id=2, slices_per_row=0, sampler=None,
            vocab=None, tiles=False, prefix_ids=None, prefix_counts=None):
    import torch

    dev = torch.device("cuda:0")
    B, stride = logits.shape
    V = stride if vocab is None else vocab
    dtype = "bf16" if logits.dtype == np.uint16 else "f32"
    H = 0 if history is None else history.shape[1]
    own = sampler is None
    if own:
        sampler = S.Sampler(V, B, dtype=dtype, top_k_capacity=top_k_capacity, history_capacity=max(H, 0),
                            slices_per_row=slices_per_row)
    lg = to_dev(logits, dev, torch)
    seeds = np.zeros(B, np.uint32) if seeds is None else seeds
    steps = np.zeros(B, np.uint64) if steps is None else steps
    out = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    kcap = top_k_capacity
    tid = torch.zeros((B, kcap), dtype=torch.int32, device=dev)
    tlg = torch.zeros((B, kcap), dtype=torch.float32, device=dev)
    tpr = torch.zeros((B, kcap), dtype=torch.float32, device=dev)
    if history is not None and history_len is None:
        history_len = np.full(B, H, np.uint32)
    kw = {}
    if tiles:
        # the tile records of these logits (as the projection's epilogue writes them), then the tile step
        rec = torch.full((B, 2 * S.tile_count(V) + 2), -1, dtype=torch.int32, device=dev)
        S.tile_records(lg, rec, vocab=V)
        kw["tile_records"] = rec
    if prefix_ids is not None:
        kw["prefix_ids"] = to_dev(prefix_ids, dev, torch)
        kw["prefix_counts"] = to_dev(prefix_counts, dev, torch)
    sampler.step(lg, S.params_tensor(params, dev), out, **kw, history=to_dev(history, dev, torch),
                 history_len=to_dev(history_len, dev, torch), seen=to_dev(seen, dev, torch),
                 allowed=to_dev(allowed, dev, torch), eos_token_id=eos_token_id, seeds=to_dev(seeds, dev, torch),
                 steps=to_dev(steps, dev, torch), rng=rng, topk_ids=tid, topk_logits=tlg, topk_probs=tpr)
    torch.cuda.synchronize()
    o = out.cpu().numpy().view(np.uint32)
    res = {
        "out": o,
        "token_id": o[:, 0].copy(),
        "selected_logit_bits": o[:, 1].copy(),
        "flags": o[:, 2].copy(),
        "topk_ids": tid.cpu().numpy().view(np.uint32),
        "topk_logits": tlg.cpu().numpy(),
        "topk_probs": tpr.cpu().numpy(),
    }
    if own:
        sampler.close()
    return res


def assert_parity(gpu, ref, params, *, label="", prob_rtol=1e-5):
    """Bit-exact token ids, records and survivor sets; probabilities within prob_rtol."""
    B = gpu["out"].shape[0]
    bad = np.nonzero((gpu["out"] != ref["out"]).any(axis=1))[0]
    assert bad.size == 0, (
        f"{label}: {bad.size}/{B} rows differ; first row {bad[0]}: gpu {gpu['out'][bad[0]].tolist()} "
        f"oracle {ref['out'][bad[0]].tolist()} params {params[bad[0]]}"
    )
    np.testing.assert_array_equal(gpu["topk_ids"], ref["topk_ids"], err_msg=f"{label}: survivor ids")
    np.testing.assert_array_equal(gpu["topk_logits"].view(np.uint32), ref["topk_logits"].view(np.uint32),
                                  err_msg=f"{label}: survivor logits")
    np.testing.assert_allclose(gpu["topk_probs"], ref["topk_probs"], rtol=prob_rtol, atol=0,
                               err_msg=f"{label}: post-filter probabilities")
