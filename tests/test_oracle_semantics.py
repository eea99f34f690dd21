"""Pins nro_sample_batch (CPU only): the reference's own sampler tests, the
literal partition/merge restatement, brute force on tiny vocabularies and
closed forms."""
import json
import os

import numpy as np
import pytest

from oracle.oracle import ROW_PARAMS

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_sampler_tests.json")))


def _logits(V, fill, sparse, B=1):
    x = np.full((B, V), fill, np.float32)
    for t, v in sparse.items():
        x[:, int(t)] = v
    return x


def test_reference_greedy_vector(oracle):
    g = GOLDEN["greedy_selects_largest_logit"]
    x = _logits(g["vocab_size"], g["fill"], g["sparse_logits"])
    p = oracle.make_params(1, method=oracle.METHOD_GREEDY)
    r = oracle.sample(x, p, top_k_capacity=1, steps=np.array([g["stream_tick"]], np.uint64))
    assert list(r["out"][0].view(np.uint8)) == g["expected_output_bytes"]


def _equal_winner_case(oracle, g, **kw):
    x = _logits(g["vocab_size"], g["fill"], g["sparse_logits"])
    p = oracle.make_params(1, temperature=g["temperature"], top_k=g["top_k"], top_p=g["top_p"])
    got = []
    for tick in g["ticks"]:
        r = oracle.sample(
            x,
            p,
            top_k_capacity=g["top_k_capacity"],
            seeds=np.array([g["seed"]], np.uint32),
            steps=np.array([tick], np.uint64),
            **kw,
        )
        assert r["selected_logit_bits"][0] == g["expected_logit_bits"]
        assert r["flags"][0] == 1
        got.append(int(r["token_id"][0]))
    assert got == g["expected_tokens"]


def test_reference_top_k_4_vector(oracle):
    _equal_winner_case(oracle, GOLDEN["top_k_4_equal_winners"])


def test_reference_top_k_4_vector_literal(oracle):
    _equal_winner_case(oracle, GOLDEN["top_k_4_equal_winners"], literal_partitions=4)


def test_reference_top_64_vector(oracle):
    _equal_winner_case(oracle, GOLDEN["top_64_top_p_095"])


def _penalty_sequence(oracle, g, literal=0):
    V = g["vocab_size"]
    seen = np.zeros((1, (V + 31) // 32), np.uint32)
    snapshot = None
    p = oracle.make_params(
        1,
        top_k=g["top_k"],
        repetition_penalty=g.get("repetition_penalty", 1.0),
        presence_penalty=g.get("presence_penalty", 0.0),
    )
    for step in g["steps"]:
        if step.get("capture"):
            snapshot = seen.copy()
        if step.get("restore"):
            seen[:] = snapshot
        oracle.record_tokens(seen[0], V, step["record_before"])
        x = _logits(V, g["fill"], step["logits"])
        r = oracle.sample(x, p, top_k_capacity=g["top_k_capacity"], seen=seen, literal_partitions=literal)
        assert int(r["token_id"][0]) == step["expected_token"], step


@pytest.mark.parametrize("literal", [0, 4])
def test_reference_repetition_sequence(oracle, literal):
    _penalty_sequence(oracle, GOLDEN["repetition_penalty_sequence"], literal)


@pytest.mark.parametrize("literal", [0, 4])
def test_reference_presence_capture_restore(oracle, literal):
    _penalty_sequence(oracle, GOLDEN["presence_penalty_capture_restore"], literal)


def test_reference_speculative_views(oracle):
    g = GOLDEN["speculative_views_isolate_presence_state"]
    V = g["vocab_size"]
    parent = np.zeros((V + 31) // 32, np.uint32)
    oracle.record_tokens(parent, V, g["runner_recorded"])
    p = oracle.make_params(2, top_k=g["top_k"], presence_penalty=g["presence_penalty"])
    seen = np.stack([parent.copy(), parent.copy()])
    x = np.zeros((2, V), np.float32)
    for i, lane in enumerate(g["lanes"]):
        oracle.record_tokens(seen[i], V, lane["prefix"])
        x[i] = _logits(V, g["fill"], lane["logits"])[0]
    r = oracle.sample(
        x, p, top_k_capacity=g["top_k_capacity"], seen=seen, steps=np.array([l["stream_tick"] for l in g["lanes"]], np.uint64)
    )
    assert list(r["token_id"]) == [l["expected_token"] for l in g["lanes"]]
    x0 = _logits(V, g["fill"], g["parent_after"]["logits"])
    r = oracle.sample(x0, p[:1], top_k_capacity=g["top_k_capacity"], seen=parent[None])
    assert int(r["token_id"][0]) == g["parent_after"]["expected_token"]


def _brute_topk(v, k):
    ids = [i for i in range(len(v)) if not np.isnan(v[i]) and v[i] != -np.inf]
    ids.sort(key=lambda i: (-float(v[i]), i))
    return ids[:k]


def _random_case(rng, B, V, kcap, with_hist=True, with_mask=False, dup_values=False, dtype=np.float32):
    if dup_values:
        x = rng.integers(-3, 3, size=(B, V)).astype(np.float32)
    else:
        x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    if dtype == np.uint16:
        x = (x.view(np.uint32) >> 16).astype(np.uint16)
    params = np.zeros(B, dtype=ROW_PARAMS)
    params["method"] = rng.integers(0, 2, B)
    params["temperature"] = rng.uniform(0.3, 1.5, B)
    params["top_k"] = rng.integers(1, kcap + 1, B)
    params["top_p"] = rng.uniform(0.2, 1.0, B)
    params["min_p"] = np.where(rng.random(B) < 0.5, 0.0, rng.uniform(0, 0.3, B))
    params["repetition_penalty"] = rng.uniform(0.8, 1.5, B)
    params["frequency_penalty"] = rng.uniform(0, 0.6, B)
    params["presence_penalty"] = rng.uniform(-0.5, 0.6, B)
    kw = {}
    if with_hist:
        H = 16
        kw["history"] = rng.integers(0, V + 3, size=(B, H)).astype(np.uint32)
        kw["history_len"] = rng.integers(0, H + 1, B).astype(np.uint32)
    if with_mask:
        W = (V + 31) // 32
        kw["allowed"] = rng.integers(0, 2**32, size=(B, W), dtype=np.uint64).astype(np.uint32)
        kw["allowed"][0] = 0
    kw["seeds"] = rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32)
    kw["steps"] = rng.integers(0, 2**40, B, dtype=np.uint64)
    return x, params, kw


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("rng_mode", [0, 1])
def test_fast_matches_literal_restatement(oracle, seed, rng_mode):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(3, 200))
    x, params, kw = _random_case(rng, 8, V, 16, with_mask=seed % 2 == 1, dup_values=seed % 3 == 0,
                                 dtype=np.uint16 if seed == 4 else np.float32)
    a = oracle.sample(x, params, top_k_capacity=16, rng=rng_mode, **kw)
    for G in (1, 3, 128):
        b = oracle.sample(x, params, top_k_capacity=16, rng=rng_mode, literal_partitions=G, **kw)
        for key in ("out", "topk_ids", "topk_logits", "topk_probs"):
            np.testing.assert_array_equal(a[key], b[key], err_msg=f"{key} G={G}")


@pytest.mark.parametrize("seed", range(4))
def test_topk_sets_match_brute_force(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    V = 97
    x, params, kw = _random_case(rng, 6, V, 12, with_hist=False, dup_values=seed % 2 == 0)
    x[0, 5] = np.nan
    x[1, :50] = -np.inf
    params["method"] = 1
    params["min_p"] = 0.0
    r = oracle.sample(x, params, top_k_capacity=12, **kw)
    for row in range(6):
        k = int(params["top_k"][row])
        ids = _brute_topk(x[row], k)
        got = [int(i) for i in r["topk_ids"][row][: len(ids)]]
        assert got == ids
        assert all(int(i) == oracle.PAD_ID for i in r["topk_ids"][row][len(ids):k])


def test_equal_weights_closed_form(oracle):
    # n equal winners, p = 1: the draw is floor(u * n) exactly.
    V, n = 300, 37
    ids = sorted(np.random.default_rng(7).choice(V, n, replace=False).tolist())
    x = np.full((1, V), -50.0, np.float32)
    x[0, ids] = 3.0
    p = oracle.make_params(1, top_k=n, temperature=0.9)
    for step in range(40):
        u = oracle.random_unit(oracle.RNG_PHILOX, 99, step, 0)
        r = oracle.sample(x, p, top_k_capacity=64, rng=oracle.RNG_PHILOX,
                          seeds=np.array([99], np.uint32), steps=np.array([step], np.uint64))
        assert int(r["token_id"][0]) == ids[int(np.floor(np.float64(u) * n))]
        probs = r["topk_probs"][0][:n]
        np.testing.assert_allclose(probs, 1.0 / n, rtol=1e-6)


def test_k_one_is_argmax_and_probs_sum_to_one(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 500)).astype(np.float32)
    p = oracle.make_params(16, top_k=1, temperature=0.5)
    r = oracle.sample(x, p, top_k_capacity=8)
    np.testing.assert_array_equal(r["token_id"], np.argmax(x, axis=1))
    p = oracle.make_params(16, top_k=8, top_p=0.7)
    r = oracle.sample(x, p, top_k_capacity=8)
    s = r["topk_probs"].sum(axis=1)
    np.testing.assert_allclose(s, 1.0, rtol=1e-6)


def test_min_p_cut_in_raw_logit_space(oracle):
    # weights at T=1: logits 0, -1, -2, -3; min_p = e^-1.5 keeps ranks 0 and 1 only.
    x = np.array([[0.0, -1.0, -2.0, -3.0] + [-100.0] * 4], np.float32)
    p = oracle.make_params(1, top_k=4, min_p=float(np.exp(-1.5)))
    r = oracle.sample(x, p, top_k_capacity=4)
    probs = r["topk_probs"][0]
    assert probs[2] == 0 and probs[3] == 0
    np.testing.assert_allclose(probs[:2], [1 / (1 + np.exp(-1)), np.exp(-1) / (1 + np.exp(-1))], rtol=1e-6)


def test_greedy_quirks(oracle):
    p = oracle.make_params(1, method=oracle.METHOD_GREEDY)
    # all -inf with V < 1024: the reference's padded lane V wins with LOWEST_FLOAT
    x = np.full((1, 10), -np.inf, np.float32)
    r = oracle.sample(x, p, top_k_capacity=1)
    assert int(r["token_id"][0]) == 10
    assert r["selected_logit_bits"][0] == np.float32(-3.4028234663852886e38).view(np.uint32)
    # a NaN as lane 0's first value persists through the tree
    x = np.zeros((1, 4096), np.float32)
    x[0, 0] = np.nan
    x[0, 77] = 5.0
    r = oracle.sample(x, p, top_k_capacity=1)
    assert int(r["token_id"][0]) == 0
    # a NaN later in a lane never wins
    x = np.zeros((1, 4096), np.float32)
    x[0, 1024 + 5] = np.nan
    x[0, 77] = 5.0
    r = oracle.sample(x, p, top_k_capacity=1)
    assert int(r["token_id"][0]) == 77
    # ties: smaller id
    x = np.zeros((1, 3000), np.float32)
    x[0, [2999, 1500, 40]] = 1.0
    assert int(oracle.sample(x, p, top_k_capacity=1)["token_id"][0]) == 40


def test_mask_all_zero_falls_back_to_eos(oracle):
    x = np.random.default_rng(0).standard_normal((3, 100)).astype(np.float32)
    allowed = np.full((3, 4), 0xFFFFFFFF, np.uint32)
    allowed[1] = 0
    allowed[2] = 0
    allowed[2, 3] = 0xFFFF0000  # bits beyond V=100 only: still empty
    p = oracle.make_params(3, top_k=5)
    r = oracle.sample(x, p, top_k_capacity=8, allowed=allowed, eos_token_id=2)
    assert list(r["token_id"][1:]) == [2, 2]
    assert list(r["flags"][1:]) == [3, 3]
    assert r["token_id"][0] != 2 or x[0].argmax() == 2


def test_frequency_penalty_counts_duplicates(oracle):
    x = np.zeros((1, 64), np.float32)
    x[0, 3] = 5.0
    x[0, 4] = 4.0
    p = oracle.make_params(1, top_k=1, frequency_penalty=0.4)
    # count(3) = 3: 5 - 1.2 = 3.8 < 4 -> 4 wins; with count 2: 4.2 > 4 -> 3 wins
    r = oracle.sample(x, p, top_k_capacity=1, history=np.array([[3, 3, 3, 9]], np.uint32))
    assert int(r["token_id"][0]) == 4
    r = oracle.sample(x, p, top_k_capacity=1, history=np.array([[3, 3, 9, 9]], np.uint32))
    assert int(r["token_id"][0]) == 3
    r = oracle.sample(x, p, top_k_capacity=1, history=np.array([[3, 3, 3, 9]], np.uint32),
                      history_len=np.array([2], np.uint32))
    assert int(r["token_id"][0]) == 3
