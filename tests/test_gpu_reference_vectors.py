"""The reference's own sampler tests, run on the GPU through the C ABI with a
runner that mirrors VulkanResidentSamplerRunner
(runtime-rs/src/vulkan_stream_circuit/tests/component_transducer_sampler_tests.rs:317-984)."""
import json
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_sampler_tests.json")))


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _dev_logits(torch, V, fill, sparse):
    x = np.full(V, fill, np.float32)
    for t, v in sparse.items():
        x[int(t)] = v
    return torch.from_numpy(x).to("cuda:0")


def test_greedy_selects_largest_logit_and_carries_tick():
    import torch
    from llmoop_amd.sampler import SamplerRunner, SamplerSpec

    g = GOLDEN["greedy_selects_largest_logit"]
    _say("reference greedy")
    V = g["vocab_size"]
    spec = SamplerSpec(sampler_id="greedy_sampler", method="greedy", top_k=0, top_k_capacity=1,
                       logits_byte_capacity=V * 4)
    r = SamplerRunner(spec, history_capacity_activations=g["history_capacity"], random_seed=0)
    r.write_stream_control(0, g["stream_tick"], g["history_capacity"])
    run = r.run(_dev_logits(torch, V, g["fill"], g["sparse_logits"]))
    assert run.token_id == g["expected_token"]
    assert run.selected_logit_bits == g["expected_logit_bits"]
    assert run.control_flags == g["expected_flags"]
    assert list(r.read_output_bytes()) == g["expected_output_bytes"]
    words = r.stream_control_words()
    after = g["expected_stream_control_after"]
    assert words[:3] == [after["token"], after["tick_low"], after["tick_high"]]
    assert r.completed_run_at(g["stream_tick"]) == run


@pytest.mark.parametrize("case", ["top_k_4_equal_winners", "top_64_top_p_095"])
def test_equal_winner_sequences(case):
    import torch
    from llmoop_amd.sampler import SamplerRunner, SamplerSpec

    g = GOLDEN[case]
    _say(f"reference {case}")
    V = g["vocab_size"]
    spec = SamplerSpec(sampler_id="temperature_top_k_top_p_sampler", method="temperature_top_k_top_p",
                       temperature=g["temperature"], top_k=g["top_k"], top_p=g["top_p"],
                       top_k_capacity=g["top_k_capacity"], logits_byte_capacity=V * 4,
                       scratch_byte_capacity=4 * g["top_k"] * 8)
    r = SamplerRunner(spec, history_capacity_activations=32, random_seed=g["seed"])
    r.write_stream_control(0, 0, 32)
    logits = _dev_logits(torch, V, g["fill"], g["sparse_logits"])
    got = []
    for _ in g["ticks"]:
        run = r.run(logits)
        assert run.selected_logit_bits == g["expected_logit_bits"]
        assert run.control_flags == 1
        got.append(run.token_id)
    assert got == g["expected_tokens"]


def test_undersized_scratch_is_rejected():
    from llmoop_amd.sampler import SamplerError, SamplerSpec

    g = GOLDEN["top_k_4_equal_winners"]
    spec = SamplerSpec(sampler_id="x", method="temperature_top_k_top_p", top_k=4, top_k_capacity=4,
                       logits_byte_capacity=64 * 4, scratch_byte_capacity=4 * 4 * 8 - 8)
    with pytest.raises(SamplerError) as e:
        spec.validate(64 * 4, 32, 4)
    assert "invalid resident sampling spec" in str(e.value)


@pytest.mark.parametrize("case,runtime", [("repetition_penalty_sequence", False),
                                          ("presence_penalty_capture_restore", True)])
def test_penalty_sequences(case, runtime):
    import torch
    from llmoop_amd.sampler import SamplerRunner, SamplerSpec

    g = GOLDEN[case]
    _say(f"reference {case}")
    V = g["vocab_size"]
    spec = SamplerSpec(sampler_id="s", method="temperature_top_k_top_p", top_k=g["top_k"],
                       top_k_capacity=g["top_k_capacity"], runtime_parameterized=runtime,
                       repetition_penalty=g.get("repetition_penalty", 1.0),
                       presence_penalty=g.get("presence_penalty", 0.0), logits_byte_capacity=V * 4,
                       scratch_byte_capacity=4 * g["top_k_capacity"] * 8)
    r = SamplerRunner(spec, history_capacity_activations=32, random_seed=g["seed"])
    for i, step in enumerate(g["steps"]):
        if step.get("capture"):
            r.capture_token_state()
        if step.get("restore"):
            r.restore_token_state()
        if case == "repetition_penalty_sequence" and i == 3:
            # the reference writes 9 into stream-control word 0 and runs record_current_token
            r.write_stream_control(9, int(r.stream_control_words()[1]))
            r.record_current_token()
        elif step["record_before"]:
            r.record_input_tokens(step["record_before"])
        run = r.run(_dev_logits(torch, V, g["fill"], step["logits"]))
        assert run.token_id == step["expected_token"], (i, step)


def test_speculative_views_isolate_presence_state():
    import torch
    from llmoop_amd.sampler import SamplerRunner, SamplerSpec

    g = GOLDEN["speculative_views_isolate_presence_state"]
    _say("reference speculative views")
    V = g["vocab_size"]
    spec = SamplerSpec(sampler_id="runtime_sampler", method="temperature_top_k_top_p", top_k=g["top_k"],
                       top_k_capacity=g["top_k_capacity"], runtime_parameterized=True,
                       presence_penalty=g["presence_penalty"], logits_byte_capacity=V * 4,
                       scratch_byte_capacity=4 * g["top_k_capacity"] * 8)
    r = SamplerRunner(spec, history_capacity_activations=32, random_seed=7, max_lanes=2)
    r.record_input_tokens(g["runner_recorded"])
    lanes = g["lanes"]
    batched = torch.stack([_dev_logits(torch, V, g["fill"], lane["logits"]) for lane in lanes])
    runs = r.sample_lanes(batched, [l["prefix"] for l in lanes], [l["stream_tick"] for l in lanes])
    assert [x.token_id for x in runs] == [l["expected_token"] for l in lanes]
    for lane in lanes:
        assert r.completed_run_at(lane["stream_tick"]).token_id == lane["expected_token"]
    parent = r.run(_dev_logits(torch, V, g["fill"], g["parent_after"]["logits"]))
    assert parent.token_id == g["parent_after"]["expected_token"]


def test_record_tokens_rejects_oversized_batch():
    from llmoop_amd.sampler import SamplerError, SamplerRunner, SamplerSpec

    spec = SamplerSpec(sampler_id="s", method="temperature_top_k_top_p", top_k=1, top_k_capacity=1,
                       presence_penalty=1.0, logits_byte_capacity=64 * 4, scratch_byte_capacity=8)
    r = SamplerRunner(spec, history_capacity_activations=32, random_seed=1)
    with pytest.raises(SamplerError):
        r.record_input_tokens(list(range(65)))
    with pytest.raises(SamplerError):
        r.record_input_tokens([])
