"""Writes tests/golden/reference_sampler_tests.json.

The fixture restates, as data, the inputs and expected results of the
reference's own sampler tests. Expected values come from the formulas and
literals written in those tests, not from any sampler implementation:

  runtime-rs/src/vulkan_stream_circuit/tests/component_transducer_sampler_tests.rs
    resident_greedy_sampler_selects_largest_logit                       (317-406)
    resident_temperature_top_k_top_p_sampler_matches_explicit_random_signal (409-533)
    resident_repetition_sampler_tracks_prompt_and_feedback_tokens_on_gpu    (536-643)
    resident_runtime_sampler_applies_presence_penalty_from_gpu_state        (646-750)
    speculative_sampler_views_isolate_hypothetical_presence_state           (753-877)
    resident_temperature_top_64_sampler_matches_explicit_random_signal      (880-984)
  runtime-rs/src/vulkan_stream_circuit/tests/fixture_model_mount.rs:1-62 (runtime override)

Run: python tests/golden/make_reference_vectors.py
"""
import json
import os
import struct


def test_hash_u32(v: int) -> int:
    # fixture_model_helpers.rs:679-686 (the tests' own copy of the shader hash)
    v &= 0xFFFFFFFF
    v ^= v >> 16
    v = (v * 0x7FEB352D) & 0xFFFFFFFF
    v ^= v >> 15
    v = (v * 0x846CA68B) & 0xFFFFFFFF
    v ^= v >> 16
    return v


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def main() -> None:
    cases = {}

    cases["greedy_selects_largest_logit"] = {
        "vocab_size": 65536,
        "fill": 0.0,
        "sparse_logits": {"7": 3.5, "1024": 9.25},
        "stream_tick": 0x0000_0007_FFFF_FFFF,
        "history_capacity": 8,
        "expected_token": 1024,
        "expected_logit_bits": f32_bits(9.25),
        "expected_flags": 0,
        "expected_output_bytes": [0x00, 0x04, 0x00, 0x00, 0x00, 0x00, 0x14, 0x41, 0, 0, 0, 0, 0, 0, 0, 0],
        "expected_stream_control_after": {"token": 1024, "tick_low": 0, "tick_high": 8},
    }

    seed = 0x5EED1234
    top = [7, 8, 19, 51]
    cases["top_k_4_equal_winners"] = {
        "vocab_size": 64,
        "fill": -100.0,
        "sparse_logits": {str(t): 2.0 for t in top},
        "temperature": 1.0,
        "top_k": 4,
        "top_p": 1.0,
        "top_k_capacity": 4,
        "seed": seed,
        "ticks": list(range(16)),
        "expected_tokens": [top[((test_hash_u32(seed ^ t) >> 8) * 4) >> 24] for t in range(16)],
        "expected_logit_bits": f32_bits(2.0),
        "expected_flags": 1,
    }

    cases["repetition_penalty_sequence"] = {
        "vocab_size": 64,
        "fill": -100.0,
        "repetition_penalty": 1.1,
        "top_k": 1,
        "top_k_capacity": 1,
        "seed": 7,
        "steps": [
            {"logits": {"7": 10.0, "8": 9.6}, "record_before": [], "expected_token": 7},
            {"logits": {"7": 10.0, "8": 9.6}, "record_before": [7], "expected_token": 8},
            {"logits": {"7": -1.0, "8": -1.05}, "record_before": [], "expected_token": 8},
            {"logits": {"9": 5.0, "10": 4.8}, "record_before": [9], "expected_token": 10},
        ],
    }

    cases["presence_penalty_capture_restore"] = {
        "vocab_size": 64,
        "fill": -100.0,
        "presence_penalty": 1.5,
        "top_k": 1,
        "top_k_capacity": 8,
        "seed": 7,
        "steps": [
            {"logits": {"7": 10.0, "8": 9.0}, "record_before": [], "expected_token": 7},
            {"logits": {"7": 10.0, "8": 9.0}, "record_before": [7], "expected_token": 8},
            {"logits": {"7": -1.0, "9": -1.25}, "record_before": [], "expected_token": 9},
            {"capture": True, "logits": {"11": 10.0, "12": 9.0}, "record_before": [11], "expected_token": 12},
            {"restore": True, "logits": {"11": 10.0, "12": 9.0}, "record_before": [], "expected_token": 11},
        ],
    }

    cases["speculative_views_isolate_presence_state"] = {
        "vocab_size": 64,
        "fill": -100.0,
        "presence_penalty": 1.5,
        "top_k": 1,
        "top_k_capacity": 8,
        "runner_recorded": [7],
        "lanes": [
            {"logits": {"8": 10.0, "11": 9.0}, "prefix": [8], "stream_tick": 0, "expected_token": 11},
            {"logits": {"10": 10.0, "12": 9.0}, "prefix": [9, 10], "stream_tick": 1, "expected_token": 12},
        ],
        "parent_after": {"logits": {"8": 10.0, "11": 9.0}, "expected_token": 8},
    }

    V = 262144
    k = 64
    seed = 46
    top64 = sorted((i * 4093 + 7) % V for i in range(k))
    cases["top_64_top_p_095"] = {
        "vocab_size": V,
        "fill": -100.0,
        "sparse_logits": {str(t): 2.0 for t in top64},
        "temperature": 1.0,
        "top_k": k,
        "top_p": 0.95,
        "top_k_capacity": k,
        "seed": seed,
        "ticks": list(range(16)),
        "nucleus": 61,
        "expected_tokens": [top64[((test_hash_u32(seed ^ t) >> 8) * 61) >> 24] for t in range(16)],
        "expected_logit_bits": f32_bits(2.0),
    }

    cases["runtime_override_promotes_greedy"] = {
        "compiled": {
            "sampler_id": "greedy_sampler",
            "method": "greedy",
            "temperature": 1.0,
            "top_k": 1,
            "top_p": 1.0,
            "min_p": 0.0,
            "presence_penalty": 0.0,
            "repetition_penalty": 1.0,
            "top_k_capacity": 256,
        },
        "sampled_override": {
            "temperature": 0.7,
            "top_k": 40,
            "top_p": 0.95,
            "min_p": 0.02,
            "presence_penalty": 0.5,
            "repetition_penalty": 1.1,
        },
        "expected_sampled": {
            "method": "temperature_top_k_top_p",
            "sampler_id": "runtime_temperature_top_k_top_p_sampler",
            "temperature": 0.7,
            "top_k": 40,
            "top_p": 0.95,
            "min_p": 0.02,
            "presence_penalty": 0.5,
            "repetition_penalty": 1.1,
            "runtime_parameterized": True,
        },
        "penalized_greedy_override": {"presence_penalty": 0.25},
        "expected_penalized_greedy_method": "greedy",
        "invalid_override": {"top_k": 257},
        "expected_error_contains": "capacity 256",
    }

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_sampler_tests.json")
    with open(path, "w") as f:
        json.dump(cases, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main()
