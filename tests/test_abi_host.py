"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, and its host-only spec logic matches the reference runner
(sampler.rs:56-160, fixture_model_mount.rs:1-62)."""
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_sampler_tests.json")))


@pytest.fixture(scope="module")
def S():
    from llmoop_amd import sampler

    sampler.load_library()
    return sampler


def test_header_symbols_are_exported(S):
    header = open(os.path.join(ROOT, "include", "nerve_sampler.h")).read()
    declared = set(re.findall(r"^\s*(?:int|uint32_t|const char \*)\s*(nerve_\w+)\s*\(", header, re.M))
    assert declared, "no declarations parsed"
    assert declared == set(S.EXPORTED_SYMBOLS)
    lib = S.load_library()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.nerve_sampler_abi_version() == 2


def test_ctypes_structs_match_the_header(S, tmp_path):
    """The Python binding's struct layouts equal the C header's (offsets from a
    host program compiled against include/nerve_sampler.h)."""
    import ctypes
    import subprocess

    structs = {"nerve_sampler_batch": S._Batch, "nerve_sampler_desc": S._Desc,
               "nerve_sampler_spec": S._Spec, "nerve_sampler_runtime_config": S._RuntimeConfig}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "nerve_sampler.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, value = line.split()
        got[(cname, field)] = int(value)
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for fname, _ in cls._fields_:
            assert got[(cname, fname)] == getattr(cls, fname).offset, (cname, fname)


def test_runtime_override_promotes_greedy(S):
    g = GOLDEN["runtime_override_promotes_greedy"]
    compiled = S.SamplerSpec(**g["compiled"], logits_byte_capacity=128, scratch_byte_capacity=128 * 256 * 8)
    sampled = S.RuntimeConfig(**g["sampled_override"]).apply_to(compiled)
    exp = g["expected_sampled"]
    assert sampled.method == exp["method"]
    assert sampled.sampler_id == exp["sampler_id"]
    for name in ("temperature", "top_p", "min_p", "presence_penalty", "repetition_penalty"):
        assert sampled.__dict__[name] == pytest.approx(exp[name], rel=0, abs=0) or \
            abs(sampled.__dict__[name] - exp[name]) < 1e-7
    assert sampled.top_k == exp["top_k"]
    assert sampled.runtime_parameterized
    assert S.kernel_role_matches("runtime_partition_top_k", True, sampled.method)
    assert not S.kernel_role_matches("runtime_sample_logits", True, sampled.method)

    greedy = S.RuntimeConfig(**g["penalized_greedy_override"]).apply_to(compiled)
    assert greedy.method == g["expected_penalized_greedy_method"]
    assert S.kernel_role_matches("runtime_sample_logits", True, greedy.method)

    with pytest.raises(S.SamplerError) as e:
        S.RuntimeConfig(**g["invalid_override"]).apply_to(compiled)
    assert g["expected_error_contains"] in str(e.value)
    assert e.value.code == S.ERR_UNSUPPORTED_RUNTIME_SAMPLING_OVERRIDE


def test_promotion_defaults_and_empty_override(S):
    compiled = S.SamplerSpec(top_k_capacity=32, logits_byte_capacity=128)
    assert S.RuntimeConfig().apply_to(compiled) == compiled
    promoted = S.RuntimeConfig(temperature=0.5).apply_to(compiled)
    assert (promoted.top_k, promoted.top_p, promoted.min_p) == (32, 1.0, 0.0)
    big = S.SamplerSpec(top_k_capacity=256, logits_byte_capacity=128)
    assert S.RuntimeConfig(top_p=0.5).apply_to(big).top_k == 50


@pytest.mark.parametrize(
    "override",
    [
        {"temperature": 0.0},
        {"temperature": float("inf")},
        {"top_k": 0},
        {"top_p": 0.0},
        {"top_p": 1.5},
        {"min_p": -0.1},
        {"min_p": 1.01},
        {"repetition_penalty": 0.0},
        {"presence_penalty": float("nan")},
    ],
)
def test_invalid_overrides_rejected(S, override):
    compiled = S.SamplerSpec(method="temperature_top_k_top_p", top_k=5, top_k_capacity=64,
                             logits_byte_capacity=4096)
    with pytest.raises(S.SamplerError):
        S.RuntimeConfig(**override).apply_to(compiled)


def test_greedy_rejects_min_p_override(S):
    compiled = S.SamplerSpec(logits_byte_capacity=128)
    with pytest.raises(S.SamplerError):
        S.RuntimeConfig(min_p=0.1, presence_penalty=0.0).apply_to(
            S.SamplerSpec(method="greedy", top_k_capacity=0, logits_byte_capacity=128))
    assert S.RuntimeConfig(presence_penalty=0.25).apply_to(compiled).method == "greedy"


def test_validate_spec(S):
    spec = S.SamplerSpec(method="temperature_top_k_top_p", top_k=4, top_k_capacity=4, logits_byte_capacity=256,
                         scratch_byte_capacity=4 * 4 * 8)
    spec.validate(256, 32, 4)
    with pytest.raises(S.SamplerError) as e:
        S.SamplerSpec(**{**spec.__dict__, "scratch_byte_capacity": 4 * 4 * 8 - 8}).validate(256, 32, 4)
    assert "invalid resident sampling spec" in str(e.value)
    with pytest.raises(S.SamplerError) as e:
        spec.validate(128, 32, 4)
    assert e.value.code == S.ERR_INVALID_LOGITS_BYTE_CAPACITY
    with pytest.raises(S.SamplerError) as e:
        spec.validate(256, 0, 4)
    assert e.value.code == S.ERR_ZERO_HISTORY_CAPACITY


def test_create_without_gpu_fails_cleanly(S):
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(S.SamplerError) as e:
        S.Sampler(1000, 4)
    assert e.value.code in (S.ERR_HIP, S.ERR_INVALID_ARGUMENT)


def test_fused_entry_points_reject_bad_arguments(S):
    """The LM-head projection, the tile records and the tile step check their
    arguments before any device call (placeholder pointers are never touched)."""
    lib = S.load_library()
    P = 0x1000  # 16-byte aligned placeholder
    bad = [
        # input_size not a multiple of 64
        lambda: lib.nerve_lm_head_project(P, 100, P, 100, 4, 100, 1000, 1.0, P, 1000, None, 0, None),
        # stride below input_size
        lambda: lib.nerve_lm_head_project(P, 32, P, 64, 4, 64, 1000, 1.0, P, 1000, None, 0, None),
        # misaligned frames
        lambda: lib.nerve_lm_head_project(P + 2, 64, P, 64, 4, 64, 1000, 1.0, P, 1000, None, 0, None),
        # logits stride below the vocabulary
        lambda: lib.nerve_lm_head_project(P, 64, P, 64, 4, 64, 1000, 1.0, P, 999, None, 0, None),
        # tile stride below ceil(V/64)
        lambda: lib.nerve_lm_head_project(P, 64, P, 64, 4, 64, 1000, 1.0, P, 1000, P, 15, None),
        # non-finite scale
        lambda: lib.nerve_lm_head_project(P, 64, P, 64, 4, 64, 1000, float("inf"), P, 1000, None, 0, None),
        # tile records: unknown dtype, short stride, misaligned records
        lambda: lib.nerve_tile_records(P, 7, 1000, 4, 1000, P, 16, None),
        lambda: lib.nerve_tile_records(P, 0, 1000, 4, 1000, P, 15, None),
        lambda: lib.nerve_tile_records(P, 0, 1000, 4, 1000, P + 4, 16, None),
        # tile step without records
        lambda: lib.nerve_sampler_step_tiles(P, P, None, 16, None),
    ]
    for i, call in enumerate(bad):
        rc = call()
        assert rc != S.NERVE_OK, f"case {i} accepted"
        assert lib.nerve_sampler_last_error(), f"case {i} left no message"
    # nothing to do: empty batches succeed without touching the device
    assert lib.nerve_lm_head_project(None, 0, None, 0, 0, 64, 1000, 1.0, None, 0, None, 0, None) == S.NERVE_OK
    assert lib.nerve_tile_records(None, 0, 0, 0, 1000, None, 0, None) == S.NERVE_OK
