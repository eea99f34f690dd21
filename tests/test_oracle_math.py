"""Pins the oracle's arithmetic primitives (CPU only).

- hash_u32: the reference tests' helper (fixture_model_helpers.rs:679-686),
  checked through the expected token sequences written into the golden fixture
  and against an independent restatement here.
- Philox4x32-10: the Random123 known-answer vectors (Salmon et al., SC'11).
- exp/log: libm within 2 ulp over dense sweeps, plus exact special values.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_sampler_tests.json")


def _py_hash(v):
    v &= 0xFFFFFFFF
    v ^= v >> 16
    v = (v * 0x7FEB352D) & 0xFFFFFFFF
    v ^= v >> 15
    v = (v * 0x846CA68B) & 0xFFFFFFFF
    v ^= v >> 16
    return v


def test_hash_matches_reference_helper(oracle):
    rng = np.random.default_rng(1)
    for v in [0, 1, 0x5EED1234, 0xFFFFFFFF, *rng.integers(0, 2**32, 200, dtype=np.uint64).tolist()]:
        assert oracle.hash_u32(int(v)) == _py_hash(int(v))


def test_reference_hash_draw_reproduces_golden_index_formula(oracle):
    g = json.load(open(GOLDEN))["top_k_4_equal_winners"]
    top = [7, 8, 19, 51]
    for tick, expected in zip(g["ticks"], g["expected_tokens"]):
        u = oracle.random_unit(oracle.RNG_REFERENCE_HASH, g["seed"], tick, 0)
        assert top[int(np.floor(np.float32(u) * np.float32(4.0)))] == expected


@pytest.mark.parametrize(
    "ctr,key,expected",
    [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        (
            [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344],
            [0xA4093822, 0x299F31D0],
            [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1],
        ),
    ],
)
def test_philox_known_answers(oracle, ctr, key, expected):
    assert oracle.philox4x32_10(ctr, key) == expected


def _ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def test_exp_within_two_ulp_of_libm(oracle):
    xs = np.concatenate(
        [
            np.linspace(-87.0, 88.5, 20001, dtype=np.float32),
            np.linspace(-1.0, 1.0, 20001, dtype=np.float32),
            np.random.default_rng(3).uniform(-30, 0, 20000).astype(np.float32),
        ]
    )
    got = np.array([oracle.expf(float(x)) for x in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(got, want).max() <= 2


def test_exp_special_values(oracle):
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(-0.0) == 1.0
    assert oracle.expf(float("-inf")) == 0.0
    assert oracle.expf(float("inf")) == float("inf")
    assert np.isnan(oracle.expf(float("nan")))
    assert oracle.expf(89.0) == float("inf")
    assert oracle.expf(-104.0) == 0.0
    # subnormal results round once, like libm to within an ulp
    for x in [-90.0, -100.0, -103.0, -87.5]:
        got = np.float32(oracle.expf(x))
        want = np.float32(np.exp(np.float64(np.float32(x))))
        assert _ulp_diff(got, want) <= 1


def test_log_within_two_ulp_of_libm(oracle):
    xs = np.concatenate(
        [
            np.geomspace(1e-30, 1.0, 20000).astype(np.float32),
            np.linspace(0.5, 2.0, 5001, dtype=np.float32),
            np.array([1e-40, 1e-44, 3.4e38], np.float32),
        ]
    )
    got = np.array([oracle.logf(float(x)) for x in xs], np.float32)
    want = np.log(xs.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(got, want).max() <= 2
    assert oracle.logf(1.0) == 0.0


def test_order_key_is_monotone_and_merges_signed_zero(oracle):
    L = oracle.lib()
    vals = np.array([-np.inf, -3.4028235e38, -1.0, -1e-45, 0.0, 1e-45, 1.0, 3.4028235e38, np.inf], np.float32)
    keys = [L.nro_order_key(float(v)) for v in vals]
    assert keys == sorted(keys) and len(set(keys)) == len(keys)
    assert L.nro_order_key(-0.0) == L.nro_order_key(0.0)
    assert L.nro_order_key(float("nan")) == 0
