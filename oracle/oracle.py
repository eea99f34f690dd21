"""ctypes front end of the CPU oracle (oracle/nerve_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, where it is the checker (or the timed CPU
baseline), never the thing measured or shipped.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1
METHOD_GREEDY = 0
METHOD_TOP_K_TOP_P = 1
RNG_REFERENCE_HASH = 0
RNG_PHILOX = 1
FLAG_SAMPLED = 1
FLAG_EOS_FALLBACK = 2
PAD_ID = 0xFFFFFFFF

ROW_PARAMS = np.dtype(
    [
        ("method", "<u4"),
        ("temperature", "<f4"),
        ("top_k", "<u4"),
        ("top_p", "<f4"),
        ("min_p", "<f4"),
        ("repetition_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("presence_penalty", "<f4"),
    ]
)


class _Batch(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_uint32),
        ("vocab_size", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("top_k_capacity", ctypes.c_uint32),
        ("logits", ctypes.c_void_p),
        ("logits_row_stride", ctypes.c_uint64),
        ("params", ctypes.c_void_p),
        ("history", ctypes.c_void_p),
        ("history_len", ctypes.c_void_p),
        ("history_stride", ctypes.c_uint32),
        ("seen", ctypes.c_void_p),
        ("seen_stride", ctypes.c_uint32),
        ("allowed", ctypes.c_void_p),
        ("allowed_stride", ctypes.c_uint32),
        ("seeds", ctypes.c_void_p),
        ("steps", ctypes.c_void_p),
        ("rng", ctypes.c_uint32),
        ("eos_token_id", ctypes.c_uint32),
        ("out", ctypes.c_void_p),
        ("topk_ids", ctypes.c_void_p),
        ("topk_logits", ctypes.c_void_p),
        ("topk_probs", ctypes.c_void_p),
    ]


_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.nro_hash_u32.restype = ctypes.c_uint32
        _lib.nro_hash_u32.argtypes = [ctypes.c_uint32]
        _lib.nro_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib.nro_expf.restype = ctypes.c_float
        _lib.nro_expf.argtypes = [ctypes.c_float]
        _lib.nro_logf.restype = ctypes.c_float
        _lib.nro_logf.argtypes = [ctypes.c_float]
        _lib.nro_order_key.restype = ctypes.c_uint32
        _lib.nro_order_key.argtypes = [ctypes.c_float]
        _lib.nro_random_unit.restype = ctypes.c_float
        _lib.nro_random_unit.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32]
        _lib.nro_configured_logit.restype = ctypes.c_float
        _lib.nro_configured_logit.argtypes = [ctypes.c_float, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        _lib.nro_sample_batch.restype = ctypes.c_int
        _lib.nro_sample_batch.argtypes = [ctypes.POINTER(_Batch), ctypes.c_int]
        _lib.nro_sample_row_literal.restype = ctypes.c_int
        _lib.nro_sample_row_literal.argtypes = [ctypes.POINTER(_Batch), ctypes.c_uint32, ctypes.c_uint32]
        _lib.nro_record_tokens.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32]
    return _lib


def hash_u32(v: int) -> int:
    return int(lib().nro_hash_u32(v & 0xFFFFFFFF))


def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32))
    o = np.zeros(4, dtype=np.uint32)
    lib().nro_philox4x32_10(c.ctypes.data, k.ctypes.data, o.ctypes.data)
    return [int(x) for x in o]


def expf(x: float) -> float:
    return float(np.float32(lib().nro_expf(float(x))))


def logf(x: float) -> float:
    return float(np.float32(lib().nro_logf(float(x))))


def random_unit(rng: int, seed: int, step: int, row: int) -> float:
    return float(lib().nro_random_unit(rng, seed & 0xFFFFFFFF, step, row))


def record_tokens(seen: np.ndarray, vocab_size: int, ids) -> None:
    assert seen.dtype == np.uint32 and seen.flags.c_contiguous
    a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32))
    lib().nro_record_tokens(seen.ctypes.data, vocab_size, a.ctypes.data, len(a))


def make_params(batch: int, **kw) -> np.ndarray:
    p = np.zeros(batch, dtype=ROW_PARAMS)
    p["method"] = METHOD_TOP_K_TOP_P
    p["temperature"] = 1.0
    p["top_k"] = 1
    p["top_p"] = 1.0
    p["min_p"] = 0.0
    p["repetition_penalty"] = 1.0
    p["frequency_penalty"] = 0.0
    p["presence_penalty"] = 0.0
    for name, value in kw.items():
        p[name] = value
    return p


def _ptr(a):
    return None if a is None else a.ctypes.data


def sample(
    logits: np.ndarray,
    params: np.ndarray,
    *,
    top_k_capacity: int,
    vocab_size: int | None = None,
    history: np.ndarray | None = None,
    history_len: np.ndarray | None = None,
    seen: np.ndarray | None = None,
    allowed: np.ndarray | None = None,
    seeds: np.ndarray | None = None,
    steps: np.ndarray | None = None,
    rng: int = RNG_REFERENCE_HASH,
    eos_token_id: int = 2,
    threads: int = 1,
    literal_partitions: int = 0,
) -> dict:
    """Run the oracle on a [B, V] logits array (float32, or uint16 holding bf16 bits).

    literal_partitions > 0 runs the literal partition/merge restatement row by
    row with that many partitions instead of the fast path.
    """
    if logits.dtype == np.float32:
        dtype = DTYPE_F32
    elif logits.dtype == np.uint16:
        dtype = DTYPE_BF16
    else:
        raise TypeError("logits must be float32 or uint16 (bf16 bits)")
    logits = np.ascontiguousarray(logits)
    B, stride = logits.shape
    V = stride if vocab_size is None else vocab_size
    params = np.ascontiguousarray(params, dtype=ROW_PARAMS)
    assert params.shape == (B,)
    seeds = np.ascontiguousarray(np.zeros(B, np.uint32) if seeds is None else seeds, dtype=np.uint32)
    steps = np.ascontiguousarray(np.zeros(B, np.uint64) if steps is None else steps, dtype=np.uint64)
    b = _Batch()
    b.batch = B
    b.vocab_size = V
    b.dtype = dtype
    b.top_k_capacity = top_k_capacity
    b.logits = logits.ctypes.data
    b.logits_row_stride = stride
    b.params = params.ctypes.data
    keep = [logits, params, seeds, steps]
    if history is not None:
        history = np.ascontiguousarray(history, dtype=np.uint32)
        history_len = np.ascontiguousarray(
            np.full(B, history.shape[1], np.uint32) if history_len is None else history_len, dtype=np.uint32
        )
        b.history = history.ctypes.data
        b.history_len = history_len.ctypes.data
        b.history_stride = history.shape[1]
        keep += [history, history_len]
    if seen is not None:
        seen = np.ascontiguousarray(seen, dtype=np.uint32)
        b.seen = seen.ctypes.data
        b.seen_stride = seen.shape[1]
        keep.append(seen)
    if allowed is not None:
        allowed = np.ascontiguousarray(allowed, dtype=np.uint32)
        b.allowed = allowed.ctypes.data
        b.allowed_stride = allowed.shape[1]
        keep.append(allowed)
    b.seeds = seeds.ctypes.data
    b.steps = steps.ctypes.data
    b.rng = rng
    b.eos_token_id = eos_token_id
    out = np.zeros((B, 4), np.uint32)
    topk_ids = np.zeros((B, top_k_capacity), np.uint32)
    topk_logits = np.zeros((B, top_k_capacity), np.float32)
    topk_probs = np.zeros((B, top_k_capacity), np.float32)
    b.out = out.ctypes.data
    b.topk_ids = topk_ids.ctypes.data
    b.topk_logits = topk_logits.ctypes.data
    b.topk_probs = topk_probs.ctypes.data
    L = lib()
    if literal_partitions:
        for r in range(B):
            if L.nro_sample_row_literal(ctypes.byref(b), r, literal_partitions) != 0:
                raise RuntimeError("oracle literal path rejected the batch")
    else:
        if L.nro_sample_batch(ctypes.byref(b), threads) != 0:
            raise RuntimeError("oracle rejected the batch")
    del keep
    return {
        "token_id": out[:, 0].copy(),
        "selected_logit_bits": out[:, 1].copy(),
        "flags": out[:, 2].copy(),
        "out": out,
        "topk_ids": topk_ids,
        "topk_logits": topk_logits,
        "topk_probs": topk_probs,
    }
