"""Seeded synthetic inputs of the five benchmark configurations.

C1..C5 follow the configuration list that the benchmark is quoted on:
  C1 greedy argmax, B=1, V=32000, f32 ~ N(0, 2.0), one random index +8.0
  C2 T=0.8, top-k 40, Philox draw, B=32, V=32000, f32 ~ N(0, 3.0), 5 spikes/row ~ U(6, 12)
  C3 rep 1.1 + freq 0.5 + presence 0.3 over a 512-id history ~ U[0, V), T=0.7, top-k 50,
     top-p 0.9, Philox; B=64, V=151936, bf16 ~ N(0, 2.5)
  C4 C3's chain plus a packed allowed-token mask (contiguous spans covering 2% of V at random
     offsets plus 200 scattered ids); B=128, V=128256, f32 ~ N(0, 2.5); some rows all-zero -> EOS 2
  C5 B=256, V=151936, bf16 ~ Student-t(df=4) * 2.0, 2048-id history, full penalty chain,
     top-k 50, top-p 0.9, T ~ U[0.5, 1.2] per row, Philox, consecutive steps
  C5P C5 with each row's 2048 history ids drawn from that row's own 200 largest raw logits:
     the penalties push the row's top tokens below the others (a decode row repeating itself)
Logits are returned as float32 or as uint16 arrays holding bf16 bits
(round-to-nearest-even from float32).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .sampler import METHOD_GREEDY, METHOD_TEMPERATURE_TOP_K_TOP_P, RNG_PHILOX, ROW_PARAMS


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


@dataclass
class Workload:
    name: str
    vocab: int
    batch: int
    dtype: str                       # "f32" | "bf16"
    logits: np.ndarray               # [B, V] float32 or uint16 (bf16 bits)
    params: np.ndarray               # [B] ROW_PARAMS
    top_k_capacity: int
    rng: int
    seeds: np.ndarray                # [B] uint32
    steps: np.ndarray                # [B] uint64
    history: np.ndarray | None = None
    history_len: np.ndarray | None = None
    allowed: np.ndarray | None = None
    eos_token_id: int = 2
    description: str = ""
    extra: dict = field(default_factory=dict)

    def algorithmic_bytes(self) -> int:
        """Once-through HBM bytes of one step: logits, history ids, mask words,
        per-row T/seed/step and the 12-byte output (see the bench's roofline)."""
        esize = 4 if self.dtype == "f32" else 2
        per_row = self.vocab * esize + 4 + 4 + 8 + 12
        if self.history is not None:
            per_row += 4 * self.history.shape[1]
        if self.allowed is not None:
            per_row += 4 * ((self.vocab + 31) // 32)
        return per_row * self.batch


def _params(B, **kw):
    p = np.zeros(B, dtype=ROW_PARAMS)
    p["method"] = METHOD_TEMPERATURE_TOP_K_TOP_P
    p["temperature"] = 1.0
    p["top_k"] = 1
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    for k, v in kw.items():
        p[k] = v
    return p


def _mask(rng, B, V, empty_rows):
    W = (V + 31) // 32
    bits = np.zeros((B, V), dtype=bool)
    span_total = int(0.02 * V)
    for r in range(B):
        left = span_total
        while left > 0:
            n = int(min(left, rng.integers(64, 1024)))
            off = int(rng.integers(0, V - n))
            bits[r, off:off + n] = True
            left -= n
        bits[r, rng.integers(0, V, 200)] = True
    bits[empty_rows] = False
    padded = np.zeros((B, W * 32), dtype=bool)
    padded[:, :V] = bits
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    w = (padded.reshape(B, W, 32).astype(np.uint64) * weights).sum(axis=2)
    return w.astype(np.uint32)


def make(name: str, seed: int = 1234, step: int = 0, batch: int | None = None, input_size: int = 4096) -> Workload:
    rng = np.random.default_rng(seed)
    name = name.upper()
    if name == "L5":
        # C5's sampling settings on logits from an LM-head projection: frames
        # [B, input_size] bf16 ~ N(0, 1), weight [V, input_size] bf16 ~ N(0, 0.04^2),
        # made on the device by lm_head_inputs(); float32 logits, std ~ 0.04 sqrt(input_size)
        w = make("C5", seed=seed, step=step, batch=batch)
        w.name = "L5"
        w.dtype = "f32"
        w.logits = None
        w.extra.update(input_size=input_size, scale=1.0, seed=seed)
        w.description = (f"LM head + step: B={w.batch}, input_size={input_size}, V={w.vocab}, bf16 frames and weight, "
                         "f32 logits, C5's penalties and sampling")
        return w
    if name == "C1":
        B, V = batch or 1, 32000
        x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
        x[np.arange(B), rng.integers(0, V, B)] += 8.0
        return Workload("C1", V, B, "f32", x, _params(B, method=METHOD_GREEDY), 1, RNG_PHILOX,
                        rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32), np.full(B, step, np.uint64),
                        description="greedy argmax, B=1, V=32000, f32")
    if name == "C2":
        B, V = batch or 32, 32000
        x = (rng.standard_normal((B, V)) * 3.0).astype(np.float32)
        for r in range(B):
            x[r, rng.integers(0, V, 5)] = rng.uniform(6, 12, 5)
        return Workload("C2", V, B, "f32", x, _params(B, temperature=0.8, top_k=40), 40, RNG_PHILOX,
                        rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32), np.full(B, step, np.uint64),
                        description="T=0.8, top-k 40, Philox, B=32, V=32000, f32")
    if name in ("C3", "C4"):
        if name == "C3":
            B, V, dtype = batch or 64, 151936, "bf16"
        else:
            B, V, dtype = batch or 128, 128256, "f32"
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
        H = 512
        hist = rng.integers(0, V, (B, H)).astype(np.uint32)
        p = _params(B, temperature=0.7, top_k=50, top_p=0.9, repetition_penalty=1.1, frequency_penalty=0.5,
                    presence_penalty=0.3)
        w = Workload(name, V, B, dtype, x if dtype == "f32" else to_bf16_bits(x), p, 64, RNG_PHILOX,
                     rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32), np.full(B, step, np.uint64),
                     history=hist, history_len=np.full(B, H, np.uint32))
        if name == "C4":
            empty = [r for r in range(B) if r % 16 == 5]
            w.allowed = _mask(rng, B, V, empty)
            w.extra["empty_rows"] = empty
            w.description = "full chain + allowed mask, B=128, V=128256, f32, H=512"
        else:
            w.description = "full chain, B=64, V=151936, bf16, H=512"
        return w
    if name in ("C5", "C5P"):
        B, V = batch or 256, 151936
        x = (rng.standard_t(4, size=(B, V)) * 2.0).astype(np.float32)
        H = 2048
        hist = rng.integers(0, V, (B, H)).astype(np.uint32)
        if name == "C5P":
            top = np.argpartition(-x, 200, axis=1)[:, :200]
            hist = np.take_along_axis(top, rng.integers(0, 200, (B, H)), axis=1).astype(np.uint32)
        p = _params(B, temperature=rng.uniform(0.5, 1.2, B).astype(np.float32), top_k=50, top_p=0.9,
                    repetition_penalty=1.1, frequency_penalty=0.5, presence_penalty=0.3)
        return Workload(name, V, B, "bf16", to_bf16_bits(x), p, 64, RNG_PHILOX,
                        rng.integers(0, 2**32, B, dtype=np.uint64).astype(np.uint32), np.full(B, step, np.uint64),
                        history=hist, history_len=np.full(B, H, np.uint32),
                        description="large-batch decode: B=256, V=151936, bf16 Student-t, H=2048, per-row T"
                        + (", history from each row's own top 200" if name == "C5P" else ""))
    raise ValueError(f"unknown workload {name}")


def lm_head_inputs(w: Workload, device):
    """Seeded bf16 frames [B, D] and weight [V, D] of an L5 workload, made on the device."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(w.extra["seed"]))
    D = int(w.extra["input_size"])
    frames = torch.randn((w.batch, D), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)
    weight = torch.empty((w.vocab, D), device=device, dtype=torch.bfloat16)
    for v0 in range(0, w.vocab, 16384):  # in chunks: the float32 staging stays small
        v1 = min(w.vocab, v0 + 16384)
        weight[v0:v1] = (torch.randn((v1 - v0, D), generator=g, device=device) * 0.04).to(torch.bfloat16)
    return frames, weight
