"""Python front end of libnerve_sampler.so (the gfx950 sampling stage).

Thin ctypes binding over the C ABI in include/nerve_sampler.h, plus a
`SamplerRunner` that mirrors the reference runner's per-stream surface
(run / record_input_tokens / capture_token_state / restore_token_state /
completed_run_at; runtime-rs/src/vulkan_stream_circuit/sampler.rs:748-873)
and `sample_lanes` (batched_output_projection.rs:316-371) on top of the one
batched launch. Device memory and streams come from PyTorch; all sampling
arithmetic runs in the HIP kernels. There is no CPU fallback: loading fails
loudly if the library is missing or the device is not gfx950.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# NERVE_SAMPLER_LIBRARY selects another build of the same library (for
# example one compiled with different launch parameters)
LIB_PATH = os.environ.get("NERVE_SAMPLER_LIBRARY") or os.path.join(HERE, "libnerve_sampler.so")

NERVE_OK = 0
ERR_INVALID_LOGITS_BYTE_CAPACITY = 1
ERR_ZERO_HISTORY_CAPACITY = 2
ERR_HISTORY_CAPACITY_OVERFLOW = 3
ERR_TOKEN_BATCH_CAPACITY_EXCEEDED = 4
ERR_INVALID_KERNEL_ROLE = 5
ERR_UNSUPPORTED_RUNTIME_SAMPLING_OVERRIDE = 6
ERR_INVALID_SAMPLING_SPEC = 7
ERR_HIP = 8
ERR_INVALID_ARGUMENT = 9
ERR_BATCH_CAPACITY_EXCEEDED = 10

DTYPE_F32 = 0
DTYPE_BF16 = 1
METHOD_GREEDY = 0
METHOD_TEMPERATURE_TOP_K_TOP_P = 1
RNG_REFERENCE_HASH = 0
RNG_PHILOX = 1
FLAG_SAMPLED = 1
FLAG_EOS_FALLBACK = 2
BATCH_APPEND_HISTORY = 1
BATCH_CONSECUTIVE_TICKS = 2
FEEDBACK_ENABLED = 1
FEEDBACK_CANCEL_REQUESTED = 2
STOP_REASON_NONE = 0
STOP_REASON_EOS = 1
STOP_REASON_CANCELLED = 2
FEEDBACK_HEADER_WORDS = 12
DESC_NO_SCRATCH = 1
TOKEN_BATCH_CAPACITY = 64
PAD_ID = 0xFFFFFFFF

METHOD_NAMES = {"greedy": METHOD_GREEDY, "temperature_top_k_top_p": METHOD_TEMPERATURE_TOP_K_TOP_P}

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


class SamplerError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"nerve sampler error {code}: {message}")
        self.code = code


class _Spec(ctypes.Structure):
    _fields_ = [
        ("sampler_id", ctypes.c_char * 64),
        ("method", ctypes.c_uint32),
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("top_k_capacity", ctypes.c_uint32),
        ("runtime_parameterized", ctypes.c_uint32),
        ("logits_byte_capacity", ctypes.c_uint64),
        ("output_byte_capacity", ctypes.c_uint64),
        ("scratch_byte_capacity", ctypes.c_uint64),
    ]


class _RuntimeConfig(ctypes.Structure):
    _fields_ = [
        ("has_temperature", ctypes.c_uint32),
        ("has_top_k", ctypes.c_uint32),
        ("has_top_p", ctypes.c_uint32),
        ("has_min_p", ctypes.c_uint32),
        ("has_presence_penalty", ctypes.c_uint32),
        ("has_repetition_penalty", ctypes.c_uint32),
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("presence_penalty", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
    ]


class _Desc(ctypes.Structure):
    _fields_ = [
        ("vocab_size", ctypes.c_uint32),
        ("max_batch", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("top_k_capacity", ctypes.c_uint32),
        ("history_capacity", ctypes.c_uint32),
        ("slices_per_row", ctypes.c_uint32),
        ("device", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
    ]


class _Batch(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_uint32),
        ("rng", ctypes.c_uint32),
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
        ("eos_token_id", ctypes.c_uint32),
        ("seeds", ctypes.c_void_p),
        ("steps", ctypes.c_void_p),
        ("stream_control", ctypes.c_void_p),
        ("output_ring", ctypes.c_void_p),
        ("ring_stride", ctypes.c_uint32),
        ("out", ctypes.c_void_p),
        ("topk_ids", ctypes.c_void_p),
        ("topk_logits", ctypes.c_void_p),
        ("topk_probs", ctypes.c_void_p),
        ("flags", ctypes.c_uint32),
        ("prefix_stride", ctypes.c_uint32),
        ("tick_base", ctypes.c_uint64),
        ("prefix_ids", ctypes.c_void_p),
        ("prefix_counts", ctypes.c_void_p),
        ("feedback_control", ctypes.c_void_p),
        ("stop_tokens", ctypes.c_void_p),
        ("feedback_stride", ctypes.c_uint32),
        ("stop_stride", ctypes.c_uint32),
    ]


EXPORTED_SYMBOLS = (
    "nerve_sampler_apply_runtime_config",
    "nerve_sampler_validate_spec",
    "nerve_sampler_kernel_role_matches",
    "nerve_sampler_create",
    "nerve_sampler_destroy",
    "nerve_sampler_step",
    "nerve_sampler_step_static_scratch",
    "nerve_sampler_record_tokens",
    "nerve_sampler_copy_token_state",
    "nerve_sampler_last_error",
    "nerve_sampler_abi_version",
    "nerve_sampler_slices_per_row",
    "nerve_sampler_step_tiles",
    "nerve_tile_records",
    "nerve_lm_head_project",
)

TILE_COLUMNS = 64  # vocabulary columns per tile record

_lib = None


def load_library() -> ctypes.CDLL:
    """Loads the in-tree library; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc, gfx950) first")
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    u32 = ctypes.c_uint32
    lib.nerve_sampler_apply_runtime_config.argtypes = [P, P, P, ctypes.c_char_p, ctypes.c_size_t]
    lib.nerve_sampler_validate_spec.argtypes = [P, ctypes.c_uint64, u32, u32]
    lib.nerve_sampler_kernel_role_matches.argtypes = [ctypes.c_char_p, u32, u32]
    lib.nerve_sampler_create.argtypes = [P, ctypes.POINTER(P)]
    lib.nerve_sampler_destroy.argtypes = [P]
    lib.nerve_sampler_step.argtypes = [P, P, P]
    lib.nerve_sampler_step_static_scratch.argtypes = [P, P, P]
    lib.nerve_sampler_record_tokens.argtypes = [P, P, u32, u32, P, u32, P, u32, P]
    lib.nerve_sampler_copy_token_state.argtypes = [P, P, P, u32, u32, P]
    lib.nerve_sampler_last_error.restype = ctypes.c_char_p
    lib.nerve_sampler_abi_version.restype = u32
    lib.nerve_sampler_slices_per_row.restype = u32
    lib.nerve_sampler_slices_per_row.argtypes = [P]
    lib.nerve_sampler_step_tiles.argtypes = [P, P, P, u32, P]
    lib.nerve_tile_records.argtypes = [P, u32, u32, u32, u32, P, u32, P]
    lib.nerve_lm_head_project.argtypes = [P, u32, P, u32, u32, u32, u32, ctypes.c_float, P, u32, P, u32, P]
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != NERVE_OK:
        msg = load_library().nerve_sampler_last_error().decode(errors="replace")
        raise SamplerError(rc, msg)


# ---- spec surface (host only) -------------------------------------------------


@dataclass
class SamplerSpec:
    """VulkanResidentSamplerSpec (sampler.rs:29-44)."""

    sampler_id: str = "greedy_sampler"
    method: str = "greedy"
    temperature: float = 1.0
    top_k: int = 1
    top_p: float = 1.0
    min_p: float = 0.0
    presence_penalty: float = 0.0
    repetition_penalty: float = 1.0
    top_k_capacity: int = 1
    runtime_parameterized: bool = False
    logits_byte_capacity: int = 0
    output_byte_capacity: int = 16
    scratch_byte_capacity: int = 0

    def _to_c(self) -> _Spec:
        s = _Spec()
        s.sampler_id = self.sampler_id.encode()[:63]
        s.method = METHOD_NAMES.get(self.method, 0xFFFFFFFF)
        for name in ("temperature", "top_k", "top_p", "min_p", "presence_penalty", "repetition_penalty",
                     "top_k_capacity", "logits_byte_capacity", "output_byte_capacity", "scratch_byte_capacity"):
            setattr(s, name, getattr(self, name))
        s.runtime_parameterized = int(self.runtime_parameterized)
        return s

    @staticmethod
    def _from_c(s: _Spec) -> "SamplerSpec":
        inv = {v: k for k, v in METHOD_NAMES.items()}
        return SamplerSpec(
            sampler_id=s.sampler_id.decode(),
            method=inv.get(s.method, "unknown"),
            temperature=s.temperature,
            top_k=s.top_k,
            top_p=s.top_p,
            min_p=s.min_p,
            presence_penalty=s.presence_penalty,
            repetition_penalty=s.repetition_penalty,
            top_k_capacity=s.top_k_capacity,
            runtime_parameterized=bool(s.runtime_parameterized),
            logits_byte_capacity=s.logits_byte_capacity,
            output_byte_capacity=s.output_byte_capacity,
            scratch_byte_capacity=s.scratch_byte_capacity,
        )

    def validate(self, logits_byte_capacity: int, history_capacity_activations: int, partition_count: int) -> None:
        """Construction-time checks (sampler.rs:259-382); raises SamplerError."""
        s = self._to_c()
        _check(load_library().nerve_sampler_validate_spec(ctypes.byref(s), logits_byte_capacity,
                                                          history_capacity_activations, partition_count))


@dataclass
class RuntimeConfig:
    """VulkanResidentSamplerRuntimeConfig (sampler.rs:46-54); None = not set."""

    temperature: float | None = None
    top_k: int | None = None
    top_p: float | None = None
    min_p: float | None = None
    presence_penalty: float | None = None
    repetition_penalty: float | None = None

    def apply_to(self, default: SamplerSpec) -> SamplerSpec:
        """sampler.rs:66-141 through the C ABI; raises SamplerError."""
        c = _RuntimeConfig()
        for name in ("temperature", "top_k", "top_p", "min_p", "presence_penalty", "repetition_penalty"):
            v = getattr(self, name)
            if v is not None:
                setattr(c, "has_" + name, 1)
                setattr(c, name, v)
        src = default._to_c()
        dst = _Spec()
        msg = ctypes.create_string_buffer(512)
        _check(load_library().nerve_sampler_apply_runtime_config(ctypes.byref(src), ctypes.byref(c), ctypes.byref(dst),
                                                                 msg, 512))
        return SamplerSpec._from_c(dst)


def kernel_role_matches(role: str, runtime_parameterized: bool, method: str) -> bool:
    return bool(load_library().nerve_sampler_kernel_role_matches(role.encode(), int(runtime_parameterized),
                                                                  METHOD_NAMES.get(method, 0xFFFFFFFF)))


# ---- device sampler -----------------------------------------------------------


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _rows(t):
    """A 2-D tensor with unit element stride and its row stride in elements
    (single-row tensors may carry any stride in dim 0, e.g. 0 after [None])."""
    if t is None:
        return None, 0
    if t.dim() != 2 or t.stride(1) != 1 or (t.shape[0] > 1 and t.stride(0) < t.shape[1]):
        t = t.contiguous()
    return t, (t.stride(0) if t.shape[0] > 1 else t.shape[1])


def _stream_arg(stream, device: int):
    """hipStream_t for a launch: the given handle, else torch's current stream
    on `device`, so launches order after the copies torch enqueued."""
    if stream is None:
        import torch

        stream = torch.cuda.current_stream(device).cuda_stream
    return ctypes.c_void_p(stream)


class Sampler:
    """One handle of the batched device sampler (nerve_sampler_create)."""

    def __init__(self, vocab_size: int, max_batch: int, *, dtype: str = "f32", top_k_capacity: int = 64,
                 history_capacity: int = 0, slices_per_row: int = 0, device: int = 0, flags: int = 0):
        lib = load_library()
        d = _Desc()
        d.vocab_size = vocab_size
        d.max_batch = max_batch
        d.dtype = DTYPE_BF16 if dtype == "bf16" else DTYPE_F32
        d.top_k_capacity = top_k_capacity
        d.history_capacity = history_capacity
        d.slices_per_row = slices_per_row
        d.device = device
        d.flags = flags
        h = ctypes.c_void_p()
        _check(lib.nerve_sampler_create(ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        self.vocab_size = vocab_size
        self.max_batch = max_batch
        self.dtype = dtype
        self.top_k_capacity = top_k_capacity
        self.history_capacity = history_capacity
        self.device = device

    @property
    def slices_per_row(self) -> int:
        return int(load_library().nerve_sampler_slices_per_row(self._h))

    def close(self) -> None:
        if getattr(self, "_h", None):
            load_library().nerve_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, logits, params, out, *, history=None, history_len=None, seen=None, allowed=None,
             eos_token_id: int = 2, seeds=None, steps=None, rng: int = RNG_REFERENCE_HASH, stream_control=None,
             output_ring=None, topk_ids=None, topk_logits=None, topk_probs=None, stream=None, flags: int = 0,
             tick_base: int = 0, seen_shared: bool = False, prefix_ids=None, prefix_counts=None,
             feedback_control=None, stop_tokens=None, entry: str = "nerve_sampler_step",
             tile_records=None) -> None:
        """Launches one step. All array arguments are torch tensors on the device:
        logits [B, stride] (float32, or bfloat16/int16 bits), params uint8 [B*32] holding ROW_PARAMS records,
        out int32 [B, 4], optional history int32 [B, H] + history_len int32 [B], seen / allowed int32 [B, W]
        (seen [1, W] with seen_shared: one bitmap for every row), seeds int32 [B], steps int64 [B],
        stream_control int32 [B, 5], output_ring int32 [B, R], topk_* [B, top_k_capacity];
        prefix_ids int32 [B, P] with prefix_counts int32 [B], or [n] without counts (row r takes ids[:r+1]);
        feedback_control int32 [B, F] or [F] (one block for every row), stop_tokens int32 [B, W] or [W].
        `entry` selects the C entry point (nerve_sampler_step or nerve_sampler_step_static_scratch);
        tile_records int32 [B, 2 * ceil(V/64) or more] (the projection's records of these logits)
        selects nerve_sampler_step_tiles."""
        b = _Batch()
        logits, lstride = _rows(logits)
        B = logits.shape[0]
        b.batch = B
        b.rng = rng
        b.logits = logits.data_ptr()
        b.logits_row_stride = lstride
        b.params = params.data_ptr()
        if history is not None:
            history, b.history_stride = _rows(history)
            b.history = history.data_ptr()
            b.history_len = history_len.data_ptr()
        if seen is not None:
            seen, b.seen_stride = _rows(seen)
            b.seen = seen.data_ptr()
            if seen_shared:
                b.seen_stride = 0
        if allowed is not None:
            allowed, b.allowed_stride = _rows(allowed)
            b.allowed = allowed.data_ptr()
        b.eos_token_id = eos_token_id
        b.seeds = _ptr(seeds)
        b.steps = _ptr(steps)
        b.stream_control = _ptr(stream_control)
        if output_ring is not None:
            if not output_ring.is_contiguous():
                raise ValueError("output_ring must be contiguous (it is written in place)")
            b.output_ring = output_ring.data_ptr()
            b.ring_stride = output_ring.shape[1]
        b.out = out.data_ptr()
        b.topk_ids = _ptr(topk_ids)
        b.topk_logits = _ptr(topk_logits)
        b.topk_probs = _ptr(topk_probs)
        b.flags = flags
        b.tick_base = tick_base
        if prefix_ids is not None:
            if prefix_ids.dim() == 1:
                b.prefix_stride = 0
            else:
                prefix_ids, b.prefix_stride = _rows(prefix_ids)
            b.prefix_ids = prefix_ids.data_ptr()
            b.prefix_counts = _ptr(prefix_counts)
        if feedback_control is not None:
            if not feedback_control.is_contiguous():
                raise ValueError("feedback_control must be contiguous (it is written in place)")
            b.feedback_control = feedback_control.data_ptr()
            b.feedback_stride = 0 if feedback_control.dim() == 1 else feedback_control.shape[1]
        if stop_tokens is not None:
            b.stop_tokens = stop_tokens.data_ptr()
            b.stop_stride = 0 if stop_tokens.dim() == 1 else _rows(stop_tokens)[1]
        if tile_records is not None:
            recs, rstride = _rows(tile_records)
            _check(load_library().nerve_sampler_step_tiles(self._h, ctypes.byref(b), recs.data_ptr(), rstride // 2,
                                                           _stream_arg(stream, self.device)))
            return
        _check(getattr(load_library(), entry)(self._h, ctypes.byref(b), _stream_arg(stream, self.device)))

    def record_tokens(self, seen, ids, counts, max_count: int, stream=None) -> None:
        """seen int32 [rows, W]; ids int32 [rows, n]; counts int32 [rows] (device)."""
        if not seen.is_contiguous():
            raise ValueError("seen must be contiguous (it is written in place)")
        ids, ids_stride = _rows(ids)
        s = _stream_arg(stream, self.device)
        _check(load_library().nerve_sampler_record_tokens(self._h, seen.data_ptr(), seen.shape[1], seen.shape[0],
                                                          ids.data_ptr(), ids_stride, counts.data_ptr(), max_count,
                                                          s))

    def copy_token_state(self, dst, src, stream=None) -> None:
        s = _stream_arg(stream, self.device)
        if not (dst.is_contiguous() and src.is_contiguous()) or dst.shape != src.shape:
            raise ValueError("token-state copies need contiguous tensors of one shape")
        _check(load_library().nerve_sampler_copy_token_state(self._h, dst.data_ptr(), src.data_ptr(), dst.shape[0],
                                                             dst.shape[1], s))


def params_tensor(params: np.ndarray, device):
    """ROW_PARAMS records -> uint8 device tensor."""
    import torch

    raw = np.ascontiguousarray(params, dtype=ROW_PARAMS).view(np.uint8)
    return torch.from_numpy(raw.copy()).to(device)


def make_params(batch: int, **kw) -> np.ndarray:
    p = np.zeros(batch, dtype=ROW_PARAMS)
    p["method"] = METHOD_TEMPERATURE_TOP_K_TOP_P
    p["temperature"] = 1.0
    p["top_k"] = 1
    p["top_p"] = 1.0
    p["repetition_penalty"] = 1.0
    for k, v in kw.items():
        p[k] = v
    return p


@dataclass
class SamplerRun:
    """VulkanResidentSamplerRun (sampler.rs:1221-1230)."""

    sampler_id: str
    token_id: int
    selected_logit_bits: int
    control_flags: int


@dataclass
class _RunnerState:
    seen: object = None
    snapshot: object = None
    stream_control: object = None
    ring: object = None


class SamplerRunner:
    """One decode stream over the batched sampler, with the reference runner's
    surface: run, record_input_tokens, capture/restore_token_state,
    completed_run_at, read_output_bytes (sampler.rs:748-873), and
    sample_lanes for B independent views over a [B, V] logits buffer
    (batched_output_projection.rs:316-371)."""

    def __init__(self, spec: SamplerSpec, *, history_capacity_activations: int, random_seed: int, device="cuda:0",
                 max_lanes: int = 1):
        import torch

        spec.validate(spec.logits_byte_capacity, history_capacity_activations, 1)
        self.torch = torch
        self.spec = spec
        self.device = torch.device(device)
        self.vocab_size = spec.logits_byte_capacity // 4
        self.history_capacity = history_capacity_activations
        self.seed = random_seed
        kcap = max(1, spec.top_k_capacity if spec.runtime_parameterized else max(spec.top_k, 1))
        self.kcap = kcap
        self.sampler = Sampler(self.vocab_size, max(1, max_lanes), dtype="f32", top_k_capacity=kcap,
                               device=self.device.index or 0)
        W = (self.vocab_size + 31) // 32
        self.words = W
        i32 = torch.int32
        self.seen = torch.zeros((1, W), dtype=i32, device=self.device)
        self.snapshot = torch.zeros((1, W), dtype=i32, device=self.device)
        self.stream_control = torch.zeros((1, 5), dtype=i32, device=self.device)
        self.stream_control[0, 4] = history_capacity_activations
        self.ring = torch.zeros((1, 4 + 4 * history_capacity_activations), dtype=i32, device=self.device)
        self.out = torch.zeros((1, 4), dtype=i32, device=self.device)
        self.seeds = torch.full((max(1, max_lanes),), random_seed & 0xFFFFFFFF, dtype=torch.int64).to(i32).to(self.device)
        method = METHOD_NAMES[spec.method]
        self.params = params_tensor(make_params(
            max(1, max_lanes), method=method, temperature=spec.temperature, top_k=max(spec.top_k, 1),
            top_p=spec.top_p, min_p=spec.min_p, repetition_penalty=spec.repetition_penalty,
            presence_penalty=spec.presence_penalty), self.device)
        self.token_state_active = spec.repetition_penalty != 1.0 or spec.presence_penalty != 0.0 or \
            spec.runtime_parameterized

    def set_stream_tick(self, tick: int) -> None:
        self.stream_control[0, 1] = int(np.uint32(tick & 0xFFFFFFFF).view(np.int32))
        self.stream_control[0, 2] = int(np.uint32((tick >> 32) & 0xFFFFFFFF).view(np.int32))

    def write_stream_control(self, token: int, tick: int, capacity: int | None = None) -> None:
        self.stream_control[0, 0] = int(np.uint32(token).view(np.int32))
        self.set_stream_tick(tick)
        if capacity is not None:
            self.stream_control[0, 4] = capacity

    def run(self, logits) -> SamplerRun:
        """logits: float32 device tensor [V] or [1, V]."""
        lg = logits.reshape(1, -1)
        self.sampler.step(lg, self.params, self.out, seen=self.seen if self.token_state_active else None,
                          seeds=self.seeds, rng=RNG_REFERENCE_HASH, stream_control=self.stream_control,
                          output_ring=self.ring)
        return self.completed_run()

    def completed_run(self) -> SamplerRun:
        w = self.ring[0, :4].cpu().numpy().view(np.uint32)
        return SamplerRun(self.spec.sampler_id, int(w[0]), int(w[1]), int(w[2]))

    def completed_run_at(self, stream_tick: int) -> SamplerRun:
        slot = (stream_tick & 0xFFFFFFFF) % self.history_capacity
        w = self.ring[0, 4 + 4 * slot: 8 + 4 * slot].cpu().numpy().view(np.uint32)
        return SamplerRun(self.spec.sampler_id, int(w[0]), int(w[1]), int(w[2]))

    def read_output_bytes(self) -> bytes:
        return self.ring[0, :4].cpu().numpy().view(np.uint32).tobytes()

    def stream_control_words(self):
        return [int(x) for x in self.stream_control[0].cpu().numpy().view(np.uint32)]

    def record_input_tokens(self, token_ids) -> None:
        if not self.token_state_active:
            return
        n = len(token_ids)
        if n == 0 or n > TOKEN_BATCH_CAPACITY:
            raise SamplerError(ERR_TOKEN_BATCH_CAPACITY_EXCEEDED,
                               f"sampler repetition-state batch requests {n} tokens, capacity is {TOKEN_BATCH_CAPACITY}")
        torch = self.torch
        ids = torch.tensor(np.asarray(token_ids, np.uint32).view(np.int32)[None], device=self.device)
        counts = torch.tensor([n], dtype=torch.int32, device=self.device)
        self.sampler.record_tokens(self.seen, ids, counts, n)

    def record_current_token(self) -> None:
        """record_seen_token.comp.template: the token in stream-control word 0."""
        ids = self.stream_control[:, :1].contiguous()
        counts = self.torch.ones(1, dtype=self.torch.int32, device=self.device)
        self.sampler.record_tokens(self.seen, ids, counts, 1)

    def capture_token_state(self) -> None:
        self.sampler.copy_token_state(self.snapshot, self.seen)

    def restore_token_state(self) -> None:
        self.sampler.copy_token_state(self.seen, self.snapshot)

    def sample_lanes(self, logits, token_prefixes, stream_ticks, dynamic_state_capacities=None, *,
                     consecutive_from: int | None = None) -> list[SamplerRun]:
        """Per-lane views over a [B, V] logits buffer (batched_output_projection.rs:316-371): lane i
        samples with the runner's seen state plus its prefix tokens (added on the device by the step
        itself, the runner's bitmap shared by every lane and left unchanged), at its own tick, and
        writes the runner's ring slot for that tick. One launch; one device-to-host copy of B records."""
        torch = self.torch
        B = len(token_prefixes)
        if B == 0 or B > self.sampler.max_batch:
            raise SamplerError(ERR_BATCH_CAPACITY_EXCEEDED, f"cannot sample {B} lanes")
        if len(stream_ticks) != B:
            raise SamplerError(ERR_INVALID_ARGUMENT, f"{B} token lanes and {len(stream_ticks)} stream ticks")
        kw = {}
        if self.token_state_active:
            n = max((len(p) for p in token_prefixes), default=0)
            if n > TOKEN_BATCH_CAPACITY:
                raise SamplerError(ERR_TOKEN_BATCH_CAPACITY_EXCEEDED,
                                   f"sampler repetition-state batch requests {n} tokens, capacity is {TOKEN_BATCH_CAPACITY}")
            kw["seen"] = self.seen
            kw["seen_shared"] = True
            if n:
                ids = np.zeros((B, n), np.uint32)
                counts = np.zeros(B, np.int32)
                for i, p in enumerate(token_prefixes):
                    ids[i, :len(p)] = p
                    counts[i] = len(p)
                kw["prefix_ids"] = torch.from_numpy(ids.view(np.int32)).to(self.device)
                kw["prefix_counts"] = torch.from_numpy(counts).to(self.device)
        caps = list(dynamic_state_capacities or [self.history_capacity] * B)
        scn = np.zeros((B, 5), np.uint32)
        for i, t in enumerate(stream_ticks):
            scn[i, 1] = t & 0xFFFFFFFF
            scn[i, 2] = t >> 32
            scn[i, 4] = caps[i]
        sc = torch.from_numpy(scn.view(np.int32)).to(self.device)
        ring = torch.zeros((B, self.ring.shape[1]), dtype=torch.int32, device=self.device)
        out = torch.zeros((B, 4), dtype=torch.int32, device=self.device)
        self.sampler.step(logits, self.params[: B * 32], out, seeds=self.seeds[:B], rng=RNG_REFERENCE_HASH,
                          stream_control=sc, output_ring=ring, **kw)
        slots = np.array([(t & 0xFFFFFFFF) % c for t, c in zip(stream_ticks, caps)], np.int64)
        cols = torch.from_numpy(4 + 4 * slots[:, None] + np.arange(4)[None, :]).to(self.device)
        recs = torch.gather(ring, 1, cols)  # [B, 4] ring records of each lane's tick
        self.ring[0].scatter_(0, cols.reshape(-1), recs.reshape(-1))
        recn = recs.cpu().numpy().view(np.uint32)
        return [SamplerRun(self.spec.sampler_id, int(r[0]), int(r[1]), int(r[2])) for r in recn]

    def sample_batch(self, logits, input_token_ids, start_stream_tick: int,
                     dynamic_state_capacity_activations: int | None = None) -> list[SamplerRun]:
        """sample_batch (batched_output_projection.rs:277-298): lane i samples with the prefix
        input_token_ids[..=i] at tick start + i (speculative verification of a drafted window)."""
        n = len(input_token_ids)
        cap = self.history_capacity if dynamic_state_capacity_activations is None else dynamic_state_capacity_activations
        ticks = [start_stream_tick + i for i in range(n)]
        return self.sample_lanes(logits, [list(input_token_ids[: i + 1]) for i in range(n)], ticks, [cap] * n)


# ---- LM head fused with the step --------------------------------------------------


def tile_count(vocab: int) -> int:
    return (vocab + TILE_COLUMNS - 1) // TILE_COLUMNS


def lm_head_project(frames, weight, logits, *, output_scale: float = 1.0, tile_records=None, stream=None) -> None:
    """logits[b, v] = output_scale * frames[b] . weight[v] (tied_output_projection_batch_bf16.comp.template):
    frames [B, D] and weight [V, D] bfloat16 (or int16 bits) on the device, logits float32 [B, >= V];
    tile_records int32 [B, >= 2 * ceil(V/64)] receives the tile records when given."""
    frames, fs = _rows(frames)
    weight, ws = _rows(weight)
    logits, ls = _rows(logits)
    B, D = frames.shape[0], frames.shape[1]
    V = weight.shape[0]
    if weight.shape[1] != D:
        raise ValueError("frames and weight disagree on input_size")
    rp, rs = 0, 0
    if tile_records is not None:
        tr, trs = _rows(tile_records)
        rp, rs = tr.data_ptr(), trs // 2
    dev = frames.device.index or 0
    _check(load_library().nerve_lm_head_project(frames.data_ptr(), fs, weight.data_ptr(), ws, B, D, V,
                                                float(output_scale), logits.data_ptr(), ls, rp or None, rs,
                                                _stream_arg(stream, dev)))


def tile_records(logits, records, *, vocab: int | None = None, stream=None) -> None:
    """The tile records of existing logits (float32, or bfloat16 / int16 bits) into records int32 [B, >= 2 * tiles]."""
    import torch

    lg, ls = _rows(logits)
    dtype = DTYPE_F32 if lg.dtype == torch.float32 else DTYPE_BF16
    V = ls if vocab is None else vocab
    tr, trs = _rows(records)
    dev = lg.device.index or 0
    _check(load_library().nerve_tile_records(lg.data_ptr(), dtype, ls, lg.shape[0], V, tr.data_ptr(), trs // 2,
                                             _stream_arg(stream, dev)))
