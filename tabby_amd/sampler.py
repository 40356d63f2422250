"""Python host side of the MI355X sampler, over the C ABI of ``include/tabby_sampler.h``.

The names mirror the reference's sampling surface so a caller of the reference finds the
same things:

* ``SeededRandom``      -- mulberry32, src/engine/sampler.ts:105-119 (host RNG; it only
                           produces each row's uniform)
* ``SamplingParams`` / ``DEFAULT_SAMPLING`` -- src/engine/sampler.ts:83-98
* ``SampleOutcome``     -- src/engine/sampler.ts:121-135
* ``TopKResult``        -- src/engine/forward.ts:93-103
* ``sample(logits, params, rng)`` -- the composition encodeSampling (forward.ts:522-601)
  -> readback -> sampleFromTopK (sampler.ts:147-212) that the worker performs
  (src/worker/inference.worker.ts:162-168), done on the GPU.

Device memory and streams come from torch (``torch.cuda``); every sampling computation runs
in ``libtabby_sampler.so``. There is no CPU fallback: without the built library, importing
the binding raises.
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Union

import numpy as np

from .build import LIB_PATH

TABBY_OK, TABBY_EINVAL, TABBY_EHIP, TABBY_EEMPTY, TABBY_EDOMAIN, TABBY_ECAPACITY = range(6)
TABBY_F32, TABBY_F16 = 0, 1
TABBY_FLAG_FULL_VOCAB = 1

PARAMS_DTYPE = np.dtype([
    ("temperature", "<f8"), ("top_p", "<f8"), ("uniform", "<f8"),
    ("top_k", "<i4"), ("reserved", "<i4"),
])
RESULT_DTYPE = np.dtype([
    ("id", "<i4"), ("considered", "<u4"), ("probability", "<f8"), ("pool_mass", "<f8"),
    ("max_logit", "<f4"), ("pool_exhausted", "<i4"), ("sum_exp", "<f8"), ("status", "<i4"),
    ("topk_count", "<i4"),
])
assert PARAMS_DTYPE.itemsize == 32 and RESULT_DTYPE.itemsize == 48

EXPORTED_SYMBOLS = (
    "tabby_sampler_create", "tabby_sampler_destroy", "tabby_sampler_sample_device",
    "tabby_sampler_sample", "tabby_last_error", "tabby_version", "tabby_debug_exp",
    "tabby_debug_seq_sum", "tabby_debug_first_above", "tabby_sampler_sample_device_noalloc",
    "tabby_argmax_device", "tabby_softmax_rows_device", "tabby_debug_stream_read",
    "tabby_debug_exp_f32", "tabby_lmhead_q4_pack_device", "tabby_lmhead_q4_device",
    "tabby_sampler_sample_lmhead_q4_device",
)


class SamplingError(RuntimeError):
    """A nonzero tabby_status; ``status`` holds the code."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the C ABI library. Raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing; build it with `python -m tabby_amd.build`")
    L = ctypes.CDLL(path)
    vp, i32, u32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_int64
    L.tabby_sampler_create.argtypes = [ctypes.c_int, i32, i32, i32, ctypes.POINTER(vp)]
    L.tabby_sampler_destroy.argtypes = [vp]
    L.tabby_sampler_sample_device.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp, i32, u32, vp]
    L.tabby_sampler_sample.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, vp, i32, vp]
    L.tabby_last_error.restype = ctypes.c_char_p
    L.tabby_version.restype = ctypes.c_char_p
    L.tabby_debug_exp.argtypes = [vp, vp, i64, vp]
    L.tabby_debug_seq_sum.argtypes = [vp, i32, ctypes.c_double, vp, vp, i32, vp]
    L.tabby_debug_first_above.argtypes = [vp, i32, vp, i32, vp, vp]
    L.tabby_sampler_sample_device_noalloc.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]
    L.tabby_argmax_device.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp]
    L.tabby_softmax_rows_device.argtypes = [vp, vp, i32, i32, i32, i32, vp]
    L.tabby_debug_stream_read.argtypes = [vp, i32, i64, vp, vp]
    L.tabby_debug_exp_f32.argtypes = [vp, vp, i64, vp]
    L.tabby_lmhead_q4_pack_device.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp]
    L.tabby_lmhead_q4_device.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]
    L.tabby_sampler_sample_lmhead_q4_device.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, vp, vp]
    for name in ("tabby_sampler_create", "tabby_sampler_destroy", "tabby_sampler_sample_device",
                 "tabby_sampler_sample", "tabby_debug_exp", "tabby_debug_seq_sum",
                 "tabby_debug_first_above", "tabby_sampler_sample_device_noalloc",
                 "tabby_argmax_device", "tabby_softmax_rows_device", "tabby_debug_stream_read",
                 "tabby_debug_exp_f32", "tabby_lmhead_q4_pack_device", "tabby_lmhead_q4_device",
                 "tabby_sampler_sample_lmhead_q4_device"):
        getattr(L, name).restype = ctypes.c_int
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != TABBY_OK:
        msg = load_library().tabby_last_error().decode("utf-8", "replace")
        raise SamplingError(rc, msg)


# ---------------------------------------------------------------------------------------
# The reference's value types.
# ---------------------------------------------------------------------------------------

class SeededRandom:
    """mulberry32 (src/engine/sampler.ts:105-119): u32 arithmetic, 32-bit uniforms."""

    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFF

    def next(self) -> float:
        s = (self.state + 0x6D2B79F5) & 0xFFFFFFFF
        self.state = s
        t = ((s ^ (s >> 15)) * (s | 1)) & 0xFFFFFFFF
        t ^= (t + (((t ^ (t >> 7)) * (t | 61)) & 0xFFFFFFFF)) & 0xFFFFFFFF
        return ((t ^ (t >> 14)) & 0xFFFFFFFF) / 4294967296.0


@dataclass
class SamplingParams:
    """src/engine/sampler.ts:83-91. topK = 0 means the whole vocabulary here."""

    temperature: float
    topK: int
    topP: float
    seed: int = 0


DEFAULT_SAMPLING = SamplingParams(temperature=0.7, topK=40, topP=0.9, seed=0)


@dataclass
class SampleOutcome:
    """src/engine/sampler.ts:121-135."""

    id: int
    probability: float
    consideredCount: int
    poolMass: float
    poolExhausted: bool


@dataclass
class TopKResult:
    """src/engine/forward.ts:93-103 (sumExp is carried in f64)."""

    maxLogit: float
    sumExp: float
    ids: List[int] = field(default_factory=list)
    logits: List[float] = field(default_factory=list)


SAMPLE_HEADER_FLOATS = 2  # forward.ts:127-129: [maxLogit, sumExp, (value, index) * k]


def encode_sample_block(top: TopKResult, k: Optional[int] = None) -> bytes:
    """A TopKResult as the sample block a decode step reads back (forward.ts:127-157): f32
    words [maxLogit, sumExp, then (value, index) per candidate], each index a u32 written
    into its word. ``k`` defaults to all of the result's candidates."""
    n = len(top.ids) if k is None else int(k)
    if not 0 <= n <= len(top.ids) or len(top.logits) != len(top.ids):
        raise ValueError(f"encode_sample_block: k must be within the result's {len(top.ids)} candidates")
    block = np.zeros(SAMPLE_HEADER_FLOATS + 2 * n, dtype=np.float32)
    block[0] = top.maxLogit
    block[1] = top.sumExp
    block[SAMPLE_HEADER_FLOATS::2] = np.asarray(top.logits[:n], dtype=np.float32)
    block.view(np.uint32)[SAMPLE_HEADER_FLOATS + 1::2] = np.asarray(top.ids[:n], dtype=np.uint32)
    return block.tobytes()


def decode_sample_block(raw: bytes, k: int) -> TopKResult:
    """forward.ts:142-157: the first k candidates of a sample block, read through an f32 and
    a u32 view of the same bytes."""
    as_float = np.frombuffer(raw, dtype=np.float32)
    as_uint = np.frombuffer(raw, dtype=np.uint32)
    if SAMPLE_HEADER_FLOATS + 2 * k > as_float.size:
        raise ValueError(f"decode_sample_block: the block holds {(as_float.size - SAMPLE_HEADER_FLOATS) // 2} "
                         f"candidates, asked for {k}")
    slots = SAMPLE_HEADER_FLOATS + 2 * np.arange(k)
    return TopKResult(float(as_float[0]), float(as_float[1]),
                      [int(v) for v in as_uint[slots + 1]], [float(v) for v in as_float[slots]])


def outcome_of(rec) -> SampleOutcome:
    return SampleOutcome(id=int(rec["id"]), probability=float(rec["probability"]),
                         consideredCount=int(rec["considered"]), poolMass=float(rec["pool_mass"]),
                         poolExhausted=bool(rec["pool_exhausted"]))


def make_params(params: Union[SamplingParams, Sequence[SamplingParams]], rows: int,
                rng: Union[SeededRandom, Sequence[float], np.ndarray, float, None]) -> np.ndarray:
    """Packs per-row params. A SeededRandom is advanced once per row with temperature > 0,
    in row order, as the reference advances it once per non-greedy token (sampler.ts:194)."""
    if isinstance(params, SamplingParams):
        params = [params] * rows
    if len(params) != rows:
        raise ValueError(f"expected {rows} SamplingParams, got {len(params)}")
    for p in params:
        # A NaN or +inf temperature is refused on every path (sampler.ts would sample NaN
        # weights), before any uniform is drawn.
        if not p.temperature < math.inf:
            raise ValueError(f"temperature must not be NaN or +Infinity, got {p.temperature}")
    out = np.zeros(rows, dtype=PARAMS_DTYPE)
    explicit = None
    if rng is not None and not isinstance(rng, SeededRandom):
        explicit = np.broadcast_to(np.asarray(rng, dtype=np.float64), (rows,))
    for r, p in enumerate(params):
        out[r]["temperature"] = p.temperature
        out[r]["top_p"] = p.topP
        out[r]["top_k"] = p.topK
        if explicit is not None:
            out[r]["uniform"] = explicit[r]
        elif isinstance(rng, SeededRandom) and p.temperature > 0:
            out[r]["uniform"] = rng.next()
    return out


# ---------------------------------------------------------------------------------------
# The sampler handle.
# ---------------------------------------------------------------------------------------

def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return TABBY_F32
    if t.dtype == torch.float16:
        return TABBY_F16
    raise TypeError(f"logits must be float32 or float16, got {t.dtype}")


class GpuSampler:
    """Owns the device scratch for sampling up to rows_max rows of up to vocab_max logits
    with top_k up to k_max (the sampling part of ForwardPass, forward.ts:243-248)."""

    def __init__(self, vocab_max: int, rows_max: int = 1, k_max: int = 64, device: int = 0):
        self._lib = load_library()
        h = ctypes.c_void_p()
        _check(self._lib.tabby_sampler_create(device, vocab_max, rows_max, k_max, ctypes.byref(h)))
        self._h = h
        self.vocab_max, self.rows_max, self.k_max, self.device = vocab_max, rows_max, k_max, device

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.tabby_sampler_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _stream(stream):
        import torch
        if stream is None:
            stream = torch.cuda.current_stream()
        return ctypes.c_void_p(stream.cuda_stream)

    def sample_params(self, logits, params: np.ndarray, topk_cap: int = 0, stream=None):
        """Host-parameter entry (tabby_sampler_sample). ``logits`` is a CUDA tensor [V] or
        [R, V]; returns (results structured array, topk ids, topk logits)."""
        if not logits.is_cuda:
            raise ValueError("logits must be a device (cuda) tensor")
        x = logits if logits.dim() == 2 else logits.reshape(1, -1)
        if not x.is_contiguous():
            raise ValueError("logits must be contiguous")
        rows, vocab = int(x.shape[0]), int(x.shape[1])
        params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
        if params.shape != (rows,):
            raise ValueError(f"params must have shape ({rows},), got {params.shape}")
        results = np.zeros(rows, dtype=RESULT_DTYPE)
        ids = np.zeros((rows, max(topk_cap, 0)), dtype=np.int32)
        vals = np.zeros((rows, max(topk_cap, 0)), dtype=np.float32)
        _check(self._lib.tabby_sampler_sample(
            self._h, ctypes.c_void_p(x.data_ptr()), _dtype_code(x), rows, vocab,
            params.ctypes.data, results.ctypes.data,
            ids.ctypes.data if topk_cap > 0 else None, vals.ctypes.data if topk_cap > 0 else None,
            topk_cap, self._stream(stream)))
        return results, ids, vals

    def sample_device(self, logits, params_dev, results_dev, topk_ids=None, topk_logits=None,
                      flags: int = 0, stream=None) -> None:
        """Device-resident entry (tabby_sampler_sample_device); asynchronous. ``params_dev``
        and ``results_dev`` are uint8 CUDA tensors holding PARAMS_DTYPE / RESULT_DTYPE rows."""
        x = logits if logits.dim() == 2 else logits.reshape(1, -1)
        rows, vocab = int(x.shape[0]), int(x.shape[1])
        cap = int(topk_ids.shape[-1]) if topk_ids is not None else 0
        _check(self._lib.tabby_sampler_sample_device(
            self._h, ctypes.c_void_p(x.data_ptr()), _dtype_code(x), rows, vocab,
            ctypes.c_void_p(params_dev.data_ptr()), ctypes.c_void_p(results_dev.data_ptr()),
            ctypes.c_void_p(topk_ids.data_ptr()) if cap else None,
            ctypes.c_void_p(topk_logits.data_ptr()) if cap else None, cap, flags,
            self._stream(stream)))

    def argmax_device(self, logits, ids_dev, max_dev=None, stream=None) -> None:
        """Greedy fast path (tabby_argmax_device): ``ids_dev`` (int32 CUDA tensor [rows])
        receives each row's argmax, ``max_dev`` (float32, optional) its value.
        Asynchronous."""
        x = logits if logits.dim() == 2 else logits.reshape(1, -1)
        if not x.is_contiguous():
            raise ValueError("logits must be contiguous")
        rows, vocab = int(x.shape[0]), int(x.shape[1])
        if ids_dev.numel() < rows or (max_dev is not None and max_dev.numel() < rows):
            raise ValueError("ids_dev / max_dev must hold one entry per row")
        _check(self._lib.tabby_argmax_device(
            self._h, ctypes.c_void_p(x.data_ptr()), _dtype_code(x), rows, vocab,
            ctypes.c_void_p(ids_dev.data_ptr()),
            ctypes.c_void_p(max_dev.data_ptr()) if max_dev is not None else None,
            self._stream(stream)))

    def argmax(self, logits, stream=None):
        """argmax of each row (sampler.ts:13-23) on the GPU: an int for a 1-D ``logits``,
        a list of ints for [rows, vocab]."""
        import torch
        x = logits if logits.dim() == 2 else logits.reshape(1, -1)
        ids = torch.empty(int(x.shape[0]), dtype=torch.int32, device=x.device)
        self.argmax_device(x, ids, stream=stream)
        out = [int(v) for v in ids.cpu().tolist()]
        return out[0] if logits.dim() == 1 else out

    def sample_lmhead_q4_device(self, head: "LmHeadQ4", hidden_states, params_dev, results_dev,
                                stream=None) -> None:
        """The lm_head fused with sampling (tabby_sampler_sample_lmhead_q4_device): one call
        samples each row of ``hidden_states`` (float32 CUDA [rows, hidden], rows <= 8) from the
        logits ``head`` would produce, without writing them. Asynchronous."""
        x = hidden_states if hidden_states.dim() == 2 else hidden_states.reshape(1, -1)
        _check(self._lib.tabby_sampler_sample_lmhead_q4_device(
            self._h, ctypes.c_void_p(head.packed.data_ptr()), ctypes.c_void_p(head.scales.data_ptr()),
            ctypes.c_void_p(head.bias.data_ptr()) if head.bias is not None else None,
            ctypes.c_void_p(x.data_ptr()), int(x.shape[0]), head.vocab, head.hidden, head.block,
            ctypes.c_void_p(params_dev.data_ptr()), ctypes.c_void_p(results_dev.data_ptr()),
            self._stream(stream)))

    def sample_lmhead_q4(self, head: "LmHeadQ4", hidden_states, params: np.ndarray, stream=None):
        """Host-parameter convenience over sample_lmhead_q4_device: returns the results
        structured array (synchronises)."""
        import torch
        x = hidden_states if hidden_states.dim() == 2 else hidden_states.reshape(1, -1)
        rows = int(x.shape[0])
        p = torch.from_numpy(np.ascontiguousarray(params, dtype=PARAMS_DTYPE).view(np.uint8).copy()).to(x.device)
        res = torch.zeros(rows * RESULT_DTYPE.itemsize, dtype=torch.uint8, device=x.device)
        self.sample_lmhead_q4_device(head, x, p, res, stream=stream)
        return res.cpu().numpy().view(RESULT_DTYPE)

    def sample(self, logits, params: SamplingParams, rng) -> SampleOutcome:
        """One row: sample(logits, {temperature, topK, topP}, rng) -> SampleOutcome."""
        res, _, _ = self.sample_params(logits, make_params(params, 1, rng))
        return outcome_of(res[0])

    def sample_batch(self, logits, params, rng) -> List[SampleOutcome]:
        rows = int(logits.shape[0])
        res, _, _ = self.sample_params(logits, make_params(params, rows, rng))
        return [outcome_of(r) for r in res]

    def top_k(self, logits, k: int) -> TopKResult:
        """The GPU half alone (encodeSampling's TopKResult) for one row."""
        p = make_params(SamplingParams(temperature=0.0, topK=k, topP=1.0), 1, 0.0)
        vocab = int(logits.shape[-1])
        cap = vocab if k <= 0 else min(k, vocab)
        res, ids, vals = self.sample_params(logits, p, topk_cap=cap)
        n = int(res[0]["topk_count"])
        return TopKResult(maxLogit=float(res[0]["max_logit"]), sumExp=float(res[0]["sum_exp"]),
                          ids=[int(v) for v in ids[0, :n]], logits=[float(v) for v in vals[0, :n]])


def sample_device_noalloc(logits, params_dev, results_dev, k_max: int, topk_ids=None, topk_logits=None,
                          stream=None) -> None:
    """The allocation-free device-resident entry (tabby_sampler_sample_device_noalloc): no
    handle, scratch in the library's fixed per-GPU array; k_max <= 256, no whole-vocabulary
    pools. Asynchronous; same buffers as GpuSampler.sample_device."""
    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    rows, vocab = int(x.shape[0]), int(x.shape[1])
    cap = int(topk_ids.shape[-1]) if topk_ids is not None else 0
    _check(load_library().tabby_sampler_sample_device_noalloc(
        ctypes.c_void_p(x.data_ptr()), _dtype_code(x), rows, vocab, int(k_max),
        ctypes.c_void_p(params_dev.data_ptr()), ctypes.c_void_p(results_dev.data_ptr()),
        ctypes.c_void_p(topk_ids.data_ptr()) if cap else None,
        ctypes.c_void_p(topk_logits.data_ptr()) if cap else None, cap, GpuSampler._stream(stream)))


_default: Optional[GpuSampler] = None


def sample(logits, params: SamplingParams, rng) -> SampleOutcome:
    """Module-level drop-in: one row, a cached handle grown to fit."""
    global _default
    vocab = int(logits.shape[-1])
    k = max(params.topK, 1)
    if _default is None or _default.vocab_max < vocab or _default.k_max < min(k, 1024):
        if _default is not None:
            _default.close()
        _default = GpuSampler(vocab_max=vocab, rows_max=1, k_max=max(64, min(k, 1024)))
    return _default.sample(logits, params, rng)


def argmax(logits) -> Union[int, List[int]]:
    """Module-level drop-in for sampler.ts's argmax (lines 13-23), on the GPU: one row (1-D)
    gives an int, [rows, vocab] a list."""
    global _default
    x = logits if logits.dim() == 2 else logits.reshape(1, -1)
    rows, vocab = int(x.shape[0]), int(x.shape[1])
    if _default is None or _default.vocab_max < vocab or _default.rows_max < rows:
        k = _default.k_max if _default is not None else 64
        if _default is not None:
            _default.close()
        _default = GpuSampler(vocab_max=vocab, rows_max=rows, k_max=k)
    return _default.argmax(logits)


def softmax_rows(x, n_rows: int, row_len: int, causal_period: int = 0, causal_offset: int = 0,
                 out=None, stream=None):
    """softmaxRows (src/reference/cpu.ts:238-264), the softmax_rows kernel's contract, on the
    GPU and bit for bit the CPU reference's: ``x`` is a float32 CUDA tensor of n_rows *
    row_len entries; returns ``out`` (a new tensor, as the CPU reference returns a copy, or
    ``x`` itself for the in-place form the kernel runs). Asynchronous."""
    import torch
    if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 CUDA tensor")
    if x.numel() != n_rows * row_len:
        raise ValueError(f"x holds {x.numel()} entries, expected {n_rows} x {row_len}")
    if out is None:
        out = torch.empty_like(x)
    elif out.dtype != torch.float32 or out.numel() != x.numel() or not out.is_contiguous():
        raise ValueError("out must be a contiguous float32 tensor shaped like x")
    _check(load_library().tabby_softmax_rows_device(
        ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(out.data_ptr()), int(n_rows), int(row_len),
        int(causal_period), int(causal_offset), GpuSampler._stream(stream)))
    return out


class LmHeadQ4:
    """The lm_head's int4 weights on the device in this library's layout
    (tabby_lmhead_q4_pack_device), made from the reference's layout: ``words`` u32
    [vocab, hidden / 8] and ``scales_f16`` f16 bits [vocab, hidden / block] (numpy or CUDA
    tensors), optional ``bias`` f32 [vocab]."""

    def __init__(self, words, scales_f16, vocab: int, hidden: int, block: int = 32, bias=None,
                 device: str = "cuda"):
        import torch
        w = torch.as_tensor(np.ascontiguousarray(words).view(np.int32) if isinstance(words, np.ndarray)
                            else words).to(device).contiguous()
        sc = torch.as_tensor(np.ascontiguousarray(scales_f16).view(np.int16)
                             if isinstance(scales_f16, np.ndarray) else scales_f16).to(device).contiguous()
        self.vocab, self.hidden, self.block = int(vocab), int(hidden), int(block)
        if w.numel() != self.vocab * self.hidden // 8 or sc.numel() != self.vocab * self.hidden // self.block:
            raise ValueError("words / scales do not match vocab x hidden / block")
        self.packed = torch.empty_like(w)
        self.scales = torch.empty_like(sc)
        self.bias = None if bias is None else torch.as_tensor(np.asarray(bias, np.float32)).to(device).contiguous()
        _check(load_library().tabby_lmhead_q4_pack_device(
            ctypes.c_void_p(w.data_ptr()), ctypes.c_void_p(sc.data_ptr()), self.vocab, self.hidden,
            self.block, ctypes.c_void_p(self.packed.data_ptr()), ctypes.c_void_p(self.scales.data_ptr()),
            GpuSampler._stream(None)))

    def logits(self, hidden_states, out=None, stream=None):
        """The lm_head matmul (tabby_lmhead_q4_device): float32 CUDA [rows, vocab]."""
        import torch
        x = hidden_states if hidden_states.dim() == 2 else hidden_states.reshape(1, -1)
        if x.dtype != torch.float32 or not x.is_contiguous():
            raise ValueError("hidden states must be a contiguous float32 tensor")
        rows = int(x.shape[0])
        y = out if out is not None else torch.empty((rows, self.vocab), dtype=torch.float32, device=x.device)
        _check(load_library().tabby_lmhead_q4_device(
            ctypes.c_void_p(self.packed.data_ptr()), ctypes.c_void_p(self.scales.data_ptr()),
            ctypes.c_void_p(self.bias.data_ptr()) if self.bias is not None else None,
            ctypes.c_void_p(x.data_ptr()), rows, self.vocab, self.hidden, self.block,
            ctypes.c_void_p(y.data_ptr()), GpuSampler._stream(stream)))
        return y


def stream_read(src, sink, stream=None) -> None:
    """The measurement diagnostic tabby_debug_stream_read over a [rows, row_floats] float32
    CUDA tensor: one plain read with the sampling kernels' loads. ``sink`` is an int32 CUDA
    tensor of at least ``rows`` entries. Asynchronous."""
    rows, row_floats = int(src.shape[0]), int(src.shape[1])
    _check(load_library().tabby_debug_stream_read(
        ctypes.c_void_p(src.data_ptr()), rows, row_floats, ctypes.c_void_p(sink.data_ptr()),
        GpuSampler._stream(stream)))


def device_exp(x) -> "object":
    """The device f64 exp over a CUDA float64 tensor (diagnostic)."""
    import torch
    y = torch.empty_like(x)
    _check(load_library().tabby_debug_exp(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                          x.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return y


def device_exp_f32(x):
    """fround(Math.exp(x)) over a CUDA float32 tensor of arguments <= 0, as the row softmax
    computes it (diagnostic)."""
    import torch
    y = torch.empty_like(x)
    _check(load_library().tabby_debug_exp_f32(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()),
                                              x.numel(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return y


def device_seq_sum(terms, stop_at: float = float("inf"), wide: int = 0, in_place: bool = False):
    """The device's sequential f64 partial sums of a CUDA float64 tensor (diagnostic):
    returns (prefix sums actually written, as a CUDA tensor, count). ``wide``: 0 the
    one-term-per-lane form, 1 the 16-terms-per-lane form used for long sums, 2 that form
    taken by a four-wave workgroup, 3 by an eight-wave workgroup, 4 the register form (at
    most 64 terms, term i in lane i). ``in_place``: the sums are written over (a copy of)
    the terms."""
    import torch
    t = terms.contiguous().clone() if in_place else terms.contiguous()
    out = t if in_place else torch.zeros_like(t)
    cnt = torch.zeros(1, dtype=torch.int32, device=t.device)
    stream = torch.cuda.current_stream()
    _check(load_library().tabby_debug_seq_sum(ctypes.c_void_p(t.data_ptr()), int(t.numel()),
                                              float(stop_at), ctypes.c_void_p(out.data_ptr()),
                                              ctypes.c_void_p(cnt.data_ptr()), int(wide),
                                              ctypes.c_void_p(stream.cuda_stream)))
    n = int(cnt.item())
    return out[:n], n


def device_first_above(c, targets):
    """The device's draw search over a non-decreasing CUDA float64 tensor ``c`` (diagnostic):
    for each target, the first i with target < c[i], or len(c) - 1 when there is none."""
    import torch
    c = c.contiguous()
    t = targets.contiguous()
    out = torch.empty(t.numel(), dtype=torch.int32, device=c.device)
    _check(load_library().tabby_debug_first_above(ctypes.c_void_p(c.data_ptr()), int(c.numel()),
                                                  ctypes.c_void_p(t.data_ptr()), int(t.numel()),
                                                  ctypes.c_void_p(out.data_ptr()),
                                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    return out
