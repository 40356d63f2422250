"""Python handle on the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import this module.
It wraps the C restatement (``tabby_oracle.c``, built by ``oracle/Makefile`` into
``oracle/_build/``) and the Node restatement (``sampler_oracle.js`` via ``node_driver.js``).
The reference functions each one follows are listed in ``tabby_oracle.h``.
"""
from __future__ import annotations

import contextlib
import ctypes
import json
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtabby_oracle.so")
NODE_DRIVER = os.path.join(HERE, "node_driver.js")


class Outcome(ctypes.Structure):
    _fields_ = [
        ("id", ctypes.c_int32),
        ("considered", ctypes.c_uint32),
        ("probability", ctypes.c_double),
        ("pool_mass", ctypes.c_double),
        ("pool_exhausted", ctypes.c_int32),
        ("status", ctypes.c_int32),
    ]

    def as_dict(self) -> dict:
        return {
            "id": self.id,
            "considered": self.considered,
            "probability": self.probability,
            "pool_mass": self.pool_mass,
            "pool_exhausted": bool(self.pool_exhausted),
            "status": self.status,
        }


def build() -> None:
    """Compile the C oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def load(path: str) -> ctypes.CDLL:
    """Loads a build of tabby_oracle.c at `path` with its ctypes signatures."""
    L = ctypes.CDLL(path)
    P = ctypes.POINTER
    L.tabby_oracle_mulberry32_fill.argtypes = [ctypes.c_uint32, P(ctypes.c_double), ctypes.c_int64]
    L.tabby_oracle_exp.argtypes = [ctypes.c_double]
    L.tabby_oracle_exp.restype = ctypes.c_double
    L.tabby_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.tabby_oracle_f16_to_f32.restype = ctypes.c_float
    L.tabby_oracle_argmax.argtypes = [P(ctypes.c_float), ctypes.c_int32]
    L.tabby_oracle_argmax.restype = ctypes.c_int32
    L.tabby_oracle_topk.argtypes = [P(ctypes.c_float), ctypes.c_int32, ctypes.c_int32,
                                    P(ctypes.c_int32), P(ctypes.c_float)]
    L.tabby_oracle_topk.restype = ctypes.c_int32
    L.tabby_oracle_sum_exp.argtypes = [P(ctypes.c_float), ctypes.c_int32, ctypes.c_float]
    L.tabby_oracle_sum_exp.restype = ctypes.c_double
    L.tabby_oracle_sample_from_topk.argtypes = [
        P(ctypes.c_int32), P(ctypes.c_float), ctypes.c_int32, ctypes.c_double,
        ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double, P(Outcome)]
    L.tabby_oracle_sample_row.argtypes = [
        P(ctypes.c_float), ctypes.c_int32, ctypes.c_int32, ctypes.c_double, ctypes.c_double,
        ctypes.c_double, P(Outcome), P(ctypes.c_int32), P(ctypes.c_float), ctypes.c_int32,
        P(ctypes.c_float), P(ctypes.c_double)]
    L.tabby_oracle_softmax_rows.argtypes = [P(ctypes.c_float), P(ctypes.c_float), ctypes.c_int32,
                                            ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
    L.tabby_oracle_softmax_rows.restype = None
    L.tabby_oracle_matmul_quantized.argtypes = [P(ctypes.c_uint32), P(ctypes.c_float), P(ctypes.c_float),
                                                ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                ctypes.c_int32, ctypes.c_int32, P(ctypes.c_float),
                                                P(ctypes.c_float)]
    L.tabby_oracle_matmul_quantized.restype = None
    return L


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = load(LIB_PATH)
    return _lib


@contextlib.contextmanager
def using(library: ctypes.CDLL):
    """Routes every function of this module through `library` (a build from `load`) for
    the duration; the tests use it to run their pins against deliberately broken builds."""
    global _lib
    saved = lib()
    _lib = library
    try:
        yield
    finally:
        _lib = saved


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def mulberry32(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().tabby_oracle_mulberry32_fill(seed & 0xFFFFFFFF, _ptr(out, ctypes.c_double), n)
    return out


def exp(x: float) -> float:
    return lib().tabby_oracle_exp(float(x))


def exp_array(x: np.ndarray) -> np.ndarray:
    f = lib().tabby_oracle_exp
    return np.array([f(float(v)) for v in np.asarray(x, dtype=np.float64)], dtype=np.float64)


def f16_to_f32(bits: int) -> float:
    return lib().tabby_oracle_f16_to_f32(bits)


def argmax(row: np.ndarray) -> int:
    row = np.ascontiguousarray(row, dtype=np.float32)
    return lib().tabby_oracle_argmax(_ptr(row, ctypes.c_float), row.size)


def matmul_quantized(words: np.ndarray, scales: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int,
                     bits: int = 4, block_size: int = 32, bias=None) -> np.ndarray:
    """matmulQuantized (src/reference/cpu.ts:352-393): y [n_tokens, out_dim] f32 for x
    [n_tokens, in_dim] f32, words u32 [out_dim * in_dim * bits / 32], scales f32
    [out_dim * in_dim / block_size]."""
    words = np.ascontiguousarray(words, dtype=np.uint32).reshape(-1)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    y = np.empty((x.shape[0], out_dim), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().tabby_oracle_matmul_quantized(_ptr(words, ctypes.c_uint32), _ptr(scales, ctypes.c_float),
                                        _ptr(x, ctypes.c_float), x.shape[0], out_dim, in_dim, bits,
                                        block_size, _ptr(b, ctypes.c_float) if b is not None else None,
                                        _ptr(y, ctypes.c_float))
    return y


def softmax_rows(x: np.ndarray, n_rows: int, row_len: int, causal_period: int = 0,
                 causal_offset: int = 0) -> np.ndarray:
    """softmaxRows (src/reference/cpu.ts:238-264): a new f32 array [n_rows * row_len]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size == n_rows * row_len
    out = np.empty_like(x)
    lib().tabby_oracle_softmax_rows(_ptr(x, ctypes.c_float), _ptr(out, ctypes.c_float), n_rows,
                                    row_len, causal_period, causal_offset)
    return out


def topk(row: np.ndarray, k: int):
    row = np.ascontiguousarray(row, dtype=np.float32)
    k = min(k, row.size)
    ids = np.empty(k, dtype=np.int32)
    vals = np.empty(k, dtype=np.float32)
    lib().tabby_oracle_topk(_ptr(row, ctypes.c_float), row.size, k, _ptr(ids, ctypes.c_int32),
                            _ptr(vals, ctypes.c_float))
    return ids, vals


def sum_exp(row: np.ndarray, max_logit: float) -> float:
    row = np.ascontiguousarray(row, dtype=np.float32)
    return lib().tabby_oracle_sum_exp(_ptr(row, ctypes.c_float), row.size, max_logit)


def sample_from_topk(ids, logits, max_logit, sum_exp_value, temperature, top_p, uniform) -> dict:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = Outcome()
    lib().tabby_oracle_sample_from_topk(_ptr(ids, ctypes.c_int32), _ptr(logits, ctypes.c_float),
                                        ids.size, max_logit, sum_exp_value, temperature, top_p,
                                        uniform, ctypes.byref(out))
    return out.as_dict()


def sample_row(row: np.ndarray, top_k: int, temperature: float, top_p: float, uniform: float,
               topk_cap: int = 0) -> dict:
    """Whole path for one row; adds max_logit, sum_exp and (if topk_cap) the sorted pool."""
    row = np.ascontiguousarray(row, dtype=np.float32)
    out = Outcome()
    cap = max(0, int(topk_cap))
    ids = np.zeros(max(cap, 1), dtype=np.int32)
    vals = np.zeros(max(cap, 1), dtype=np.float32)
    mx = ctypes.c_float(0)
    se = ctypes.c_double(0)
    lib().tabby_oracle_sample_row(_ptr(row, ctypes.c_float), row.size, int(top_k),
                                  float(temperature), float(top_p), float(uniform),
                                  ctypes.byref(out), _ptr(ids, ctypes.c_int32),
                                  _ptr(vals, ctypes.c_float), cap, ctypes.byref(mx),
                                  ctypes.byref(se))
    d = out.as_dict()
    d["max_logit"] = mx.value
    d["sum_exp"] = se.value
    if cap:
        k_eff = row.size if (top_k <= 0 or top_k >= row.size) else top_k
        m = min(cap, k_eff)
        d["topk_ids"] = ids[:m].copy()
        d["topk_values"] = vals[:m].copy()
    return d


def sample_batch(logits: np.ndarray, top_k, temperature, top_p, uniform, topk_cap: int = 0,
                 workers: int = 8) -> list:
    """Row-parallel over threads (ctypes releases the GIL during each C call)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    rows = logits.shape[0]

    def one(r):
        return sample_row(logits[r], int(top_k[r]), float(temperature[r]), float(top_p[r]),
                          float(uniform[r]), topk_cap)

    if rows == 1 or workers <= 1:
        return [one(r) for r in range(rows)]
    with ThreadPoolExecutor(max_workers=min(workers, rows)) as pool:
        return list(pool.map(one, range(rows)))


# --------------------------------------------------------------------------------------
# Node restatement
# --------------------------------------------------------------------------------------

def node_available() -> bool:
    return shutil.which("node") is not None


def node_exp(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    with tempfile.TemporaryDirectory() as d:
        src, dst = os.path.join(d, "x.f64"), os.path.join(d, "y.f64")
        x.tofile(src)
        subprocess.run(["node", NODE_DRIVER, "exp", src, dst], check=True)
        return np.fromfile(dst, dtype=np.float64)


def node_mulberry32(seed: int, n: int) -> np.ndarray:
    with tempfile.TemporaryDirectory() as d:
        dst = os.path.join(d, "y.f64")
        subprocess.run(["node", NODE_DRIVER, "mulberry", str(seed & 0xFFFFFFFF), str(n), dst],
                       check=True)
        return np.fromfile(dst, dtype=np.float64)


def _write_spec(d, logits, top_k, temperature, top_p, uniform, **extra):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    lp = os.path.join(d, "logits.f32")
    logits.tofile(lp)
    spec = {
        "logits": lp, "rows": int(logits.shape[0]), "vocab": int(logits.shape[1]),
        "topK": [int(v) for v in top_k], "temperature": [float(v) for v in temperature],
        "topP": [float(v) for v in top_p], "uniform": [float(v) for v in uniform],
        "out": os.path.join(d, "out.json"),
    }
    spec.update(extra)
    sp = os.path.join(d, "spec.json")
    with open(sp, "w") as f:
        json.dump(spec, f)
    return sp, spec


def node_sample_batch(logits, top_k, temperature, top_p, uniform, topk_cap: int = 0) -> list:
    with tempfile.TemporaryDirectory() as d:
        sp, spec = _write_spec(d, logits, top_k, temperature, top_p, uniform, topkCap=int(topk_cap))
        subprocess.run(["node", NODE_DRIVER, "sample", sp], check=True)
        with open(spec["out"]) as f:
            return json.load(f)


def node_bench(logits, top_k, temperature, top_p, uniform, seconds: float, threads: int = 1,
               max_rows: int = 0) -> dict:
    """Times sampleRow in Node on rows cycled from `logits` for about `seconds`."""
    with tempfile.TemporaryDirectory() as d:
        sp, _ = _write_spec(d, logits, top_k, temperature, top_p, uniform, seconds=seconds,
                            threads=threads, maxRows=max_rows)
        r = subprocess.run(["node", NODE_DRIVER, "bench", sp], check=True, capture_output=True,
                           text=True)
        return json.loads(r.stdout.strip().splitlines()[-1])


def node_softmax_rows(x: np.ndarray, n_rows: int, row_len: int, causal_period: int = 0,
                      causal_offset: int = 0) -> np.ndarray:
    """softmaxRows restated in JS, run by Node with V8's Math.exp and Math.fround."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    with tempfile.TemporaryDirectory() as d:
        src, dst, sp = os.path.join(d, "x.f32"), os.path.join(d, "y.f32"), os.path.join(d, "s.json")
        x.tofile(src)
        with open(sp, "w") as f:
            json.dump({"x": src, "nRows": int(n_rows), "rowLen": int(row_len),
                       "period": int(causal_period), "offset": int(causal_offset), "out": dst}, f)
        subprocess.run(["node", NODE_DRIVER, "softmax", sp], check=True)
        return np.fromfile(dst, dtype=np.float32)


def node_argmax(logits: np.ndarray) -> list:
    """argmax of each row, restated in JS and run by Node."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    with tempfile.TemporaryDirectory() as d:
        lp, sp, out = os.path.join(d, "l.f32"), os.path.join(d, "s.json"), os.path.join(d, "o.json")
        logits.tofile(lp)
        with open(sp, "w") as f:
            json.dump({"logits": lp, "rows": int(logits.shape[0]), "vocab": int(logits.shape[1]),
                       "out": out}, f)
        subprocess.run(["node", NODE_DRIVER, "argmax", sp], check=True)
        with open(out) as f:
            return json.load(f)


def node_matmul_quantized(words, scales, x, out_dim: int, in_dim: int, bits: int = 4,
                          block_size: int = 32, bias=None) -> np.ndarray:
    """matmulQuantized restated in JS, run by Node (Math.fround)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    with tempfile.TemporaryDirectory() as d:
        paths = {k: os.path.join(d, k) for k in ("w", "s", "x", "b", "y", "spec")}
        np.ascontiguousarray(words, np.uint32).tofile(paths["w"])
        np.ascontiguousarray(scales, np.float32).tofile(paths["s"])
        x.tofile(paths["x"])
        if bias is not None:
            np.ascontiguousarray(bias, np.float32).tofile(paths["b"])
        with open(paths["spec"], "w") as f:
            json.dump({"words": paths["w"], "scales": paths["s"], "x": paths["x"],
                       "bias": paths["b"] if bias is not None else None, "nTokens": int(x.shape[0]),
                       "outDim": int(out_dim), "inDim": int(in_dim), "bits": int(bits),
                       "blockSize": int(block_size), "out": paths["y"]}, f)
        subprocess.run(["node", NODE_DRIVER, "matmulq", paths["spec"]], check=True)
        return np.fromfile(paths["y"], dtype=np.float32).reshape(x.shape[0], out_dim)
