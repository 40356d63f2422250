"""Writes the committed golden vectors under tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``). Needs ``node`` (the image's Node 12).

The reference sampler is TypeScript and cannot run here (no TS toolchain, and its
`generateGreedy` uses syntax Node 12 rejects), and the reference commits no logits or
sampling vectors. So the expected values come from two sources:

* ``sampling_fixture.json`` -- the reference's own CPU fixture (tests/sampling.test.ts:206-250:
  a four-candidate TopKResult and its assertions), with each outcome's values worked out in
  closed form below (exp of integers, the cumulative weights, the cut), not by any oracle.
* ``softmax_vectors.json`` (``--softmax``) -- softmaxRows outputs of the Node restatement
  (V8's Math.exp and Math.fround) on integer-derived scores (``softmax_input``): every output
  bit for small cases, a SHA-256 of the output bytes for long ones.
* ``exp_f32_hard.json`` (``--exp-f32``) -- f32 arguments whose exp sits within 2^-46 of an f32
  rounding boundary (``hard_exp_f32_arguments``), with V8's fround(Math.exp(x)) for each.
* ``node_vectors.json`` -- outputs of the Node restatement (oracle/sampler_oracle.js), which
  runs V8's own Math.exp and Array.prototype.sort comparator the reference runs on: mulberry32
  streams, Math.exp over assorted arguments, and sampled outcomes (+ sorted pool ids) of
  small workloads. Their logits are integer-derived from mulberry32 draws (`golden_logits`),
  exactly representable in f32 and reproducible without libm; a SHA-256 of each workload's
  bytes is stored so a test can prove it regenerated the same inputs.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from tabby_amd.synth import mulberry32_stream  # noqa: E402

MULBERRY_SEEDS = (0, 1, 7, 42, 12345, 0xDEADBEEF, 0xFFFFFFFF)
TOPK_CAP = 16

# name -> (rows, vocab, seed, kind, top_k choices, temperatures, top_ps)
WORKLOADS = {
    "fine": (8, 4096, 101, "fine", (1, 5, 40, 64, 0), (0.0, 0.5, 1.0, 2.0), (0.5, 0.9, 1.0)),
    "ties_neg_inf": (8, 1000, 202, "coarse_neg_inf", (0, 7, 64, 1024), (0.7, 1.0), (0.9, 0.98, 1.0)),
    "whole_vocab": (4, 3000, 303, "fine", (0,), (0.3, 1.0), (0.95,)),
    "special": (6, 512, 404, "special", (1, 40, 0), (0.0, 0.7, 1.0), (0.9, 1.0)),
}


def golden_logits(rows: int, vocab: int, seed: int, kind: str) -> np.ndarray:
    """Integer-derived f32 logits (every value exact in f32; no transcendental functions).

    fine:            top 24 bits of a mulberry32 draw, scaled to [-16, 16) in steps of 2^-19
    coarse_neg_inf:  multiples of 0.25 in [-8, 8) (heavy ties), 30 % -inf, -0 canonicalised
    special:         rows chosen to hit edge cases: all equal; +0/-0 mixes; one finite value
                     among -inf; a max shared by many ids; two spikes; a ramp
    """
    out = np.empty((rows, vocab), dtype=np.float32)
    for r in range(rows):
        u = mulberry32_stream((seed * 7919 + r * 104729) & 0xFFFFFFFF, vocab)
        bits = (u * 4294967296.0).astype(np.uint64)
        if kind == "fine":
            out[r] = ((bits >> np.uint64(8)).astype(np.float64) - 8388608.0) / 524288.0
        elif kind == "coarse_neg_inf":
            q = ((bits >> np.uint64(26)).astype(np.float64) - 32.0) * 0.25
            q[q == 0.0] = 0.0
            mask = mulberry32_stream((seed * 31 + r) & 0xFFFFFFFF, vocab) < 0.3
            q[mask] = -np.inf
            out[r] = q
        elif kind == "special":
            case = r % 6
            if case == 0:
                out[r] = 1.5
            elif case == 1:
                out[r] = np.where(bits % np.uint64(3) == 0, 0.0, -0.0)
                out[r, 5] = -1.0
            elif case == 2:
                out[r] = -np.inf
                out[r, vocab // 3] = -2.0
            elif case == 3:
                out[r] = ((bits >> np.uint64(28)).astype(np.float64)) * 0.5
            elif case == 4:
                out[r] = -3.0
                out[r, 17] = 4.0
                out[r, 300] = 4.0 - 2.0 ** -20
            else:
                out[r] = np.arange(vocab, dtype=np.float64)[::-1] / 64.0
        else:
            raise ValueError(kind)
    return out


def golden_params(rows: int, seed: int, ks, ts, ps):
    pick = mulberry32_stream((seed * 65537 + 11) & 0xFFFFFFFF, 4 * rows).reshape(rows, 4)
    k = np.asarray(ks, np.int32)[(pick[:, 0] * len(ks)).astype(int)]
    t = np.asarray(ts, np.float64)[(pick[:, 1] * len(ts)).astype(int)]
    p = np.asarray(ps, np.float64)[(pick[:, 2] * len(ps)).astype(int)]
    return k, t, p, pick[:, 3].copy()


def workload(name: str):
    rows, vocab, seed, kind, ks, ts, ps = WORKLOADS[name]
    logits = golden_logits(rows, vocab, seed, kind)
    k, t, p, u = golden_params(rows, seed, ks, ts, ps)
    return logits, k, t, p, u


def exp_arguments() -> np.ndarray:
    u = mulberry32_stream(0xE4F, 6000)
    ln2 = math.log(2.0)
    parts = [
        -60.0 + 61.0 * u[:2000],             # the sampler's range: (l - m)/T and l - m
        -745.5 + 1455.5 * u[2000:3000],       # the whole finite range, incl. under/overflow
        (u[3000:3500] - 0.5) * 2.0 ** -26,    # |x| < 2^-27: the 1 + x branch
        (u[3500:4000] - 0.5) * ln2,           # |x| < ln2/2: no reduction
        np.round((u[4000:4500] - 0.5) * 200) * ln2 / 2 + (u[4500:5000] - 0.5) * 1e-9,  # k*ln2/2
        np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 709.782712893384, 709.79, -708.39641853226408,
                  -745.13321910194111, -745.14, -37.0, -40.0, 2.0 ** -28, -(2.0 ** -28)]),
    ]
    return np.concatenate(parts)


def closed_form_fixture() -> dict:
    """tests/sampling.test.ts:206-250 with every expected value derived by hand."""
    e = [math.exp(-i) for i in range(4)]  # exp(l - maxLogit) for l = 10, 9, 8, 7
    s1 = sum(e)                            # 1 + e^-1 + e^-2 + e^-3
    w = [v / s1 for v in e]                # weights at T = 1
    c = list(np.cumsum(w))

    def first_reaching(p):
        return next(i for i, ci in enumerate(c) if ci >= p) + 1

    return {
        "source": "reference tests/sampling.test.ts:206-250",
        "top": {"maxLogit": 10.0, "sumExp": 2.5, "ids": [1, 2, 3, 4], "logits": [10.0, 9.0, 8.0, 7.0]},
        "cases": [
            {"name": "argmax at temperature 0", "temperature": 0.0, "topP": 1.0, "sumExp": 2.5,
             "expect": {"id": 1, "consideredCount": 1, "probability": 1.0 / 2.5,
                        "poolMass": s1 / 2.5, "poolExhausted": False}},
            {"name": "wide (topP 1)", "temperature": 1.0, "topP": 1.0, "sumExp": 2.5,
             "expect": {"consideredCount": 4, "poolMass": s1 / 2.5, "poolExhausted": False}},
            {"name": "narrow (topP 0.5)", "temperature": 1.0, "topP": 0.5, "sumExp": 2.5,
             "expect": {"consideredCount": first_reaching(0.5), "id": 1,
                        "poolMass": s1 / 2.5, "poolExhausted": False}},
            {"name": "clipped by k (sumExp 100)", "temperature": 1.0, "topP": 0.9, "sumExp": 100.0,
             "expect": {"poolMass": s1 / 100.0, "poolExhausted": True,
                        "consideredCount": first_reaching(0.9)}},
        ],
        "weights_T1": w,
        "spread": {"temperature": 2.0, "topP": 1.0, "seed": 12345, "draws": 200, "min_distinct": 2},
    }


# name -> (n_rows, row_len, causal_period, causal_offset, kind): inputs of softmax_vectors.json
SOFTMAX_CASES = {
    # The reference's own kernel test: nHeads 3 x nTokens 5, randomF32(75, 0x50f7, 4),
    # softmaxRows(scores, 15, 5, 5) (tests/kernels.test.ts:457-473).
    "reference_causal_3x5": (15, 5, 5, 0, "reference"),
    # Decode-like: 4 heads x 6 new queries over 10 positions, 4 of them cached (posStart 4).
    "attention_offset": (24, 10, 6, 4, "scores"),
    "whole_rows_300": (8, 300, 0, 0, "scores"),
    "long_rows_5000": (3, 5000, 0, 0, "scores"),
    "quantised_ties": (6, 777, 0, 0, "ties"),
    "special_rows": (7, 64, 0, 0, "special"),
}


def softmax_input(name: str) -> np.ndarray:
    """f32 scores for SOFTMAX_CASES[name], reproducible from mulberry32 without libm.

    reference: randomF32 of tests/support.ts:19-24 -- fround((u * 2 - 1) * scale), scale 4
    scores:    top 24 bits of a draw scaled to [-24, 24) in steps of 2^-18 (exps from 1 down
               to subnormal f32 and zero)
    ties:      multiples of 0.5 in [-8, 8) (long runs of equal terms: exact half-ulp ties)
    special:   NaN, +inf, all -inf, a single finite entry among -inf, +0/-0 mixes, all equal,
               and entries 100 apart (exps that underflow)
    """
    n_rows, row_len, _, _, kind = SOFTMAX_CASES[name]
    n = n_rows * row_len
    if kind == "reference":
        u = mulberry32_stream(0x50F7, n)
        return ((u * 2.0 - 1.0) * 4.0).astype(np.float32)
    u = mulberry32_stream(sum(map(ord, name)) * 7919 & 0xFFFFFFFF, n)
    bits = (u * 4294967296.0).astype(np.uint64)
    if kind == "scores":
        return (((bits >> np.uint64(8)).astype(np.float64) - 8388608.0) / 349525.33333333331).astype(np.float32)
    if kind == "ties":
        return (((bits >> np.uint64(27)).astype(np.float64) - 16.0) * 0.5).astype(np.float32)
    x = (((bits >> np.uint64(8)).astype(np.float64) - 8388608.0) / 1048576.0).reshape(n_rows, row_len)
    x[0, 9] = np.nan
    x[1, 3] = np.inf
    x[2, :] = -np.inf
    x[3, :] = -np.inf
    x[3, 40] = -7.0
    x[4, :] = np.where(bits[4 * row_len:5 * row_len] % np.uint64(2) == 0, 0.0, -0.0)
    x[5, :] = 2.5
    x[6, :] = -100.0 * (np.arange(row_len) % 3)
    return x.astype(np.float32).reshape(-1)


def softmax_vectors(o) -> dict:
    out = {}
    for name, (n_rows, row_len, period, offset, _) in SOFTMAX_CASES.items():
        x = softmax_input(name)
        y = o.node_softmax_rows(x, n_rows, row_len, period, offset)
        rec = {"n_rows": n_rows, "row_len": row_len, "causal_period": period, "causal_offset": offset,
               "x_sha256": hashlib.sha256(x.tobytes()).hexdigest(),
               "y_sha256": hashlib.sha256(y.tobytes()).hexdigest()}
        if y.size <= 2048:
            rec["y_bits"] = [int(v) for v in y.view(np.uint32)]
        out[name] = rec
    return {"source": "oracle/sampler_oracle.js softmaxRows (V8 Math.exp, Math.fround)", "cases": out}


def hard_exp_f32_arguments(limit_bits: int = 46) -> np.ndarray:
    """Every f32 d in [-20, -2^-10) whose e^d (numpy's f64 exp) lies within 2^-limit_bits of
    its own size from a rounding boundary of f32 (the midpoint between two neighbours, or
    below a power of two the narrower one): the arguments where rounding a fast f64 exp to
    f32 could differ from rounding V8's. A scan of 120 M values (about 20 s)."""
    start = int(np.float32(-2.0 ** -10).view(np.uint32))
    stop = int(np.float32(-20.0).view(np.uint32))
    hits = []
    for lo in range(start, stop, 1 << 22):
        d = np.arange(lo, min(lo + (1 << 22), stop), dtype=np.uint64).astype(np.uint32).view(np.float32)
        e = np.exp(d.astype(np.float64))
        y = e.astype(np.float32)
        res = e - y.astype(np.float64)
        yb = y.view(np.uint32)
        ex = ((yb >> 23) & 0xFF).astype(np.int64)
        half = np.ldexp(1.0, np.maximum(ex, 1) - 151)
        half = np.where((res < 0) & ((yb & 0x7FFFFF) == 0) & (ex > 1), half * 0.5, half)
        hits.append(d[(half - np.abs(res)) / e < 2.0 ** -limit_bits])
    return np.concatenate(hits)


def exp_f32_vectors(o) -> dict:
    x = hard_exp_f32_arguments()
    y = o.node_exp(x.astype(np.float64)).astype(np.float32)  # fround(Math.exp(x)) in V8
    return {"source": "node Math.exp, rounded to f32 (Math.fround)",
            "x_bits": [int(v) for v in x.view(np.uint32)], "y_bits": [int(v) for v in y.view(np.uint32)]}


def main() -> None:
    import oracle as o

    if "--exp-f32" in sys.argv:
        with open(os.path.join(HERE, "exp_f32_hard.json"), "w") as f:
            json.dump(exp_f32_vectors(o), f, separators=(",", ":"))
        print("wrote exp_f32_hard.json")
        return

    if "--softmax" in sys.argv:
        with open(os.path.join(HERE, "softmax_vectors.json"), "w") as f:
            json.dump(softmax_vectors(o), f, separators=(",", ":"))
        print("wrote softmax_vectors.json")
        return

    if not o.node_available():
        raise SystemExit("node is required to write the golden vectors")
    vec = {"mulberry32": {}, "exp": {}, "workloads": {}, "topk_cap": TOPK_CAP}
    for seed in MULBERRY_SEEDS:
        vec["mulberry32"][str(seed)] = [float(v) for v in o.node_mulberry32(seed, 64)]
    x = exp_arguments()
    y = o.node_exp(x)
    vec["exp"] = {"x": [float(v) for v in x], "y": [float(v) for v in y]}
    for name in WORKLOADS:
        logits, k, t, p, u = workload(name)
        outs = o.node_sample_batch(logits, k, t, p, u, topk_cap=TOPK_CAP)
        vec["workloads"][name] = {
            "sha256": hashlib.sha256(logits.tobytes()).hexdigest(),
            "outcomes": outs,
        }
    with open(os.path.join(HERE, "node_vectors.json"), "w") as f:
        json.dump(vec, f, separators=(",", ":"))
    with open(os.path.join(HERE, "sampling_fixture.json"), "w") as f:
        json.dump(closed_form_fixture(), f, indent=1)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
