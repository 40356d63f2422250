"""Pins of the CPU oracle (oracle/tabby_oracle.c) -- CPU only.

Each part of the reference path is checked against something other than a retyping of its
own formula: the reference's hand fixture worked out in closed form, the Node restatement
running V8's own Math.exp and sort (committed vectors in tests/golden/, and live when node
is on PATH), brute force over tiny inputs, library routines (numpy's stable sort, numpy's
f16 widening), and inverse-CDF counting for the draw.
"""
import hashlib
import itertools
import json
import math
import os

import numpy as np
import pytest

from tabby_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def vectors():
    return _load("node_vectors.json")


@pytest.fixture(scope="module")
def fixture():
    return _load("sampling_fixture.json")


def _golden_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


# ---- mulberry32 (sampler.ts:105-119) -------------------------------------------------------

def test_mulberry32_matches_node_vectors(oracle, vectors):
    for seed, expected in vectors["mulberry32"].items():
        got = oracle.mulberry32(int(seed), len(expected))
        assert got.tolist() == expected, f"seed {seed}"


def test_mulberry32_closed_form_stream_matches_oracle(oracle):
    # synth's vectorised closed form (state = seed + i*golden) against the C stepper.
    for seed in (0, 3, 0x9E3779B9, 0xFFFFFFFF):
        assert np.array_equal(synth.mulberry32_stream(seed, 100_000), oracle.mulberry32(seed, 100_000))


def test_mulberry32_host_class_matches_oracle(oracle):
    from tabby_amd.sampler import SeededRandom
    rng = SeededRandom(12345)
    assert [rng.next() for _ in range(1000)] == oracle.mulberry32(12345, 1000).tolist()


@pytest.mark.skipif(not __import__("oracle").node_available(), reason="node not on PATH")
def test_mulberry32_million_outputs_match_node_live(oracle):
    for seed in (0, 42, 0xDEADBEEF):
        assert np.array_equal(oracle.node_mulberry32(seed, 1_000_000), oracle.mulberry32(seed, 1_000_000))


def test_mulberry32_outputs_are_32_bit_fractions(oracle):
    u = oracle.mulberry32(99, 50_000)
    assert np.all((u >= 0) & (u < 1))
    assert np.array_equal(u * 4294967296.0, np.floor(u * 4294967296.0))


# ---- exp: V8's Math.exp (fdlibm's method) -------------------------------------------------

def test_exp_matches_v8_vectors(oracle, vectors):
    x = np.array(vectors["exp"]["x"])
    y = np.array(vectors["exp"]["y"])
    got = oracle.exp_array(x)
    bad = np.nonzero(got.view(np.uint64) != y.view(np.uint64))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}"


@pytest.mark.skipif(not __import__("oracle").node_available(), reason="node not on PATH")
def test_exp_matches_v8_live(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-60, 1, 800_000), rng.uniform(-746, 710, 200_000)])
    bad = np.nonzero(oracle.exp_array(x).view(np.uint64) != oracle.node_exp(x).view(np.uint64))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r}"


def test_exp_special_values_and_accuracy(oracle):
    assert oracle.exp(0.0) == 1.0 and oracle.exp(-0.0) == 1.0
    assert oracle.exp(1.0) == math.e
    assert oracle.exp(float("-inf")) == 0.0 and oracle.exp(float("inf")) == float("inf")
    assert math.isnan(oracle.exp(float("nan")))
    assert oracle.exp(710.0) == float("inf") and oracle.exp(-746.0) == 0.0
    # Within 1 ulp of the correctly rounded value (fdlibm's bound), checked in extended
    # precision through expm1 of the small remainder around exact multiples of ln2.
    rng = np.random.default_rng(2)
    for x in rng.uniform(-700, 700, 2000):
        y = oracle.exp(float(x))
        ref = math.exp(x)
        assert abs(y - ref) <= 1.0 * math.ulp(ref), x


# ---- f16 widening (tests/support.ts:61-74) ------------------------------------------------

def test_f16_widening_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


# ---- top-k order (sampler.ts:25-30) and argmax (sampler.ts:13-23) --------------------------

def _definition_topk(row, k):
    """The reference comparator spelled as a sort key: value descending, id ascending."""
    return sorted(range(len(row)), key=lambda i: (-float(row[i]), i))[:k]


def test_topk_brute_force_all_tiny_tie_heavy_rows(oracle):
    values = np.array([-np.inf, -1.0, -0.0, 0.0, 0.5, 1.0], dtype=np.float32)
    for n in range(1, 6):
        for combo in itertools.product(range(len(values)), repeat=n):
            row = values[list(combo)]
            for k in range(1, n + 1):
                ids, vals = oracle.topk(row, k)
                assert ids.tolist() == _definition_topk(row, k), (row, k)
                assert np.array_equal(vals, row[ids])


def test_topk_matches_stable_library_sort(oracle):
    rng = np.random.default_rng(3)
    for trial in range(40):
        n = int(rng.integers(1, 5000))
        row = (np.round(rng.normal(0, 2, n) * 2) / 2).astype(np.float32)
        row[rng.random(n) < 0.2] = -np.inf
        row[row == 0] = np.where(rng.random(int((row == 0).sum())) < 0.5, 0.0, -0.0)
        k = int(rng.integers(1, n + 1))
        order = np.argsort(-row.astype(np.float64), kind="stable")[:k]
        ids, _ = oracle.topk(row, k)
        assert np.array_equal(ids, order), trial


def test_topk_special_rows(oracle):
    assert oracle.topk(np.full(100, 1.5, np.float32), 10)[0].tolist() == list(range(10))
    row = np.full(50, -np.inf, np.float32)
    assert oracle.topk(row, 5)[0].tolist() == [0, 1, 2, 3, 4]
    row = np.array([-0.0, 0.0, -0.0, -1.0], np.float32)  # -0 equals +0: ties go by id
    assert oracle.topk(row, 4)[0].tolist() == [0, 1, 2, 3]


def test_argmax_is_lowest_index_of_max(oracle):
    rng = np.random.default_rng(4)
    for _ in range(200):
        row = rng.integers(-3, 3, int(rng.integers(1, 300))).astype(np.float32)
        assert oracle.argmax(row) == int(np.argmax(row)) == int(oracle.topk(row, 1)[0][0])


# ---- sumExp (tests/sampling.test.ts:73-77) --------------------------------------------------

def test_sum_exp_is_sequential_f64_sum(oracle):
    rng = np.random.default_rng(5)
    row = rng.normal(0, 3, 10_000).astype(np.float32)
    m = float(row.max())
    s = oracle.sum_exp(row, m)
    assert math.isclose(s, math.fsum(math.exp(float(v) - m) for v in row), rel_tol=1e-13)
    assert oracle.sum_exp(np.zeros(7, np.float32), 0.0) == 7.0
    assert oracle.sum_exp(np.array([3.0, -np.inf], np.float32), 3.0) == 1.0


# ---- sampleFromTopK (sampler.ts:147-212): the reference's hand fixture ----------------------

def _fixture_case(oracle, fixture, case, uniform=0.0):
    top = fixture["top"]
    return oracle.sample_from_topk(top["ids"], top["logits"], top["maxLogit"], case["sumExp"],
                                   case["temperature"], case["topP"], uniform)


def test_fixture_outcomes_match_closed_forms(oracle, fixture):
    for case in fixture["cases"]:
        for u in (0.0, 0.3, 0.999):
            out = _fixture_case(oracle, fixture, case, u)
            for key, want in case["expect"].items():
                field = {"consideredCount": "considered", "poolMass": "pool_mass",
                         "poolExhausted": "pool_exhausted"}.get(key, key)
                got = out[field]
                if isinstance(want, float):
                    assert math.isclose(got, want, rel_tol=1e-15), (case["name"], key, got, want)
                else:
                    assert got == want, (case["name"], key, got, want)


def test_fixture_assertions_of_the_reference(oracle, fixture):
    cases = {c["name"]: c for c in fixture["cases"]}
    wide = _fixture_case(oracle, fixture, cases["wide (topP 1)"], 0.5)
    narrow = _fixture_case(oracle, fixture, cases["narrow (topP 0.5)"], 0.5)
    assert 1 <= narrow["considered"] < wide["considered"]
    clipped = _fixture_case(oracle, fixture, cases["clipped by k (sumExp 100)"], 0.5)
    assert clipped["pool_mass"] < 0.9 and clipped["pool_exhausted"]
    sp = fixture["spread"]
    top = fixture["top"]
    u = oracle.mulberry32(sp["seed"], sp["draws"])
    chosen = {oracle.sample_from_topk(top["ids"], top["logits"], top["maxLogit"], top["sumExp"],
                                      sp["temperature"], sp["topP"], float(x))["id"] for x in u}
    assert len(chosen) >= sp["min_distinct"]


def test_fixture_probability_is_exact_term_of_chosen(oracle, fixture):
    top = fixture["top"]
    w = fixture["weights_T1"]
    c = np.cumsum(w)
    for u in np.linspace(0, 0.999, 37):
        out = oracle.sample_from_topk(top["ids"], top["logits"], 10.0, 2.5, 1.0, 1.0, float(u))
        i = int(np.searchsorted(c, u * c[-1], side="right"))  # first i with u*total < c_i
        assert out["id"] == top["ids"][i]
        assert math.isclose(out["probability"], math.exp(-i) / 2.5, rel_tol=1e-15)


def test_greedy_does_not_depend_on_uniform(oracle, fixture):
    top = fixture["top"]
    a = oracle.sample_from_topk(top["ids"], top["logits"], 10.0, 2.5, 0.0, 0.9, 0.0)
    b = oracle.sample_from_topk(top["ids"], top["logits"], 10.0, 2.5, 0.0, 0.9, 0.99)
    assert a == b and a["id"] == 1 and a["considered"] == 1


def test_shift_invariance_of_the_tail(oracle, fixture):
    # Integer logits shifted by 700: every l - max is unchanged exactly, so every outcome
    # must be bit-identical (and nothing may overflow: the max is subtracted first).
    top = fixture["top"]
    shifted = [v + 700.0 for v in top["logits"]]
    for T, p, u in ((1.0, 1.0, 0.3), (0.5, 0.9, 0.8), (2.0, 0.5, 0.1), (0.0, 1.0, 0.5)):
        a = oracle.sample_from_topk(top["ids"], top["logits"], 10.0, 2.5, T, p, u)
        b = oracle.sample_from_topk(top["ids"], shifted, 710.0, 2.5, T, p, u)
        assert a == b, (T, p, u)
    row = np.array([3.0, 1.0, 2.0, 3.0, -1.0], np.float32)
    a = oracle.sample_row(row, 0, 0.7, 0.9, 0.6, topk_cap=5)
    b = oracle.sample_row(row + 700.0, 0, 0.7, 0.9, 0.6, topk_cap=5)
    assert a["sum_exp"] == b["sum_exp"] and a["id"] == b["id"] and a["probability"] == b["probability"]


def test_draw_intervals_are_half_open(oracle):
    # Four equal candidates: the weights are exactly 1/4 and every running sum is exact, so
    # u = j/4 lies on a boundary; u in [c_(i-1), c_i) picks i (sampler.ts: target < running).
    ids = np.array([7, 3, 9, 1], np.int32)
    logits = np.zeros(4, np.float32)
    for u, want in ((0.0, 7), (0.2, 7), (0.25, 3), (0.5, 9), (0.75, 1), (0.99, 1)):
        assert oracle.sample_from_topk(ids, logits, 0.0, 4.0, 1.0, 1.0, u)["id"] == want, u
    # Top-p reached exactly at a boundary: c_1 = 0.5 >= 0.5 cuts after two candidates.
    assert oracle.sample_from_topk(ids, logits, 0.0, 4.0, 1.0, 0.5, 0.9)["considered"] == 2


# ---- the draw: inverse CDF ------------------------------------------------------------------

def test_draw_is_inverse_cdf_over_a_grid(oracle):
    rng = np.random.default_rng(6)
    for trial in range(30):
        k = int(rng.integers(1, 12))
        logits = np.sort(rng.normal(0, 2, k).astype(np.float32))[::-1].copy()
        ids = rng.permutation(1000)[:k].astype(np.int32)
        T = float(rng.choice([0.3, 0.7, 1.0, 2.5]))
        p = float(rng.choice([0.5, 0.8, 1.0]))
        m = float(logits[0])
        s = np.array([math.exp((float(l) - m) / T) for l in logits])
        w = s / s.sum()
        c = np.cumsum(w)
        cut = k if p >= 1.0 else int(np.argmax(c >= p)) + 1 if np.any(c >= p) else k
        grid = (np.arange(400) + 0.5) / 400
        counts = np.zeros(k)
        for u in grid:
            out = oracle.sample_from_topk(ids, logits, m, 10.0, T, p, float(u))
            j = int(np.nonzero(ids == out["id"])[0][0])
            assert j < cut and out["considered"] == cut
            counts[j] += 1
        # Each kept candidate owns a share of [0,1) equal to its weight over the kept mass.
        share = w[:cut] / c[cut - 1]
        assert np.all(np.abs(counts[:cut] / len(grid) - share) <= 1.0 / len(grid) + 1e-12), trial


# ---- whole rows: the C oracle against the Node restatement ---------------------------------

def _compare_outcome(name, r, o, n):
    assert o["id"] == n["id"], (name, r)
    assert o["considered"] == n["consideredCount"], (name, r)
    assert o["probability"] == n["probability"], (name, r)
    assert o["pool_mass"] == n["poolMass"], (name, r)
    assert bool(o["pool_exhausted"]) == n["poolExhausted"], (name, r)
    assert o["sum_exp"] == n["sumExp"] and o["max_logit"] == n["maxLogit"], (name, r)
    assert o["topk_ids"].tolist() == n["topIds"], (name, r)


def test_golden_workloads_regenerate_bit_for_bit(vectors):
    g = _golden_module()
    for name, entry in vectors["workloads"].items():
        logits = g.workload(name)[0]
        assert hashlib.sha256(logits.tobytes()).hexdigest() == entry["sha256"], name


def test_c_oracle_matches_node_vectors(oracle, vectors):
    g = _golden_module()
    cap = vectors["topk_cap"]
    for name, entry in vectors["workloads"].items():
        logits, k, t, p, u = g.workload(name)
        outs = oracle.sample_batch(logits, k, t, p, u, topk_cap=cap)
        for r, (o, n) in enumerate(zip(outs, entry["outcomes"])):
            _compare_outcome(name, r, o, n)


@pytest.mark.skipif(not __import__("oracle").node_available(), reason="node not on PATH")
def test_c_oracle_matches_node_live_on_benchmark_shapes(oracle):
    # A slice of config 3 (full vocabulary width) and tie/-inf rows of config 5.
    for w in (synth.config(3, rows=6), synth.config(5, rows=3), synth.config(4, rows=2)):
        lf = w.logits_f32()
        outs = oracle.sample_batch(lf, w.top_k, w.temperature, w.top_p, w.uniform, topk_cap=20)
        node = oracle.node_sample_batch(lf, w.top_k, w.temperature, w.top_p, w.uniform, topk_cap=20)
        for r, (o, n) in enumerate(zip(outs, node)):
            _compare_outcome(w.name, r, o, n)


def test_rows_outside_the_contract_are_flagged(oracle):
    row = np.zeros(10, np.float32)
    row[3] = np.nan
    assert oracle.sample_row(row, 5, 0.7, 0.9, 0.5)["status"] != 0
    assert oracle.sample_row(np.full(10, -np.inf, np.float32), 5, 0.7, 0.9, 0.5)["status"] != 0


# ---- softmaxRows (src/reference/cpu.ts:238-264) --------------------------------------------

def _same_f32(a_bits, b_bits):
    """Bitwise equality of f32 arrays (as uint32), any NaN equal to any NaN: a NaN's sign and
    payload are not part of the result (V8 stores one canonical NaN, x86 arithmetic makes
    another)."""
    a = np.asarray(a_bits, np.uint32)
    b = np.asarray(b_bits, np.uint32)
    nan_a = (a & 0x7FFFFFFF) > 0x7F800000
    nan_b = (b & 0x7FFFFFFF) > 0x7F800000
    return (a == b) | (nan_a & nan_b)


def _canonical_nan(y):
    """A copy with every NaN as the one quiet NaN V8 stores (0x7FC00000)."""
    y = np.array(y, dtype=np.float32)
    y[np.isnan(y)] = np.float32("nan")
    return y


@pytest.fixture(scope="module")
def softmax_vectors():
    return _load("softmax_vectors.json")


def test_softmax_matches_node_vectors(oracle, softmax_vectors):
    # Bit for bit against the Node restatement (V8's Math.exp and Math.fround), committed.
    gm = _golden_module()
    for name, rec in softmax_vectors["cases"].items():
        x = gm.softmax_input(name)
        assert hashlib.sha256(x.tobytes()).hexdigest() == rec["x_sha256"], name
        y = oracle.softmax_rows(x, rec["n_rows"], rec["row_len"], rec["causal_period"],
                                rec["causal_offset"])
        if "y_bits" in rec:
            want = np.asarray(rec["y_bits"], np.uint32)
            bad = np.nonzero(~_same_f32(y.view(np.uint32), want))[0]
            assert bad.size == 0, f"{name}: {bad.size} entries differ, first at {bad[:5]}"
        else:
            assert hashlib.sha256(_canonical_nan(y).tobytes()).hexdigest() == rec["y_sha256"], name


@pytest.mark.skipif(not __import__("oracle").node_available(), reason="node not on PATH")
def test_softmax_matches_node_live(oracle):
    rng = np.random.default_rng(5)
    for n_rows, row_len, period, offset in ((40, 37, 8, 29), (5, 4100, 0, 0), (33, 1, 0, 0)):
        x = (rng.normal(0, 6, n_rows * row_len)).astype(np.float32)
        a = oracle.softmax_rows(x, n_rows, row_len, period, offset)
        b = oracle.node_softmax_rows(x, n_rows, row_len, period, offset)
        assert np.all(_same_f32(a.view(np.uint32), b.view(np.uint32))), (n_rows, row_len)


def test_softmax_closed_forms(oracle):
    # n equal entries: every exp is exp(0) = 1, the f32 sum is n (exact), out = fround(1 / n).
    for n in (1, 2, 3, 7, 64, 1000):
        y = oracle.softmax_rows(np.full(n, -3.25, np.float32), 1, n)
        assert np.all(y == np.float32(1.0 / n)), n
    # One finite entry among -inf: exp(-inf - m) = 0 elsewhere.
    x = np.full(9, -np.inf, np.float32)
    x[4] = 0.5
    assert oracle.softmax_rows(x, 1, 9).tolist() == [0, 0, 0, 0, 1, 0, 0, 0, 0]
    # Two entries ln 3 apart: weights 3/4 and 1/4 up to f32 rounding.
    y = oracle.softmax_rows(np.array([math.log(3.0), 0.0], np.float32), 1, 2)
    assert abs(y[0] - 0.75) < 2e-7 and abs(y[1] - 0.25) < 2e-7
    # A NaN or +inf entry makes the row's valid prefix NaN (Math.max propagates NaN;
    # inf - inf is NaN); all -inf is NaN too (-inf - -inf). The masked rest is still 0.
    for bad in (np.nan, np.inf):
        x = np.array([1.0, bad, 2.0, 0.5, 0.25, -1.0], np.float32)
        y = oracle.softmax_rows(x, 2, 3, 2, 1)  # row 0 covers 2 entries, row 1 all 3
        assert np.isnan(y[0]) and np.isnan(y[1]) and y[2] == 0 and np.all(np.isfinite(y[3:]))
    assert np.all(np.isnan(oracle.softmax_rows(np.full(3, -np.inf, np.float32), 1, 3)))


def test_softmax_reference_kernel_test_assertions(oracle):
    # tests/kernels.test.ts:457-487 on its own input: masked entries exactly 0, each row's
    # valid prefix sums to 1 to 5 decimals, and every entry within 1e-6 of the f64 softmax.
    gm = _golden_module()
    x = gm.softmax_input("reference_causal_3x5")
    y = oracle.softmax_rows(x, 15, 5, 5, 0).reshape(15, 5)
    xs = x.reshape(15, 5).astype(np.float64)
    for row in range(15):
        valid = row % 5 + 1
        assert np.all(y[row, valid:] == 0)
        assert abs(float(np.sum(y[row].astype(np.float64))) - 1.0) < 5e-6
        e = np.exp(xs[row, :valid] - xs[row, :valid].max())
        assert np.max(np.abs(y[row, :valid] - e / e.sum())) < 1e-6


def test_softmax_rows_match_float64_math(oracle):
    # Against numpy's f64 softmax: the f32 steps stay within the error of an f32 sequential
    # sum of `valid` terms (valid * 2^-24 relative) plus a few ulps. Scores near +120 make
    # exp overflow f32 unless the max is subtracted first; a wrong mask or a sum over the
    # wrong range fails too.
    rng = np.random.default_rng(11)
    for n_rows, row_len, period, offset, shift in ((12, 50, 4, 46, 0.0), (6, 2000, 0, 0, 120.0),
                                                   (16, 16, 16, 0, -60.0)):
        x = (rng.normal(0, 5, (n_rows, row_len)) + shift).astype(np.float32)
        y = oracle.softmax_rows(x.reshape(-1), n_rows, row_len, period, offset).reshape(n_rows, row_len)
        for r in range(n_rows):
            valid = offset + r % period + 1 if period else row_len
            v = x[r, :valid].astype(np.float64)
            e = np.exp(v - v.max())
            ref = e / e.sum()
            tol = (valid * 2.0 ** -24 + 1e-6) * np.maximum(ref, 1e-3)
            assert np.all(np.abs(y[r, :valid] - ref) <= tol), (r, valid)
            assert np.all(y[r, valid:] == 0)


def test_exp_rounded_to_f32_on_hard_arguments(oracle):
    # fround(Math.exp(x)) where e^x sits within 2^-46 of an f32 rounding boundary: the oracle's
    # exp (bit for bit V8's) rounded to f32 gives V8's answers (committed from Node).
    d = _load("exp_f32_hard.json")
    x = np.asarray(d["x_bits"], np.uint32).view(np.float32)
    want = np.asarray(d["y_bits"], np.uint32)
    got = oracle.exp_array(x.astype(np.float64)).astype(np.float32).view(np.uint32)
    assert x.size >= 40 and np.array_equal(got, want)


# ---- matmulQuantized (src/reference/cpu.ts:352-393) ----------------------------------------

def _dequant_f64(words, scales, out_dim, in_dim, bits, block):
    per = 8 if bits == 4 else 4
    shift = 32 // per
    raw = np.stack([(words >> np.uint32(shift * j)) & np.uint32((1 << shift) - 1) for j in range(per)], 1)
    raw = raw.reshape(out_dim, in_dim).astype(np.float64)
    centred = raw - 8 if bits == 4 else np.where(raw > 127, raw - 256, raw)
    return centred * np.repeat(np.asarray(scales, np.float64).reshape(out_dim, in_dim // block), block, axis=1)


def test_matmul_quantized_on_the_reference_test_shapes(oracle):
    # tests/quant.test.ts:122-177: weights randomF32(rows * cols, seed, 0.05) quantized by
    # quantizeQ4, f16-rounded scales, x = randomF32(cols, seed ^ 0x1234); the reference
    # accepts a max abs error of 1e-4 against matmulQuantized. Here: the C restatement and
    # the Node one (Math.fround) agree bit for bit, and both are within the f32 steps' error
    # of the f64 product of the dequantized weights.
    for rows, cols in ((8, 32), (17, 96), (64, 896), (896, 4864)):
        seed = rows * 31 + cols
        w = synth.random_f32(rows * cols, seed, 0.05)
        words, _, scales = synth.quantize_q4(w, rows, cols, 32)
        x = synth.random_f32(cols, seed ^ 0x1234)
        y = oracle.matmul_quantized(words, scales, x, rows, cols)
        if oracle.node_available():
            yn = oracle.node_matmul_quantized(words, scales, x, rows, cols)
            assert np.array_equal(y.view(np.uint32), yn.view(np.uint32)), (rows, cols)
        W = _dequant_f64(words, scales, rows, cols, 4, 32)
        ref = x.astype(np.float64) @ W.T
        bound = (np.abs(x.astype(np.float64)) @ np.abs(W).T) * cols * 2.0 ** -23 + 1e-12
        assert np.all(np.abs(y[0] - ref) <= bound), (rows, cols)
        assert np.max(np.abs(y[0] - ref)) < 1e-4


def test_matmul_quantized_bias_bits8_and_batches(oracle):
    rng = np.random.default_rng(3)
    out_dim, in_dim = 40, 128
    for bits, block in ((4, 32), (4, 64), (8, 32), (8, 128)):
        words = rng.integers(0, 2 ** 32, out_dim * in_dim * bits // 32, dtype=np.uint64).astype(np.uint32)
        scales = rng.normal(0, 0.01, out_dim * in_dim // block).astype(np.float16).astype(np.float32)
        bias = rng.normal(0, 1, out_dim).astype(np.float32)
        x = rng.normal(0, 2, (3, in_dim)).astype(np.float32)
        y = oracle.matmul_quantized(words, scales, x, out_dim, in_dim, bits, block, bias)
        ref = x.astype(np.float64) @ _dequant_f64(words, scales, out_dim, in_dim, bits, block).T + bias
        assert np.max(np.abs(y - ref)) < 1e-4, (bits, block)
        if oracle.node_available():
            yn = oracle.node_matmul_quantized(words, scales, x, out_dim, in_dim, bits, block, bias)
            assert np.array_equal(y.view(np.uint32), yn.view(np.uint32)), (bits, block)


def test_matmul_quantized_closed_form(oracle):
    # One word of codes 0..7 (values -8..-1) against x = 1..8 and scale 0.5, and one of 8..15
    # (values 0..7) against x = 1: partial sums are small integers, exact in f32.
    words = np.array([0x76543210, 0xFEDCBA98, 0x00000000, 0x88888888], np.uint32)
    scales = np.array([0.5], np.float32)
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 2, 2, 2, 2, 2, 2, 9, 9, 9, 9, 9, 9, 9, 9],
                 np.float32)
    y = oracle.matmul_quantized(words, scales, x, 1, 32)
    # sum((j - 8) * (j + 1)) = -120; sum(j for j in 0..7) = 28; 8 * (-8) * 2 = -128; codes 8 -> 0.
    assert y.tolist() == [[(-120 + 28 - 128 + 0) * 0.5]]
