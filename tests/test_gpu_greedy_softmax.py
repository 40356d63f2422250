"""GPU parity of the greedy fast path (tabby_argmax_device) and the attention row softmax
(tabby_softmax_rows_device), through the C ABI, against the CPU oracle: ids bit-exact
(argmax, src/engine/sampler.ts:13-23), softmax outputs bit-exact (softmaxRows,
src/reference/cpu.ts:238-264; any NaN equal to any NaN)."""
import os

import numpy as np
import pytest

from tabby_amd import sampler as S

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _torch():
    import torch
    assert torch.cuda.is_available(), "needs an MI355X"
    return torch


def _same_f32(a, b):
    a = np.asarray(a, np.float32).view(np.uint32)
    b = np.asarray(b, np.float32).view(np.uint32)
    nan_a = (a & 0x7FFFFFFF) > 0x7F800000
    nan_b = (b & 0x7FFFFFFF) > 0x7F800000
    return (a == b) | (nan_a & nan_b)


# ---- argmax --------------------------------------------------------------------------------

def _gpu_argmax(logits_np, dtype="f32"):
    torch = _torch()
    rows, vocab = logits_np.shape
    x = torch.from_numpy(logits_np.astype(np.float16 if dtype == "f16" else np.float32)).cuda()
    ids = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    mx = torch.zeros(rows, dtype=torch.float32, device="cuda")
    with S.GpuSampler(vocab_max=vocab, rows_max=rows, k_max=64) as g:
        g.argmax_device(x, ids, mx)
        torch.cuda.synchronize()
    return ids.cpu().numpy(), mx.cpu().numpy()


@pytest.mark.parametrize("rows,vocab", [(1, 1), (1, 7), (3, 4096), (1, 49152), (1, 151936), (64, 151936),
                                        (256, 151936), (300, 100003), (5, 151937), (1024, 2048)])
def test_argmax_matches_oracle(oracle, rows, vocab):
    rng = np.random.default_rng(rows * 1000 + vocab)
    # Integer values: many exact ties, so the lowest-index rule decides most rows.
    logits = rng.integers(-40, 40, (rows, vocab)).astype(np.float32)
    print(f"argmax rows={rows} vocab={vocab}", flush=True)
    ids, mx = _gpu_argmax(logits)
    want = np.array([oracle.argmax(logits[r]) for r in range(rows)])
    assert np.array_equal(ids, want), np.nonzero(ids != want)[0][:5]
    assert np.array_equal(mx, logits[np.arange(rows), want])


def test_argmax_special_rows(oracle):
    vocab = 5000
    rows = []
    r = np.full(vocab, -np.inf, np.float32); rows.append(r)                  # all -inf -> 0
    r = np.full(vocab, -np.inf, np.float32); r[0] = np.nan; r[9] = 3; rows.append(r)  # NaN first -> 0
    r = np.zeros(vocab, np.float32); r[1::2] = -0.0; rows.append(r)          # +0/-0 equal -> 0
    r = np.full(vocab, -1.0, np.float32); r[100] = np.nan; r[4999] = 2; rows.append(r)  # NaN skipped
    r = np.full(vocab, 7.5, np.float32); rows.append(r)                       # all equal -> 0
    r = np.full(vocab, np.nan, np.float32); r[3] = -np.inf; rows.append(r)    # NaN first, -inf -> 0
    r = np.full(vocab, np.nan, np.float32); r[0] = -np.inf; r[77] = -5; rows.append(r)  # -> 77
    r = np.full(vocab, -3.0, np.float32); r[4096] = np.inf; r[4097] = np.inf; rows.append(r)  # +inf -> 4096
    r = -np.arange(vocab, dtype=np.float32)[::-1].copy(); rows.append(r)     # max at the end
    logits = np.stack(rows)
    ids, mx = _gpu_argmax(logits)
    want = np.array([oracle.argmax(logits[i]) for i in range(len(rows))])
    assert want.tolist() == [0, 0, 0, 4999, 0, 0, 77, 4096, vocab - 1]
    assert np.array_equal(ids, want)
    assert np.all(_same_f32(mx, logits[np.arange(len(rows)), want]))


@pytest.mark.parametrize("rows,vocab", [(64, 151936), (64, 4099), (256, 151936), (260, 4099)])
def test_argmax_f16(oracle, rows, vocab):
    rng = np.random.default_rng(vocab + rows)
    h = rng.normal(0, 3, (rows, vocab)).astype(np.float16)
    h[5, :] = np.float16(1.0)
    h[6, 123] = np.float16(np.nan)
    ids, mx = _gpu_argmax(h, "f16")
    wide = h.astype(np.float32)
    want = np.array([oracle.argmax(wide[r]) for r in range(rows)])
    assert np.array_equal(ids, want)
    assert np.array_equal(mx, wide[np.arange(rows), want])


def test_argmax_agrees_with_greedy_sampling(oracle):
    # The one-candidate pool's id (sampleFromTopK at T = 0) is the argmax.
    torch = _torch()
    from tabby_amd import synth
    w = synth.config(3, rows=32)
    x = torch.from_numpy(w.logits).cuda()
    with S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=64) as g:
        params = np.zeros(w.rows, dtype=S.PARAMS_DTYPE)
        params["temperature"], params["top_k"], params["top_p"] = 0.0, 1, 1.0
        res, _, _ = g.sample_params(x, params)
        ids = g.argmax(x)
    assert ids == res["id"].tolist()
    assert ids == [oracle.argmax(w.logits[r]) for r in range(w.rows)]


def test_argmax_rejects_beyond_the_handle():
    torch = _torch()
    x = torch.zeros((4, 100), dtype=torch.float32, device="cuda")
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    with S.GpuSampler(vocab_max=100, rows_max=2, k_max=8) as g:
        with pytest.raises(S.SamplingError) as e:
            g.argmax_device(x, ids)
        assert e.value.status == S.TABBY_ECAPACITY


# ---- softmax_rows --------------------------------------------------------------------------

def _gpu_softmax(x_np, n_rows, row_len, period=0, offset=0, in_place=False):
    torch = _torch()
    x = torch.from_numpy(np.ascontiguousarray(x_np, np.float32).reshape(-1)).cuda()
    if in_place:
        y = S.softmax_rows(x, n_rows, row_len, period, offset, out=x)
        assert y.data_ptr() == x.data_ptr()
    else:
        y = S.softmax_rows(x, n_rows, row_len, period, offset)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _check_softmax(oracle, x, n_rows, row_len, period=0, offset=0, in_place=False):
    print(f"softmax n_rows={n_rows} row_len={row_len} period={period} offset={offset} "
          f"in_place={in_place}", flush=True)
    got = _gpu_softmax(x, n_rows, row_len, period, offset, in_place)
    want = oracle.softmax_rows(x, n_rows, row_len, period, offset)
    bad = np.nonzero(~_same_f32(got, want))[0]
    assert bad.size == 0, (f"{bad.size} of {want.size} differ; first at {bad[0]}: "
                           f"gpu {got[bad[0]]!r} oracle {want[bad[0]]!r}")


def test_softmax_golden_cases(oracle):
    import importlib.util
    import json
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
    gm = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gm)
    with open(os.path.join(HERE, "golden", "softmax_vectors.json")) as f:
        cases = json.load(f)["cases"]
    for name, rec in cases.items():
        x = gm.softmax_input(name)
        got = _gpu_softmax(x, rec["n_rows"], rec["row_len"], rec["causal_period"], rec["causal_offset"])
        if "y_bits" in rec:
            want = np.asarray(rec["y_bits"], np.uint32).view(np.float32)
            assert np.all(_same_f32(got, want)), name
        _check_softmax(oracle, x, rec["n_rows"], rec["row_len"], rec["causal_period"], rec["causal_offset"])


@pytest.mark.parametrize("row_len", [1, 3, 4, 64, 100, 256, 260, 512, 1000, 1024, 2048, 3000, 4096, 4097, 10000])
def test_softmax_every_row_length(oracle, row_len):
    rng = np.random.default_rng(row_len)
    n_rows = 9
    x = rng.normal(0, 4, n_rows * row_len).astype(np.float32)
    _check_softmax(oracle, x, n_rows, row_len)
    period = min(n_rows, row_len)
    _check_softmax(oracle, x, n_rows, row_len, period, row_len - period)


@pytest.mark.parametrize("row_len", [1, 3, 100, 257, 511, 512])
def test_softmax_many_short_rows(oracle, row_len):
    # Batches of at least 256 rows of at most 512 entries take the lane-per-row kernel:
    # a ragged last block, causal prefixes, in place and not, ties and NaN rows.
    rng = np.random.default_rng(row_len + 40)
    n_rows = 256 + 37
    x = rng.normal(0, 4, (n_rows, row_len)).astype(np.float32)
    x[5] = np.round(x[5])
    x[6, row_len // 2] = np.nan
    x = x.reshape(-1)
    _check_softmax(oracle, x, n_rows, row_len)
    _check_softmax(oracle, x, n_rows, row_len, min(row_len, 64), row_len - min(row_len, 64), in_place=True)


@pytest.mark.parametrize("row_len", [512, 4096, 6000])
def test_softmax_in_place(oracle, row_len):
    rng = np.random.default_rng(row_len + 1)
    x = rng.normal(0, 2, 40 * row_len).astype(np.float32)
    _check_softmax(oracle, x, 40, row_len, in_place=True)
    _check_softmax(oracle, x, 40, row_len, 8, row_len - 8, in_place=True)


@pytest.mark.parametrize("row_len", [300, 2048, 5000])
def test_softmax_ties_and_underflow(oracle, row_len):
    # Quantised scores: long runs of equal exps, so the f32 running sum meets exact half-ulp
    # ties; scores spread over [-120, 0]: exps down to subnormal f32 and zero.
    rng = np.random.default_rng(row_len + 2)
    q = (rng.integers(-16, 16, 16 * row_len) * 0.5).astype(np.float32)
    _check_softmax(oracle, q, 16, row_len)
    ones = np.zeros(4 * row_len, np.float32)  # all exps 1: the sum crosses every power of two
    _check_softmax(oracle, ones, 4, row_len)
    wide = (-rng.random(16 * row_len) * 120.0).astype(np.float32)
    _check_softmax(oracle, wide, 16, row_len)


def test_softmax_attention_shapes(oracle):
    # Prefill (14 heads x 512 queries over 512 positions, causal) and decode steps (14 heads x
    # 1 query over a growing cache: causal_offset = posStart).
    rng = np.random.default_rng(3)
    x = rng.normal(0, 3, 14 * 512 * 512).astype(np.float32)
    _check_softmax(oracle, x, 14 * 512, 512, 512, 0)
    for total in (1, 17, 1024, 4095, 8191):
        y = rng.normal(0, 3, 14 * total).astype(np.float32)
        _check_softmax(oracle, y, 14, total, 1, total - 1)


def test_softmax_special_rows(oracle):
    row_len = 300
    x = np.random.default_rng(9).normal(0, 1, (6, row_len)).astype(np.float32)
    x[0, 17] = np.nan
    x[1, 299] = np.inf
    x[2, :] = -np.inf
    x[3, :] = -np.inf
    x[3, 150] = 1e30
    x[4, :] = np.where(np.arange(row_len) % 2 == 0, 0.0, -0.0)
    x[5, :] = np.float32(3.0e38)
    _check_softmax(oracle, x.reshape(-1), 6, row_len)
    _check_softmax(oracle, x.reshape(-1), 6, row_len, 6, 200)


def test_softmax_rejects_bad_arguments():
    torch = _torch()
    x = torch.zeros(40, dtype=torch.float32, device="cuda")
    with pytest.raises(S.SamplingError) as e:
        S.softmax_rows(x, 4, 10, 4, 7)  # the last row would cover 11 > 10 entries
    assert e.value.status == S.TABBY_EINVAL
    lib = S.load_library()
    import ctypes
    rc = lib.tabby_softmax_rows_device(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr() + 8),
                                       4, 10, 0, 0, None)
    assert rc == S.TABBY_EINVAL  # out overlaps x without being x


def test_device_exp_f32_matches_v8(oracle):
    # The softmax's f32 exps: the fast f64 exp with its rounding check, against fround of the
    # oracle's (V8's) exp -- on the committed arguments closest to an f32 rounding boundary
    # (the check's fallback path), a million random ones, and special values.
    import json
    torch = _torch()
    with open(os.path.join(HERE, "golden", "exp_f32_hard.json")) as f:
        hard = np.asarray(json.load(f)["x_bits"], np.uint32).view(np.float32)
    rng = np.random.default_rng(17)
    rand = np.concatenate([-rng.random(600_000) * 20, -rng.random(300_000) * 110,
                           -rng.random(100_000) * 1e-6]).astype(np.float32)
    special = np.array([0.0, -0.0, -np.inf, np.nan, -87.3, -88.7, -103.2, -103.97, -104.0, -149 * 0.6931,
                        -745.2, -1e30, -np.finfo(np.float32).tiny], np.float32)
    x = np.concatenate([hard, rand, special])
    got = S.device_exp_f32(torch.from_numpy(x).cuda()).cpu().numpy()
    want = oracle.exp_array(x.astype(np.float64)).astype(np.float32)
    bad = np.nonzero(~_same_f32(got, want))[0]
    assert bad.size == 0, (f"{bad.size} differ; first x={x[bad[0]]!r}: device {got[bad[0]]!r} "
                           f"oracle {want[bad[0]]!r}")


def test_softmax_row_of_hard_exp_arguments(oracle):
    import json
    with open(os.path.join(HERE, "golden", "exp_f32_hard.json")) as f:
        hard = np.asarray(json.load(f)["x_bits"], np.uint32).view(np.float32)
    row = np.concatenate([[0.0], hard]).astype(np.float32)  # x - max = x exactly
    _check_softmax(oracle, row, 1, row.size)
    many = np.tile(row, 1100)
    _check_softmax(oracle, many, 1100, row.size)
