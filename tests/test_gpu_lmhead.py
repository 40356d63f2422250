"""GPU parity of the lm_head path through the C ABI: the int4 matmul (tabby_lmhead_q4_device)
bit for bit against the CPU restatement of matmulQuantized (src/reference/cpu.ts:352-393),
and the lm_head fused with sampling (tabby_sampler_sample_lmhead_q4_device) against the oracle
sampler on the oracle's logits: ids and consideredCount exact, probability / poolMass /
sumExp within 1e-5 relative, maxLogit exact."""
import numpy as np
import pytest

from tabby_amd import sampler as S
from tabby_amd import synth

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    assert torch.cuda.is_available(), "needs an MI355X"
    return torch


_HEADS = {}


def _head(vocab, hidden, block, seed=7, bias=False):
    key = (vocab, hidden, block, seed, bias)
    if key not in _HEADS:
        words, f16, f32 = synth.lm_head_q4(vocab, hidden, block, seed)
        b = np.random.default_rng(seed).normal(0, 0.5, vocab).astype(np.float32) if bias else None
        _HEADS[key] = (S.LmHeadQ4(words, f16, vocab, hidden, block, bias=b), words, f32, b)
    return _HEADS[key]


@pytest.mark.parametrize("rows,cols", [(8, 32), (17, 96), (64, 896), (896, 4864)])
def test_gemv_on_the_reference_test_shapes(oracle, rows, cols):
    # tests/quant.test.ts:122-177's cases (rows = output rows, cols = the reduction), quantized
    # the reference's way; bit for bit (the reference asks 1e-4).
    torch = _torch()
    seed = rows * 31 + cols
    w = synth.random_f32(rows * cols, seed, 0.05)
    words, f16, f32 = synth.quantize_q4(w, rows, cols, 32)
    x = synth.random_f32(cols, seed ^ 0x1234).reshape(1, cols)
    head = S.LmHeadQ4(words, f16, rows, cols, 32)
    got = head.logits(torch.from_numpy(x).cuda()).cpu().numpy()
    want = oracle.matmul_quantized(words, f32, x, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows", [1, 3, 8, 11])
@pytest.mark.parametrize("block,bias", [(32, False), (64, True), (128, False)])
def test_gemv_lm_head_shape(oracle, rows, block, bias):
    # Qwen2.5-0.5B's lm_head: 151,936 x 896; eleven rows take two passes over the weights.
    torch = _torch()
    vocab, hidden = 151936, 896
    head, words, f32, b = _head(vocab, hidden, block, bias=bias)
    x = synth.hidden_states(rows, hidden, seed=rows)
    print(f"gemv rows={rows} block={block} bias={bias}", flush=True)
    got = head.logits(torch.from_numpy(x).cuda()).cpu().numpy()
    want = oracle.matmul_quantized(words, f32, x, vocab, hidden, 4, block, b)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad[0].size == 0, (bad[0].size, got[bad][:3], want[bad][:3])


def _params(rows, seed, k_choices=(1, 7, 40, 64), ts=(0.0, 0.7, 1.3), ps=(0.8, 0.95, 1.0)):
    u = synth.mulberry32_stream(seed, 4 * rows).reshape(rows, 4)
    p = np.zeros(rows, dtype=S.PARAMS_DTYPE)
    p["top_k"] = np.asarray(k_choices)[(u[:, 0] * len(k_choices)).astype(int)]
    p["temperature"] = np.asarray(ts)[(u[:, 1] * len(ts)).astype(int)]
    p["top_p"] = np.asarray(ps)[(u[:, 2] * len(ps)).astype(int)]
    p["uniform"] = u[:, 3]
    return p


def _check_rows(oracle, res, logits, params, ctx):
    for r in range(len(params)):
        o = oracle.sample_row(logits[r], int(params[r]["top_k"]), float(params[r]["temperature"]),
                              float(params[r]["top_p"]), float(params[r]["uniform"]))
        g = res[r]
        c = f"{ctx} row {r} k={params[r]['top_k']} T={params[r]['temperature']} p={params[r]['top_p']}"
        assert int(g["status"]) == 0, c
        assert int(g["id"]) == o["id"], c
        assert int(g["considered"]) == o["considered"], c
        assert np.float32(g["max_logit"]) == np.float32(o["max_logit"]), c
        for f in ("probability", "pool_mass", "sum_exp"):
            assert abs(float(g[f]) - o[f]) <= 1e-5 * abs(o[f]), (c, f, float(g[f]), o[f])
        assert bool(g["pool_exhausted"]) == o["pool_exhausted"] or abs(o["pool_mass"] - params[r]["top_p"]) < 1e-5, c


@pytest.mark.parametrize("vocab,hidden,rows", [(151936, 896, 1), (151936, 896, 8), (151936, 896, 5),
                                               (50000, 896, 3), (100, 64, 2), (1024, 32, 4), (2048 + 7, 128, 8)])
def test_fused_lm_head_sampling_matches_oracle(oracle, vocab, hidden, rows):
    torch = _torch()
    head, words, f32, b = _head(vocab, hidden, 32, seed=vocab + hidden)
    x = synth.hidden_states(rows, hidden, seed=vocab + rows)
    params = _params(rows, vocab * 7 + rows)
    logits = oracle.matmul_quantized(words, f32, x, vocab, hidden)
    print(f"fused vocab={vocab} hidden={hidden} rows={rows}", flush=True)
    with S.GpuSampler(vocab_max=vocab, rows_max=8, k_max=64) as g:
        res = g.sample_lmhead_q4(head, torch.from_numpy(x).cuda(), params)
    _check_rows(oracle, res, logits, params, f"vocab {vocab}")


def test_fused_matches_unfused_on_the_device(oracle):
    # The fused pass against the unfused one (the matmul writes logits, the sampler reads them)
    # on the same device weights: ids, counts and the exact maxLogit equal; many draws.
    torch = _torch()
    vocab, hidden, rows = 151936, 896, 8
    head, _, _, _ = _head(vocab, hidden, 32)
    x = torch.from_numpy(synth.hidden_states(rows, hidden, seed=99)).cuda()
    with S.GpuSampler(vocab_max=vocab, rows_max=rows, k_max=64) as g:
        logits = head.logits(x)
        for trial in range(6):
            params = _params(rows, 1000 + trial, ts=(0.5, 1.0, 2.0), ps=(0.9, 0.99))
            fused = g.sample_lmhead_q4(head, x, params)
            plain, _, _ = g.sample_params(logits, params)
            for f in ("id", "considered", "status", "max_logit"):
                assert np.array_equal(fused[f], plain[f]), (trial, f)
            for f in ("probability", "pool_mass", "sum_exp"):
                assert np.allclose(fused[f], plain[f], rtol=2e-5, atol=0), (trial, f)


def test_fused_rows_outside_its_pools_report_einval(oracle):
    torch = _torch()
    vocab, hidden = 4096, 64
    head, words, f32, _ = _head(vocab, hidden, 32)
    x = synth.hidden_states(4, hidden, seed=5)
    params = _params(4, 77, k_choices=(40,))
    params["top_k"] = [40, 0, 65, 1]
    with S.GpuSampler(vocab_max=vocab, rows_max=4, k_max=128) as g:
        res = g.sample_lmhead_q4(head, torch.from_numpy(x).cuda(), params)
    assert res["status"].tolist() == [0, S.TABBY_EINVAL, S.TABBY_EINVAL, 0]
    logits = oracle.matmul_quantized(words, f32, x, vocab, hidden)
    _check_rows(oracle, res[[0, 3]], logits[[0, 3]], params[[0, 3]], "in-contract rows")


def test_fused_rejects_more_than_eight_rows():
    torch = _torch()
    head, _, _, _ = _head(4096, 64, 32)
    x = torch.zeros((9, 64), dtype=torch.float32, device="cuda")
    with S.GpuSampler(vocab_max=4096, rows_max=16, k_max=64) as g:
        with pytest.raises(S.SamplingError) as e:
            g.sample_lmhead_q4(head, x, _params(9, 1))
        assert e.value.status == S.TABBY_EINVAL


@pytest.mark.parametrize("crowded_slices", [[0], [3, 90, 170], [0, 10, 50, 100, 200, 237]])
def test_fused_crowded_top(oracle, crowded_slices):
    # Rows whose top lies in a few slices: 64 rows of each named 640-row slice get all codes 15
    # (+7 * scale) and positive scales against positive activations, so the bound from the
    # slices' first entries admits whole lists -- up to 6 x 64 = 384 entries, beyond the
    # bounded merge's 256, which then hands the row to the general merge. Ties among equal
    # rows go to the lower id.
    torch = _torch()
    vocab, hidden, block = 151936, 896, 32
    words, f16, f32 = synth.lm_head_q4(vocab, hidden, block, seed=3)
    words = words.reshape(vocab, hidden // 8).copy()
    f16 = f16.reshape(vocab, hidden // block).copy()
    for sl in crowded_slices:
        rows = np.arange(sl * 640, sl * 640 + 64)
        words[rows] = 0xFFFFFFFF
        f16[rows] = np.float16(0.006 + 0.0001 * (sl % 3)).view(np.uint16)
    f32 = f16.view(np.float16).astype(np.float32).reshape(-1)
    head = S.LmHeadQ4(words.reshape(-1), f16.reshape(-1), vocab, hidden, block)
    x = np.abs(synth.hidden_states(3, hidden, seed=8))
    params = _params(3, 4242, k_choices=(40, 64), ts=(0.7, 1.0), ps=(0.9, 1.0))
    logits = oracle.matmul_quantized(words.reshape(-1), f32, x, vocab, hidden)
    with S.GpuSampler(vocab_max=vocab, rows_max=3, k_max=64) as g:
        res = g.sample_lmhead_q4(head, torch.from_numpy(x).cuda(), params)
    _check_rows(oracle, res, logits, params, f"crowded {crowded_slices}")
