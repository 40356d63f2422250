"""The allocation-free entry (tabby_sampler_sample_device_noalloc) against the handle's
device-resident entry on the same inputs: two calls in a row, the second smaller, each
covering a different launch shape. Ids, counts, maxima, statuses and top-k lists bit for
bit; the f64 outputs within 1e-5 relative (sum-exp repeats run to run only to ~1e-9)."""
import numpy as np
import pytest

from tabby_amd import sampler as S
from tabby_amd import synth

from parity import params_of

pytestmark = pytest.mark.gpu


def _device_buffers(w, cap):
    import torch
    x = torch.from_numpy(np.ascontiguousarray(w.logits)).cuda()
    pd = torch.from_numpy(params_of(w).view(np.uint8).copy()).cuda()
    rd = torch.zeros(w.rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    ids = torch.full((w.rows, cap), -7, dtype=torch.int32, device="cuda")
    vals = torch.zeros((w.rows, cap), dtype=torch.float32, device="cuda")
    return x, pd, rd, ids, vals


def _results(rd, ids, vals):
    return rd.cpu().numpy().view(S.RESULT_DTYPE).copy(), ids.cpu().numpy(), vals.cpu().numpy()


def _same(a, b, ctx):
    ra, ia, va = a
    rb, ib, vb = b
    for f in ("id", "considered", "max_logit", "status", "topk_count", "pool_exhausted"):
        assert ra[f].tobytes() == rb[f].tobytes(), f"{ctx}: {f}"
    for f in ("probability", "pool_mass", "sum_exp"):
        np.testing.assert_allclose(ra[f], rb[f], rtol=1e-5, atol=0, err_msg=f"{ctx}: {f}")
    for r in range(ra.shape[0]):
        n = int(ra["topk_count"][r])
        assert np.array_equal(ia[r, :n], ib[r, :n]), f"{ctx}: row {r} top-k ids"
        assert np.array_equal(va[r, :n].view(np.uint32), vb[r, :n].view(np.uint32)), f"{ctx}: row {r} top-k logits"


def _one(w, k_max, cap, ctx):
    import torch
    print(f"[no-alloc] {ctx}: {w.rows} x {w.vocab}, k_max {k_max}", flush=True)
    x, pd, rd, ids, vals = _device_buffers(w, cap)
    with S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=k_max) as g:
        g.sample_device(x, pd, rd, ids, vals)
        want = _results(rd, ids, vals)
    rd.zero_()
    ids.fill_(-7)
    S.sample_device_noalloc(x, pd, rd, k_max, ids, vals)
    torch.cuda.synchronize()
    got = _results(rd, ids, vals)
    _same(got, want, ctx)
    return got


def test_no_alloc_matches_device_entry_two_calls():
    # First call: 200 rows of 151,936 (one-wave slices, packed lists of 21 slices per row);
    # second, smaller: 8 rows of 100,000 (each row in parts, merged by the second kernel).
    w1 = synth.config(3, rows=200)
    w1.top_k[:] = np.resize(np.array([1, 20, 50, 100, 256], np.int32), 200)
    _one(w1, 256, 64, "call 1, slices")
    w2 = synth.random_workload(rows=8, vocab=100000, seed=5, ties=True, neg_inf_frac=0.2,
                               k_choices=(1, 50, 64, 200), temperatures=(0.0, 0.7, 1.0))
    _one(w2, 256, 64, "call 2, parts")


def test_no_alloc_parts_across_calls():
    # Calls whose rows are cut into different numbers of parts share the scratch: ten parts
    # (a row of 151,936), then four (17 rows of 100,000), then ten again.
    _one(synth.config(2), 64, 50, "parts: one row of 151,936")
    w = synth.random_workload(rows=17, vocab=100000, seed=17, k_choices=(1, 50, 64), temperatures=(0.0, 0.8))
    _one(w, 64, 50, "parts: 17 rows of 100,000")
    _one(synth.config(2), 64, 50, "parts: one row of 151,936 again")


def test_no_alloc_per_row_kernel_and_statuses():
    # 256 rows: one workgroup per row, no lists in scratch; a -inf row and a whole-vocabulary
    # row come back with their statuses as from the handle's entry.
    w = synth.config(3, rows=256, vocab=30000)
    w.logits[3] = -np.inf
    w.top_k[7] = 0
    _one(w, 64, 50, "per-row kernel")
    w2 = synth.config(1)
    _one(w2, 64, 40, "one row of 49,152")


def test_no_alloc_rejects_beyond_its_limits():
    import torch
    x = torch.zeros(2, 1000, device="cuda")
    pd = torch.zeros(2 * S.PARAMS_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    rd = torch.zeros(2 * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    with pytest.raises(S.SamplingError, match="k_max") as e:
        S.sample_device_noalloc(x, pd, rd, 257)
    assert e.value.status == S.TABBY_ECAPACITY
