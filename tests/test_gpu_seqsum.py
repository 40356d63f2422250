"""The device's parallel evaluation of left-to-right f64 sums (the sequential sums of
sampler.ts:156-203) against numpy's sequential cumsum, bit for bit."""
import numpy as np
import pytest

from tabby_amd import sampler as S

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[0, 1, 2, 3], ids=["lds", "wide", "block", "block8"])
def wide(request):
    return request.param


def _check(terms, stop_at=np.inf, wide=0):
    import torch
    terms = np.ascontiguousarray(terms, dtype=np.float64)
    prefix, n = S.device_seq_sum(torch.from_numpy(terms).cuda(), stop_at, wide)
    expected = np.cumsum(terms)  # numpy's cumsum is a sequential left-to-right loop
    hits = np.nonzero(expected >= stop_at)[0]
    want_n = int(hits[0]) + 1 if hits.size else terms.size
    assert n == want_n, (n, want_n)
    got = prefix.cpu().numpy()
    bad = np.nonzero(got.view(np.uint64) != expected[:n].view(np.uint64))[0]
    assert bad.size == 0, f"{bad.size} differ, first at {bad[0]}: {got[bad[0]]!r} vs {expected[bad[0]]!r}"


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 63, 64, 65, 1023, 1024, 1025, 4096, 4097, 8193, 20000])
def test_sorted_exponential_terms(n, wide):
    rng = np.random.default_rng(n)
    l = np.sort(rng.normal(0, 3, n))[::-1]
    _check(np.exp((l - l[0]) / 0.7), wide=wide)


def test_many_binade_crossings_and_flat_terms(wide):
    _check(np.ones(5000), wide=wide)                  # integer sums: a crossing at every power of two
    _check(np.full(3000, 1.0 / 3.0), wide=wide)
    _check(np.linspace(1.0, 1e-3, 7000), wide=wide)


def test_exact_half_ulp_ties_round_to_even(wide):
    # 1 + 2^-53 is a tie (stays 1), then terms that make odd and even sums alternate.
    t = [1.0] + [2.0 ** -53] * 40 + [2.0 ** -52] + [2.0 ** -53] * 40 + [3 * 2.0 ** -53] * 30
    _check(np.array(t), wide=wide)
    rng = np.random.default_rng(7)
    base = np.ldexp(1.0, -rng.integers(40, 56, 3000).astype(np.int64))
    _check(np.concatenate([[0.75], np.sort(base)[::-1]]), wide=wide)


def test_dense_ties_long(wide):
    # Terms that fall on half an ulp of the running sum on most steps, past the short path.
    pattern = np.array([2.0 ** -53, 3 * 2.0 ** -53, 2.0 ** -52, 5 * 2.0 ** -54, 2.0 ** -53, 7 * 2.0 ** -54])
    _check(np.concatenate([[1.0], np.tile(pattern, 600)]), wide=wide)
    _check(np.concatenate([[1.5], np.tile(pattern[::-1], 500)]), wide=wide)


@pytest.mark.parametrize("stop", [np.inf, 0.98])
def test_quantised_logit_terms(stop, wide):
    # Weights of logits on a 0.25 grid (few distinct values, many repeats), sorted, as in
    # BASELINE config 5; the top-p stop variant cuts inside the run.
    rng = np.random.default_rng(5)
    levels = np.sort(np.round(rng.normal(0, 2, 1024) * 4) / 4)[::-1]
    s = np.exp(levels - levels[0])
    _check(s / s.sum() if np.isfinite(stop) else s, stop, wide)


def test_tiny_and_zero_terms(wide):
    _check(np.concatenate([[1.0], np.full(100, 1e-300), np.zeros(200), [5e-324] * 10]), wide=wide)


@pytest.mark.parametrize("stop", [0.5, 0.9, 0.95, 0.999999, 1.0])
def test_stop_at_threshold(stop, wide):
    rng = np.random.default_rng(11)
    l = np.sort(rng.normal(0, 1, 3000))[::-1]
    s = np.exp(l - l[0])
    w = s / s.sum()
    _check(w, stop, wide)
