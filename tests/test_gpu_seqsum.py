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


def _check_in_place(terms, stop_at=np.inf, wide=0):
    """The same sums written over their own terms (whole-vocabulary heads run the running
    sums that way): every partial sum up to the stop bit for bit."""
    import torch
    terms = np.ascontiguousarray(terms, dtype=np.float64)
    prefix, n = S.device_seq_sum(torch.from_numpy(terms).cuda(), stop_at, wide, in_place=True)
    expected = np.cumsum(terms)
    hits = np.nonzero(expected >= stop_at)[0]
    want_n = int(hits[0]) + 1 if hits.size else terms.size
    assert n == want_n, (n, want_n)
    got = prefix.cpu().numpy()
    bad = np.nonzero(got.view(np.uint64) != expected[:n].view(np.uint64))[0]
    assert bad.size == 0, f"{bad.size} differ, first at {bad[0]}: {got[bad[0]]!r} vs {expected[bad[0]]!r}"


@pytest.mark.parametrize("n", [300, 16385, 40000])
@pytest.mark.parametrize("stop", [np.inf, 0.9, 0.999])
def test_in_place_with_binade_events(n, stop, wide):
    # Normalised weights of a flat, tied head (many binade crossings below 1: every event
    # restarts a step after thread 0 has rewritten the event's term) and integer-valued terms
    # (a crossing at each power of two).
    rng = np.random.default_rng(n)
    levels = np.sort(np.round(rng.normal(0, 1, n) * 4) / 4)[::-1]
    s = np.exp((levels - levels[0]) / 2.0)
    _check_in_place(s / s.sum(), stop, wide)
    if not np.isfinite(stop):
        _check_in_place(np.ones(n), stop, wide)


def _stop_terms(n, seed):
    rng = np.random.default_rng(seed)
    l = np.sort(rng.normal(0, 1.5, n))[::-1]
    s = np.exp(l - l[0])
    return s / s.sum()


@pytest.mark.parametrize("n", [9, 40, 65, 256])
def test_short_sums_with_stop_past_the_serial_prefix(n, wide):
    # Sums of at most 256 terms with a top-p stop take their first 8 terms one by one and
    # the rest by the scan from term 8: stops exactly at the 8th and 9th partial sums, just
    # above them, and late.
    w = _stop_terms(n, n)
    c = np.cumsum(w)
    stops = [c[7], c[8], np.nextafter(c[7], 2.0), np.nextafter(c[8], 2.0), c[n - 2], c[n - 1]]
    if n > 20:
        stops.append(c[n // 2])
    for st in stops:
        _check(w, st, wide)


@pytest.mark.parametrize("n", [9, 40, 65, 256])
def test_short_sums_binade_and_tie_after_the_serial_prefix(n, wide):
    # The 8th partial sum is 1 + 2^-52 (odd); term 9 is half its ulp, an exact tie that
    # rounds to the even sum; then terms that cross into [2, 4).
    head = [1.0, 2.0 ** -52] + [0.0] * 6
    t = np.array(head + [2.0 ** -53] + [0.75] * (n - 9), dtype=np.float64)[:n]
    c = np.cumsum(t)
    for st in (np.inf, c[8], c[min(n - 1, 9)], c[-1]):
        _check(t, st, wide)
    # A crossing of 1.0 at term 9 itself, then small terms.
    t2 = np.array([0.5] + [1.0 / 16] * 7 + [0.25] + [2.0 ** -20] * (n - 9), dtype=np.float64)[:n]
    c2 = np.cumsum(t2)
    for st in (np.inf, c2[8], np.nextafter(c2[8], 0.0), c2[-1]):
        _check(t2, st, wide)


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 100, 4095, 4096, 4097, 5000, 60000, 151936])
def test_draw_search_first_above(n):
    # The whole-vocabulary draw: the first i with target < c[i] over non-decreasing running
    # sums (long tie runs included), or n - 1 when none, against a brute-force search.
    import torch
    rng = np.random.default_rng(n + 7)
    for trial in range(4):
        inc = rng.random(n)
        inc[rng.random(n) < (0.2 if trial % 2 else 0.9)] = 0.0  # runs of equal sums
        c = np.cumsum(inc)
        c = c / max(c[-1], 1.0)
        probes = np.concatenate([rng.random(300) * (c[-1] + 0.01), c[rng.integers(0, n, 200)],
                                 np.nextafter(c[rng.integers(0, n, 100)], -1.0), [0.0, -1.0, c[-1], c[-1] + 1]])
        want = np.minimum(np.searchsorted(c, probes, side="right"), n - 1)
        got = S.device_first_above(torch.from_numpy(c).cuda(), torch.from_numpy(probes).cuda()).cpu().numpy()
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"n={n} trial {trial}: {bad.size} wrong, first target {probes[bad[0]]!r}: "
                               f"got {got[bad[0]]}, want {want[bad[0]]}")


@pytest.mark.parametrize("n", [1, 2, 9, 15, 16, 17, 33, 50, 63, 64])
def test_register_form_short_sums(n):
    # Pools of at most 64 finish with term i in lane i (wide = 4): sorted weights at several
    # temperatures, with and without a top-p stop at every position, integer terms (a binade
    # crossing at each power of two), exact half-ulp ties, and quantised-logit weights.
    rng = np.random.default_rng(100 + n)
    l = np.sort(rng.normal(0, 3, n))[::-1]
    for T in (0.05, 0.7, 2.0, 50.0):
        s = np.exp((l - l[0]) / T)
        _check(s, wide=4)
        w = s / s.sum()
        c = np.cumsum(w)
        for st in np.unique(np.concatenate([c, np.nextafter(c, 2.0), [0.5, 0.9, 0.95]])):
            _check(w, st, wide=4)
    _check(np.ones(n), wide=4)
    _check(np.ones(n), float(max(1, n // 2)), wide=4)
    t = ([1.0] + [2.0 ** -53] * 20 + [2.0 ** -52] + [2.0 ** -53] * 20 + [3 * 2.0 ** -53] * 22)[:n]
    _check(np.array(t), wide=4)
    q = np.sort(np.round(rng.normal(0, 2, n) * 4) / 4)[::-1]
    e = np.exp(q - q[0])
    _check(e / e.sum(), wide=4)
    _check(e / e.sum(), 0.98, wide=4)
    _check(np.concatenate([[1.0], np.full(n - 1, 1e-300)]), wide=4)
