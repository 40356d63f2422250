"""GPU parity: libtabby_sampler.so (through its C ABI) against the CPU oracle on identical
seeded logits and uniforms. Ids, candidate sets and counts must be bit-exact; the f64
probabilities within 1e-5 relative (the tolerance of BASELINE.json's north_star)."""
import numpy as np
import pytest

from tabby_amd import sampler as S
from tabby_amd import synth

from parity import REL_TOL, compare, params_of, rel, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def _log(name, stats):
    print(f"[parity] {name}: {stats}", flush=True)


@pytest.mark.parametrize("greedy", [False, True])
def test_config1_single_row_49152(oracle, greedy):
    w = synth.config(1)
    if greedy:
        w.temperature[:] = 0.0
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=40)
    _log(f"config1 greedy={greedy}", compare(w, res, ids, vals, run_oracle(oracle, w, 40), 40))


def test_config2_single_row_151936_spiky(oracle):
    w = synth.config(2)
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=50)
    _log("config2", compare(w, res, ids, vals, run_oracle(oracle, w, 50), 50))


def test_config3_batch_256(oracle):
    w = synth.config(3)
    res, ids, vals = run_gpu(w, k_max=128, topk_cap=100)
    _log("config3", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))


def test_config5_ties_neg_inf_k1024(oracle):
    w = synth.config(5, rows=128)
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=1024)
    _log("config5[128 rows]", compare(w, res, ids, vals, run_oracle(oracle, w, 1024), 1024))


def test_config5_sorted_slice_lists(oracle):
    # 256 rows: one pool_row_kernel workgroup per row (its list selected in the kernel).
    w = synth.config(5, rows=256)
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=1024)
    _log("config5[256 rows]", compare(w, res, ids, vals, run_oracle(oracle, w, 1024), 1024))


def test_large_pool_capacity_mixed_k(oracle):
    # k_max 1024 sends every row through the 256-lane slices; small and large k mix, with
    # ties and -inf, on few enough slices per row for the sorted-list merge.
    w = synth.random_workload(rows=192, vocab=20000, seed=17, ties=True, neg_inf_frac=0.3,
                              k_choices=(1, 64, 300, 1024))
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=1024)
    _log("k_max 1024 mixed", compare(w, res, ids, vals, run_oracle(oracle, w, 1024), 1024))


@pytest.mark.parametrize("dtype,vocab", [(np.float32, 20000), (np.float16, 20000), (np.float16, 20001),
                                         (np.float32, 3000)])
def test_pool_row_kernel_batches(oracle, dtype, vocab):
    # Batches of >= 256 rows with k_max 1024 take pool_row_kernel: k from 1 to 1024 with ties
    # and -inf, rows whose every element is a candidate (all equal: the shared list spills past
    # its 8,192 LDS entries to global memory), whole-vocabulary rows (handed to the head path),
    # a vocabulary shorter than the 16 waves' first chunks (3,000), and f16 rows of odd length
    # (one-element loads).
    rows = 256
    w = synth.random_workload(rows=rows, vocab=vocab, seed=vocab + rows, ties=True, neg_inf_frac=0.2,
                              k_choices=(1, 64, 100, 200, 300, 1024), temperatures=(0.0, 0.7, 1.0, 2.0),
                              top_ps=(0.5, 0.9, 0.98, 1.0))
    for r in range(0, rows, 16):
        w.logits[r, :] = 1.25  # all equal
        w.top_k[r] = 1024
    w.top_k[5::32] = 0  # whole vocabulary
    if dtype == np.float16:
        w.logits = w.logits.astype(np.float16)
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=64)
    _log(f"pool row kernel {dtype.__name__} V={vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_pool_row_kernel_rows_outside_contract(oracle):
    # The pool kernel ends every row but a head pass's whole-vocabulary ones: rows with -inf
    # only, NaN or +inf report EDOMAIN, topK above k_max and whole-vocabulary rows without
    # TABBY_FLAG_FULL_VOCAB report EINVAL, and the other rows (pools of 40 to 600) are sampled.
    import torch
    rows, vocab = 256, 3000
    x = torch.randn(rows, vocab, device="cuda")
    x[5] = float("-inf")
    x[77, 1234] = float("nan")
    x[200, 9] = float("inf")
    p = S.make_params(S.SamplingParams(0.7, 40, 0.9), rows, 0.25)
    p["top_k"] = np.array([40, 100, 200, 600], np.int32)[np.arange(rows) % 4]
    p["uniform"] = (np.arange(rows) * 0.618034) % 1.0
    p["top_k"][[9, 130]] = 2000
    p["top_k"][[13, 250]] = 0
    with S.GpuSampler(vocab_max=vocab, rows_max=rows, k_max=1024) as g:
        pd = torch.from_numpy(p.view(np.uint8).copy()).cuda()
        rd = torch.zeros(rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
        g.sample_device(x, pd, rd)
        res = rd.cpu().numpy().view(S.RESULT_DTYPE)
    logits = x.cpu().numpy()
    for r in range(rows):
        want = (S.TABBY_EDOMAIN if r in (5, 77, 200) else S.TABBY_EINVAL if r in (9, 130, 13, 250) else 0)
        assert res["status"][r] == want, f"row {r}"
        if want == 0:
            o = oracle.sample_row(logits[r], int(p[r]["top_k"]), float(p[r]["temperature"]),
                                  float(p[r]["top_p"]), float(p[r]["uniform"]))
            assert (int(res["id"][r]), int(res["considered"][r])) == (o["id"], o["considered"]), f"row {r}"


def test_pool_row_kernel_batch_with_head_pass(oracle):
    # 256 rows with k_max 1024 and TABBY_FLAG_FULL_VOCAB: pool_row_kernel samples the pools
    # (k 50, 300, 1000) and writes the statuses itself, and hands the whole-vocabulary rows
    # (k 0) to merge_kernel and the head kernels, which skip the rows it ended.
    import torch
    w = synth.random_workload(rows=256, vocab=4000, seed=31, k_choices=(0, 50, 300, 1000), ties=True,
                              neg_inf_frac=0.05)
    w.logits[17] = -np.inf
    w.logits[140, 7] = np.nan
    params = np.zeros(w.rows, dtype=S.PARAMS_DTYPE)
    params["temperature"], params["top_p"], params["uniform"], params["top_k"] = (
        w.temperature, w.top_p, w.uniform, w.top_k)
    params["top_k"][99] = 2000  # above k_max: EINVAL
    x = torch.from_numpy(np.ascontiguousarray(w.logits)).cuda()
    pd = torch.from_numpy(params.view(np.uint8).copy()).cuda()
    rd = torch.zeros(w.rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    with S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=1024) as g:
        g.sample_device(x, pd, rd, flags=S.TABBY_FLAG_FULL_VOCAB)
        res = rd.cpu().numpy().view(S.RESULT_DTYPE).copy()
    logits = w.logits_f32()
    sampled = 0
    for r in range(w.rows):
        if r in (17, 140):
            assert int(res["status"][r]) == S.TABBY_EDOMAIN, f"row {r}"
            continue
        if r == 99:
            assert int(res["status"][r]) == S.TABBY_EINVAL, f"row {r}"
            continue
        k, T, p, u = (int(params[r]["top_k"]), float(params[r]["temperature"]), float(params[r]["top_p"]),
                      float(params[r]["uniform"]))
        o = oracle.sample_row(logits[r], k, T, p, u)
        c = f"row {r}: k={k} T={T} p={p} u={u!r}"
        assert int(res["status"][r]) == o["status"] == 0, c
        assert (int(res["id"][r]), int(res["considered"][r])) == (o["id"], o["considered"]), c
        assert np.float32(res["max_logit"][r]) == np.float32(o["max_logit"]), c
        for f in ("probability", "pool_mass", "sum_exp"):
            assert rel(float(res[f][r]), o[f]) < REL_TOL, (c, f)
        sampled += 1
    assert sampled == w.rows - 3
    _log("pool rows with a head pass", {"rows": sampled})


def _f32_keys(x):
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return np.where(b >> 31 == 1, (~b) & 0xFFFFFFFF, b | 0x80000000)


def _pool_guess_candidates(row, kk, vec):
    """The candidates pool_row_kernel's guessed first bound leaves in a row (at least 128 chunks
    of 1,024; vec: elements per lane per load, 4 for f32 and 8 for f16): its sample is each
    wave's first two claims -- claim v takes chunk (v mod 16) s + v // 16 below 16 s, s the
    largest power of two with 16 s <= chunks -- and the bound is the top 22 key bits of the
    (kk/2)-th largest of the sample's 4,096 group maxima (a lane's elements 4g .. 4g + 3 of its
    first chunk and of its second; element e of lane l sits at (e // vec) 64 vec + l vec +
    e % vec in its chunk)."""
    row = row.astype(np.float32)
    n = row.size
    nch = -(-n // 1024)
    s = 1
    while 32 * s <= nch:
        s *= 2
    chunk = lambda v: (v % 16) * s + v // 16 if v < 16 * s else v
    e = np.arange(16).reshape(4, 1, 4)
    lanes = np.arange(64).reshape(1, 64, 1)
    at = (e // vec) * 64 * vec + lanes * vec + e % vec  # [group, lane, element of the group]
    gm = []
    for w in range(16):
        xa = row[chunk(w) * 1024 + at]
        xb = row[chunk(16 + w) * 1024 + at]
        gm.append(np.maximum(xa.max(2), xb.max(2)).ravel())
    keys = np.clip(_f32_keys(np.concatenate(gm)), 0x007FFFFF, 0xFF800000)
    t = np.sort(keys)[::-1][kk // 2 - 1] & ~np.uint64(0x3FF)
    return int(np.count_nonzero(_f32_keys(row) >= t))


@pytest.mark.parametrize("dtype,V", [(np.float32, 151936), (np.float16, 151936), (np.float32, 151937)])
def test_pool_row_kernel_guessed_bound(oracle, dtype, V):
    # Rows of 151,936 (149 chunks) take pool_row_kernel's guessed first bound: the (k/2)-th
    # largest group maximum of a sample of 32 chunks spread over the row. Rows 0-3 put their
    # largest values in exactly those chunks, so the guess leaves fewer than k candidates and
    # the row's candidates are taken again at the certain bound (rows 0-2: the sampled chunks
    # drawn around 10, the rest around 0; row 3: one value near 20 in every group of the
    # sample, the rest around 0). Rows 4-5 are sorted ascending and descending, row 6 has a
    # sample of -inf (no guess: every element is a candidate), row 7 a sample of one value;
    # the other rows are config-5-like (ties, -inf) with k from 1 to 1,024. f16 rows load
    # eight elements per lane at a time and an odd vocabulary one, which changes the groups
    # (and row 3's layout).
    rows = 256
    vec = 1 if V % 8 else 4 if dtype == np.float32 else 8
    w = synth.random_workload(rows=rows, vocab=V, seed=5150, ties=True, neg_inf_frac=0.3,
                              k_choices=(1, 64, 300, 1024), temperatures=(0.7, 1.0), top_ps=(0.5, 0.98, 1.0),
                              sigma=2.0)
    rng = np.random.default_rng(5150)
    sample = np.zeros(V, dtype=bool)
    for v in range(32):
        c = (v % 16) * 8 + v // 16
        sample[c * 1024:(c + 1) * 1024] = True
    for r, k in ((0, 1024), (1, 300), (2, 1000), (3, 1024), (4, 1024), (5, 1024), (6, 1024), (7, 1024)):
        w.top_k[r] = k
        w.logits[r] = rng.standard_normal(V).astype(np.float32)
    for r in range(3):
        w.logits[r, sample] += 10.0
    # Row 3: the first of lane l's elements 4g .. 4g + 3, for even lanes, in every sampled chunk
    # (element e of lane l sits at (e // vec) 64 vec + l vec + e % vec in its chunk).
    big = np.zeros(V, dtype=bool)
    e, lane = np.meshgrid(np.arange(0, 16, 4), np.arange(0, 64, 2))
    first = ((e // vec) * 64 * vec + lane * vec + e % vec).ravel()
    for v in range(32):
        big[((v % 16) * 8 + v // 16) * 1024 + first] = True
    w.logits[3, big] = 20.0 + rng.random(int(big.sum())).astype(np.float32)
    w.logits[4] = np.sort(w.logits[4])
    w.logits[5] = np.sort(w.logits[5])[::-1]
    w.logits[6, sample] = -np.inf
    w.logits[7, sample] = 5.0
    w.top_p[:4] = (0.98, 0.5, 0.98, 0.9)
    if dtype == np.float16:
        w.logits = w.logits.astype(np.float16)
    for r in range(4):  # the premise: the guess leaves fewer than k candidates
        assert _pool_guess_candidates(w.logits[r], int(w.top_k[r]), vec) < int(w.top_k[r]), f"row {r}"
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=64)
    _log(f"pool kernel guessed bound {dtype.__name__}",
         compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_pool_row_kernel_guessed_bound_k_sweep(oracle):
    # 256 rows of 131,072 (exactly the 128 chunks from which pool_row_kernel guesses its first
    # bound), k from 2 to 1,024 in steps of 4 with ties and -inf; every fourth row has its
    # sampled chunks raised by 3, so that some guesses fall short (those rows are taken again)
    # and others only just hold.
    V, rows = 131072, 256
    w = synth.random_workload(rows=rows, vocab=V, seed=7331, ties=True, neg_inf_frac=0.2,
                              k_choices=tuple(range(2, 1025, 4)), temperatures=(0.0, 0.7, 1.0),
                              top_ps=(0.5, 0.95, 1.0), sigma=2.0)
    sample = np.zeros(V, dtype=bool)
    for v in range(32):
        c = (v % 16) * 8 + v // 16
        sample[c * 1024:(c + 1) * 1024] = True
    for r in range(0, rows, 4):
        w.logits[r, sample] += 3.0
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=64)
    _log("pool kernel guessed bound, k sweep", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


@pytest.mark.parametrize("it", range(8))
def test_pool_row_kernel_random_batches(oracle, it):
    # Seeded random batches for the large-pool kernel: k from 257 to 1,024, vocabularies of
    # 131,072 to 262,144 (odd ones too), ties or not, -inf, f16 or f32, and rows whose
    # first-bound sample is raised or lowered against the rest of the row.
    rng = np.random.default_rng(4242 + it)
    V = int(rng.choice([131072, 131075, 151936, 152064, 200000, 262144]))
    rows = int(rng.choice([256, 300, 512]))
    w = synth.random_workload(rows=rows, vocab=V, seed=int(rng.integers(1, 1 << 30)),
                              ties=bool(rng.integers(0, 2)), neg_inf_frac=float(rng.choice([0.0, 0.1, 0.5])),
                              k_choices=tuple(int(x) for x in rng.integers(257, 1025, 8)),
                              temperatures=(0.0, 0.5, 1.0, 2.0), top_ps=(0.5, 0.9, 0.98, 1.0),
                              sigma=float(rng.choice([1.0, 2.0, 3.0])))
    nch = -(-V // 1024)
    s = 1
    while 32 * s <= nch:
        s *= 2
    sample = np.zeros(V, dtype=bool)
    for v in range(32):
        c = (v % 16) * s + v // 16
        sample[c * 1024:min((c + 1) * 1024, V)] = True
    for r in range(rows):
        u = rng.random()
        if u < 0.15:
            w.logits[r, sample] += float(rng.uniform(0.5, 6.0))
        elif u < 0.25:
            w.logits[r, sample] -= float(rng.uniform(0.5, 6.0))
    if rng.random() < 0.3:
        w.logits = w.logits.astype(np.float16)
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=32)
    _log(f"pool kernel random batch {it} (V={V}, rows={rows}, {w.logits.dtype})",
         compare(w, res, ids, vals, run_oracle(oracle, w, 32), 32))


@pytest.mark.parametrize("it", range(16))
def test_random_batches_every_launch_shape(oracle, it):
    # Seeded random batches over every launch shape the plan picks: 1 to 600 rows, vocabularies
    # of 1 to 200,000 (odd ones too), k_max 64 to 1,024 with k up to it and whole-vocabulary
    # rows, ties, -inf, greedy and sampled rows, f16 or f32.
    rng = np.random.default_rng(9000 + it)
    rows = int(rng.choice([1, 2, 3, 7, 16, 64, 100, 129, 200, 256, 300, 512, 600]))
    V = int(rng.choice([1, 5, 64, 1000, 4097, 16385, 49152, 100003, 131072, 151936, 200000]))
    if rows * V > 600 * 151936:
        V = 151936
    kmax = int(rng.choice([64, 128, 256, 1024]))
    kc = [int(k) for k in rng.integers(1, kmax + 1, 4)] + ([0] if rng.random() < 0.3 else [])
    w = synth.random_workload(rows=rows, vocab=V, seed=int(rng.integers(1, 1 << 30)), ties=bool(rng.integers(0, 2)),
                              neg_inf_frac=float(rng.choice([0.0, 0.05, 0.3])), k_choices=tuple(kc),
                              temperatures=(0.0, 0.3, 0.7, 1.0, 2.0), top_ps=(0.5, 0.9, 0.98, 1.0),
                              sigma=float(rng.choice([1.0, 3.0])))
    w.logits[~np.isfinite(w.logits).any(axis=1), 0] = 0.0  # no row of only -inf (outside the contract)
    if rng.random() < 0.3:
        w.logits = w.logits.astype(np.float16)
    cap = min(kmax, 32)
    res, ids, vals = run_gpu(w, k_max=kmax, topk_cap=cap)
    _log(f"random batch {it} (rows={rows}, V={V}, k_max={kmax}, {w.logits.dtype})",
         compare(w, res, ids, vals, run_oracle(oracle, w, cap), cap))


def test_f16_input_finite_k(oracle):
    w = synth.config(4, rows=16)
    w.top_k[:] = np.array([1, 20, 50, 100] * 4, np.int32)
    w.temperature[:] = 0.3
    res, ids, vals = run_gpu(w, k_max=128, topk_cap=100)
    _log("f16 finite k", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))


@pytest.mark.parametrize("vocab", [1, 3, 64, 203, 1000, 4097, 16385, 49153])
def test_awkward_vocab_sizes(oracle, vocab):
    # Non-multiples of 4 take the scalar-load path; sizes straddle the slice lengths.
    w = synth.random_workload(rows=6, vocab=vocab, seed=vocab, k_choices=(1, 5, 40, 64))
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    _log(f"vocab {vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_ties_and_neg_inf(oracle):
    w = synth.random_workload(rows=32, vocab=20000, seed=7, ties=True, neg_inf_frac=0.5,
                              k_choices=(1, 7, 64, 256))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=256)
    _log("ties+neg_inf", compare(w, res, ids, vals, run_oracle(oracle, w, 256), 256))


@pytest.mark.parametrize("k", [20, 50, 64])
def test_first_chunk_unrepresentative(oracle, k):
    # Vocab 147,456 on 4 rows is cut into 36 slices of 4,096, and each slice's first chunk
    # sets its starting theta. Rows 0-1 put one large value per lane in the first 256
    # elements of every 4,096-block and keep the rest small (the first chunk holds the whole
    # top of the slice); row 2 is sorted ascending (every first chunk is its slice's
    # smallest: a low theta, many candidates, many prunes); row 3 descending.
    V = 147456
    w = synth.random_workload(rows=4, vocab=V, seed=41, k_choices=(k,), temperatures=(0.7,),
                              top_ps=(0.9,), sigma=1.0)
    big = np.zeros(V, dtype=bool)
    big[(np.arange(V) % 4096 < 256) & (np.arange(V) % 4 == 0)] = True
    rng = np.random.default_rng(k)
    for r in (0, 1):
        w.logits[r, big] = (20.0 + rng.standard_normal(int(big.sum()))).astype(np.float32)
    w.logits[2] = np.sort(w.logits[2])
    w.logits[3] = np.sort(w.logits[3])[::-1]
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=k)
    _log(f"unrepresentative first chunk k={k}", compare(w, res, ids, vals, run_oracle(oracle, w, k), k))


def test_all_equal_row_takes_lowest_ids(oracle):
    w = synth.random_workload(rows=2, vocab=5000, seed=3, k_choices=(64,))
    w.logits[:] = 1.5
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    assert np.array_equal(ids[0], np.arange(64)) and np.array_equal(ids[1], np.arange(64))
    compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64)


def test_signed_zero_ties(oracle):
    w = synth.random_workload(rows=4, vocab=3000, seed=11, k_choices=(50,))
    w.logits[:] = -1.0
    w.logits[:, ::3] = 0.0
    w.logits[:, 1::3] = -0.0  # equal to +0 for the comparator: order by id
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=50)
    compare(w, res, ids, vals, run_oracle(oracle, w, 50), 50)


def test_k_at_least_vocab_takes_whole_row(oracle):
    w = synth.random_workload(rows=4, vocab=100, seed=5, k_choices=(100, 200, 0))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=100)
    compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100)


def assert_same_result(a, b):
    """Two runs of the same rows: ids, counts, flags, max and the top-k lists bit for bit.
    The row kernel's waves claim chunks in whatever order they run and keep sum-exp as f32
    terms relative to each lane's running max, so sum-exp -- and the probability and poolMass
    divided by it -- repeat to those terms' rounding (~1e-9 relative; the contract's
    tolerance is 1e-5)."""
    for f in ("id", "considered", "max_logit", "status", "topk_count"):
        assert a[0][f].tobytes() == b[0][f].tobytes(), f
    for f in ("probability", "pool_mass", "sum_exp"):
        np.testing.assert_allclose(a[0][f], b[0][f], rtol=1e-6, atol=0, err_msg=f)
    assert np.array_equal(a[1], b[1]) and np.array_equal(a[2].view(np.uint32), b[2].view(np.uint32))


@pytest.mark.parametrize("rows", [1, 32, 256])
def test_repeatable(rows):
    w = synth.config(3, rows=rows)
    assert_same_result(run_gpu(w, k_max=128, topk_cap=100), run_gpu(w, k_max=128, topk_cap=100))


def test_reuse_handle_across_calls(oracle):
    # The arrival counters reset themselves; a second call on the same handle must agree.
    w = synth.random_workload(rows=8, vocab=30000, seed=21)
    with S.GpuSampler(vocab_max=30000, rows_max=8, k_max=64) as g:
        first = run_gpu(w, sampler=g, topk_cap=64)
        second = run_gpu(w, sampler=g, topk_cap=64)
    assert_same_result(first, second)
    compare(w, *first, run_oracle(oracle, w, 64), 64)


def test_rejects_topk_above_capacity():
    import torch
    x = torch.zeros(1, 1000, device="cuda")
    with S.GpuSampler(vocab_max=1000, rows_max=1, k_max=64) as g:
        p = S.make_params(S.SamplingParams(0.7, 65, 0.9), 1, 0.5)
        with pytest.raises(S.SamplingError, match="topK"):
            g.sample_params(x, p)


@pytest.mark.parametrize("fill", ["all_neg_inf", "nan", "pos_inf"])
def test_rows_outside_contract_report_edomain(fill):
    import torch
    x = torch.randn(3, 2000, device="cuda")
    if fill == "all_neg_inf":
        x[1] = float("-inf")
    elif fill == "nan":
        x[1, 17] = float("nan")
    else:
        x[1, 17] = float("inf")
    with S.GpuSampler(vocab_max=2000, rows_max=3, k_max=64) as g:
        p = S.make_params(S.SamplingParams(0.7, 40, 0.9), 3, 0.25)
        with pytest.raises(S.SamplingError) as e:
            g.sample_params(x, p)
        assert e.value.status == S.TABBY_EDOMAIN
        # The other rows are still sampled: run the device form and look at statuses.
        pd = torch.from_numpy(p.view(np.uint8).copy()).cuda()
        rd = torch.zeros(3 * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
        g.sample_device(x, pd, rd)
        res = rd.cpu().numpy().view(S.RESULT_DTYPE)
        assert list(res["status"]) == [0, S.TABBY_EDOMAIN, 0]


def test_device_exp_matches_oracle_exp(oracle):
    import torch
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-60, 1, 400_000), rng.uniform(-750, 712, 100_000),
                        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 709.78, -745.2])])
    y = S.device_exp(torch.from_numpy(x).cuda()).cpu().numpy()
    expected = oracle.exp_array(x)
    bad = np.nonzero(y.view(np.uint64) != expected.view(np.uint64))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at x={x[bad[0]]!r}"


def test_module_level_sample_matches_oracle(oracle):
    import torch
    w = synth.config(1)
    rng = S.SeededRandom(42)
    out = S.sample(torch.from_numpy(w.logits[0]).cuda(), S.SamplingParams(0.7, 40, 0.9), rng)
    u = S.SeededRandom(42).next()
    o = oracle.sample_row(w.logits[0], 40, 0.7, 0.9, u)
    assert out.id == o["id"] and out.consideredCount == o["considered"]


# ---- whole-vocabulary pools (top_k = 0): the head path -----------------------------------

def test_config4_f16_full_vocab_top_p(oracle):
    w = synth.config(4)
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    _log("config4", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


@pytest.mark.parametrize("temperature", [0.0, 0.3, 1.0])
def test_full_vocab_temperatures(oracle, temperature):
    w = synth.config(4, rows=8)
    w.temperature[:] = temperature
    w.top_p[:] = np.array([0.5, 0.9, 0.95, 0.99, 1.0, 0.95, 0.8, 1.0])
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    _log(f"full vocab T={temperature}", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_full_vocab_head_threshold_extremes(oracle):
    # The head's threshold (the smallest key with (l - max)/T >= -37.5 in f64) for
    # temperatures from 1e-4 (a head of ties at the max) to 1e3 (the whole row) and rows whose
    # max sits at 0, +300, -500 and +1e4 (keys far from 1.0 in both directions).
    temps, offsets = (1e-4, 0.01, 3.0, 1e3), (0.0, 300.0, -500.0, 1e4)
    w = synth.random_workload(rows=16, vocab=20000, seed=77, k_choices=(0,), temperatures=(1.0,),
                              top_ps=(0.9,), ties=True, sigma=2.0)
    for r in range(16):
        w.temperature[r] = temps[r % 4]
        w.top_p[r] = (0.5, 0.9, 0.99, 1.0)[(r // 4 + r) % 4]
        w.logits[r] = (w.logits[r].astype(np.float64) + offsets[r // 4]).astype(np.float32)
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    _log("full vocab head threshold extremes", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_full_vocab_flat_row_takes_batched_head(oracle):
    # A hot temperature puts every element in the head: H = V, several sort batches.
    w = synth.random_workload(rows=2, vocab=20000, seed=31, k_choices=(0,), temperatures=(50.0,),
                              top_ps=(0.9, 1.0), sigma=1.0)
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64)


def test_full_vocab_all_equal_and_ties(oracle):
    w = synth.random_workload(rows=3, vocab=9000, seed=41, k_choices=(0,), temperatures=(0.7,),
                              top_ps=(0.9,), ties=True, neg_inf_frac=0.3)
    w.logits[0] = 2.0
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=64)
    compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64)


def test_full_vocab_mixed_with_finite_rows(oracle):
    w = synth.config(3, rows=12, vocab=30000)
    w.top_k[::3] = 0
    res, ids, vals = run_gpu(w, k_max=128, topk_cap=100)
    compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("topk_cap,k_max", [(0, 64), (16, 64), (16, 1024), (300, 1024)])
def test_full_vocab_fast_finish_edges(oracle, dtype, topk_cap, k_max):
    # Whole-vocabulary rows that the merge's sorted top list may finish (head_fast_kernel) or
    # must hand to the sorted head: fewer finite entries than the list (the rest -inf), a spike
    # over a band of ~150 distinct small terms under top-p 0.5 (their ulp counts tie now and
    # then: the sorted head decides those rows), a plateau whose mass pushes the total past its
    # binade, and greedy rows.
    rows, vocab = 32, 30000
    w = synth.random_workload(rows=rows, vocab=vocab, seed=5150 + topk_cap, k_choices=(0,),
                              temperatures=(0.7,), top_ps=(0.95,), sigma=2.0)
    rng = np.random.default_rng(5150)
    for r in range(rows):
        kind = r % 4
        if kind == 0:  # ten finite entries
            keep = rng.choice(vocab, 10, replace=False)
            row = np.full(vocab, -np.inf, np.float32)
            row[keep] = rng.normal(0, 2, 10).astype(np.float32)
            w.logits[r] = row
            w.temperature[r], w.top_p[r] = (0.7, 1.0) if r % 8 == 0 else (0.0, 0.9)
        elif kind == 1:  # spike + band of distinct terms in [2^-8, 2^-7): P_N < 2 with the band
            row = rng.normal(-20, 1, vocab).astype(np.float32)
            row[rng.integers(vocab)] = 10.0
            band = rng.choice(vocab, 150, replace=False)
            row[band] = (10.0 + rng.uniform(np.log(2.0 ** -8), np.log(2.0 ** -7), 150)).astype(np.float32)
            w.logits[r] = row
            w.temperature[r], w.top_p[r] = 1.0, 0.5
        elif kind == 2:  # a plateau of 3,000 near the max: its mass leaves P_N's binade
            row = rng.normal(0, 2, vocab).astype(np.float32)
            row[rng.choice(vocab, 3000, replace=False)] = (12.0 - rng.uniform(0, 0.5, 3000)).astype(np.float32)
            row[rng.integers(vocab)] = 12.0
            w.logits[r] = row
            w.temperature[r], w.top_p[r] = 1.0, 0.05 + 0.1 * (r % 3)
        else:  # config-4-like spikes, greedy every other row
            w.temperature[r] = 0.0 if r % 8 == 3 else 0.3
    w.logits[:] = w.logits.astype(dtype).astype(np.float32)
    if dtype == np.float16:
        w.logits = w.logits.astype(np.float16)
    # k_max 1024: the list comes from merge_kernel (pools above 256); a 300-entry list is too
    # long to hand over, and those rows take the sorted head.
    res, ids, vals = run_gpu(w, k_max=k_max, topk_cap=topk_cap)
    _log(f"full vocab fast finish {dtype.__name__} cap={topk_cap} k_max={k_max}",
         compare(w, res, ids, vals, run_oracle(oracle, w, topk_cap), topk_cap))


def test_full_vocab_rejects_list_above_k_max():
    import torch
    x = torch.zeros(1, 5000, device="cuda")
    with S.GpuSampler(vocab_max=5000, rows_max=1, k_max=64) as g:
        p = S.make_params(S.SamplingParams(0.7, 0, 0.9), 1, 0.5)
        with pytest.raises(S.SamplingError, match="topk_cap"):
            g.sample_params(x, p, topk_cap=65)


# ---- batches of at least as many rows as CUs: the per-row kernel -------------------------
# (row_kernel: one workgroup per row, chunks claimed from an LDS counter, a first bound
# shared by the row's waves, lists merged in LDS.)

def test_row_kernel_mixed_k_ties_neg_inf(oracle):
    # 264 rows of 20,000: ten waves per row (not a power of two), pools up to 256 (four
    # registers per list), ties and -inf, greedy and sampled rows.
    w = synth.random_workload(rows=264, vocab=20000, seed=53, ties=True, neg_inf_frac=0.3,
                              k_choices=(1, 5, 50, 64, 65, 100, 200, 256))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=256)
    _log("row kernel mixed k", compare(w, res, ids, vals, run_oracle(oracle, w, 256), 256))


def test_row_kernel_f16_finite_k(oracle):
    w = synth.config(4, rows=256, vocab=40000)
    w.top_k[:] = np.array([1, 20, 50, 100] * 64, np.int32)
    w.temperature[:] = np.array([0.0, 0.3, 0.7, 1.0] * 64)
    res, ids, vals = run_gpu(w, k_max=128, topk_cap=100)
    _log("row kernel f16", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))


@pytest.mark.parametrize("vocab", [1, 3, 1000, 2049, 4096])
def test_row_kernel_small_vocab(oracle, vocab):
    # One or two waves per row; rows shorter than their k; a row's first chunk partial.
    w = synth.random_workload(rows=256, vocab=vocab, seed=61 + vocab, k_choices=(1, 2, 40, 64, 256))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=64)
    _log(f"row kernel vocab {vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_row_kernel_with_full_vocab_rows(oracle):
    # Whole-vocabulary rows among finite ones: the per-row kernel hands them to the head
    # kernels.
    w = synth.random_workload(rows=256, vocab=12000, seed=71, k_choices=(0, 1, 50, 256),
                              temperatures=(0.0, 0.3, 1.0), top_ps=(0.9, 0.95, 1.0))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=64)
    _log("row kernel + full vocab", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_row_kernel_rows_outside_contract():
    import torch
    rows = 256
    x = torch.randn(rows, 3000, device="cuda")
    x[5] = float("-inf")
    x[77, 1234] = float("nan")
    x[200, 9] = float("inf")
    with S.GpuSampler(vocab_max=3000, rows_max=rows, k_max=64) as g:
        p = S.make_params(S.SamplingParams(0.7, 40, 0.9), rows, 0.25)
        pd = torch.from_numpy(p.view(np.uint8).copy()).cuda()
        rd = torch.zeros(rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
        g.sample_device(x, pd, rd)
        res = rd.cpu().numpy().view(S.RESULT_DTYPE)
    bad = {5, 77, 200}
    for r in range(rows):
        assert res["status"][r] == (S.TABBY_EDOMAIN if r in bad else 0), f"row {r}"


def test_row_kernel_f16_unaligned_vocab(oracle):
    # f16 rows whose length is not a multiple of 8: element loads instead of 16-byte vectors.
    w = synth.config(4, rows=256, vocab=4097)
    w.top_k[:] = np.array([1, 7, 64, 200] * 64, np.int32)
    w.temperature[:] = np.array([0.0, 0.5, 1.0, 2.0] * 64)
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=200)
    _log("row kernel f16 vocab 4097", compare(w, res, ids, vals, run_oracle(oracle, w, 200), 200))


def test_row_kernel_300_rows(oracle):
    # More rows than CUs, not a multiple of 8, with -inf and ties.
    w = synth.random_workload(rows=300, vocab=30000, seed=83, ties=True, neg_inf_frac=0.1,
                              k_choices=(1, 50, 128))
    res, ids, vals = run_gpu(w, k_max=128, topk_cap=128)
    _log("row kernel 300 rows", compare(w, res, ids, vals, run_oracle(oracle, w, 128), 128))


def test_row_kernel_shared_bound_adversarial(oracle):
    # The row kernel's first bound is the k-th largest of the union of the waves' top lane
    # maxima over their first two chunks. Rows built against it, 16 waves per row: the top
    # of the row inside wave 0's first chunk; the top packed into one lane of every chunk (a
    # lane maximum stands for one of its 16 elements); ascending rows (every first chunk is
    # the smallest); the top in the last chunks only (claimed last).
    V = 60000
    w = synth.random_workload(rows=256, vocab=V, seed=97, ties=False,
                              k_choices=(1, 50, 64, 65, 128, 129, 200, 256), sigma=1.0)
    rng = np.random.default_rng(97)
    pos = np.arange(V)
    one_lane = ((pos % 1024) % 256) // 4 == 0  # lane 0 of every 1,024-element chunk
    for r in range(256):
        kind = r % 4
        if kind == 0:
            w.logits[r, :1024] = (12.0 + rng.standard_normal(1024)).astype(np.float32)
        elif kind == 1:
            w.logits[r, one_lane] = (12.0 + rng.standard_normal(int(one_lane.sum()))).astype(np.float32)
        elif kind == 2:
            w.logits[r] = np.sort(w.logits[r])
        else:
            w.logits[r, V - 4096:] = (12.0 + rng.standard_normal(4096)).astype(np.float32)
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=256)
    _log("row kernel shared bound", compare(w, res, ids, vals, run_oracle(oracle, w, 256), 256))


@pytest.mark.parametrize("rows", [1, 5, 17, 64])
def test_row_kernel_parts(oracle, rows):
    # Fewer rows than half the CUs: each row is split into parts of one 16-wave workgroup
    # each (seven parts of 100,000 here, four at 64 rows), and a second kernel merges the
    # parts' sorted lists; ties, -inf, pools up to 256, greedy and whole-vocabulary rows.
    w = synth.random_workload(rows=rows, vocab=100000, seed=101 + rows, ties=True, neg_inf_frac=0.2,
                              k_choices=(0, 1, 50, 64, 65, 256), temperatures=(0.0, 0.3, 1.0))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=64)
    _log(f"row kernel parts, {rows} rows", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


def test_row_kernel_parts_across_calls(oracle):
    # Calls on one handle whose rows are cut into different numbers of parts (ten for a row
    # of 151,936, seven and four for rows of 100,000): each call's part lists and statistics
    # replace the previous call's in the handle's scratch, whatever their number.
    with S.GpuSampler(vocab_max=151936, rows_max=64, k_max=64) as g:
        for i, (rows, vocab) in enumerate([(1, 151936), (5, 100000), (1, 151936), (64, 100000),
                                           (3, 151936), (1, 151936)]):
            w = synth.random_workload(rows=rows, vocab=vocab, seed=900 + i, k_choices=(1, 20, 50, 64),
                                      temperatures=(0.0, 0.7, 1.0), top_ps=(0.9, 1.0))
            res, ids, vals = run_gpu(w, k_max=64, topk_cap=50, sampler=g)
            _log(f"parts call {i}: {rows} x {vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 50), 50))


@pytest.mark.parametrize("vocab", [33000, 49152])
def test_row_kernel_one_workgroup_few_rows(oracle, vocab):
    # Rows of two or three parts' length with few rows: one 16-wave workgroup per row
    # streams and finishes it alone.
    w = synth.random_workload(rows=3, vocab=vocab, seed=7 + vocab, k_choices=(1, 40, 256))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=40)
    _log(f"row kernel one workgroup, vocab {vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 40), 40))


@pytest.mark.parametrize("dtype,vocab", [("f32", 65537), ("f16", 65544), ("f16", 65539)])
def test_row_kernel_parts_ragged(oracle, dtype, vocab):
    # Parts whose last one is short and ends inside a chunk; an odd vocabulary (element
    # loads instead of 16-byte vectors) and f16 rows, aligned and not.
    w = synth.random_workload(rows=2, vocab=vocab, seed=131 + vocab, ties=True, neg_inf_frac=0.1,
                              k_choices=(1, 50, 256), temperatures=(0.0, 0.8))
    if dtype == "f16":
        w.logits = w.logits.astype(np.float16)
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=50)
    _log(f"row kernel parts ragged {dtype} {vocab}", compare(w, res, ids, vals, run_oracle(oracle, w, 50), 50))


def test_full_vocab_huge_tied_head_draw(oracle):
    # Found by a randomized sweep: row 6 (k = 0, T = 2.0, top-p 0.9, u = 0.753) of this
    # workload has a 90 K-entry head of quantised logits, and its draw lands inside a run of
    # 3,573 tied values (positions 13,293 / 13,294). The 64-ary draw search skipped the
    # entries between its last valid probe and its upper bound and drew one position late.
    w = synth.random_workload(rows=200, vocab=100000, seed=770792225, ties=True, neg_inf_frac=0.1,
                              k_choices=(2, 0, 0), temperatures=(0.0, 0.3, 0.7, 1.0, 2.0),
                              top_ps=(0.5, 0.9, 0.95, 1.0))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=40)
    _log("huge tied head", compare(w, res, ids, vals, run_oracle(oracle, w, 40), 40))


U_GRID = (0.0, 0.001, 0.1, 0.25, 0.5, 0.6180339887, 0.75, 0.9, 0.999, 0.9999999998)


@pytest.mark.parametrize("vocab,ties", [(12000, False), (12000, True), (60000, False), (60000, True)])
def test_full_vocab_long_cuts_draw_grid(oracle, vocab, ties):
    # Whole-vocabulary rows whose cut is long (hot temperatures, top-p near 1): heads below
    # 16,384 entries (sums and draw from LDS) and above (from global memory), with and without
    # long tie runs, every row drawn at each point of a grid of uniforms.
    temps, tops = (1.0, 2.0, 50.0), (0.9, 0.99)
    combos = [(t, p, u) for t in temps for p in tops for u in U_GRID]
    w = synth.random_workload(rows=len(combos), vocab=vocab, seed=vocab + int(ties), ties=ties,
                              neg_inf_frac=0.05 if ties else 0.0, k_choices=(0,))
    for r, (t, p, u) in enumerate(combos):
        w.temperature[r], w.top_p[r], w.uniform[r] = t, p, u
    res, ids, vals = run_gpu(w, k_max=64, topk_cap=16)
    _log(f"full vocab long cuts V={vocab} ties={ties}",
         compare(w, res, ids, vals, run_oracle(oracle, w, 16), 16))


@pytest.mark.parametrize("offset", [-500.0, 100.0, 300.0, 1000.0])
def test_sum_exp_shift_invariant(oracle, offset):
    # Logits far from 0: sum-exp, poolMass and the probabilities are relative to the row max
    # (sampler.ts:156-157; tests/sampling.test.ts:73-77), so their accuracy must not depend on
    # where the row sits. Pools of 1, 50, 256 and the whole vocabulary; three kernel paths
    # (the per-row kernel at 256 rows, parts at 8 rows, the two-kernel path at 130 rows).
    for rows in (256, 8, 130):
        w = synth.config(3, rows=rows, vocab=30000 if rows == 256 else 151936)
        w.logits = (w.logits.astype(np.float64) + offset).astype(np.float32)
        w.top_k[:] = np.resize(np.array([1, 50, 256, 0], np.int32), rows)
        res, ids, vals = run_gpu(w, k_max=256, topk_cap=50)
        _log(f"shift {offset:+} rows {rows}", compare(w, res, ids, vals, run_oracle(oracle, w, 50), 50))


def test_config5_full_512_rows(oracle):
    # BASELINE config 5 at its stated size: one slice per row of the 256-lane slice kernel.
    w = synth.config(5)
    assert w.rows == 512
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=1024)
    _log("config5[512 rows]", compare(w, res, ids, vals, run_oracle(oracle, w, 1024), 1024))


@pytest.mark.parametrize("rows", [129, 192, 197, 255])
def test_row_kernel_batches_between_half_and_all_cus(oracle, rows):
    # 129-255 rows with pools up to 256: one 16-wave workgroup per row, as at 256 rows, with
    # the other CUs idle; pools of 1 to 224 take the small-pool path, 256 the sorted merge.
    w = synth.config(3, rows=rows)
    w.top_k[:] = np.resize(np.array([1, 20, 50, 100, 200, 256], np.int32), rows)
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=100)
    _log(f"row kernel {rows} rows", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))


@pytest.mark.parametrize("rows", [64, 61])
def test_wave_kernel_short_rows(oracle, rows):
    # Up to half as many rows as CUs whose rows are too short for two parts take the one-wave
    # slice kernel and its merge kernel; 64 rows (a multiple of 8) place each row's slices on
    # the XCD of its merge, 61 do not.
    w = synth.random_workload(rows=rows, vocab=12000, seed=61 + rows, ties=True, neg_inf_frac=0.1,
                              k_choices=(1, 20, 50, 100, 256), temperatures=(0.0, 0.7, 1.3))
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=100)
    _log(f"wave kernel {rows} short rows", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))


def test_headline_workload_device_form(oracle):
    # The bench's headline exactly: 256 x 151,936 f32, k 50 and top-p 0.9 on every row, k_max
    # 64, device-resident parameters and results, no top-k output.
    import torch
    w = synth.config(3)
    w.top_k[:] = 50
    w.top_p[:] = 0.9
    x = torch.from_numpy(w.logits).cuda()
    pd = torch.from_numpy(params_of(w).view(np.uint8).copy()).cuda()
    rd = torch.zeros(w.rows * S.RESULT_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    with S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=64) as g:
        g.sample_device(x, pd, rd)
        res = rd.cpu().numpy().view(S.RESULT_DTYPE)
    _log("headline device form", compare(w, res, None, None, run_oracle(oracle, w, 0), 0))


def test_exact_boundary_draws_large_pools(oracle):
    # The same boundaries for pools of 257..1024 (the merge kernel's workgroup tail): equal top
    # values make every running sum j/K, so top-p and the target sit on them and the fast
    # sums must hand over to the exact ones; other rows have clear margins.
    V = 30000
    rows = 12
    w = synth.random_workload(rows=rows, vocab=V, seed=977, k_choices=(300,), temperatures=(1.0,),
                              top_ps=(0.5,), sigma=1.0)
    for r in range(rows):
        K = (300, 512, 1024)[r % 3]
        w.top_k[r] = K
        if r < 6:
            w.logits[r, :] = np.minimum(w.logits[r, :], 3.0)
            pos = (np.arange(K) * 997 + r * 13) % V
            w.logits[r, pos] = 7.5
            j = 1 + (r * 37) % (K - 1)
            w.top_p[r] = j / K
            w.uniform[r] = ((r * 53) % K) / K
            w.temperature[r] = (1.0, 0.5, 2.0)[r % 3]
        else:
            w.temperature[r] = (0.7, 1.0, 1.5)[r % 3]
            w.top_p[r] = (0.9, 0.98, 1.0)[(r // 3) % 3]
    res, ids, vals = run_gpu(w, k_max=1024, topk_cap=32)
    _log("exact boundaries, large pools", compare(w, res, ids, vals, run_oracle(oracle, w, 32), 32))


@pytest.mark.parametrize("rows", [256, 4])
def test_exact_boundary_draws(oracle, rows):
    # Pools whose running sums land exactly on top-p and on the draw's target: the top K
    # values are equal, so every weight is 1/K and the running sums are j/K exactly. The
    # cut and the draw then sit on a boundary, where only the sequential sums decide (the
    # fast parallel sums must hand over to the exact ones). 256 rows take the per-row kernel
    # (pools of 65..256 its two- and four-register tails), 4 rows the parts and the merge
    # kernel.
    V = 20000
    w = synth.random_workload(rows=rows, vocab=V, seed=211 + rows, k_choices=(4,), temperatures=(1.0,),
                              top_ps=(0.5,), sigma=1.0)
    for r in range(rows):
        K = (4, 8, 16, 64, 100, 128, 200, 256)[r % 8]
        w.logits[r, :] = np.minimum(w.logits[r, :], 3.0)
        pos = (np.arange(K) * 997 + r * 13) % V
        w.logits[r, pos] = 7.5
        w.top_k[r] = K
        j = 1 + (r // 4) % (K - 1)
        w.top_p[r] = j / K
        w.temperature[r] = (1.0, 0.5, 2.0)[(r // 8) % 3]
        w.uniform[r] = ((r // 24) % K) / K if r % 3 else 0.5
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=64)
    _log(f"exact boundaries, {rows} rows", compare(w, res, ids, vals, run_oracle(oracle, w, 64), 64))


@pytest.mark.parametrize("rows", [256, 4])
def test_small_pool_takes_of_65_to_256(oracle, rows):
    # Pools of at most 256 are selected from the waves' unsorted lists through a 256-bin key
    # histogram. Ties at the K-th largest put more entries in its bin than K: 100, 120, 200 or
    # 250 equal maxima under pools of 50, 64, 100, 128, 200 and 256 take 65..256 entries
    # (sorted in two or four registers); 300 equal maxima take more than 256 (the sorted
    # merge); other rows have pools of 65..256 over N(0, 3^2) logits with and without top-p.
    V = 40000
    w = synth.random_workload(rows=rows, vocab=V, seed=404 + rows, k_choices=(65, 100, 128, 129, 200, 256),
                              temperatures=(0.6, 1.0, 1.7), top_ps=(0.8, 0.95, 1.0), sigma=3.0)
    for r in range(rows):
        if r % 3 == 0:
            ties = (100, 120, 200, 250, 300)[(r // 3) % 5]
            K = (50, 64, 100, 128, 200, 256)[(r // 15) % 6]
            w.logits[r, :] = np.minimum(w.logits[r, :], 4.0)
            w.logits[r, (np.arange(ties) * 331 + r) % V] = 9.0
            w.top_k[r] = K
    res, ids, vals = run_gpu(w, k_max=256, topk_cap=100)
    _log(f"small-pool takes of 65..256, {rows} rows", compare(w, res, ids, vals, run_oracle(oracle, w, 100), 100))
