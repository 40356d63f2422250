"""Shared helpers of the parity tests: run a workload through the C ABI, run it through the
CPU oracle, and compare to the bar the sampler is held to -- bit-exact ids, candidate sets,
counts and maxima; probabilities, pool mass and sum-exp within 1e-5 relative."""
from __future__ import annotations

import numpy as np

from tabby_amd import sampler as S
from tabby_amd.synth import Workload

REL_TOL = 1e-5  # normalised probabilities within 1e-5 relative


def params_of(w: Workload) -> np.ndarray:
    p = np.zeros(w.rows, dtype=S.PARAMS_DTYPE)
    p["temperature"] = w.temperature
    p["top_p"] = w.top_p
    p["uniform"] = w.uniform
    p["top_k"] = w.top_k
    return p


def run_gpu(w: Workload, k_max: int | None = None, topk_cap: int = 0, sampler=None):
    import torch
    dev = torch.from_numpy(np.ascontiguousarray(w.logits)).cuda()
    kmax = k_max or max(1, int(w.top_k.max()))
    own = sampler is None
    g = sampler or S.GpuSampler(vocab_max=w.vocab, rows_max=w.rows, k_max=kmax)
    try:
        res, ids, vals = g.sample_params(dev, params_of(w), topk_cap=topk_cap)
    finally:
        if own:
            g.close()
    return res, ids, vals


def run_oracle(oracle, w: Workload, topk_cap: int = 0, workers: int = 16):
    return oracle.sample_batch(w.logits_f32(), w.top_k, w.temperature, w.top_p, w.uniform,
                               topk_cap=topk_cap, workers=workers)


def rel(a: float, b: float) -> float:
    return abs(a - b) / max(abs(b), 1e-300)


def compare(w: Workload, res, ids, vals, expected, topk_cap: int = 0) -> dict:
    """Asserts parity row by row; returns summary statistics for the log."""
    worst_prob = worst_mass = worst_sum = 0.0
    boundary_rows = 0
    for r in range(w.rows):
        o = expected[r]
        g = res[r]
        ctx = (f"{w.name} row {r}: k={int(w.top_k[r])} T={w.temperature[r]} "
               f"p={w.top_p[r]} u={w.uniform[r]!r}")
        assert g["status"] == o["status"] == 0, f"{ctx}: status gpu={g['status']} oracle={o['status']}"
        assert int(g["id"]) == o["id"], f"{ctx}: id gpu={int(g['id'])} oracle={o['id']}"
        assert int(g["considered"]) == o["considered"], f"{ctx}: consideredCount"
        assert np.float32(g["max_logit"]) == np.float32(o["max_logit"]), f"{ctx}: maxLogit"
        worst_prob = max(worst_prob, rel(float(g["probability"]), o["probability"]))
        worst_mass = max(worst_mass, rel(float(g["pool_mass"]), o["pool_mass"]))
        worst_sum = max(worst_sum, rel(float(g["sum_exp"]), o["sum_exp"]))
        assert rel(float(g["probability"]), o["probability"]) < REL_TOL, f"{ctx}: probability"
        assert rel(float(g["pool_mass"]), o["pool_mass"]) < REL_TOL, f"{ctx}: poolMass"
        assert rel(float(g["sum_exp"]), o["sum_exp"]) < REL_TOL, f"{ctx}: sumExp"
        # poolExhausted compares poolMass with topP; within the sum-exp tolerance of the
        # boundary the flag is decided by ulps of sumExp, so only rows clear of it must agree.
        if abs(o["pool_mass"] - w.top_p[r]) > REL_TOL * w.top_p[r]:
            assert bool(g["pool_exhausted"]) == o["pool_exhausted"], f"{ctx}: poolExhausted"
        else:
            boundary_rows += 1
        if topk_cap:
            n = int(g["topk_count"])
            assert n == len(o["topk_ids"]), f"{ctx}: topk count {n} vs {len(o['topk_ids'])}"
            assert np.array_equal(ids[r, :n], o["topk_ids"]), f"{ctx}: top-k ids differ"
            assert np.array_equal(vals[r, :n].view(np.uint32), o["topk_values"].view(np.uint32)), \
                f"{ctx}: top-k logits differ"
    return {"rows": w.rows, "worst_prob_rel": worst_prob, "worst_mass_rel": worst_mass,
            "worst_sumexp_rel": worst_sum, "boundary_rows": boundary_rows}
