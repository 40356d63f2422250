"""The Node host (tabby_amd/node: N-API addon + index.js) against the CPU oracle."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from tabby_amd import synth
from tabby_amd.build import NODE_ADDON

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER = os.path.join(HERE, "node_host.js")

needs_node = pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(NODE_ADDON),
                                reason="node or the built addon is missing")


def _node(*args, timeout=120):
    r = subprocess.run(["node", DRIVER, *args], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]
    return r.stdout


@needs_node
def test_addon_loads_without_a_gpu():
    out = json.loads(_node("load").strip().splitlines()[-1])
    assert out["version"].startswith("tabby_sampler")


def _run(w, tmp_path, k_max, cap):
    lp = tmp_path / "logits.bin"
    f16 = w.logits.dtype == np.float16
    (w.logits.view(np.uint16) if f16 else w.logits).tofile(lp)
    spec = {"logits": str(lp), "dtype": "f16" if f16 else "f32", "rows": w.rows, "vocab": w.vocab,
            "topK": [int(v) for v in w.top_k], "temperature": [float(v) for v in w.temperature],
            "topP": [float(v) for v in w.top_p], "uniform": [float(v) for v in w.uniform],
            "topkCap": cap, "kMax": k_max, "out": str(tmp_path / "out.json")}
    sp = tmp_path / "spec.json"
    sp.write_text(json.dumps(spec))
    _node("sample", str(sp))
    return json.loads((tmp_path / "out.json").read_text())


def _check(w, outs, oracle, cap):
    ref = oracle.sample_batch(w.logits_f32(), w.top_k, w.temperature, w.top_p, w.uniform, topk_cap=cap)
    for r, (g, o) in enumerate(zip(outs, ref)):
        ctx = f"{w.name} row {r}"
        assert g["id"] == o["id"], ctx
        assert g["consideredCount"] == o["considered"], ctx
        assert abs(g["probability"] - o["probability"]) <= 1e-5 * o["probability"], ctx
        assert abs(g["poolMass"] - o["pool_mass"]) <= 1e-5 * o["pool_mass"], ctx
        if cap:
            assert g["top"]["ids"] == o["topk_ids"].tolist(), ctx
            assert g["top"]["maxLogit"] == o["max_logit"], ctx


@needs_node
@pytest.mark.gpu
def test_node_batch_matches_oracle(oracle, tmp_path):
    w = synth.config(3, rows=16, vocab=49152)
    _check(w, _run(w, tmp_path, 128, 100), oracle, 100)


@needs_node
@pytest.mark.gpu
def test_node_f16_whole_vocab_matches_oracle(oracle, tmp_path):
    w = synth.config(4, rows=4, vocab=30000)
    _check(w, _run(w, tmp_path, 64, 64), oracle, 64)


@needs_node
@pytest.mark.gpu
def test_node_ties_neg_inf_matches_oracle(oracle, tmp_path):
    w = synth.random_workload(rows=8, vocab=20000, seed=77, ties=True, neg_inf_frac=0.3,
                              k_choices=(1, 7, 64, 200))
    _check(w, _run(w, tmp_path, 256, 200), oracle, 200)


@needs_node
@pytest.mark.gpu
def test_node_sample_api_rng_and_errors(oracle):
    rep = json.loads(_node("api").strip().splitlines()[-1])
    row = np.array(rep["row"], dtype=np.float32)
    # Greedy: argmax, one candidate considered, the uniform not consumed (sampler.ts:159-167).
    assert rep["greedy"]["id"] == oracle.argmax(row) and rep["greedy"]["consideredCount"] == 1
    assert rep["stateAfterGreedy"] == 42
    # DEFAULT_SAMPLING (T 0.7, k 40, p 0.9) with the first draw of SeededRandom(42).
    u = oracle.mulberry32(42, 1)[0]
    o = oracle.sample_row(row, 40, 0.7, 0.9, float(u))
    assert rep["sampled"]["id"] == o["id"] and rep["sampled"]["consideredCount"] == o["considered"]
    assert rep["stateAfterSample"] == (42 + 0x6D2B79F5) & 0xFFFFFFFF
    # forward.ts:348-351: topK out of range is rejected before any GPU work or RNG use.
    assert "topK must be between 0 and 64, got 65" in rep["topKError"]
    assert rep["stateAfterError"] == rep["stateAfterSample"]
