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
    # A NaN or +inf temperature throws before any uniform is drawn; -0 is greedy (T <= 0).
    assert rep["temperatureErrors"] == ["temperature must not be NaN or +Infinity, got NaN",
                                        "temperature must not be NaN or +Infinity, got Infinity"]
    assert rep["stateAfterTemperatureErrors"] == rep["stateAfterSample"]
    assert rep["negZero"]["id"] == oracle.argmax(row) and rep["negZero"]["consideredCount"] == 1
    assert rep["stateAfterNegZero"] == rep["stateAfterSample"]


@needs_node
def test_pool_size_is_the_workers_rule():
    # inference.worker.ts:118-123: T <= 0 -> 1; else min(64, max(1, topK || 64)).
    out = subprocess.run(["node", "-e", (
        "const t = require(process.argv[1]);"
        "const cases = [[0.7, 40], [0, 40], [-1, 0], [0.7, 0], [1.0, 100], [0.5, 1], [0.5, 64], [0.5, 65]];"
        "console.log(JSON.stringify(cases.map(([T, k]) => t.poolSize({temperature: T, topK: k}))));"
        "console.log(JSON.stringify([t.poolSize({temperature: 1, topK: 0}, 256), t.poolSize({temperature: 1, topK: 300}, 256)]));"),
        os.path.join(os.path.dirname(HERE), "tabby_amd", "node", "index.js")],
        capture_output=True, text=True, check=True).stdout.splitlines()
    assert json.loads(out[0]) == [40, 1, 1, 64, 64, 1, 64, 64]
    assert json.loads(out[1]) == [256, 256]


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [5000, 151936])
def test_decode_loop_seeded_determinism(vocab):
    # sampling.test.ts:151-204 on a synthetic model: seed 42 replays identically, seed 43
    # differs, temperature 0 does not depend on the seed -- and every run's ids equal the CPU
    # restatement's replay of the worker's loop (sampleFromTopK over a poolSize pool).
    r = json.loads(_node("decode", str(vocab), timeout=300).strip().splitlines()[-1])
    assert r["seed42"]["tokens"] == r["seed42again"]["tokens"]
    assert r["seed43"]["tokens"] != r["seed42"]["tokens"]
    assert r["greedy1"]["tokens"] == r["greedy999"]["tokens"]
    assert len(r["seed42"]["tokens"]) == 24 and not r["seed42"]["stopped"]
    for name in ("seed42", "seed43", "greedy1", "topK0"):
        assert r[name]["tokens"] == r["cpu"][name]["tokens"], name
    # One 48-byte result read back per token (the reference reads (2 + 2k) * 4 bytes).
    assert r["seed42"]["readbackPerToken"] == 48
    assert r["seed42"]["totalReadback"] == 48 * 24
    # Stop token: the loop ends at its first occurrence, which is emitted.
    stop = r["stop"]
    assert stop["stopped"] and stop["tokens"] == r["cpu"]["stop"]["tokens"]
    assert stop["tokens"][-1] == r["stopId"] and r["stopId"] not in stop["tokens"][:-1]
    assert [i for _, i in stop["seen"]] == list(range(len(stop["tokens"])))
    # A cancel during the third decode: the prefill's token and two decodes' are emitted.
    c = r["cancelInFlight"]
    assert c["cancelled"] and c["decodes"] == 3 and c["tokens"] == r["seed42"]["tokens"][:3]
    # A cancel before anything is emitted.
    assert r["cancelFirst"]["cancelled"] and r["cancelFirst"]["tokens"] == []


@needs_node
@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [4999, 151936])
def test_generate_greedy_and_argmax(vocab):
    # sampler.ts:54-76 with the argmax on the GPU: the same ids as the CPU argmax loop, onToken
    # per step, a stop token ends it, an aborted signal throws before the next forward.
    r = json.loads(_node("greedy", str(vocab), timeout=300).strip().splitlines()[-1])
    assert r["plain"]["tokens"] == r["cpuTokens"] and not r["plain"]["stopped"]
    assert r["seen"] == [[t, i] for i, t in enumerate(r["cpuTokens"])]
    assert r["stopped"]["stopped"] and r["stopped"]["tokens"] == r["cpuTokens"][:5]
    assert r["abortError"] == "AbortError" and r["abortedTokens"] == r["cpuTokens"][:4]
    assert all(g == c for g, c in r["special"]), r["special"]


@needs_node
@pytest.mark.gpu
def test_node_softmax_rows_bit_exact(oracle, tmp_path):
    rng = np.random.default_rng(21)
    for n_rows, row_len, period, offset in ((15, 5, 5, 0), (28, 700, 14, 686), (3, 5000, 0, 0)):
        x = rng.normal(0, 4, n_rows * row_len).astype(np.float32)
        xp, yp, sp = tmp_path / "x.f32", tmp_path / "y.f32", tmp_path / "s.json"
        x.tofile(xp)
        sp.write_text(json.dumps({"x": str(xp), "nRows": n_rows, "rowLen": row_len, "period": period,
                                  "offset": offset, "out": str(yp)}))
        _node("softmax", str(sp))
        got = np.fromfile(yp, dtype=np.float32)
        want = oracle.softmax_rows(x, n_rows, row_len, period, offset)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n_rows, row_len)
