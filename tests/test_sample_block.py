"""The sample block a decode step reads back (src/engine/forward.ts:127-157): the layout
[maxLogit, sumExp, (value, index) * k] as f32 words with each index a u32 in its word, written
and read by the Python and Node hosts alike. CPU only."""
import base64
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from tabby_amd import sampler as S
from tabby_amd.build import NODE_ADDON

HERE = os.path.dirname(os.path.abspath(__file__))

TOP = S.TopKResult(maxLogit=17.25, sumExp=3.0517578125,
                   ids=[151935, 0, 7, 2**31 + 5, 42], logits=[17.25, -0.0, 3.5, float("-inf"), 1e-30])


def test_layout_matches_the_reference_words():
    raw = S.encode_sample_block(TOP)
    f = np.frombuffer(raw, dtype=np.float32)
    u = np.frombuffer(raw, dtype=np.uint32)
    assert f.size == 2 + 2 * len(TOP.ids)
    assert f[0] == np.float32(17.25) and f[1] == np.float32(3.0517578125)
    for i, (idx, v) in enumerate(zip(TOP.ids, TOP.logits)):
        assert u[3 + 2 * i] == idx  # the index: u32 bits in the odd word, not a float value
        assert f[2 + 2 * i].tobytes() == np.float32(v).tobytes()  # -0.0 and -inf kept bit for bit


def test_round_trip_and_prefix():
    for k in (0, 1, 3, len(TOP.ids)):
        got = S.decode_sample_block(S.encode_sample_block(TOP), k)
        assert got.ids == TOP.ids[:k]
        assert [np.float32(v).tobytes() for v in got.logits] == [np.float32(v).tobytes() for v in TOP.logits[:k]]
        assert got.maxLogit == 17.25 and got.sumExp == np.float32(3.0517578125)
    # a block of k slots read for fewer candidates
    assert S.decode_sample_block(S.encode_sample_block(TOP), 2).ids == TOP.ids[:2]
    # sumExp travels as f32, as in the reference's sampleOut buffer
    assert S.decode_sample_block(S.encode_sample_block(S.TopKResult(1.0, 1.0 / 3.0, [], [])), 0).sumExp \
        == float(np.float32(1.0 / 3.0))


def test_rejects_bad_sizes():
    with pytest.raises(ValueError):
        S.encode_sample_block(TOP, len(TOP.ids) + 1)
    with pytest.raises(ValueError):
        S.decode_sample_block(S.encode_sample_block(TOP, 2), 3)


@pytest.mark.skipif(shutil.which("node") is None or not os.path.exists(NODE_ADDON),
                    reason="node or the built addon is missing")
def test_node_host_writes_and_reads_the_same_bytes():
    block = S.encode_sample_block(TOP)
    spec = {"top": {"maxLogit": TOP.maxLogit, "sumExp": TOP.sumExp, "ids": TOP.ids,
                    "logits": [v if np.isfinite(v) else None for v in TOP.logits]},
            "k": len(TOP.ids), "block64": base64.b64encode(block).decode()}
    # JSON has no -inf: send the block for the decode check, and encode a finite copy
    spec["top"]["logits"] = [17.25, -0.0, 3.5, -1e30, 1e-30]
    r = subprocess.run(["node", os.path.join(HERE, "node_host.js"), "wire", json.dumps(spec)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    finite = S.TopKResult(TOP.maxLogit, TOP.sumExp, TOP.ids, [17.25, -0.0, 3.5, -1e30, 1e-30])
    assert base64.b64decode(out["encoded"]) == S.encode_sample_block(finite)
    dec = out["decoded"]
    assert dec["ids"] == TOP.ids and dec["maxLogit"] == 17.25
    assert dec["logits"][:3] == [17.25, 0.0, 3.5] and dec["logits"][3] is None  # -inf: JSON null
