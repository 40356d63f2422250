"""The C ABI boundary without a GPU: the library loads, exports exactly what
include/tabby_sampler.h declares, and the Python host side mirrors the reference's
value types. No sampling call is made here (that needs an MI355X)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from tabby_amd import build as B
from tabby_amd import sampler as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tabby_sampler.h")


def declared_symbols():
    text = open(HEADER).read()
    return re.findall(r"TABBY_API\s+[\w\s\*]+?\b(tabby_\w+)\s*\(", text)


def test_header_declares_the_bound_symbols():
    assert sorted(declared_symbols()) == sorted(S.EXPORTED_SYMBOLS)


def test_header_cites_the_reference_for_each_entry_point():
    text = open(HEADER).read()
    for name in declared_symbols():
        if name in ("tabby_last_error", "tabby_version"):
            continue
        block = text[:text.index(name)].rsplit("*/", 2)[-2]
        if "no counterpart in the" in " ".join(block.split()):
            # An addition of this library (the allocation-free entry, the measurement
            # diagnostic): its comment says so and names the callers it is for.
            assert "cannot allocate" in block or "for measurements" in block, \
                f"{name} does not name its callers"
            continue
        assert re.search(r"\.ts:\d+", block), f"{name} has no reference citation"


def test_library_exports_every_declared_symbol():
    assert os.path.exists(B.LIB_PATH), "build the library first (python -m tabby_amd.build)"
    lib = ctypes.CDLL(B.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", B.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    tabby = {s for s in exported if s.startswith("tabby_")}
    assert tabby == set(declared_symbols()), tabby ^ set(declared_symbols())


def test_timeline_library_adds_only_its_reader():
    # The timeline build (row kernel phase stamps for bench.py --timeline) exports the same
    # boundary plus tabby_debug_timeline; the plain library does not export the reader.
    assert os.path.exists(B.TIMELINE_LIB_PATH), "build the library first (python -m tabby_amd.build)"
    out = subprocess.run(["nm", "-D", "--defined-only", B.TIMELINE_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    tabby = {s for s in exported if s.startswith("tabby_")}
    assert tabby == set(declared_symbols()) | {"tabby_debug_timeline"}


def test_version_and_last_error_are_callable_without_a_device():
    lib = S.load_library()
    assert lib.tabby_version().decode().startswith("tabby")
    assert isinstance(lib.tabby_last_error(), bytes)


def test_struct_layouts_match_the_header():
    # tabby_row_params: 3 doubles + 2 int32 = 32 B; tabby_row_result: 48 B.
    assert S.PARAMS_DTYPE.itemsize == 32 and S.RESULT_DTYPE.itemsize == 48
    assert [S.RESULT_DTYPE.fields[n][1] for n in ("id", "considered", "probability", "pool_mass",
                                                   "max_logit", "pool_exhausted", "sum_exp",
                                                   "status", "topk_count")] == [0, 4, 8, 16, 24, 28, 32, 40, 44]
    text = open(HEADER).read()
    for field in ("temperature", "top_p", "uniform", "top_k", "reserved"):
        assert re.search(rf"\b{field};", text), field


def test_status_codes_match_the_header():
    text = open(HEADER).read()
    for name in ("TABBY_OK", "TABBY_EINVAL", "TABBY_EHIP", "TABBY_EEMPTY", "TABBY_EDOMAIN",
                 "TABBY_ECAPACITY"):
        m = re.search(rf"{name}\s*=\s*(\d+)", text)
        assert m and int(m.group(1)) == getattr(S, name), name


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(S, "_lib", None)
    with pytest.raises(ImportError, match="missing"):
        S.load_library(str(tmp_path / "nope.so"))


def test_default_sampling_and_params_packing():
    d = S.DEFAULT_SAMPLING  # sampler.ts:93-98
    assert (d.temperature, d.topK, d.topP, d.seed) == (0.7, 40, 0.9, 0)
    p = S.make_params(S.SamplingParams(0.5, 20, 0.8), 3, [0.1, 0.2, 0.3])
    assert p.dtype == S.PARAMS_DTYPE and p.shape == (3,)
    assert np.all(p["top_k"] == 20) and np.all(p["reserved"] == 0)
    assert p["uniform"].tolist() == [0.1, 0.2, 0.3]


def test_rng_is_advanced_only_for_non_greedy_rows():
    # sampler.ts:159-167 + :194 -- a greedy row consumes no uniform.
    params = [S.SamplingParams(0.7, 40, 0.9), S.SamplingParams(0.0, 40, 0.9),
              S.SamplingParams(1.0, 5, 1.0)]
    p = S.make_params(params, 3, S.SeededRandom(9))
    ref = S.SeededRandom(9)
    a, b = ref.next(), ref.next()
    assert p["uniform"].tolist() == [a, 0.0, b]


def test_nan_and_inf_temperature_refused_before_any_uniform():
    # A NaN or +inf temperature is refused (the device form gives TABBY_EINVAL for the row);
    # the host raises before advancing the RNG. -0 and -inf are greedy (T <= 0) and draw none.
    for t in (float("nan"), float("inf")):
        rng = S.SeededRandom(9)
        with pytest.raises(ValueError, match="temperature must not be NaN or \\+Infinity"):
            S.make_params([S.SamplingParams(0.7, 40, 0.9), S.SamplingParams(t, 40, 0.9)], 2, rng)
        assert rng.state == 9
    p = S.make_params([S.SamplingParams(-0.0, 40, 0.9), S.SamplingParams(float("-inf"), 40, 0.9)], 2,
                      S.SeededRandom(9))
    assert p["uniform"].tolist() == [0.0, 0.0]
