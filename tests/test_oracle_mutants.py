"""The oracle's pins must reject plausible mistakes -- CPU only.

Each case copies oracle/tabby_oracle.c to a temporary directory, plants one mistake in the
copy (a flipped comparison, a dropped term, a wrong constant or index), builds it with gcc,
routes the oracle module through the broken build, and requires at least one of the pins in
test_oracle.py to fail. The committed oracle source is never modified.
"""
import os
import shutil
import subprocess

import pytest

import test_oracle as pins

ORACLE_SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")

MUTANTS = {
    "ties by id descending": ("return (a->id > b->id) - (a->id < b->id);",
                              "return (a->id < b->id) - (a->id > b->id);"),
    "values ascending": ("if (a->value > b->value) return -1;\n  if (a->value < b->value) return 1;",
                         "if (a->value > b->value) return 1;\n  if (a->value < b->value) return -1;"),
    "argmax keeps the last tie": ("if (row[i] > best_value)", "if (row[i] >= best_value)"),
    "top-p strict comparison": ("if (cumulative >= top_p) {", "if (cumulative > top_p) {"),
    "draw non-strict comparison": ("if (target < running) {", "if (target <= running) {"),
    "total over the whole pool": ("for (int32_t i = 0; i < cut; ++i) total += weights[i];",
                                  "for (int32_t i = 0; i < count; ++i) total += weights[i];"),
    "probability from the scaled weights": ("out->probability = exact[chosen];",
                                            "out->probability = weights[chosen];"),
    "greedy only below zero": ("if (temperature <= 0.0) {", "if (temperature < 0.0) {"),
    "exhausted flag inverted": ("if (pool_mass < top_p) exhausted = 1;",
                                "if (pool_mass > top_p) exhausted = 1;"),
    "weights without the max": ("weights[i] = tabby_oracle_exp(((double)logits[i] - max_logit) / temperature);",
                                "weights[i] = tabby_oracle_exp((double)logits[i] / temperature);"),
    "sumExp without the max": ("sum += tabby_oracle_exp((double)row[i] - (double)max_logit);",
                               "sum += tabby_oracle_exp((double)row[i]);"),
    "poolMass skips the first term": ("for (int32_t i = 0; i < count; ++i) pool_mass += exact[i];",
                                      "for (int32_t i = 1; i < count; ++i) pool_mass += exact[i];"),
    "mulberry32 shift": ("uint32_t t = (s ^ (s >> 15)) * (s | 1u);",
                         "uint32_t t = (s ^ (s >> 16)) * (s | 1u);"),
    "mulberry32 increment": ("*state + 0x6d2b79f5u", "*state + 0x6d2b79f3u"),
    "exp drops the P5 term": ("t * (kP4 + t * kP5)", "t * (kP4)"),
    "exp without the e special case": ("if (x == 1.0) return kE;", ""),
    "exp ln2 low part sign": ("lo = t * kLn2Lo;", "lo = -t * kLn2Lo;"),
    "exp tiny-argument branch": ("return 1.0 + x;", "return 1.0;"),
    "f16 subnormal scale": ("ldexp((double)mantissa / 1024.0, -14)", "ldexp((double)mantissa / 1024.0, -15)"),
    "f16 exponent bias": ("exponent - 15)", "exponent - 14)"),
    "softmax causal prefix one short": ("causal_offset + (row % causal_period) + 1",
                                        "causal_offset + (row % causal_period)"),
    "softmax without the max": ("(float)((double)o[i] - (double)max_v)", "(float)((double)o[i])"),
    "softmax tail not zeroed": ("for (int32_t i = valid; i < row_len; ++i) o[i] = 0.0f;", ""),
    "q4 offset seven": ("(int32_t)raw - 8 :", "(int32_t)raw - 7 :"),
    "q4 scale of the wrong block": ("const float scale = srow[w / words_per_block];",
                                    "const float scale = srow[(w + 1) / words_per_block % blocks_per_row];"),
    "q4 bias skipped": ("if (bias) acc = (float)((double)acc + (double)bias[m]);", ""),
    "q4 products not rounded to f32": ("const float prod = (float)((double)centred * (double)xt[k0 + lane]);",
                                       "const double prod = (double)centred * (double)xt[k0 + lane];"),
    "softmax sum skips the first exp": ("    o[i] = e;\n      sum = (float)((double)sum + (double)e);",
                                        "    o[i] = e;\n      if (i > 0) sum = (float)((double)sum + (double)e);"),
}


def _battery(oracle, vectors, fixture):
    """Cheap pins first; stops at the first failure."""
    checks = [
        lambda: pins.test_fixture_outcomes_match_closed_forms(oracle, fixture),
        lambda: pins.test_fixture_assertions_of_the_reference(oracle, fixture),
        lambda: pins.test_fixture_probability_is_exact_term_of_chosen(oracle, fixture),
        lambda: pins.test_greedy_does_not_depend_on_uniform(oracle, fixture),
        lambda: pins.test_shift_invariance_of_the_tail(oracle, fixture),
        lambda: pins.test_draw_intervals_are_half_open(oracle),
        lambda: pins.test_mulberry32_matches_node_vectors(oracle, vectors),
        lambda: pins.test_exp_matches_v8_vectors(oracle, vectors),
        lambda: pins.test_exp_special_values_and_accuracy(oracle),
        lambda: pins.test_f16_widening_exhaustive(oracle),
        lambda: pins.test_topk_special_rows(oracle),
        lambda: pins.test_argmax_is_lowest_index_of_max(oracle),
        lambda: pins.test_topk_matches_stable_library_sort(oracle),
        lambda: pins.test_sum_exp_is_sequential_f64_sum(oracle),
        lambda: pins.test_draw_is_inverse_cdf_over_a_grid(oracle),
        lambda: pins.test_c_oracle_matches_node_vectors(oracle, vectors),
        lambda: pins.test_softmax_closed_forms(oracle),
        lambda: pins.test_softmax_reference_kernel_test_assertions(oracle),
        lambda: pins.test_softmax_rows_match_float64_math(oracle),
        lambda: pins.test_softmax_matches_node_vectors(oracle, pins._load("softmax_vectors.json")),
        lambda: pins.test_matmul_quantized_closed_form(oracle),
        lambda: pins.test_matmul_quantized_bias_bits8_and_batches(oracle),
        lambda: pins.test_matmul_quantized_on_the_reference_test_shapes(oracle),
    ]
    for i, check in enumerate(checks):
        try:
            check()
        except AssertionError:
            return i
    return None


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pins_reject_mutant(oracle, tmp_path, name):
    vectors = pins._load("node_vectors.json")
    fixture = pins._load("sampling_fixture.json")
    src = open(os.path.join(ORACLE_SRC, "tabby_oracle.c")).read()
    old, new = MUTANTS[name]
    assert src.count(old) == 1, f"mutation anchor not found once: {old!r}"
    (tmp_path / "tabby_oracle.c").write_text(src.replace(old, new))
    shutil.copy(os.path.join(ORACLE_SRC, "tabby_oracle.h"), tmp_path / "tabby_oracle.h")
    so = tmp_path / "libmutant.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-o", str(so),
                    str(tmp_path / "tabby_oracle.c"), "-lm"], check=True)
    with oracle.using(oracle.load(str(so))):
        caught = _battery(oracle, vectors, fixture)
    assert caught is not None, f"no pin rejects the mutant '{name}'"


def test_unmutated_copy_passes_the_battery(oracle, tmp_path):
    vectors = pins._load("node_vectors.json")
    fixture = pins._load("sampling_fixture.json")
    shutil.copy(os.path.join(ORACLE_SRC, "tabby_oracle.c"), tmp_path / "tabby_oracle.c")
    shutil.copy(os.path.join(ORACLE_SRC, "tabby_oracle.h"), tmp_path / "tabby_oracle.h")
    so = tmp_path / "libcopy.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-o", str(so),
                    str(tmp_path / "tabby_oracle.c"), "-lm"], check=True)
    with oracle.using(oracle.load(str(so))):
        assert _battery(oracle, vectors, fixture) is None
