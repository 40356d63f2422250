"""bench.py's command-line contract that needs no GPU: it measures one GPU only and says so."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "8"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that did not happen


def test_bench_secondary_modes_refuse_more_than_one_gpu():
    # The diagnostic modes (--timeline loads the timeline build of the library) keep the same
    # one-GPU contract and print no JSON line when refused.
    for mode in ("--timeline", "--read-ceiling"):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), mode, "--gpus", "2"],
                           capture_output=True, text=True, timeout=60)
        assert r.returncode == 2, mode
        assert "one GPU only" in r.stderr, mode
        assert r.stdout == "", mode
