"""bench.py's host-side contract, without a GPU: the multi-GPU refusal and the guard that
keeps a failing extra configuration from costing the run its JSON line."""
import subprocess
import sys

import bench


def test_extra_records_an_exception_instead_of_raising():
    def boom(x):
        raise RuntimeError(f"no {x}")

    assert bench._extra(boom, "box") == {"error": "RuntimeError: no box"}
    assert bench._extra(lambda a, b: {"v": a + b}, 1, 2) == {"v": 3}


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, bench.__file__, "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""
