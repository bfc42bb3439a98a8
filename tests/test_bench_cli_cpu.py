"""bench.py's command-line contract, checked without a GPU: more than one GPU
is refused with a message before anything touches the device, and the
percentile helper used for the per-replay spread is the nearest-rank one."""

import os
import subprocess
import sys

from conftest import ROOT

sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_percentiles_nearest_rank():
    p = bench.percentiles([5.0, 1.0, 3.0, 2.0, 4.0])
    assert p == {"median": 3.0, "p10": 1.0, "p90": 5.0, "samples": 5}
    p = bench.percentiles([float(i) for i in range(101)])
    assert (p["median"], p["p10"], p["p90"]) == (50.0, 10.0, 90.0)
