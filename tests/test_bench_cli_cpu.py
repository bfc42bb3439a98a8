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


def test_zipf_targets_closed_forms():
    """Water-filled Zipf row targets: they sum to T*k, never exceed T, fall
    with rank; s = 0 is uniform; without saturation n_r is proportional to
    r^-s; at the T=4096 MoE workload the most popular expert saturates."""
    t = bench.zipf_targets(128, 4096, 8, 1.1)
    assert abs(sum(t) - 4096 * 8) < 1e-3
    assert max(t) == 4096.0 and t[1] < 4096.0  # exactly one saturated expert
    assert all(a >= b for a, b in zip(t, t[1:]))
    assert min(t) > 32.0  # every expert keeps some rows under Zipf(1.1)
    u = bench.zipf_targets(16, 100, 4, 0.0)
    assert all(abs(v - 25.0) < 1e-6 for v in u)
    z = bench.zipf_targets(8, 10000, 1, 2.0)  # T*k = T: nothing saturates
    for r in range(1, 8):
        assert abs(z[r] / z[0] - (r + 1) ** -2.0) < 1e-9


def test_zipf_router_bias_fit():
    """The fitted bias routes a synthetic 4096-token batch (router logits of
    N(0,1) tokens and N(0, 0.02) weights) to within 2% L1 of the Zipf(1.1)
    targets, with the most popular expert taking every token."""
    import torch

    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, 2048, generator=g)
    w = torch.randn(128, 2048, generator=g) * 0.02
    bias, tgt = bench.zipf_router_bias(x, w, 8)
    idx = torch.topk(x @ w.t() + bias, 8, dim=1).indices
    h = bench.routing_histogram(idx, tgt, 4096)
    assert h["l1_vs_target"] < 0.02
    assert h["achieved_rows_top8"][0] == 4096
    assert h["touched_experts"] == 128 and h["experts_below_32_rows"] == 0
