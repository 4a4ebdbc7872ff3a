"""CPU checks of bench.py's contract: the one-GPU guard, the committed traffic
record lookup and the synthetic selection of the north-star workload."""

import json
import os
import subprocess
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, cwd=ROOT, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_traffic_record_matches_only_its_workload():
    with open(bench.TRAFFIC_FILE) as f:
        rec = json.load(f)
    assert rec["workload"] == "T32768_H16_D128_r0.25_seed2"
    for name, ent in rec["kernels"].items():
        assert ent["bytes_per_launch"] == ent["read_bytes"] + ent["write_bytes"]
        assert bench.measured_traffic(name, 32768, 16, 128, 0.25, 2) == ent["bytes_per_launch"]
    assert bench.measured_traffic("logo_sq_bwd_dkv", 16384, 16, 128, 0.25, 2) is None
    assert bench.measured_traffic("no_such_kernel", 32768, 16, 128, 0.25, 2) is None


def test_markov_selection_ratio_and_runs():
    g = torch.Generator()
    g.manual_seed(2)
    sel = bench.markov_mask(32768, 0.25, 8, g)
    assert sel.dtype == np.bool_ and sel.shape == (32768,)
    assert abs(sel.mean() - 0.25) < 0.03
    # mean length of the selected runs is about 8 (P(1 -> 0) = 1/8)
    starts = np.flatnonzero(sel & ~np.concatenate(([False], sel[:-1])))
    assert 6.0 < sel.sum() / len(starts) < 10.0
