"""bench.py's host-side contract, on the CPU (no device is touched)."""
import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_clock_warmup_runs_the_step_for_the_requested_time(monkeypatch):
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    calls = []
    out = bench._clock_warmup(lambda i: calls.append(i), 0.05)
    assert out["s"] >= 0.05 and out["steps"] == len(calls) >= 10
    assert out["steps"] % 10 == 0 and set(calls) == {0}
    calls.clear()
    assert bench._clock_warmup(lambda i: calls.append(i), 0.0)["steps"] == 0
    assert calls == []


def test_workload_is_baseline_config_2():
    assert bench.SHAPE == (2, 16, 2048, 64)
    assert bench.pairs(2, 16, 2048) == 67141632
    assert bench.kernel_flops_per_pair(64) == {"ca_fwd": 256, "ca_bwd_dkdv": 512, "ca_bwd_dq": 128}
