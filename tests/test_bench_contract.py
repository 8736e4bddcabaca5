"""The bench line's contract pieces that need no GPU: the refusal of more than one GPU, and the committed rocprofv3
summaries it reads (HBM traffic and MFMA counters) for every decode workload."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

WORKLOADS = ["cfg1", "cfg2", "cfg3", "cfg3-bf16", "cfg4", "cfg4-swa128", "cfg5"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stdout + r.stderr


@pytest.mark.parametrize("wl", WORKLOADS)
def test_committed_counter_summaries(wl):
    traffic, source = bench._traffic(wl)
    assert traffic and traffic > 0 and "profiles/traffic_" in source
    mc = bench._mfma_counters(wl)
    assert mc is not None and mc["workload"] == wl
    assert 0.0 <= mc["mfma_busy_pct"] <= 100.0 and mc["mfma_flops_per_step"] > 0
    assert os.path.exists(os.path.join(ROOT, mc["source"])), mc["source"]


def test_missing_summaries_read_as_none():
    assert bench._traffic("no-such-workload") == (None, None)
    assert bench._mfma_counters("no-such-workload") is None
