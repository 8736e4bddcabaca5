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


def test_mfma_counters_match_the_issued_instructions():
    """The committed counter passes read exactly the MFMA work the kernels issue by construction. cfg3 (FP8 rows): per
    16-key tile, and once per row for the own row (a one-key tile), 8 scaled FP8 16x16x128 MFMAs for the latent QK
    (the query's two e4m3 parts over 4 blocks), 2 bf16 16x16x32 for the rope and 32 bf16 16x16x16 for PV. cfg2: per
    32-key tile and KV head, 16 bf16 16x16x32 (8 QK steps over two half-tiles, 8 PV d-tiles)."""
    import torch

    from sglang_neuron_amd import workloads

    spec = workloads.MLA_CONFIG
    lo, hi = spec["lens"]
    lens = torch.randint(lo, hi + 1, (spec["B"],), generator=workloads.gen(3))
    tiles = int(((lens - 1 + 15) // 16).sum()) + spec["B"]
    mc = bench._mfma_counters("cfg3")
    assert mc["mfma_flops_per_step"] == tiles * (2 * 16 * 16 * 32 * 2 + 32 * 16 * 16 * 16 * 2)
    assert mc["mfma_f8_flops_per_step"] == tiles * 8 * 16 * 16 * 128 * 2
    g2 = workloads.GQA_CONFIGS[2]
    tiles2 = g2["B"] * -(-(4096 - 1) // 32) * g2["G"]
    assert bench._mfma_counters("cfg2")["mfma_flops_per_step"] == tiles2 * 16 * 16 * 16 * 32 * 2
