"""Parity over seeded random shapes beyond the configs: GQA (head dims, groups, pages, windows, sinks, FP8 and bf16),
absorbed MLA (head counts, pages, FP8 and bf16 rows) and DSA (pages, index counts, short rows), each against the
oracle with the pools bit-exact after the step. The shapes are drawn once from fixed seeds, so every run checks the
same cases."""

import random

import pytest
import torch

from sglang_neuron_amd import workloads
from tests.conftest import announce
from tests._harness import (assert_close_attn, cache_bytes, dsa_gpu_pool, dsa_gpu_step, dsa_oracle, gqa_gpu_decode,
                            gqa_gpu_pool, gqa_oracle, mla_gpu_decode, mla_gpu_pool, mla_oracle)

pytestmark = pytest.mark.gpu


def _gqa_shape(seed: int) -> dict:
    r = random.Random(seed)
    G = r.choice([1, 2, 4, 8])
    group = r.choice([g for g in (1, 2, 4, 8, 16) if G * g <= 64])
    lo = r.randint(1, 2000)
    return {"B": r.randint(1, 9), "H": G * group, "G": G, "d": r.choice([64, 128]), "P": r.choice([16, 32, 64, 128]),
            "fp8": r.random() < 0.6, "lens": (lo, lo + r.randint(0, 3000)),
            "window": r.choice([0, 0, r.randint(16, 700)]), "sinks": r.random() < 0.4}


def _mla_shape(seed: int) -> dict:
    r = random.Random(seed)
    lo = r.randint(1, 3000)
    return {"B": r.randint(1, 12), "H": r.choice([8, 16, 20, 32]), "P": r.choice([16, 64, 128]),
            "lens": (lo, lo + r.randint(0, 5000))}


def _dsa_shape(seed: int) -> dict:
    r = random.Random(seed)
    P = r.choice([16, 64, 128])
    per = r.choice([1024, 4096, 8192])
    k = r.choice([64, 256, 512, 1024, 2048])
    return {"B": r.randint(1, 8), "P": P, "pool_positions": per, "n_indices": k,
            "recent": min(r.choice([8, 64, 128]), k),  # the recent window is part of the index list
            "short_rows": tuple(r.randint(2, per) for _ in range(r.randint(0, 2)))}


GQA_SEEDS = list(range(9100, 9112))
MLA_SEEDS = list(range(9200, 9208))
DSA_SEEDS = list(range(9300, 9306))


@pytest.mark.parametrize("seed", GQA_SEEDS)
def test_gqa_random_shape(seed):
    over = _gqa_shape(seed)
    case = workloads.gqa_case(2, overrides=over)
    announce(f"gqa random {seed}: {over}")
    want, kc_o, vc_o, ks_o, vs_o = gqa_oracle(case)
    kc, vc, ks, vs = gqa_gpu_pool(case)
    out = gqa_gpu_decode(case, kc, vc, ks, vs)
    torch.cuda.synchronize()
    assert_close_attn(out, want, f"gqa {seed}")
    assert torch.equal(cache_bytes(kc), cache_bytes(kc_o)), "K pool differs"
    assert torch.equal(cache_bytes(vc), cache_bytes(vc_o)), "V pool differs"


@pytest.mark.parametrize("seed", MLA_SEEDS)
def test_mla_random_shape(seed):
    over = _mla_shape(seed)
    bf16 = seed % 2 == 1
    case = workloads.mla_case(overrides=over)
    announce(f"mla random {seed}: {over} bf16={bf16}")
    want, cache_o, scale_o = mla_oracle(case, bf16=bf16)
    cache, scale = mla_gpu_pool(case, bf16=bf16)
    out = mla_gpu_decode(case, cache, scale)
    torch.cuda.synchronize()
    assert_close_attn(out, want, f"mla {seed}")
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"
    if not bf16:
        assert torch.equal(scale.cpu(), scale_o), "row scales differ"


@pytest.mark.parametrize("seed", DSA_SEEDS)
def test_dsa_random_shape(seed):
    over = _dsa_shape(seed)
    case = workloads.dsa_case(overrides=over)
    announce(f"dsa random {seed}: {over}")
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache)
    torch.cuda.synchronize()
    assert_close_attn(ctx, want_ctx, f"dsa {seed}")
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4), (lse.cpu() - want_lse).abs().max()
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"
