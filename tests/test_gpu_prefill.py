"""Segmented prefill attention over the FP8 or bf16 pool (ops.prefill_attention, the reference's segmented_attention) against
the CPU oracle (oracle/attention.segmented_prefill) on the same pool bytes: within the attention bar."""

from __future__ import annotations

import random

import pytest
import torch

from conftest import announce
from _harness import assert_close_attn
from oracle import attention as oatt
from sglang_neuron_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, H, G, d, P, priors, lens, spare_pages=5, bf16=False):
    """A pool holding every request's prior and chunk (stored by ops.kv_store_mha with per-head absmax scales), its
    table, the chunk queries and their row offsets."""
    g = torch.Generator().manual_seed(seed)
    R = len(priors)
    spans = [p + s for p, s in zip(priors, lens)]
    pages = [-(-x // P) for x in spans]
    nb = sum(pages) + spare_pages + 1
    width = max(pages) + 2
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = torch.full((R, width), -1, dtype=torch.int32)
    used = 0
    for r, n in enumerate(pages):
        table[r, :n] = perm[used:used + n].to(torch.int32)
        used += n
    k_tok = [torch.randn(x, G, d, generator=g).to(torch.bfloat16) for x in spans]
    v_tok = [torch.randn(x, G, d, generator=g).to(torch.bfloat16) for x in spans]
    k_all, v_all = torch.cat(k_tok), torch.cat(v_tok)
    ks = (k_all.float().abs().amax(dim=(0, 2)) / 448.0).clamp(min=1e-6)
    vs = (v_all.float().abs().amax(dim=(0, 2)) / 448.0).clamp(min=1e-6)
    slots = torch.cat([table[r, torch.arange(x) // P].to(torch.int64) * P + torch.arange(x) % P
                       for r, x in enumerate(spans)])
    kc = torch.zeros(nb, G, P, d, dtype=torch.bfloat16 if bf16 else torch.float8_e4m3fn, device=DEV)
    vc = torch.zeros_like(kc)
    if bf16:
        ks = vs = None
        ops.kv_store_mha(k_all.to(DEV), v_all.to(DEV), slots.to(DEV), kc, vc)
    else:
        ops.kv_store_mha(k_all.to(DEV), v_all.to(DEV), slots.to(DEV), kc, vc, ks.to(DEV), vs.to(DEV))
    T = sum(lens)
    q = torch.randn(T, H, d, generator=g).to(torch.bfloat16)
    q_start = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    return q, kc, vc, ks, vs, table, q_start, torch.tensor(priors, dtype=torch.int32)


CASES = [
    ("qwen3-8b-chunks", 1, dict(H=32, G=8, d=128, P=16, priors=(0, 100, 1000), lens=(64, 200, 37)), 0, False),
    ("gpt-oss-swa-sinks", 2, dict(H=8, G=1, d=64, P=16, priors=(300, 0), lens=(150, 129)), 128, True),
    ("group3-page64", 3, dict(H=12, G=4, d=64, P=64, priors=(70, 5), lens=(33, 90)), 0, True),
    ("long-prior", 4, dict(H=8, G=2, d=128, P=16, priors=(40000,), lens=(8,)), 0, False),
    ("window-1000-page32", 5, dict(H=16, G=4, d=128, P=32, priors=(5000,), lens=(300,)), 1000, False),
    ("mha-d128", 6, dict(H=4, G=4, d=128, P=16, priors=(17, 250), lens=(140, 3)), 0, False),
    ("empty-request", 7, dict(H=8, G=2, d=64, P=16, priors=(40, 9, 0), lens=(20, 0, 33)), 0, False),
    ("bf16-qwen3-0.6b", 8, dict(H=16, G=8, d=128, P=16, priors=(0, 300, 77), lens=(128, 45, 200), bf16=True), 0, False),
    ("bf16-swa-sinks-d64", 10, dict(H=8, G=2, d=64, P=32, priors=(500, 3), lens=(70, 130), bf16=True), 96, True),
    ("bf16-long-prior", 11, dict(H=4, G=1, d=128, P=16, priors=(34000,), lens=(20,), bf16=True), 0, False),
    ("fp8-long-window-page64", 13, dict(H=16, G=4, d=128, P=64, priors=(70000, 3000), lens=(100, 70)), 40000, True),
    # pages that are multiples of 16 but not powers of two (the tile's page lookups divide)
    ("fp8-page48-window", 14, dict(H=16, G=4, d=128, P=48, priors=(3000, 7), lens=(90, 60)), 500, False),
    ("bf16-page48-sinks", 15, dict(H=8, G=2, d=64, P=48, priors=(100,), lens=(70,), bf16=True), 0, True),
]


@pytest.mark.parametrize("name,seed,cfg,window,sinks", CASES, ids=[c[0] for c in CASES])
def test_prefill_attention_matches_oracle(name, seed, cfg, window, sinks):
    announce(f"prefill {name}: {cfg} window={window} sinks={sinks}")
    q, kc, vc, ks, vs, table, q_start, priors = _case(seed, **cfg)
    H, d = cfg["H"], cfg["d"]
    sk = torch.randn(H, generator=torch.Generator().manual_seed(seed + 50)) if sinks else None
    scale = d ** -0.5
    bf16 = cfg.get("bf16", False)
    out = ops.prefill_attention(q.to(DEV), kc, vc, table.to(DEV), q_start.to(DEV), priors.to(DEV),
                                max_q_len=max(cfg["lens"]) + 7, sm_scale=scale,
                                k_scale=None if bf16 else ks.to(DEV), v_scale=None if bf16 else vs.to(DEV),
                                sinks=None if sk is None else sk.to(DEV), window=window)
    torch.cuda.synchronize()
    kh, vh = (kc.cpu(), vc.cpu()) if bf16 else (kc.cpu().view(torch.uint8), vc.cpu().view(torch.uint8))
    want = oatt.segmented_prefill(q, kh, vh, table, q_start, priors, sm_scale=scale, k_scale=ks, v_scale=vs, sinks=sk,
                                  window=window)
    assert_close_attn(out.cpu(), want, name)


def _random_shape(seed: int):
    r = random.Random(seed)
    G = r.choice([1, 2, 4, 8])
    group = r.choice([g for g in (1, 2, 4, 8, 16) if G * g <= 64])
    R = r.randint(1, 3)
    cfg = dict(H=G * group, G=G, d=r.choice([64, 128]), P=r.choice([16, 32, 48, 64, 128]),
               priors=tuple(r.randint(0, 3000) for _ in range(R)), lens=tuple(r.randint(1, 200) for _ in range(R)),
               bf16=r.random() < 0.35)
    return cfg, r.choice([0, 0, r.randint(16, 1500)]), r.random() < 0.4


RANDOM_SEEDS = list(range(9400, 9410))


@pytest.mark.parametrize("seed", RANDOM_SEEDS)
def test_prefill_random_shape(seed):
    """Seeded random shapes (groups, head dims, pages including non-powers of two, requests, windows, sinks, FP8 and
    bf16 pools), drawn once from fixed seeds, against the oracle."""
    cfg, window, sinks = _random_shape(seed)
    test_prefill_attention_matches_oracle(f"random-{seed}", seed, cfg, window, sinks)


def test_segmented_attention_reference_signature():
    """ops.segmented_attention takes the reference's arguments (one request, q [heads, S, d], sink [heads, 1])."""
    announce("prefill segmented_attention signature")
    q, kc, vc, ks, vs, table, q_start, priors = _case(9, H=8, G=2, d=128, P=16, priors=(77,), lens=(50,))
    sk = torch.randn(8, 1)
    out = ops.segmented_attention(q.transpose(0, 1).contiguous().to(DEV), k_cache=kc, v_cache=vc,
                                  block_tables=table.to(DEV), prior_tokens=torch.tensor([[77]]), block_size=16,
                                  kv_segment_size=512, scale=0.1, sliding_window=None, sink=sk.to(DEV),
                                  k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == (8, 50, 128)
    want = oatt.segmented_prefill(q, kc.cpu().view(torch.uint8), vc.cpu().view(torch.uint8), table, q_start, priors,
                                  sm_scale=0.1, k_scale=ks, v_scale=vs, sinks=sk.reshape(-1))
    assert_close_attn(out.transpose(0, 1).cpu(), want, "segmented_attention")


def test_prefill_rejects_bad_pages_and_missing_scales():
    q = torch.zeros(4, 8, 64, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(3, 2, 16, 64, dtype=torch.float8_e4m3fn, device=DEV)
    args = (q, kc, kc, torch.zeros(1, 2, dtype=torch.int32, device=DEV), torch.tensor([0, 4], dtype=torch.int32,
                                                                                      device=DEV),
            torch.tensor([0], dtype=torch.int32, device=DEV))
    one = torch.ones(2, device=DEV)
    with pytest.raises(ValueError):
        ops.prefill_attention(*args, max_q_len=4, sm_scale=1.0)  # an FP8 pool without its scales
    kc8 = torch.zeros(3, 2, 8, 64, dtype=torch.float8_e4m3fn, device=DEV)
    with pytest.raises(ValueError):
        ops.prefill_attention(q, kc8, kc8, *args[3:], max_q_len=4, sm_scale=1.0, k_scale=one, v_scale=one)
    # more workgroups than the kernel numbers in 32 bits: refused before any launch
    many = 65535
    with pytest.raises(ValueError, match="exceed the grid"):
        ops.prefill_attention(q, kc, kc, torch.zeros(many, 2, dtype=torch.int32, device=DEV),
                              torch.zeros(many + 1, dtype=torch.int32, device=DEV),
                              torch.zeros(many, dtype=torch.int32, device=DEV), max_q_len=2 ** 31 - 1, sm_scale=1.0,
                              k_scale=one, v_scale=one)


def test_prefill_takes_int64_tables_and_checks_host_offsets():
    """An int64 block table, q_start and prior_lens are converted (as the decode wrappers do); with a host copy of
    q_start, offsets that do not run from 0 to T or a chunk past max_q_len are refused before the launch."""
    announce("prefill int64 operands and host offsets")
    q, kc, vc, ks, vs, table, q_start, priors = _case(12, H=8, G=2, d=64, P=16, priors=(30, 5), lens=(40, 25))
    args = dict(max_q_len=40, sm_scale=0.125, k_scale=ks.to(DEV), v_scale=vs.to(DEV))
    out = ops.prefill_attention(q.to(DEV), kc, vc, table.to(torch.int64).to(DEV), q_start.to(torch.int64).to(DEV),
                                priors.to(torch.int64).to(DEV), host_q_start=q_start, **args)
    torch.cuda.synchronize()
    want = oatt.segmented_prefill(q, kc.cpu().view(torch.uint8), vc.cpu().view(torch.uint8), table, q_start, priors,
                                  sm_scale=0.125, k_scale=ks, v_scale=vs)
    assert_close_attn(out.cpu(), want, "int64 operands")
    dev_args = (q.to(DEV), kc, vc, table.to(DEV), q_start.to(DEV), priors.to(DEV))
    with pytest.raises(ValueError, match="max_q_len"):
        ops.prefill_attention(*dev_args, host_q_start=q_start, **{**args, "max_q_len": 39})
    with pytest.raises(ValueError, match="from 0 to T"):
        ops.prefill_attention(*dev_args, host_q_start=q_start - 1, **args)
