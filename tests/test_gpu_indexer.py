"""The DSA indexer on the GPU (ops.index_key_store, ops.indexer_scores, ops.topk_positions) against the oracle
(oracle/indexer.py): the key store bit-exact; scores within one bf16 rounding of the fp32 reference (the sum order
differs) and dead keys exactly -1e30; the top-k exact: the k largest values, ties at the threshold taken at the
lowest positions."""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from oracle import indexer as oix
from sglang_neuron_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pool(seed, B, width, P, spare=4):
    g = torch.Generator().manual_seed(seed)
    pages = -(-width // P)
    nb = B * pages + spare + 1
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = perm[:B * pages].reshape(B, pages).to(torch.int32)
    keys = torch.randn(nb * P, 128, generator=g).to(torch.bfloat16) * 1.5
    cache = oix.pack_index_keys(keys).reshape(nb, P, 128)
    return g, table, cache


def test_index_key_store_bit_exact():
    announce("indexer key store")
    g = torch.Generator().manual_seed(1)
    nb, P = 12, 64
    keys = (torch.randn(300, 128, generator=g) * 200).to(torch.bfloat16)  # past +-448 too
    keys[0, :4] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.0])
    slots = torch.randperm(nb * P, generator=g)[:300].to(torch.int64)
    slots[5], slots[9] = -1, nb * P + 3  # skipped
    cache = torch.full((nb, P, 128), 0x11, dtype=torch.uint8)
    want = cache.clone()
    oix.index_key_store(keys, slots, want)
    got = cache.to(DEV)
    ops.index_key_store(keys.to(DEV), slots.to(DEV), got)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


SCORES = [("h64-p64", 2, 64, 64, (5000, 3333, 1), 5000), ("h32-p16", 3, 32, 16, (700, 1000), 1000),
          ("h16-ragged-width", 4, 16, 64, (100, 37, 0), 300), ("h128", 5, 128, 64, (2000,), 2048)]


@pytest.mark.parametrize("name,seed,H,P,limits,width", SCORES, ids=[s[0] for s in SCORES])
def test_indexer_scores_match_oracle(name, seed, H, P, limits, width):
    B = len(limits)
    announce(f"indexer scores {name}: B={B} H={H} P={P} width={width}")
    g, table, cache = _pool(seed, B, width, P)
    table[0, 1] = -1  # an invalid page: dead keys
    q = torch.randn(B, H, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(B, H, generator=g) * H ** -0.5
    lim = torch.tensor(limits, dtype=torch.int32)
    got = ops.indexer_scores(q.to(DEV), w.to(DEV), cache.to(DEV), table.to(DEV), lim.to(DEV), width)
    torch.cuda.synchronize()
    want = oix.indexer_scores(q, w, cache, table, lim, width).float()
    got = got.cpu().float()
    dead = want <= -5e29
    assert torch.equal(got[dead], want[dead]), "dead keys must score -1e30"
    err = (got[~dead] - want[~dead]).abs()
    bound = want[~dead].abs() * 2.0 ** -7 + 2e-4  # one bf16 rounding (and fp32 sum order under cancellation)
    assert bool((err <= bound).all()), f"{name}: max err {float(err.max())}"


def _deterministic_topk(row: torch.Tensor, k: int) -> set:
    """The selection with ties taken at the lowest positions (sort by value desc, then position), dead keys as -1."""
    r = row.float().tolist()
    order = sorted(range(len(r)), key=lambda e: (-r[e], e))[:k]
    return {e if r[e] > -5e29 else -1 for e in order}


TOPK = [("ties", 6, 3, 3000, 300), ("k2048-of-8192", 7, 2, 8192, 2048), ("k-all", 8, 2, 700, 700),
        ("dead-tail", 9, 2, 1500, 1200), ("multi-chunk", 12, 2, 20000, 2048), ("odd-width", 13, 2, 9001, 1000),
        ("row-in-registers-max", 14, 1, 131072, 2048), ("streamed-row", 15, 1, 140001, 2048)]


@pytest.mark.parametrize("name,seed,B,N,k", TOPK, ids=[t[0] for t in TOPK])
def test_topk_positions_exact(name, seed, B, N, k):
    announce(f"topk {name}: B={B} N={N} k={k}")
    g = torch.Generator().manual_seed(seed)
    s = (torch.randint(-300, 300, (B, N), generator=g).float() / 16).to(torch.bfloat16)  # heavy ties
    if name == "dead-tail":
        s[:, 1000:] = -1e30
    got = ops.topk_positions(s.to(DEV), k)
    torch.cuda.synchronize()
    got = got.cpu()
    _, vals = oix.topk_positions(s, k)
    for b in range(B):
        live = got[b] >= 0
        assert len(set(got[b][live].tolist())) == int(live.sum()), "duplicate positions"
        # the selected values are exactly the k largest
        dead_v = torch.tensor(-1e30).to(torch.bfloat16).float()  # what a dead key scores in bf16
        sel = torch.cat([s[b, got[b][live].long()].float(), dead_v.repeat(int((~live).sum()))])
        assert torch.equal(torch.sort(sel, descending=True).values, torch.sort(vals[b], descending=True).values)
        # and, ties taken at the lowest positions, exactly the deterministic selection
        assert set(got[b].tolist()) == _deterministic_topk(s[b], k)


def test_scores_then_topk_select_every_clear_winner():
    """GPU scores then GPU top-k: every key whose oracle score clears the oracle's k-th value by more than two bf16
    roundings is selected (the scores may differ by one rounding, so the threshold's neighbourhood may differ)."""
    announce("indexer scores + topk")
    B, H, P, width, k = 2, 64, 64, 6000, 512
    g, table, cache = _pool(11, B, width, P)
    q = torch.randn(B, H, 128, generator=g).to(torch.bfloat16)
    w = torch.rand(B, H, generator=g) * H ** -0.5
    lim = torch.tensor([6000, 4100], dtype=torch.int32)
    sc = ops.indexer_scores(q.to(DEV), w.to(DEV), cache.to(DEV), table.to(DEV), lim.to(DEV), width)
    pos = ops.topk_positions(sc, k).cpu()
    want = oix.indexer_scores(q, w, cache, table, lim, width).float()
    for b in range(B):
        kth = torch.topk(want[b], k).values[-1]
        clear = torch.nonzero(want[b] > kth * (1 + 2 * 2.0 ** -7) + 1e-6).flatten().tolist()
        assert set(clear) <= set(pos[b].tolist())
