"""Pins of the indexer oracle (oracle/indexer.py): the key store's cast, the score by explicit float64 loops, and the
top-k selection against a full sort."""

from __future__ import annotations

import math

import torch

from oracle import fp8 as ofp8
from oracle import indexer as oix


def test_pack_index_keys_is_the_clamped_e4m3fn_cast():
    x = torch.tensor([0.0, 1.1, -1.1, 500.0, -1e6, 448.0, 2.0 ** -9, 3.3])
    got = oix.pack_index_keys(x)
    want = ofp8.quantize(x.clamp(-448, 448), torch.tensor(1.0))
    assert torch.equal(got, want)
    assert got[1].item() == ofp8.quantize(torch.tensor([1.125]), torch.tensor(1.0))[0].item()  # 1.1 -> 1.125
    assert torch.equal(got[3:5].view(torch.float8_e4m3fn).float(), torch.tensor([448.0, -448.0]))


def test_indexer_scores_brute_force():
    g = torch.Generator().manual_seed(3)
    B, H, d, P, nb = 2, 3, 8, 4, 9
    q = torch.randn(B, H, d, generator=g).to(torch.bfloat16)
    w = torch.randn(B, H, generator=g)
    cache = oix.pack_index_keys(torch.randn(nb, P, d, generator=g) * 2)
    table = torch.tensor([[3, 5, -1, 2], [7, 1, 4, 8]], dtype=torch.int32)
    limits = torch.tensor([10, 14])
    width = 16
    got = oix.indexer_scores(q, w, cache, table, limits, width)
    keys = cache.view(torch.float8_e4m3fn).float()
    for b in range(B):
        for e in range(width):
            page = int(table[b, e // P])
            if page < 0 or e >= int(limits[b]):
                assert got[b, e].float().item() == -1e30 or math.isclose(got[b, e].float().item(), -1e30, rel_tol=1e-2)
                continue
            tot = 0.0
            for h in range(H):
                raw = sum(float(q[b, h, i]) * float(keys[page, e % P, i]) for i in range(d)) / math.sqrt(d)
                tot += float(w[b, h]) * max(raw, 0.0)
            want = torch.tensor(tot).to(torch.bfloat16).float().item()
            assert abs(got[b, e].float().item() - want) <= abs(want) * 2 ** -7 + 1e-6, (b, e)


def test_topk_positions_against_a_full_sort():
    g = torch.Generator().manual_seed(5)
    s = (torch.randint(-20, 20, (3, 300), generator=g).float() / 4).to(torch.bfloat16)  # many ties
    s[1, 250:] = -1e30  # dead keys
    for k in (1, 17, 64, 280):
        pos, vals = oix.topk_positions(s, k)
        for b in range(3):
            srt = torch.sort(s[b].float(), descending=True).values[:k]
            assert torch.equal(torch.sort(vals[b], descending=True).values, srt)
            live = vals[b] > -5e29
            assert torch.equal(s[b, pos[b][live].long()].float(), vals[b][live])
            assert bool((pos[b][~live] == -1).all())
