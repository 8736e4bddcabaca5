"""Pins of the page-item oracle (oracle/page_items.py): the item addressing against the pools' own tensor indexing,
pack by explicit byte loops, and the invariants tying pack, unpack and copy together."""

from __future__ import annotations

import torch

from oracle import page_items as opi


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8).reshape(-1)


def test_item_is_the_pools_page():
    """ptr + p * item_len (memory_pool.py:193-202) is page p of the pool tensors: [nb, H, P, d] K/V buffers (item
    H * P * d * itemsize) and the MLA row buffer [slots, 1, 576] (item P * 576)."""
    g = torch.Generator().manual_seed(0)
    kv = torch.randint(0, 256, (5, 3, 16, 64), dtype=torch.uint8, generator=g)
    il = 3 * 16 * 64
    for p in range(5):
        assert torch.equal(opi.item(_bytes(kv), il, p), kv[p].reshape(-1))
    kvb = torch.randn(4, 2, 16, 8, generator=g).to(torch.bfloat16)  # a bf16 pool: item in bytes
    for p in range(4):
        assert torch.equal(opi.item(_bytes(kvb), 2 * 16 * 8 * 2, p), _bytes(kvb[p]))
    P = 16
    rows = torch.randint(0, 256, (3 * P, 1, 576), dtype=torch.uint8, generator=g)
    for p in range(3):
        assert torch.equal(opi.item(_bytes(rows), P * 576, p), rows[p * P:(p + 1) * P].reshape(-1))


def test_pack_by_byte_loops():
    g = torch.Generator().manual_seed(1)
    item_lens = [16, 32, 48]
    regions = [torch.randint(0, 256, (il * n,), dtype=torch.uint8, generator=g) for il, n in zip(item_lens, (6, 4, 3))]
    pages = [2, 0, 5, 1, -1]  # 5 is outside regions 1 and 2, -1 outside all
    want = []
    for reg, il in zip(regions, item_lens):
        n = reg.numel() // il
        for p in pages:
            for b in range(il):
                want.append(int(reg[p * il + b]) if 0 <= p < n else 0)
    assert opi.pack(regions, item_lens, pages).tolist() == want


def test_round_trips_and_copy_agree():
    g = torch.Generator().manual_seed(2)
    item_lens = [32, 64]
    src = [torch.randint(0, 256, (il * 7,), dtype=torch.uint8, generator=g) for il in item_lens]
    sp, dp = [3, 6, 0, 9], [1, 4, 5, 2]  # source page 9 is outside: skipped by copy and unpack
    # pack then unpack at the same pages restores those items and nothing else
    back = [torch.zeros_like(r) for r in src]
    opi.unpack(opi.pack(src, item_lens, sp), back, item_lens, sp)
    for r, il in zip(range(2), item_lens):
        for p in range(7):
            want = src[r][p * il:(p + 1) * il] if p in sp else torch.zeros(il, dtype=torch.uint8)
            assert torch.equal(back[r][p * il:(p + 1) * il], want)
    # copy == unpack(pack(src, sp), dst, dp) where every source page is inside
    dst_a = [torch.full_like(r, 7) for r in src]
    dst_b = [torch.full_like(r, 7) for r in src]
    opi.copy(src, dst_a, item_lens, sp[:3], dp[:3])
    opi.unpack(opi.pack(src, item_lens, sp[:3]), dst_b, item_lens, dp[:3])
    assert all(torch.equal(a, b) for a, b in zip(dst_a, dst_b))
    # an outside source page leaves its destination item alone
    dst_c = [torch.full_like(r, 7) for r in src]
    opi.copy(src, dst_c, item_lens, [9], [2])
    assert all(bool((d == 7).all()) for d in dst_c)


def test_copy_into_a_replicated_page_addresses_source_items():
    """A destination page of k source items (a replicated DCP page): block j of page p is source-item index
    p * k + j (dcp_stripes.py:146-161)."""
    g = torch.Generator().manual_seed(3)
    il, k = 48, 2
    src = [torch.randint(0, 256, (il * 4,), dtype=torch.uint8, generator=g)]
    dst = [torch.zeros(il * k * 3, dtype=torch.uint8)]
    opi.copy(src, dst, [il], [0, 1, 3], [2 * k + 1, 0 * k + 0, 1 * k + 1])
    page = lambda p: dst[0][p * il * k:(p + 1) * il * k]  # noqa: E731
    assert torch.equal(page(2)[il:], src[0][0:il])
    assert torch.equal(page(0)[:il], src[0][il:2 * il])
    assert torch.equal(page(1)[il:], src[0][3 * il:4 * il])
    assert int(page(2)[:il].sum()) == 0 and int(page(0)[il:].sum()) == 0
