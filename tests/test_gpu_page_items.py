"""Page items on the GPU (ops.pack_page_items / unpack_page_items / copy_page_items, through the C ABI) against the
oracle (oracle/page_items.py) on the pools' own regions: bit-exact. Then a transfer between two pools followed by a
decode on each: the same output."""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from oracle import page_items as opi
from sglang_neuron_amd import ops
from sglang_neuron_amd.mem_cache.memory_pool import NeuronMHATokenToKVPool, NeuronMLATokenToKVPool

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP8 = torch.float8_e4m3fn


def _fill(t: torch.Tensor, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    b = t.view(torch.uint8)
    b.copy_(torch.randint(0, 256, b.shape, dtype=torch.uint8, generator=g))


def _mha_pool(seed: int, layers=3, size=16 * 40, P=16, H=8, d=128, dtype=FP8) -> NeuronMHATokenToKVPool:
    pool = NeuronMHATokenToKVPool(size, P, dtype, H, d, layers, DEV)
    for i, t in enumerate(pool.k_buffer + pool.v_buffer):
        _fill(t, seed * 100 + i)
    return pool


def _host_regions(pool_bufs):
    return [t.contiguous().view(torch.uint8).reshape(-1).cpu() for t in pool_bufs]


def test_pack_matches_oracle_on_an_mha_pool():
    announce("page items pack, MHA FP8 pool")
    pool = _mha_pool(1)
    infos = pool.get_contiguous_buf_infos()
    pages = torch.tensor([3, 0, 17, 40, 41, -1, 25], dtype=torch.int32)  # 41 and -1 are outside: zeros
    wire = ops.pack_page_items(infos, pages.to(DEV))
    torch.cuda.synchronize()
    want = opi.pack(_host_regions(pool.k_buffer + pool.v_buffer), infos[2], pages.tolist())
    assert wire.numel() == ops.page_items_wire_bytes(infos, pages.numel()) == want.numel()
    assert torch.equal(wire.cpu(), want)


def test_unpack_matches_oracle_on_a_bf16_pool():
    announce("page items unpack, MHA bf16 pool")
    pool = _mha_pool(2, dtype=torch.bfloat16, H=2, d=64)
    infos = pool.get_contiguous_buf_infos()
    pages = torch.tensor([5, 2, 39, 44, 11], dtype=torch.int32)  # 44 is outside: skipped
    n = ops.page_items_wire_bytes(infos, pages.numel())
    wire = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=torch.Generator().manual_seed(3))
    regions = _host_regions(pool.k_buffer + pool.v_buffer)
    opi.unpack(wire, regions, infos[2], pages.tolist())
    ops.unpack_page_items(wire.to(DEV), infos, pages.to(DEV))
    torch.cuda.synchronize()
    for got, want in zip(_host_regions(pool.k_buffer + pool.v_buffer), regions):
        assert torch.equal(got, want)


def test_pack_over_more_regions_than_one_launch_holds():
    """130 regions of mixed item sizes: two launches of 65; the wire offsets run across them."""
    announce("page items pack, 130 regions")
    g = torch.Generator().manual_seed(4)
    item_lens = [16 * (1 + (r % 5)) for r in range(130)]
    bufs = [torch.randint(0, 256, (il * (6 + r % 3),), dtype=torch.uint8, generator=g) for r, il in enumerate(item_lens)]
    dev_bufs = [b.to(DEV) for b in bufs]
    infos = ([b.data_ptr() for b in dev_bufs], [b.numel() for b in dev_bufs], item_lens)
    pages = torch.tensor([1, 7, 0, 5, 6], dtype=torch.int32)  # 6 and 7 are outside some regions
    wire = ops.pack_page_items(infos, pages.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(wire.cpu(), opi.pack(bufs, item_lens, pages.tolist()))
    back = [torch.zeros_like(b) for b in dev_bufs]
    ops.unpack_page_items(wire, ([b.data_ptr() for b in back], [b.numel() for b in back], item_lens), pages.to(DEV))
    torch.cuda.synchronize()
    want = [torch.zeros_like(b) for b in bufs]
    opi.unpack(wire.cpu(), want, item_lens, pages.tolist())
    assert all(torch.equal(a.cpu(), b) for a, b in zip(back, want))


def test_copy_between_mla_pools_with_their_scales():
    """A transfer of an MLA pool moves the row pages and this build's per-slot row scales (get_scale_buf_infos)."""
    announce("page items copy, MLA pools")
    P = 16
    src = NeuronMLATokenToKVPool(P * 20, P, FP8, 512, 64, 2, DEV)
    dst = NeuronMLATokenToKVPool(P * 24, P, FP8, 512, 64, 2, DEV)
    for i, t in enumerate(src.kv_buffer + dst.kv_buffer):
        _fill(t, 50 + i)
    for i, t in enumerate(src.row_scale + dst.row_scale):
        t.copy_(torch.rand(t.shape, generator=torch.Generator().manual_seed(60 + i)).to(DEV))
    sp = torch.tensor([4, 1, 19, 22, 8], dtype=torch.int32)  # source 22 is outside (21 pages): skipped
    dp = torch.tensor([10, 24, 3, 5, 0], dtype=torch.int32)
    for infos_of in (lambda p: p.get_contiguous_buf_infos(), lambda p: p.get_scale_buf_infos()):
        s_inf, d_inf = infos_of(src), infos_of(dst)
        ptr_to_t = {t.data_ptr(): t for t in src.kv_buffer + src.row_scale + dst.kv_buffer + dst.row_scale}
        host_src = [ptr_to_t[p].contiguous().view(torch.uint8).reshape(-1).cpu() for p in s_inf[0]]
        host_dst = [ptr_to_t[p].contiguous().view(torch.uint8).reshape(-1).cpu() for p in d_inf[0]]
        opi.copy(host_src, host_dst, s_inf[2], sp.tolist(), dp.tolist())
        ops.copy_page_items(s_inf, d_inf, sp.to(DEV), dp.to(DEV))
        torch.cuda.synchronize()
        for p, want in zip(d_inf[0], host_dst):
            assert torch.equal(ptr_to_t[p].contiguous().view(torch.uint8).reshape(-1).cpu(), want)


def test_copy_into_replicated_pages():
    """Destination pages twice the source item (a replicated DCP page): blocks addressed in source items."""
    announce("page items copy, replicated blocks")
    g = torch.Generator().manual_seed(7)
    il = 4096
    src = torch.randint(0, 256, (il * 6,), dtype=torch.uint8, generator=g).to(DEV)
    dst = torch.zeros(il * 2 * 5, dtype=torch.uint8, device=DEV)
    sp, dp = torch.tensor([0, 5, 2], dtype=torch.int32), torch.tensor([9, 0, 4], dtype=torch.int32)
    ops.copy_page_items(([src.data_ptr()], [src.numel()], [il]), ([dst.data_ptr()], [dst.numel()], [2 * il]),
                        sp.to(DEV), dp.to(DEV))
    want = torch.zeros(il * 10, dtype=torch.uint8)
    opi.copy([src.cpu()], [want], [il], sp.tolist(), dp.tolist())
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), want)


def test_transfer_then_decode_matches():
    """A request's pages moved from a 'prefill' pool to other pages of a 'decode' pool (every layer's K and V): a GQA
    decode over the destination table gives exactly the source's output."""
    announce("page items transfer then decode")
    P, H, G, d, L = 16, 16, 8, 128, 300
    src, dst = _mha_pool(8, layers=2, size=P * 30, P=P, H=G, d=d), _mha_pool(9, layers=2, size=P * 40, P=P, H=G, d=d)
    for i, t in enumerate(src.k_buffer + src.v_buffer):  # finite e4m3fn bytes (|x| <= 16), random signs
        g = torch.Generator().manual_seed(200 + i)
        b = torch.randint(0, 0x58, t.shape, dtype=torch.uint8, generator=g)
        t.view(torch.uint8).copy_(b | (torch.randint(0, 2, t.shape, dtype=torch.uint8, generator=g) << 7))
    n = -(-L // P)
    sp = torch.randperm(30, generator=torch.Generator().manual_seed(10))[:n].to(torch.int32) + 1
    dp = torch.randperm(40, generator=torch.Generator().manual_seed(11))[:n].to(torch.int32) + 1
    ops.copy_page_items(src.get_contiguous_buf_infos(), dst.get_contiguous_buf_infos(), sp.to(DEV), dp.to(DEV))
    g = torch.Generator().manual_seed(12)
    q = torch.randn(1, H, d, generator=g).to(torch.bfloat16).to(DEV)
    kn = torch.randn(1, G, d, generator=g).to(torch.bfloat16).to(DEV)
    vn = torch.randn(1, G, d, generator=g).to(torch.bfloat16).to(DEV)
    lens = torch.tensor([L], dtype=torch.int64, device=DEV)
    one = torch.ones(G, device=DEV)
    for layer in range(2):
        outs = []
        for pool, pages in ((src, sp), (dst, dp)):
            kc, vc = pool.get_kv_buffer(layer)
            outs.append(ops.paged_decode_gqa(q, kc, vc, pages.reshape(1, -1).to(DEV), lens, kn, vn, sm_scale=d ** -0.5,
                                             k_scale=one, v_scale=one))
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1])


def test_page_items_reject_bad_regions():
    buf = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    pages = torch.zeros(2, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):  # an item of 24 bytes is not whole 16-byte vectors
        ops.pack_page_items(([buf.data_ptr()], [4096], [24]), pages)
    with pytest.raises(ValueError):  # a wire buffer too small
        ops.pack_page_items(([buf.data_ptr()], [4096], [1024]), pages, wire=torch.zeros(1024, dtype=torch.uint8,
                                                                                          device=DEV))
