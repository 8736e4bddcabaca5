"""KV-store parity: the HIP store kernels against the oracle, bit-exact (BASELINE.json's bar for the store)."""

import pytest
import torch

from oracle import fp8 as ofp8
from oracle import store as ost
from sglang_neuron_amd import ops
from tests.conftest import announce
from tests._harness import cache_bytes

pytestmark = pytest.mark.gpu
ALL_BF16 = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def test_fp8_conversion_instruction_exact():
    announce("diag fp8->bf16 on all 256 bytes")
    b = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = ops.diag_fp8_to_bf16(b.cuda()).cpu().view(torch.bfloat16).float()
    want = b.view(torch.float8_e4m3fn).float()
    finite = torch.isfinite(want)
    assert torch.equal(got[finite], want[finite])
    assert bool(torch.isnan(got[~finite]).all())


@pytest.mark.parametrize("scales", [(1.0, 1.0, 1.0, 1.0), (2 ** -6, 0.5, 1 / 448, 0.0123),
                                    (0.0173, 3.3e-3, 0.771, 1.7e-4), (0.02931, 5.5, 1 / 3, 6.1e-5)])
def test_mha_store_every_bf16_pattern(scales):
    announce(f"kv_store_mha all bf16 patterns scales={scales}")
    G, d, P = 4, 128, 16
    T = (1 << 16) // (G * d)
    k = ALL_BF16.reshape(T, G, d)
    v = ALL_BF16.flip(0).reshape(T, G, d)
    nb = T // P + 3
    g = torch.Generator().manual_seed(5)
    slots = torch.randperm((nb - 1) * P, generator=g)[:T] + P  # distinct, never page 0
    ks = torch.tensor(scales, dtype=torch.float32)
    vs = ks.flip(0).contiguous()
    kc = torch.zeros(nb, G, P, d, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ost.kv_store_mha(k, v, slots, kc, vc, ks, vs)
    kg = torch.zeros(nb, G, P, d, dtype=torch.float8_e4m3fn, device="cuda")
    vg = torch.zeros_like(kg)
    ops.kv_store_mha(k.cuda(), v.cuda(), slots.cuda(), kg, vg, ks.cuda(), vs.cuda())
    assert torch.equal(cache_bytes(kg), kc)
    assert torch.equal(cache_bytes(vg), vc)


@pytest.mark.parametrize("ckpt", [(0.0123, 3.0 / 448.0, 0.02931, 2 ** -6), (1 / 448, 4.67 / 448, 0.5, 7.5)])
def test_mha_store_multiplier_mode_every_bf16_pattern(ckpt):
    """The GPT-OSS decode write (SNA_DTYPE_FP8_E4M3FN_MUL): e4m3fn(bf16(x * m)) with m the loader's inverted bf16
    scales, every bf16 pattern (NaN included: both write 0x7F) against the oracle, bit for bit."""
    announce(f"kv_store_mha multiplier mode all bf16 patterns ckpt={ckpt}")
    G, d, P = 4, 128, 16
    T = (1 << 16) // (G * d)
    k = ALL_BF16.reshape(T, G, d)
    v = ALL_BF16.flip(0).reshape(T, G, d)
    nb = T // P + 3
    g = torch.Generator().manual_seed(15)
    slots = torch.randperm((nb - 1) * P, generator=g)[:T] + P
    km = ofp8.inverted_scale(torch.tensor(ckpt, dtype=torch.float32))
    vm = km.flip(0).contiguous()
    kc = torch.zeros(nb, G, P, d, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ost.kv_store_mha(k, v, slots, kc, vc, km, vm, scales_multiply=True)
    kg = torch.zeros(nb, G, P, d, dtype=torch.float8_e4m3fn, device="cuda")
    vg = torch.zeros_like(kg)
    ops.kv_store_mha(k.cuda(), v.cuda(), slots.cuda(), kg, vg, km.cuda(), vm.cuda(), scales_multiply=True)
    assert torch.equal(cache_bytes(kg), kc)
    assert torch.equal(cache_bytes(vg), vc)
    # and the divide with the same heads' dequantization scales writes other bytes somewhere (the modes differ)
    kd = torch.zeros_like(kg)
    ops.kv_store_mha(k.cuda(), v.cuda(), slots.cuda(), kd, torch.zeros_like(kg),
                     torch.tensor(ckpt, dtype=torch.float32).cuda(), torch.tensor(ckpt, dtype=torch.float32).cuda())
    assert not torch.equal(cache_bytes(kd), kc)


def test_mha_store_bf16_and_redirect():
    announce("kv_store_mha bf16 + out-of-pool slot")
    G, d, P, nb = 2, 64, 16, 5
    g = torch.Generator().manual_seed(6)
    k = torch.randn(3, G, d, generator=g).to(torch.bfloat16)
    v = torch.randn(3, G, d, generator=g).to(torch.bfloat16)
    slots = torch.tensor([17, 40, nb * P + 3])  # the last one is past the pool -> slot 0
    kc = torch.zeros(nb, G, P, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    ost.kv_store_mha(k, v, slots, kc, vc)
    kg, vg = torch.zeros_like(kc).cuda(), torch.zeros_like(vc).cuda()
    ops.kv_store_mha(k.cuda(), v.cuda(), slots.cuda(), kg, vg)
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    assert torch.equal(kc[0, :, 0], k[2])  # redirected to slot 0: page 0, offset 0


def test_absmax_scale_exact():
    announce("kv_absmax_scale")
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(1000, 8, 128, generator=g) * torch.linspace(0.1, 3, 8)[None, :, None]).to(torch.bfloat16)
    x[:, 5] = 0
    got = ops.kv_absmax_scale(x.cuda()).cpu()
    want = ofp8.absmax_scale(x, dims=(0, 2))
    assert torch.equal(got, want)


@pytest.mark.parametrize("n", [1, 37, 300])
def test_mla_store_per_token(n):
    announce(f"kv_store_mla n={n}")
    g = torch.Generator().manual_seed(8 + n)
    rows = torch.randn(n, 576, generator=g) * torch.exp2(torch.randint(-8, 8, (n, 1), generator=g).float())
    rows = rows.to(torch.bfloat16)
    if n > 2:
        rows[1] = 0
    nslots = 64 * (n // 64 + 3)
    slots = torch.randperm(nslots - 64, generator=g)[:n] + 64
    cache = torch.zeros(nslots, 576, dtype=torch.uint8)
    scale = torch.zeros(nslots, dtype=torch.float32)
    ost.kv_store_mla(rows, slots, cache, scale)
    cg = torch.zeros(nslots, 576, dtype=torch.uint8, device="cuda")
    sg = torch.zeros(nslots, dtype=torch.float32, device="cuda")
    ops.kv_store_mla(rows.cuda(), slots.cuda(), cg, sg)
    assert torch.equal(cg.cpu(), cache)
    assert torch.equal(sg.cpu(), scale)


def test_mla_store_every_bf16_pattern():
    announce("kv_store_mla all bf16 patterns")
    # 65536 patterns over rows of 576 (the tail row padded with ones)
    n = -(-(1 << 16) // 576)
    flat = torch.ones(n * 576, dtype=torch.bfloat16)
    flat[: 1 << 16] = ALL_BF16
    rows = flat.reshape(n, 576)
    # NaN and Inf patterns become 1 here so that every row keeps a finite scale (an infinite element makes the row's
    # scale infinite and every byte zero); the MHA sweep covers the quantizer on them
    bad = ~torch.isfinite(rows.float())
    rows = torch.where(bad, torch.ones_like(rows), rows)
    slots = torch.arange(n) + 64
    cache = torch.zeros(n + 128, 576, dtype=torch.uint8)
    scale = torch.zeros(n + 128, dtype=torch.float32)
    ost.kv_store_mla(rows, slots, cache, scale)
    cg, sg = cache.clone().cuda() * 0, scale.clone().cuda() * 0
    ops.kv_store_mla(rows.cuda(), slots.cuda(), cg, sg)
    assert torch.equal(sg.cpu(), scale)
    assert torch.equal(cg.cpu(), cache)


@pytest.mark.parametrize("kv_scale", [2.0 ** -6, 1.0, 0.0173])
def test_dsa_pack_and_scatter(kv_scale):
    announce(f"kv_store_dsa kv_scale={kv_scale}")
    g = torch.Generator().manual_seed(11)
    n = 200
    rows = torch.randn(n, 576, generator=g).to(torch.bfloat16)
    nrows = 64 * 8
    slots = torch.randperm(nrows, generator=g)[:n]
    slots[3] = -1        # skipped
    slots[4] = nrows + 9  # skipped
    cache = torch.randint(0, 255, (nrows, 640), generator=g, dtype=torch.int32).to(torch.uint8)
    cg = cache.clone().cuda()
    ost.kv_store_dsa(rows, slots, cache, kv_scale)
    ops.kv_store_dsa(rows.cuda(), slots.cuda(), cg, kv_scale)
    assert torch.equal(cg.cpu(), cache)
