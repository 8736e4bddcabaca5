"""QKV writer parity: the HIP norm + RoPE + store kernel against the oracle (oracle/qkv.py), bit for bit: Q, the K
pool and the V pool, with and without the QK norm (the oracle sums the norm's squares in the writer's order)."""


import pytest
import torch

from oracle import qkv as oqkv
from sglang_neuron_amd import ops
from tests.conftest import announce

pytestmark = pytest.mark.gpu

CASES = [
    # name, T, Hq, Hkv, d, P, fp8, norm
    ("qwen3-8b-fp8-norm", 300, 32, 8, 128, 16, True, True),
    ("qwen3-8b-fp8", 300, 32, 8, 128, 16, True, False),
    ("qwen3-0.6b-bf16-norm", 257, 16, 8, 128, 16, False, True),
    ("gpt-oss-share-bf16", 129, 8, 1, 64, 16, False, False),
    ("gpt-oss-share-fp8-page64", 200, 8, 1, 64, 64, True, False),
    # d 64 with the norm: the lane sums fold through xor shuffles instead of DPP rotations
    ("d64-bf16-norm", 129, 8, 2, 64, 16, False, True),
    ("d64-fp8-norm", 77, 4, 4, 64, 16, True, True),
    # a page size that is not a power of two: the slot's page and offset by division
    ("fp8-page24-norm", 61, 4, 2, 128, 24, True, True),
    ("bf16-page24", 50, 4, 2, 64, 24, False, False),
]


def _inputs(T, Hq, Hkv, d, P, fp8, norm, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * d, generator=g) * 2.0).to(torch.bfloat16)
    pos = torch.arange(T, dtype=torch.float64)[:, None] + 1000.0
    inv = 1.0 / (1.0e6 ** (torch.arange(d // 2, dtype=torch.float64) * 2 / d))
    ang = torch.cat([pos * inv, pos * inv], dim=-1)
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    nb = (T + P - 1) // P + 2
    slots = torch.randperm((nb - 1) * P, generator=g)[:T] + P  # distinct slots past the reserved page
    slots[T // 3] = -1                                          # out of pool: slot 0
    qn = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16) if norm else None
    kn = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16) if norm else None
    ks = (0.5 + torch.rand(Hkv, generator=g)) * 0.02 if fp8 else None
    vs = (0.5 + torch.rand(Hkv, generator=g)) * 0.02 if fp8 else None
    return qkv, cos, sin, slots, qn, kn, ks, vs, nb


@pytest.mark.parametrize("name,T,Hq,Hkv,d,P,fp8,norm", CASES, ids=[c[0] for c in CASES])
def test_qkv_writer_matches_oracle(name, T, Hq, Hkv, d, P, fp8, norm):
    announce(f"qkv {name}: T={T} Hq={Hq} Hkv={Hkv} d={d} P={P} fp8={fp8} norm={norm}")
    qkv, cos, sin, slots, qn, kn, ks, vs, nb = _inputs(T, Hq, Hkv, d, P, fp8, norm, 7)
    dt = torch.uint8 if fp8 else torch.bfloat16
    kc_o, vc_o = torch.zeros(nb, Hkv, P, d, dtype=dt), torch.zeros(nb, Hkv, P, d, dtype=dt)
    q_o = oqkv.qkv_norm_rope_store(qkv, cos, sin, Hq, Hkv, d, kc_o, vc_o, slots, qn, kn, 1e-6, ks, vs)
    dev = "cuda"
    gdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    kc = torch.zeros(nb, Hkv, P, d, dtype=gdt, device=dev)
    vc = torch.zeros(nb, Hkv, P, d, dtype=gdt, device=dev)
    q = ops.qkv_norm_rope_store(qkv.to(dev), cos=cos.to(dev), sin=sin.to(dev), num_q_heads=Hq, num_kv_heads=Hkv,
                                d_head=d, k_cache=kc, v_cache=vc, slot_mapping=slots.to(dev),
                                q_norm=None if qn is None else qn.to(dev), k_norm=None if kn is None else kn.to(dev),
                                norm_eps=1e-6, k_scale=None if ks is None else ks.to(dev),
                                v_scale=None if vs is None else vs.to(dev))
    torch.cuda.synchronize()
    kb = kc.cpu().view(torch.uint8) if fp8 else kc.cpu()
    vb = vc.cpu().view(torch.uint8) if fp8 else vc.cpu()
    assert torch.equal(vb, vc_o), "V pool differs"
    # with the QK norm too: the oracle sums the squares in the order the writer's lanes do (oracle.qkv.sum_of_squares)
    assert torch.equal(q.cpu(), q_o), "Q differs"
    assert torch.equal(kb, kc_o), "K pool differs"


@pytest.mark.parametrize("fp8,norm", [(True, True), (True, False), (False, True), (False, False)])
def test_qkv_writer_nan_and_inf_bits(fp8, norm):
    """NaN (both signs, assorted payloads) and infinities in the projection output and the rotation rows: Q and K
    against the oracle with NaN exactly where the oracle has NaN and every other value bit for bit (a NaN's bits are
    not fixed by the reference: torch's float to bf16 conversion writes 0x7FC0 or 0xFFFF depending on its code path,
    and an FP8 byte of a NaN is 0x7F or 0xFF by that NaN's sign); V, copied or quantized from the input, bit for bit
    (a bf16 pool keeps the input's bits, an FP8 byte of a NaN is its sign | 0x7F). Covers the kernel's uniform NaN
    branch (a wave with a NaN takes the exact quantizer, one without the fast one)."""
    announce(f"qkv NaN/inf fp8={fp8} norm={norm}")
    T, Hq, Hkv, d, P = 96, 8, 2, 128, 16
    qkv, cos, sin, slots, qn, kn, ks, vs, nb = _inputs(T, Hq, Hkv, d, P, fp8, norm, 11)
    g = torch.Generator().manual_seed(12)
    i16 = lambda v: v - (1 << 16) if v >= 1 << 15 else v  # noqa: E731  (a bf16 bit pattern as int16)
    bits = qkv.view(torch.int16)
    specials = torch.tensor([i16(v) for v in (0x7FC0, 0xFFC0, 0x7F81, 0xFFFF, 0x7FA5, 0x7F80, 0xFF80)],
                            dtype=torch.int16)
    where = torch.randperm(bits.numel(), generator=g)[:60]  # a few tokens' rows, most rows clean
    bits.view(-1)[where] = specials[torch.arange(60) % len(specials)]
    cos.view(torch.int16)[5, 3] = i16(0x7F80)   # +inf: inf * 0 and inf - inf reach the sums
    sin.view(torch.int16)[9, 70] = i16(0xFF80)
    dt = torch.uint8 if fp8 else torch.bfloat16
    kc_o, vc_o = torch.zeros(nb, Hkv, P, d, dtype=dt), torch.zeros(nb, Hkv, P, d, dtype=dt)
    q_o = oqkv.qkv_norm_rope_store(qkv, cos, sin, Hq, Hkv, d, kc_o, vc_o, slots, qn, kn, 1e-6, ks, vs)
    dev = "cuda"
    gdt = torch.float8_e4m3fn if fp8 else torch.bfloat16
    kc = torch.zeros(nb, Hkv, P, d, dtype=gdt, device=dev)
    vc = torch.zeros(nb, Hkv, P, d, dtype=gdt, device=dev)
    q = ops.qkv_norm_rope_store(qkv.to(dev), cos=cos.to(dev), sin=sin.to(dev), num_q_heads=Hq, num_kv_heads=Hkv,
                                d_head=d, k_cache=kc, v_cache=vc, slot_mapping=slots.to(dev),
                                q_norm=None if qn is None else qn.to(dev), k_norm=None if kn is None else kn.to(dev),
                                norm_eps=1e-6, k_scale=None if ks is None else ks.to(dev),
                                v_scale=None if vs is None else vs.to(dev))
    torch.cuda.synchronize()
    as_bits = lambda t: t.contiguous().view(torch.uint8)  # noqa: E731

    def same_up_to_nan_bits(got, want, what):
        if got.dtype == torch.uint8:  # FP8 bytes: 0x7F / 0xFF are NaN
            gn, wn = (got & 0x7F) == 0x7F, (want & 0x7F) == 0x7F
        else:
            gn, wn = torch.isnan(got.float()), torch.isnan(want.float())
        assert torch.equal(gn, wn), f"{what}: NaN at different places"
        assert torch.equal(as_bits(got[~gn]), as_bits(want[~wn])), f"{what}: non-NaN values differ"

    assert bool(torch.isnan(q_o.float()).any()), "the case must reach NaN outputs"
    same_up_to_nan_bits(q.cpu(), q_o, "Q")
    same_up_to_nan_bits(kc.cpu().view(torch.uint8) if fp8 else kc.cpu(), kc_o, "K pool")
    assert torch.equal(as_bits(vc.cpu()), as_bits(vc_o)), "V pool bits differ"


def test_qkv_writer_norm_within_a_bf16_step_of_the_reference_formula():
    """The writer's normed Q (no RoPE: angle 0) against the reference's literal _rms, gamma * (x32 *
    torch.rsqrt(x32.pow(2).mean(-1) + eps)).to(bf16) (qkv_paged.py:40-42): at most one bf16 step of the normed value
    (times gamma) apart, so the writer cannot drift from the reference's normalisation."""
    announce("qkv norm vs the literal reference formula")
    T, Hq, Hkv, d, P = 200, 8, 2, 128, 16
    g = torch.Generator().manual_seed(31)
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * d, generator=g) * 2.0).to(torch.bfloat16)
    cos, sin = torch.ones(T, d, dtype=torch.bfloat16), torch.zeros(T, d, dtype=torch.bfloat16)
    qn = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kn = torch.ones(d, dtype=torch.bfloat16)
    nb = T // P + 2
    dev = "cuda"
    kc = torch.zeros(nb, Hkv, P, d, dtype=torch.bfloat16, device=dev)
    q = ops.qkv_norm_rope_store(qkv.to(dev), cos=cos.to(dev), sin=sin.to(dev), num_q_heads=Hq, num_kv_heads=Hkv,
                                d_head=d, k_cache=kc, v_cache=torch.zeros_like(kc),
                                slot_mapping=(torch.arange(T) + P).to(dev), q_norm=qn.to(dev), k_norm=kn.to(dev),
                                norm_eps=1e-6).cpu()
    x32 = qkv[:, :Hq * d].reshape(T, Hq, d).float()
    normed = (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    want = qn * normed
    step = torch.exp2(torch.floor(torch.log2(normed.float().abs().clamp(min=1e-30))) - 7) * qn.float().abs()
    assert bool(((q.float() - want.float()).abs() <= 2 * step + 1e-30).all())
    assert float((q != want).float().mean()) < 0.05


def test_qkv_writer_rejects_bad_arguments():
    dev = "cuda"
    kc = torch.zeros(4, 2, 16, 64, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qkv = torch.zeros(3, 8 * 64, dtype=torch.bfloat16, device=dev)
    cs = torch.zeros(3, 64, dtype=torch.bfloat16, device=dev)
    slots = torch.zeros(3, dtype=torch.int64, device=dev)
    with pytest.raises(ValueError):  # one gamma without the other
        ops.qkv_norm_rope_store(qkv, cos=cs, sin=cs, num_q_heads=4, num_kv_heads=2, d_head=64, k_cache=kc,
                                v_cache=vc, slot_mapping=slots, q_norm=torch.ones(64, dtype=torch.bfloat16,
                                                                                   device=dev))
    with pytest.raises(ValueError):  # an FP8 cache without scales
        kf = torch.zeros(4, 2, 16, 64, dtype=torch.float8_e4m3fn, device=dev)
        ops.qkv_norm_rope_store(qkv, cos=cs, sin=cs, num_q_heads=4, num_kv_heads=2, d_head=64, k_cache=kf,
                                v_cache=torch.zeros_like(kf), slot_mapping=slots)
