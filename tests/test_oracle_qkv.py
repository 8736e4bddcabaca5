"""Pins of the QKV writer oracle (oracle/qkv.py) by closed forms and a float64 restatement that does not share its
rounding steps."""

import math

import pytest
import torch

from oracle import qkv as oqkv
from oracle import store as ost


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def test_rope_at_angle_zero_is_the_identity():
    t = _bf16((5, 3, 64), 1)
    c, s = torch.ones(5, 1, 64, dtype=torch.bfloat16), torch.zeros(5, 1, 64, dtype=torch.bfloat16)
    assert torch.equal(oqkv.rope(t, c, s), t)


def test_rope_at_a_quarter_turn_is_rotate_half():
    t = _bf16((4, 2, 128), 2)
    c, s = torch.zeros(4, 1, 128, dtype=torch.bfloat16), torch.ones(4, 1, 128, dtype=torch.bfloat16)
    want = torch.cat([-t[..., 64:], t[..., :64]], dim=-1)
    assert torch.equal(oqkv.rope(t, c, s), want)


def test_rope_is_a_complex_rotation_within_three_bf16_roundings():
    T, H, d = 7, 4, 128
    t = _bf16((T, H, d), 3)
    pos = torch.arange(T, dtype=torch.float64)[:, None] * 37.0
    inv = 1.0 / (10000.0 ** (torch.arange(d // 2, dtype=torch.float64) * 2 / d))
    ang = torch.cat([pos * inv, pos * inv], dim=-1)
    c, s = ang.cos().to(torch.bfloat16)[:, None], ang.sin().to(torch.bfloat16)[:, None]
    out = oqkv.rope(t, c, s).double()
    z = torch.complex(t[..., :d // 2].double(), t[..., d // 2:].double())
    w = torch.complex(c[..., :d // 2].double(), s[..., :d // 2].double())
    r = z * w
    want = torch.cat([r.real, r.imag], dim=-1)
    mag = (t[..., :d // 2].double().abs() * c[..., :d // 2].double().abs()
           + t[..., d // 2:].double().abs() * s[..., :d // 2].double().abs()).repeat(1, 1, 2)
    assert bool(((out - want).abs() <= 3 * 2.0 ** -8 * (mag + out.abs()) + 1e-30).all())


def test_rms_of_a_constant_magnitude_head_has_its_closed_form():
    """|x_i| = a for every i: x * rsqrt(a^2 + eps) with unit gamma, so eps shows when a^2 is near it."""
    d, eps = 128, 1e-6
    for a in (2.0 ** -10, 0.5, 3.0):
        sign = torch.where(torch.arange(d) % 3 == 0, -1.0, 1.0)
        x = (sign * a).to(torch.bfloat16).reshape(1, 1, d)
        got = oqkv.rms(x, torch.ones(d, dtype=torch.bfloat16), eps).double()
        want = sign.double() * a / math.sqrt(a * a + eps)
        assert bool(((got.reshape(-1) - want).abs() <= 2.0 ** -8 * want.abs()).all()), a


def test_writer_stores_the_rotated_k_and_the_raw_v():
    """The cache writes are the pinned MHA store of (rotated K, V); Q is returned rotated."""
    T, Hq, Hkv, d, P, nb = 6, 4, 2, 64, 16, 4
    qkv = _bf16((T, (Hq + 2 * Hkv) * d), 4)
    g = torch.Generator().manual_seed(5)
    ang = torch.rand(T, d // 2, generator=g, dtype=torch.float64) * 6.28
    cos = torch.cat([ang.cos(), ang.cos()], -1).to(torch.bfloat16)
    sin = torch.cat([ang.sin(), ang.sin()], -1).to(torch.bfloat16)
    slots = torch.tensor([17, 18, 40, 63, -1, 5000])
    for fp8 in (False, True):
        dt = torch.uint8 if fp8 else torch.bfloat16
        kc, vc = torch.zeros(nb, Hkv, P, d, dtype=dt), torch.zeros(nb, Hkv, P, d, dtype=dt)
        ks = vs = torch.tensor([0.02, 0.03]) if fp8 else None
        q = oqkv.qkv_norm_rope_store(qkv, cos, sin, Hq, Hkv, d, kc, vc, slots, k_scale=ks, v_scale=vs)
        c, s = cos.reshape(T, 1, d), sin.reshape(T, 1, d)
        qs, k, v = qkv.split([Hq * d, Hkv * d, Hkv * d], -1)
        assert torch.equal(q, oqkv.rope(qs.reshape(T, Hq, d), c, s))
        kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
        ost.kv_store_mha(oqkv.rope(k.reshape(T, Hkv, d), c, s).contiguous(), v.reshape(T, Hkv, d).contiguous(), slots,
                         kc2, vc2, ks, vs)
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
        # out-of-pool slots (-1, 5000) went to slot 0, the reserved page
        assert bool((kc[0, :, 0] != 0).any())


def test_sum_of_squares_order_is_a_full_sum():
    """The oracle's fixed-order fp32 sum of squares against a float64 sum of the same squares: within the bound any
    summation order of d fp32 terms keeps (a dropped, doubled or misindexed term is off by far more); on small
    integers, where every partial sum is exact in fp32, equal to torch's own reduction."""
    g = torch.Generator().manual_seed(5)
    for d in (64, 128):
        x = torch.randn(7, 3, d, generator=g).to(torch.bfloat16).float()
        got = oqkv.sum_of_squares(x)[..., 0].double()
        want = (x.double() ** 2).sum(-1)
        assert bool(((got - want).abs() <= d * 2.0 ** -23 * want).all()), d
        ints = torch.randint(-40, 41, (5, 2, d), generator=g).float()
        assert torch.equal(oqkv.sum_of_squares(ints)[..., 0], ints.pow(2).sum(-1))
        # a term placed by hand: only element j is non-zero
        for j in (0, 7, 8, d // 2, d - 1):
            e = torch.zeros(1, d)
            e[0, j] = 3.0
            assert float(oqkv.sum_of_squares(e)) == 9.0, j


def test_recip_sqrt_rounds_each_step_to_the_nearest_float32():
    """recip_sqrt's square root is the float32 nearest the exact root and its reciprocal the float32 nearest the exact
    1 / root: checked with exact rationals (Fraction) against both float32 neighbours, on random positive values
    across exponents and on exact squares."""
    from fractions import Fraction

    import numpy as np

    g = torch.Generator().manual_seed(11)
    v = torch.exp(torch.randn(400, generator=g) * 4.0)
    v = torch.cat([v, torch.tensor([1.0, 4.0, 0.25, 2.0 ** -20, 3.0, 1e-6])])
    got = oqkv.recip_sqrt(v)
    for vi, ri in zip(v.tolist(), got.tolist()):
        a = Fraction(vi)
        r = np.float32(ri)
        # a candidate root (a float32 near sqrt(a)), shown to be the nearest: a lies on its side of the squared
        # midpoint towards each float32 neighbour
        root = np.float32(np.sqrt(np.float64(vi)))
        for cand in (np.nextafter(root, np.float32(0)), np.nextafter(root, np.float32(np.inf))):
            mid = (Fraction(float(cand)) + Fraction(float(root))) / 2
            assert (a - mid * mid) * (Fraction(float(root)) - mid) >= 0, (vi, float(root), float(cand))
        # r is the float32 nearest 1 / root
        rr = 1 / Fraction(float(root))
        for cand in (np.nextafter(r, np.float32(0)), np.nextafter(r, np.float32(np.inf))):
            assert abs(Fraction(float(r)) - rr) <= abs(Fraction(float(cand)) - rr), (vi, ri)


def _literal_rms(x, gamma, eps):
    """The reference's _rms exactly as written (ops/attention/qkv_paged.py:40-42), in torch's own order."""
    x32 = x.float()
    return gamma.reshape(-1) * (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)


@pytest.mark.parametrize("d,scale", [(128, 1.0), (64, 3.0), (128, 1e-3)])
def test_rms_matches_the_reference_formula_within_a_bf16_step(d, scale):
    """oracle.rms fixes the sum order and rounds sqrt and 1 / sqrt once each; against the reference's literal
    torch.rsqrt(x32.pow(2).mean(-1) + eps) the normed value may move by at most one bf16 step (before gamma's product,
    which both round the same way), and most values are equal."""
    g = torch.Generator().manual_seed(d)
    x = (torch.randn(400, 8, d, generator=g) * scale).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    ones = torch.ones(d, dtype=torch.bfloat16)
    got, want = oqkv.rms(x, ones, 1e-6), _literal_rms(x, ones, 1e-6)
    step = torch.exp2(torch.floor(torch.log2(want.float().abs().clamp(min=1e-30))) - 7)  # one bf16 ulp at |want|
    assert bool(((got.float() - want.float()).abs() <= step).all())
    assert float((got != want).float().mean()) < 0.05
    with_gamma = oqkv.rms(x, gamma, 1e-6)
    assert bool(((with_gamma.float() - _literal_rms(x, gamma, 1e-6).float()).abs()
                 <= 2 * step * gamma.float().abs().max()).all())
