"""Pins the oracle's FP8 quantizer (torch's cast behind the reference's divide-and-clamp) against an independent
restatement from the e4m3fn definition, over every bf16 bit pattern, and against the reference's known answer."""

import numpy as np
import pytest
import torch

from oracle import fp8

ALL_BF16 = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
SCALES = [1.0, 0.5, 2.0 ** -6, 1.0 / 448.0, 3.0 / 448.0, 0.0123, 7.5, 1e-3, 5.0 / 448.0 * 1.0001]


def test_reference_known_answer():
    # models/kimi_k3/kernels/decode/mla_decode_torch.py:89-96: quantize_fp8_e4m3fn([1.1, 500.0]) -> [1.125, 448.]
    q = fp8.quantize(torch.tensor([1.1, 500.0]), 1.0)
    assert fp8.dequantize(q, 1.0).tolist() == [1.125, 448.0]
    assert q.tolist() == [57, 126]


def test_value_table_is_the_format():
    v = fp8.e4m3fn_values()
    assert v[0x7E] == 448.0 and v[0x08] == 2.0 ** -6 and v[0x01] == 2.0 ** -9
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF])
    finite = v[~np.isnan(v)]
    assert len(finite) == 254  # +-0 count twice
    # the bytes decode through torch to the same values
    t = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    assert np.array_equal(np.isnan(t), np.isnan(v))
    assert np.array_equal(t[~np.isnan(t)], v[~np.isnan(v)])


@pytest.mark.parametrize("scale", SCALES)
def test_quantize_matches_definition_on_every_bf16(scale):
    got = fp8.quantize(ALL_BF16, scale).numpy()
    x = (ALL_BF16.float() / torch.tensor(scale, dtype=torch.float32)).numpy()
    clamped = np.clip(x, -448.0, 448.0)  # numpy's clip keeps NaN
    want = fp8.e4m3fn_rne_spec(clamped)
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]


def test_unclamped_cast_matches_definition():
    # the cast itself (no clamp): RNE, NaN above the 464 midpoint, ties to even
    x = torch.tensor([447.9, 448.0, 455.9, 456.0, 463.9, 464.0, 470.0, 480.0, float("inf"), float("nan"),
                      2 ** -10, 3 * 2 ** -11, 2 ** -9, 1e-9, -2 ** -10, -0.0])
    got = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, fp8.e4m3fn_rne_spec(x.numpy()))


def test_bf16_cast_matches_definition():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1 << 16, generator=g) * torch.exp2(torch.randint(-30, 30, (1 << 16,), generator=g).float())
    got = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, fp8.bf16_rne_spec(x.numpy()))


def test_absmax_scale_rule():
    x = torch.tensor([[0.0, 0.0], [-3.0, 2.0]]).to(torch.bfloat16)
    s = fp8.absmax_scale(x, dims=-1)
    assert s.tolist() == [1.0, float(torch.tensor(3.0) / 448.0)]
    # the largest magnitude lands on +-448 exactly (or its neighbour below when the division rounds down)
    q = fp8.quantize(x[1], s[1])
    assert abs(fp8.dequantize(q, 1.0)[0].item()) in (448.0, 416.0)


def test_dequant_error_bound():
    # |dequant(quant(x)) - x| <= half an e4m3fn ulp at x's binade, times the scale
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, generator=g).to(torch.bfloat16)
    s = fp8.absmax_scale(x, dims=0)
    y = fp8.dequantize(fp8.quantize(x, s), s)
    xf = x.float()
    e = torch.floor(torch.log2((xf / s).abs().clamp(min=2 ** -6)))
    ulp = torch.exp2(e - 3) * s
    assert bool(((y - xf).abs() <= ulp / 2 + 1e-12).all())


# ---- the GPT-OSS decode write: bf16 product with the inverted scale, then the cast ----

# multipliers as the reference's loader makes them from checkpoint scales (1 / bf16(s), rounded to bf16): cfg4-like
# absmax / 448 values, odd ones, and powers of two (whose product needs no rounding)
CKPT_SCALES = [0.0123, 1.0 / 448.0, 3.0 / 448.0, 0.02931, 4.67 / 448.0, 2.0 ** -6, 0.5, 7.5]


def _mul_definition(x_bf16: torch.Tensor, m: float) -> np.ndarray:
    """Bytes by the definitions: the exact float64 product, rounded to bf16's 8 significant bits (ties to even, by
    the significand), clamped to +-448, cast by nearest-value search."""
    p = x_bf16.double().numpy() * float(m)  # exact: two 8-bit significands
    r = fp8.bf16_round_spec(p)
    return fp8.e4m3fn_rne_spec(np.clip(r, -448.0, 448.0).astype(np.float32))


@pytest.mark.parametrize("s", CKPT_SCALES)
def test_quantize_mul_matches_definition_on_every_bf16(s):
    m = fp8.inverted_scale(s)
    got = fp8.quantize_mul(ALL_BF16, m).numpy()
    nan = torch.isnan(ALL_BF16).numpy()
    want = _mul_definition(ALL_BF16, float(m))
    assert np.array_equal(got[~nan], want[~nan]), np.nonzero(got[~nan] != want[~nan])[0][:10]
    assert (got[nan] == 0x7F).all()  # NaN in: the canonical NaN byte


def test_quantize_mul_is_the_reference_formula_on_finite_values():
    # (k * k_scale).clamp(-448, 448).to(e4m3fn) with bf16 k and k_scale (attention_decode.py:259-260)
    g = torch.Generator().manual_seed(4)
    k = (torch.randn(5000, generator=g) * 3).to(torch.bfloat16)
    ks = torch.tensor([[1.0 / 0.0123]]).to(torch.bfloat16)
    want = (k * ks).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1)
    assert torch.equal(fp8.quantize_mul(k, ks.float()).reshape(-1), want)


def test_inverted_scale_is_the_loaders_rule():
    # 1.0 / bf16(s): an IEEE float32 division of bf16 operands, rounded to bf16 (common.py:481-485)
    for s in CKPT_SCALES + [1.0, 3.3e-3, 1e-4]:
        sb = np.float32(torch.tensor(s).to(torch.bfloat16).float().item())
        q32 = np.float32(1.0) / sb
        want = fp8.bf16_rne_spec(np.array([q32]))[0]
        got = fp8.inverted_scale(s).to(torch.bfloat16).view(torch.int16).item() & 0xFFFF
        assert got == int(want), (s, hex(got), hex(int(want)))
    assert float(fp8.inverted_scale(2.0 ** -6)) == 64.0


def test_bf16_round_spec_matches_the_bit_layout_rule():
    # the significand rounding and the binary32 bit rule agree wherever both apply (bf16's normal range)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1 << 16, generator=g, dtype=torch.float64) * torch.exp2(
        torch.randint(-100, 100, (1 << 16,), generator=g).double())
    x32 = x.float().numpy()
    a = fp8.bf16_round_spec(x32.astype(np.float64))
    b = fp8.bf16_rne_spec(x32).view(np.int16).astype(np.int32) << 16
    b = b.astype(np.uint32).view(np.float32).astype(np.float64)
    assert np.array_equal(a, b)


def test_divide_and_multiply_writes_differ_on_cfg4_data():
    """The two FP8 writes are not interchangeable: on N(0,1) tokens with an absmax / 448 scale the GPT-OSS decode
    write (bf16 product with the inverted bf16 scale) and the divide give different bytes for a few percent of the
    elements; with a power-of-two scale they agree."""
    g = torch.Generator().manual_seed(1004)
    x = torch.randn(1 << 16, generator=g).to(torch.bfloat16)
    s = fp8.absmax_scale(x, dims=0)
    div = fp8.quantize(x, s)
    mul = fp8.quantize_mul(x, fp8.inverted_scale(s))
    frac = float((div != mul).double().mean())
    assert 0.005 < frac < 0.1, frac
    p2 = torch.tensor(2.0 ** -6)
    assert torch.equal(fp8.quantize(x, p2), fp8.quantize_mul(x, fp8.inverted_scale(p2)))
