"""FP8 e4m3fn quantization as the reference computes it, plus an independent restatement from the format's definition
that pins it. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py)."""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

FP8_MAX = 448.0  # utils/dtype_utils.py:6 (_FP8_E4M3FN_MAX)


def quantize(x: Tensor, scale) -> Tensor:
    """uint8 e4m3fn bytes of ``x`` (any float dtype) stored with dequantization scale ``scale`` (broadcastable):
    e4m3fn(clamp(float(x) / scale, -448, 448)).

    Follows the reference's write path: ``(x.float() / scale).clamp(-FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(fp8)`` in
    _torch_qkv (ops/attention/qkv.py:69-70), _quantize (ops/attention/swa_fused.py:73-75), and the latent half of
    pack_kv_rows (models/glm52/kernels/decode/attention/mla/mla_decode_attention_torch.py:219-220). The division is
    fp32 (torch's elementwise true division)."""
    s = torch.as_tensor(scale, dtype=torch.float32)
    return (x.float() / s).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def quantize_mul(x: Tensor, multiplier) -> Tensor:
    """uint8 e4m3fn bytes of ``x`` stored by the GPT-OSS decode write with quantization multiplier ``multiplier``
    (broadcastable; each a bf16 value): e4m3fn(clamp(bf16(bf16(x) * bf16(m)), -448, 448)).

    Follows ``(k * k_scale).clamp(-FP8_CLAMP_MAX, FP8_CLAMP_MAX).to(torch.float8_e4m3fn)`` of _torch_attention_decode
    (ops/attention/attention_decode.py:259-260): k is the bf16 step token and k_scale the bf16 inverted checkpoint scale
    (models/gpt_oss/mxfp4/common.py:481-485), so the product is a bf16 tensor. A NaN element's byte is not fixed by
    that formula: torch's bf16 product writes NaN as 0x7FC0 or as 0xFFFF depending on whether the element falls in its
    vectorized loop, which casts to 0x7F or 0xFF. Here it is 0x7F, bf16's canonical NaN cast (the HIP store's too)."""
    m = torch.as_tensor(multiplier, dtype=torch.float32).to(torch.bfloat16)
    xb = x.to(torch.bfloat16)
    q = (xb * m).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)
    return torch.where(torch.isnan(xb), torch.full_like(q, 0x7F), q)


def dequantize_mul(b: Tensor, multiplier) -> Tensor:
    """float32 values of e4m3fn bytes stored with quantization multiplier m: byte / m (the dequantization the GPT-OSS
    model folds into its softmax scale and output projection, models/gpt_oss/mxfp4/model_decode.py:62-70)."""
    return b.view(torch.float8_e4m3fn).float() / torch.as_tensor(multiplier, dtype=torch.float32)


def inverted_scale(scale) -> Tensor:
    """The GPT-OSS multiplier of a dequantization scale, as the reference's loader computes it: ``1.0 /
    scale.to(bfloat16)``, a bf16 value, here as float32 (models/gpt_oss/mxfp4/common.py:481-485)."""
    return (1.0 / torch.as_tensor(scale, dtype=torch.float32).to(torch.bfloat16)).float()


def dequantize(b: Tensor, scale) -> Tensor:
    """float32 values of e4m3fn bytes times their dequantization scale."""
    return b.view(torch.float8_e4m3fn).float() * torch.as_tensor(scale, dtype=torch.float32)


def absmax_scale(x: Tensor, dims) -> Tensor:
    """Dequantization scale absmax / 448 over ``dims`` (fp32), 1 where the absmax is 0; NaN elements are left out
    of the absmax (an infinite one makes the scale infinite). This is the per-KV-head
    (cfg2) and per-token (cfg3) calibration: an extension with no reference counterpart (the reference's FP8 KV
    scale is one per-tensor checkpoint value, models/gpt_oss/mxfp4/common.py:475-487)."""
    a = x.float().abs()
    m = torch.where(torch.isnan(a), torch.zeros_like(a), a).amax(dim=dims)  # NaN elements do not count
    return torch.where(m > 0, m / FP8_MAX, torch.ones_like(m))


# ---- independent restatement from the OCP definition (the pin of torch's cast) ----

def e4m3fn_values() -> np.ndarray:
    """float64 value of each of the 256 codes (NaN for 0x7F / 0xFF), from the definition: bias 7, 3 mantissa bits,
    subnormals m * 2^-9, no infinities."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 15 and m == 7:
            out[code] = np.nan
        elif e == 0:
            out[code] = s * m * 2.0 ** -9
        else:
            out[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def e4m3fn_rne_spec(x: np.ndarray) -> np.ndarray:
    """uint8 codes of float32 ``x`` by nearest-value search, ties to the even code (mantissa LSB 0). A magnitude past
    the midpoint between 448 and the next binade step (464), and NaN, give the NaN code with the sign of x. This is the
    behaviour of an unsaturated cast, which the reference relies on only behind its clamp."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    vals = e4m3fn_values()
    pos_codes = np.arange(0, 0x7F)  # 0x00..0x7E: the finite non-negative codes, in increasing value
    pos_vals = vals[pos_codes]
    a = np.abs(x)
    idx = np.clip(np.searchsorted(pos_vals, a), 1, len(pos_vals) - 1)
    lo, hi = pos_vals[idx - 1], pos_vals[idx]
    dlo, dhi = a - lo, hi - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((pos_codes[idx] & 1) == 0))
    code = np.where(pick_hi, pos_codes[idx], pos_codes[idx - 1])
    code = np.where(a <= 0.0, 0, code)
    # above the largest finite value: ties at 464 round to 448 (even), anything larger is NaN
    over = a > 464.0
    tie = a == 464.0
    code = np.where(tie, 0x7E, code)
    code = np.where(a > 448.0, np.where(over, 0x7F, 0x7E), code)
    code = np.where(np.isnan(x), 0x7F, code)
    sign = np.signbit(x).astype(np.int64) << 7
    return (code | sign).astype(np.uint8)


def bf16_round_spec(x: np.ndarray) -> np.ndarray:
    """float64 values of float64 ``x`` rounded to bf16's 8 significant bits, ties to even, by the significand (frexp):
    a restatement independent of the binary32 bit layout. Exact for results in bf16's normal range; a magnitude that
    rounds past bf16's largest finite value becomes infinite. (Results below 2^-126 keep 8 bits, as bf16 subnormals do
    not; the e4m3fn cast sends every such value to a signed zero.)"""
    x = np.asarray(x, dtype=np.float64)
    mant, exp = np.frexp(x)
    r = np.ldexp(np.rint(mant * 256.0) / 256.0, exp)
    big = (2.0 - 2.0 ** -7) * 2.0 ** 127
    return np.where(np.isfinite(x) & (np.abs(r) > big), np.copysign(np.inf, x), r)


def bf16_rne_spec(x: np.ndarray) -> np.ndarray:
    """uint16 bf16 codes of float32 ``x``, round to nearest even (NaN -> 0x7FC0), from the binary32 layout."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(np.asarray(x, dtype=np.float32)), np.uint16(0x7FC0), r)
