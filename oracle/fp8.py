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


def bf16_rne_spec(x: np.ndarray) -> np.ndarray:
    """uint16 bf16 codes of float32 ``x``, round to nearest even (NaN -> 0x7FC0), from the binary32 layout."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(np.asarray(x, dtype=np.float32)), np.uint16(0x7FC0), r)
