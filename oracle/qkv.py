"""The QKV writer after the projection, as the reference's torch path computes it (CPU). TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Follows _rms and _torch_qkv_paged (ops/attention/qkv_paged.py:40-68): per-head RMSNorm of Q and K before RoPE (when
gammas are given), rotate-half RoPE ``t * c + cat(-t[d/2:], t[:d/2]) * s`` in the activation dtype, K and V written at
the token slots. The FP8 write is _torch_qkv's divide-and-clamp (ops/attention/qkv.py:69-70, 78-80), the same
quantization as the MHA store."""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from . import store


def sum_of_squares(x32: Tensor) -> Tensor:
    """The fp32 sum of x32^2 over the last dim (a multiple of 8) in one fixed order: each square rounded (pow(2)),
    each run of 8 consecutive squares summed in sequence, then the runs folded in halves (the second half added onto
    the first) until one is left. The reference's mean leaves this order to its backend (torch's CPU reduction, the
    Neuron compiler), where a different order can move a normed value by one bf16 step; this is the order the HIP
    writer's lanes reduce in, so its stores can be compared bit for bit."""
    sq = x32 * x32
    runs = sq.reshape(*sq.shape[:-1], -1, 8)
    acc = runs[..., 0]
    for e in range(1, 8):
        acc = acc + runs[..., e]
    while acc.shape[-1] > 1:
        h = acc.shape[-1] // 2
        acc = acc[..., :h] + acc[..., h:]
    return acc


def recip_sqrt(v: Tensor) -> Tensor:
    """1 / sqrt(v) for float32 v (>= 0), the square root and the reciprocal each rounded to the nearest float32: each
    is computed in float64 (numpy, the hardware's IEEE sqrt and divide) and rounded once to float32, which gives the
    correctly rounded float32 result for both operations (53 >= 2 * 24 + 2 bits). torch's float32 CPU sqrt and
    reciprocal are not correctly rounded on every host (two x86 hosts here disagree by one ulp on a fifth of the
    values), so the oracle does not use them."""
    a = v.detach().cpu().contiguous().numpy().astype(np.float64)
    s = np.sqrt(a).astype(np.float32).astype(np.float64)
    return torch.from_numpy((1.0 / s).astype(np.float32)).to(v.device)


def rms(x: Tensor, gamma: Tensor, eps: float) -> Tensor:
    """_rms (qkv_paged.py:40-42): gamma * (x32 * rsqrt(mean(x32^2) + eps)).to(x.dtype), the mean as the sum of
    squares (sum_of_squares) over d, rsqrt as 1 / sqrt (recip_sqrt: each correctly rounded)."""
    x32 = x.float()
    mean = sum_of_squares(x32) / x32.shape[-1]
    return gamma.reshape(-1) * (x32 * recip_sqrt(mean + eps)).to(x.dtype)


def rope(t: Tensor, c: Tensor, s: Tensor) -> Tensor:
    """rope (qkv_paged.py:61-62): t [T, H, d], c / s [T, 1, d], in t's dtype."""
    d = t.shape[-1]
    return t * c + torch.cat([-t[..., d // 2:], t[..., :d // 2]], dim=-1) * s


def qkv_norm_rope_store(qkv: Tensor, cos: Tensor, sin: Tensor, num_q_heads: int, num_kv_heads: int, d_head: int,
                        k_cache: Tensor, v_cache: Tensor, slots: Tensor, q_norm=None, k_norm=None, eps: float = 1e-6,
                        k_scale=None, v_scale=None) -> Tensor:
    """qkv [T, (q + 2 kv) * d] bf16 (the projection's output), cos / sin [T, d] bf16; the caches [blocks, kv, page, d]
    (bf16, or uint8 holding e4m3fn with per-head scales) are written in place. Returns Q [T, q, d] bf16.
    (qkv_paged.py:52-68 after its `hidden @ weights + bias`.)"""
    T = qkv.shape[0]
    q, k, v = qkv.split([num_q_heads * d_head, num_kv_heads * d_head, num_kv_heads * d_head], dim=-1)
    q, k, v = q.reshape(T, -1, d_head), k.reshape(T, -1, d_head), v.reshape(T, -1, d_head)
    if q_norm is not None:
        q, k = rms(q, q_norm, eps), rms(k, k_norm, eps)
    c, s = cos.reshape(T, 1, d_head), sin.reshape(T, 1, d_head)
    q, k = rope(q, c, s), rope(k, c, s)
    store.kv_store_mha(k.contiguous(), v.contiguous(), slots, k_cache, v_cache, k_scale, v_scale)
    return q.contiguous()
