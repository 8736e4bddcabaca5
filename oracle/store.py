"""KV-pool stores as the reference computes them (CPU, in place). TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

FP8 caches are handled as uint8 byte tensors: CPU indexing has no fp8 kernels (the reference does the same,
ops/attention/swa_fused.py:84-86)."""

from __future__ import annotations

import torch
from torch import Tensor

from . import fp8

ROPE_BYTES = 128     # models/glm52/kernels/decode/attention/mla/kv_row_layout.py:38
LATENT_BYTES = 512   # kv_row_layout.py:41
ROW_BYTES = 640      # kv_row_layout.py:44


def redirect_slots(slots: Tensor, num_slots: int) -> Tensor:
    """A slot < 0 or >= the pool goes to slot 0, SGLang's reserved page (ops/attention/attention_decode.py:290-291;
    models/deepseek_v2/model.py:67-69)."""
    s = slots.to(torch.int64).reshape(-1)
    return torch.where((s < 0) | (s >= num_slots), torch.zeros_like(s), s)


def kv_store_mha(k: Tensor, v: Tensor, slots: Tensor, k_cache: Tensor, v_cache: Tensor, k_scale=None,
                 v_scale=None, scales_multiply: bool = False) -> None:
    """Write k, v [T, G, d] (bf16) into caches [blocks, G, page, d] at (slot // page, head, slot % page).

    bf16 cache: a copy (ops/attention/attention_decode_paged.py:174-176, index_copy_ of the row).
    uint8 (FP8) cache: quantize with the per-head scales [G], then index_put_ (attention_decode.py:288-300). The
    quantize is qkv.py:69-70's divide-and-clamp by dequantization scales, or, with ``scales_multiply``, the GPT-OSS
    decode write by multipliers, e4m3fn(bf16(k * k_scale)) (attention_decode.py:259-260)."""
    nb, G, P, d = k_cache.shape
    T = k.shape[0]
    s = redirect_slots(slots, nb * P)
    index = ((s // P).repeat_interleave(G), torch.arange(G).repeat(T), (s % P).repeat_interleave(G))
    if k_cache.dtype == torch.uint8:
        ks = torch.as_tensor(k_scale, dtype=torch.float32).reshape(1, G, 1)
        vs = torch.as_tensor(v_scale, dtype=torch.float32).reshape(1, G, 1)
        quant = fp8.quantize_mul if scales_multiply else fp8.quantize
        kq = quant(k.reshape(T, G, d), ks)
        vq = quant(v.reshape(T, G, d), vs)
        k_cache.index_put_(index, kq.reshape(T * G, d))
        v_cache.index_put_(index, vq.reshape(T * G, d))
    else:
        k_cache.index_put_(index, k.reshape(T * G, d).to(k_cache.dtype))
        v_cache.index_put_(index, v.reshape(T * G, d).to(v_cache.dtype))


def kv_store_mla(rows: Tensor, slots: Tensor, cache: Tensor, row_scale: Tensor | None = None) -> None:
    """Write compact rows [T, 576] into ``cache`` [slots, 576] at ``slots`` (models/deepseek_v2/model.py:64-70,
    ``flat[slots] = rows``, out-of-pool slots to slot 0). uint8 (FP8) cache: each row gets its own scale
    s_t = absmax(row_t) / 448 (1 for a zero row) in ``row_scale``; this per-token scale is an extension with no
    reference counterpart."""
    flat = cache.reshape(-1, rows.shape[-1])  # a view: the writes land in cache
    s = redirect_slots(slots, flat.shape[0])
    if flat.dtype == torch.uint8:
        sc = fp8.absmax_scale(rows, dims=-1)  # [T]
        q = fp8.quantize(rows, sc[:, None])
        flat[s] = q
        row_scale.reshape(-1)[s] = sc
    else:
        flat[s] = rows.to(flat.dtype)


def latent_byte_offset(c: int) -> int:
    """Byte of latent dim c in the 640-byte row (kv_row_layout.py:62-84): c = 256a + 128b + p -> 128 + 256a + 2p + b."""
    a, rem = divmod(c, 256)
    b, p = divmod(rem, 128)
    return ROPE_BYTES + 256 * a + 2 * p + b


def latent_byte_map(c_dim: int = 512) -> Tensor:
    """Byte offset of each latent dim, as an index tensor (kv_row_layout / _latent_byte_map,
    mla_decode_attention_torch.py:231-233)."""
    return torch.tensor([latent_byte_offset(c) for c in range(c_dim)], dtype=torch.int64)


def pack_kv_rows(rows: Tensor, kv_scale: float) -> Tensor:
    """[n, 640] uint8 rows of logical bf16 rows [n, 576] in [k_pe 64 | latent 512] order: bf16(k_pe / kv_scale) at
    bytes [0, 128), then e4m3fn(clamp(latent / kv_scale)) at the permuted latent bytes
    (mla_decode_attention_torch.py:204-221; ml_dtypes' float32 -> bfloat16 / float8_e4m3fn casts are the IEEE/OCP
    round-to-nearest-even ones that torch's casts also implement, which tests/test_oracle_fp8.py pins)."""
    n = rows.shape[0]
    vals = rows.float()
    out = torch.zeros(n, ROW_BYTES, dtype=torch.uint8)
    rope = (vals[:, :64] / kv_scale).to(torch.bfloat16)
    out[:, :ROPE_BYTES] = rope.view(torch.uint8).reshape(n, 128)
    out[:, latent_byte_map()] = fp8.quantize(vals[:, 64:], kv_scale)
    return out


def unpack_kv_row(rows: Tensor, kv_scale: float) -> Tensor:
    """[n, 576] float32 values of packed rows [n, 640]: [k_pe 64 | latent 512] (mla_decode_attention_torch.py:224-228)."""
    n = rows.shape[0]
    rope = rows[:, :ROPE_BYTES].contiguous().view(torch.bfloat16).float() * kv_scale
    lat = rows[:, latent_byte_map()].contiguous().view(torch.float8_e4m3fn).float() * kv_scale
    return torch.cat([rope.reshape(n, 64), lat.reshape(n, 512)], dim=1)


def kv_store_dsa(rows: Tensor, slots: Tensor, cache: Tensor, kv_scale: float) -> None:
    """Pack and scatter (in place) rows [T, 576] to flat cache rows; a slot < 0 or past the cache is skipped
    (_scatter, mla_decode_attention_torch.py:193-201)."""
    flat = cache.reshape(-1, ROW_BYTES)
    packed = pack_kv_rows(rows, kv_scale)
    s = slots.reshape(-1).to(torch.int64)
    for i in range(s.numel()):
        if 0 <= int(s[i]) < flat.shape[0]:
            flat[int(s[i])] = packed[i]
