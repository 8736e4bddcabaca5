"""KV pools in the block layout the HIP decode kernels read, with the reference pools' interface.

Mirrors sglang_neuron/mem_cache/memory_pool.py (NeuronMHATokenToKVPool :45-211, NeuronMLATokenToKVPool :306-428):
same class names, constructor arguments, buffer shapes and bookkeeping calls, so a plugin that registers these
classes as SGLang's pool kinds finds what the reference's callers use. SGLang itself is not importable here, so the
classes stand alone instead of subclassing SGLang's KVCache; the attributes SGLang reads from its own pools are set
by hand.

Differences from the reference, all on the write path the reference leaves to its compiled graphs:

  * ``set_kv_buffer`` (MHA) and ``set_mla_kv_buffer`` / ``set_kv_buffer`` (MLA) are implemented (the reference raises,
    :178-179, :414-418) with the HIP store kernels: FP8 e4m3fn quantization, bit-exact with the reference's
    ``e4m3fn(clamp(x / s, +-448))``, scattered to token slots, out-of-pool slots redirected to the reserved slot 0.
  * FP8 scales are tensors of the pool: per layer and KV head for MHA (``k_scale[layer]``, ``v_scale[layer]`` [G]
    fp32), per token slot for MLA (``row_scale[layer]`` [slots] fp32, set by the store from each row's absmax). An
    MHA layer's scales are dequantization scales s (stores divide: e4m3fn(x / s), qkv.py:69-70), or, set with
    ``inverted=True``, the GPT-OSS model's inverted bf16 scales m (gpt_oss/mxfp4/common.py:481-485), which its decode
    multiplies by (e4m3fn(bf16(x * m)), attention_decode.py:259-260) and its prefill divides by bf16(1 / m)
    (gpt_oss/mxfp4/model_prefill.py:41-43).
  * K stays unpacked ``[blocks, kv_heads, page, head_dim]``: ``fp8_packed_k`` is False (the packed
    ``[.., page/2, d, 2]`` K of :133-137 is a Trainium-kernel layout).

Page 0 is reserved: a pool of ``size`` tokens has ``size // page_size + 1`` blocks (:20-21, :106-107).
"""

from __future__ import annotations

import logging
from typing import List, Optional, Tuple, Union

import torch
from torch import Tensor

from .. import ops

logger = logging.getLogger(__name__)

GB = 1024 ** 3
FP8 = torch.float8_e4m3fn

# SGLang pool keyword arguments naming features these pools do not build. A pool accepts such an argument only when it
# leaves the feature off (absent, None or False); any other value is a ValueError, as the reference pools refuse them
# (mem_cache/memory_pool.py:260-282 for the MHA pool, :432 for the MLA pool). The head-dim arguments must repeat the
# pool's own head dim: K and V pages share it on every layer.
_FEATURES_NOT_BUILT = {
    "mha": ("post_capture_active", "quant_method", "kv_cache_layout", "enable_kv_cache_copy"),
    "mla": ("use_dsa", "override_kv_cache_dim", "dcp_replicated"),
}
_SAME_HEAD_DIM = ("v_head_dim", "swa_head_dim", "swa_v_head_dim")


def _check_pool_kwargs(kind: str, kwargs: dict, head_dim: Optional[int] = None) -> None:
    """Raise ValueError naming every keyword argument of ``kwargs`` that asks ``kind``'s pool for something it does not
    build: a feature switched on, or (with ``head_dim``) a second head dim."""
    asked = [f"{name}={kwargs[name]!r}" for name in _FEATURES_NOT_BUILT[kind]
             if kwargs.get(name) not in (None, False)]
    if head_dim is not None:
        asked += [f"{name}={kwargs[name]!r}" for name in _SAME_HEAD_DIM if kwargs.get(name) not in (None, head_dim)]
    if asked:
        raise ValueError(f"the {kind.upper()} KV pool (one head dim, FP8 or bf16 pages) does not support "
                         f"{', '.join(sorted(asked))}")


def _layer_id(layer) -> int:
    return int(layer if isinstance(layer, int) else getattr(layer, "layer_id"))


def _scale_tensor(scale: Union[float, Tensor], n: int, device) -> Tensor:
    t = torch.as_tensor(scale, dtype=torch.float32, device=device).reshape(-1)
    if t.numel() == 1:
        t = t.expand(n)
    if t.numel() != n:
        raise ValueError(f"a scale of {t.numel()} entries for {n} KV heads")
    return t.contiguous()


class NeuronMHATokenToKVPool:
    """The MHA/GQA pool: per layer K and V ``[num_blocks, head_num, page_size, head_dim]`` in the cache dtype (bf16 or
    float8_e4m3fn), head-major pages (``kv_head_major``), plus the FP8 dequantization scales per layer and KV head.
    Constructor arguments as the reference's (memory_pool.py:56-69)."""

    kv_head_major = True
    kv_cp_size = 1
    kv_cp_rank = 0
    publishes_kv_layer_ids = True

    def __init__(self, size: int, page_size: int, dtype: torch.dtype, head_num: int, head_dim: int, layer_num: int,
                 device: Union[str, torch.device], enable_memory_saver: bool = False,
                 start_layer: Optional[int] = None, end_layer: Optional[int] = None, **kwargs):
        _check_pool_kwargs("mha", kwargs, head_dim)
        if enable_memory_saver:
            raise ValueError("the KV pool does not support enable_memory_saver")
        if size % page_size:
            raise ValueError(f"a pool of {size} tokens is not whole pages of {page_size}")
        if dtype not in (torch.bfloat16, FP8):
            raise ValueError(f"the HIP decode path reads bf16 or float8_e4m3fn caches, not {dtype}")
        self.size = int(size)
        self.page_size = int(page_size)
        self.dtype = dtype
        self.store_dtype = dtype
        self.head_num = int(head_num)
        self.head_dim = int(head_dim)
        self.k_head_dim = self.v_head_dim = self.head_dim
        self.layer_num = int(layer_num)
        self.start_layer = int(start_layer or 0)
        self.end_layer = int(end_layer if end_layer is not None else self.start_layer + self.layer_num - 1)
        self.device = torch.device(device)
        self.block_size = self.page_size
        self.num_blocks = self.size // self.page_size + 1
        self.k_buffer: List[Tensor] = []
        self.v_buffer: List[Tensor] = []
        self.k_scale: List[Tensor] = []
        self.v_scale: List[Tensor] = []
        self.scales_inverted: List[bool] = []  # per layer: the scales are GPT-OSS multipliers m, not divisors s
        self._create_buffers()
        self.mem_usage = self.get_kv_size_bytes() / GB
        logger.info("KV pool: layers=%d blocks=%d page=%d kv_heads=%d head_dim=%d dtype=%s (%.2f GB)", self.layer_num,
                    self.num_blocks, self.page_size, self.head_num, self.head_dim, self.store_dtype, self.mem_usage)

    @property
    def fp8_packed_k(self) -> bool:
        """K is kept unpacked in every dtype."""
        return False

    def _create_buffers(self) -> None:
        _, shape = self.get_kv_buffer_shape()
        for _ in range(self.layer_num):
            self.k_buffer.append(torch.zeros(shape, dtype=self.store_dtype, device=self.device))
            self.v_buffer.append(torch.zeros(shape, dtype=self.store_dtype, device=self.device))
            self.k_scale.append(torch.ones(self.head_num, dtype=torch.float32, device=self.device))
            self.v_scale.append(torch.ones(self.head_num, dtype=torch.float32, device=self.device))
            self.scales_inverted.append(False)

    def _idx(self, layer_id: int) -> int:
        i = layer_id - self.start_layer
        if not 0 <= i < self.layer_num:
            raise IndexError(f"layer {layer_id} is outside this pool's layers [{self.start_layer}, "
                             f"{self.start_layer + self.layer_num})")
        return i

    # access (memory_pool.py:163-176)
    def get_key_buffer(self, layer_id: int) -> Tensor:
        return self.k_buffer[self._idx(layer_id)]

    def get_value_buffer(self, layer_id: int) -> Tensor:
        return self.v_buffer[self._idx(layer_id)]

    def get_kv_buffer(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        return self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

    def get_kv_scales(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """The layer's FP8 scales [head_num] fp32 (K, V): dequantization scales, or the GPT-OSS multipliers when
        ``kv_scales_inverted(layer_id)``."""
        i = self._idx(layer_id)
        return self.k_scale[i], self.v_scale[i]

    def kv_scales_inverted(self, layer_id: int) -> bool:
        """Whether the layer's scales are GPT-OSS multipliers m (a byte is worth byte / m) rather than dequantization
        scales."""
        return self.scales_inverted[self._idx(layer_id)]

    def prefill_kv_scales(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        """The dequantization scales the layer's prefill writers divide by: the layer's scales, or for multipliers m
        ``1 / m`` rounded to bf16, as the reference's GPT-OSS prefill computes them (model_prefill.py:41-43)."""
        i = self._idx(layer_id)
        if not self.scales_inverted[i]:
            return self.k_scale[i], self.v_scale[i]
        return (ops.prefill_write_scale(self.k_scale[i]).to(self.device),
                ops.prefill_write_scale(self.v_scale[i]).to(self.device))

    def get_kv_layer_ids(self) -> List[int]:
        layers = list(range(self.start_layer, self.start_layer + self.layer_num))
        return layers + layers

    # writes
    def set_kv_scales(self, layer_id: int, k_scale: Union[float, Tensor], v_scale: Union[float, Tensor], *,
                      inverted: bool = False) -> None:
        """Set the layer's scales (a float or one per KV head): dequantization scales, or with ``inverted`` the GPT-OSS
        model's inverted scales (its ``attn.k_scale`` / ``attn.v_scale``, bf16 values: 1 / bf16(checkpoint scale),
        gpt_oss/mxfp4/common.py:481-485), which the layer's decode then multiplies by."""
        i = self._idx(layer_id)
        if inverted:
            k_scale = torch.as_tensor(k_scale).detach().float().cpu().to(torch.bfloat16).float()
            v_scale = torch.as_tensor(v_scale).detach().float().cpu().to(torch.bfloat16).float()
        self.k_scale[i] = _scale_tensor(k_scale, self.head_num, self.device)
        self.v_scale[i] = _scale_tensor(v_scale, self.head_num, self.device)
        self.scales_inverted[i] = bool(inverted)

    def calibrate_kv_scales(self, layer_id: int, cache_k: Tensor, cache_v: Tensor,
                            inverted: bool = False) -> Tuple[Tensor, Tensor]:
        """Per-KV-head absmax / 448 scales of bf16 tokens [T, head_num, head_dim] (the HIP absmax kernel), set as the
        layer's scales and returned. With ``inverted`` they stand for a GPT-OSS checkpoint's scales: the layer gets
        the multipliers the reference's loader makes of them (ops.inverted_kv_scale), which are returned."""
        k = cache_k.reshape(-1, self.head_num, self.head_dim)
        v = cache_v.reshape(-1, self.head_num, self.head_dim)
        ks, vs = ops.kv_absmax_scale(k), ops.kv_absmax_scale(v)
        if inverted:
            ks, vs = ops.inverted_kv_scale(ks).to(self.device), ops.inverted_kv_scale(vs).to(self.device)
        self.set_kv_scales(layer_id, ks, vs, inverted=inverted)
        return ks, vs

    def set_kv_buffer(self, layer, loc: Tensor, cache_k: Tensor, cache_v: Tensor,
                      k_scale: Optional[Union[float, Tensor]] = None, v_scale: Optional[Union[float, Tensor]] = None,
                      layer_id_override: Optional[int] = None) -> None:
        """Store tokens [T, head_num, head_dim] (bf16) at slots ``loc`` [T] of layer ``layer`` (a layer id or an object
        with ``layer_id``). SGLang's signature; ``k_scale`` / ``v_scale``, when given, are the dequantization scales
        (the stored value is x / scale) and become the layer's. A layer of GPT-OSS multipliers is written as its
        decode writes (e4m3fn(bf16(x * m)), attention_decode.py:259-260). The reference pool raises here
        (memory_pool.py:178-179)."""
        layer_id = layer_id_override if layer_id_override is not None else _layer_id(layer)
        i = self._idx(layer_id)
        if k_scale is not None or v_scale is not None:
            self.set_kv_scales(layer_id, 1.0 if k_scale is None else k_scale, 1.0 if v_scale is None else v_scale)
        fp8 = self.store_dtype == FP8
        ops.kv_store_mha(cache_k.reshape(-1, self.head_num, self.head_dim),
                         cache_v.reshape(-1, self.head_num, self.head_dim), loc, self.k_buffer[i], self.v_buffer[i],
                         self.k_scale[i] if fp8 else None, self.v_scale[i] if fp8 else None,
                         scales_multiply=fp8 and self.scales_inverted[i])

    def set_kv_buffer_prefill(self, layer, loc: Tensor, cache_k: Tensor, cache_v: Tensor) -> None:
        """Store a prefill chunk's tokens [T, head_num, head_dim] (bf16) at ``loc`` as the reference's prefill writers
        do: divided by the layer's dequantization scales, which for GPT-OSS multipliers m are bf16(1 / m)
        (qkv.py:69-70 with model_prefill.py:41-43). For a layer of dequantization scales this is set_kv_buffer."""
        i = self._idx(_layer_id(layer))
        fp8 = self.store_dtype == FP8
        ks, vs = self.prefill_kv_scales(_layer_id(layer)) if fp8 else (None, None)
        ops.kv_store_mha(cache_k.reshape(-1, self.head_num, self.head_dim),
                         cache_v.reshape(-1, self.head_num, self.head_dim), loc, self.k_buffer[i], self.v_buffer[i],
                         ks, vs)

    # bookkeeping (memory_pool.py:182-202)
    def get_kv_size_bytes(self) -> int:
        per = self.num_blocks * self.head_num * self.page_size * self.head_dim * self.store_dtype.itemsize
        return per * 2 * self.layer_num

    def get_kv_buffer_shape(self):
        """Per-layer K and V buffer shapes (equal: K is unpacked)."""
        shape = torch.Size((self.num_blocks, self.head_num, self.page_size, self.head_dim))
        return shape, shape

    def get_contiguous_buf_infos(self):
        """(ptrs, lens, item_lens): K buffers then V buffers; a page of one layer is item_len bytes at ptr + p *
        item_len."""
        item_len = self.head_num * self.page_size * self.head_dim * self.store_dtype.itemsize
        ptrs = [t.data_ptr() for t in self.k_buffer] + [t.data_ptr() for t in self.v_buffer]
        lens = [t.numel() * t.element_size() for t in self.k_buffer + self.v_buffer]
        return ptrs, lens, [item_len] * (2 * self.layer_num)

    def get_cpu_copy(self, *args, **kwargs):
        raise NotImplementedError("KV host offload is not part of this build")

    def load_cpu_copy(self, *args, **kwargs):
        raise NotImplementedError("KV host offload is not part of this build")


class NeuronMLATokenToKVPool:
    """The absorbed-MLA pool: per layer one compact row per token slot, ``kv_buffer[layer]`` [size + page_size, 1,
    kv_lora_rank + qk_rope_head_dim] in row order [latent | rope] (models/deepseek_v2/model.py:110). bf16 rows as the
    reference's DeepSeek-V2 pool holds them (memory_pool.py:306-351, models/catalog.py:230-231), or FP8 stored as
    uint8 (memory_pool.py:313-315) with one fp32 dequantization scale per slot in ``row_scale[layer]`` (bf16 pools
    have no row scales). Constructor arguments as SGLang's MLATokenToKVPool."""

    publishes_kv_layer_ids = True

    def __init__(self, size: int, page_size: int, dtype: torch.dtype, kv_lora_rank: int, qk_rope_head_dim: int,
                 layer_num: int, device: Union[str, torch.device], enable_memory_saver: bool = False,
                 start_layer: Optional[int] = None, end_layer: Optional[int] = None, **kwargs):
        _check_pool_kwargs("mla", kwargs)
        if enable_memory_saver:
            raise ValueError("the MLA pool does not support enable_memory_saver")
        if dtype not in (FP8, torch.uint8, torch.bfloat16):
            raise ValueError(f"the HIP MLA decode reads bf16 rows or FP8 rows with per-token scales, not {dtype}")
        if kv_lora_rank + qk_rope_head_dim != 576 or qk_rope_head_dim != 64:
            raise ValueError("the HIP MLA decode reads 576-wide rows (kv_lora_rank 512 + rope 64)")
        if page_size % 16:
            raise ValueError(f"the HIP MLA decode reads pages that are whole 16-slot tiles, not {page_size}")
        self.size = int(size)
        self.page_size = int(page_size)
        self.fp8 = dtype != torch.bfloat16
        self.dtype = FP8 if self.fp8 else torch.bfloat16
        self.store_dtype = torch.uint8 if self.fp8 else torch.bfloat16
        self.kv_lora_rank = int(kv_lora_rank)
        self.qk_rope_head_dim = int(qk_rope_head_dim)
        self.kv_cache_dim = self.kv_lora_rank + self.qk_rope_head_dim
        self.layer_num = int(layer_num)
        self.start_layer = int(start_layer or 0)
        self.end_layer = int(end_layer if end_layer is not None else self.start_layer + self.layer_num - 1)
        self.model_layer_ids = list(range(self.start_layer, self.start_layer + self.layer_num))
        self.device = torch.device(device)
        self.kv_buffer: List[Tensor] = [
            torch.zeros((self.size + self.page_size, 1, self.kv_cache_dim), dtype=self.store_dtype, device=self.device)
            for _ in range(self.layer_num)]
        self.row_scale: List[Tensor] = [torch.ones(self.size + self.page_size, dtype=torch.float32, device=self.device)
                                        for _ in range(self.layer_num)] if self.fp8 else []
        self.mem_usage = self.get_kv_size_bytes() / GB

    @property
    def num_blocks(self) -> int:
        """Pages of the pool, the reserved page 0 included (memory_pool.py:353-356)."""
        return self.size // self.page_size + 1

    def _idx(self, layer_id: int) -> int:
        i = layer_id - self.start_layer
        if not 0 <= i < self.layer_num:
            raise IndexError(f"layer {layer_id} is outside this pool's layers")
        return i

    def get_key_buffer(self, layer_id: int) -> Tensor:
        return self.kv_buffer[self._idx(layer_id)]

    def get_value_buffer(self, layer_id: int) -> Tensor:
        """V is the latent part of the same rows (the first kv_lora_rank bytes)."""
        return self.kv_buffer[self._idx(layer_id)][..., :self.kv_lora_rank]

    def get_kv_buffer(self, layer_id: int) -> Tuple[Tensor, Tensor]:
        return self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

    def get_row_scale(self, layer_id: int) -> Optional[Tensor]:
        """The layer's per-slot fp32 scales (FP8 rows), None for bf16 rows."""
        i = self._idx(layer_id)
        return self.row_scale[i] if self.fp8 else None

    def get_block_buffer(self, layer_id: int) -> Tensor:
        """The layer's rows as blocks [num_blocks, page_size, kv_cache_dim] of the stored bytes, a view
        (memory_pool.py:358-364)."""
        if self.size % self.page_size:
            raise ValueError(f"an MLA pool of {self.size} tokens is not whole {self.page_size}-token pages")
        return self.kv_buffer[self._idx(layer_id)].view(self.num_blocks, self.page_size, self.kv_cache_dim)

    def get_kv_layer_ids(self) -> List[int]:
        return list(self.model_layer_ids)

    def set_mla_kv_buffer(self, layer, loc: Tensor, cache_k_nope: Tensor, cache_k_rope: Tensor) -> None:
        """Store rows [latent | rope] built from ``cache_k_nope`` [T, 1, 512] and ``cache_k_rope`` [T, 1, 64] at
        slots ``loc``, each quantized with its own absmax / 448 scale (the reference raises, memory_pool.py:417-418)."""
        rows = torch.cat([cache_k_nope.reshape(-1, self.kv_lora_rank), cache_k_rope.reshape(-1, self.qk_rope_head_dim)],
                         dim=-1)
        self._store(_layer_id(layer), loc, rows)

    def set_kv_buffer(self, layer, loc: Tensor, cache_k: Tensor, cache_v: Optional[Tensor] = None, *args,
                      **kwargs) -> None:
        """Store full rows ``cache_k`` [T, 1, 576] at slots ``loc`` (``cache_v`` is unused: V is the rows' latent)."""
        self._store(_layer_id(layer), loc, cache_k.reshape(-1, self.kv_cache_dim))

    def _store(self, layer_id: int, loc: Tensor, rows: Tensor) -> None:
        i = self._idx(layer_id)
        ops.kv_store_mla(rows, loc, self.kv_buffer[i], self.row_scale[i] if self.fp8 else None)

    def get_kv_size_bytes(self) -> int:
        rows = (self.size + self.page_size) * self.layer_num
        return rows * (self.kv_cache_dim * self.store_dtype.itemsize + (4 if self.fp8 else 0))

    def get_contiguous_buf_infos(self):
        """(ptrs, lens, item_lens) of each layer's rows: page p is item_len bytes at ptr + p * item_len
        (memory_pool.py:404-412)."""
        ptrs = [t.data_ptr() for t in self.kv_buffer]
        lens = [t.numel() * t.element_size() for t in self.kv_buffer]
        return ptrs, lens, [t[0].numel() * t.element_size() * self.page_size for t in self.kv_buffer]

    def get_scale_buf_infos(self):
        """(ptrs, lens, item_lens) of each layer's per-slot fp32 row scales, paged like the rows (page p is page_size *
        4 bytes at ptr + p * item_len). The reference's MLA pool has no such scales; a transfer of this pool moves
        these items beside the rows of get_contiguous_buf_infos. A bf16 pool has none: empty lists."""
        ptrs = [t.data_ptr() for t in self.row_scale]
        lens = [t.numel() * t.element_size() for t in self.row_scale]
        return ptrs, lens, [self.page_size * 4] * len(self.row_scale)

    def get_cpu_copy(self, *args, **kwargs):
        raise NotImplementedError("KV host offload is not part of this build")

    def load_cpu_copy(self, *args, **kwargs):
        raise NotImplementedError("KV host offload is not part of this build")


class NeuronDSATokenToKVPool:
    """The DSA (DeepSeek sparse attention) row pool of the GLM-5 decode: per layer ``[num_blocks, 1, page_size, 640]``
    uint8 rows ``[bf16(k_pe / kv_scale) 128 B | e4m3fn(latent / kv_scale) 512 B, permuted]``
    (models/glm52/kernels/decode/attention/mla/kv_row_layout.py:38-99), one per-tensor ``kv_scale`` per layer."""

    ROW_BYTES = 640

    def __init__(self, size: int, page_size: int, layer_num: int, device: Union[str, torch.device],
                 kv_scale: float = 1.0, start_layer: Optional[int] = None, **kwargs):
        if size % page_size:
            raise ValueError(f"a pool of {size} tokens is not whole pages of {page_size}")
        self.size = int(size)
        self.page_size = int(page_size)
        self.layer_num = int(layer_num)
        self.start_layer = int(start_layer or 0)
        self.device = torch.device(device)
        self.num_blocks = self.size // self.page_size + 1
        self.kv_scale: List[float] = [float(kv_scale)] * self.layer_num
        self.kv_buffer: List[Tensor] = [
            torch.zeros((self.num_blocks, 1, self.page_size, self.ROW_BYTES), dtype=torch.uint8, device=self.device)
            for _ in range(self.layer_num)]

    def _idx(self, layer_id: int) -> int:
        i = layer_id - self.start_layer
        if not 0 <= i < self.layer_num:
            raise IndexError(f"layer {layer_id} is outside this pool's layers")
        return i

    def get_key_buffer(self, layer_id: int) -> Tensor:
        return self.kv_buffer[self._idx(layer_id)]

    def get_kv_scale(self, layer_id: int) -> float:
        return self.kv_scale[self._idx(layer_id)]

    def set_kv_buffer(self, layer, loc: Tensor, rows: Tensor, *args, **kwargs) -> None:
        """Pack rows [T, 576] bf16 ([k_pe 64 | latent 512]) and scatter them to slots ``loc``; a negative or
        out-of-pool slot is skipped (mla_decode_attention_torch.py:193-201)."""
        i = self._idx(_layer_id(layer))
        ops.kv_store_dsa(rows.reshape(-1, 576), loc, self.kv_buffer[i], self.kv_scale[i])

    def get_kv_size_bytes(self) -> int:
        return self.num_blocks * self.page_size * self.ROW_BYTES * self.layer_num


# Kind aliases under the names the reference registers with SGLang (memory_pool.py:213)
NeuronMHATokenToKVPoolKind = NeuronMHATokenToKVPool


def full_attention_pool(pool):
    """The pool itself (this build has no hybrid linear-attention pools); the reference's helper of that name
    unwraps SGLang's hybrid pool."""
    return pool
