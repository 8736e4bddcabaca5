"""Tensor-level entry points of the HIP path. Each checks shapes, dtypes and devices on the host, then calls the C ABI
on torch's current stream. There is no CPU or eager fallback: without the built library, or with CPU tensors, these
raise.

Reference interfaces each function stands in for are cited per function (paths under
/root/reference/sglang_neuron).
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence, Union

import torch
from torch import Tensor

from . import _lib

FP8 = torch.float8_e4m3fn
_cu_count: dict[int, int] = {}


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    """The current HIP stream of `device` (its raw handle: torch's own accessor, a few hundred ns, where building the
    torch.cuda.Stream object costs microseconds a call)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return _raw_stream(idx)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None) or \
    (lambda idx: torch.cuda.current_stream(idx).cuda_stream)


def _num_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_count:
        _cu_count[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_count[idx]


def _need(cond: bool, msg) -> None:
    """Raise ValueError(msg) unless cond; msg is a string or, where building it costs (a formatted message on a hot
    path), a callable that returns it."""
    if not cond:
        raise ValueError(msg() if callable(msg) else msg)


def _on_gpu(*ts: Optional[Tensor]) -> torch.device:
    """The device of the given tensors (None entries skipped): every one a GPU tensor on the same GPU, else
    ValueError (compared by device index, which get_device gives without building a torch.device per tensor)."""
    first = None
    idx = -1
    for t in ts:
        if t is None:
            continue
        i = t.get_device()
        if first is None:
            first, idx = t, i
        if i < 0 or i != idx:
            _need(t.is_cuda, "the HIP path takes device tensors (got a CPU tensor); there is no CPU fallback")
            _need(False, lambda: f"tensors on {t.device} and {first.device}")
    assert first is not None
    _need(idx >= 0, "the HIP path takes device tensors (got a CPU tensor); there is no CPU fallback")
    return first.device


def _contig(t: Tensor, name: str, dtype: Optional[torch.dtype] = None) -> Tensor:
    if dtype is not None:
        _need(t.dtype == dtype, lambda: f"{name} must be {dtype}, got {t.dtype}")
    return t if t.is_contiguous() else t.contiguous()


def _as(t: Tensor, dtype: torch.dtype) -> Tensor:
    """t converted to dtype, t itself when it already is (skipping Tensor.to's argument parsing on the hot path)."""
    return t if t.dtype == dtype else t.to(dtype)


def cache_dtype_code(dtype: torch.dtype, scales_multiply: bool = False) -> int:
    """The C ABI's cache dtype code. ``scales_multiply``: an FP8 cache whose scales are the GPT-OSS quantization
    multipliers m (SNA_DTYPE_FP8_E4M3FN_MUL) rather than dequantization scales."""
    if dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dtype in (FP8, torch.uint8):
        return _lib.DTYPE_FP8_E4M3FN_MUL if scales_multiply else _lib.DTYPE_FP8_E4M3FN
    raise ValueError(f"unsupported cache dtype {dtype} (bf16 or float8_e4m3fn)")


def inverted_kv_scale(scale: Union[float, Tensor]) -> Tensor:
    """The GPT-OSS quantization multiplier of a checkpoint's dequantization scale, as the reference's loader makes it:
    ``1.0 / scale.to(bfloat16)``, a bf16 value (models/gpt_oss/mxfp4/common.py:481-485), returned as fp32. Computed on
    the host, so every device gets the same bits."""
    s = torch.as_tensor(scale).detach().to("cpu", torch.float32)
    return (1.0 / s.to(torch.bfloat16)).float()


def prefill_write_scale(multiplier: Union[float, Tensor]) -> Tensor:
    """The dequantization scale the reference's GPT-OSS prefill writes with, from the decode's multiplier m:
    ``1.0 / m`` as bf16 (models/gpt_oss/mxfp4/model_prefill.py:41-43), returned as fp32 (host)."""
    m = torch.as_tensor(multiplier).detach().to("cpu", torch.float32)
    return (1.0 / m.to(torch.bfloat16)).float()


# ------------------------------------------------------------------------------------------------------------------
# stores
# ------------------------------------------------------------------------------------------------------------------

def kv_store_mha(k: Tensor, v: Tensor, slots: Tensor, k_cache: Tensor, v_cache: Tensor,
                 k_scale: Optional[Tensor] = None, v_scale: Optional[Tensor] = None,
                 scales_multiply: bool = False) -> None:
    """Write the tokens' K/V [T, kv_heads, d] bf16 into one layer's caches [blocks, kv_heads, page, d] at ``slots``
    [T] (int64); FP8 caches quantize with the per-head dequantization scales [kv_heads] (e4m3fn(x / s), qkv.py:69-70),
    or, with ``scales_multiply``, with the GPT-OSS multipliers m (e4m3fn(bf16(x * m)), attention_decode.py:259-260).
    Out-of-pool slots write slot 0, as the reference's write does (ops/attention/attention_decode.py:288-300)."""
    dev = _on_gpu(k, v, slots, k_cache, v_cache, k_scale, v_scale)
    nb, G, P, d = k_cache.shape
    _need(v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype, "K and V caches differ")
    k = _contig(k.reshape(-1, G, d), "k", torch.bfloat16)
    v = _contig(v.reshape(-1, G, d), "v", torch.bfloat16)
    _need(k.shape == v.shape, lambda: f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    slots = _contig(_as(slots.reshape(-1), torch.int64), "slots")
    _need(slots.numel() == k.shape[0], lambda: f"{slots.numel()} slots for {k.shape[0]} tokens")
    code = cache_dtype_code(k_cache.dtype, scales_multiply)
    if code != _lib.DTYPE_BF16:
        _need(k_scale is not None and v_scale is not None, "an FP8 cache needs k_scale and v_scale")
        k_scale = _contig(_as(k_scale.reshape(-1), torch.float32), "k_scale")
        v_scale = _contig(_as(v_scale.reshape(-1), torch.float32), "v_scale")
        _need(k_scale.numel() == G and v_scale.numel() == G, lambda: f"scales must have {G} entries (one per KV head)")
    _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    rc = _lib.load().sna_kv_store_mha(_ptr(k), _ptr(v), _ptr(slots), k.shape[0], _ptr(k_scale), _ptr(v_scale),
                                      _ptr(k_cache), _ptr(v_cache), nb, G, P, d, code, _stream(dev))
    _lib.check(rc, "kv_store_mha")


def qkv_norm_rope_store(qkv: Tensor, *, cos: Tensor, sin: Tensor, num_q_heads: int, num_kv_heads: int, d_head: int,
                        k_cache: Tensor, v_cache: Tensor, slot_mapping: Tensor, q_norm: Optional[Tensor] = None,
                        k_norm: Optional[Tensor] = None, norm_eps: float = 1e-6, k_scale: Optional[Tensor] = None,
                        v_scale: Optional[Tensor] = None, q_out: Optional[Tensor] = None) -> Tensor:
    """The writer after the QKV projection: ``qkv`` [T, (q + 2 kv) * d] bf16 (the projection with its bias), per-head
    RMSNorm of Q and K when ``q_norm`` / ``k_norm`` [d] are given, rotate-half RoPE by ``cos`` / ``sin`` [T, d] (or
    [1, T, d]), K and V stored at ``slot_mapping`` [T] into the layer's caches [blocks, kv, page, d] (bf16, or FP8 with
    per-KV-head ``k_scale`` / ``v_scale``). Returns Q [T, q, d] bf16; the caches are written in place.

    Stands in for _torch_qkv_paged after its projection (ops/attention/qkv_paged.py:45-68) and for _torch_qkv's rope
    and FP8 write (ops/attention/qkv.py:57-85)."""
    dev = _on_gpu(qkv, cos, sin, k_cache, v_cache, slot_mapping, q_norm, k_norm, k_scale, v_scale, q_out)
    nb, G, P, d = k_cache.shape
    _need(G == num_kv_heads and d == d_head,
          lambda: f"caches {tuple(k_cache.shape)} for {num_kv_heads} heads of {d_head}")
    _need(v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype, "K and V caches differ")
    _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    width = (num_q_heads + 2 * num_kv_heads) * d_head
    qkv = qkv.reshape(-1, qkv.shape[-1])
    _need(qkv.dtype == torch.bfloat16 and qkv.shape[-1] == width and qkv.stride(-1) == 1,
          lambda: f"qkv must be bf16 [T, {width}] with unit column stride")
    T = qkv.shape[0]
    cos = _contig(cos.reshape(-1, d_head), "cos", torch.bfloat16)
    sin = _contig(sin.reshape(-1, d_head), "sin", torch.bfloat16)
    _need(cos.shape[0] == T and sin.shape[0] == T, lambda: f"cos/sin need {T} rows")
    slots = _contig(_as(slot_mapping.reshape(-1), torch.int64), "slot_mapping")
    _need(slots.numel() == T, lambda: f"{slots.numel()} slots for {T} tokens")
    _need((q_norm is None) == (k_norm is None), "give both QK-norm gammas or neither")
    if q_norm is not None:
        q_norm = _contig(q_norm.reshape(-1), "q_norm", torch.bfloat16)
        k_norm = _contig(k_norm.reshape(-1), "k_norm", torch.bfloat16)
        _need(q_norm.numel() == d_head and k_norm.numel() == d_head, lambda: f"QK-norm gammas need {d_head} entries")
    code = cache_dtype_code(k_cache.dtype)
    if code == _lib.DTYPE_FP8_E4M3FN:
        _need(k_scale is not None and v_scale is not None, "an FP8 cache needs k_scale and v_scale")
        k_scale = _contig(k_scale.reshape(-1).float().expand(G) if k_scale.numel() == 1 else k_scale.reshape(-1).float(),
                          "k_scale")
        v_scale = _contig(v_scale.reshape(-1).float().expand(G) if v_scale.numel() == 1 else v_scale.reshape(-1).float(),
                          "v_scale")
        _need(k_scale.numel() == G and v_scale.numel() == G, lambda: f"scales need 1 or {G} entries")
    if q_out is None:
        q_out = torch.empty(T, num_q_heads, d_head, dtype=torch.bfloat16, device=dev)
    _need(q_out.shape == (T, num_q_heads, d_head) and q_out.dtype == torch.bfloat16 and q_out.is_contiguous(),
          "bad q_out tensor")
    rc = _lib.load().sna_qkv_norm_rope_store(
        _ptr(qkv), qkv.stride(0), T, num_q_heads, num_kv_heads, d_head, _ptr(q_norm), _ptr(k_norm), float(norm_eps),
        _ptr(cos), _ptr(sin), cos.stride(0), _ptr(slots), _ptr(q_out), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale),
        _ptr(v_scale), nb, P, code, _stream(dev))
    _lib.check(rc, "qkv_norm_rope_store")
    return q_out


def kv_absmax_scale(x: Tensor) -> Tensor:
    """Per-head dequantization scales [H] fp32 of x [T, H, d] bf16: absmax / 448, or 1 for an all-zero head."""
    dev = _on_gpu(x)
    _need(x.dim() == 3, lambda: f"x must be [T, H, d], got {tuple(x.shape)}")
    x = _contig(x, "x", torch.bfloat16)
    T, H, d = x.shape
    lib = _lib.load()
    ws = torch.empty(max(int(lib.sna_absmax_workspace_bytes(T, H)), 4), dtype=torch.uint8, device=dev)
    out = torch.empty(H, dtype=torch.float32, device=dev)
    rc = lib.sna_kv_absmax_scale(_ptr(x), T, H, d, _ptr(out), _ptr(ws), ws.numel(), _stream(dev))
    _lib.check(rc, "kv_absmax_scale")
    return out


def kv_store_mla(rows: Tensor, slots: Tensor, cache: Tensor, row_scale: Optional[Tensor] = None) -> None:
    """Write compact MLA rows [T, 576] bf16 into a layer's rows [slots, 576] (or [slots, 1, 576]) at ``slots``; an
    FP8 (uint8-stored) cache gets one scale per token in ``row_scale`` [slots]. Out-of-pool slots write slot 0
    (models/deepseek_v2/model.py:64-70)."""
    dev = _on_gpu(rows, slots, cache, row_scale)
    flat = cache.reshape(cache.shape[0], -1)
    n_slots, dim = flat.shape
    rows = _contig(rows.reshape(-1, dim), "rows", torch.bfloat16)
    slots = _contig(_as(slots.reshape(-1), torch.int64), "slots")
    _need(slots.numel() == rows.shape[0], lambda: f"{slots.numel()} slots for {rows.shape[0]} rows")
    code = cache_dtype_code(cache.dtype)
    if code == _lib.DTYPE_FP8_E4M3FN:
        _need(row_scale is not None and row_scale.numel() == n_slots and row_scale.dtype == torch.float32
              and row_scale.is_contiguous(), lambda: f"an FP8 MLA cache needs a contiguous fp32 row_scale of {n_slots}")
    _need(cache.is_contiguous(), "cache must be contiguous")
    rc = _lib.load().sna_kv_store_mla(_ptr(rows), _ptr(slots), rows.shape[0], dim, _ptr(cache), _ptr(row_scale),
                                      n_slots, code, _stream(dev))
    _lib.check(rc, "kv_store_mla")


def kv_store_dsa(rows: Tensor, slots: Tensor, cache: Tensor, kv_scale: float) -> None:
    """Pack rows [T, 576] bf16 ([k_pe 64 | latent 512]) into the 640-byte layout and scatter them to ``slots``
    (flat rows of ``cache`` [..., 640] uint8); a negative or out-of-cache slot is skipped
    (models/glm52/kernels/decode/attention/mla/mla_decode_attention_torch.py:193-221)."""
    dev = _on_gpu(rows, slots, cache)
    _need(cache.dtype == torch.uint8 and cache.shape[-1] == 640 and cache.is_contiguous(),
          "the DSA cache is contiguous uint8 [..., 640]")
    rows = _contig(rows.reshape(-1, 576), "rows", torch.bfloat16)
    slots = _contig(_as(slots.reshape(-1), torch.int64), "slots")
    _need(slots.numel() == rows.shape[0], lambda: f"{slots.numel()} slots for {rows.shape[0]} rows")
    n_rows = cache.numel() // 640
    rc = _lib.load().sna_kv_store_dsa(_ptr(rows), _ptr(slots), rows.shape[0], float(kv_scale), _ptr(cache), n_rows,
                                      _stream(dev))
    _lib.check(rc, "kv_store_dsa")


# ------------------------------------------------------------------------------------------------------------------
# planning
# ------------------------------------------------------------------------------------------------------------------

def plan_decode(kind: int, B: int, *, host_seq_lens: Union[Tensor, Sequence[int], None] = None,
                max_seq_len: int = -1, window: int = 0, n_keys_per_row: int = 0, ctas_per_item: int = 1,
                num_cus: int = 0, gqa_depth: int = 0) -> _lib.SplitPlan:
    """The split-K plan of a decode launch (sna_plan_decode): exact from host seq_lens, or a bound from
    ``max_seq_len``. ``gqa_depth`` (2 or 3) asks for a GQA plan shape (see sna_split_plan.depth); 0 lets the planner pick."""
    plan = _lib.SplitPlan()
    plan.depth = int(gqa_depth)
    arr = None
    if host_seq_lens is not None:
        t = torch.as_tensor(host_seq_lens, dtype=torch.int32).reshape(-1).cpu().contiguous()
        _need(t.numel() == B, lambda: f"{t.numel()} host seq_lens for {B} rows")
        arr = t
    rc = _lib.load().sna_plan_decode(kind, None if arr is None else arr.data_ptr(), B, max_seq_len, window,
                                     n_keys_per_row, ctas_per_item, num_cus, plan)
    _lib.check(rc, "plan_decode")
    return plan


def _row_splits(L: int, window: int, split_tiles: int) -> int:
    """A GQA row's split count: its key tiles of 32 from its window's first key to its last prior key, over
    split_tiles (the kernels' splits_of)."""
    if L <= 1:
        return 0
    hi, lo = L - 1, (L - window if window > 0 and L - window > 0 else 0)
    if hi <= lo:
        return 0
    return (-(-hi // 32) - lo // 32 + split_tiles - 1) // split_tiles


def _gqa_device_split_tiles(tiles, n_work: int) -> int:
    """The split size a device-split GQA launch computes from its rows' tile counts (gqa_device_item): the least size
    at least 4, ceil(total / items) and min(longest, 8) (at most max(longest, 4)) whose items, max(1, ceil(tiles /
    size)) a row, fit items = max(n_work, B); then at least a 64th of the longest row."""
    B = len(tiles)
    items = max(n_work, B, 1)
    total, mx = sum(tiles), max(tiles, default=0)
    cap = max(mx, 4)
    lo = min(max(4, -(-total // items), min(mx, 8)), cap)
    hi = min(cap, max(lo, -(-total // (items - B)))) if items > B else cap
    while lo < hi:
        mid = (lo + hi) // 2
        if sum(max(1, -(-t // mid)) for t in tiles) <= items:
            hi = mid
        else:
            lo = mid + 1
    return max(lo, -(-mx // 64))


def check_plan_lengths(plan: _lib.SplitPlan, kind: int, host_seq_lens, window: int = 0) -> None:
    """Refuse a plan that cannot serve these lengths (host copies): a GQA plan whose item map or split count misses a
    split some row needs (those keys would be dropped), an MLA plan made for other key counts (its launch is cut by
    the plan's). Raises ValueError naming the first row."""
    lens = [int(x) for x in torch.as_tensor(host_seq_lens).reshape(-1).tolist()]
    _need(len(lens) == plan.batch, lambda: f"a plan for {plan.batch} rows, {len(lens)} lengths")
    if kind == _lib.KIND_GQA:
        if plan.device_split:
            # the launch sizes its splits from the device's lengths (gqa_device_item): a row must fit the plan's
            # split count
            tiles = [_row_splits(L, window, 1) for L in lens]
            st = _gqa_device_split_tiles(tiles, plan.n_work)
            for b, t in enumerate(tiles):
                _need(max(1, -(-t // st)) <= max(plan.max_splits, 1),
                      lambda: f"row {b}: seq_len {lens[b]} is past the plan's bound (at most {plan.max_splits} splits)")
            return
        need = [_row_splits(L, window, plan.split_tiles) for L in lens]
        if plan.work_n > 0:
            have = [0] * len(lens)
            for i in range(plan.work_n):
                have[(plan.work[i] & 0x7FFFFFFF) >> 6] += 1
        else:
            have = [max(plan.max_splits, 1)] * len(lens)
        for b, (n, h) in enumerate(zip(need, have)):
            _need(n <= h,
                  lambda: f"row {b}: seq_len {lens[b]} needs {n} splits, the plan runs {h} (made for other lengths)")
        _need(sum(need) <= plan.n_work,
              lambda: f"the lengths need {sum(need)} split items, the plan runs {plan.n_work}")
    elif kind == _lib.KIND_MLA:
        for b, L in enumerate(lens):
            if plan.device_split:  # a bound: the launch cuts its split from the device's lengths
                _need(L - 1 <= plan.row_keys[b],
                      lambda: f"row {b}: seq_len {L} is past the plan's bound {plan.row_keys[b] + 1}")
                continue
            _need(plan.row_keys[b] == max(L - 1, 0),
                  lambda: f"row {b}: seq_len {L}, the plan was made for {plan.row_keys[b] + 1} "
                          "(its launch is cut by them)")


def check_decode_operands(seq_lens: Tensor, block_table: Tensor, new_slots: Optional[Tensor], page_size: int,
                          num_blocks: int, active: Optional[Tensor] = None) -> None:
    """Refuse a decode batch whose host operands the kernels cannot serve (sna_check_decode_operands): a seq_len
    outside [1, 2^31 - 1], a block table too narrow for a row or naming a page outside the pool inside a row's pages,
    a live row's new slot that is outside the pool, on the reserved page 0, or not at its position on its last page,
    two live rows writing one slot. Host (CPU) tensors: seq_lens [B] int, block_table [B, W] int32, new_slots [B] int
    or None, active [B] (1 = live) or None (then a row is live unless it is a padding row: seq_len 1 written to page 0
    or outside the pool). Raises ValueError naming the row.

    The refusals of the reference's decode_operands (attention/mla_operands.py:54-97)."""
    for t in (seq_lens, block_table, new_slots, active):
        _need(t is None or not t.is_cuda, "check_decode_operands takes host copies of the operands")
    lens = seq_lens.reshape(-1).to(torch.int64).contiguous()
    B = lens.numel()
    _need(block_table.dim() == 2 and block_table.shape[0] == B, lambda: f"block_table must be [{B}, width]")
    table = block_table.to(torch.int32).contiguous()
    slots = None if new_slots is None else new_slots.reshape(-1).to(torch.int64).contiguous()
    _need(slots is None or slots.numel() == B, lambda: f"new_slots must have {B} entries")
    act = None if active is None else active.reshape(-1).to(torch.int32).contiguous()
    _need(act is None or act.numel() == B, lambda: f"active must have {B} entries")
    rc = _lib.load().sna_check_decode_operands(lens.data_ptr(), table.data_ptr(), table.stride(0), table.shape[1],
                                               None if slots is None else slots.data_ptr(),
                                               None if act is None else act.data_ptr(), B, int(page_size),
                                               int(num_blocks))
    _lib.check(rc, "check_decode_operands")


def workspace_bytes(plan: _lib.SplitPlan, heads: int, dim_v: int) -> int:
    return int(_lib.load().sna_decode_workspace_bytes(plan, heads, dim_v))


def _stream_workspace_arg(ws: Optional[Tensor], plan: _lib.SplitPlan, heads: int, device) -> Tensor:
    if ws is None:
        return stream_workspace(plan, heads, device)
    _need(ws.dtype == torch.uint8 and ws.is_contiguous() and ws.device == device, "workspace must be contiguous uint8 "
          "on the decode's device")
    _need(ws.numel() >= workspace_bytes(plan, heads, 512), lambda: f"workspace of {ws.numel()} bytes, the plan needs "
          f"{workspace_bytes(plan, heads, 512)}")
    return ws


def stream_row_chunks(kind: int, B: int, heads: int, n_keys_per_row: int = 0, spec: int = 1) -> list[tuple[int, int]]:
    """Row ranges [r0, r1) that split an MLA / DSA batch into launches each one plan can hold: at most MAX_PLAN_ROWS
    rows, at most STREAM_MAX_COUNTERS merge counters (rows x 16-head groups), and for DSA at most MAX_CTAS workgroups
    of at most SPARSE_MAX_RANGE_KEYS keys (a row of K keys takes ceil(K / 2048) of them), whole sequences of ``spec``
    query tokens each (a token attends its siblings' rows in its own launch). One range for the batches of the
    measured configurations; the launches of a split batch run one after another on the stream."""
    groups = (heads + 15) // 16
    rows = min(_lib.MAX_PLAN_ROWS, _lib.STREAM_MAX_COUNTERS // groups)
    if kind == _lib.KIND_DSA:
        pieces = max(1, -(-int(n_keys_per_row) // _lib.SPARSE_MAX_RANGE_KEYS))
        _need(pieces <= _lib.MAX_CTAS, lambda: f"a DSA row of {n_keys_per_row} keys needs more than {_lib.MAX_CTAS} "
              "workgroups")
        rows = min(rows, _lib.MAX_CTAS // pieces)
    rows -= rows % spec
    _need(rows >= spec, lambda: f"a sequence of {spec} query tokens does not fit one launch")
    return [(r0, min(B, r0 + rows)) for r0 in range(0, B, rows)] or [(0, 0)]


def _plans_of(plan, kind: int, B: int, heads: int, n_keys: int = 0, spec: int = 1):
    """(row chunks, plans) of a caller's plan argument: one plan for the whole batch, or a list with one plan per
    range of stream_row_chunks."""
    if isinstance(plan, _lib.SplitPlan):
        return [(0, B)], [plan]
    chunks = stream_row_chunks(kind, B, heads, n_keys, spec)
    plans = list(plan)
    _need(len(plans) == len(chunks),
          lambda: f"{len(plans)} plans for the {len(chunks)} launches a batch of {B} rows takes")
    return chunks, plans


def stream_workspace(plan: _lib.SplitPlan, heads: int, device: torch.device) -> Tensor:
    """A workspace for an MLA / DSA plan: zeroed, so its counter block starts at zero (each completed launch leaves it
    zero again, so one workspace serves every later call ordered on one stream)."""
    return torch.zeros(max(workspace_bytes(plan, heads, 512), 256), dtype=torch.uint8, device=device)


def stream_workspace_status(ws: Tensor) -> int:
    """The status word of an MLA / DSA workspace, cleared as it is read (sna_stream_workspace_status): 0 when every
    launch on it since the last read found its counter block clean, else WS_DIRTY_ARRIVAL (a row's merge could not be
    trusted) and / or WS_DIRTY_DONE (the counters may not return to zero by themselves: reset_stream_workspace).
    Waits for the current stream."""
    _need(ws.is_cuda and ws.dtype == torch.uint8 and ws.is_contiguous(), "workspace must be a contiguous uint8 GPU "
          "tensor")
    status = ctypes.c_int32(0)
    rc = _lib.load().sna_stream_workspace_status(_ptr(ws), ws.numel(), ctypes.addressof(status), _stream(ws.device))
    _lib.check(rc, "stream_workspace_status")
    return int(status.value)


def reset_stream_workspace(ws: Tensor) -> None:
    """Zero an MLA / DSA workspace's counter block on the current stream (sna_stream_workspace_reset: a fill kernel,
    so it may be captured in a graph)."""
    _need(ws.is_cuda and ws.dtype == torch.uint8 and ws.is_contiguous(), "workspace must be a contiguous uint8 GPU "
          "tensor")
    _lib.check(_lib.load().sna_stream_workspace_reset(_ptr(ws), ws.numel(), _stream(ws.device)),
               "stream_workspace_reset")


def _host_lens(seq_lens: Tensor, host_seq_lens) -> Optional[Tensor]:
    if host_seq_lens is not None:
        return torch.as_tensor(host_seq_lens, dtype=torch.int32).reshape(-1)
    if not seq_lens.is_cuda:
        return seq_lens.reshape(-1).to(torch.int32)
    return None


# ------------------------------------------------------------------------------------------------------------------
# decode attention
# ------------------------------------------------------------------------------------------------------------------

class Prepared:
    """One or more C-ABI calls with validated, bound arguments, launched again on every call. It keeps its tensors
    (inputs, outputs, workspace) alive and returns its outputs. The bench runs its timed loop through these, so host
    work stays out of the timing, and every public decode function below is prepare + one launch. The launches go to
    the stream that was current when it was prepared (bound like the pointers): prepare it on the stream it will run
    on, e.g. inside a graph capture to capture it."""

    def __init__(self, calls, keep, outputs, what):
        self._calls = calls        # [(fn, args)]
        self._keep = keep
        self.outputs = outputs
        self._what = what

    def __call__(self):
        for fn, args in self._calls:
            rc = fn(*args)
            if rc:
                _lib.check(rc, self._what)
        return self.outputs


def prepare_paged_decode_gqa(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                             k_new: Tensor, v_new: Tensor, *, sm_scale: float, k_scale: Optional[Tensor] = None,
                             v_scale: Optional[Tensor] = None, sinks: Optional[Tensor] = None, window: int = 0,
                             new_slots: Optional[Tensor] = None, out: Optional[Tensor] = None,
                             host_seq_lens=None, plan: Optional[_lib.SplitPlan] = None,
                             library_scratch: bool = False, scales_multiply: bool = False) -> Prepared:
    """paged_decode_gqa's checks and argument binding, launched by calling the result. With ``library_scratch`` the
    call is sna_paged_decode_gqa_noalloc: no workspace tensor is allocated, the split partials go to the library's
    per-GPU scratch array (at most NOALLOC_SCRATCH_BYTES; calls that overlap on one GPU race). With
    ``scales_multiply`` the FP8 scales are the GPT-OSS quantization multipliers m (a cached byte is worth byte / m,
    and the step's token is stored as e4m3fn(bf16(x * m)), attention_decode.py:259-260)."""
    dev = _on_gpu(q, k_cache, v_cache, block_table, seq_lens, k_new, v_new, k_scale, v_scale, sinks, new_slots, out)
    _need(q.dim() == 3, lambda: f"q must be [B, H, d], got {tuple(q.shape)}")
    B, H, d = q.shape
    nb, G, P, dk = k_cache.shape
    _need(dk == d and v_cache.shape == k_cache.shape and v_cache.dtype == k_cache.dtype,
          lambda: f"caches {tuple(k_cache.shape)} / {tuple(v_cache.shape)} do not match q's head_dim {d}")
    _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    _need(H % G == 0, lambda: f"{H} query heads over {G} KV heads")
    code = cache_dtype_code(k_cache.dtype, scales_multiply)
    q = _contig(q, "q", torch.bfloat16)
    k_new = _contig(k_new.reshape(B, G, d), "k_new", torch.bfloat16)
    v_new = _contig(v_new.reshape(B, G, d), "v_new", torch.bfloat16)
    _need(block_table.dim() == 2 and block_table.shape[0] == B, lambda: f"block_table must be [{B}, width]")
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    _need(table.stride(1) == 1, "block_table rows must be contiguous")
    lens = _contig(_as(seq_lens.reshape(-1), torch.int32), "seq_lens")
    _need(lens.numel() == B, lambda: f"{lens.numel()} seq_lens for {B} rows")
    if code != _lib.DTYPE_BF16:
        _need(k_scale is not None and v_scale is not None, "an FP8 cache needs k_scale and v_scale")
        k_scale = _contig(_as(k_scale.reshape(-1), torch.float32), "k_scale")
        v_scale = _contig(_as(v_scale.reshape(-1), torch.float32), "v_scale")
        _need(k_scale.numel() == G and v_scale.numel() == G, "one k/v scale per KV head")
    if sinks is not None:
        sinks = _contig(_as(sinks.reshape(-1), torch.float32), "sinks")
        _need(sinks.numel() == H, lambda: f"{sinks.numel()} sinks for {H} heads")
    if new_slots is not None:
        new_slots = _contig(_as(new_slots.reshape(-1), torch.int64), "new_slots")
        _need(new_slots.numel() == B, lambda: f"{new_slots.numel()} new slots for {B} rows")
    if out is None:
        out = torch.empty(B, H, d, dtype=torch.bfloat16, device=dev)
    _need(out.shape == (B, H, d) and out.dtype == torch.bfloat16 and out.is_contiguous(), "bad out tensor")
    hl = _host_lens(seq_lens, host_seq_lens)
    if plan is None:
        plan = plan_decode(_lib.KIND_GQA, B, host_seq_lens=hl, max_seq_len=table.shape[1] * P, window=window,
                           ctas_per_item=G, num_cus=_num_cus(dev))
    elif hl is not None:
        check_plan_lengths(plan, _lib.KIND_GQA, hl, window)
    lib = _lib.load()
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), _ptr(table), table.stride(0),
            table.shape[1], _ptr(lens), _ptr(k_new), _ptr(v_new), _ptr(new_slots), _ptr(sinks), int(window),
            float(sm_scale), _ptr(out), B, H, G, d, P, nb, code, plan)
    keep = (q, k_cache, v_cache, k_scale, v_scale, table, lens, k_new, v_new, new_slots, sinks, out, plan)
    if library_scratch:
        return Prepared([(lib.sna_paged_decode_gqa_noalloc, args + (_stream(dev),))], keep, out,
                        "paged_decode_gqa_noalloc")
    ws = torch.empty(max(workspace_bytes(plan, H, d), 16), dtype=torch.uint8, device=dev)
    return Prepared([(lib.sna_paged_decode_gqa, args + (_ptr(ws), ws.numel(), _stream(dev)))], keep + (ws,), out,
                    "paged_decode_gqa")


def paged_decode_gqa(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                     k_new: Tensor, v_new: Tensor, **kw) -> Tensor:
    """GQA decode of q [B, H, d] over a layer's paged caches [blocks, G, page, d], the step's token k_new / v_new
    [B, G, d] attended in-band (and stored at ``new_slots`` when given). Keyword arguments: sm_scale, k_scale,
    v_scale (FP8), scales_multiply (the scales are GPT-OSS multipliers), sinks, window, new_slots, out,
    host_seq_lens, plan. Returns [B, H, d] bf16.

    Stands in for the attention core of _torch_attention_decode_paged (ops/attention/attention_decode_paged.py:
    159-177) and _torch_attention_decode (ops/attention/attention_decode.py:259-300)."""
    return prepare_paged_decode_gqa(q, k_cache, v_cache, block_table, seq_lens, k_new, v_new, **kw)()


def paged_decode_gqa_multi(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                           k_new: Tensor, v_new: Tensor, *, sm_scale: float, new_slots: Tensor,
                           k_scale: Optional[Tensor] = None, v_scale: Optional[Tensor] = None,
                           sinks: Optional[Tensor] = None, window: int = 0, scales_multiply: bool = False,
                           host_seq_lens=None) -> Tensor:
    """GQA decode of S active tokens per row: q [B, S, H, d], the step's K/V k_new / v_new [B, S, G, d] stored at
    new_slots [B, S], seq_lens [B] counting the prior and the S tokens (token j at position L - S + j). Token j
    attends the row's prior and active tokens 0 .. j. Returns [B, S, H, d] bf16.

    The S tokens are stored first (kv_store_mha), then each (row, token) decodes as a row of its own whose length
    ends at that token: its earlier active tokens are then pool keys holding the bytes the store wrote, which are the
    values the reference attends in its last S slots (dequantized FP8 or bf16), so this is the reference's triu mask
    over the active slots. A window must hold the S tokens (S <= window), as the reference's mask does not window
    them. Stands in for _torch_attention_decode with X [B, S, Hd] (ops/attention/attention_decode.py:226-300)."""
    dev = _on_gpu(q, k_cache, v_cache, block_table, seq_lens, k_new, v_new, new_slots, k_scale, v_scale, sinks)
    _need(q.dim() == 4, lambda: f"q must be [B, S, H, d], got {tuple(q.shape)}")
    B, S, H, d = q.shape
    nb, G, P, _ = k_cache.shape
    _need(k_new.shape == (B, S, G, d) and v_new.shape == (B, S, G, d),
          lambda: f"k_new / v_new must be [{B}, {S}, {G}, {d}]")
    _need(new_slots.numel() == B * S, lambda: f"new_slots must be [{B}, {S}]")
    _need(window <= 0 or S <= window, lambda: f"{S} active tokens do not fit a window of {window}")
    hl = _host_lens(seq_lens, host_seq_lens)
    if hl is not None:
        _need(int(hl.min()) >= S if B else True, lambda: f"a row holds its {S} active tokens: seq_lens >= {S}")
    kv_store_mha(k_new.reshape(B * S, G, d), v_new.reshape(B * S, G, d), new_slots.reshape(-1), k_cache, v_cache,
                 k_scale, v_scale, scales_multiply=scales_multiply)
    j = torch.arange(S, device=dev, dtype=torch.int32)
    lens = (seq_lens.reshape(B, 1).to(torch.int32) - S + 1 + j).reshape(-1)
    rows = torch.arange(B, device=dev).repeat_interleave(S)
    table = block_table.index_select(0, rows)
    host_rows = None if hl is None else (hl.reshape(B, 1).to(torch.int32) - S + 1 + j.cpu()).reshape(-1)
    out = paged_decode_gqa(q.reshape(B * S, H, d), k_cache, v_cache, table, lens, k_new.reshape(B * S, G, d),
                           v_new.reshape(B * S, G, d), sm_scale=sm_scale, k_scale=k_scale, v_scale=v_scale,
                           sinks=sinks, window=window, scales_multiply=scales_multiply, host_seq_lens=host_rows)
    return out.reshape(B, S, H, d)


def prepare_mla_decode(ql_nope: Tensor, q_pe: Tensor, cache: Tensor, row_scale: Optional[Tensor], block_table: Tensor,
                       seq_lens: Tensor, compact_new: Tensor, *, sm_scale: float, page_size: int,
                       new_slots: Optional[Tensor] = None, out: Optional[Tensor] = None, host_seq_lens=None,
                       plan: Optional[_lib.SplitPlan] = None, workspace: Optional[Tensor] = None) -> Prepared:
    """mla_decode's checks and argument binding, launched by calling the result. ``workspace``: a uint8 tensor from
    stream_workspace (zeroed once, reused by calls ordered on one stream), or None for a new one.

    The plan: an exact one (from host lengths: ``host_seq_lens``, or seq_lens on the host) cuts the launch by those
    lengths, so a call with one must carry the host lengths it is checked against; a device-split plan
    (plan_decode(KIND_MLA, B, max_seq_len=bound)) lets the launch cut its split from the device's seq_lens, so one
    prepared (or captured) launch serves any lengths up to the bound. Without a plan: exact from host lengths when
    there are any, else a device split bounded by the block table's width."""
    dev = _on_gpu(ql_nope, q_pe, cache, row_scale, block_table, seq_lens, compact_new, new_slots, out)
    B, H, lat = ql_nope.shape
    _need(lat == 512 and q_pe.shape == (B, H, 64), "ql_nope [B, H, 512] and q_pe [B, H, 64]")
    # rows as the pool holds them: [slots, 576], [slots, 1, 576] or the block view [blocks, page, 576]
    _need(cache.shape[-1] == 576 and cache.is_contiguous(), lambda: f"MLA rows must be contiguous [.., 576], got "
          f"{tuple(cache.shape)}")
    code = cache_dtype_code(cache.dtype)
    n_slots = cache.numel() // 576
    P = int(page_size)
    _need(n_slots % P == 0, lambda: f"{n_slots} rows are not whole pages of {P}")
    nb = n_slots // P
    if code == _lib.DTYPE_FP8_E4M3FN:
        _need(row_scale is not None and row_scale.numel() == n_slots and row_scale.dtype == torch.float32 and
              row_scale.is_contiguous(), "FP8 rows need row_scale: contiguous fp32 with one entry per row")
    else:
        row_scale = None  # bf16 rows carry no scale
    ql_nope = _contig(ql_nope, "ql_nope", torch.bfloat16)
    q_pe = _contig(q_pe, "q_pe", torch.bfloat16)
    compact_new = _contig(compact_new.reshape(B, 576), "compact_new", torch.bfloat16)
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    _need(table.dim() == 2 and table.shape[0] == B and table.stride(1) == 1,
          lambda: f"block_table must be [{B}, width]")
    lens = _contig(_as(seq_lens.reshape(-1), torch.int32), "seq_lens")
    _need(lens.numel() == B, lambda: f"{lens.numel()} seq_lens for {B} rows")
    if new_slots is not None:
        new_slots = _contig(_as(new_slots.reshape(-1), torch.int64), "new_slots")
        _need(new_slots.numel() == B, lambda: f"{new_slots.numel()} new slots for {B} rows")
    if out is None:
        out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    _need(out.shape == (B, H, 512) and out.dtype == torch.bfloat16 and out.is_contiguous(), "bad out tensor")
    hl = _host_lens(seq_lens, host_seq_lens)
    if plan is not None:
        chunks, plans = _plans_of(plan, _lib.KIND_MLA, B, H)
        for (r0, r1), pl in zip(chunks, plans):
            if hl is not None:
                check_plan_lengths(pl, _lib.KIND_MLA, hl[r0:r1])
            else:
                _need(bool(pl.device_split), "an exact MLA plan is cut by host lengths: pass host_seq_lens (or use a "
                      "device-split plan, plan_decode(KIND_MLA, B, max_seq_len=...), for lengths only the device "
                      "holds)")
    else:
        chunks = stream_row_chunks(_lib.KIND_MLA, B, H)
        bound = table.shape[1] * P
        plans = [plan_decode(_lib.KIND_MLA, r1 - r0, host_seq_lens=None if hl is None else hl[r0:r1],
                             max_seq_len=bound, ctas_per_item=(H + 15) // 16, num_cus=_num_cus(dev))
                 for r0, r1 in chunks]
    ws = _stream_workspace_arg(workspace, max(plans, key=lambda p: workspace_bytes(p, H, 512)), H, dev)
    lib = _lib.load()
    calls = []
    for (r0, r1), pl in zip(chunks, plans):
        calls.append((lib.sna_mla_decode, (
            _ptr(ql_nope[r0:r1]), _ptr(q_pe[r0:r1]), _ptr(cache), _ptr(row_scale), _ptr(table[r0:r1]),
            table.stride(0), table.shape[1], _ptr(lens[r0:r1]), _ptr(compact_new[r0:r1]),
            None if new_slots is None else _ptr(new_slots[r0:r1]), float(sm_scale), _ptr(out[r0:r1]), r1 - r0, H, P,
            nb, code, pl, _ptr(ws), ws.numel(), _stream(dev))))
    keep = (ql_nope, q_pe, cache, row_scale, table, lens, compact_new, new_slots, out, ws, plans)
    return Prepared(calls, keep, out, "mla_decode")


def mla_decode(ql_nope: Tensor, q_pe: Tensor, cache: Tensor, row_scale: Tensor, block_table: Tensor,
               seq_lens: Tensor, compact_new: Tensor, **kw) -> Tensor:
    """Absorbed-MLA decode of ql_nope [B, H, 512] / q_pe [B, H, 64] over a layer's rows [slots, 576]: FP8 (uint8 or
    float8 storage) with per-token scales ``row_scale`` [slots], or bf16 (``row_scale`` unused, may be None); the
    history through ``block_table`` and the own row ``compact_new`` [B, 576] in-band (stored at ``new_slots`` when
    given). Keyword arguments: sm_scale, page_size,
    new_slots, out, host_seq_lens, plan. Returns [B, H, 512] bf16.

    Stands in for mla_decode (ops/attention/mla.py:32-53)."""
    return prepare_mla_decode(ql_nope, q_pe, cache, row_scale, block_table, seq_lens, compact_new, **kw)()


def prepare_mla_decode_sparse(q_absorbed: Tensor, q_pe: Tensor, cache: Tensor, kv_scale: float, indices: Tensor,
                              block_table: Tensor, positions: Tensor, own_rows: Tensor, *, sm_scale: float,
                              page_size: int, new_slots: Optional[Tensor] = None,
                              plan: Optional[_lib.SplitPlan] = None, workspace: Optional[Tensor] = None,
                              spec: int = 1) -> Prepared:
    """mla_decode_sparse's checks and argument binding (with ``new_slots``, the own rows are stored by the same launch),
    launched by calling the result."""
    dev = _on_gpu(q_absorbed, q_pe, cache, indices, block_table, positions, own_rows, new_slots)
    B, H, lat = q_absorbed.shape
    _need(lat == 512 and q_pe.shape == (B, H, 64), "q_absorbed [B, H, 512] and q_pe [B, H, 64]")
    _need(cache.dtype == torch.uint8 and cache.shape[-1] == 640 and cache.is_contiguous(), "cache [..., 640] uint8")
    n_rows = cache.numel() // 640
    P = int(page_size)
    _need(n_rows % P == 0, lambda: f"{n_rows} rows are not whole pages of {P}")
    q_absorbed = _contig(q_absorbed, "q_absorbed", torch.bfloat16)
    q_pe = _contig(q_pe, "q_pe", torch.bfloat16)
    own_rows = _contig(own_rows.reshape(B, 576), "own_rows", torch.bfloat16)
    idx = _contig(_as(indices.reshape(B, -1), torch.int32), "indices")
    K = idx.shape[1]
    spec = int(spec)
    _need(spec >= 1 and B % spec == 0, lambda: f"{B} query tokens are not whole sequences of {spec}")
    S = B // spec
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
    _need(table.dim() == 2 and table.shape[0] == S and table.stride(1) == 1,
          lambda: f"block_table must be [{S}, width] (one row per sequence)")
    pos = _contig(_as(positions.reshape(-1), torch.int32), "positions")
    _need(pos.numel() == B, lambda: f"{pos.numel()} positions for {B} rows")
    nkeys = K + spec - 1  # a row's keys: its index list, then its spec - 1 siblings' own rows
    if plan is not None:
        chunks, plans = _plans_of(plan, _lib.KIND_DSA, B, H, nkeys, spec)
    else:
        chunks = stream_row_chunks(_lib.KIND_DSA, B, H, nkeys, spec)
        plans = [plan_decode(_lib.KIND_DSA, r1 - r0, n_keys_per_row=nkeys, ctas_per_item=(H + 15) // 16,
                             num_cus=_num_cus(dev)) for r0, r1 in chunks]
    ws = _stream_workspace_arg(workspace, max(plans, key=lambda p: workspace_bytes(p, H, 512)), H, dev)
    ctx = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)
    lib = _lib.load()
    calls = []
    fused_slots = new_slots
    if new_slots is not None:
        new_slots = _contig(_as(new_slots.reshape(-1), torch.int64), "new_slots")
        _need(new_slots.numel() == B, lambda: f"{new_slots.numel()} new slots for {B} rows")
        fused_slots = new_slots
        if len(chunks) > 1:
            # The reference stores every own row before any gather (mla_decode_attention_torch.py steps 0-1): one
            # launch keeps that order in itself, several store the whole batch's rows first
            calls.append((lib.sna_kv_store_dsa, (_ptr(own_rows), _ptr(new_slots), B, float(kv_scale), _ptr(cache),
                                                 n_rows, _stream(dev))))
            fused_slots = None
    for (r0, r1), pl in zip(chunks, plans):
        calls.append((lib.sna_mla_decode_sparse, (
            _ptr(q_absorbed[r0:r1]), _ptr(q_pe[r0:r1]), _ptr(cache), float(kv_scale), _ptr(idx[r0:r1]), K,
            _ptr(table[r0 // spec:r1 // spec]), table.stride(0), table.shape[1], _ptr(pos[r0:r1]),
            _ptr(own_rows[r0:r1]), None if fused_slots is None else _ptr(fused_slots[r0:r1]), float(sm_scale),
            _ptr(ctx[r0:r1]), _ptr(lse[r0:r1]), r1 - r0, spec, H, P, n_rows // P, pl, _ptr(ws), ws.numel(),
            _stream(dev))))
    keep = (q_absorbed, q_pe, cache, idx, table, pos, own_rows, new_slots, ctx, lse, ws, plans)
    return Prepared(calls, keep, (ctx, lse), "mla_decode_sparse")


def mla_decode_sparse(q_absorbed: Tensor, q_pe: Tensor, cache: Tensor, kv_scale: float, indices: Tensor,
                      block_table: Tensor, positions: Tensor, own_rows: Tensor, **kw) -> tuple[Tensor, Tensor]:
    """DSA sparse decode: q_absorbed [B, H, 512], q_pe [B, H, 64], the 640-byte row cache, ``indices`` [B, K] int32
    global positions (-1 empty), ``block_table`` [B / spec, W] (one row per sequence), ``positions`` [B], own rows
    [B, 576] ([k_pe | latent]); ``spec`` query tokens per sequence (default 1; GLM's MTP verify runs 8): each token
    also attends its sequence's other own rows at their positions (kept iff at or before its own). With
    ``new_slots`` the launch also stores the own rows there, and a gather of such a slot attends the stored bytes
    (the reference stores them first, steps 0-1); without, the caller has stored them. Keyword arguments: sm_scale,
    page_size, new_slots, plan, spec. Returns (ctx [B, H, 512] bf16, lse [B, H] fp32).

    Stands in for mla_decode_attention_torch_ref with one token per sequence and one CP rank
    (models/glm52/kernels/decode/attention/mla/mla_decode_attention_torch.py:38-130)."""
    return prepare_mla_decode_sparse(q_absorbed, q_pe, cache, kv_scale, indices, block_table, positions, own_rows,
                                     **kw)()


def lse_combine(o_parts: Tensor, lse_parts: Tensor) -> tuple[Tensor, Tensor]:
    """Merge partial attention results o_parts [n, rows, dim] fp32 (each normalized) with their natural-log LSEs
    [n, rows]: out = sum_i exp(lse_i - LSE) o_i. The reference's DCP merge (ops/attention/attention_decode.py:
    277-285)."""
    dev = _on_gpu(o_parts, lse_parts)
    n, rows, dim = o_parts.shape
    o_parts = _contig(o_parts, "o_parts", torch.float32)
    lse_parts = _contig(lse_parts.reshape(n, rows), "lse_parts", torch.float32)
    out = torch.empty(rows, dim, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(rows, dtype=torch.float32, device=dev)
    rc = _lib.load().sna_lse_combine(_ptr(o_parts), _ptr(lse_parts), n, rows, dim, _ptr(out), _ptr(lse), _stream(dev))
    _lib.check(rc, "lse_combine")
    return out, lse


# ------------------------------------------------------------------------------------------------------------------
# prefill attention over the pool
# ------------------------------------------------------------------------------------------------------------------

def prefill_attention(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, q_start: Tensor,
                      prior_lens: Tensor, *, max_q_len: int, sm_scale: float, k_scale: Optional[Tensor] = None,
                      v_scale: Optional[Tensor] = None, sinks: Optional[Tensor] = None, window: int = 0,
                      out: Optional[Tensor] = None, host_q_start=None, scales_multiply: bool = False) -> Tensor:
    """Prefill attention of a batch of chunks: q [T, H, d] bf16 (request r's rows q_start[r] .. q_start[r + 1], at
    positions prior_lens[r] + i), every key read from one layer's caches [blocks, G, page, d] (FP8 with per-KV-head
    scales k_scale / v_scale [G], dequantization scales or, with ``scales_multiply``, GPT-OSS multipliers m whose
    bytes are worth byte / m; or bf16) through ``block_table`` [R, width] (store the chunk's K/V first, with
    kv_store_mha). Causal, optionally windowed (keys
    (p - window, p]) and with sinks [H]. ``max_q_len`` bounds the chunk lengths (a host int). Returns [T, H, d] bf16.
    ``host_q_start``: a host copy of q_start; with it the offsets are checked (0 first, non-decreasing, T last, no
    chunk longer than max_q_len: a row past the bound would be left unwritten) before the launch.

    Stands in for segmented_attention (ops/attention/attention_segmented_cte.py:21-75) over a batch."""
    dev = _on_gpu(q, k_cache, v_cache, block_table, q_start, prior_lens, k_scale, v_scale, sinks, out)
    T, H, d = q.shape
    nb, G, P, dk = k_cache.shape
    _need(dk == d and tuple(v_cache.shape) == tuple(k_cache.shape), "q, k_cache and v_cache disagree on shape")
    _need(H % G == 0, lambda: f"{H} query heads over {G} KV heads")
    R = prior_lens.shape[0]
    _need(q_start.shape == (R + 1,), lambda: f"q_start must be [{R + 1}]")
    _need(block_table.dim() == 2 and block_table.shape[0] >= R and block_table.stride(1) == 1,
          "block_table must be [R, width] with unit column stride")
    q = _contig(q, "q", torch.bfloat16)
    qs = q_start.to(torch.int32).contiguous()
    pl = prior_lens.to(torch.int32).contiguous()
    table = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32).contiguous()
    if host_q_start is not None:
        hq = [int(x) for x in torch.as_tensor(host_q_start).reshape(-1).tolist()]
        _need(len(hq) == R + 1 and hq[0] == 0 and hq[-1] == T,
              lambda: f"q_start must run from 0 to T = {T} over {R + 1} "
              f"entries, got {hq[:4]}{'...' if len(hq) > 4 else ''} ending {hq[-1] if hq else None}")
        lens = [hq[r + 1] - hq[r] for r in range(R)]
        _need(min(lens, default=0) >= 0, "q_start must not decrease")
        _need(max(lens, default=0) <= int(max_q_len),
              lambda: f"a chunk of {max(lens)} queries exceeds max_q_len {max_q_len}")
    code = cache_dtype_code(k_cache.dtype, scales_multiply)
    ks = vs = None
    if code != _lib.DTYPE_BF16:
        _need(k_scale is not None and v_scale is not None, "an FP8 pool needs k_scale and v_scale")
        ks = _contig(_as(k_scale.reshape(-1), torch.float32), "k_scale")
        vs = _contig(_as(v_scale.reshape(-1), torch.float32), "v_scale")
        _need(ks.numel() == G and vs.numel() == G, lambda: f"k_scale and v_scale must have {G} entries")
    sk = None if sinks is None else _contig(_as(sinks.reshape(-1), torch.float32), "sinks")
    if sk is not None:
        _need(sk.numel() == H, lambda: f"sinks must have {H} entries")
    if out is None:
        out = torch.empty(T, H, d, dtype=torch.bfloat16, device=dev)
    _need(out.shape == (T, H, d) and out.dtype == torch.bfloat16 and out.is_contiguous(), "out must be [T, H, d] bf16")
    if T == 0 or R == 0:
        return out
    rc = _lib.load().sna_prefill_attention(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(ks), _ptr(vs), _ptr(table), table.stride(0), table.shape[1],
        _ptr(qs), _ptr(pl), R, int(max_q_len), _ptr(sk), float(sm_scale), int(window), _ptr(out), H, G, d, P, nb,
        code, _stream(dev))
    _lib.check(rc, "prefill_attention")
    return out


def segmented_attention(q: Tensor, *, k_cache: Tensor, v_cache: Tensor, block_tables: Tensor, prior_tokens,
                        block_size: int, kv_segment_size: int, scale: float, sliding_window: Optional[int],
                        sink: Optional[Tensor], k_scale: Optional[Tensor] = None,
                        v_scale: Optional[Tensor] = None) -> Tensor:
    """The reference's signature (ops/attention/attention_segmented_cte.py:21-47) for one request: q [heads, S, d],
    caches [pages, kv_heads, page, d] (FP8, unpacked K, or bf16), block_tables [1, blocks], prior_tokens (an int or a 1-element
    tensor), sink [heads, 1] or None; returns [heads, S, d]. The per-KV-head scales k_scale / v_scale are this pool's
    (the reference folds its per-tensor scale into ``scale``); ``kv_segment_size`` is the Trainium kernel's tiling and
    has no role here."""
    del kv_segment_size
    heads, S, d = q.shape
    _need(block_size == k_cache.shape[2],
          lambda: f"block_size {block_size} differs from the cache's page {k_cache.shape[2]}")
    dev = q.device
    prior = int(torch.as_tensor(prior_tokens).reshape(-1)[0])
    out = prefill_attention(
        q.transpose(0, 1).contiguous(), k_cache, v_cache, block_tables[:1].to(dev),
        torch.tensor([0, S], dtype=torch.int32, device=dev), torch.tensor([prior], dtype=torch.int32, device=dev),
        max_q_len=S, sm_scale=scale, k_scale=k_scale, v_scale=v_scale, sinks=None if sink is None else sink.reshape(-1),
        window=int(sliding_window or 0), host_q_start=[0, S])
    return out.transpose(0, 1).contiguous()


# ------------------------------------------------------------------------------------------------------------------
# DSA indexer
# ------------------------------------------------------------------------------------------------------------------

def index_key_store(keys: Tensor, slots: Tensor, cache: Tensor) -> None:
    """Write index-key rows keys [T, d] (bf16) at ``slots`` [T] (int64) of an index-key cache [blocks, page, d]
    (uint8 or float8_e4m3fn) as e4m3fn(clamp(key, +-448)); out-of-cache slots are skipped
    (indexer_torch.py:44-53, :228-234)."""
    dev = _on_gpu(keys, slots, cache)
    d = cache.shape[-1]
    keys = _contig(keys.reshape(-1, d), "keys", torch.bfloat16)
    slots = _contig(slots.reshape(-1), "slots", torch.int64)
    _need(slots.numel() == keys.shape[0], "one slot per key row")
    _need(cache.dtype in (torch.uint8, FP8) and cache.is_contiguous(), "the index-key cache is contiguous e4m3fn bytes")
    rc = _lib.load().sna_index_key_store(_ptr(keys), _ptr(slots), keys.shape[0], d, _ptr(cache), cache.numel() // d,
                                         _stream(dev))
    _lib.check(rc, "index_key_store")


def indexer_scores(q: Tensor, w: Tensor, keys: Tensor, block_table: Tensor, limits: Tensor, width: int, *,
                   out: Optional[Tensor] = None) -> Tensor:
    """[B, width] bf16 index scores of every cached key: sum over heads of w[b, h] * relu(q[b, h] . key * d^-0.5),
    clamped to -1e30 for keys at or past ``limits[b]`` (the positions before the query's own) or on invalid pages.
    q [B, H, 128] bf16 (rotated), w [B, H] fp32 (scaled by H^-0.5), keys [blocks, page, 128] e4m3fn bytes read through
    ``block_table`` [B, W]. The score of indexer_kv_score_torch_ref (indexer_torch.py:254-268)."""
    dev = _on_gpu(q, w, keys, block_table, limits, out)
    B, H, d = q.shape
    nb, P, dk = keys.shape
    _need(dk == d, "q and the keys disagree on head_dim")
    _need(w.shape == (B, H) and limits.shape == (B,), lambda: f"w must be [{B}, {H}] and limits [{B}]")
    _need(block_table.dim() == 2 and block_table.shape[0] >= B and block_table.stride(1) == 1,
          "block_table must be [B, W] with unit column stride")
    q = _contig(q, "q", torch.bfloat16)
    w = _contig(w.float(), "w")
    lim = _contig(limits, "limits", torch.int32)
    table = block_table if block_table.dtype == torch.int32 else _contig(block_table, "block_table", torch.int32)
    _need(keys.dtype in (torch.uint8, FP8) and keys.is_contiguous(), "keys must be contiguous e4m3fn bytes")
    if out is None:
        out = torch.empty(B, width, dtype=torch.bfloat16, device=dev)
    _need(out.shape[0] == B and out.shape[1] >= width and out.dtype == torch.bfloat16 and out.stride(1) == 1,
          lambda: f"out must be [{B}, >= {width}] bf16")
    rc = _lib.load().sna_indexer_scores(_ptr(q), _ptr(w), _ptr(keys), _ptr(table), table.stride(0), table.shape[1],
                                        _ptr(lim), B, H, d, P, nb, int(width), _ptr(out), out.stride(0), _stream(dev))
    _lib.check(rc, "indexer_scores")
    return out


def topk_positions(scores: Tensor, k: int) -> Tensor:
    """[B, k] int32 positions of the k largest bf16 scores [B, N] per row: those above the k-th largest value, then
    its ties (lowest positions), each in position order; -1 for a selected dead key (score <= -1e30 / 2). The
    selection of indexer_topk_local_torch_ref (indexer_torch.py:296-309)."""
    dev = _on_gpu(scores)
    _need(scores.dim() == 2 and scores.dtype == torch.bfloat16 and scores.stride(1) == 1, "scores must be [B, N] bf16")
    B, N = scores.shape
    _need(1 <= k <= N, lambda: f"k {k} must be in [1, {N}]")
    out = torch.empty(B, k, dtype=torch.int32, device=dev)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.sna_topk_workspace_bytes(B, N)), 4), dtype=torch.uint8, device=dev)
    rc = lib.sna_topk_positions(_ptr(scores), scores.stride(0), B, N, int(k), _ptr(out), out.stride(0), _ptr(ws),
                                ws.numel(), _stream(dev))
    _lib.check(rc, "topk_positions")
    return out


# ------------------------------------------------------------------------------------------------------------------
# decode metadata on the device
# ------------------------------------------------------------------------------------------------------------------

def block_table(req_to_token: Tensor, req_pool_indices: Tensor, seq_lens: Tensor, page_size: int, width: int, *,
                seq_lens_i32: Optional[Tensor] = None) -> Tensor:
    """[B, width] int32 block table from req_to_token [rows, context] int32 (device), req_pool_indices [B] and
    seq_lens [B] (int64, device): floor(req_to_token[row_b, j * page] / page) while j * page < seq_len_b, else -1.
    ``seq_lens_i32`` [B] int32, when given, receives seq_lens narrowed (what the decode entry points take).
    With width = ceil(max seq_len / page) this is NeuronAttnBackend._block_table (attention/backend.py:114-130)."""
    dev = _on_gpu(req_to_token, req_pool_indices, seq_lens, seq_lens_i32)
    _need(req_to_token.dim() == 2 and req_to_token.dtype == torch.int32 and req_to_token.stride(1) == 1,
          "req_to_token must be [rows, context] int32 with unit column stride")
    B = req_pool_indices.shape[0]
    _need(seq_lens.shape == (B,), lambda: f"seq_lens must be [{B}]")
    _need(width >= 1 and page_size >= 1, lambda: f"width {width} and page_size {page_size} must be positive")
    rows = _contig(req_pool_indices, "req_pool_indices", torch.int64)
    lens = _contig(seq_lens, "seq_lens", torch.int64)
    if seq_lens_i32 is not None:
        _need(seq_lens_i32.shape == (B,) and seq_lens_i32.dtype == torch.int32 and seq_lens_i32.is_contiguous(),
              lambda: f"seq_lens_i32 must be a contiguous [{B}] int32 tensor")
    table = torch.empty(B, width, dtype=torch.int32, device=dev)
    rc = _lib.load().sna_block_table(_ptr(req_to_token), req_to_token.shape[0], req_to_token.shape[1],
                                     req_to_token.stride(0), _ptr(rows), _ptr(lens), B, page_size, width, _ptr(table),
                                     _ptr(seq_lens_i32), _stream(dev))
    _lib.check(rc, "block_table")
    return table


def window_blocks(window: int, page_size: int, table_width: int, align_blocks: int = 1) -> int:
    """Table columns a decode row's sliding window of ``window`` keys spans: its window - 1 prior keys and the new
    token's page, rounded up to ``align_blocks``, at most the table's width (model_executor/graph_runner.py:871-882;
    the reference aligns to its Trainium kernel's shard size, which this path does not need: align 1)."""
    _need(window >= 1 and page_size >= 1 and align_blocks >= 1, "window, page_size and align_blocks must be >= 1")
    n = -(-(window - 1) // page_size) + 1
    n = -(-n // align_blocks) * align_blocks
    return min(n, table_width)


def window_table(block_table: Tensor, seq_lens: Tensor, page_size: int, n_blocks: int) -> tuple[Tensor, Tensor]:
    """A sliding-window layer's (trimmed table [B, n_blocks] int32, position offset [B] int32) from the full
    ``block_table`` [B, width] int32 and ``seq_lens`` [B] int64: columns from start_b = max((seq_len_b - 1) // page
    - n_blocks + 1, 0), -1 past the table; offset_b = start_b * page (model_executor/graph_runner.py:1121-1133)."""
    dev = _on_gpu(block_table, seq_lens)
    _need(block_table.dim() == 2 and block_table.dtype == torch.int32 and block_table.stride(1) == 1,
          "block_table must be [B, width] int32 with unit column stride")
    B, width = block_table.shape
    _need(seq_lens.shape == (B,), lambda: f"seq_lens must be [{B}]")
    _need(n_blocks >= 1, "n_blocks must be >= 1")
    lens = _contig(seq_lens, "seq_lens", torch.int64)
    trimmed = torch.empty(B, n_blocks, dtype=torch.int32, device=dev)
    offset = torch.empty(B, dtype=torch.int32, device=dev)
    if B == 0:
        return trimmed, offset
    rc = _lib.load().sna_window_table(_ptr(block_table), block_table.stride(0), width, _ptr(lens), B, page_size,
                                      n_blocks, _ptr(trimmed), _ptr(offset), _stream(dev))
    _lib.check(rc, "window_table")
    return trimmed, offset


def diag_fp8_to_bf16(x: Tensor) -> Tensor:
    """The gathered-page conversion instruction applied to bytes x (uint8): bf16 bits as int16 view."""
    dev = _on_gpu(x)
    x = _contig(x.reshape(-1), "x", torch.uint8)
    out = torch.empty(x.numel(), dtype=torch.int16, device=dev)
    rc = _lib.load().sna_diag_fp8_to_bf16(_ptr(x), _ptr(out), x.numel(), _stream(dev))
    _lib.check(rc, "diag_fp8_to_bf16")
    return out


def default_sm_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


# ------------------------------------------------------------------------------------------------------------------
# page items: what a prefill-decode transfer moves
# ------------------------------------------------------------------------------------------------------------------

def _regions(infos, what: str):
    """Host arrays (ptrs u64, lens i64, item_lens i64) of a pool's get_contiguous_buf_infos() triple."""
    ptrs, lens, items = (list(x) for x in infos)
    _need(len(ptrs) == len(lens) == len(items), lambda: f"{what}: ptrs, lens and item_lens differ in length")
    n = len(ptrs)
    return ((ctypes.c_uint64 * n)(*[int(x) for x in ptrs]), (ctypes.c_int64 * n)(*[int(x) for x in lens]),
            (ctypes.c_int64 * n)(*[int(x) for x in items]), n)


def _pages(pages: Tensor, what: str) -> Tensor:
    _need(pages.dim() == 1, lambda: f"{what}: pages must be 1-D")
    return pages.to(torch.int32).contiguous()


def page_items_wire_bytes(infos, n_pages: int) -> int:
    """Bytes of the wire buffer holding n_pages pages of every region of ``infos`` (a pool's
    get_contiguous_buf_infos(): (ptrs, lens, item_lens), mem_cache/memory_pool.py:193-202)."""
    _, _, items, n = _regions(infos, "page_items_wire_bytes")
    return int(_lib.load().sna_page_items_wire_bytes(items, n, int(n_pages)))


def pack_page_items(infos, pages: Tensor, wire: Optional[Tensor] = None) -> Tensor:
    """The items (region r, pages[i]) of ``infos``'s regions gathered into one uint8 wire buffer, region-major (region
    r's items at n_pages * (item bytes of the regions before r), item i at + i * item_lens[r]); a page outside a
    region packs as zeros. ``pages``: device int tensor [n]."""
    dev = _on_gpu(pages)
    p = _pages(pages, "pack_page_items")
    ptrs, lens, items, n = _regions(infos, "pack_page_items")
    lib = _lib.load()
    need = int(lib.sna_page_items_wire_bytes(items, n, p.numel()))
    if wire is None:
        wire = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    _on_gpu(pages, wire)
    _need(wire.dtype == torch.uint8 and wire.is_contiguous(), "wire must be contiguous uint8")
    rc = lib.sna_page_items_pack(ptrs, lens, items, n, _ptr(p), p.numel(), _ptr(wire), wire.numel(), _stream(dev))
    _lib.check(rc, "page_items_pack")
    return wire[:need]


def unpack_page_items(wire: Tensor, infos, pages: Tensor) -> None:
    """Scatters a wire buffer of pack_page_items' layout into the items (region r, pages[i]) of ``infos``'s regions; a
    page outside a region is skipped. ``pages`` must be distinct."""
    dev = _on_gpu(wire, pages)
    p = _pages(pages, "unpack_page_items")
    _need(wire.dtype == torch.uint8 and wire.is_contiguous(), "wire must be contiguous uint8")
    ptrs, lens, items, n = _regions(infos, "unpack_page_items")
    rc = _lib.load().sna_page_items_unpack(_ptr(wire), wire.numel(), ptrs, lens, items, n, _ptr(p), p.numel(),
                                           _stream(dev))
    _lib.check(rc, "page_items_unpack")


def copy_page_items(src_infos, dst_infos, src_pages: Tensor, dst_pages: Tensor) -> None:
    """The transfer's WRITE list on one GPU: item (r, src_pages[i]) of the source pool's regions to item (r,
    dst_pages[i]) of the destination's (disaggregation/state_transfer.py:9-10), items of the source's item_lens[r]
    bytes (a destination page holding several source items is addressed in source-item units). A page outside its
    region is skipped; ``dst_pages`` must be distinct."""
    dev = _on_gpu(src_pages, dst_pages)
    sp, dp = _pages(src_pages, "copy_page_items"), _pages(dst_pages, "copy_page_items")
    _need(sp.numel() == dp.numel(), "copy_page_items: src_pages and dst_pages differ in length")
    s_ptrs, s_lens, items, n = _regions(src_infos, "copy_page_items")
    d_ptrs, d_lens, _, n_dst = _regions((dst_infos[0], dst_infos[1], src_infos[2]), "copy_page_items")
    _need(n == n_dst, lambda: f"copy_page_items: {n} source regions, {n_dst} destination regions")
    rc = _lib.load().sna_page_items_copy(s_ptrs, s_lens, d_ptrs, d_lens, items, n, _ptr(sp), _ptr(dp), sp.numel(),
                                         _stream(dev))
    _lib.check(rc, "page_items_copy")
