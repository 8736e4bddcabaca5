"""The attention backend: per-forward metadata from SGLang's ForwardBatch, and the decode forward on the HIP path.

Mirrors sglang_neuron/attention/backend.py: ``NeuronForwardMetadata`` (:29-38) and ``NeuronAttnBackend`` (:41-148)
with the same constructor, hooks and ``build_metadata`` / ``_block_table`` semantics. The reference leaves
``forward_decode`` (and ``forward_extend``) to its compiled graphs and raises (:143-148); here they run: the step's
new K/V (or MLA row) is stored at ``out_cache_loc`` when ``save_kv_cache`` is set, then the paged split-K decode (or,
for an extend batch on the MHA pool, the segmented prefill attention) runs over the pool, all on torch's current
stream.

Metadata conventions (attention/backend.py:5-8, :114-130): ``block_table[b, j] = req_to_token[row_b, j * page] //
page`` (int32), -1 where ``j * page >= seq_len_b`` when the batch has more than one row; ``seq_lens`` count the new
token; an idle batch gets a (0, 1) table. Padded rows use seq_len 1 (``get_cuda_graph_seq_len_fill_value``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from .. import _lib, ops
from ..mem_cache.memory_pool import NeuronDSATokenToKVPool, NeuronMHATokenToKVPool, NeuronMLATokenToKVPool


@dataclass
class NeuronForwardMetadata:
    is_prefill: bool
    batch_size: int  # real number of requests
    num_tokens: int  # real number of tokens in this forward
    block_table: Tensor  # [bs, max_blocks] int32 (CPU), -1 padded
    slot_mapping: Tensor  # [num_tokens] int64 (CPU)
    seq_lens: Tensor  # [bs] int64 (CPU) total lens (prefix + new)
    positions: Tensor  # [num_tokens] int64 (CPU)
    cached_seq_len: int = 0


@dataclass
class _DecodeState:
    """The device copies and split-K plans of one decode forward, shared by its layers."""
    meta: NeuronForwardMetadata
    table: Tensor  # [bs, max_blocks] int32, device
    seq_lens: Tensor  # [bs] int32, device
    slots: Tensor  # [bs] int64, device
    positions: Tensor  # [bs] int32, device
    plans: dict
    host_lens: Optional[Tensor] = None  # [bs] host seq_lens when known (exact split plans), else None
    max_len: int = -1  # a bound on seq_lens (plans when host_lens is None)


@dataclass
class _ExtendState:
    """The device copies of one extend forward, shared by its layers."""
    meta: NeuronForwardMetadata
    table: Tensor  # [bs, max_blocks] int32, device
    slots: Tensor  # [T] int64, device
    q_start: Tensor  # [bs + 1] int32, device (a cumsum of the host's extend lengths: 0 first, T last, steps <= max_q_len)
    prior: Tensor  # [bs] int32, device (extend_prefix_lens)
    max_q_len: int


def _real_sizes(fb) -> tuple:
    """(requests, tokens) of a ForwardBatch without the padding SGLang's DP attention adds on the eager path, which
    keeps the real sizes in ``_original_batch_size`` / ``_original_num_tokens`` (attention/backend.py:86-93)."""
    n_req = getattr(fb, "_original_batch_size", None)
    n_tok = getattr(fb, "_original_num_tokens", None)
    return (int(fb.batch_size) if n_req is None else int(n_req),
            int(fb.out_cache_loc.shape[0]) if n_tok is None else int(n_tok))


def _seq_lens_source(fb) -> Tensor:
    """The batch's seq_lens, from its host copy when it carries one."""
    host = getattr(fb, "seq_lens_cpu", None)
    return fb.seq_lens if host is None else host


def _first(t: Tensor, n: int, device) -> Tensor:
    """The first n entries of a batch tensor as int64 on ``device``."""
    return t[:n].to(device=device, dtype=torch.int64)


def _idle_metadata(positions: Tensor, device) -> NeuronForwardMetadata:
    """The metadata of an idle (or empty) batch: no rows, a (0, 1) block table of -1."""
    none = torch.zeros((0,), dtype=torch.long, device=device)
    return NeuronForwardMetadata(is_prefill=False, batch_size=0, num_tokens=0,
                                 block_table=torch.full((0, 1), -1, dtype=torch.int32, device=device),
                                 slot_mapping=none, seq_lens=none.clone(), positions=positions)


def _need_positions_fit(seq_lens: Tensor) -> None:
    """A decode row's length must be in [1, 2^31 - 1]: positions are int32 in the kernels (attention/mla_operands.py:
    73)."""
    lo, hi = int(seq_lens.min()), int(seq_lens.max())
    if lo < 1 or hi > 2 ** 31 - 1:
        raise ValueError(f"decode seq_lens must lie in [1, 2^31 - 1], got [{lo}, {hi}]")


def host_block_table(req_to_token: Tensor, rows: Tensor, seq_lens: Tensor, page_size: int) -> Tensor:
    """The decode block table on the host: [n, ceil(max seq_len / page)] int32 whose column j of row i is the page of
    the row's token j * page (``req_to_token[rows[i], j * page] // page``) while that token lies inside the row
    (j * page < seq_lens[i]), else -1. The reference's NeuronAttnBackend._block_table (attention/backend.py:114-130)
    gives the same entries; ``req_to_token`` is SGLang's [rows, context] int32 map on the CPU."""
    first_token = torch.arange(0, -(-int(seq_lens.max()) // page_size) * page_size, page_size, dtype=torch.int64)
    slots = req_to_token.index_select(0, rows.to(torch.int64)).index_select(1, first_token)
    table = torch.div(slots, page_size, rounding_mode="floor").to(torch.int32)
    table.masked_fill_(first_token.unsqueeze(0) >= seq_lens.to(torch.int64).unsqueeze(1), -1)
    return table.contiguous()


class NeuronAttnBackend:
    """The attention backend of the HIP decode path. ``model_runner`` provides ``req_to_token_pool`` (with
    ``req_to_token`` [rows, context] int32), ``token_to_kv_pool`` (one of this package's pools) and ``page_size``.

    With req_to_token on the host (the reference's arrangement) a decode forward's metadata is built as the
    reference builds it (``build_metadata``) and uploaded once per forward. With req_to_token on the GPU (SGLang's
    own arrangement there) it is built on the device (``build_device_metadata``): the block table by a gather
    kernel, nothing read back; only the batch's longest length is taken from ``seq_lens_cpu`` when the batch carries
    it, to size the table and plan the splits exactly."""

    def __init__(self, model_runner):
        self.model_runner = model_runner
        self.req_to_token_pool = model_runner.req_to_token_pool
        self.token_to_kv_pool = model_runner.token_to_kv_pool
        self.page_size = int(model_runner.page_size)

    # SGLang's hooks: the metadata's consumers build it themselves (attention/backend.py:56-76)
    def init_forward_metadata(self, forward_batch):
        return None

    def init_forward_metadata_out_graph(self, forward_batch, in_capture: bool = False):
        return None

    def init_forward_metadata_in_graph(self, forward_batch):
        return None

    def init_cuda_graph_state(self, max_bs: int, max_num_tokens: int):
        return None

    def get_cpu_graph_seq_len_fill_value(self) -> int:
        return self.get_cuda_graph_seq_len_fill_value()

    def get_cuda_graph_seq_len_fill_value(self) -> int:
        # padded (idle) rows: seq_len 1, so req_to_token[0, 0] (the reserved page) is read
        return 1

    def build_metadata(self, fb) -> NeuronForwardMetadata:
        """Exact (unpadded) host metadata of a ForwardBatch, the reference's NeuronForwardMetadata semantics
        (attention/backend.py:29-40, 78-112): the batch's real requests and tokens only, CPU int64 seq_lens /
        slot_mapping / positions, and the block table of ``host_block_table``. An idle batch gets a (0, 1) table."""
        n_req, n_tok = _real_sizes(fb)
        positions = _first(fb.positions, n_tok, "cpu")
        if fb.forward_mode.is_idle() or n_req == 0:
            return _idle_metadata(positions[:0], torch.device("cpu"))
        lens = _first(_seq_lens_source(fb), n_req, "cpu")
        extend = bool(fb.forward_mode.is_extend())
        slots = _first(fb.out_cache_loc, n_tok, "cpu")
        table = host_block_table(self.req_to_token_pool.req_to_token, _first(fb.req_pool_indices, n_req, "cpu"), lens,
                                 self.page_size)
        return NeuronForwardMetadata(
            is_prefill=extend, batch_size=n_req, num_tokens=int(slots.numel()), block_table=table, slot_mapping=slots,
            seq_lens=lens, positions=positions,
            cached_seq_len=int(fb.extend_prefix_lens[:n_req].max()) if extend else 0)

    def build_device_metadata(self, fb, device: torch.device) -> NeuronForwardMetadata:
        """A batch's metadata with req_to_token on the GPU, built there: ``block_table`` [bs, width] int32 by
        ``ops.block_table`` (the reference's _block_table, attention/backend.py:114-130, entry for entry when width
        is the longest row's page count), ``slot_mapping`` / ``seq_lens`` / ``positions`` as device views of the
        batch's own tensors. ``width`` is ceil(max seq_len / page) from ``seq_lens_cpu`` when the batch has it, else
        req_to_token's context width in pages (a bound)."""
        n_req, n_tok = _real_sizes(fb)
        if fb.forward_mode.is_idle() or n_req == 0:
            return _idle_metadata(torch.zeros((0,), dtype=torch.long, device=device), device)
        r2t = self.req_to_token_pool.req_to_token
        page = self.page_size
        lens_cpu = getattr(fb, "seq_lens_cpu", None)
        longest = int(lens_cpu[:n_req].max()) if lens_cpu is not None else int(r2t.shape[1])
        lens = _first(fb.seq_lens, n_req, device)
        table = ops.block_table(r2t, _first(fb.req_pool_indices, n_req, device), lens, page,
                                max(1, -(-longest // page)))
        return NeuronForwardMetadata(
            is_prefill=bool(fb.forward_mode.is_extend()), batch_size=n_req, num_tokens=n_tok, block_table=table,
            slot_mapping=_first(fb.out_cache_loc, n_tok, device), seq_lens=lens,
            positions=_first(fb.positions, n_tok, device))

    # ---- decode ----
    def _decode_state(self, fb, device: torch.device) -> _DecodeState:
        st = getattr(fb, "_sna_decode_state", None)
        if st is not None and st.table.device == device:
            return st
        on_device = self.req_to_token_pool.req_to_token.is_cuda
        meta = self.build_device_metadata(fb, device) if on_device else self.build_metadata(fb)
        if meta.is_prefill:
            raise NotImplementedError("forward_decode got an extend batch: this build runs the decode path only")
        if meta.num_tokens != meta.batch_size:
            raise ValueError(f"a decode batch has one new token per row ({meta.num_tokens} tokens, {meta.batch_size} "
                             "rows)")
        if on_device:
            # the operands live on the device: only the host lengths (when the batch carries them) are checked
            lens_cpu = getattr(fb, "seq_lens_cpu", None)
            host_lens = lens_cpu[:meta.batch_size].to(torch.long) if lens_cpu is not None else None
            max_len = meta.block_table.shape[1] * self.page_size
            if host_lens is not None and meta.batch_size:
                _need_positions_fit(host_lens)
        else:
            host_lens, max_len = meta.seq_lens, -1
            if meta.batch_size:
                ops.check_decode_operands(meta.seq_lens, meta.block_table, meta.slot_mapping, self.page_size,
                                          int(self.token_to_kv_pool.num_blocks))
        st = _DecodeState(meta=meta, table=meta.block_table.to(device), seq_lens=meta.seq_lens.to(device, torch.int32),
                          slots=meta.slot_mapping.to(device), positions=meta.positions.to(device, torch.int32),
                          plans={}, host_lens=host_lens, max_len=max_len)
        try:
            fb._sna_decode_state = st
        except AttributeError:
            pass
        return st

    def _extend_state(self, fb, device: torch.device) -> _ExtendState:
        st = getattr(fb, "_sna_extend_state", None)
        if st is not None and st.table.device == device:
            return st
        on_device = self.req_to_token_pool.req_to_token.is_cuda
        meta = self.build_device_metadata(fb, device) if on_device else self.build_metadata(fb)
        if not meta.is_prefill:
            raise ValueError("forward_extend got a batch that is not an extend batch")
        bs = meta.batch_size
        ext_cpu = getattr(fb, "extend_seq_lens_cpu", None)
        ext = torch.as_tensor(ext_cpu if ext_cpu is not None else fb.extend_seq_lens.cpu(), dtype=torch.long)[:bs]
        prefix = torch.as_tensor(fb.extend_prefix_lens, device=device).to(torch.int32)[:bs]
        if int(ext.sum()) != meta.num_tokens:
            raise ValueError(f"extend lengths sum to {int(ext.sum())}, the batch has {meta.num_tokens} tokens")
        q_start = torch.zeros(bs + 1, dtype=torch.int32)
        q_start[1:] = torch.cumsum(ext, 0)
        st = _ExtendState(meta=meta, table=meta.block_table.to(device), slots=meta.slot_mapping.to(device),
                          q_start=q_start.to(device), prior=prefix, max_q_len=int(ext.max()) if bs else 0)
        try:
            fb._sna_extend_state = st
        except AttributeError:
            pass
        return st

    def forward_extend(self, q: Tensor, k: Optional[Tensor], v: Optional[Tensor], layer, forward_batch,
                       save_kv_cache: bool = True, **kwargs) -> Tensor:
        """An extend (prefill) step of ``layer`` on the MHA pool: the chunk's K/V [T, G * d] stored at
        ``out_cache_loc`` (when ``save_kv_cache``), then segmented prefill attention (ops.prefill_attention): request
        r's ``extend_seq_lens[r]`` new tokens, at positions ``extend_prefix_lens[r] + i``, attend to its prior and
        causally to themselves, every key read from the pool. q [T, H * d] or [T, H, d]; ``layer`` as in
        forward_decode (window, sinks). Returns [T, H * d] bf16. The reference leaves extend to its compiled graphs
        and raises (attention/backend.py:143-145). FP8 and bf16 pools."""
        if q.device.type != "cuda":
            raise RuntimeError("forward_extend runs on the GPU (there is no CPU path)")
        pool = self.token_to_kv_pool
        if not isinstance(pool, NeuronMHATokenToKVPool):
            raise NotImplementedError(f"forward_extend runs on the MHA pool, not {type(pool).__name__}")
        st = self._extend_state(forward_batch, q.device)
        T = st.meta.num_tokens
        layer_id = int(layer.layer_id)
        H, G = int(layer.tp_q_head_num), int(layer.tp_k_head_num)
        d = int(getattr(layer, "head_dim", pool.head_dim))
        if G != pool.head_num or d != pool.head_dim:
            raise ValueError(f"layer {layer_id} has {G} KV heads of {d}, the pool {pool.head_num} of {pool.head_dim}")
        window = getattr(layer, "sliding_window_size", None)
        window = int(window) if window is not None and int(window) > 0 else 0
        sinks = kwargs.get("sinks")
        if sinks is None:
            sinks = getattr(layer, "sinks", None)
        if save_kv_cache:
            pool.set_kv_buffer_prefill(layer, st.slots, k.reshape(T, G, d), v.reshape(T, G, d))
        k_cache, v_cache = pool.get_kv_buffer(layer_id)
        k_scale, v_scale = pool.get_kv_scales(layer_id)
        out = ops.prefill_attention(q.reshape(T, H, d), k_cache, v_cache, st.table, st.q_start, st.prior,
                                    max_q_len=st.max_q_len, sm_scale=float(layer.scaling), k_scale=k_scale,
                                    v_scale=v_scale, sinks=sinks, window=window,
                                    scales_multiply=pool.kv_scales_inverted(layer_id))
        return out.reshape(T, H * d)

    def forward_decode(self, q: Tensor, k: Optional[Tensor], v: Optional[Tensor], layer, forward_batch,
                       save_kv_cache: bool = True, **kwargs) -> Tensor:
        """One decode step of ``layer``: the new K/V of every row stored at ``out_cache_loc`` (when ``save_kv_cache``)
        and attended in-band, the history read from the pool through the block table.

        GQA (MHA pool): q [bs, H * d] or [bs, H, d], k / v [bs, G * d] or [bs, G, d]; ``layer`` gives ``layer_id``,
        ``tp_q_head_num``, ``tp_k_head_num``, ``head_dim``, ``scaling`` and optionally ``sliding_window_size`` (> 0:
        a window of that many keys, the new one included) and ``sinks`` [H] (or the ``sinks`` keyword). Returns
        [bs, H * d] bf16.

        MLA (MLA pool): q [bs, H, 576] absorbed ([q_nope W_uk 512 | q_pe 64]), k the new compact rows [bs, 576]
        ([latent | rope]); v is unused. Returns [bs, H * 512] bf16.

        DSA (DSA pool): as MLA with k the new rows in [k_pe | latent] order and the ``topk_indices`` keyword [bs, K]
        int32 (global positions, -1 empty). Returns [bs, H * 512] bf16; the LSE [bs, H] is kept in
        ``self.last_lse``."""
        if q.device.type != "cuda":
            raise RuntimeError("forward_decode runs on the GPU (there is no CPU path)")
        pool = self.token_to_kv_pool
        st = self._decode_state(forward_batch, q.device)
        bs = st.meta.batch_size
        layer_id = int(layer.layer_id)
        if isinstance(pool, NeuronMHATokenToKVPool):
            return self._decode_gqa(q, k, v, layer, layer_id, st, bs, save_kv_cache, kwargs.get("sinks"))
        if isinstance(pool, NeuronMLATokenToKVPool):
            return self._decode_mla(q, k, layer, layer_id, st, bs, save_kv_cache)
        if isinstance(pool, NeuronDSATokenToKVPool):
            return self._decode_dsa(q, k, layer, layer_id, st, bs, save_kv_cache, kwargs.get("topk_indices"))
        raise TypeError(f"unsupported KV pool {type(pool).__name__}")

    def _decode_gqa(self, q, k, v, layer, layer_id, st, bs, save, sinks):
        pool: NeuronMHATokenToKVPool = self.token_to_kv_pool
        H, G = int(layer.tp_q_head_num), int(layer.tp_k_head_num)
        d = int(getattr(layer, "head_dim", pool.head_dim))
        if G != pool.head_num or d != pool.head_dim:
            raise ValueError(f"layer {layer_id} has {G} KV heads of {d}, the pool {pool.head_num} of {pool.head_dim}")
        window = getattr(layer, "sliding_window_size", None)
        window = int(window) if window is not None and int(window) > 0 else 0
        if sinks is None:
            sinks = getattr(layer, "sinks", None)
        key = ("gqa", window, G)
        if key not in st.plans:
            st.plans[key] = ops.plan_decode(_lib.KIND_GQA, bs, host_seq_lens=st.host_lens, max_seq_len=st.max_len,
                                            window=window, ctas_per_item=G, num_cus=ops._num_cus(q.device))
        k_cache, v_cache = pool.get_kv_buffer(layer_id)
        k_scale, v_scale = pool.get_kv_scales(layer_id)
        fp8 = pool.store_dtype == ops.FP8
        out = ops.paged_decode_gqa(
            q.reshape(bs, H, d), k_cache, v_cache, st.table, st.seq_lens, k.reshape(bs, G, d), v.reshape(bs, G, d),
            sm_scale=float(layer.scaling), k_scale=k_scale if fp8 else None, v_scale=v_scale if fp8 else None,
            sinks=sinks, window=window, new_slots=st.slots if save else None, plan=st.plans[key],
            scales_multiply=fp8 and pool.kv_scales_inverted(layer_id))
        return out.reshape(bs, H * d)

    def _decode_mla(self, q, k, layer, layer_id, st, bs, save):
        pool: NeuronMLATokenToKVPool = self.token_to_kv_pool
        H = int(layer.tp_q_head_num)
        q = q.reshape(bs, H, 576)
        key = ("mla", H)
        if key not in st.plans:
            # exact plans from host lengths; without a host copy, a device split bounded by the table's width (the
            # launch reads the device's lengths, nothing is read back)
            chunks = ops.stream_row_chunks(_lib.KIND_MLA, bs, H)
            bound = st.table.shape[1] * pool.page_size
            plans = [ops.plan_decode(_lib.KIND_MLA, r1 - r0,
                                     host_seq_lens=None if st.host_lens is None else st.host_lens[r0:r1],
                                     max_seq_len=bound, ctas_per_item=(H + 15) // 16, num_cus=ops._num_cus(q.device))
                     for r0, r1 in chunks]
            ws = ops.stream_workspace(max(plans, key=lambda p: ops.workspace_bytes(p, H, 512)), H, q.device)
            st.plans[key] = (plans, ws)
        plans, ws = st.plans[key]
        out = ops.mla_decode(
            q[..., :512], q[..., 512:], pool.get_key_buffer(layer_id), pool.get_row_scale(layer_id), st.table,
            st.seq_lens, k.reshape(bs, 576), sm_scale=float(layer.scaling), page_size=pool.page_size,
            new_slots=st.slots if save else None, plan=plans, workspace=ws, host_seq_lens=st.host_lens)
        return out.reshape(bs, H * 512)

    def _decode_dsa(self, q, k, layer, layer_id, st, bs, save, topk_indices):
        pool: NeuronDSATokenToKVPool = self.token_to_kv_pool
        if topk_indices is None:
            raise ValueError("a DSA decode needs topk_indices [bs, K]")
        H = int(layer.tp_q_head_num)
        q = q.reshape(bs, H, 576)
        idx = topk_indices.reshape(bs, -1)
        key = ("dsa", H, idx.shape[1])
        if key not in st.plans:
            chunks = ops.stream_row_chunks(_lib.KIND_DSA, bs, H, idx.shape[1])
            plans = [ops.plan_decode(_lib.KIND_DSA, r1 - r0, n_keys_per_row=idx.shape[1], ctas_per_item=(H + 15) // 16,
                                     num_cus=ops._num_cus(q.device)) for r0, r1 in chunks]
            ws = ops.stream_workspace(max(plans, key=lambda p: ops.workspace_bytes(p, H, 512)), H, q.device)
            st.plans[key] = (plans, ws)
        plans, ws = st.plans[key]
        ctx, lse = ops.mla_decode_sparse(
            q[..., :512], q[..., 512:], pool.get_key_buffer(layer_id), pool.get_kv_scale(layer_id), idx, st.table,
            st.positions, k.reshape(bs, 576), sm_scale=float(layer.scaling), page_size=pool.page_size,
            new_slots=st.slots if save else None, plan=plans, workspace=ws)
        self.last_lse = lse
        return ctx.reshape(bs, H * 512)
