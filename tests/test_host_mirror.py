"""The host-side mirror of the reference's KV pool and attention backend, on the CPU: metadata semantics checked by
brute force, pool shapes and bookkeeping, refusals, and that nothing computes without the GPU path."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from sglang_neuron_amd import ops
from sglang_neuron_amd.attention import NeuronAttnBackend
from sglang_neuron_amd.mem_cache import NeuronDSATokenToKVPool, NeuronMHATokenToKVPool, NeuronMLATokenToKVPool


class _Mode:
    def __init__(self, kind: str):
        self.kind = kind

    def is_extend(self):
        return self.kind == "extend"

    def is_idle(self):
        return self.kind == "idle"

    def is_decode(self):
        return self.kind == "decode"


def _runner(req_to_token: torch.Tensor, pool, page: int):
    return SimpleNamespace(req_to_token_pool=SimpleNamespace(req_to_token=req_to_token), token_to_kv_pool=pool,
                           page_size=page)


def _batch(rows, lens, mode="decode", slots=None):
    lens = torch.as_tensor(lens, dtype=torch.int64)
    bs = len(lens)
    slots = torch.arange(bs, dtype=torch.int64) if slots is None else torch.as_tensor(slots)
    return SimpleNamespace(forward_mode=_Mode(mode), batch_size=bs, req_pool_indices=torch.as_tensor(rows),
                           seq_lens=lens, seq_lens_cpu=lens, out_cache_loc=slots, positions=lens - 1,
                           extend_prefix_lens=torch.zeros(bs, dtype=torch.int64))


def _brute_table(r2t: np.ndarray, rows, lens, page: int) -> np.ndarray:
    """block_table[b, j] = req_to_token[row_b, j * page] // page while j * page < len_b, else -1 (one row: no -1)."""
    width = (max(lens) + page - 1) // page
    out = np.empty((len(rows), width), dtype=np.int64)
    for b, (r, L) in enumerate(zip(rows, lens)):
        for j in range(width):
            live = j * page < L or len(rows) == 1
            out[b, j] = r2t[r, j * page] // page if live else -1
    return out


@pytest.mark.parametrize("page,lens", [(16, [1, 17, 64, 300]), (64, [1000, 5]), (16, [33]), (1, [3, 9, 2])])
def test_block_table_matches_brute_force(page, lens):
    g = torch.Generator().manual_seed(7)
    rows = [3, 0, 5, 1][:len(lens)]
    ctx = 1024
    r2t = torch.randint(0, 1 << 20, (8, ctx), generator=g, dtype=torch.int32)
    backend = NeuronAttnBackend(_runner(r2t, None, page))
    meta = backend.build_metadata(_batch(rows, lens))
    want = _brute_table(r2t.numpy(), rows, lens, page)
    assert meta.block_table.dtype == torch.int32
    assert np.array_equal(meta.block_table.numpy(), want)
    assert meta.batch_size == len(lens) and meta.num_tokens == len(lens)
    assert meta.seq_lens.tolist() == lens and meta.positions.tolist() == [L - 1 for L in lens]
    assert not meta.is_prefill


def test_idle_batch_metadata():
    backend = NeuronAttnBackend(_runner(torch.zeros(2, 16, dtype=torch.int32), None, 16))
    meta = backend.build_metadata(_batch([0], [1], mode="idle"))
    assert meta.batch_size == 0 and meta.num_tokens == 0
    assert tuple(meta.block_table.shape) == (0, 1) and meta.block_table.dtype == torch.int32
    assert backend.get_cuda_graph_seq_len_fill_value() == 1
    assert backend.init_forward_metadata(None) is None


def test_block_table_follows_in_place_req_to_token_writes():
    r2t = torch.zeros(2, 64, dtype=torch.int32)
    backend = NeuronAttnBackend(_runner(r2t, None, 16))
    fb = _batch([1], [20])
    assert backend.build_metadata(fb).block_table.tolist() == [[0, 0]]
    r2t[1, 0] = 5 * 16
    r2t[1, 16] = 9 * 16 + 3
    assert backend.build_metadata(fb).block_table.tolist() == [[5, 9]]


def test_mha_pool_shapes_and_bookkeeping():
    pool = NeuronMHATokenToKVPool(size=128, page_size=16, dtype=torch.float8_e4m3fn, head_num=4, head_dim=64,
                                  layer_num=3, device="cpu", start_layer=2)
    assert pool.num_blocks == 128 // 16 + 1
    k_shape, v_shape = pool.get_kv_buffer_shape()
    assert k_shape == v_shape == torch.Size((9, 4, 16, 64))
    assert not pool.fp8_packed_k and pool.kv_head_major
    k, v = pool.get_kv_buffer(3)
    assert k.dtype == torch.float8_e4m3fn and tuple(k.shape) == tuple(k_shape)
    assert pool.get_kv_size_bytes() == 9 * 4 * 16 * 64 * 1 * 2 * 3
    ptrs, lens, items = pool.get_contiguous_buf_infos()
    assert len(ptrs) == len(lens) == len(items) == 6
    assert lens == [9 * 4 * 16 * 64] * 6 and items == [4 * 16 * 64] * 6
    assert pool.get_kv_layer_ids() == [2, 3, 4, 2, 3, 4]
    ks, vs = pool.get_kv_scales(4)
    assert ks.tolist() == [1.0] * 4 and vs.tolist() == [1.0] * 4
    pool.set_kv_scales(4, 0.5, torch.tensor([1.0, 2.0, 3.0, 4.0]))
    assert pool.get_kv_scales(4)[0].tolist() == [0.5] * 4 and pool.get_kv_scales(4)[1].tolist() == [1, 2, 3, 4]
    with pytest.raises(IndexError):
        pool.get_key_buffer(5)


@pytest.mark.parametrize("kw", [{"quant_method": "fp8"}, {"kv_cache_layout": "NHD"}, {"v_head_dim": 32},
                                {"enable_kv_cache_copy": True}])
def test_mha_pool_refuses_options_it_does_not_have(kw):
    with pytest.raises(ValueError):
        NeuronMHATokenToKVPool(64, 16, torch.bfloat16, 2, 64, 1, "cpu", **kw)


def test_mha_pool_refuses_bad_sizes_and_dtypes():
    with pytest.raises(ValueError):
        NeuronMHATokenToKVPool(60, 16, torch.bfloat16, 2, 64, 1, "cpu")
    with pytest.raises(ValueError):
        NeuronMHATokenToKVPool(64, 16, torch.float16, 2, 64, 1, "cpu")
    with pytest.raises(ValueError):
        NeuronMHATokenToKVPool(64, 16, torch.bfloat16, 2, 64, 1, "cpu", enable_memory_saver=True)


def test_mla_pool_shapes_and_views():
    pool = NeuronMLATokenToKVPool(256, 64, torch.float8_e4m3fn, 512, 64, 2, "cpu")
    assert pool.num_blocks == 5
    assert tuple(pool.kv_buffer[0].shape) == (256 + 64, 1, 576) and pool.kv_buffer[0].dtype == torch.uint8
    blk = pool.get_block_buffer(1)
    assert tuple(blk.shape) == (5, 64, 576) and blk.data_ptr() == pool.kv_buffer[1].data_ptr()
    assert tuple(pool.get_value_buffer(0).shape) == (320, 1, 512)
    assert tuple(pool.get_row_scale(0).shape) == (320,)
    ptrs, lens, items = pool.get_contiguous_buf_infos()
    assert lens == [320 * 576] * 2 and items == [576 * 64] * 2
    for bad in ({"dtype": torch.float16}, {"page_size": 8}):
        args = dict(size=256, page_size=64, dtype=torch.float8_e4m3fn, kv_lora_rank=512, qk_rope_head_dim=64,
                    layer_num=1, device="cpu")
        args.update(bad)
        with pytest.raises(ValueError):
            NeuronMLATokenToKVPool(**args)
    with pytest.raises(ValueError):
        NeuronMLATokenToKVPool(256, 64, torch.float8_e4m3fn, 512, 64, 1, "cpu", use_dsa=True)


def test_mla_pool_bf16_rows():
    """bf16 rows as the reference's DeepSeek-V2 pool holds them: no row scales, 1152-byte rows."""
    pool = NeuronMLATokenToKVPool(256, 128, torch.bfloat16, 512, 64, 2, "cpu")
    assert pool.kv_buffer[0].dtype == torch.bfloat16 and tuple(pool.kv_buffer[0].shape) == (256 + 128, 1, 576)
    assert pool.get_row_scale(0) is None and pool.get_scale_buf_infos() == ([], [], [])
    ptrs, lens, items = pool.get_contiguous_buf_infos()
    assert lens == [384 * 1152] * 2 and items == [1152 * 128] * 2
    assert pool.get_kv_size_bytes() == 2 * 384 * 1152


def test_dsa_pool_shapes():
    pool = NeuronDSATokenToKVPool(128, 64, 2, "cpu", kv_scale=2.0 ** -6)
    assert tuple(pool.get_key_buffer(1).shape) == (3, 1, 64, 640)
    assert pool.get_kv_scale(0) == 2.0 ** -6


def test_no_cpu_compute_path():
    """Writes and decodes refuse CPU tensors: the HIP path is the only one."""
    pool = NeuronMHATokenToKVPool(64, 16, torch.bfloat16, 2, 64, 1, "cpu")
    k = torch.zeros(3, 2, 64, dtype=torch.bfloat16)
    with pytest.raises((ValueError, RuntimeError)):
        pool.set_kv_buffer(0, torch.arange(3), k, k)
    backend = NeuronAttnBackend(_runner(torch.zeros(2, 64, dtype=torch.int32), pool, 16))
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=4, tp_k_head_num=2, head_dim=64, scaling=0.125)
    with pytest.raises(RuntimeError):
        backend.forward_decode(torch.zeros(1, 4 * 64, dtype=torch.bfloat16), k[:1], k[:1], layer, _batch([0], [5]))


@pytest.mark.parametrize("page", [1, 4, 16, 64])
@pytest.mark.parametrize("window", [1, 2, 15, 16, 17, 128, 1000])
def test_window_blocks_cover_every_window_and_no_more(window, page):
    """ops.window_blocks (graph_runner.py:871-882 without the Trainium alignment): the window's keys [L - W, L - 1]
    of any row fall in the trimmed table's columns (start = (L - 1) // page - nb + 1), and some row needs all nb of
    them; by brute force over L."""
    nb = ops.window_blocks(window, page, 10**6)
    need = 0
    for L in range(1, 3 * window + 4 * page):
        first, last = max(L - window, 0) // page, (L - 1) // page
        start = max((L - 1) // page - nb + 1, 0)
        assert start <= first and last <= start + nb - 1, (L, first, last, start, nb)
        need = max(need, last - first + 1)
    assert need == nb
    assert ops.window_blocks(window, page, 3) == min(nb, 3)
    assert ops.window_blocks(window, page, 10**6, align_blocks=4) == -(-nb // 4) * 4


def test_device_metadata_refuses_cpu_tensors():
    r2t = torch.zeros(4, 64, dtype=torch.int32)
    with pytest.raises(ValueError):
        ops.block_table(r2t, torch.arange(2), torch.tensor([3, 5]), 16, 4)
    with pytest.raises(ValueError):
        ops.window_table(torch.zeros(2, 4, dtype=torch.int32), torch.tensor([3, 5]), 16, 2)
