"""The decode step through the reference-shaped interface (pool set_kv_buffer + backend forward_decode) against the
CPU oracle: outputs within the attention bar, pools bit-exact after the step."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from conftest import announce
from _harness import assert_close_attn, dsa_oracle, gqa_oracle, mla_oracle
from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import store as ost
from sglang_neuron_amd import workloads
from sglang_neuron_amd.attention import NeuronAttnBackend
from sglang_neuron_amd.mem_cache import NeuronDSATokenToKVPool, NeuronMHATokenToKVPool, NeuronMLATokenToKVPool

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Decode:
    def is_extend(self):
        return False

    def is_idle(self):
        return False


def _req_to_token(table: torch.Tensor, lens, page: int) -> torch.Tensor:
    """req_to_token [B, context] of the case's pages: slot of (b, pos) = table[b, pos // page] * page + pos % page."""
    B = table.shape[0]
    ctx = table.shape[1] * page
    pos = torch.arange(ctx)
    r2t = table.to(torch.int64).clamp(min=0)[:, pos // page] * page + pos % page
    return r2t.to(torch.int32).reshape(B, ctx)


def _backend(pool, table, lens, page, device_r2t=False):
    r2t = _req_to_token(table, lens, page)
    runner = SimpleNamespace(req_to_token_pool=SimpleNamespace(req_to_token=r2t.to(DEV) if device_r2t else r2t),
                             token_to_kv_pool=pool, page_size=page)
    return NeuronAttnBackend(runner)


def _batch(lens, new_slots, positions=None, host_lens=True):
    lens = lens.to(torch.int64)
    B = lens.numel()
    return SimpleNamespace(forward_mode=_Decode(), batch_size=B, req_pool_indices=torch.arange(B), seq_lens=lens.to(DEV),
                           seq_lens_cpu=lens if host_lens else None, out_cache_loc=new_slots.to(DEV),
                           positions=(lens - 1 if positions is None else positions).to(DEV), extend_prefix_lens=None)


GQA = [("cfg1", 1, {}), ("cfg2-small", 2, {"B": 4, "lens": (100, 700)}),
       ("cfg4-sinks", 4, {"B": 6, "lens": (30, 600)}), ("cfg4-swa", 4, {"B": 5, "lens": (10, 500), "window": 128})]


@pytest.mark.parametrize("name,cfg,over", GQA, ids=[g[0] for g in GQA])
def test_backend_gqa_decode(name, cfg, over):
    case = workloads.gqa_case(cfg, overrides=over)
    want, kc_o, vc_o, ks_o, vs_o = gqa_oracle(case)
    announce(f"backend gqa {name}: B={case.B} H={case.H} G={case.G} d={case.d} fp8={case.fp8}")
    dtype = torch.float8_e4m3fn if case.fp8 else torch.bfloat16
    pool = NeuronMHATokenToKVPool(size=(case.num_blocks - 1) * case.P, page_size=case.P, dtype=dtype,
                                  head_num=case.G, head_dim=case.d, layer_num=2, device=DEV)
    layer = SimpleNamespace(layer_id=1, tp_q_head_num=case.H, tp_k_head_num=case.G, head_dim=case.d,
                            scaling=case.sm_scale, sliding_window_size=case.window if case.window else -1,
                            sinks=None if case.sinks is None else case.sinks.to(DEV))
    if case.fp8:
        # cfg4: the GPT-OSS model's inverted scales (the layer's decode multiplies by them)
        pool.calibrate_kv_scales(1, torch.cat([case.k_prior, case.k_new]).to(DEV),
                                 torch.cat([case.v_prior, case.v_new]).to(DEV), inverted=case.scales_multiply)
        assert pool.kv_scales_inverted(1) == case.scales_multiply
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.k_prior.to(DEV), case.v_prior.to(DEV))
    backend = _backend(pool, case.block_table, case.seq_lens, case.P)
    fb = _batch(case.seq_lens, case.new_slots)
    out = backend.forward_decode(case.q.reshape(case.B, -1).to(DEV), case.k_new.to(DEV), case.v_new.to(DEV), layer, fb)
    torch.cuda.synchronize()
    assert out.shape == (case.B, case.H * case.d)
    assert_close_attn(out.reshape(case.B, case.H, case.d), want, name)
    k, v = pool.get_kv_buffer(1)
    assert torch.equal(k.cpu().view(torch.uint8), kc_o.view(torch.uint8)), "K pool differs"
    assert torch.equal(v.cpu().view(torch.uint8), vc_o.view(torch.uint8)), "V pool differs"
    if case.fp8:
        ks, vs = pool.get_kv_scales(1)
        assert torch.equal(ks.cpu(), ks_o) and torch.equal(vs.cpu(), vs_o), "scales differ"


def test_backend_gqa_decode_without_save_leaves_pool():
    case = workloads.gqa_case(2, overrides={"B": 3, "lens": (50, 200)})
    want, *_ = gqa_oracle(case)
    announce("backend gqa no-save")
    pool = NeuronMHATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, case.G, case.d, 1, DEV)
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, tp_k_head_num=case.G, head_dim=case.d,
                            scaling=case.sm_scale)
    pool.calibrate_kv_scales(0, torch.cat([case.k_prior, case.k_new]).to(DEV),
                             torch.cat([case.v_prior, case.v_new]).to(DEV))
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.k_prior.to(DEV), case.v_prior.to(DEV))
    before = pool.get_key_buffer(0).clone()
    backend = _backend(pool, case.block_table, case.seq_lens, case.P)
    out = backend.forward_decode(case.q.to(DEV), case.k_new.to(DEV), case.v_new.to(DEV), layer,
                                 _batch(case.seq_lens, case.new_slots), save_kv_cache=False)
    torch.cuda.synchronize()
    assert_close_attn(out.reshape(case.B, case.H, case.d), want, "no-save")
    assert torch.equal(pool.get_key_buffer(0).view(torch.uint8), before.view(torch.uint8))


def test_backend_mla_decode():
    case = workloads.mla_case(overrides={"B": 4, "lens": (1, 3000)})
    want, cache_o, scale_o = mla_oracle(case)
    announce(f"backend mla: B={case.B} lens={case.seq_lens.tolist()}")
    pool = NeuronMLATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, 512, 64, 1, DEV)
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, scaling=case.sm_scale)
    T = case.prior_slots.numel()
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.prior_rows.reshape(T, 1, 576).to(DEV))
    backend = _backend(pool, case.block_table, case.seq_lens, case.P)
    q = torch.cat([case.ql_nope, case.q_pe], dim=-1).to(DEV)
    out = backend.forward_decode(q, case.compact_new.to(DEV), None, layer, _batch(case.seq_lens, case.new_slots))
    torch.cuda.synchronize()
    assert_close_attn(out.reshape(case.B, case.H, 512), want, "mla")
    assert torch.equal(pool.kv_buffer[0].cpu().reshape(-1, 576), cache_o), "row pool differs"
    written = torch.cat([case.prior_slots, case.new_slots])
    assert torch.equal(pool.row_scale[0].cpu()[written], scale_o[written]), "row scales differ"


def test_backend_mla_decode_bf16_pool():
    """The reference's DeepSeek-V2 serving pool: bf16 rows at page 128 (models/catalog.py:230-231)."""
    case = workloads.mla_case(overrides={"B": 4, "P": 128, "lens": (1, 3000)})
    want, cache_o, _ = mla_oracle(case, bf16=True)
    announce(f"backend mla bf16: B={case.B} lens={case.seq_lens.tolist()}")
    pool = NeuronMLATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.bfloat16, 512, 64, 1, DEV)
    assert pool.get_row_scale(0) is None and pool.get_scale_buf_infos() == ([], [], [])
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, scaling=case.sm_scale)
    T = case.prior_slots.numel()
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.prior_rows.reshape(T, 1, 576).to(DEV))
    backend = _backend(pool, case.block_table, case.seq_lens, case.P)
    q = torch.cat([case.ql_nope, case.q_pe], dim=-1).to(DEV)
    out = backend.forward_decode(q, case.compact_new.to(DEV), None, layer, _batch(case.seq_lens, case.new_slots))
    torch.cuda.synchronize()
    assert_close_attn(out.reshape(case.B, case.H, 512), want, "mla bf16")
    assert torch.equal(pool.kv_buffer[0].cpu().reshape(-1, 576).view(torch.int16), cache_o.view(torch.int16)), \
        "row pool differs"


def test_backend_mla_set_mla_kv_buffer_matches_full_rows():
    case = workloads.mla_case(overrides={"B": 2, "lens": (40, 90)})
    announce("backend mla set_mla_kv_buffer")
    T = case.prior_slots.numel()
    a = NeuronMLATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, 512, 64, 1, DEV)
    b = NeuronMLATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, 512, 64, 1, DEV)
    rows = case.prior_rows.to(DEV)
    a.set_kv_buffer(0, case.prior_slots.to(DEV), rows.reshape(T, 1, 576))
    b.set_mla_kv_buffer(0, case.prior_slots.to(DEV), rows[:, :512].reshape(T, 1, 512), rows[:, 512:].reshape(T, 1, 64))
    torch.cuda.synchronize()
    assert torch.equal(a.kv_buffer[0], b.kv_buffer[0]) and torch.equal(a.row_scale[0], b.row_scale[0])


def test_backend_dsa_decode():
    case = workloads.dsa_case(overrides={"B": 3, "pool_positions": 2048, "n_indices": 256, "recent": 32,
                                         "short_rows": (200,)})
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    announce(f"backend dsa: B={case.B} K={case.indices.shape[1]}")
    pool = NeuronDSATokenToKVPool((case.num_blocks - 1) * case.P, case.P, 1, DEV, kv_scale=case.kv_scale)
    case.fill_rows(lambda v, s: pool.set_kv_buffer(0, s.to(DEV), v.to(DEV)))
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, scaling=case.sm_scale)
    backend = _backend(pool, case.block_table, case.positions.to(torch.int64) + 1, case.P)
    q = torch.cat([case.q_absorbed, case.q_pe], dim=-1).to(DEV)
    fb = _batch(case.positions.to(torch.int64) + 1, case.new_slots, positions=case.positions.to(torch.int64))
    out = backend.forward_decode(q, case.own_rows.to(DEV), None, layer, fb, topk_indices=case.indices.to(DEV))
    torch.cuda.synchronize()
    assert_close_attn(out.reshape(case.B, case.H, 512), want_ctx, "dsa")
    assert torch.allclose(backend.last_lse.cpu(), want_lse, atol=2e-3, rtol=1e-4)
    assert torch.equal(pool.get_key_buffer(0).cpu().reshape(-1, 640), cache_o), "row pool differs"


DEVICE_META = [("cfg2-small", 2, {"B": 4, "lens": (100, 700)}), ("cfg4-swa", 4, {"B": 5, "lens": (10, 500), "window": 128})]


@pytest.mark.parametrize("host_lens", [True, False], ids=["seq_lens_cpu", "bound"])
@pytest.mark.parametrize("name,cfg,over", DEVICE_META, ids=[g[0] for g in DEVICE_META])
def test_backend_gqa_device_metadata(name, cfg, over, host_lens):
    """req_to_token on the GPU: the block table is built there (ops.block_table). With seq_lens_cpu the step is the
    host-metadata step bit for bit; without it (a plan from req_to_token's width) it stays within the bar."""
    case = workloads.gqa_case(cfg, overrides=over)
    want, kc_o, *_ = gqa_oracle(case)
    announce(f"backend gqa device metadata {name} host_lens={host_lens}")
    pool = NeuronMHATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, case.G, case.d, 1, DEV)
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, tp_k_head_num=case.G, head_dim=case.d,
                            scaling=case.sm_scale, sliding_window_size=case.window if case.window else -1,
                            sinks=None if case.sinks is None else case.sinks.to(DEV))
    pool.calibrate_kv_scales(0, torch.cat([case.k_prior, case.k_new]).to(DEV),
                             torch.cat([case.v_prior, case.v_new]).to(DEV), inverted=case.scales_multiply)
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.k_prior.to(DEV), case.v_prior.to(DEV))
    args = (case.q.reshape(case.B, -1).to(DEV), case.k_new.to(DEV), case.v_new.to(DEV), layer)
    host = _backend(pool, case.block_table, case.seq_lens, case.P).forward_decode(*args, _batch(case.seq_lens,
                                                                                                 case.new_slots))
    dev = _backend(pool, case.block_table, case.seq_lens, case.P, device_r2t=True)
    fb = _batch(case.seq_lens, case.new_slots, host_lens=host_lens)
    out = dev.forward_decode(*args, fb)
    torch.cuda.synchronize()
    assert fb._sna_decode_state.table.is_cuda
    if host_lens:
        assert torch.equal(out, host)
    assert_close_attn(out.reshape(case.B, case.H, case.d), want, name)
    assert torch.equal(pool.get_key_buffer(0).cpu().view(torch.uint8), kc_o.view(torch.uint8)), "K pool differs"


@pytest.mark.parametrize("host_lens", [True, False], ids=["seq_lens_cpu", "bound"])
def test_backend_mla_device_metadata(host_lens):
    case = workloads.mla_case(overrides={"B": 4, "lens": (1, 3000)})
    want, cache_o, _ = mla_oracle(case)
    announce(f"backend mla device metadata host_lens={host_lens}")
    pool = NeuronMLATokenToKVPool((case.num_blocks - 1) * case.P, case.P, torch.float8_e4m3fn, 512, 64, 1, DEV)
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=case.H, scaling=case.sm_scale)
    T = case.prior_slots.numel()
    pool.set_kv_buffer(layer, case.prior_slots.to(DEV), case.prior_rows.reshape(T, 1, 576).to(DEV))
    q = torch.cat([case.ql_nope, case.q_pe], dim=-1).to(DEV)
    host = _backend(pool, case.block_table, case.seq_lens, case.P).forward_decode(
        q, case.compact_new.to(DEV), None, layer, _batch(case.seq_lens, case.new_slots))
    dev = _backend(pool, case.block_table, case.seq_lens, case.P, device_r2t=True)
    out = dev.forward_decode(q, case.compact_new.to(DEV), None, layer,
                             _batch(case.seq_lens, case.new_slots, host_lens=host_lens))
    torch.cuda.synchronize()
    if host_lens:
        assert torch.equal(out, host)
    assert_close_attn(out.reshape(case.B, case.H, 512), want, "mla device metadata")
    assert torch.equal(pool.kv_buffer[0].cpu().reshape(-1, 576), cache_o), "row pool differs"


class _Extend:
    def is_extend(self):
        return True

    def is_idle(self):
        return False


EXTEND = [("qwen3-8b-shape", 21, dict(H=32, G=8, d=128, P=16), (50, 0, 300), (40, 70, 5), 0, False, False),
          ("gpt-oss-share-swa-sinks", 22, dict(H=8, G=1, d=64, P=16), (200, 17), (150, 33), 128, True, True)]


@pytest.mark.parametrize("device_r2t", [False, True], ids=["host-r2t", "device-r2t"])
@pytest.mark.parametrize("name,seed,shape,priors,ext,window,sinks,inverted", EXTEND, ids=[e[0] for e in EXTEND])
def test_backend_extend_then_decode(name, seed, shape, priors, ext, window, sinks, inverted, device_r2t):
    """An extend batch through forward_extend (its K/V stored, then segmented prefill attention over the pool), then
    one decode step through forward_decode over the pool the extend wrote: attention within the bar against the
    oracle's segmented prefill and decode on the pool's bytes, the pool bit-exact against the oracle's store. The
    GPT-OSS case keeps the model's inverted scales m: its prior and decoded tokens are written as the decode writes
    them (bf16(x * m)), its extend chunk as the prefill writes it (x / bf16(1 / m), model_prefill.py:41-43)."""
    H, G, d, P = shape["H"], shape["G"], shape["d"], shape["P"]
    R = len(priors)
    announce(f"backend extend+decode {name} device_r2t={device_r2t}")
    g = torch.Generator().manual_seed(seed)
    totals = [p + e + 1 for p, e in zip(priors, ext)]  # prior, the extend chunk, one decoded token
    pages = [-(-x // P) for x in totals]
    nb = sum(pages) + 3
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = torch.full((R, max(pages)), -1, dtype=torch.int32)
    used = 0
    for r, n in enumerate(pages):
        table[r, :n] = perm[used:used + n].to(torch.int32)
        used += n
    slot_of = lambda r, pos: int(table[r, pos // P]) * P + pos % P  # noqa: E731
    ks_tok = [torch.randn(x, G, d, generator=g).to(torch.bfloat16) for x in totals]
    vs_tok = [torch.randn(x, G, d, generator=g).to(torch.bfloat16) for x in totals]
    pool = NeuronMHATokenToKVPool((nb - 1) * P, P, torch.float8_e4m3fn, G, d, 1, DEV)
    kscale, vscale = pool.calibrate_kv_scales(0, torch.cat(ks_tok).to(DEV), torch.cat(vs_tok).to(DEV),
                                              inverted=inverted)
    sk = torch.randn(H, generator=g) if sinks else None
    layer = SimpleNamespace(layer_id=0, tp_q_head_num=H, tp_k_head_num=G, head_dim=d, scaling=d ** -0.5,
                            sliding_window_size=window if window else -1, sinks=None if sk is None else sk.to(DEV))
    prior_slots = torch.tensor([slot_of(r, i) for r in range(R) for i in range(priors[r])], dtype=torch.int64)
    if prior_slots.numel():
        pool.set_kv_buffer(layer, prior_slots.to(DEV), torch.cat([ks_tok[r][:priors[r]] for r in range(R)]).to(DEV),
                           torch.cat([vs_tok[r][:priors[r]] for r in range(R)]).to(DEV))
    backend = _backend(pool, table, torch.tensor(totals), P, device_r2t=device_r2t)

    # extend
    ext_slots = torch.tensor([slot_of(r, priors[r] + i) for r in range(R) for i in range(ext[r])], dtype=torch.int64)
    k_ext = torch.cat([ks_tok[r][priors[r]:priors[r] + ext[r]] for r in range(R)])
    v_ext = torch.cat([vs_tok[r][priors[r]:priors[r] + ext[r]] for r in range(R)])
    T = sum(ext)
    q_ext = torch.randn(T, H, d, generator=g).to(torch.bfloat16)
    seq_ext = torch.tensor([p + e for p, e in zip(priors, ext)], dtype=torch.int64)
    fb = SimpleNamespace(forward_mode=_Extend(), batch_size=R, req_pool_indices=torch.arange(R),
                         seq_lens=seq_ext.to(DEV), seq_lens_cpu=seq_ext, extend_seq_lens=torch.tensor(ext).to(DEV),
                         extend_seq_lens_cpu=list(ext), extend_prefix_lens=torch.tensor(priors).to(DEV),
                         out_cache_loc=ext_slots.to(DEV),
                         positions=torch.cat([torch.arange(p, p + e) for p, e in zip(priors, ext)]).to(DEV))
    out = backend.forward_extend(q_ext.reshape(T, H * d).to(DEV), k_ext.reshape(T, G * d).to(DEV),
                                 v_ext.reshape(T, G * d).to(DEV), layer, fb)
    torch.cuda.synchronize()
    kc_o = torch.zeros(nb, G, P, d, dtype=torch.uint8)
    vc_o = torch.zeros_like(kc_o)
    ost.kv_store_mha(torch.cat([ks_tok[r][:priors[r]] for r in range(R)]),
                     torch.cat([vs_tok[r][:priors[r]] for r in range(R)]), prior_slots, kc_o, vc_o, kscale.cpu(),
                     vscale.cpu(), inverted)
    # the chunk: divided by the prefill's scales (the multipliers' bf16 inverses for the GPT-OSS layer)
    pk = ofp8.inverted_scale(kscale.cpu()) if inverted else kscale.cpu()
    pv = ofp8.inverted_scale(vscale.cpu()) if inverted else vscale.cpu()
    ost.kv_store_mha(k_ext, v_ext, ext_slots, kc_o, vc_o, pk, pv)
    k_pool, v_pool = (t.cpu().view(torch.uint8) for t in pool.get_kv_buffer(0))
    assert torch.equal(k_pool, kc_o) and torch.equal(v_pool, vc_o), "pool after extend differs"
    q_start = torch.tensor([0] + torch.tensor(ext).cumsum(0).tolist(), dtype=torch.int32)
    want = oatt.segmented_prefill(q_ext, k_pool, v_pool, table, q_start, torch.tensor(priors), sm_scale=d ** -0.5,
                                  k_scale=kscale.cpu(), v_scale=vscale.cpu(), sinks=sk, window=window,
                                  scales_multiply=inverted)
    assert_close_attn(out.reshape(T, H, d).cpu(), want, f"{name} extend")

    # one decode step over the pool the extend wrote
    L = torch.tensor(totals, dtype=torch.int64)
    new_slots = torch.tensor([slot_of(r, totals[r] - 1) for r in range(R)], dtype=torch.int64)
    k_new = torch.stack([ks_tok[r][-1] for r in range(R)])
    v_new = torch.stack([vs_tok[r][-1] for r in range(R)])
    q_dec = torch.randn(R, H, d, generator=g).to(torch.bfloat16)
    out_d = backend.forward_decode(q_dec.reshape(R, H * d).to(DEV), k_new.reshape(R, G * d).to(DEV),
                                   v_new.reshape(R, G * d).to(DEV), layer, _batch(L, new_slots))
    torch.cuda.synchronize()
    want_d = oatt.paged_decode_gqa(q_dec, k_pool, v_pool, table, L, k_new, v_new, sm_scale=d ** -0.5,
                                   k_scale=kscale.cpu(), v_scale=vscale.cpu(), sinks=sk, window=window,
                                   scales_multiply=inverted)
    assert_close_attn(out_d.reshape(R, H, d).cpu(), want_d, f"{name} decode after extend")
    # the decode's fused store wrote the new tokens as the layer's decode does
    ost.kv_store_mha(k_new, v_new, new_slots, kc_o, vc_o, kscale.cpu(), vscale.cpu(), inverted)
    k_pool, v_pool = (t.cpu().view(torch.uint8) for t in pool.get_kv_buffer(0))
    assert torch.equal(k_pool, kc_o) and torch.equal(v_pool, vc_o), "pool after the decode differs"
