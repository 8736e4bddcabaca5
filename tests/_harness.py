"""Shared builders for the parity tests: the same seeded case materialized twice, in the CPU oracle and through the HIP
path, and the comparison bar (bit-exact stores; max-abs 2e-2 and mean-abs 2e-3 for bf16 attention outputs with fp32
accumulation, the tolerance BASELINE.json's north star states)."""

from __future__ import annotations

import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import store as ost
from sglang_neuron_amd import ops, workloads

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def assert_close_attn(got: torch.Tensor, want: torch.Tensor, what: str = "") -> None:
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape, (g.shape, w.shape)
    assert bool(torch.isfinite(g).all()), f"{what}: non-finite output"
    diff = (g - w).abs()
    mx, mean = float(diff.max()) if diff.numel() else 0.0, float(diff.mean()) if diff.numel() else 0.0
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e} (bar {MAX_ABS}), mean-abs {mean:.3e} " \
                                               f"(bar {MEAN_ABS})"


# ---- GQA ----

def gqa_scales(case: workloads.GqaCase):
    """Per-KV-head absmax scales over every K (V) token of the case, prior and new (oracle); for a GPT-OSS case
    (``scales_multiply``) the multipliers the reference's loader makes of them."""
    k_all = torch.cat([case.k_prior.cpu(), case.k_new.cpu()], dim=0)
    v_all = torch.cat([case.v_prior.cpu(), case.v_new.cpu()], dim=0)
    ks, vs = ofp8.absmax_scale(k_all, dims=(0, 2)), ofp8.absmax_scale(v_all, dims=(0, 2))
    if case.scales_multiply:
        return ofp8.inverted_scale(ks), ofp8.inverted_scale(vs)
    return ks, vs


def gqa_oracle(case: workloads.GqaCase):
    """(out [B, H, d], k_cache, v_cache, k_scale, v_scale) on the CPU: prefill store, decode, then the new token's store."""
    G, d, P, nb = case.G, case.d, case.P, case.num_blocks
    dt = torch.uint8 if case.fp8 else torch.bfloat16
    kc = torch.zeros(nb, G, P, d, dtype=dt)
    vc = torch.zeros(nb, G, P, d, dtype=dt)
    ks = vs = None
    if case.fp8:
        ks, vs = gqa_scales(case)
    mul = case.scales_multiply
    ost.kv_store_mha(case.k_prior.cpu(), case.v_prior.cpu(), case.prior_slots.cpu(), kc, vc, ks, vs, mul)
    out = oatt.paged_decode_gqa(case.q.cpu(), kc, vc, case.block_table, case.seq_lens, case.k_new.cpu(),
                                case.v_new.cpu(), sm_scale=case.sm_scale, k_scale=ks, v_scale=vs,
                                sinks=case.sinks, window=case.window, scales_multiply=mul)
    ost.kv_store_mha(case.k_new.cpu(), case.v_new.cpu(), case.new_slots.cpu(), kc, vc, ks, vs, mul)
    return out, kc, vc, ks, vs


def gqa_gpu_pool(case: workloads.GqaCase, dev="cuda"):
    """(k_cache, v_cache, k_scale, v_scale) on the GPU, filled by the HIP store (scales by the HIP absmax kernel)."""
    return workloads.gqa_pool(case, dev)


def gqa_gpu_decode(case: workloads.GqaCase, kc, vc, ks, vs, dev="cuda", store_new=True):
    return ops.paged_decode_gqa(case.q.to(dev), kc, vc, case.block_table.to(dev), case.seq_lens.to(dev),
                                case.k_new.to(dev), case.v_new.to(dev), sm_scale=case.sm_scale, k_scale=ks,
                                v_scale=vs, sinks=None if case.sinks is None else case.sinks.to(dev),
                                window=case.window, new_slots=case.new_slots.to(dev) if store_new else None,
                                host_seq_lens=case.seq_lens, scales_multiply=case.scales_multiply)


def cache_bytes(c: torch.Tensor) -> torch.Tensor:
    return c.detach().cpu().contiguous().view(torch.uint8)


# ---- MLA ----

def mla_oracle(case: workloads.MlaCase, bf16: bool = False):
    """(out, cache, row_scale) on the CPU: prefill rows, decode, then the own row's store. ``bf16``: a bf16 row pool
    (row_scale None)."""
    n = case.num_blocks * case.P
    cache = torch.zeros(n, 576, dtype=torch.bfloat16 if bf16 else torch.uint8)
    scale = None if bf16 else torch.zeros(n, dtype=torch.float32)
    ost.kv_store_mla(case.prior_rows.cpu(), case.prior_slots.cpu(), cache, scale)
    out = oatt.mla_decode(case.ql_nope.cpu(), case.q_pe.cpu(), cache, scale, case.block_table, case.seq_lens,
                          case.compact_new.cpu(), sm_scale=case.sm_scale, page_size=case.P)
    ost.kv_store_mla(case.compact_new.cpu(), case.new_slots.cpu(), cache, scale)
    return out, cache, scale


def mla_gpu_pool(case: workloads.MlaCase, dev="cuda", bf16: bool = False):
    return workloads.mla_pool(case, dev, bf16)


def mla_gpu_decode(case: workloads.MlaCase, cache, scale, dev="cuda", store_new=True):
    return ops.mla_decode(case.ql_nope.to(dev), case.q_pe.to(dev), cache, scale, case.block_table.to(dev),
                          case.seq_lens.to(dev), case.compact_new.to(dev), sm_scale=case.sm_scale, page_size=case.P,
                          new_slots=case.new_slots.to(dev) if store_new else None, host_seq_lens=case.seq_lens)


# ---- DSA ----

def dsa_oracle(case: workloads.DsaCase):
    """(ctx, lse, cache) on the CPU: every prior row stored, then the reference's six steps."""
    n = case.num_blocks * case.P
    cache = torch.zeros(n, 640, dtype=torch.uint8)
    case.fill_rows(lambda v, s: ost.kv_store_dsa(v, s, cache, case.kv_scale))
    ctx, lse, cache2 = oatt.mla_decode_sparse(case.q_absorbed.cpu(), case.q_pe.cpu(), cache, case.kv_scale,
                                              case.indices, case.block_table, case.positions, case.own_rows.cpu(),
                                              case.new_slots.cpu(), sm_scale=case.sm_scale, page_size=case.P,
                                              spec=case.spec)
    return ctx, lse, cache2


def dsa_gpu_pool(case: workloads.DsaCase, dev="cuda", gen_device="cpu"):
    return workloads.dsa_pool(case, dev, gen_device)


def dsa_gpu_step(case: workloads.DsaCase, cache, dev="cuda", fused=True):
    """The step as the path runs it: the sparse decode storing the own rows in the same launch (fused), or the store
    kernel first and then the decode."""
    slots = case.new_slots.to(dev)
    if not fused:
        ops.kv_store_dsa(case.own_rows.to(dev), slots, cache, case.kv_scale)
    return ops.mla_decode_sparse(case.q_absorbed.to(dev), case.q_pe.to(dev), cache, case.kv_scale,
                                 case.indices.to(dev), case.block_table.to(dev), case.positions.to(dev),
                                 case.own_rows.to(dev), sm_scale=case.sm_scale, page_size=case.P,
                                 new_slots=slots if fused else None, spec=case.spec)
