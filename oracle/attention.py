"""Decode attention as the reference's torch paths compute it (CPU, fp32 accumulation). TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Conventions shared with the reference: a row of seq_len L decodes the token at position L - 1, reads its prior from
the pool through the block table (positions < L - 1), and appends its own token in-band, always visible
(ops/attention/attention_decode_paged.py:165-169; ops/attention/attention_decode.py:262-269; ops/attention/mla.py:
46-50). Scores and softmax are fp32; outputs are cast to bf16 once.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch import Tensor

from . import fp8
from . import store as st


def _dequant_cache(cache: Tensor, scale: Optional[Tensor], G: int, multiply: bool = False) -> Tensor:
    """A head-major cache [blocks, G, page, d] as float32 values (uint8 = FP8 bytes, times the per-head dequantization
    scale, or over the per-head GPT-OSS multiplier)."""
    if cache.dtype == torch.uint8:
        sc = torch.as_tensor(scale, dtype=torch.float32).reshape(1, G, 1, 1)
        return fp8.dequantize_mul(cache, sc) if multiply else fp8.dequantize(cache, sc)
    return cache.float()


def paged_decode_gqa(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                     k_new: Tensor, v_new: Tensor, *, sm_scale: float, k_scale=None, v_scale=None,
                     sinks: Optional[Tensor] = None, window: int = 0, scales_multiply: bool = False) -> Tensor:
    """[B, H, d] bf16 GQA decode of q [B, H, d] over caches [blocks, G, page, d] (bf16, or uint8 FP8 bytes with
    per-KV-head dequantization scales [G], or with ``scales_multiply`` the GPT-OSS multipliers [G]: a byte is worth
    byte / m and the new token is stored as fp8.quantize_mul writes it, attention_decode.py:259-260).

    Follows _torch_attention_decode_paged (attention_decode_paged.py:159-173) for the gather, visibility and GQA
    head mapping (q head h reads KV head h // group, :170), and _torch_attention_decode (attention_decode.py:259-276)
    for the FP8 path: the new token attends as dequant(quant(x)) (:259-269), and a sink logit per head joins the
    softmax as an extra column that is then dropped (:274-275). Visibility of a prior key at position p: its table
    entry is >= 0 (and inside the pool), p < L - 1 (attention_decode_paged.py:166), and, with a window W,
    p >= L - W (the window [L - W, L - 1], gpt_oss/attention_masks.py:47-52 with attention_decode_mask.py:72-77).
    The reference folds the FP8 dequantization into the softmax scale and the output projection
    (gpt_oss/mxfp4/model_decode.py:62-70); here K and V are dequantized, which is the same arithmetic."""
    B, H, d = q.shape
    nb, G, P, _ = k_cache.shape
    group = H // G
    Wt = block_table.shape[1]
    table = block_table.to(torch.int64)
    out = torch.empty(B, H, d, dtype=torch.bfloat16)
    key_pos = torch.arange(Wt * P)
    for b in range(B):  # one row at a time bounds the gathered copy's memory
        L = int(seq_lens[b])
        tb = table[b]
        page_ok = (tb >= 0) & (tb < nb)
        rows = tb.clamp(min=0, max=nb - 1)
        keys = _dequant_cache(k_cache[rows], k_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(G, Wt * P, d)
        vals = _dequant_cache(v_cache[rows], v_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(G, Wt * P, d)
        visible = page_ok.repeat_interleave(P) & (key_pos < L - 1)
        if window > 0:
            visible &= key_pos >= L - window
        if k_cache.dtype == torch.uint8:
            ks = torch.as_tensor(k_scale, dtype=torch.float32).reshape(G, 1)
            vs = torch.as_tensor(v_scale, dtype=torch.float32).reshape(G, 1)
            if scales_multiply:
                kn = fp8.dequantize_mul(fp8.quantize_mul(k_new[b], ks), ks)
                vn = fp8.dequantize_mul(fp8.quantize_mul(v_new[b], vs), vs)
            else:
                kn = fp8.dequantize(fp8.quantize(k_new[b], ks), ks)
                vn = fp8.dequantize(fp8.quantize(v_new[b], vs), vs)
        else:
            kn, vn = k_new[b].float(), v_new[b].float()
        keys = torch.cat([keys, kn.reshape(G, 1, d)], dim=1)
        vals = torch.cat([vals, vn.reshape(G, 1, d)], dim=1)
        vis = torch.cat([visible, torch.ones(1, dtype=torch.bool)])
        qb = q[b].float().reshape(G, group, d)
        scores = torch.einsum("gjd,gsd->gjs", qb, keys) * sm_scale
        scores = scores.masked_fill(~vis[None, None, :], float("-inf"))
        if sinks is not None:
            sk = sinks.float().reshape(G, group, 1)
            scores = torch.cat([scores, sk], dim=-1)
            probs = torch.softmax(scores, dim=-1)[..., :-1]
        else:
            probs = torch.softmax(scores, dim=-1)
        out[b] = torch.einsum("gjs,gsd->gjd", probs, vals).reshape(H, d).to(torch.bfloat16)
    return out


def paged_decode_gqa_multi(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, seq_lens: Tensor,
                           k_new: Tensor, v_new: Tensor, *, sm_scale: float, k_scale=None, v_scale=None,
                           sinks: Optional[Tensor] = None, window: int = 0,
                           scales_multiply: bool = False) -> Tensor:
    """[B, S, H, d] bf16 GQA decode of S active tokens per row: q [B, S, H, d], the step's K/V k_new / v_new
    [B, S, G, d], seq_lens [B] counting the prior and the S tokens, so token j sits at position L - S + j.

    Follows _torch_attention_decode (ops/attention/attention_decode.py:226-276) for X [B, S, Hd]: the prior is
    gathered through the row's table (positions < L - S, pages >= 0), the S tokens go in the last S slots as their
    FP8-rounded values (:259-269), and token j sees the prior (within its window: positions >= L - S + j - W + 1,
    gpt_oss/attention_masks.py:47-52) and active tokens 0 .. j (the mask's triu over the active slots,
    attention_decode_mask.py:64-81); a sink column per head joins the softmax and is dropped (:274-275)."""
    B, S, H, d = q.shape
    nb, G, P, _ = k_cache.shape
    group = H // G
    Wt = block_table.shape[1]
    table = block_table.to(torch.int64)
    fp8_cache = k_cache.dtype == torch.uint8
    out = torch.empty(B, S, H, d, dtype=torch.bfloat16)
    key_pos = torch.arange(Wt * P)
    for b in range(B):
        L = int(seq_lens[b])
        tb = table[b]
        page_ok = (tb >= 0) & (tb < nb)
        rows = tb.clamp(min=0, max=nb - 1)
        keys = _dequant_cache(k_cache[rows], k_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(G, Wt * P, d)
        vals = _dequant_cache(v_cache[rows], v_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(G, Wt * P, d)
        prior_vis = page_ok.repeat_interleave(P) & (key_pos < L - S)
        if fp8_cache:
            ks = torch.as_tensor(k_scale, dtype=torch.float32).reshape(1, G, 1)
            vs = torch.as_tensor(v_scale, dtype=torch.float32).reshape(1, G, 1)
            if scales_multiply:
                kn = fp8.dequantize_mul(fp8.quantize_mul(k_new[b], ks), ks)
                vn = fp8.dequantize_mul(fp8.quantize_mul(v_new[b], vs), vs)
            else:
                kn = fp8.dequantize(fp8.quantize(k_new[b], ks), ks)
                vn = fp8.dequantize(fp8.quantize(v_new[b], vs), vs)
        else:
            kn, vn = k_new[b].float(), v_new[b].float()
        keys = torch.cat([keys, kn.permute(1, 0, 2)], dim=1)  # [G, W*P + S, d]
        vals = torch.cat([vals, vn.permute(1, 0, 2)], dim=1)
        for j in range(S):
            pos = L - S + j
            vis = prior_vis.clone()
            if window > 0:
                vis &= key_pos >= pos - window + 1
            act = torch.arange(S) <= j
            vis = torch.cat([vis, act])
            qb = q[b, j].float().reshape(G, group, d)
            scores = torch.einsum("gjd,gsd->gjs", qb, keys) * sm_scale
            scores = scores.masked_fill(~vis[None, None, :], float("-inf"))
            if sinks is not None:
                scores = torch.cat([scores, sinks.float().reshape(G, group, 1)], dim=-1)
                probs = torch.softmax(scores, dim=-1)[..., :-1]
            else:
                probs = torch.softmax(scores, dim=-1)
            out[b, j] = torch.einsum("gjs,gsd->gjd", probs, vals).reshape(H, d).to(torch.bfloat16)
    return out


def segmented_prefill(q: Tensor, k_cache: Tensor, v_cache: Tensor, block_table: Tensor, q_start, prior_lens, *,
                      sm_scale: float, k_scale=None, v_scale=None, sinks: Optional[Tensor] = None,
                      window: int = 0, scales_multiply: bool = False) -> Tensor:
    """[T, H, d] bf16 prefill attention of a chunk's queries q [T, H, d] over caches [blocks, G, page, d] (bf16, or
    uint8 FP8 bytes with per-KV-head scales [G]: dequantization scales, or with ``scales_multiply`` GPT-OSS multipliers
    m, a byte worth byte / m) into which the chunk's own K/V were stored first. Request r owns rows
    q_start[r] .. q_start[r + 1] of q, at positions prior_lens[r] + i, and table row r.

    Follows _torch_segmented_attention (ops/attention/attention_segmented_cte.py:50-75): keys are gathered through the
    row's whole block table, -1 entries read as page 0 (:57-60); key k is visible to the query at position p iff
    k < prior + S and k <= p, and, with a window W, k > p - W (:62-66); scores are fp32 (:68); a sink per head joins
    the softmax as an extra column that is dropped (:70-73); PV is fp32 and the output cast once (:74). GQA maps q
    head h to KV head h // group (:56-57). The reference folds FP8 scales into ``scale`` (the caller's); here K and V
    are dequantized, the same arithmetic."""
    T, H, d = q.shape
    nb, G, P, _ = k_cache.shape
    group = H // G
    out = torch.empty(T, H, d, dtype=torch.bfloat16)
    qs = [int(x) for x in torch.as_tensor(q_start).tolist()]
    pl = [int(x) for x in torch.as_tensor(prior_lens).tolist()]
    for r in range(len(pl)):
        a, b_, prior = qs[r], qs[r + 1], pl[r]
        S = b_ - a
        if S == 0:
            continue
        span = prior + S
        n_pages = -(-span // P)
        pages = block_table[r, :n_pages].to(torch.int64).clamp(min=0)
        keys = _dequant_cache(k_cache[pages], k_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(
            G, n_pages * P, d)[:, :span]
        vals = _dequant_cache(v_cache[pages], v_scale, G, scales_multiply).permute(1, 0, 2, 3).reshape(
            G, n_pages * P, d)[:, :span]
        q_pos = torch.arange(S).unsqueeze(1) + prior
        k_pos = torch.arange(span).unsqueeze(0)
        allowed = (k_pos < prior + S) & (k_pos <= q_pos)
        if window > 0:
            allowed &= k_pos > q_pos - window
        qr = q[a:b_].float().reshape(S, G, group, d).permute(1, 2, 0, 3)  # [G, group, S, d]
        scores = torch.einsum("gjsd,gkd->gjsk", qr, keys) * sm_scale
        scores = scores.masked_fill(~allowed[None, None], float("-inf"))
        if sinks is not None:
            sk = sinks.float().reshape(G, group, 1, 1).expand(G, group, S, 1)
            probs = torch.softmax(torch.cat([scores, sk], dim=-1), dim=-1)[..., :-1]
        else:
            probs = torch.softmax(scores, dim=-1)
        o = torch.einsum("gjsk,gkd->gjsd", probs, vals)  # [G, group, S, d]
        out[a:b_] = o.permute(2, 0, 1, 3).reshape(S, H, d).to(torch.bfloat16)
    return out


def token_slots(block_table: Tensor, page: int, width: int) -> Tensor:
    """[rows, width] token slots of each row's first ``width`` positions, -1 past its pages (ops/attention/mla.py:
    16-21)."""
    positions = torch.arange(width)
    pages = block_table[:, positions // page].to(torch.int64)
    return torch.where(pages >= 0, pages * page + positions % page, torch.full_like(pages, -1))


def mla_decode(ql_nope: Tensor, q_pe: Tensor, cache: Tensor, row_scale: Optional[Tensor], block_table: Tensor,
               seq_lens: Tensor, compact_new: Tensor, *, sm_scale: float, page_size: int) -> Tensor:
    """[B, H, 512] bf16 absorbed-MLA decode (ops/attention/mla.py:44-53) over rows [slots, 576]: bf16, or uint8
    FP8 bytes with one dequantization scale per slot (``row_scale``, this path's extension). History is positions
    < seq_len - 1 read at token_slots(block_table); the own row ``compact_new`` [B, 576] is appended, always valid,
    as dequant(quant(row)) with its own per-token scale for FP8. scores = (ql_nope . latent + q_pe . k_pe) * scale
    (mla.py:24-29), fp32 softmax, out = probs . latent."""
    B, H, latent = ql_nope.shape
    flat = cache.reshape(-1, 576)
    n_rows = flat.shape[0]
    width = block_table.shape[1] * page_size
    slots = token_slots(block_table, page_size, width)
    out = torch.empty(B, H, latent, dtype=torch.bfloat16)
    for b in range(B):
        L = int(seq_lens[b])
        sl = slots[b]
        ok = (sl >= 0) & (sl < n_rows)
        rows = sl.clamp(min=0, max=n_rows - 1)
        if flat.dtype == torch.uint8:
            hist = fp8.dequantize(flat[rows], row_scale.reshape(-1)[rows][:, None])
            ns = fp8.absmax_scale(compact_new[b], dims=-1)
            new = fp8.dequantize(fp8.quantize(compact_new[b], ns), ns)
        else:
            hist = flat[rows].float()
            new = compact_new[b].float()
        keys = torch.cat([hist, new[None]], dim=0)  # [width + 1, 576]
        valid = torch.cat([ok & (torch.arange(width) < L - 1), torch.ones(1, dtype=torch.bool)])
        scores = (ql_nope[b].float() @ keys[:, :latent].T + q_pe[b].float() @ keys[:, latent:].T) * sm_scale
        probs = torch.softmax(scores.masked_fill(~valid[None], float("-inf")), dim=-1)
        out[b] = (probs @ keys[:, :latent]).to(torch.bfloat16)
    return out


def mla_decode_sparse(q_absorbed: Tensor, q_pe: Tensor, cache: Tensor, kv_scale: float, indices: Tensor,
                      block_table: Tensor, positions: Tensor, own_rows: Tensor, new_slots: Tensor, *,
                      sm_scale: float, page_size: int, inplace: bool = False,
                      spec: int = 1) -> tuple[Tensor, Tensor, Tensor]:
    """(ctx [B, H, 512] bf16, lse [B, H] fp32, cache) of the DSA absorbed-MLA decode of B query tokens, ``spec`` per
    sequence (sequence s owns tokens s * spec .. s * spec + spec - 1 and table row s), on one CP rank:
    mla_decode_attention_torch_ref (models/glm52/kernels/decode/attention/mla/mla_decode_attention_torch.py:38-130)
    with cp_degree = 1, cp_rank = 0.

    Steps 0-1 pack ``own_rows`` [B, 576] ([k_pe | latent] order) and scatter them at ``new_slots`` into a copy of
    ``cache`` [rows, 640] before any read. Step 2, per token: each index pos >= 0 resolves to row
    table[s, pos // P] * P + pos % P (_gather_token_keys, :162-179; dropped when its block is past the table,
    unallocated, or the row is outside the cache), and the sequence's spec own rows are appended from their packed
    bytes at their positions (:185-189). Step 4 keeps key_pos <= the token's position (its own row and its earlier
    siblings). Step 5 gives ctx = softmax . latent and lse = max + log(sum) (:117-121); a token with no kept key gives
    ctx 0 and lse -inf (:122-128). ``inplace`` writes the own rows into ``cache`` itself instead of a copy (the
    reference copies, :193-196; the CPU baseline times the in-place form)."""
    B, H, _ = q_absorbed.shape
    P = page_size
    if not inplace:
        cache = cache.clone()
    st.kv_store_dsa(own_rows, new_slots, cache, kv_scale)
    flat = cache.reshape(-1, st.ROW_BYTES)
    n_rows = flat.shape[0]
    packed_own = st.pack_kv_rows(own_rows.reshape(B, 576), kv_scale)
    ctx = torch.empty(B, H, 512, dtype=torch.bfloat16)
    lse = torch.empty(B, H, dtype=torch.float32)
    Wt = block_table.shape[1]
    for b in range(B):
        seq = b // spec
        sel = indices[b].to(torch.int64)
        pos_q = int(positions[b])
        blk = torch.where(sel >= 0, sel // P, torch.full_like(sel, -1))
        in_table = (blk >= 0) & (blk < Wt)
        tab = torch.where(in_table, block_table[seq].to(torch.int64)[blk.clamp(min=0, max=Wt - 1)],
                          torch.full_like(sel, -1))
        row = tab * P + sel % P
        resident = in_table & (tab >= 0) & (row >= 0) & (row < n_rows)
        key_pos = torch.where(resident, sel.float(), torch.full_like(sel, 1 << 30, dtype=torch.float32))
        keys = torch.zeros(sel.numel(), 576)
        if bool(resident.any()):
            keys[resident] = st.unpack_kv_row(flat[row[resident]], kv_scale)
        own = st.unpack_kv_row(packed_own[seq * spec:(seq + 1) * spec], kv_scale)  # the sequence's own rows
        keys = torch.cat([keys, own], dim=0)
        key_pos = torch.cat([key_pos, positions[seq * spec:(seq + 1) * spec].float()])
        k_pe, latent = keys[:, :64], keys[:, 64:]
        scores = sm_scale * (q_absorbed[b].float() @ latent.T + q_pe[b].float() @ k_pe.T)  # [H, K+1]
        keep = key_pos <= float(pos_q)
        scores = scores.masked_fill(~keep[None], float("-inf"))
        row_max = scores.amax(dim=-1, keepdim=True)
        shifted = torch.exp(scores - row_max)
        row_sum = shifted.sum(dim=-1, keepdim=True)
        c = (shifted / row_sum) @ latent
        l = (row_max.squeeze(-1) + torch.log(row_sum.squeeze(-1))).float()
        if not bool(keep.any()):
            c = torch.zeros_like(c)
            l = torch.full_like(l, float("-inf"))
        ctx[b] = c.to(torch.bfloat16)
        lse[b] = l
    return ctx, lse, cache


def lse_merge(o_parts: Tensor, lse_parts: Tensor) -> tuple[Tensor, Tensor]:
    """(out [rows, dim] bf16, lse [rows]) of normalized partials o_parts [n, rows, dim] with natural-log LSEs
    [n, rows]: LSE = logsumexp(lse_i), out = sum_i exp(lse_i - LSE) o_i. The reference's DCP merge
    (ops/attention/attention_decode.py:281-284)."""
    merged = torch.logsumexp(lse_parts.float(), dim=0)
    w = torch.exp(lse_parts.float() - merged[None])
    w = torch.where(torch.isfinite(merged)[None], w, torch.zeros_like(w))
    out = (o_parts.float() * w[..., None]).sum(dim=0)
    return out.to(torch.bfloat16), merged


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
