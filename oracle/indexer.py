"""The DeepSeek-sparse-attention indexer's decode step as the reference's torch path computes it: the fp8 index-key
store, the head-weighted ReLU score over a request's cached keys, and the top-k selection. TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Follows models/glm52/kernels/decode/attention/indexer/indexer_torch.py, from the point where the projections are
done (the query and key rotated, the head weights computed: model work outside this path):
  - pack_indexer_keys_fp8 (:44-53): a key row stored as clamp(key, +-448) cast to e4m3fn, no scale;
  - indexer_kv_score_torch_ref's score (:254-268): raw = q_rot . key * d^-0.5 in fp32, relu, weighted by
    w = (hidden @ weights_proj) * H^-0.5 and summed over heads, clamped by the residency mask (a key at a position
    >= the query's own position scores -MASK_BOUND), narrowed to bf16 once;
  - indexer_topk_local_torch_ref's selection (:296-309): the topk largest scores (ties at the threshold in any
    order: the reference compares the selected multiset), a selected dead key (score <= -MASK_BOUND / 2) labelled -1.
"""

from __future__ import annotations

import torch
from torch import Tensor

MASK_BOUND = 1.0e30
KEY_FP8_MAX = 448.0


def pack_index_keys(keys: Tensor) -> Tensor:
    """[..., d] float keys -> e4m3fn bytes (uint8): clamp to +-448, then cast (pack_indexer_keys_fp8, :44-53)."""
    return keys.float().clamp(-KEY_FP8_MAX, KEY_FP8_MAX).to(torch.float8_e4m3fn).view(torch.uint8)


def index_key_store(keys: Tensor, slots: Tensor, cache: Tensor) -> None:
    """Write key rows [T, d] (bf16) at ``slots`` [T] of an index-key cache [blocks, page, d] (uint8): the slot's row
    takes pack_index_keys(key); slots outside the cache are skipped (indexer_torch.py:228-234)."""
    flat = cache.view(-1, cache.shape[-1])
    for i, s in enumerate(slots.tolist()):
        if 0 <= s < flat.shape[0]:
            flat[s] = pack_index_keys(keys[i])


def indexer_scores(q: Tensor, w: Tensor, cache: Tensor, block_table: Tensor, limits: Tensor, width: int) -> Tensor:
    """[B, width] bf16 index scores: row b scores its logical keys e < width, key e read at page block_table[b, e //
    P], offset e % P of the cache [blocks, P, d] (uint8 e4m3fn bytes); q [B, H, d] (bf16, already rotated), w [B, H]
    fp32 (already scaled by H^-0.5). Key e is live iff e < limits[b] (the residency mask: positions before the
    query's own) and its page is valid; a dead key scores -MASK_BOUND (the clamp of :266-267)."""
    B, H, d = q.shape
    nb, P, _ = cache.shape
    keys_all = cache.view(torch.float8_e4m3fn).float().reshape(nb * P, d)
    out = torch.empty(B, width, dtype=torch.bfloat16)
    e = torch.arange(width)
    for b in range(B):
        col = e // P
        page = torch.full((width,), -1, dtype=torch.int64)
        inside = col < block_table.shape[1]
        page[inside] = block_table[b, col[inside]].to(torch.int64)
        ok = (page >= 0) & (page < nb) & (e < int(limits[b]))
        rows = page.clamp(min=0) * P + e % P
        keys = keys_all[rows]
        raw = torch.einsum("hd,ed->he", q[b].float(), keys) * (float(d) ** -0.5)
        score = torch.einsum("h,he->e", w[b].float(), torch.relu(raw))
        score = torch.minimum(score, torch.where(ok, torch.tensor(MASK_BOUND), torch.tensor(-MASK_BOUND)))
        out[b] = score.to(torch.bfloat16)
    return out


def topk_positions(scores: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """(positions [B, k] int32, values [B, k] fp32) of the k largest scores per row (torch.topk), -1 for a selected
    dead key (score <= -MASK_BOUND / 2), as indexer_topk_local_torch_ref labels them (:296-309)."""
    top = torch.topk(scores.float(), k, dim=-1, largest=True)
    pos = top.indices.to(torch.int32)
    pos = torch.where(top.values > -0.5 * MASK_BOUND, pos, torch.full_like(pos, -1))
    return pos, top.values
