"""Decode metadata as the reference's backend and runtime build it (host, numpy/torch). TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py)."""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor


def block_table(req_to_token: np.ndarray, req_pool_indices: np.ndarray, seq_lens: np.ndarray, page: int) -> Tensor:
    """[bs, max_blocks] int32: each request's page representatives divided by the page, -1 past its own pages when
    bs != 1 (NeuronAttnBackend._block_table, attention/backend.py:114-130)."""
    rows = np.asarray(req_pool_indices)
    lens = np.asarray(seq_lens)
    max_blocks = (int(lens.max()) + page - 1) // page
    table = (req_to_token[rows, : max_blocks * page : page] // page).astype(np.int32, copy=False)
    if len(rows) != 1:
        live = np.arange(0, max_blocks * page, page) < lens[:, None]
        table = np.where(live, table, np.int32(-1))
    return torch.from_numpy(np.ascontiguousarray(table))


def swa_trimmed_table(block_table: Tensor, seq_lens: Tensor, window: int, page: int, width: int) -> tuple[Tensor,
                                                                                                           Tensor]:
    """(trimmed table [B, width], per-row position offset [B]) of a sliding-window layer: the table from column
    start = max((L - 1) // page - width + 1, 0), -1 past the table (model_executor/graph_runner.py:1124-1136)."""
    ctx = seq_lens.to(torch.long) - 1
    start = torch.clamp(ctx // page - width + 1, min=0)
    gather = (start[:, None] + torch.arange(width)[None, :]).clamp(max=block_table.shape[1] - 1)
    trimmed = block_table.gather(1, gather)
    valid = (torch.arange(width)[None, :] + start[:, None]) < block_table.shape[1]
    trimmed = torch.where(valid, trimmed, torch.full_like(trimmed, -1))
    return trimmed, (start * page).to(torch.int32)
