"""Decode metadata built on the device (ops.block_table, ops.window_table) against the oracle's restatement of the
reference's host builders (attention/backend.py:114-130, model_executor/graph_runner.py:1121-1133): bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import metadata as omd
from sglang_neuron_amd import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _r2t(rows: int, ctx: int, seed: int) -> np.ndarray:
    g = np.random.default_rng(seed)
    return g.integers(0, 1 << 20, size=(rows, ctx), dtype=np.int32)


CASES = [("bs1", 1, 16, 5000, 1), ("bs8-p16", 8, 16, 5000, 2), ("bs33-p64", 33, 64, 9000, 3),
         ("bs5-p1", 5, 1, 300, 4), ("bs64-p128", 64, 128, 20000, 5)]


@pytest.mark.parametrize("name,B,page,ctx,seed", CASES, ids=[c[0] for c in CASES])
def test_block_table_matches_reference_builder(name, B, page, ctx, seed):
    announce(f"block_table {name}: B={B} page={page} ctx={ctx}")
    r2t = _r2t(B + 7, ctx, seed)
    g = np.random.default_rng(seed + 100)
    rows = g.permutation(B + 7)[:B].astype(np.int64)
    lens = g.integers(1, ctx + 1, size=B).astype(np.int64)
    lens[0] = ctx  # a row spanning the whole context
    if B > 2:
        lens[1] = 1  # only its new token
        lens[2] = page  # exactly one page
    want = omd.block_table(r2t, rows, lens, page)
    width = want.shape[1]
    lens32 = torch.empty(B, dtype=torch.int32, device=DEV)
    got = ops.block_table(torch.from_numpy(r2t).to(DEV), torch.from_numpy(rows).to(DEV),
                          torch.from_numpy(lens).to(DEV), page, width, seq_lens_i32=lens32)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want), name
    assert torch.equal(lens32.cpu(), torch.from_numpy(lens).to(torch.int32))


def test_block_table_bounds():
    """A wider table than the rows need, a row index outside req_to_token, a zero length, a strided req_to_token
    view and columns past its width: -1 there, the reference's entries elsewhere."""
    announce("block_table bounds")
    page, ctx = 16, 200
    full = _r2t(12, ctx + 40, 7)
    r2t = torch.from_numpy(full).to(DEV)[:, :ctx]  # row stride ctx + 40
    rows = torch.tensor([3, -1, 12, 5, 0], dtype=torch.int64)
    lens = torch.tensor([50, 30, 30, 0, 400], dtype=torch.int64)
    width = 30  # 480 tokens: past the context (200) and past every row
    got = ops.block_table(r2t, rows.to(DEV), lens.to(DEV), page, width).cpu()
    want = torch.full((5, width), -1, dtype=torch.int32)
    want[0, :4] = torch.from_numpy(full[3, 0:50:page] // page)
    want[4, :13] = torch.from_numpy(full[0, 0:ctx:page] // page)  # columns whose first token is inside the context
    assert torch.equal(got, want)


WINDOWS = [(1, 16), (16, 16), (17, 16), (128, 16), (128, 64), (1000, 64), (4096, 16)]


@pytest.mark.parametrize("window,page", WINDOWS, ids=[f"w{w}-p{p}" for w, p in WINDOWS])
def test_window_table_matches_reference_trim(window, page):
    announce(f"window_table w={window} page={page}")
    g = np.random.default_rng(window * 131 + page)
    B, ctx = 24, 6000
    r2t = _r2t(B, ctx, window)
    lens = g.integers(1, ctx + 1, size=B).astype(np.int64)
    lens[:4] = [1, window, window + 1, ctx]
    table = omd.block_table(r2t, np.arange(B), lens, page)
    nb = ops.window_blocks(window, page, table.shape[1])
    want_t, want_off = omd.swa_trimmed_table(table, torch.from_numpy(lens), window, page, nb)
    got_t, got_off = ops.window_table(table.to(DEV), torch.from_numpy(lens).to(DEV), page, nb)
    torch.cuda.synchronize()
    assert torch.equal(got_t.cpu(), want_t)
    assert torch.equal(got_off.cpu(), want_off)


def test_window_table_of_a_strided_table():
    announce("window_table strided")
    page, B = 16, 6
    big = torch.arange(B * 50, dtype=torch.int32).reshape(B, 50)
    lens = torch.tensor([1, 100, 300, 500, 640, 800], dtype=torch.int64)
    view = big[:, :40]  # row stride 50, width 40
    nb = ops.window_blocks(128, page, 40)
    want_t, want_off = omd.swa_trimmed_table(view.contiguous(), lens, 128, page, nb)
    got_t, got_off = ops.window_table(big.to(DEV)[:, :40], lens.to(DEV), page, nb)
    assert torch.equal(got_t.cpu(), want_t) and torch.equal(got_off.cpu(), want_off)
