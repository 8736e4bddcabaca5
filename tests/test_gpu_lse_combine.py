"""The exported LSE merge of partial attention results (sna_lse_combine through ops.lse_combine) against the oracle's
lse_merge (the reference's DCP merge, ops/attention/attention_decode.py:277-285): 1 to 64 parts, parts whose LSE is
-inf (an empty shard: context 0, mla_decode_attention_torch.py:122-128), rows whose parts are all -inf, and a merge of
split partials that equals the whole attention."""

import math

import pytest
import torch

from oracle import attention as oatt
from sglang_neuron_amd import ops
from tests.conftest import announce
from tests._harness import assert_close_attn

pytestmark = pytest.mark.gpu


def _parts(n, rows, dim, seed, empty_frac=0.0, empty_rows=()):
    g = torch.Generator().manual_seed(seed)
    o = torch.randn(n, rows, dim, generator=g)
    lse = torch.randn(n, rows, generator=g) * 4.0
    if empty_frac:
        empty = torch.rand(n, rows, generator=g) < empty_frac
        lse[empty] = -math.inf
        o[empty] = 0.0
    for r in empty_rows:
        lse[:, r] = -math.inf
        o[:, r] = 0.0
    return o, lse


@pytest.mark.parametrize("n,rows,dim,empty_frac,empty_rows", [
    (1, 7, 512, 0.0, ()),
    (2, 33, 128, 0.0, ()),
    (3, 16, 64, 0.3, ()),
    (16, 40, 512, 0.2, (5,)),
    (64, 9, 512, 0.5, (0, 8)),
])
def test_lse_combine_matches_oracle(n, rows, dim, empty_frac, empty_rows):
    o, lse = _parts(n, rows, dim, 100 + n, empty_frac, empty_rows)
    announce(f"lse_combine n={n} rows={rows} dim={dim} empty={empty_frac} empty_rows={empty_rows}")
    want, want_lse = oatt.lse_merge(o, lse)
    got, got_lse = ops.lse_combine(o.cuda(), lse.cuda())
    torch.cuda.synchronize()
    assert_close_attn(got, want, f"lse_combine n={n}")
    g, w = got_lse.cpu(), want_lse
    assert torch.equal(torch.isneginf(g), torch.isneginf(w)), "rows with no part differ"
    fin = torch.isfinite(w)
    assert torch.allclose(g[fin], w[fin], atol=1e-5, rtol=1e-5), (g[fin] - w[fin]).abs().max()
    for r in empty_rows:
        assert torch.equal(got[r].cpu(), torch.zeros(dim, dtype=torch.bfloat16)), f"empty row {r} is not zero"


def test_lse_combine_of_splits_is_the_whole_attention():
    """Attention over 300 keys in 5 shards, each normalized with its own LSE, merges to attention over all keys."""
    g = torch.Generator().manual_seed(9)
    q = torch.randn(6, 64, generator=g, dtype=torch.float64)
    k = torch.randn(300, 64, generator=g, dtype=torch.float64)
    v = torch.randn(300, 64, generator=g, dtype=torch.float64)
    s = q @ k.T / 8.0
    whole = torch.softmax(s, dim=-1) @ v
    parts, lses = [], []
    for lo in range(0, 300, 60):
        sl = s[:, lo:lo + 60]
        parts.append(torch.softmax(sl, dim=-1) @ v[lo:lo + 60])
        lses.append(torch.logsumexp(sl, dim=-1))
    announce("lse_combine of 5 shards")
    got, got_lse = ops.lse_combine(torch.stack(parts).float().cuda(), torch.stack(lses).float().cuda())
    torch.cuda.synchronize()
    assert_close_attn(got, whole.float(), "shards")
    assert torch.allclose(got_lse.cpu().double(), torch.logsumexp(s, dim=-1), atol=1e-4)


def test_lse_combine_refuses_bad_shapes():
    with pytest.raises(ValueError):
        ops.lse_combine(torch.zeros(2, 3, 4, device="cuda", dtype=torch.float16), torch.zeros(2, 3, device="cuda"))
