"""Pins of the oracle's stores (oracle/store.py), each against something other than its own code: an explicit
per-token, per-head loop for the slot arithmetic, untouched bytes outside the written slots, the reference's stated
properties of the DSA row layout, and pack/unpack round trips against the FP8 definition."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import store as ost


def _rand_bf16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("fp8", [False, True])
def test_mha_store_slot_arithmetic_by_loop(fp8):
    nb, G, P, d, T = 5, 3, 4, 8, 9
    k, v = _rand_bf16((T, G, d), 1), _rand_bf16((T, G, d), 2)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(nb * P, generator=g)[:T]
    slots[2] = -5          # out of pool -> slot 0
    slots[7] = nb * P + 3  # past the pool -> slot 0
    dt = torch.uint8 if fp8 else torch.bfloat16
    sentinel = 0x55 if fp8 else 7.0
    kc = torch.full((nb, G, P, d), sentinel, dtype=dt)
    vc = kc.clone()
    ks = torch.tensor([0.5, 1.0, 0.03125]) if fp8 else None
    vs = torch.tensor([2.0, 0.25, 1.0]) if fp8 else None
    ost.kv_store_mha(k, v, slots, kc, vc, ks, vs)
    want_k = torch.full_like(kc, sentinel)
    want_v = want_k.clone()
    for t in range(T):  # in order: a later token to the same slot wins, as the scatter does
        s = int(slots[t])
        s = 0 if s < 0 or s >= nb * P else s
        for h in range(G):
            if fp8:
                want_k[s // P, h, s % P] = ofp8.quantize(k[t, h], float(ks[h]))
                want_v[s // P, h, s % P] = ofp8.quantize(v[t, h], float(vs[h]))
            else:
                want_k[s // P, h, s % P] = k[t, h]
                want_v[s // P, h, s % P] = v[t, h]
    # two tokens redirected to slot 0: the reference's index_put_ leaves either; compare everything else exactly
    keep = torch.ones(nb, G, P, dtype=torch.bool)
    keep[0, :, 0] = False
    assert torch.equal(kc[keep], want_k[keep]) and torch.equal(vc[keep], want_v[keep])
    # the redirected slot holds one of the two redirected tokens
    cands = [ofp8.quantize(k[t], ks.reshape(G, 1)) if fp8 else k[t] for t in (2, 7)]
    assert any(torch.equal(kc[0, :, 0], c) for c in cands)


def test_mha_store_multiplier_mode_by_loop():
    """The GPT-OSS decode write (scales_multiply): every byte against the definition of its element, e4m3fn of the
    exact product rounded to bf16 and clamped, at (slot // page, head, slot % page)."""
    nb, G, P, d, T = 4, 2, 4, 8, 6
    k, v = _rand_bf16((T, G, d), 5) * 7, _rand_bf16((T, G, d), 6)
    slots = torch.tensor([4, 9, 15, 5, 12, 6])
    m = ofp8.inverted_scale(torch.tensor([0.0123, 3.0 / 448.0]))
    kc = torch.zeros(nb, G, P, d, dtype=torch.uint8)
    vc = torch.zeros_like(kc)
    ost.kv_store_mha(k, v, slots, kc, vc, m, m.flip(0), scales_multiply=True)
    vals = ofp8.e4m3fn_values()
    for t in range(T):
        s = int(slots[t])
        for h in range(G):
            for src, cache, mh in ((k, kc, float(m[h])), (v, vc, float(m.flip(0)[h]))):
                for i in range(d):
                    p = float(src[t, h, i]) * mh
                    r = float(ofp8.bf16_round_spec(np.array([p]))[0])
                    r = min(max(r, -448.0), 448.0)
                    byte = int(cache[s // P, h, s % P, i])
                    # the nearest code (ties are rare enough at these values to be checked by the spec's search)
                    assert byte == int(ofp8.e4m3fn_rne_spec(np.array([r], dtype=np.float32))[0]), (t, h, i)
                    assert abs(vals[byte] - r) <= abs(r) * 2 ** -4 + 2 ** -10
    # untouched elsewhere
    written = {(int(s) // P, int(s) % P) for s in slots}
    for pg in range(nb):
        for off in range(P):
            if (pg, off) not in written:
                assert int(kc[pg, :, off].abs().sum()) == 0


def test_mla_store_per_token_scale_by_loop():
    n, T = 12, 5
    rows = _rand_bf16((T, 576), 4) * 3
    rows[1] = 0  # an all-zero row: scale 1, bytes 0
    slots = torch.tensor([3, 0, 11, 7, 50])
    cache = torch.full((n, 576), 0x33, dtype=torch.uint8)
    scale = torch.full((n,), -1.0)
    ost.kv_store_mla(rows, slots, cache, scale)
    for t in range(T):
        s = int(slots[t]) if int(slots[t]) < n else 0
        if t in (1, 4):
            continue  # slot 0: token 4 (redirected) overwrites token 1; checked below
        amax = np.float32(max(abs(float(x)) for x in rows[t].float()))
        sc = float(amax / np.float32(448.0)) if amax > 0 else 1.0  # the fp32 division of the scale rule
        assert float(scale[s]) == sc
        assert torch.equal(cache[s], ofp8.quantize(rows[t], sc))
    assert torch.equal(cache[0], ofp8.quantize(rows[4], float(scale[0])))
    untouched = [i for i in range(n) if i not in (3, 0, 11, 7)]
    assert bool((cache[untouched] == 0x33).all()) and bool((scale[untouched] == -1.0).all())
    assert torch.equal(ofp8.quantize(rows[1], 1.0), torch.zeros(576, dtype=torch.uint8))


def test_dsa_latent_map_is_the_stated_bijection():
    """The reference's contract (kv_row_layout.py:62-84): a bijection from [0, 512) onto [128, 640); read as 16-bit
    words, word w of the latent holds dims 256 (w // 128) + w % 128 (low byte) and that + 128 (high byte)."""
    m = ost.latent_byte_map().tolist()
    assert sorted(m) == list(range(128, 640))
    for w in range(256):
        lo_dim = 256 * (w // 128) + w % 128
        assert m[lo_dim] == 128 + 2 * w and m[lo_dim + 128] == 128 + 2 * w + 1


@pytest.mark.parametrize("kv_scale", [1.0, 2.0 ** -6, 0.37])
def test_dsa_pack_unpack_round_trip(kv_scale):
    rows = _rand_bf16((6, 576), 5)
    packed = ost.pack_kv_rows(rows, kv_scale)
    back = ost.unpack_kv_row(packed, kv_scale)
    rope_want = (rows[:, :64].float() / kv_scale).to(torch.bfloat16).float() * kv_scale
    lat_want = ofp8.dequantize(ofp8.quantize(rows[:, 64:], kv_scale), kv_scale)
    assert torch.equal(back[:, :64], rope_want)
    assert torch.equal(back[:, 64:], lat_want)


def test_dsa_store_skips_invalid_slots():
    cache = torch.full((8, 640), 0x11, dtype=torch.uint8)
    rows = _rand_bf16((4, 576), 6)
    ost.kv_store_dsa(rows, torch.tensor([2, -1, 8, 5]), cache, 0.5)
    packed = ost.pack_kv_rows(rows, 0.5)
    assert torch.equal(cache[2], packed[0]) and torch.equal(cache[5], packed[3])
    assert bool((cache[[0, 1, 3, 4, 6, 7]] == 0x11).all())
