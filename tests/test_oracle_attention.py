"""Pins of the oracle's decode attention (oracle/attention.py) and metadata (oracle/metadata.py): float64 brute force
with explicit loops over keys on tiny inputs, closed forms, invariances, and block tables built by hand."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import metadata as omd
from oracle import store as ost


def _bf16(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _softmax_attend(q, keys, vals, scale, sink=None):
    """float64 softmax attention of one query over key/value lists, by explicit loops."""
    s = [sum(float(q[i]) * float(k[i]) for i in range(len(q))) * scale for k in keys]
    m = max(s + ([sink] if sink is not None else []))
    e = [math.exp(x - m) for x in s]
    den = sum(e) + (math.exp(sink - m) if sink is not None else 0.0)
    return [sum(e[j] * float(vals[j][i]) for j in range(len(keys))) / den for i in range(len(vals[0]))]


def _gqa_case(seed, B=3, H=4, G=2, d=8, P=4, fp8=False, window=0, sinks=False, mul=False):
    g = torch.Generator().manual_seed(seed)
    lens = [1, 6, 11][:B]
    pages = [(L + P - 1) // P for L in lens]
    nb = sum(pages) + 2
    perm = (torch.randperm(nb - 1, generator=g) + 1).tolist()
    W = max(pages)
    table = torch.full((B, W), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        table[b, :n] = torch.tensor(perm[o:o + n], dtype=torch.int32)
        o += n
    dt = torch.uint8 if fp8 else torch.bfloat16
    kc = torch.zeros(nb, G, P, d, dtype=dt)
    vc = torch.zeros(nb, G, P, d, dtype=dt)
    kp, vp, slots = [], [], []
    for b, L in enumerate(lens):
        for p in range(L - 1):
            slots.append(int(table[b, p // P]) * P + p % P)
    T = len(slots)
    kp, vp = _bf16((T, G, d), g), _bf16((T, G, d), g)
    ks = torch.rand(G, generator=g) * 0.01 + 0.004 if fp8 else None
    vs = torch.rand(G, generator=g) * 0.01 + 0.004 if fp8 else None
    if mul:  # GPT-OSS multipliers: the bf16 inverses of the scales
        ks, vs = ofp8.inverted_scale(ks), ofp8.inverted_scale(vs)
    ost.kv_store_mha(kp, vp, torch.tensor(slots), kc, vc, ks, vs, mul)
    q, kn, vn = _bf16((B, H, d), g), _bf16((B, G, d), g), _bf16((B, G, d), g)
    sk = torch.randn(H, generator=g) if sinks else None
    return dict(q=q, kc=kc, vc=vc, table=table, lens=torch.tensor(lens), kn=kn, vn=vn, ks=ks, vs=vs, sinks=sk,
                P=P, G=G, window=window, slots=slots, mul=mul)


def _brute_gqa(c, scale):
    """Loops: row b, head h -> KV head h // (H / G); prior keys at positions p < L - 1 (and >= L - W) read from
    page table[b, p // P] at offset p % P; then the new token."""
    q, P, G = c["q"], c["P"], c["G"]
    B, H, d = q.shape
    out = torch.empty(B, H, d, dtype=torch.float64)
    for b in range(B):
        L = int(c["lens"][b])
        for h in range(H):
            g = h // (H // G)
            keys, vals = [], []
            for p in range(L - 1):
                if c["window"] and p < L - c["window"]:
                    continue
                page = int(c["table"][b, p // P])
                kb, vb = c["kc"][page, g, p % P], c["vc"][page, g, p % P]
                if c["ks"] is not None:
                    # float64 values: byte * s, or for multipliers byte / m
                    kf = kb.view(torch.float8_e4m3fn).double()
                    vf = vb.view(torch.float8_e4m3fn).double()
                    kms, vms = float(c["ks"][g]), float(c["vs"][g])
                    kb, vb = (kf / kms, vf / vms) if c["mul"] else (kf * kms, vf * vms)
                keys.append(kb.double())
                vals.append(vb.double())
            kn, vn = c["kn"][b, g], c["vn"][b, g]
            if c["ks"] is not None:
                kms, vms = float(c["ks"][g]), float(c["vs"][g])
                if c["mul"]:
                    # the decode write of the new token: the bf16 product, cast (attention_decode.py:259-260)
                    kn = torch.tensor(ofp8.e4m3fn_values()[_mul_bytes(kn, kms)]) / kms
                    vn = torch.tensor(ofp8.e4m3fn_values()[_mul_bytes(vn, vms)]) / vms
                else:
                    kn = ofp8.dequantize(ofp8.quantize(kn, kms), kms)
                    vn = ofp8.dequantize(ofp8.quantize(vn, vms), vms)
            keys.append(kn.double())
            vals.append(vn.double())
            sink = None if c["sinks"] is None else float(c["sinks"][h])
            out[b, h] = torch.tensor(_softmax_attend(q[b, h].double(), keys, vals, scale, sink))
    return out


def _mul_bytes(x, m: float) -> np.ndarray:
    """e4m3fn codes of bf16 x written with multiplier m, from the definitions: the exact product rounded to bf16's 8
    significant bits, clamped, cast by nearest-value search."""
    r = ofp8.bf16_round_spec(x.double().numpy() * m)
    return ofp8.e4m3fn_rne_spec(np.clip(r, -448.0, 448.0).astype(np.float32)).astype(np.int64)


def _oracle_gqa(c, scale):
    return oatt.paged_decode_gqa(c["q"], c["kc"], c["vc"], c["table"], c["lens"], c["kn"], c["vn"], sm_scale=scale,
                                 k_scale=c["ks"], v_scale=c["vs"], sinks=c["sinks"], window=c["window"],
                                 scales_multiply=c["mul"])


@pytest.mark.parametrize("fp8,window,sinks,mul", [(False, 0, False, False), (True, 0, False, False),
                                                  (True, 0, True, False), (False, 3, False, False),
                                                  (True, 4, True, False), (True, 0, True, True), (True, 4, True, True)])
def test_gqa_matches_float64_brute_force(fp8, window, sinks, mul):
    c = _gqa_case(11, fp8=fp8, window=window, sinks=sinks, mul=mul)
    scale = 1 / math.sqrt(8)
    got = _oracle_gqa(c, scale).double()
    want = _brute_gqa(c, scale)
    # the oracle rounds its output to bf16 once: half an ulp of bf16 at these magnitudes
    assert torch.allclose(got, want, atol=1e-2, rtol=8e-3), (got - want).abs().max()


def test_gqa_single_key_returns_its_value():
    c = _gqa_case(12)
    c["lens"] = torch.tensor([1, 1, 1])  # no prior: only the new token
    out = _oracle_gqa(c, 0.3)
    want = c["vn"].repeat_interleave(2, dim=1)  # head h reads KV head h // 2
    assert torch.equal(out, want)


def test_gqa_equal_keys_give_the_mean_of_values():
    c = _gqa_case(13)
    b, L = 2, int(c["lens"][2])
    key = c["kn"][b]
    for p in range(L - 1):  # every prior key of row 2 equal to the new key
        page = int(c["table"][b, p // c["P"]])
        c["kc"][page, :, p % c["P"]] = key
    out = _oracle_gqa(c, 0.5)[b].float()
    vals = [c["vc"][int(c["table"][b, p // c["P"]]), :, p % c["P"]].float() for p in range(L - 1)]
    vals.append(c["vn"][b].float())
    mean = torch.stack(vals).mean(0).repeat_interleave(2, dim=0)
    assert torch.allclose(out, mean, atol=8e-3, rtol=8e-3)


def test_gqa_minus_inf_sink_is_no_sink_and_wide_window_is_full():
    c = _gqa_case(14, sinks=True)
    base = _oracle_gqa(dict(c, sinks=None), 0.4)
    assert torch.equal(_oracle_gqa(dict(c, sinks=torch.full((4,), float("-inf"))), 0.4), base)
    assert torch.equal(_oracle_gqa(dict(c, sinks=None, window=100), 0.4), base)
    # a finite sink only shrinks the weights: the output moves toward 0
    with_sink = _oracle_gqa(dict(c, sinks=torch.full((4,), 3.0)), 0.4).float()
    assert bool((with_sink.abs() <= base.float().abs() + 1e-2).all())


def test_gqa_fp8_scale_one_on_representable_values_is_the_bf16_result():
    c = _gqa_case(15)
    vals = torch.tensor(ofp8.e4m3fn_values(), dtype=torch.float32)
    vals = vals[vals.abs() <= 4]
    g = torch.Generator().manual_seed(9)
    for key in ("kc", "vc"):
        pick = vals[torch.randint(0, vals.numel(), c[key].shape, generator=g)]
        c[key] = pick.to(torch.bfloat16)
    for key in ("kn", "vn"):
        c[key] = vals[torch.randint(0, vals.numel(), c[key].shape, generator=g)].to(torch.bfloat16)
    bf = _oracle_gqa(c, 0.35)
    f8 = dict(c, kc=ofp8.quantize(c["kc"], 1.0), vc=ofp8.quantize(c["vc"], 1.0), ks=torch.ones(2), vs=torch.ones(2))
    assert torch.equal(_oracle_gqa(f8, 0.35), bf)


def test_gqa_page_permutation_invariance():
    c = _gqa_case(16, fp8=True)
    nb = c["kc"].shape[0]
    g = torch.Generator().manual_seed(17)
    perm = torch.cat([torch.zeros(1, dtype=torch.long), torch.randperm(nb - 1, generator=g) + 1])  # new id of page i
    kc2, vc2 = torch.empty_like(c["kc"]), torch.empty_like(c["vc"])
    kc2[perm], vc2[perm] = c["kc"], c["vc"]
    table2 = torch.where(c["table"] >= 0, perm[c["table"].clamp(min=0).long()].to(torch.int32), c["table"])
    assert torch.equal(_oracle_gqa(dict(c, kc=kc2, vc=vc2, table=table2), 0.3), _oracle_gqa(c, 0.3))


def test_lse_merge_of_splits_is_the_whole():
    g = torch.Generator().manual_seed(18)
    q, keys, vals = torch.randn(8, generator=g), torch.randn(20, 8, generator=g), torch.randn(20, 5, generator=g)
    s = keys @ q
    full = torch.softmax(s, 0) @ vals
    parts, lses = [], []
    for lo, hi in ((0, 7), (7, 13), (13, 20)):
        ss = s[lo:hi]
        parts.append((torch.softmax(ss, 0) @ vals[lo:hi])[None])
        lses.append(torch.logsumexp(ss, 0).reshape(1))
    out, lse = oatt.lse_merge(torch.stack(parts), torch.stack(lses))
    assert torch.allclose(out.float().reshape(-1), full, atol=1e-2)
    assert torch.allclose(lse.reshape(-1), torch.logsumexp(s, 0).reshape(-1), atol=1e-5)


def _mla_case(seed, B=2, H=3, P=4):
    g = torch.Generator().manual_seed(seed)
    lens = [3, 9][:B]
    pages = [(L + P - 1) // P for L in lens]
    nb = sum(pages) + 1
    table = torch.full((B, max(pages)), -1, dtype=torch.int32)
    perm = (torch.randperm(nb - 1, generator=g) + 1).tolist()
    o = 0
    for b, n in enumerate(pages):
        table[b, :n] = torch.tensor(perm[o:o + n], dtype=torch.int32)
        o += n
    cache = torch.zeros(nb * P, 576, dtype=torch.uint8)
    scale = torch.zeros(nb * P)
    slots = [int(table[b, p // P]) * P + p % P for b, L in enumerate(lens) for p in range(L - 1)]
    rows = _bf16((len(slots), 576), g)
    ost.kv_store_mla(rows, torch.tensor(slots), cache, scale)
    return dict(ql=_bf16((B, H, 512), g), qpe=_bf16((B, H, 64), g), cache=cache, scale=scale, table=table,
                lens=torch.tensor(lens), new=_bf16((B, 576), g), P=P)


def test_mla_matches_float64_brute_force():
    c = _mla_case(21)
    sm = 1 / math.sqrt(192)
    got = oatt.mla_decode(c["ql"], c["qpe"], c["cache"], c["scale"], c["table"], c["lens"], c["new"], sm_scale=sm,
                          page_size=c["P"]).double()
    B, H, _ = c["ql"].shape
    for b in range(B):
        L = int(c["lens"][b])
        keys = []
        for p in range(L - 1):
            s = int(c["table"][b, p // c["P"]]) * c["P"] + p % c["P"]
            keys.append(ofp8.dequantize(c["cache"][s], float(c["scale"][s])).double())
        ns = float(ofp8.absmax_scale(c["new"][b], dims=-1))
        keys.append(ofp8.dequantize(ofp8.quantize(c["new"][b], ns), ns).double())
        for h in range(H):
            q = torch.cat([c["ql"][b, h], c["qpe"][b, h]]).double()
            want = _softmax_attend(q, keys, [k[:512] for k in keys], sm)
            assert torch.allclose(got[b, h], torch.tensor(want, dtype=torch.float64), atol=1e-2, rtol=8e-3)


def test_dsa_all_prior_indices_match_a_dense_brute_force():
    g = torch.Generator().manual_seed(31)
    B, H, P, per = 2, 2, 4, 12
    W = per // P
    table = torch.tensor([[3, 1, 5], [2, 6, 4]], dtype=torch.int32)
    cache = torch.zeros(7 * P, 640, dtype=torch.uint8)
    kv = 0.5
    for b in range(B):
        slots = torch.tensor([int(table[b, p // P]) * P + p % P for p in range(per)])
        ost.kv_store_dsa(_bf16((per, 576), g), slots, cache, kv)
    positions = torch.tensor([7, 11], dtype=torch.int32)
    idx = torch.full((B, per), -1, dtype=torch.int32)
    for b in range(B):
        idx[b, :int(positions[b])] = torch.arange(int(positions[b]))  # every prior position
    own = _bf16((B, 576), g)
    new_slots = torch.tensor([int(table[b, int(positions[b]) // P]) * P + int(positions[b]) % P for b in range(B)])
    qa, qpe = _bf16((B, H, 512), g), _bf16((B, H, 64), g)
    ctx, lse, cache2 = oatt.mla_decode_sparse(qa, qpe, cache, kv, idx, table, positions, own, new_slots,
                                              sm_scale=0.0625, page_size=P)
    for b in range(B):
        keys = []
        for p in range(int(positions[b]) + 1):  # the prior positions, then the own row (stored at its position)
            s = int(table[b, p // P]) * P + p % P
            row = ost.unpack_kv_row(cache2[s][None], kv)[0].double()  # [k_pe | latent]
            keys.append(row)
        for h in range(H):
            q = torch.cat([qpe[b, h], qa[b, h]]).double()
            want = _softmax_attend(q, keys, [k[64:] for k in keys], 0.0625)
            assert torch.allclose(ctx[b, h].double(), torch.tensor(want, dtype=torch.float64), atol=1e-2, rtol=8e-3)
            s = [float((q * k).sum()) * 0.0625 for k in keys]
            assert float(lse[b, h]) == pytest.approx(float(torch.logsumexp(torch.tensor(s), 0)), abs=1e-4)


@pytest.mark.parametrize("spec", [1, 3])
def test_dsa_speculative_tokens_match_a_float64_brute_force(spec):
    """spec query tokens per sequence (MTP verify): token j of sequence s attends its own index list through table
    row s, then every own row of its sequence at that token's position, kept iff at or before its own (so its
    earlier siblings and itself), each key decoded from its packed bytes; by explicit float64 loops over keys."""
    g = torch.Generator().manual_seed(40 + spec)
    S, H, P, K, kv = 2, 2, 4, 6, 0.25
    B = S * spec
    table = torch.tensor([[3, 1, 5, 8], [2, 6, 4, 7]], dtype=torch.int32)
    cache = torch.zeros(9 * P, 640, dtype=torch.uint8)
    base = [9, 5]  # each sequence's first speculative position; its prior is positions < base
    for s_ in range(S):
        slots = torch.tensor([int(table[s_, p // P]) * P + p % P for p in range(base[s_])])
        ost.kv_store_dsa(_bf16((base[s_], 576), g), slots, cache, kv)
    positions = torch.tensor([base[b // spec] + b % spec for b in range(B)], dtype=torch.int32)
    idx = torch.full((B, K), -1, dtype=torch.int32)
    for b in range(B):
        prior = base[b // spec]
        sel = torch.randperm(prior, generator=g)[:K - 1]
        idx[b, :sel.numel()] = sel.to(torch.int32)
    idx[0, K - 1] = 30  # a block past the table's width: dropped
    own = _bf16((B, 576), g)
    new_slots = torch.tensor([int(table[b // spec, int(positions[b]) // P]) * P + int(positions[b]) % P
                              for b in range(B)])
    qa, qpe = _bf16((B, H, 512), g), _bf16((B, H, 64), g)
    ctx, lse, cache2 = oatt.mla_decode_sparse(qa, qpe, cache, kv, idx, table, positions, own, new_slots,
                                              sm_scale=0.0625, page_size=P, spec=spec)
    packed = ost.pack_kv_rows(own, kv)
    for b in range(B):
        s_, qpos = b // spec, int(positions[b])
        keys = []
        for e in idx[b].tolist():
            if e < 0 or e // P >= table.shape[1] or e > qpos:
                continue
            r = int(table[s_, e // P]) * P + e % P
            keys.append(ost.unpack_kv_row(cache2[r][None], kv)[0].double())
        for i in range(spec):  # the sequence's own rows, at their positions
            if int(positions[s_ * spec + i]) <= qpos:
                keys.append(ost.unpack_kv_row(packed[s_ * spec + i][None], kv)[0].double())
        assert len(keys) == sum(1 for e in idx[b].tolist() if 0 <= e <= qpos and e // P < 4) + b % spec + 1
        for h in range(H):
            q = torch.cat([qpe[b, h], qa[b, h]]).double()
            want = _softmax_attend(q, keys, [k[64:] for k in keys], 0.0625)
            assert torch.allclose(ctx[b, h].double(), torch.tensor(want, dtype=torch.float64), atol=1e-2, rtol=8e-3)
            sc = [float((q * k).sum()) * 0.0625 for k in keys]
            assert float(lse[b, h]) == pytest.approx(float(torch.logsumexp(torch.tensor(sc), 0)), abs=1e-4)


def test_block_table_by_hand():
    page = 4
    r2t = np.arange(6 * 40, dtype=np.int64).reshape(6, 40) * 3 % 997
    rows, lens = np.array([4, 1, 2]), np.array([9, 1, 16])
    got = omd.block_table(r2t, rows, lens, page).numpy()
    want = np.full((3, 4), -1)
    for i, (r, L) in enumerate(zip(rows, lens)):
        for j in range(4):
            if j * page < L:
                want[i, j] = r2t[r, j * page] // page
    assert np.array_equal(got, want)
    one = omd.block_table(r2t, np.array([5]), np.array([3]), page).numpy()  # one row: no -1
    assert np.array_equal(one, [[r2t[5, 0] // page]])


def test_swa_trimmed_table_by_hand():
    table = torch.arange(1, 11, dtype=torch.int32).reshape(1, 10)
    trimmed, off = omd.swa_trimmed_table(table, torch.tensor([37]), window=8, page=4, width=3)
    # ctx 36 -> column 9 is the last; start = 9 - 3 + 1 = 7
    assert trimmed.tolist() == [[8, 9, 10]] and off.tolist() == [28]
    trimmed, off = omd.swa_trimmed_table(table, torch.tensor([5]), window=8, page=4, width=3)
    assert trimmed.tolist() == [[1, 2, 3]] and off.tolist() == [0]


def _prefill_case(seed, H=4, G=2, d=8, P=4, priors=(7, 0, 3), lens=(5, 3, 6), nb=40, fp8=False):
    g = torch.Generator().manual_seed(seed)
    R = len(priors)
    width = max(-(-(p + s) // P) for p, s in zip(priors, lens)) + 1
    perm = torch.randperm(nb - 1, generator=g) + 1
    table = torch.full((R, width), -1, dtype=torch.int32)
    used = 0
    for r, (p, s) in enumerate(zip(priors, lens)):
        n = -(-(p + s) // P)
        table[r, :n] = perm[used:used + n].to(torch.int32)
        used += n
    kf = torch.randn(nb, G, P, d, generator=g)
    vf = torch.randn(nb, G, P, d, generator=g)
    if fp8:
        ks, vs = torch.rand(G, generator=g) * 0.02 + 0.005, torch.rand(G, generator=g) * 0.02 + 0.005
        kc = ofp8.quantize(kf, ks.reshape(1, G, 1, 1))
        vc = ofp8.quantize(vf, vs.reshape(1, G, 1, 1))
    else:
        ks = vs = None
        kc, vc = kf.to(torch.bfloat16), vf.to(torch.bfloat16)
    T = sum(lens)
    q = torch.randn(T, H, d, generator=g).to(torch.bfloat16)
    q_start = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)
    return q, kc, vc, table, q_start, torch.tensor(priors, dtype=torch.int32), ks, vs


@pytest.mark.parametrize("window", [0, 3])
@pytest.mark.parametrize("sinks", [False, True])
def test_segmented_prefill_brute_force(window, sinks):
    """Explicit float64 loops over (request, query, head, key) on a tiny case."""
    q, kc, vc, table, q_start, priors, _, _ = _prefill_case(11)
    H, d, P, G = q.shape[1], q.shape[2], kc.shape[2], kc.shape[1]
    sk = torch.randn(H) if sinks else None
    got = oatt.segmented_prefill(q, kc, vc, table, q_start, priors, sm_scale=0.3, sinks=sk, window=window)
    for r in range(len(priors)):
        for i in range(int(q_start[r + 1] - q_start[r])):
            row, pos = int(q_start[r]) + i, int(priors[r]) + i
            for h in range(H):
                kvh = h // (H // G)
                logits, vals = [], []
                for k in range(pos + 1):
                    if window and k <= pos - window:
                        continue
                    page = int(table[r, k // P])
                    kk = kc[page, kvh, k % P].double()
                    logits.append(float((q[row, h].double() * kk).sum()) * 0.3)
                    vals.append(vc[page, kvh, k % P].double())
                m = max(logits + ([float(sk[h])] if sinks else []))
                w = [math.exp(x - m) for x in logits]
                den = sum(w) + (math.exp(float(sk[h]) - m) if sinks else 0.0)
                want = sum(wi * v for wi, v in zip(w, vals)) / den
                assert torch.allclose(got[row, h].double(), want, atol=1e-2, rtol=8e-3), (r, i, h)


@pytest.mark.parametrize("fp8", [False, True])
def test_segmented_prefill_last_query_is_the_decode_of_its_position(fp8):
    """The chunk's last query sees exactly what a decode of that position sees (its own token as the new key):
    oracle/attention.segmented_prefill against oracle/attention.paged_decode_gqa, itself pinned above."""
    q, kc, vc, table, q_start, priors, ks, vs = _prefill_case(5, priors=(9, 0, 14), lens=(4, 6, 2), fp8=fp8)
    G, P = kc.shape[1], kc.shape[2]
    sk = torch.randn(q.shape[1])
    for window in (0, 5):
        got = oatt.segmented_prefill(q, kc, vc, table, q_start, priors, sm_scale=0.25, k_scale=ks, v_scale=vs,
                                     sinks=sk, window=window)
        for r in range(len(priors)):
            last, L = int(q_start[r + 1]) - 1, int(priors[r] + q_start[r + 1] - q_start[r])
            page, off = int(table[r, (L - 1) // P]), (L - 1) % P
            deq = (lambda c, s: ofp8.dequantize(c[page, :, off], s.reshape(G, 1))) if fp8 else \
                (lambda c, s: c[page, :, off].float())
            # the new token's K/V as the decode receives them: the pool's values (exact under quantize for FP8)
            kn, vn = deq(kc, ks), deq(vc, vs)
            want = oatt.paged_decode_gqa(q[last:last + 1], kc, vc, table[r:r + 1], torch.tensor([L]),
                                         kn.unsqueeze(0).to(torch.bfloat16) if not fp8 else kn.unsqueeze(0),
                                         vn.unsqueeze(0).to(torch.bfloat16) if not fp8 else vn.unsqueeze(0),
                                         sm_scale=0.25, k_scale=ks, v_scale=vs, sinks=sk, window=window)
            assert torch.allclose(got[last].float(), want[0].float(), atol=1e-2, rtol=1e-2), (r, window)


def test_segmented_prefill_is_chunking_invariant():
    """One chunk of 9 tokens == chunks of 4 and 5 (the second at prior + 4) over the same pool."""
    q, kc, vc, table, _, _, _, _ = _prefill_case(8, priors=(6,), lens=(9,))
    whole = oatt.segmented_prefill(q, kc, vc, table, torch.tensor([0, 9]), torch.tensor([6]), sm_scale=0.5, window=4)
    two = oatt.segmented_prefill(q, kc, vc, table.repeat(2, 1), torch.tensor([0, 4, 9]), torch.tensor([6, 10]),
                                 sm_scale=0.5, window=4)
    assert torch.equal(whole, two)


def _multi_case(seed, B=2, S=3, H=4, G=2, d=8, P=4, mul=True):
    """Rows of S active tokens over a small FP8 pool (GPT-OSS multipliers) or a bf16 one."""
    g = torch.Generator().manual_seed(seed)
    lens = [9, 14][:B]
    pages = [(L + P - 1) // P for L in lens]
    nb = sum(pages) + 2
    perm = (torch.randperm(nb - 1, generator=g) + 1).tolist()
    table = torch.full((B, max(pages)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        table[b, :n] = torch.tensor(perm[o:o + n], dtype=torch.int32)
        o += n
    fp8 = mul is not None
    ks = torch.rand(G, generator=g) * 0.01 + 0.004 if fp8 else None
    vs = torch.rand(G, generator=g) * 0.01 + 0.004 if fp8 else None
    if mul:
        ks, vs = ofp8.inverted_scale(ks), ofp8.inverted_scale(vs)
    dt = torch.uint8 if fp8 else torch.bfloat16
    kc, vc = torch.zeros(nb, G, P, d, dtype=dt), torch.zeros(nb, G, P, d, dtype=dt)
    slots = [int(table[b, p // P]) * P + p % P for b, L in enumerate(lens) for p in range(L - S)]
    T = len(slots)
    ost.kv_store_mha(_bf16((T, G, d), g), _bf16((T, G, d), g), torch.tensor(slots), kc, vc, ks, vs, bool(mul))
    q, kn, vn = _bf16((B, S, H, d), g), _bf16((B, S, G, d), g), _bf16((B, S, G, d), g)
    new = torch.tensor([[int(table[b, p // P]) * P + p % P for p in range(L - S, L)] for b, L in enumerate(lens)])
    return dict(q=q, kc=kc, vc=vc, table=table, lens=torch.tensor(lens), kn=kn, vn=vn, ks=ks, vs=vs, new=new,
                P=P, G=G, mul=bool(mul))


@pytest.mark.parametrize("mul,window,sinks", [(True, 0, True), (True, 5, True), (None, 0, False), (False, 6, False)])
def test_gqa_multi_token_matches_float64_brute_force(mul, window, sinks):
    """S active tokens per row (attention_decode.py with X [B, S, Hd]): token j of row b (position L - S + j) attends
    the prior positions < L - S on the row's pages (within its window) and active tokens 0 .. j as their FP8-rounded
    values; explicit float64 loops over keys."""
    c = _multi_case(51, mul=mul)
    B, S, H, d = c["q"].shape
    G, P = c["G"], c["P"]
    sk = torch.randn(H, generator=torch.Generator().manual_seed(3)) if sinks else None
    got = oatt.paged_decode_gqa_multi(c["q"], c["kc"], c["vc"], c["table"], c["lens"], c["kn"], c["vn"],
                                      sm_scale=0.35, k_scale=c["ks"], v_scale=c["vs"], sinks=sk, window=window,
                                      scales_multiply=c["mul"])
    vals = ofp8.e4m3fn_values()
    for b in range(B):
        L = int(c["lens"][b])
        for j in range(S):
            pos = L - S + j
            for h in range(H):
                g_ = h // (H // G)
                keys, vv = [], []
                for p in range(L - S):
                    if window and p < pos - window + 1:
                        continue
                    pg = int(c["table"][b, p // P])
                    kb, vb = c["kc"][pg, g_, p % P], c["vc"][pg, g_, p % P]
                    if c["ks"] is not None:  # byte / m for multipliers, byte * s for dequantization scales
                        kms, vms = float(c["ks"][g_]), float(c["vs"][g_])
                        kf, vf = torch.tensor(vals[kb.long().numpy()]), torch.tensor(vals[vb.long().numpy()])
                        kb, vb = (kf / kms, vf / vms) if c["mul"] else (kf * kms, vf * vms)
                    keys.append(kb.double())
                    vv.append(vb.double())
                for i in range(j + 1):  # the active tokens up to this one, as the cache holds them
                    kn, vn = c["kn"][b, i, g_], c["vn"][b, i, g_]
                    if c["ks"] is not None:
                        kms, vms = float(c["ks"][g_]), float(c["vs"][g_])
                        if c["mul"]:
                            kn = torch.tensor(vals[_mul_bytes(kn, kms)]) / kms
                            vn = torch.tensor(vals[_mul_bytes(vn, vms)]) / vms
                        else:
                            kn = torch.tensor(vals[ofp8.e4m3fn_rne_spec(np.clip(kn.float().numpy() / np.float32(kms),
                                                                                 -448, 448)).astype(np.int64)]) * kms
                            vn = torch.tensor(vals[ofp8.e4m3fn_rne_spec(np.clip(vn.float().numpy() / np.float32(vms),
                                                                                 -448, 448)).astype(np.int64)]) * vms
                    keys.append(kn.double())
                    vv.append(vn.double())
                want = _softmax_attend(c["q"][b, j, h].double(), keys, vv, 0.35,
                                       None if sk is None else float(sk[h]))
                assert torch.allclose(got[b, j, h].double(), torch.tensor(want, dtype=torch.float64), atol=1e-2, rtol=8e-3), (b, j, h)


def test_gqa_multi_token_is_stored_tokens_then_one_row_per_token():
    """The decomposition the HIP path runs: store the S tokens, then decode token j as a row whose length ends at it
    (its earlier active tokens read back from the pool) gives the multi-token oracle's outputs."""
    c = _multi_case(52, mul=True)
    B, S, H, d = c["q"].shape
    want = oatt.paged_decode_gqa_multi(c["q"], c["kc"], c["vc"], c["table"], c["lens"], c["kn"], c["vn"],
                                       sm_scale=0.35, k_scale=c["ks"], v_scale=c["vs"], window=7, scales_multiply=True)
    kc, vc = c["kc"].clone(), c["vc"].clone()
    ost.kv_store_mha(c["kn"].reshape(B * S, c["G"], d), c["vn"].reshape(B * S, c["G"], d), c["new"].reshape(-1), kc,
                     vc, c["ks"], c["vs"], True)
    lens = (c["lens"].reshape(B, 1) - S + 1 + torch.arange(S)).reshape(-1)
    got = oatt.paged_decode_gqa(c["q"].reshape(B * S, H, d), kc, vc, c["table"].repeat_interleave(S, 0), lens,
                                c["kn"].reshape(B * S, c["G"], d), c["vn"].reshape(B * S, c["G"], d), sm_scale=0.35,
                                k_scale=c["ks"], v_scale=c["vs"], window=7, scales_multiply=True)
    assert torch.allclose(got.reshape(B, S, H, d).float(), want.float(), atol=1e-2)
    assert float((got.reshape(B, S, H, d).float() - want.float()).abs().max()) <= 2 ** -7


def test_gqa_multi_token_with_one_token_is_the_single_token_decode():
    c = _multi_case(53, S=1, mul=True)
    B, S, H, d = c["q"].shape
    a = oatt.paged_decode_gqa_multi(c["q"], c["kc"], c["vc"], c["table"], c["lens"], c["kn"], c["vn"], sm_scale=0.35,
                                    k_scale=c["ks"], v_scale=c["vs"], scales_multiply=True)
    b = oatt.paged_decode_gqa(c["q"][:, 0], c["kc"], c["vc"], c["table"], c["lens"], c["kn"][:, 0], c["vn"][:, 0],
                              sm_scale=0.35, k_scale=c["ks"], v_scale=c["vs"], scales_multiply=True)
    assert torch.equal(a[:, 0], b)
