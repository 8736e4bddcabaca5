"""GQA decode parity: the HIP split-K decode (+ combine + fused store) against the oracle on seeded cases of cfg1,
cfg2 and cfg4 (full and sliding-window layers), plus the edge cases the reference's path has."""

import pytest
import torch

from sglang_neuron_amd import workloads
from tests.conftest import announce
from tests._harness import assert_close_attn, cache_bytes, gqa_gpu_decode, gqa_gpu_pool, gqa_oracle

pytestmark = pytest.mark.gpu

CASES = [
    ("cfg1", 1, {}),                                                     # full size: B8 H16 G8 d128 bf16
    ("cfg2-small", 2, {"B": 4, "lens": (4096, 4096)}),                    # FP8 per-head, L=4096, 4 rows
    ("cfg2-ragged", 2, {"B": 6, "lens": (1, 700)}),
    ("cfg4-full", 4, {"B": 6}),                                          # sinks, d64, group 8
    ("cfg4-swa", 4, {"B": 6, "window": workloads.SWA_WINDOW}),
    ("cfg4-swa-short", 4, {"B": 5, "window": 128, "lens": (1, 200)}),
    ("bf16-d64-g1", 1, {"B": 3, "H": 4, "G": 4, "d": 64, "lens": (2, 300)}),
    ("fp8-g16", 2, {"B": 2, "H": 32, "G": 2, "lens": (33, 900)}),
    ("fp8-page64", 2, {"B": 3, "P": 64, "lens": (50, 1500)}),
    # page 128: the page the reference serves Qwen3 with (docs/model-recipes/qwen3.md:126)
    ("cfg2-page128", 2, {"B": 8, "P": 128, "lens": (2000, 4096)}),
    ("bf16-page128", 1, {"B": 5, "P": 128, "lens": (100, 3000)}),
    ("cfg4-page128-sinks", 4, {"B": 6, "P": 128, "lens": (1000, 5000)}),
    # page sizes that are multiples of 16 but not powers of two (columns and in-page slots by division)
    ("fp8-page48", 2, {"B": 4, "P": 48, "lens": (50, 2000)}),
    ("cfg4-swa-page48", 4, {"B": 5, "P": 48, "window": 128, "lens": (1, 3000)}),
    ("bf16-page80", 1, {"B": 3, "P": 80, "lens": (2, 900)}),
    ("cfg2-32-splits", 2, {"B": 2, "lens": (8192, 8192)}),                # the combine's second chunk of 16 splits
    ("cfg4-64-splits", 4, {"B": 2, "lens": (8000, 8192)}),                # 4 chunks, sinks
    # GPT-OSS multipliers on other shapes (cfg4 itself runs with them): 8 KV heads, d128, and no sinks
    ("multiplier-g8-d128", 2, {"B": 4, "lens": (300, 1500), "scales_multiply": True}),
    ("multiplier-cfg4-no-sinks", 4, {"B": 5, "lens": (1, 900), "sinks": False}),
    # the bench workloads at their full sizes (the metric's cfg2 included): same seeds, same split plans
    ("cfg2-full", 2, {}),
    ("cfg4-full-size", 4, {}),
    ("cfg4-swa-full-size", 4, {"window": workloads.SWA_WINDOW}),
]


@pytest.mark.parametrize("name,cfg,over", CASES, ids=[c[0] for c in CASES])
def test_gqa_decode_matches_oracle(name, cfg, over):
    case = workloads.gqa_case(cfg, overrides=over)
    want, kc_o, vc_o, ks_o, vs_o = gqa_oracle(case)
    announce(f"gqa {name}: B={case.B} H={case.H} G={case.G} d={case.d} P={case.P} fp8={case.fp8} "
             f"window={case.window} lens={case.seq_lens.tolist()[:8]}")
    kc, vc, ks, vs = gqa_gpu_pool(case)
    if case.fp8:
        assert torch.equal(ks.cpu(), ks_o) and torch.equal(vs.cpu(), vs_o)
    out = gqa_gpu_decode(case, kc, vc, ks, vs)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    # the pool after the step (prefill + the fused store of the new token) is bit-exact
    assert torch.equal(cache_bytes(kc), cache_bytes(kc_o)), "K pool differs"
    assert torch.equal(cache_bytes(vc), cache_bytes(vc_o)), "V pool differs"


def test_gqa_single_token_rows():
    """seq_len 1 (a padding row reading nothing but its own token): the output is the new token's value."""
    case = workloads.gqa_case(2, overrides={"B": 3, "lens": (1, 1)})
    announce("gqa seq_len 1")
    want, *_ = gqa_oracle(case)
    kc, vc, ks, vs = gqa_gpu_pool(case)
    out = gqa_gpu_decode(case, kc, vc, ks, vs)
    assert_close_attn(out, want, "seq_len 1")


def test_gqa_page_permutation_invariance():
    """Moving pages to other physical ids (and the table with them) leaves the output bit-identical."""
    case = workloads.gqa_case(2, overrides={"B": 3, "lens": (500, 1200)})
    announce("gqa page permutation")
    kc, vc, ks, vs = gqa_gpu_pool(case)
    out1 = gqa_gpu_decode(case, kc, vc, ks, vs, store_new=False)
    perm = torch.randperm(case.num_blocks - 1, generator=torch.Generator().manual_seed(3)) + 1
    inv = torch.zeros(case.num_blocks, dtype=torch.int64)
    inv[perm] = torch.arange(1, case.num_blocks)
    kc2 = kc.clone()
    vc2 = vc.clone()
    kc2[inv[1:].cuda()] = kc[1:]
    vc2[inv[1:].cuda()] = vc[1:]
    t = case.block_table.clone().to(torch.int64)
    t = torch.where(t > 0, inv[t.clamp(min=0)], t).to(torch.int32)
    case.block_table = t
    out2 = gqa_gpu_decode(case, kc2, vc2, ks, vs, store_new=False)
    assert torch.equal(out1.cpu(), out2.cpu())


def test_gqa_invalid_pages_are_masked():
    """-1 table entries inside a row's range hide those keys, as the reference's visibility mask does."""
    case = workloads.gqa_case(1, overrides={"B": 2, "lens": (300, 300)})
    case.block_table[0, 3] = -1
    case.block_table[1, 0] = -1
    want, *_ = gqa_oracle(case)
    announce("gqa -1 pages")
    kc, vc, ks, vs = gqa_gpu_pool(case)
    out = gqa_gpu_decode(case, kc, vc, ks, vs)
    assert_close_attn(out, want, "-1 pages")


@pytest.mark.parametrize("window", [0, 100], ids=["full", "window100"])
@pytest.mark.parametrize("mapped", [True, False], ids=["item-map", "located"])
def test_plan_for_longer_rows_still_attends_and_stores_the_own_token(mapped, window):
    """A plan made for longer rows than the device holds (its last splits cover no key of the device's rows) still
    attends and stores every row's own token: the last split the launch runs for a row takes it, whether the plan
    carries an item map (host lengths) or the items are located from the device's lengths (a bound). The rows are
    longer by 2048 keys, a whole number of tiles, so with a window each row spans as many tiles as the plan's rows
    (a window's tile count depends on where it starts inside a tile; the plan is then valid for the device's lengths,
    as check_plan_lengths confirms), while its splits start elsewhere: the launch places them by the device's
    lengths."""
    from sglang_neuron_amd import ops

    case = workloads.gqa_case(2, overrides={"B": 4, "lens": (300, 900), "window": window})
    want, kc_o, vc_o, ks_o, vs_o = gqa_oracle(case)
    announce(f"gqa plan for longer rows mapped={mapped} window={window} lens={case.seq_lens.tolist()}")
    kc, vc, ks, vs = gqa_gpu_pool(case)
    longer = (case.seq_lens + 2048).tolist()
    if mapped:
        plan = ops.plan_decode(0, case.B, host_seq_lens=longer, window=window, ctas_per_item=case.G, num_cus=256)
        assert plan.work_n > 0
        ops.check_plan_lengths(plan, 0, case.seq_lens, window)
    else:
        plan = ops.plan_decode(0, case.B, max_seq_len=max(longer), window=window, ctas_per_item=case.G, num_cus=256)
        assert plan.work_n == 0
    assert window or plan.max_splits > 1
    out = ops.paged_decode_gqa(case.q.cuda(), kc, vc, case.block_table.cuda(), case.seq_lens.cuda(), case.k_new.cuda(),
                               case.v_new.cuda(), sm_scale=case.sm_scale, k_scale=ks, v_scale=vs, window=window,
                               new_slots=case.new_slots.cuda(), plan=plan)
    torch.cuda.synchronize()
    assert_close_attn(out, want, "plan for longer rows")
    assert torch.equal(cache_bytes(kc), cache_bytes(kc_o)), "K pool differs"
    assert torch.equal(cache_bytes(vc), cache_bytes(vc_o)), "V pool differs"


BOUND = [("cfg4-full-size", 4, {}, 8192),                                   # the bench's bound plan: 128 rows
         ("cfg4-swa", 4, {"B": 40, "window": workloads.SWA_WINDOW}, 8192),
         ("cfg2-ragged", 2, {"B": 20, "lens": (1, 3000)}, 4096),
         ("cfg1", 1, {}, 1024),
         ("cfg2-one-row-at-bound", 2, {"B": 3, "lens": (16, 16)}, 16),
         ("cfg4-300-rows", 4, {"B": 300, "lens": (1, 600)}, 2048),
         # rows of their own token only (no prior key: a split of no tile), beside rows of one tile
         ("cfg2-own-token-rows", 2, {"B": 70, "lens": (1, 3)}, 64),
         ("cfg1-short-final", 1, {"B": 9, "lens": (1, 200)}, 256)]                # one split a row, no combine


@pytest.mark.parametrize("name,cfg,over,bound", BOUND, ids=[b[0] for b in BOUND])
def test_gqa_device_split_plan_matches_oracle(name, cfg, over, bound):
    """A plan from a length bound splits on the device: every launch sizes its splits from the device's seq_lens
    (gqa_split_tiles). Against the oracle, pools bit-exact, on full, sliding-window, ragged and single-tile rows."""
    from sglang_neuron_amd import ops

    case = workloads.gqa_case(cfg, overrides=over)
    want, kc_o, vc_o, ks_o, vs_o = gqa_oracle(case)
    plan = ops.plan_decode(0, case.B, max_seq_len=bound, window=case.window, ctas_per_item=case.G,
                           num_cus=ops._num_cus(torch.device("cuda", 0)))
    announce(f"gqa device split {name}: B={case.B} bound={bound} n_work={plan.n_work} max_splits={plan.max_splits}")
    assert plan.device_split == 1 and plan.work_n == 0
    kc, vc, ks, vs = gqa_gpu_pool(case)
    out = ops.paged_decode_gqa(case.q.cuda(), kc, vc, case.block_table.cuda(), case.seq_lens.cuda(), case.k_new.cuda(),
                               case.v_new.cuda(), sm_scale=case.sm_scale, k_scale=ks, v_scale=vs,
                               sinks=None if case.sinks is None else case.sinks.cuda(), window=case.window,
                               new_slots=case.new_slots.cuda(), plan=plan, host_seq_lens=case.seq_lens,
                               scales_multiply=case.scales_multiply)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    assert torch.equal(cache_bytes(kc), cache_bytes(kc_o)), "K pool differs"
    assert torch.equal(cache_bytes(vc), cache_bytes(vc_o)), "V pool differs"


MULTI = [("cfg4-s4", 4, {"B": 8, "lens": (100, 3000)}, 4),                  # GPT-OSS multipliers, sinks
         ("cfg4-swa-s8", 4, {"B": 6, "lens": (2, 900), "window": 128}, 8),
         ("cfg2-s3", 2, {"B": 4, "lens": (40, 1000)}, 3),
         ("cfg1-bf16-s2", 1, {"B": 3, "lens": (30, 400)}, 2)]


@pytest.mark.parametrize("name,cfg,over,S", MULTI, ids=[m[0] for m in MULTI])
def test_gqa_multi_token_decode_matches_oracle(name, cfg, over, S):
    """S active tokens per row (the GPT-OSS decode's X [B, S, Hd]): the last S positions of each row are the step's
    tokens, stored by the call and attended causally; against oracle.paged_decode_gqa_multi, pools bit-exact."""
    from oracle import attention as oatt
    from oracle import store as ost
    from sglang_neuron_amd import ops

    case = workloads.gqa_case(cfg, overrides=over)
    B, G, d, P, H = case.B, case.G, case.d, case.P, case.H
    lens = case.seq_lens.clamp(min=S)
    # the prior tokens by (row, position); each row's last S positions become its active tokens
    k_at, v_at, k = {}, {}, 0
    for b, L in enumerate(case.seq_lens.tolist()):
        for pos in range(L - 1):
            k_at[(b, pos)], v_at[(b, pos)] = case.k_prior[k], case.v_prior[k]
            k += 1
        k_at[(b, L - 1)], v_at[(b, L - 1)] = case.k_new[b], case.v_new[b]
    g = torch.Generator().manual_seed(77)
    z = torch.zeros(G, d, dtype=torch.bfloat16)
    k_act = torch.stack([torch.stack([k_at.get((b, int(L) - S + j), z) for j in range(S)]) for b, L in enumerate(lens)])
    v_act = torch.stack([torch.stack([v_at.get((b, int(L) - S + j), z) for j in range(S)]) for b, L in enumerate(lens)])
    q = torch.randn(B, S, H, d, generator=g).to(torch.bfloat16)
    slot_of = lambda b, pos: int(case.block_table[b, pos // P]) * P + pos % P  # noqa: E731
    prior = [(b, pos) for b, L in enumerate(lens.tolist()) for pos in range(L - S)]
    pk = torch.stack([k_at[x] for x in prior]) if prior else torch.zeros(0, G, d, dtype=torch.bfloat16)
    pv = torch.stack([v_at[x] for x in prior]) if prior else torch.zeros(0, G, d, dtype=torch.bfloat16)
    ps = torch.tensor([slot_of(*x) for x in prior], dtype=torch.int64)
    new_slots = torch.tensor([[slot_of(b, int(L) - S + j) for j in range(S)] for b, L in enumerate(lens)])
    from tests._harness import gqa_scales
    ks, vs = gqa_scales(case) if case.fp8 else (None, None)
    mul = case.scales_multiply
    dt = torch.uint8 if case.fp8 else torch.bfloat16
    kc_o = torch.zeros(case.num_blocks, G, P, d, dtype=dt)
    vc_o = torch.zeros_like(kc_o)
    ost.kv_store_mha(pk, pv, ps, kc_o, vc_o, ks, vs, mul)
    kc = (kc_o.view(torch.float8_e4m3fn) if case.fp8 else kc_o).cuda().contiguous()
    vc = (vc_o.view(torch.float8_e4m3fn) if case.fp8 else vc_o).cuda().contiguous()
    want = oatt.paged_decode_gqa_multi(q, kc_o, vc_o, case.block_table, lens, k_act, v_act, sm_scale=case.sm_scale,
                                       k_scale=ks, v_scale=vs, sinks=case.sinks, window=case.window,
                                       scales_multiply=mul)
    ost.kv_store_mha(k_act.reshape(B * S, G, d), v_act.reshape(B * S, G, d), new_slots.reshape(-1), kc_o, vc_o, ks,
                     vs, mul)
    announce(f"gqa multi-token {name}: B={B} S={S} H={H} G={G} d={d} window={case.window}")
    out = ops.paged_decode_gqa_multi(q.cuda(), kc, vc, case.block_table.cuda(), lens.cuda(), k_act.cuda(),
                                     v_act.cuda(), sm_scale=case.sm_scale, new_slots=new_slots.cuda(),
                                     k_scale=None if ks is None else ks.cuda(), v_scale=None if vs is None else vs.cuda(),
                                     sinks=None if case.sinks is None else case.sinks.cuda(), window=case.window,
                                     scales_multiply=mul, host_seq_lens=lens)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    assert torch.equal(cache_bytes(kc), cache_bytes(kc_o)), "K pool differs"
    assert torch.equal(cache_bytes(vc), cache_bytes(vc_o)), "V pool differs"
