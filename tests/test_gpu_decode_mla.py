"""Absorbed-MLA decode parity (cfg3 shapes) and DSA sparse decode parity (cfg5 shapes): the HIP kernels against the
oracle on seeded cases, with the pools compared bit-exact after the step."""

import pytest
import torch

from sglang_neuron_amd import _lib, ops, workloads
from tests.conftest import announce
from tests._harness import (assert_close_attn, dsa_gpu_pool, dsa_gpu_step, dsa_oracle, mla_gpu_decode, mla_gpu_pool,
                            mla_oracle)

pytestmark = pytest.mark.gpu

MLA_CASES = [
    ("cfg3-small", {"B": 4, "lens": (1024, 4096)}),
    ("cfg3-ragged", {"B": 6, "lens": (1, 300)}),
    ("cfg3-long", {"B": 2, "lens": (16000, 16384)}),
    ("heads-8", {"B": 3, "H": 8, "lens": (20, 2000)}),
    ("heads-20", {"B": 2, "H": 20, "lens": (100, 1000)}),
    ("page-16", {"B": 3, "P": 16, "lens": (40, 900)}),
    ("page-48", {"B": 3, "P": 48, "lens": (40, 3000)}),                 # a page that is not a power of two
    # page 128: the page the reference serves DeepSeek-V2 with (docs/model-recipes/deepseek-v2.md:122)
    ("cfg3-page128", {"B": 6, "P": 128, "lens": (1024, 16384)}),
    ("cfg3-full", {}),                                                   # the bench workload at its full size
    # more rows than workgroups (20 heads: two head groups of 128 workgroups): ranges span several rows
    ("multi-row-ranges", {"B": 200, "H": 20, "lens": (1, 200)}),
    # more rows than one launch's plan holds (256): two launches, one after the other
    ("batch-past-one-launch", {"B": 300, "lens": (1, 120)}),
]


@pytest.mark.parametrize("name,over", MLA_CASES, ids=[c[0] for c in MLA_CASES])
def test_mla_decode_matches_oracle(name, over):
    case = workloads.mla_case(overrides=over)
    want, cache_o, scale_o = mla_oracle(case)
    announce(f"mla {name}: B={case.B} H={case.H} P={case.P} lens={case.seq_lens.tolist()[:8]}")
    cache, scale = mla_gpu_pool(case)
    out = mla_gpu_decode(case, cache, scale)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"
    assert torch.equal(scale.cpu(), scale_o), "row scales differ"


# device-split plans (a bound: the block table's width): the launch cuts its split from the device's seq_lens
DEVICE_SPLIT_CASES = [
    ("ds-cfg3-small", {"B": 4, "lens": (1024, 4096)}, False),
    ("ds-ragged", {"B": 9, "lens": (1, 300)}, False),
    ("ds-cfg3-full", {}, False),
    ("ds-one-row", {"B": 1, "lens": (7000, 7000)}, False),
    # 128 heads: 8 head groups of 32 workgroups, fewer than the 40 rows: equal ranges across rows
    ("ds-ranges-across-rows", {"B": 40, "H": 128, "lens": (1, 1500)}, False),
    ("ds-bf16-page128", {"B": 6, "P": 128, "lens": (1024, 16384)}, True),
]


@pytest.mark.parametrize("name,over,bf16", DEVICE_SPLIT_CASES, ids=[c[0] for c in DEVICE_SPLIT_CASES])
def test_mla_device_split_matches_oracle(name, over, bf16):
    dev = torch.device("cuda", 0)
    case = workloads.mla_case(overrides=over)
    want, cache_o, scale_o = mla_oracle(case, bf16=bf16)
    cache, scale = mla_gpu_pool(case, bf16=bf16)
    table = case.block_table.to(dev)
    groups = (case.H + 15) // 16
    plan = ops.plan_decode(1, case.B, max_seq_len=table.shape[1] * case.P, ctas_per_item=groups,
                           num_cus=ops._num_cus(dev))
    announce(f"mla device split {name}: B={case.B} H={case.H} P={case.P} n_ctas={plan.n_ctas} "
             f"lens={case.seq_lens.tolist()[:8]}")
    assert plan.device_split == 1
    out = ops.mla_decode(case.ql_nope.to(dev), case.q_pe.to(dev), cache, scale, table, case.seq_lens.to(dev),
                         case.compact_new.to(dev), sm_scale=case.sm_scale, page_size=case.P,
                         new_slots=case.new_slots.to(dev), plan=plan)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    assert torch.equal(cache.cpu().view(torch.uint8), cache_o.view(torch.uint8)), "row pool differs"
    if not bf16:
        assert torch.equal(scale.cpu(), scale_o), "row scales differ"


# bf16 rows, the reference's DeepSeek-V2 pool (models/catalog.py:230-231: bf16 KV at page 128)
MLA_BF16_CASES = [
    ("bf16-cfg3-page128", {"B": 8, "P": 128, "lens": (1024, 16384)}),
    ("bf16-cfg3-full", {}),
    ("bf16-ragged", {"B": 6, "lens": (1, 300)}),
    ("bf16-heads-20", {"B": 2, "H": 20, "lens": (100, 1000)}),
    ("bf16-page-16", {"B": 3, "P": 16, "lens": (40, 900)}),
    ("bf16-page-48", {"B": 3, "P": 48, "lens": (40, 3000)}),
    ("bf16-multi-row-ranges", {"B": 200, "H": 20, "lens": (1, 200)}),
]


@pytest.mark.parametrize("name,over", MLA_BF16_CASES, ids=[c[0] for c in MLA_BF16_CASES])
def test_mla_decode_bf16_rows_matches_oracle(name, over):
    case = workloads.mla_case(overrides=over)
    want, cache_o, _ = mla_oracle(case, bf16=True)
    announce(f"mla {name}: B={case.B} H={case.H} P={case.P} lens={case.seq_lens.tolist()[:8]}")
    cache, scale = mla_gpu_pool(case, bf16=True)
    out = mla_gpu_decode(case, cache, scale)
    torch.cuda.synchronize()
    assert_close_attn(out, want, name)
    assert torch.equal(cache.cpu().view(torch.int16), cache_o.view(torch.int16)), "row pool differs"


DSA_CASES = [
    ("cfg5-small", {"B": 4, "pool_positions": 4096, "n_indices": 512, "recent": 128, "short_rows": (100, 300)}),
    ("cfg5-wide", {"B": 2, "pool_positions": 8192, "n_indices": 2048, "recent": 128, "short_rows": (1500,)}),
    ("page-16", {"B": 3, "P": 16, "pool_positions": 2048, "n_indices": 100, "recent": 16, "short_rows": (40,)}),
    ("page-48", {"B": 3, "P": 48, "pool_positions": 4800, "n_indices": 300, "recent": 32, "short_rows": (200,)}),
    ("cfg5-page128", {"B": 4, "P": 128, "pool_positions": 8192, "n_indices": 2048, "recent": 128,
                      "short_rows": (600,)}),
    ("cfg5-full", {}),                                                   # the bench workload: 131072 positions per row
    # a block table past the prologue's LDS copy (20000 one-slot pages): indices resolve entry by entry
    ("page-1-wide-table", {"B": 2, "P": 1, "pool_positions": 20000, "n_indices": 256, "recent": 16,
                           "short_rows": ()}),
    # index lists past one workgroup's 2048 (each row in pieces of at most 2048 indices)
    ("indices-past-one-range", {"B": 6, "pool_positions": 8192, "n_indices": 3000, "recent": 128,
                                "short_rows": (2000,)}),
    # rows whose pieces need more than one launch's 256 workgroups: the own rows stored first, then two launches
    ("batch-past-one-launch", {"B": 130, "pool_positions": 2600, "n_indices": 2500, "recent": 64,
                               "short_rows": (1000,)}),
    # MTP verify: spec query tokens per sequence, each attending its index list and its earlier siblings' own rows
    ("spec-3-small", {"B": 3, "pool_positions": 2048, "n_indices": 256, "recent": 32, "short_rows": (300,),
                      "spec": 3}),
    ("cfg5-mtp-spec8", {"spec": workloads.DSA_MTP_SPEC}),               # GLM's MTP K7 on the full cfg5 pool
    ("spec8-three-launches", {"B": 40, "pool_positions": 3000, "n_indices": 2500, "recent": 64,
                              "short_rows": (900,), "spec": 8}),
]


@pytest.mark.parametrize("name,over", DSA_CASES, ids=[c[0] for c in DSA_CASES])
def test_dsa_decode_matches_oracle(name, over):
    case = workloads.dsa_case(overrides=over)
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    announce(f"dsa {name}: B={case.B} spec={case.spec} H={case.H} P={case.P} K={case.indices.shape[1]}")
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache)
    torch.cuda.synchronize()
    assert_close_attn(ctx, want_ctx, name)
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4), (lse.cpu() - want_lse).abs().max()
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"


def test_dsa_caller_stored_rows():
    """Without new_slots the caller stores the own rows first (sna_kv_store_dsa), and the decode only reads."""
    case = workloads.dsa_case(overrides=DSA_CASES[0][1])
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    announce("dsa caller-stored own rows")
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache, fused=False)
    assert_close_attn(ctx, want_ctx, "caller-stored")
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4)
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"


@pytest.mark.parametrize("name,over", [
    ("one-workgroup", {"B": 3, "pool_positions": 1024, "n_indices": 64, "recent": 8, "short_rows": ()}),
    ("split-rows", {"B": 3, "pool_positions": 8192, "n_indices": 2048, "recent": 64, "short_rows": ()}),
])
def test_dsa_gathers_of_slots_stored_in_the_launch(name, over):
    """Gathers of a row that this launch stores an own row to attend the stored bytes, as in the reference, which
    stores every own row before any gather: a row indexing its own position, a row whose table maps a block onto
    another row's new slot, and two rows storing to one slot (the later row's bytes land and are gathered)."""
    case = workloads.dsa_case(overrides=over)
    P = case.P
    p0 = int(case.positions[0])
    case.indices[0, 10] = p0                                   # row 0 attends its own position through an index
    case.block_table[1, 3] = case.block_table[0, p0 // P]      # row 1's block 3 is row 0's last block
    case.indices[1, 11] = 3 * P + p0 % P                       # ... and row 1 gathers row 0's new slot
    case.new_slots[2] = case.new_slots[0]                      # rows 0 and 2 store to one slot: row 2's bytes land
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    announce(f"dsa aliased gathers {name}: B={case.B} K={case.indices.shape[1]}")
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache)
    assert_close_attn(ctx, want_ctx, name)
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4)
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"


def test_dsa_invalid_indices_are_dropped():
    """Indices past the table, into unallocated blocks, or after the query's position are dropped; -1 is empty."""
    case = workloads.dsa_case(overrides={"B": 2, "pool_positions": 1024, "n_indices": 64, "recent": 8,
                                         "short_rows": ()})
    case.indices[0, 5] = 10 ** 6            # past the table
    case.indices[0, 6] = -1
    case.block_table[1, 2] = -1            # unallocated block: drops indices in [128, 192)
    case.indices[1, 7] = 150
    case.indices[1, 8] = int(case.positions[1]) + 5  # after the query position (not kept)
    want_ctx, want_lse, _ = dsa_oracle(case)
    announce("dsa invalid indices")
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache)
    assert_close_attn(ctx, want_ctx, "invalid indices")
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4)


@pytest.mark.parametrize("polls", [0, 1])
def test_split_merge_when_polls_run_out(polls):
    """A split row's owners poll a bounded number of times for the row's last partial; with the bound at 0 or 1 they
    mostly give up and retract their latent blocks, and the last workgroup to arrive merges them. Every block is still
    merged once, to the same bits as with the planner's bound (the merge's sums do not depend on which workgroup
    runs them), on two calls in a row. (The bound is forced from the host: every wait still ends.)"""
    dev = torch.device("cuda", 0)
    case = workloads.mla_case(overrides={"B": 4, "lens": (1024, 4096)})
    want, _, _ = mla_oracle(case)
    cache, scale = mla_gpu_pool(case)
    args = (case.ql_nope.to(dev), case.q_pe.to(dev), cache, scale, case.block_table.to(dev), case.seq_lens.to(dev),
            case.compact_new.to(dev))
    kw = dict(sm_scale=case.sm_scale, page_size=case.P, new_slots=case.new_slots.to(dev), host_seq_lens=case.seq_lens)
    plan = ops.plan_decode(1, case.B, host_seq_lens=case.seq_lens, ctas_per_item=1, num_cus=ops._num_cus(dev))
    announce(f"mla merge with {polls} polls: B={case.B} n_ctas={plan.n_ctas} max_splits={plan.max_splits}")
    assert plan.max_splits > 1
    base = ops.mla_decode(*args, **kw, plan=plan)
    plan.wait_polls = polls
    for _ in range(2):
        out = ops.mla_decode(*args, **kw, plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(out, base), "MLA output differs from the default plan's"
    assert_close_attn(out, want, f"mla polls={polls}")

    dcase = workloads.dsa_case(overrides=DSA_CASES[0][1])
    dplan = ops.plan_decode(2, dcase.B, n_keys_per_row=dcase.indices.shape[1], ctas_per_item=1,
                            num_cus=ops._num_cus(dev))
    assert dplan.max_splits > 1
    want_ctx, want_lse, _ = dsa_oracle(dcase)
    cache = dsa_gpu_pool(dcase)
    dargs = (dcase.q_absorbed.to(dev), dcase.q_pe.to(dev), cache, dcase.kv_scale, dcase.indices.to(dev),
             dcase.block_table.to(dev), dcase.positions.to(dev), dcase.own_rows.to(dev))
    dkw = dict(sm_scale=dcase.sm_scale, page_size=dcase.P, new_slots=dcase.new_slots.to(dev))
    base_ctx, base_lse = ops.mla_decode_sparse(*dargs, **dkw, plan=dplan)
    dplan.wait_polls = polls
    for _ in range(2):
        ctx, lse = ops.mla_decode_sparse(*dargs, **dkw, plan=dplan)
        torch.cuda.synchronize()
        assert torch.equal(ctx, base_ctx) and torch.equal(lse, base_lse), "DSA output differs from the default plan's"
    assert_close_attn(ctx, want_ctx, f"dsa polls={polls}")


def test_dirty_counter_block_is_detected_and_reset():
    """A workspace whose counter block is not zero on entry (planted from the host: a row's arrival count, then the
    finished-workgroups count) sets the launch's sticky status bit, which stream_workspace_status reports and clears.
    A clean block reads 0; after a dirty arrival the launch's own end returns the counters to zero, so the next call
    is clean and matches the oracle; after a dirty finished count the counters stay dirty until
    reset_stream_workspace, after which the call is clean and matches again. Every wait in the merge is bounded, so
    each launch ends."""
    dev = torch.device("cuda", 0)
    case = workloads.mla_case(overrides={"B": 2, "lens": (3000, 4096)})
    want, _, _ = mla_oracle(case)
    cache, scale = mla_gpu_pool(case)
    args = (case.ql_nope.to(dev), case.q_pe.to(dev), cache, scale, case.block_table.to(dev), case.seq_lens.to(dev),
            case.compact_new.to(dev))
    plan = ops.plan_decode(1, case.B, host_seq_lens=case.seq_lens, ctas_per_item=1, num_cus=ops._num_cus(dev))
    assert plan.max_splits > 3
    ws = ops.stream_workspace(plan, case.H, dev)
    kw = dict(sm_scale=case.sm_scale, page_size=case.P, new_slots=case.new_slots.to(dev), host_seq_lens=case.seq_lens,
              plan=plan, workspace=ws)
    words = ws.view(torch.int32)
    announce(f"mla dirty counters: B={case.B} n_ctas={plan.n_ctas} max_splits={plan.max_splits}")

    def clean_call():
        out = ops.mla_decode(*args, **kw)
        assert ops.stream_workspace_status(ws) == 0
        assert_close_attn(out, want, "clean call")

    clean_call()
    words[0] = 3  # row 0's arrival word (head group 0)
    ops.mla_decode(*args, **kw)
    assert ops.stream_workspace_status(ws) & _lib.WS_DIRTY_ARRIVAL
    assert ops.stream_workspace_status(ws) == 0  # read and cleared
    clean_call()  # the dirty launch's end zeroed the counters
    words[16 * 2 * _lib.STREAM_MAX_COUNTERS] = 1 << 20  # the finished-workgroups count
    ops.mla_decode(*args, **kw)
    assert ops.stream_workspace_status(ws) & _lib.WS_DIRTY_DONE
    ops.reset_stream_workspace(ws)
    torch.cuda.synchronize()
    assert int(words[:16 * 2 * _lib.STREAM_MAX_COUNTERS + 16].abs().sum()) == 0
    clean_call()


def test_dsa_pool_past_4gib():
    """A DSA pool of more than 4 GiB (150,000 unused pages mixed into the permutation): its rows take 64-bit addresses
    (the kernel's WIDE form) instead of 32-bit offsets against one buffer resource. Parity and the pool bit-exact,
    as for the smaller pools."""
    case = workloads.dsa_case(overrides={"B": 2, "pool_positions": 8192, "n_indices": 2048, "recent": 128,
                                         "short_rows": (), "extra_pages": 150_000})
    assert case.num_blocks * case.P * 640 > (1 << 32)
    far = int((case.block_table.to(torch.int64) * case.P * 640 >= (1 << 32)).sum())
    assert far > 0, "no page of the case lies past 4 GiB"
    want_ctx, want_lse, cache_o = dsa_oracle(case)
    announce(f"dsa pool past 4 GiB: {case.num_blocks * case.P * 640 / 2**30:.2f} GiB, {far} pages past 4 GiB")
    cache = dsa_gpu_pool(case)
    ctx, lse = dsa_gpu_step(case, cache)
    torch.cuda.synchronize()
    assert_close_attn(ctx, want_ctx, "pool past 4 GiB")
    assert torch.allclose(lse.cpu(), want_lse, atol=2e-3, rtol=1e-4)
    assert torch.equal(cache.cpu(), cache_o), "row pool differs"


@pytest.mark.parametrize("polls", [0, 1])
def test_multi_segment_merge_with_bounded_polls(polls):
    """Ranges that span rows (200 rows, 20 heads: two head groups of 128 workgroups): a workgroup whose range goes on
    into another row publishes its partial without polling, and the merge of every split row still completes, to the
    same bits with the poll bound forced to 0 or 1 as with the planner's, and within the oracle's tolerance."""
    dev = torch.device("cuda", 0)
    case = workloads.mla_case(overrides={"B": 200, "H": 20, "lens": (1, 200)})
    want, _, _ = mla_oracle(case)
    cache, scale = mla_gpu_pool(case)
    args = (case.ql_nope.to(dev), case.q_pe.to(dev), cache, scale, case.block_table.to(dev), case.seq_lens.to(dev),
            case.compact_new.to(dev))
    kw = dict(sm_scale=case.sm_scale, page_size=case.P, new_slots=case.new_slots.to(dev), host_seq_lens=case.seq_lens)
    plan = ops.plan_decode(1, case.B, host_seq_lens=case.seq_lens, ctas_per_item=2, num_cus=ops._num_cus(dev))
    announce(f"mla multi-segment merge, {polls} polls: B={case.B} n_ctas={plan.n_ctas} max_splits={plan.max_splits}")
    assert plan.n_ctas < case.B and plan.max_splits > 1
    base = ops.mla_decode(*args, **kw, plan=plan)
    plan.wait_polls = polls
    for _ in range(2):
        out = ops.mla_decode(*args, **kw, plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(out, base), "output differs from the default plan's"
    assert_close_attn(out, want, f"multi-segment polls={polls}")
