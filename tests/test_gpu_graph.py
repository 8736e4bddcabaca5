"""The decode launches captured in a HIP graph (torch.cuda.CUDAGraph) and replayed: GQA with split-K and its combine
pass (a plan from a length bound, which the kernels resolve against the device's lengths), absorbed MLA and DSA
(their in-launch merges reset their own counters). Each replay, with eager work and synchronizations between them,
gives the eager call's bits; the library issues no memset or copy, so nothing else is recorded."""

import pytest
import torch

from oracle import attention as oatt
from oracle import store as ost
from sglang_neuron_amd import ops, workloads
from tests.conftest import announce
from tests._harness import assert_close_attn, dsa_gpu_pool, mla_gpu_pool

pytestmark = pytest.mark.gpu
REPLAYS = 4


def _replay_matches(prepare, outputs_of):
    """Warm up eagerly, capture one call prepared inside the capture (so it binds the capture stream), then replay it
    REPLAYS times with unrelated eager work between replays; every replay's outputs equal the eager call's."""
    dev = torch.device("cuda", 0)
    eager = [t.clone() for t in outputs_of(prepare()())]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        prepare()()  # a call on the capture stream before the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        captured = prepare()
        outs = outputs_of(captured())
    for i in range(REPLAYS):
        for t in outs:
            t.fill_(0)  # eager work on the outputs between replays
        junk = torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert float(junk) == float(junk)
        for got, want in zip(outs, eager):
            assert torch.equal(got, want), f"replay {i} differs from the eager call"


def test_graph_gqa_split_and_combine():
    case = workloads.gqa_case(4, overrides={"B": 6, "lens": (1500, 5000)})
    kc, vc, ks, vs = workloads.gqa_pool(case, "cuda")
    q, table, lens = case.q.to("cuda"), case.block_table.to("cuda"), case.seq_lens.to("cuda")
    kn, vn, slots = case.k_new.to("cuda"), case.v_new.to("cuda"), case.new_slots.to("cuda")
    sinks = case.sinks.to("cuda")
    # a plan from a bound: no item map, the kernels read the device's lengths
    plan = ops.plan_decode(0, case.B, max_seq_len=table.shape[1] * case.P, ctas_per_item=case.G,
                           num_cus=ops._num_cus(q.device))
    announce(f"graph gqa: B={case.B} max_splits={plan.max_splits} work_n={plan.work_n}")
    assert plan.max_splits > 1 and plan.work_n == 0
    _replay_matches(lambda: ops.prepare_paged_decode_gqa(q, kc, vc, table, lens, kn, vn, sm_scale=case.sm_scale,
                                                         k_scale=ks, v_scale=vs, sinks=sinks, new_slots=slots,
                                                         plan=plan, scales_multiply=case.scales_multiply),
                    lambda out: [out])


def test_graph_mla():
    case = workloads.mla_case(overrides={"B": 4, "lens": (1024, 4096)})
    cache, scale = mla_gpu_pool(case)
    table, lens = case.block_table.to("cuda"), case.seq_lens.to("cuda")
    plan = ops.plan_decode(1, case.B, host_seq_lens=case.seq_lens, ctas_per_item=1,
                           num_cus=ops._num_cus(torch.device("cuda", 0)))
    ws = ops.stream_workspace(plan, case.H, torch.device("cuda", 0))
    announce(f"graph mla: B={case.B} n_ctas={plan.n_ctas} max_splits={plan.max_splits}")
    ql, qp, cn, slots = case.ql_nope.to("cuda"), case.q_pe.to("cuda"), case.compact_new.to("cuda"), \
        case.new_slots.to("cuda")
    _replay_matches(lambda: ops.prepare_mla_decode(ql, qp, cache, scale, table, lens, cn, sm_scale=case.sm_scale,
                                                   page_size=case.P, new_slots=slots, plan=plan, workspace=ws,
                                                   host_seq_lens=case.seq_lens),
                    lambda out: [out])


@pytest.mark.parametrize("bf16", [False, True], ids=["fp8-rows", "bf16-rows"])
def test_graph_mla_device_split_replays_growing_lengths(bf16):
    """One MLA decode captured once with a device-split plan (a bound: the table's width), then replayed for three
    steps in which every row grows by one token: before each replay the step's own rows and slots are copied into the
    captured inputs and the device's seq_lens are incremented, nothing is planned again. Each step's output against
    oracle.mla_decode over the pool as the oracle has it by then, and the pool (rows and scales) bit-exact after
    every step."""
    dev = torch.device("cuda", 0)
    steps = 3
    case = workloads.mla_case(overrides={"B": 5, "lens": (900, 5000)})
    L0 = case.seq_lens - (steps - 1)  # the first step's lengths; the case's prior covers every later step's rows
    P = case.P
    rows_of = {}  # (row, position) -> its compact row
    k = 0
    for b, L in enumerate(case.seq_lens.tolist()):
        for pos in range(L - 1):
            rows_of[(b, pos)] = case.prior_rows[k]
            k += 1
    for b in range(case.B):
        rows_of[(b, int(case.seq_lens[b]) - 1)] = case.compact_new[b]
    slot_of = lambda b, pos: int(case.block_table[b, pos // P]) * P + pos % P  # noqa: E731
    n = case.num_blocks * P
    cache_o = torch.zeros(n, 576, dtype=torch.bfloat16 if bf16 else torch.uint8)
    scale_o = None if bf16 else torch.zeros(n, dtype=torch.float32)
    first = [(b, pos) for b in range(case.B) for pos in range(int(L0[b]) - 1)]
    first_rows = torch.stack([rows_of[x] for x in first])
    first_slots = torch.tensor([slot_of(*x) for x in first])
    ost.kv_store_mla(first_rows, first_slots, cache_o, scale_o)
    cache = torch.zeros(n, 576, dtype=cache_o.dtype, device=dev)
    scale = None if bf16 else torch.zeros(n, dtype=torch.float32, device=dev)
    ops.kv_store_mla(first_rows.to(dev), first_slots.to(dev), cache, scale)
    table = case.block_table.to(dev)
    lens = L0.to(torch.int32).to(dev)
    ql, qp = case.ql_nope.to(dev), case.q_pe.to(dev)
    new_rows = torch.zeros(case.B, 576, dtype=torch.bfloat16, device=dev)
    new_slots = torch.zeros(case.B, dtype=torch.int64, device=dev)
    plan = ops.plan_decode(1, case.B, max_seq_len=table.shape[1] * P, ctas_per_item=1, num_cus=ops._num_cus(dev))
    assert plan.device_split == 1
    ws = ops.stream_workspace(plan, case.H, dev)
    announce(f"graph mla device split bf16={bf16}: B={case.B} n_ctas={plan.n_ctas} lens0={L0.tolist()}")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        prep = ops.prepare_mla_decode(ql, qp, cache, scale, table, lens, new_rows, sm_scale=case.sm_scale, page_size=P,
                                      new_slots=new_slots, plan=plan, workspace=ws)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            out = prep()
    torch.cuda.synchronize()
    for s_ in range(steps):
        L = L0 + s_
        rows = torch.stack([rows_of[(b, int(L[b]) - 1)] for b in range(case.B)])
        slots = torch.tensor([slot_of(b, int(L[b]) - 1) for b in range(case.B)])
        new_rows.copy_(rows.to(dev))
        new_slots.copy_(slots.to(dev))
        lens.copy_(L.to(torch.int32).to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = oatt.mla_decode(case.ql_nope, case.q_pe, cache_o, scale_o, case.block_table, L, rows,
                               sm_scale=case.sm_scale, page_size=P)
        ost.kv_store_mla(rows, slots, cache_o, scale_o)
        assert_close_attn(out, want, f"device split step {s_}")
        assert torch.equal(cache.cpu().view(torch.uint8), cache_o.view(torch.uint8)), f"step {s_}: row pool differs"
        if not bf16:
            assert torch.equal(scale.cpu(), scale_o), f"step {s_}: row scales differ"


def test_graph_dsa():
    case = workloads.dsa_case(overrides={"B": 4, "pool_positions": 4096, "n_indices": 512, "recent": 128,
                                         "short_rows": (100, 300)})
    cache = dsa_gpu_pool(case)
    dev = torch.device("cuda", 0)
    plan = ops.plan_decode(2, case.B, n_keys_per_row=case.indices.shape[1], ctas_per_item=1, num_cus=ops._num_cus(dev))
    ws = ops.stream_workspace(plan, case.H, dev)
    announce(f"graph dsa: B={case.B} n_ctas={plan.n_ctas} max_splits={plan.max_splits}")
    args = (case.q_absorbed.to(dev), case.q_pe.to(dev), cache, case.kv_scale, case.indices.to(dev),
            case.block_table.to(dev), case.positions.to(dev), case.own_rows.to(dev))
    slots = case.new_slots.to(dev)
    _replay_matches(lambda: ops.prepare_mla_decode_sparse(*args, sm_scale=case.sm_scale, page_size=case.P,
                                                          new_slots=slots, plan=plan, workspace=ws),
                    lambda out: list(out))
