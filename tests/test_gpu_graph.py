"""The decode launches captured in a HIP graph (torch.cuda.CUDAGraph) and replayed: GQA with split-K and its combine
pass (a plan from a length bound, which the kernels resolve against the device's lengths), absorbed MLA and DSA
(their in-launch merges reset their own counters). Each replay, with eager work and synchronizations between them,
gives the eager call's bits; the library issues no memset or copy, so nothing else is recorded."""

import pytest
import torch

from sglang_neuron_amd import ops, workloads
from tests.conftest import announce
from tests._harness import dsa_gpu_pool, mla_gpu_pool

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
                                                   page_size=case.P, new_slots=slots, plan=plan, workspace=ws),
                    lambda out: [out])


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
