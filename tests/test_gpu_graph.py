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


@pytest.mark.parametrize("window", [0, workloads.SWA_WINDOW], ids=["full", "swa"])
def test_graph_gqa_device_split_replays_growing_lengths(window):
    """One GQA decode (GPT-OSS shape: sinks, FP8 multipliers) captured once with a plan from a bound, which sizes its
    splits on the device, then replayed for three steps in which every row grows by one token: before each replay
    the step's K/V, slots and lengths are copied into the captured inputs, nothing is planned again. Each step's
    output against oracle.paged_decode_gqa over the pool as the oracle has it by then, and both pools bit-exact after
    every step."""
    dev = torch.device("cuda", 0)
    steps = 3
    case = workloads.gqa_case(4, overrides={"B": 7, "lens": (40, 5000), "window": window})
    L0 = case.seq_lens - (steps - 1)
    P, G, d = case.P, case.G, case.d
    kv_of = {}  # (row, position) -> (k, v) [G, d]
    k = 0
    for b, L in enumerate(case.seq_lens.tolist()):
        for pos in range(L - 1):
            kv_of[(b, pos)] = (case.k_prior[k], case.v_prior[k])
            k += 1
        kv_of[(b, L - 1)] = (case.k_new[b], case.v_new[b])
    slot_of = lambda b, pos: int(case.block_table[b, pos // P]) * P + pos % P  # noqa: E731
    ks = ops.inverted_kv_scale(ops.kv_absmax_scale(torch.cat([case.k_prior, case.k_new]).to(dev))).to(dev)
    vs = ops.inverted_kv_scale(ops.kv_absmax_scale(torch.cat([case.v_prior, case.v_new]).to(dev))).to(dev)
    ks_o, vs_o = ks.cpu(), vs.cpu()
    first = [(b, pos) for b in range(case.B) for pos in range(int(L0[b]) - 1)]
    k_first = torch.stack([kv_of[x][0] for x in first])
    v_first = torch.stack([kv_of[x][1] for x in first])
    s_first = torch.tensor([slot_of(*x) for x in first])
    kc_o = torch.zeros(case.num_blocks, G, P, d, dtype=torch.uint8)
    vc_o = torch.zeros_like(kc_o)
    ost.kv_store_mha(k_first, v_first, s_first, kc_o, vc_o, ks_o, vs_o, scales_multiply=True)
    kc = torch.zeros(case.num_blocks, G, P, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    ops.kv_store_mha(k_first.to(dev), v_first.to(dev), s_first.to(dev), kc, vc, ks, vs, scales_multiply=True)
    table = case.block_table.to(dev)
    lens = L0.to(torch.int32).to(dev)
    q, sinks = case.q.to(dev), case.sinks.to(dev)
    k_step = torch.zeros(case.B, G, d, dtype=torch.bfloat16, device=dev)
    v_step = torch.zeros_like(k_step)
    slots = torch.zeros(case.B, dtype=torch.int64, device=dev)
    plan = ops.plan_decode(0, case.B, max_seq_len=table.shape[1] * P, window=window, ctas_per_item=G,
                           num_cus=ops._num_cus(dev))
    assert plan.device_split == 1 and plan.work_n == 0
    announce(f"graph gqa device split window={window}: B={case.B} n_work={plan.n_work} lens0={L0.tolist()}")
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        prep = ops.prepare_paged_decode_gqa(q, kc, vc, table, lens, k_step, v_step, sm_scale=case.sm_scale,
                                            k_scale=ks, v_scale=vs, sinks=sinks, window=window, new_slots=slots,
                                            plan=plan, scales_multiply=True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            out = prep()
    torch.cuda.synchronize()
    for s_ in range(steps):
        L = L0 + s_
        kn = torch.stack([kv_of[(b, int(L[b]) - 1)][0] for b in range(case.B)])
        vn = torch.stack([kv_of[(b, int(L[b]) - 1)][1] for b in range(case.B)])
        sl = torch.tensor([slot_of(b, int(L[b]) - 1) for b in range(case.B)])
        k_step.copy_(kn.to(dev))
        v_step.copy_(vn.to(dev))
        slots.copy_(sl.to(dev))
        lens.copy_(L.to(torch.int32).to(dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = oatt.paged_decode_gqa(case.q, kc_o, vc_o, case.block_table, L, kn, vn, sm_scale=case.sm_scale,
                                     k_scale=ks_o, v_scale=vs_o, sinks=case.sinks, window=window,
                                     scales_multiply=True)
        ost.kv_store_mha(kn, vn, sl, kc_o, vc_o, ks_o, vs_o, scales_multiply=True)
        assert_close_attn(out, want, f"gqa device split step {s_}")
        assert torch.equal(kc.cpu().view(torch.uint8), kc_o), f"step {s_}: K pool differs"
        assert torch.equal(vc.cpu().view(torch.uint8), vc_o), f"step {s_}: V pool differs"


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
