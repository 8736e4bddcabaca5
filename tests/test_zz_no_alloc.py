"""sna_paged_decode_gqa_noalloc (the GQA decode with the library's per-GPU scratch array in place of a workspace)
against sna_paged_decode_gqa on the same inputs: two calls in a row through the C ABI, the second with a smaller
input, each bit-identical to the workspace entry point (output and the pool after the fused store) and within the
attention bar of the oracle; and a plan whose partials exceed the scratch is refused."""

import ctypes

import pytest
import torch

from sglang_neuron_amd import _lib, ops, workloads
from tests.conftest import announce
from tests._harness import assert_close_attn, cache_bytes, gqa_gpu_pool, gqa_oracle

pytestmark = pytest.mark.gpu


def _noalloc_call(case, kc, vc, ks, vs, plan):
    """One sna_paged_decode_gqa_noalloc call through ctypes, on torch's current stream; returns its output."""
    dev = "cuda"
    q = case.q.to(dev).contiguous()
    table = case.block_table.to(dev).to(torch.int32).contiguous()
    lens = case.seq_lens.to(dev).to(torch.int32).contiguous()
    kn, vn = case.k_new.to(dev).contiguous(), case.v_new.to(dev).contiguous()
    slots = case.new_slots.to(dev).to(torch.int64).contiguous()
    sinks = None if case.sinks is None else case.sinks.to(dev).float().contiguous()
    out = torch.empty(case.B, case.H, case.d, dtype=torch.bfloat16, device=dev)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    lib = _lib.load()
    rc = lib.sna_paged_decode_gqa_noalloc(
        ptr(q), ptr(kc), ptr(vc), ptr(ks), ptr(vs), ptr(table), table.stride(0), table.shape[1], ptr(lens), ptr(kn),
        ptr(vn), ptr(slots), ptr(sinks), case.window, case.sm_scale, ptr(out), case.B, case.H, case.G, case.d, case.P,
        kc.shape[0], ops.cache_dtype_code(kc.dtype, case.scales_multiply), ctypes.byref(plan),
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "paged_decode_gqa_noalloc")
    return out


def _workspace_call(case, kc, vc, ks, vs, plan):
    return ops.paged_decode_gqa(case.q.cuda(), kc, vc, case.block_table.cuda(), case.seq_lens.cuda(),
                                case.k_new.cuda(), case.v_new.cuda(), sm_scale=case.sm_scale, k_scale=ks, v_scale=vs,
                                sinks=None if case.sinks is None else case.sinks.cuda(), window=case.window,
                                new_slots=case.new_slots.cuda(), plan=plan, scales_multiply=case.scales_multiply)


# the first call spreads its rows over many splits (a large partial workspace); the second is smaller
CALLS = [("cfg4-many-splits", 4, {"B": 24, "lens": (2000, 8192)}),
         ("cfg2-small", 2, {"B": 3, "lens": (100, 900)})]


def test_noalloc_matches_workspace_entry_point_twice():
    for name, cfg, over in CALLS:
        case = workloads.gqa_case(cfg, overrides=over)
        plan = ops.plan_decode(_lib.KIND_GQA, case.B, host_seq_lens=case.seq_lens, window=case.window,
                               ctas_per_item=case.G, num_cus=ops._num_cus(torch.device("cuda")))
        need = ops.workspace_bytes(plan, case.H, case.d)
        announce(f"noalloc {name}: B={case.B} H={case.H} G={case.G} d={case.d} splits={plan.max_splits} "
                 f"partials={need} bytes")
        kc, vc, ks, vs = gqa_gpu_pool(case)
        kc2, vc2 = kc.clone(), vc.clone()
        got = _noalloc_call(case, kc, vc, ks, vs, plan)
        want = _workspace_call(case, kc2, vc2, ks, vs, plan)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), want.cpu()), f"{name}: output differs from sna_paged_decode_gqa"
        assert torch.equal(cache_bytes(kc), cache_bytes(kc2)) and torch.equal(cache_bytes(vc), cache_bytes(vc2)), \
            f"{name}: pools differ after the fused store"
        oracle_out, *_ = gqa_oracle(case)
        assert_close_attn(got, oracle_out, name)
        if name == CALLS[0][0]:
            assert plan.max_splits > 1 and need > 0, "the first call must use the scratch"


def test_noalloc_refuses_plans_past_its_scratch():
    """A plan whose partials need more than the scratch array is refused before any launch."""
    B, H, G, d = 128, 128, 1, 128
    plan = ops.plan_decode(_lib.KIND_GQA, B, host_seq_lens=[100000] * B, ctas_per_item=G, num_cus=256)
    assert ops.workspace_bytes(plan, H, d) > _lib.NOALLOC_SCRATCH_BYTES
    rc = _lib.load().sna_paged_decode_gqa_noalloc(None, None, None, None, None, None, 1, 1, None, None, None, None, None,
                                                  0, 0.1, None, B, H, G, d, 16, 1, 1, ctypes.byref(plan), None)
    assert rc == _lib.SNA_ERR_WORKSPACE and "scratch" in _lib.last_error()
