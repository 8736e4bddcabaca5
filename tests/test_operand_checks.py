"""Host refusals of a decode batch's operands (sna_check_decode_operands through ops.check_decode_operands and the
backend's host path), the refusals of the reference's decode_operands (attention/mla_operands.py:64-97), on the CPU:
each bad operand is refused with ValueError naming its row, and consistent operands (including padding rows on the
reserved page 0) pass."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from sglang_neuron_amd import ops
from sglang_neuron_amd.attention import NeuronAttnBackend
from sglang_neuron_amd.attention.backend import host_block_table
from sglang_neuron_amd.mem_cache import NeuronMHATokenToKVPool, NeuronMLATokenToKVPool

P = 16
NB = 40  # pool pages (page 0 reserved)


def _ok_batch():
    """Three live rows on disjoint pages and one padding row (seq_len 1, slot 0 on the reserved page)."""
    lens = torch.tensor([33, 16, 1, 50])
    table = torch.full((4, 4), -1, dtype=torch.int32)
    table[0, :3] = torch.tensor([5, 9, 2])
    table[1, :1] = torch.tensor([7])
    table[2, :1] = torch.tensor([0])
    table[3, :4] = torch.tensor([11, 12, 13, 14])
    slots = torch.tensor([2 * P + 0, 7 * P + 15, 0, 14 * P + 1])
    return lens, table, slots


def test_consistent_operands_pass():
    lens, table, slots = _ok_batch()
    ops.check_decode_operands(lens, table, slots, P, NB)
    ops.check_decode_operands(lens, table, None, P, NB)
    # two padding rows may share slot 0 (both are redirected to the reserved page)
    ops.check_decode_operands(torch.tensor([1, 1]), torch.zeros(2, 1, dtype=torch.int32), torch.tensor([0, 0]), P, NB)


@pytest.mark.parametrize("what,edit,match", [
    ("position past int32", lambda L, T, S: L.__setitem__(3, 2 ** 31), "int32"),
    ("empty row", lambda L, T, S: L.__setitem__(1, 0), "seq_len 0"),
    ("table too narrow", lambda L, T, S: L.__setitem__(3, 65), "block table holds 4"),
    ("-1 inside a row", lambda L, T, S: T.__setitem__((0, 1), -1), "outside the pool"),
    ("page past the pool", lambda L, T, S: T.__setitem__((3, 0), NB), "outside the pool"),
    ("slot offset vs position", lambda L, T, S: S.__setitem__(0, 2 * P + 1), "disagrees with position 32"),
    ("slot on another page", lambda L, T, S: S.__setitem__(1, 8 * P + 15), "last page is 7"),
    ("shared live slot", lambda L, T, S: (T.__setitem__((1, 0), 2), S.__setitem__(1, 2 * P + 0),
                                          L.__setitem__(1, 1)), "write slot 32"),
])
def test_each_bad_operand_is_refused(what, edit, match):
    lens, table, slots = _ok_batch()
    lens = lens.to(torch.int64)
    edit(lens, table, slots)
    with pytest.raises(ValueError, match=match):
        ops.check_decode_operands(lens, table, slots, P, NB)


@pytest.mark.parametrize("slot,match", [(0, "on the reserved page 0"), (5, "on the reserved page 0"), (NB * P + 7, "outside the pool"),
                                        (-1, "outside the pool")])
def test_live_row_slot_off_the_pool_is_refused(slot, match):
    """A live row (seq_len > 1) whose write would be redirected to the reserved slot 0 would lose its token: refused.
    The same slot on a padding row (seq_len 1) passes."""
    lens, table, slots = _ok_batch()
    slots[3] = slot
    with pytest.raises(ValueError, match=f"row 3: live row's new slot {slot} is {match}"):
        ops.check_decode_operands(lens, table, slots, P, NB)
    slots[2] = slot  # row 2 is a padding row
    slots[3] = 14 * P + 1
    ops.check_decode_operands(lens, table, slots, P, NB)


def test_explicit_active_flags():
    """With the reference's active flags, an inactive row is not checked and a live row is, whatever its length."""
    lens, table, slots = _ok_batch()
    slots[0] = 3 * P + 1  # would disagree with row 0's position and page
    with pytest.raises(ValueError, match="row 0"):
        ops.check_decode_operands(lens, table, slots, P, NB)
    ops.check_decode_operands(lens, table, slots, P, NB, active=torch.tensor([0, 1, 0, 1]))
    slots[2] = 0  # the padding row, flagged live: its slot on page 0 is refused
    with pytest.raises(ValueError, match="row 2"):
        ops.check_decode_operands(lens, table, slots, P, NB, active=torch.tensor([0, 1, 1, 1]))


def test_refusals_name_the_row():
    lens, table, slots = _ok_batch()
    slots[3] = 14 * P + 2
    with pytest.raises(ValueError, match="row 3"):
        ops.check_decode_operands(lens, table, slots, P, NB)


@pytest.mark.gpu
def test_check_takes_host_tensors_only():
    lens, table, slots = _ok_batch()
    with pytest.raises(ValueError):
        ops.check_decode_operands(lens.cuda(), table, slots, P, NB)


class _Mode:
    def __init__(self, kind):
        self.kind = kind

    def is_extend(self):
        return self.kind == "extend"

    def is_idle(self):
        return self.kind == "idle"


def _backend_and_batch(slots, lens, rows_pages):
    """A host req_to_token whose rows hold the given pages, and a decode ForwardBatch over them."""
    r2t = torch.zeros(len(rows_pages), 4 * P, dtype=torch.int32)
    for r, pages in enumerate(rows_pages):
        for j, pg in enumerate(pages):
            r2t[r, j * P:(j + 1) * P] = torch.arange(pg * P, (pg + 1) * P, dtype=torch.int32)
    pool = NeuronMHATokenToKVPool((NB - 1) * P, P, torch.bfloat16, 2, 64, 1, "cpu")
    runner = SimpleNamespace(req_to_token_pool=SimpleNamespace(req_to_token=r2t), token_to_kv_pool=pool, page_size=P)
    lens = torch.as_tensor(lens, dtype=torch.int64)
    fb = SimpleNamespace(forward_mode=_Mode("decode"), batch_size=len(lens), req_pool_indices=torch.arange(len(lens)),
                         seq_lens=lens, seq_lens_cpu=lens, out_cache_loc=torch.as_tensor(slots), positions=lens - 1,
                         extend_prefix_lens=None)
    return NeuronAttnBackend(runner), fb


def test_backend_refuses_before_any_launch():
    """The backend's host path checks the operands once per forward, when it builds the forward's decode state (the
    uploads and split plans every layer shares), before any layer launches."""
    backend, fb = _backend_and_batch([5 * P + 3, 6 * P + 3], [20, 20], [[4, 5], [9, 6]])
    st = backend._decode_state(fb, torch.device("cpu"))
    assert st.table.tolist() == [[4, 5], [9, 6]]
    backend, fb = _backend_and_batch([5 * P + 3, 5 * P + 3], [20, 20], [[4, 5], [9, 5]])
    with pytest.raises(ValueError, match="write slot"):
        backend._decode_state(fb, torch.device("cpu"))
    backend, fb = _backend_and_batch([5 * P + 3, 6 * P + 4], [20, 20], [[4, 5], [9, 6]])
    with pytest.raises(ValueError, match="row 1"):
        backend._decode_state(fb, torch.device("cpu"))


def test_metadata_drops_dp_padding():
    """A batch that DP attention padded (batch_size 4, out_cache_loc of 4) but whose real sizes are 2 rows / 2 tokens
    (_original_batch_size / _original_num_tokens) gives metadata of the 2 real rows (attention/backend.py:86-93)."""
    backend, fb = _backend_and_batch([5 * P + 3, 6 * P + 3, 0, 0], [20, 20, 1, 1], [[4, 5], [9, 6], [0], [0]])
    fb._original_batch_size, fb._original_num_tokens = 2, 2
    meta = backend.build_metadata(fb)
    assert meta.batch_size == 2 and meta.num_tokens == 2
    assert meta.block_table.tolist() == [[4, 5], [9, 6]]
    assert meta.seq_lens.tolist() == [20, 20] and meta.slot_mapping.tolist() == [5 * P + 3, 6 * P + 3]
    assert meta.positions.tolist() == [19, 19]


def test_host_block_table_single_row_and_masking():
    r2t = torch.arange(8 * 64, dtype=torch.int32).reshape(8, 64)
    t = host_block_table(r2t, torch.tensor([2, 5]), torch.tensor([17, 40]), 16)
    assert t.dtype == torch.int32 and t.tolist() == [[8, 9, -1], [20, 21, 22]]
    assert host_block_table(r2t, torch.tensor([3]), torch.tensor([33]), 16).tolist() == [[12, 13, 14]]


@pytest.mark.parametrize("kw", [{"use_dsa": True}, {"override_kv_cache_dim": 640}, {"dcp_replicated": True}])
def test_mla_pool_refuses_options_it_does_not_have(kw):
    with pytest.raises(ValueError, match=next(iter(kw))):
        NeuronMLATokenToKVPool(256, 64, torch.float8_e4m3fn, 512, 64, 1, "cpu", **kw)


def test_pools_accept_options_switched_off():
    NeuronMHATokenToKVPool(64, 16, torch.bfloat16, 2, 64, 1, "cpu", quant_method=None, enable_kv_cache_copy=False,
                           v_head_dim=64, swa_head_dim=None)
    NeuronMLATokenToKVPool(256, 64, torch.float8_e4m3fn, 512, 64, 1, "cpu", use_dsa=False, dcp_replicated=False)


def test_plan_made_for_other_lengths_is_refused():
    """A plan must hold every split the host lengths need (GQA) or be cut by exactly those lengths (MLA); a mismatch
    with the device's lengths would drop keys (the host copy is what the check can see)."""
    short = ops.plan_decode(0, 3, host_seq_lens=[100, 200, 300], ctas_per_item=8, num_cus=256)
    ops.check_plan_lengths(short, 0, [100, 200, 300])
    ops.check_plan_lengths(short, 0, [50, 1, 300])  # fewer splits than planned: the extra items run empty
    with pytest.raises(ValueError, match="row 2"):
        ops.check_plan_lengths(short, 0, [100, 200, 300 + 64 * short.split_tiles])
    bound = ops.plan_decode(0, 3, max_seq_len=1000, ctas_per_item=8, num_cus=256)
    ops.check_plan_lengths(bound, 0, [1000, 17, 640])
    with pytest.raises(ValueError, match="splits"):
        ops.check_plan_lengths(bound, 0, [1000, 1000, 64000])
    mla = ops.plan_decode(1, 2, host_seq_lens=[100, 200], ctas_per_item=1, num_cus=256)
    ops.check_plan_lengths(mla, 1, [100, 200])
    with pytest.raises(ValueError, match="row 1"):
        ops.check_plan_lengths(mla, 1, [100, 201])
