"""The C ABI on the CPU: the library loads and exports every function include/sglang_neuron_amd.h declares, with the
ctypes declarations matching; the split-K planner's host logic; host-side argument checks. No kernel is launched."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from sglang_neuron_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sglang_neuron_amd.h")


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from sglang_neuron_amd import build

        build.build(verbose=False)
    return _lib.load()


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sna_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_exported_and_bound(lib):
    names = _declared()
    assert len(names) >= 14, names
    for n in names:
        assert hasattr(lib, n), f"{n} is declared but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes declaration"
    assert set(_lib.SIGNATURES) == set(names), set(_lib.SIGNATURES) ^ set(names)


def test_header_parameter_counts_match_ctypes():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for m in re.finditer(r"\b(sna_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert len(_lib.SIGNATURES[name][1]) == n, (name, n, len(_lib.SIGNATURES[name][1]))


def test_version_and_error_string(lib):
    assert lib.sna_version() == 101
    assert isinstance(lib.sna_last_error(), bytes)


def _plan(lib, kind, lens=None, B=None, max_len=-1, window=0, keys=0, ctas=1, cus=256, depth=0):
    p = _lib.SplitPlan()
    p.depth = depth
    B = len(lens) if lens is not None else B
    arr = (ctypes.c_int32 * B)(*lens) if lens is not None else None
    rc = lib.sna_plan_decode(kind, arr, B, max_len, window, keys, ctas, cus, ctypes.byref(p))
    return rc, p


def _splits(L, window, tile, split):
    if L <= 1:
        return 0
    hi, lo = L - 1, (L - window if window > 0 and L - window > 0 else 0)
    if hi <= lo:
        return 0
    t0, t1 = lo // tile, (hi + tile - 1) // tile
    return (t1 - t0 + split - 1) // split


@pytest.mark.parametrize("kind,lens,window,ctas", [
    (_lib.KIND_GQA, [4096] * 64, 0, 8),
    (_lib.KIND_GQA, [2048 + 37 * i for i in range(128)], 0, 1),
    (_lib.KIND_GQA, [2048 + 37 * i for i in range(128)], 128, 1),
    (_lib.KIND_GQA, [1, 2, 17, 33, 1000], 0, 8),
])
def test_plan_invariants(lib, kind, lens, window, ctas):
    rc, p = _plan(lib, kind, lens, window=window, ctas=ctas)
    assert rc == 0, lib.sna_last_error()
    tile = 32
    assert p.tile == tile and p.batch == len(lens)
    n = [_splits(L, window, tile, p.split_tiles) for L in lens]
    assert p.n_work == sum(n) and p.max_splits == max(n) <= 64
    assert p.empty_rows == sum(1 for x in n if x == 0)
    assert p.depth in (2, 3)
    if p.depth == 4:  # one-round plans fit the resident target unless splits are capped
        assert p.n_work * ctas <= p.target_ctas or p.split_tiles == max((max(lens) - 1 + tile - 1) // tile, 4)
    # the item map the kernels read instead of searching seq_lens: (row, split) in launch order
    want = [(b << 6) | sp | (1 << 31 if sp == nb - 1 else 0) for b, nb in enumerate(n) for sp in range(nb)]
    if len(want) <= 512 and len(lens) <= 512:
        assert p.work_n == len(want) and list(p.work[:p.work_n]) == want
    else:
        assert p.work_n == 0
    ws = lib.sna_decode_workspace_bytes(ctypes.byref(p), 16, 512)
    assert ws == (0 if p.max_splits <= 1 else p.batch * p.max_splits * 16 * (512 + 2) * 4)


def test_plan_from_a_bound_marks_empty_rows_unknown(lib):
    # past the device split's 512 rows a GQA plan from a bound keeps the bound's split: no map (the kernels search the
    # device's seq_lens), and which rows hold only their new token is unknown
    rc, p = _plan(lib, _lib.KIND_GQA, B=600, max_len=900)
    assert rc == 0 and p.empty_rows == -1 and p.work_n == 0 and p.device_split == 0


@pytest.mark.parametrize("kind,window,max_len,B", [
    (_lib.KIND_GQA, 128, 600, 5), (_lib.KIND_GQA, 128, 129, 3), (_lib.KIND_GQA, 100, 5000, 7),
    (_lib.KIND_GQA, 1, 300, 2), (_lib.KIND_GQA, 0, 4000, 9)])
def test_plan_from_a_bound_holds_every_length_up_to_it(lib, kind, window, max_len, B):
    """Every length L <= max_len: its split count fits the plan (max_splits, and n_work for B such rows), whatever
    tile offset a window starts at. A GQA plan from a bound is a device split: the launch sizes its splits from the
    device's lengths (_device_split_tiles), so the check runs that rule on batches of B rows at each length and on
    ragged batches below the bound."""
    rc, p = _plan(lib, kind, B=B, max_len=max_len, window=window, ctas=8 if kind == _lib.KIND_GQA else 1)
    assert rc == 0, lib.sna_last_error()
    if not p.device_split:
        worst = max(_splits(L, window, p.tile, p.split_tiles) for L in range(1, max_len + 1))
        assert worst <= p.max_splits and B * worst <= p.n_work, (worst, p)
        return
    import random

    import torch

    from sglang_neuron_amd import ops
    # every row gets an item (the own token of a row with no prior key is attended in a split of no tile)
    assert kind == _lib.KIND_GQA and p.work_n == 0 and p.empty_rows == 0 and p.n_work >= B and p.max_splits >= 1
    rng = random.Random(max_len * 31 + B)
    batches = [[L] * B for L in range(1, max_len + 1)]
    batches += [[rng.randint(1, max_len) for _ in range(B)] for _ in range(200)]
    for lens in batches:
        tiles = [_splits(L, window, 32, 1) for L in lens]
        st = _device_split_tiles(tiles, p.n_work)
        counts = [max(1, -(-t // st)) for t in tiles]
        assert max(counts) <= p.max_splits and sum(counts) <= p.n_work, (lens, st, p.max_splits, p.n_work)
        ops.check_plan_lengths(p, _lib.KIND_GQA, torch.tensor(lens), window=window)


def _device_split_tiles(tiles, items):
    """The split size a device-split GQA launch computes from its rows' tile counts (gqa_device_item in
    decode_gqa.hip): the least size in [start, max(longest, 4)] whose items (max(1, ceil(tiles / size)) a row) fit
    `items`, with start = ceil(total / items) and at least 4 and min(longest, 8) tiles, then at least a 64th of the
    longest row. Found here by a linear scan over the whole range, so the kernel's bisection bracket (its upper end
    ceil(total / (items - B))) is checked against the definition."""
    B = len(tiles)
    items = max(items, B)
    total, mx = sum(tiles), max(tiles, default=0)
    cap = max(mx, 4)
    st = min(max(4, -(-total // items), min(mx, 8)), cap)
    fits = [s for s in range(st, cap + 1) if sum(max(1, -(-t // s)) for t in tiles) <= items]
    least = fits[0]
    if items > B:
        assert least <= min(cap, max(st, -(-total // (items - B))))
    return max(least, -(-mx // 64))


def test_gqa_plan_from_a_bound_is_a_device_split(lib):
    """Up to 512 rows a GQA plan from a bound splits on the device (n_work items, one per row at least, and room for
    4-tile splits of the bound); past 512 it keeps the bound's own split; with host lengths it is exact."""
    rc, p = _plan(lib, _lib.KIND_GQA, B=128, max_len=8192, ctas=1, cus=256)
    assert rc == 0 and p.device_split == 1 and p.n_work == 512 and p.max_splits == 32 and p.work_n == 0
    assert p.empty_rows == 0  # every row gets a split: no lone-token pass
    # 64 rows of the bound: the bound's split is whole rows, so every launch's is (n_work = B): one split a row
    rc, p = _plan(lib, _lib.KIND_GQA, B=64, max_len=4096, ctas=8, cus=256)
    assert rc == 0 and p.device_split == 1 and p.n_work == 64 and p.max_splits == 1
    rc, p = _plan(lib, _lib.KIND_GQA, B=600, max_len=8192, ctas=1, cus=256)
    assert rc == 0 and p.device_split == 0 and p.n_work >= 600
    rc, p = _plan(lib, _lib.KIND_GQA, [100, 4000, 9000], ctas=1, cus=256)
    assert rc == 0 and p.device_split == 0
    rc, p = _plan(lib, _lib.KIND_GQA, B=3, max_len=40, ctas=8, cus=256)
    assert rc == 0 and p.device_split == 1 and p.max_splits == 1 and p.n_work >= 3
    rc, p = _plan(lib, _lib.KIND_GQA, B=5, max_len=1, ctas=8, cus=256)  # own tokens only: a split each, no tile
    assert rc == 0 and p.device_split == 1 and p.max_splits == 1 and p.n_work == 5
    # a sliding window of 128 keys spans at most 5 tiles: one split a row, written without a combine pass
    rc, p = _plan(lib, _lib.KIND_GQA, B=128, max_len=8192, window=128, ctas=1, cus=256)
    assert rc == 0 and p.device_split == 1 and p.max_splits == 1
    assert lib.sna_decode_workspace_bytes(ctypes.byref(p), 8, 64) == 0
    rc, p = _plan(lib, _lib.KIND_GQA, B=2, max_len=32 * (1 << 17) + 64, ctas=1, cus=256)  # past the device bound
    assert rc == 0 and p.device_split == 0


def _row_tiles(keys):
    return [max((k + 15) // 16, 1) for k in keys]


def _check_stream_plan(p, keys, cus, ctas=1):
    """The MLA / DSA stream split by brute force: every row's tiles (at least one) end to end, cut into n_ctas ranges
    that start where cta_row / cta_off say. With a workgroup per row the rows are apportioned whole: no range spans
    two rows, a row's pieces differ by at most one tile, and no other apportionment of the workgroups has a shorter
    longest piece. Otherwise the ranges are equal (+-1). max_splits is the most ranges any row meets."""
    tiles = _row_tiles(keys)
    first = [0]
    for t in tiles:
        first.append(first[-1] + t)
    total = first[-1]
    n = p.n_ctas
    assert p.tile == 16 and p.total_tiles == total and list(p.row_keys[:len(keys)]) == list(keys)
    assert 1 <= n <= min(cus // ctas, 256, total)
    starts = list(p.cta_start[:n + 1])
    assert starts[0] == 0 and starts[-1] == total
    sizes = [starts[w + 1] - starts[w] for w in range(n)]
    assert min(sizes) >= 1 and p.split_tiles == max(sizes)
    for w in range(n):
        r = p.cta_row[w]
        assert first[r] <= starts[w] < first[r + 1] and starts[w] - first[r] == p.cta_off[w]
    meets = [sum(1 for w in range(n) if starts[w] < first[b + 1] and starts[w + 1] > first[b])
             for b in range(len(keys))]
    assert p.max_splits == max(meets)
    if len(keys) <= n:
        assert all(starts[w + 1] <= first[p.cta_row[w] + 1] for w in range(n)), "a range spans two rows"
        for b, t in enumerate(tiles):
            mine = [sizes[w] for w in range(n) if p.cta_row[w] == b]
            assert sum(mine) == t and max(mine) - min(mine) <= 1
        # optimality of the longest piece: fewer than n workgroups cannot give every row pieces of <= longest - 1
        shorter = max(sizes) - 1
        if shorter >= 1:
            assert sum(-(-t // shorter) for t in tiles) > n
    else:
        assert max(sizes) - min(sizes) <= 1
    assert p.empty_rows == sum(1 for k in keys if k == 0)


@pytest.mark.parametrize("lens,ctas,cus", [([1024 + 467 * i for i in range(32)], 1, 256), ([1, 5, 70000], 2, 256),
                                          ([1] * 7, 1, 256), ([16385] * 8, 1, 80), ([3000] * 256, 1, 256)])
def test_mla_stream_plan(lib, lens, ctas, cus):
    rc, p = _plan(lib, _lib.KIND_MLA, lens, ctas=ctas, cus=cus)
    assert rc == 0, lib.sna_last_error()
    _check_stream_plan(p, [L - 1 for L in lens], cus, ctas)
    ws = lib.sna_decode_workspace_bytes(ctypes.byref(p), 16 * ctas, 512)
    assert ws == 262144 + 2 * p.n_ctas * 16 * ctas * (512 + 2) * 4


def test_dsa_stream_plan(lib):
    rc, p = _plan(lib, _lib.KIND_DSA, B=16, keys=2048, ctas=1)
    assert rc == 0
    _check_stream_plan(p, [2048] * 16, 256)
    assert max(p.cta_start[w + 1] - p.cta_start[w] for w in range(p.n_ctas)) <= 2048 // 16
    rc, p = _plan(lib, _lib.KIND_DSA, B=3, keys=0, ctas=1)  # empty index lists: one tile each for the own rows
    assert rc == 0 and p.total_tiles == 3 and p.empty_rows == 3


@pytest.mark.parametrize("B,K,ctas", [(20, 3000, 1), (16, 2064, 1), (5, 4096, 1), (64, 4000, 1), (100, 2500, 2),
                                      (7, 2049, 4), (256, 2048, 1), (3, 4095, 8)])
def test_dsa_plan_ranges_fit_the_sparse_cap(lib, B, K, ctas):
    """A sparse workgroup resolves at most 2048 indices (128 tiles) in LDS: every range of a DSA plan holds at most
    that many, whole rows longer than it included (each gets enough pieces)."""
    rc, p = _plan(lib, _lib.KIND_DSA, B=B, keys=K, ctas=ctas)
    assert rc == 0, lib.sna_last_error()
    sizes = [p.cta_start[w + 1] - p.cta_start[w] for w in range(p.n_ctas)]
    assert max(sizes) <= 2048 // 16 and min(sizes) >= 1
    assert p.cta_start[p.n_ctas] == p.total_tiles == B * max((K + 15) // 16, 1)
    tiles = max((K + 15) // 16, 1)
    if B <= p.n_ctas:  # whole rows: every range inside one row
        assert all(p.cta_start[w] // tiles == (p.cta_start[w + 1] - 1) // tiles for w in range(p.n_ctas))


def test_stream_row_chunks_fit_one_plan_each(lib):
    """ops.stream_row_chunks splits a batch past one launch's limits (rows, merge counters, sparse workgroups) into
    row ranges each of which plans."""
    from sglang_neuron_amd import ops
    for kind, B, H, K in ((_lib.KIND_MLA, 300, 16, 0), (_lib.KIND_MLA, 600, 128, 0), (_lib.KIND_DSA, 300, 16, 3000),
                          (_lib.KIND_DSA, 90, 64, 9000), (_lib.KIND_MLA, 40, 16, 0)):
        chunks = ops.stream_row_chunks(kind, B, H, K)
        assert chunks[0][0] == 0 and chunks[-1][1] == B
        assert all(a[1] == b[0] for a, b in zip(chunks, chunks[1:]))
        for r0, r1 in chunks:
            lens = [1000 + 37 * i for i in range(r1 - r0)] if kind == _lib.KIND_MLA else None
            rc, _ = _plan(lib, kind, lens, B=r1 - r0, keys=K, ctas=(H + 15) // 16)
            assert rc == 0, (kind, B, H, K, r0, r1, lib.sna_last_error())
    assert ops.stream_row_chunks(_lib.KIND_MLA, 40, 16) == [(0, 40)]


def test_stream_workspace_calls_refuse_bad_arguments(lib):
    """The workspace status and reset calls refuse a null workspace or one smaller than the counter block before
    touching a device."""
    st = ctypes.c_int32(0)
    assert lib.sna_stream_workspace_status(None, 1 << 20, ctypes.addressof(st), None) == _lib.SNA_ERR_INVALID_ARGUMENT
    assert lib.sna_stream_workspace_status(ctypes.c_void_p(64), 4096, ctypes.addressof(st), None) == \
        _lib.SNA_ERR_INVALID_ARGUMENT
    assert lib.sna_stream_workspace_reset(ctypes.c_void_p(64), 4096, None) == _lib.SNA_ERR_INVALID_ARGUMENT
    assert b"counter block" in lib.sna_last_error()


def test_mla_plan_from_a_bound_is_a_device_split(lib):
    """Without host lengths an MLA plan is a device split: the launch cuts its stream from the device's seq_lens, so
    the plan fixes only the grid (a workgroup per CU and head group) and the workspace it is sized for."""
    rc, p = _plan(lib, _lib.KIND_MLA, None, B=4, max_len=3000, ctas=2, cus=256)
    assert rc == 0 and p.device_split == 1 and p.n_ctas == 128 and p.batch == 4 and p.tile == 16
    assert list(p.row_keys[:4]) == [2999] * 4
    assert lib.sna_decode_workspace_bytes(ctypes.byref(p), 32, 512) == 262144 + 2 * 128 * 32 * 514 * 4
    rc, q = _plan(lib, _lib.KIND_MLA, [100, 200])
    assert rc == 0 and q.device_split == 0
    assert _plan(lib, _lib.KIND_MLA, None, B=4, max_len=16 * 65535 + 2)[0] == _lib.SNA_ERR_UNSUPPORTED
    assert _plan(lib, _lib.KIND_MLA, None, B=4, max_len=0)[0] == _lib.SNA_ERR_UNSUPPORTED
    # a sparse decode refuses it
    rc = lib.sna_mla_decode_sparse(None, None, None, 1.0, None, 16, None, 0, 0, None, None, None, 0.1, None, None, 4,
                                   1, 16, 64, 10, ctypes.byref(p), None, 0, None)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"device-split" in lib.sna_last_error()


def test_stream_plan_refusals(lib):
    assert _plan(lib, _lib.KIND_MLA, [100] * 257)[0] == _lib.SNA_ERR_UNSUPPORTED  # past SNA_MAX_PLAN_ROWS
    assert _plan(lib, _lib.KIND_MLA, [16 * 65536])[0] == _lib.SNA_ERR_UNSUPPORTED  # a row past 65535 tiles
    assert _plan(lib, _lib.KIND_MLA, [0, 5])[0] == _lib.SNA_ERR_INVALID_ARGUMENT  # seq_len 0
    # more (row, head group) pairs than a launch's merge counters
    assert _plan(lib, _lib.KIND_MLA, [100] * 256, ctas=8)[0] == _lib.SNA_ERR_UNSUPPORTED
    assert b"merge counters" in lib.sna_last_error()
    assert _plan(lib, _lib.KIND_DSA, B=200, keys=3000)[0] == _lib.SNA_ERR_UNSUPPORTED  # 400 sparse workgroups


def test_plan_rejects_bad_arguments(lib):
    assert _plan(lib, 7, [10])[0] == _lib.SNA_ERR_INVALID_ARGUMENT
    assert _plan(lib, _lib.KIND_GQA, [10], ctas=0)[0] == _lib.SNA_ERR_INVALID_ARGUMENT
    assert _plan(lib, _lib.KIND_GQA, None, B=2, max_len=-1)[0] == _lib.SNA_ERR_INVALID_ARGUMENT
    rc = lib.sna_plan_decode(0, None, 1, 10, 0, 0, 1, 256, None)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"null plan" in lib.sna_last_error()


def test_decode_entry_checks_arguments_before_touching_the_gpu(lib):
    rc, p = _plan(lib, _lib.KIND_GQA, [100, 200], ctas=2)
    null = None
    # 5 query heads over 2 KV heads
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 0, 0, null, null, null, null, null, 0, 0.1, null,
                                  2, 5, 2, 128, 16, 10, 1, ctypes.byref(p), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"head counts" in lib.sna_last_error()
    # head_dim 96 is not built
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 0, 0, null, null, null, null, null, 0, 0.1, null,
                                  2, 4, 2, 96, 16, 10, 1, ctypes.byref(p), null, 0, null)
    assert rc == _lib.SNA_ERR_UNSUPPORTED
    # null tensors with a valid shape
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 8, 8, null, null, null, null, null, 0, 0.1, null,
                                  2, 4, 2, 128, 16, 10, 1, ctypes.byref(p), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"null pointer" in lib.sna_last_error()
    # a plan made for another batch
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 8, 8, null, null, null, null, null, 0, 0.1, null,
                                  3, 4, 2, 128, 16, 10, 1, ctypes.byref(p), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"plan" in lib.sna_last_error()
    # a plan whose item map names a row past the batch, or more entries than the map holds
    assert p.work_n == p.n_work > 0
    bad = _lib.SplitPlan.from_buffer_copy(p)
    bad.work[0] = (2 << 6) | 0
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 8, 8, null, null, null, null, null, 0, 0.1, null,
                                  2, 4, 2, 128, 16, 10, 1, ctypes.byref(bad), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"item" in lib.sna_last_error()
    # a map whose rows are not consecutive, splits in order (the kernel counts a row's splits from it)
    rc2, p2 = _plan(lib, _lib.KIND_GQA, [3000, 3000], ctas=2)
    assert rc2 == 0 and p2.work_n >= 4
    bad = _lib.SplitPlan.from_buffer_copy(p2)
    bad.work[0], bad.work[1] = bad.work[1], bad.work[0]
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 8, 8, null, null, null, null, null, 0, 0.1, null,
                                  2, 4, 2, 128, 16, 10, 1, ctypes.byref(bad), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"out of order" in lib.sna_last_error()
    bad = _lib.SplitPlan.from_buffer_copy(p2)
    bad.work[0] |= 1 << 31  # a row's first item flagged as its last
    rc = lib.sna_paged_decode_gqa(null, null, null, null, null, null, 8, 8, null, null, null, null, null, 0, 0.1, null,
                                  2, 4, 2, 128, 16, 10, 1, ctypes.byref(bad), null, 0, null)
    assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"mis-flagged" in lib.sna_last_error()
    rcm, pm = _plan(lib, _lib.KIND_MLA, [100, 200])
    assert rcm == 0 and pm.n_ctas > 0
    for field, value in (("total_tiles", 3), ("cta_off", None), ("cta_row", None)):
        bad = _lib.SplitPlan.from_buffer_copy(pm)
        if field == "total_tiles":
            bad.total_tiles = value
        elif field == "cta_off":
            bad.cta_off[1] += 1
        else:
            bad.cta_row[0] = 5
        rc = lib.sna_mla_decode(null, null, null, null, null, 0, 0, null, null, null, 0.1, null, 2, 16, 64, 10, 1,
                                ctypes.byref(bad), null, 0, null)
        assert rc == _lib.SNA_ERR_INVALID_ARGUMENT and b"plan" in lib.sna_last_error(), field
    # an empty batch is a no-op
    rc0, p0 = _plan(lib, _lib.KIND_GQA, B=0, max_len=0)
    assert rc0 == 0
    assert lib.sna_paged_decode_gqa(null, null, null, null, null, null, 0, 0, null, null, null, null, null, 0, 0.1,
                                    null, 0, 4, 2, 128, 16, 10, 1, ctypes.byref(p0), null, 0, null) == 0


def test_store_entries_check_arguments(lib):
    assert lib.sna_kv_store_mha(None, None, None, 4, None, None, None, None, 10, 2, 16, 100, 1, None) < 0
    assert lib.sna_kv_store_mla(None, None, 4, 576, None, None, 100, 1, None) < 0
    assert lib.sna_kv_store_dsa(None, None, 4, 0.5, None, 100, None) < 0
    assert lib.sna_kv_store_mha(None, None, None, 0, None, None, None, None, 10, 2, 16, 128, 0, None) == 0
