#!/usr/bin/env python
"""Benchmark of the paged decode-attention step on one MI355X (the metric of BASELINE.json).

A step is one decode of the whole batch: the new token's store, the decode kernel(s), and (GQA rows split over
several workgroups) the combine pass. The default line is cfg2 (Qwen3-8B-shaped GQA, FP8 e4m3fn KV with per-KV-head
scales, B64 H32 G8 d128, L=4096, page 16), the metric's workload, and carries every other config under "per_config".
Inputs are resident in HBM; the pool is rotated over copies whose total exceeds the 256 MB Infinity Cache several
times, so every step reads cold HBM.

One JSON line on stdout:
  value         algorithmic HBM bytes of the step / step time, GB/s (higher is better); ms_per_step beside it. The
                step time: the K steps captured in one HIP graph on the stream the kernels launch on, one untimed
                replay, then one HIP event pair (torch events) around one replay, divided by K. The same K steps
                launched one by one from the host (after W warm-up steps, one event pair around them) are reported as
                us_per_step_launched: for the small steps (cfg1, cfg4's window layer) that number is the host's
                launch rate.
  roofline      the step's kernels (cfg2: the one split-K decode kernel): their algorithmic bytes per step / the step
                time, against MI355X's 8 TB/s. traffic = FETCH_SIZE + WRITE_SIZE per step from the committed
                rocprofv3 counter summary (traffic_source says which), else null.
  cpu_baseline  the CPU oracle (a torch restatement of the reference's torch path) on a bounded sample of the same
                workload, timed on this host's cores (2 warm-ups, median of 5 runs).
  per_config    cfg1, cfg3, cfg4 (full and sliding-window layers), cfg5, cfg3 over bf16 rows and cfg5 as an MTP
                verify step (8 query tokens per sequence), each with us_per_step, its roofline and cpu_baseline.

Options: --config {1,2,3,4,4swa,5,3bf16,5mtp} prints that workload's line alone (3bf16: cfg3 over bf16 rows, the
reference's served DeepSeek-V2 pool; 5mtp: cfg5 as GLM's MTP verify, 8 query tokens per sequence); --config meta
times the device-side decode
metadata (block table, window trim) instead, --config prefill the segmented prefill attention, --config indexer the
DSA indexer, --config qkv the QKV writer, --config wire the PD page items; --all prints one line per workload;
--no-per-config drops the per_config map; --gpus above 1 is refused, because this build measures one GPU.
"""

from __future__ import annotations

import argparse
import functools
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode-attn µs/step + achieved HBM GB/s (% of peak), FP8 KV, 1 MI355X"
PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
COLD_BYTES = 1 << 30  # rotate pool copies until the rotation spans this much (4x the Infinity Cache)
COPY_CALIBRATION_BYTES = 1 << 30


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _copies(touched_bytes: int, pool_bytes: int, cap: int) -> int:
    n = max(2, math.ceil(COLD_BYTES / max(touched_bytes, 1)))
    n = min(n, cap, max(2, (64 << 30) // max(pool_bytes, 1)))
    return n


def _traffic(workload: str):
    """(FETCH_SIZE + WRITE_SIZE bytes per step, where they come from) from profiles/traffic_<workload>.json, the
    committed summary of two rocprofv3 counter passes; (None, None) when no such pass was committed."""
    p = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(p):
        return None, None
    with open(p) as f:
        d = json.load(f)
    b = d.get("bytes_per_step", d.get("bytes_per_launch"))
    return b, f"committed rocprofv3 counter passes (profiles/traffic_{workload}.json), not this run"


def _mfma_counters(workload: str):
    """The step's MFMA busy share and bf16 MFMA flops from profiles/mfma_<workload>.json, the committed summary of a
    rocprofv3 pass of the derived counters MfmaUtil and MfmaFlopsBF16; None when no such pass was committed."""
    p = os.path.join(ROOT, "profiles", f"mfma_{workload}.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)


def time_us(fn, n_steps: int, warmup: int) -> float:
    """Microseconds per call of fn(i): warmup calls, then one HIP event pair (torch events, recorded on torch's current
    stream, the stream every launch here goes to) around n_steps back-to-back calls."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n_steps):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n_steps * 1e3


def time_us_graph(fn, n_steps: int) -> float:
    """Microseconds per call of fn(i) with the n_steps calls captured in one HIP graph (torch.cuda.CUDAGraph, on the
    current stream, which the calls are bound to): one untimed replay, then one HIP event pair around one replay of
    all n_steps calls. The GPU's time for the steps, without the host's per-call launch cost (a serving loop replays
    such a graph)."""
    import torch

    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=torch.cuda.current_stream()):
        for i in range(n_steps):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / n_steps * 1e3
    del g
    return us


def cpu_threads() -> int:
    """The CPU baseline's thread count: the host's cores, capped by OMP_NUM_THREADS (a GPU box grants each GPU a share
    of its cores through it)."""
    n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() else n


def cpu_median_s(run) -> float:
    """Seconds per call of run(): 2 warm-up calls, then the median of 5 timed calls, on cpu_threads() threads."""
    import torch

    torch.set_num_threads(cpu_threads())
    for _ in range(2):
        run()
    times = []
    for _ in range(5):
        t = time.perf_counter()
        run()
        times.append(time.perf_counter() - t)
    return statistics.median(times)


# ---------------------------------------------------------------------------------------------------------------
# workloads: each returns (steps [Prepared per pool copy], description dict, alg bytes of the step, the step's kernels,
# the MFMA flops they issue, a CPU-baseline callable, and the step's two halves timed apart: "store" (the standalone
# store kernel of the step's new tokens) and "decode" (the decode without its fused store), each a callable per pool
# copy)
# ---------------------------------------------------------------------------------------------------------------

def setup_gqa(cfg: int, window: int, dev):
    import torch

    from sglang_neuron_amd import ops, workloads

    over = {"window": window} if window else {}
    t0 = time.time()
    case = workloads.gqa_case(cfg, gen_device=dev, overrides=over)
    kc, vc, ks, vs = workloads.gqa_pool(case, dev)
    pool_bytes = kc.numel() * kc.element_size() * 2
    touched = case.kv_bytes_per_step()
    n = _copies(touched, pool_bytes, 64)
    pools = [(kc, vc)] + [(kc.clone(), vc.clone()) for _ in range(n - 1)]
    torch.cuda.synchronize()
    log(f"cfg{cfg}{' swa' if window else ''}: B={case.B} H={case.H} G={case.G} d={case.d} P={case.P} "
        f"tokens={int(case.seq_lens.sum())} pool={pool_bytes / 1e6:.1f} MB x {n} copies, built in {time.time() - t0:.1f}s")
    q, table, lens = case.q, case.block_table.to(dev), case.seq_lens.to(dev)
    kn, vn, slots = case.k_new.to(dev), case.v_new.to(dev), case.new_slots.to(dev)
    sinks = None if case.sinks is None else case.sinks.to(dev)
    plan = ops.plan_decode(0, case.B, host_seq_lens=case.seq_lens, window=case.window, ctas_per_item=case.G,
                           num_cus=ops._num_cus(q.device))
    out = torch.empty(case.B, case.H, case.d, dtype=torch.bfloat16, device=dev)
    mul = case.scales_multiply
    steps = [ops.prepare_paged_decode_gqa(q, k, v, table, lens, kn, vn, sm_scale=case.sm_scale, k_scale=ks,
                                          v_scale=vs, sinks=sinks, window=case.window, new_slots=slots, out=out,
                                          plan=plan, scales_multiply=mul) for (k, v) in pools]
    legs = {"store": [functools.partial(ops.kv_store_mha, kn, vn, slots, k, v, ks, vs, scales_multiply=mul)
                      for (k, v) in pools],
            "decode": [ops.prepare_paged_decode_gqa(q, k, v, table, lens, kn, vn, sm_scale=case.sm_scale, k_scale=ks,
                                                    v_scale=vs, sinks=sinks, window=case.window, out=out, plan=plan,
                                                    scales_multiply=mul)
                       for (k, v) in pools]}
    # the step under a plan from a bound (the block table's width), as a serving graph captured once for growing
    # lengths runs it: a device split, whose launch sizes its splits and locates its items from the device's seq_lens
    plan_b = ops.plan_decode(0, case.B, max_seq_len=table.shape[1] * case.P, window=case.window, ctas_per_item=case.G,
                             num_cus=ops._num_cus(q.device))
    legs["bound_plan"] = [ops.prepare_paged_decode_gqa(q, k, v, table, lens, kn, vn, sm_scale=case.sm_scale,
                                                       k_scale=ks, v_scale=vs, sinks=sinks, window=case.window,
                                                       new_slots=slots, out=out, plan=plan_b, scales_multiply=mul)
                          for (k, v) in pools]
    tiles = 0
    for L in case.seq_lens.tolist():
        hi = L - 1
        lo = max(0, L - case.window) if case.window else 0
        if hi > lo:
            tiles += -(-hi // 32) - lo // 32
    steps_qk, dt = case.d // 32, case.d // 16
    mfma_flops = tiles * case.G * (2 * steps_qk + dt) * (16 * 16 * 32 * 2)
    name = {1: "qwen3-0.6b-gqa-bf16", 2: "qwen3-8b-gqa-fp8", 4: "gpt-oss-120b-share-fp8"}[cfg]
    desc = {"workload": f"cfg{cfg}{'-swa' + str(window) if window else ''}: {name}", "batch": case.B,
            "q_heads": case.H, "kv_heads": case.G, "head_dim": case.d, "page_size": case.P,
            "kv_dtype": ("fp8_e4m3fn, the GPT-OSS decode write (bf16 product with the inverted bf16 scale)" if mul
                         else "fp8_e4m3fn per-KV-head scale") if case.fp8 else "bf16",
            "seq_len": "4096" if cfg == 2 else f"U{list(workloads.GQA_CONFIGS[cfg]['lens'])}",
            "window": case.window or None, "sinks": case.sinks is not None, "pool_copies": n,
            "split_plan": {"split_tiles": plan.split_tiles, "n_work": plan.n_work}}

    def cpu_baseline(budget_s: float):
        from oracle import attention as oatt
        from oracle import store as ost

        kcpu = pools[0][0].cpu().view(torch.uint8) if case.fp8 else pools[0][0].cpu()
        vcpu = pools[0][1].cpu().view(torch.uint8) if case.fp8 else pools[0][1].cpu()
        kss = None if ks is None else ks.cpu()
        vss = None if vs is None else vs.cpu()
        qc, knc, vnc = q.cpu(), kn.cpu(), vn.cpu()
        sk = None if sinks is None else sinks.cpu()

        def run(nrows):
            oatt.paged_decode_gqa(qc[:nrows], kcpu, vcpu, case.block_table[:nrows], case.seq_lens[:nrows],
                                  knc[:nrows], vnc[:nrows], sm_scale=case.sm_scale, k_scale=kss, v_scale=vss,
                                  sinks=sk, window=case.window, scales_multiply=mul)
            ost.kv_store_mha(knc[:nrows], vnc[:nrows], case.new_slots[:nrows], kcpu, vcpu, kss, vss, mul)

        return _time_rows(run, case.B, budget_s)

    kernels = ["gqa_decode_kernel"] + (["gqa_combine_kernel"] if plan.max_splits > 1 else []) + \
        (["gqa_lone_token_kernel"] if bool((case.seq_lens == 1).any()) else [])
    return steps, desc, case.kv_bytes_per_step(), kernels, mfma_flops, cpu_baseline, legs


def setup_mla(dev, bf16: bool = False):
    import torch

    from sglang_neuron_amd import ops, workloads

    t0 = time.time()
    case = workloads.mla_case(gen_device=dev)
    cache, scale = workloads.mla_pool(case, dev, bf16)
    pool_bytes = cache.numel() * cache.element_size() + (0 if bf16 else scale.numel() * 4)
    n = _copies(case.kv_bytes_per_step(bf16), pool_bytes, 64)
    pools = [(cache, scale)] + [(cache.clone(), None if bf16 else scale.clone()) for _ in range(n - 1)]
    torch.cuda.synchronize()
    log(f"cfg3{'-bf16' if bf16 else ''}: B={case.B} H={case.H} P={case.P} tokens={int(case.seq_lens.sum())} "
        f"pool={pool_bytes / 1e6:.1f} MB x {n} copies, built in {time.time() - t0:.1f}s")
    table, lens = case.block_table.to(dev), case.seq_lens.to(dev)
    plan = ops.plan_decode(1, case.B, host_seq_lens=case.seq_lens, ctas_per_item=1, num_cus=ops._num_cus(table.device))
    out = torch.empty(case.B, case.H, 512, dtype=torch.bfloat16, device=dev)
    new_slots = case.new_slots.to(dev)
    hl = case.seq_lens
    steps = [ops.prepare_mla_decode(case.ql_nope, case.q_pe, c, s, table, lens, case.compact_new,
                                    sm_scale=case.sm_scale, page_size=case.P, new_slots=new_slots,
                                    out=out, plan=plan, host_seq_lens=hl) for (c, s) in pools]
    legs = {"store": [functools.partial(ops.kv_store_mla, case.compact_new, new_slots, c, s) for (c, s) in pools],
            "decode": [ops.prepare_mla_decode(case.ql_nope, case.q_pe, c, s, table, lens, case.compact_new,
                                              sm_scale=case.sm_scale, page_size=case.P, out=out, plan=plan,
                                              host_seq_lens=hl)
                       for (c, s) in pools]}
    # the step under a device-split plan from a bound (the block table's width): the launch cuts its split from the
    # device's seq_lens, as a serving graph captured once for growing lengths runs it
    plan_b = ops.plan_decode(1, case.B, max_seq_len=table.shape[1] * case.P, ctas_per_item=1,
                             num_cus=ops._num_cus(table.device))
    legs["bound_plan"] = [ops.prepare_mla_decode(case.ql_nope, case.q_pe, c, s, table, lens, case.compact_new,
                                                 sm_scale=case.sm_scale, page_size=case.P, new_slots=new_slots,
                                                 out=out, plan=plan_b) for (c, s) in pools]
    tiles = int(((case.seq_lens - 1 + 15) // 16).sum())
    # bf16 rows: 18 QK steps of 16x16x32 and 32 PV steps of 16x16x16 (bf16); FP8 rows: the latent QK as 8 scaled FP8
    # 16x16x128 (4 blocks, the query's two parts), the rope as 2 bf16 16x16x32, PV as 32 bf16 16x16x16
    if bf16:
        mfma_flops = tiles * (18 * 16 * 16 * 32 * 2 + 32 * 16 * 16 * 16 * 2)
    else:
        mfma_flops = {"bf16": tiles * (2 * 16 * 16 * 32 * 2 + 32 * 16 * 16 * 16 * 2), "fp8": tiles * 8 * 16 * 16 * 128 * 2}
    desc = {"workload": "cfg3-bf16: deepseek-v2-lite absorbed MLA, bf16 rows (the reference's served dtype)" if bf16
            else "cfg3: deepseek-v2-lite absorbed MLA", "batch": case.B, "q_heads": case.H,
            "qk_dim": 576, "v_dim": 512, "page_size": case.P,
            "kv_dtype": "bf16" if bf16 else "fp8_e4m3fn per-token scale",
            "seq_len": "U[1024, 16384]", "pool_copies": n,
            "split_plan": {"split_tiles": plan.split_tiles, "n_work": plan.n_work}}

    def cpu_baseline(budget_s: float):
        from oracle import attention as oatt
        from oracle import store as ost

        c0, s0 = pools[0][0].cpu(), None if bf16 else pools[0][1].cpu()
        ql, qp, cn = case.ql_nope.cpu(), case.q_pe.cpu(), case.compact_new.cpu()

        def run(nrows):
            oatt.mla_decode(ql[:nrows], qp[:nrows], c0, s0, case.block_table[:nrows], case.seq_lens[:nrows],
                            cn[:nrows], sm_scale=case.sm_scale, page_size=case.P)
            ost.kv_store_mla(cn[:nrows], case.new_slots[:nrows], c0, s0)

        return _time_rows(run, case.B, budget_s)

    return steps, desc, case.kv_bytes_per_step(bf16), ["mla_decode_kernel"], mfma_flops, cpu_baseline, legs


def setup_dsa(dev, spec: int = 1):
    import torch

    from sglang_neuron_amd import ops, workloads

    t0 = time.time()
    case = workloads.dsa_case(gen_device=dev, overrides={"spec": spec})
    cache = workloads.dsa_pool(case, dev, gen_device=dev)
    pool_bytes = cache.numel()
    n = _copies(case.kv_bytes_per_step(), pool_bytes, 16)
    pools = [cache] + [cache.clone() for _ in range(n - 1)]
    torch.cuda.synchronize()
    wl = "cfg5" if spec == 1 else f"cfg5-mtp{spec}"
    log(f"{wl}: B={case.B} spec={spec} H={case.H} K={case.indices.shape[1]} pool={pool_bytes / 1e9:.2f} GB x {n} "
        f"copies, built in {time.time() - t0:.1f}s")
    idx, table, pos = case.indices.to(dev), case.block_table.to(dev), case.positions.to(dev)
    T = case.B * spec
    keys = case.indices.shape[1] + spec - 1  # a token's keys: its index list, then its siblings' own rows
    plan = ops.plan_decode(2, T, n_keys_per_row=keys, ctas_per_item=1, num_cus=ops._num_cus(idx.device))
    new_slots = case.new_slots.to(dev)
    steps = [ops.prepare_mla_decode_sparse(case.q_absorbed, case.q_pe, c, case.kv_scale, idx, table, pos,
                                           case.own_rows, sm_scale=case.sm_scale, page_size=case.P,
                                           new_slots=new_slots, plan=plan, spec=spec) for c in pools]
    legs = {"store": [functools.partial(ops.kv_store_dsa, case.own_rows, new_slots, c, case.kv_scale) for c in pools],
            "decode": [ops.prepare_mla_decode_sparse(case.q_absorbed, case.q_pe, c, case.kv_scale, idx, table, pos,
                                                     case.own_rows, sm_scale=case.sm_scale, page_size=case.P,
                                                     plan=plan, spec=spec) for c in pools]}
    tiles = T * (-(-keys // 16))
    mfma_flops = tiles * (18 * 16 * 16 * 32 * 2 + 32 * 16 * 16 * 16 * 2)
    desc = {"workload": f"{wl}: glm-5.2-style DSA absorbed MLA" + (f", MTP verify ({spec} query tokens per sequence)"
                                                                    if spec > 1 else ""),
            "batch": case.B, "query_tokens_per_seq": spec, "q_heads": case.H,
            "indices_per_row": case.indices.shape[1], "pool_positions_per_seq": case.pool_positions,
            "page_size": case.P, "kv_dtype": "fp8_e4m3fn latent + bf16 rope, 640-byte rows, kv_scale 2^-6",
            "short_rows": list(workloads.DSA_CONFIG["short_rows"]), "pool_copies": n,
            "split_plan": {"split_tiles": plan.split_tiles, "n_work": plan.n_work}}

    def cpu_baseline(budget_s: float):
        from oracle import attention as oatt

        c0 = pools[0].cpu()
        qa, qp, own = case.q_absorbed.cpu(), case.q_pe.cpu(), case.own_rows.cpu()

        def run(nseq):  # the first nseq sequences (their spec tokens each)
            t = nseq * spec
            oatt.mla_decode_sparse(qa[:t], qp[:t], c0, case.kv_scale, case.indices[:t], case.block_table[:nseq],
                                   case.positions[:t], own[:t], case.new_slots[:t], sm_scale=case.sm_scale,
                                   page_size=case.P, inplace=True, spec=spec)

        return _time_rows(run, case.B, budget_s)

    return steps, desc, case.kv_bytes_per_step(), ["mla_decode_kernel"], mfma_flops, cpu_baseline, legs


def _time_rows(run, B: int, budget_s: float):
    """Time the CPU oracle on the first n rows (n sized to the budget: 2 warm-ups and 5 timed runs in about budget_s),
    median of the 5 timed runs, scaled to the whole batch."""
    import torch

    torch.set_num_threads(cpu_threads())
    t = time.perf_counter()
    run(1)
    t1 = time.perf_counter() - t
    nrows = max(1, min(B, int(budget_s / 7 / max(t1, 1e-6))))
    for _ in range(2):
        run(nrows)
    times = []
    for _ in range(5):
        t = time.perf_counter()
        run(nrows)
        times.append(time.perf_counter() - t)
    med = statistics.median(times)
    return {"value": round(med * (B / nrows) * 1e6, 1), "unit": "us/step", "cores": torch.get_num_threads(),
            "host_cpus": os.cpu_count(), "kind": "port",
            "sample": f"rows 0..{nrows - 1} of {B} (2 warm-ups, median of 5 runs, scaled x{B / nrows:.2f} to the batch)",
            "cpu": cpu_model()}


# ---------------------------------------------------------------------------------------------------------------

META_METRIC = "decode metadata build µs/step (block table from req_to_token + window trim), 1 MI355X"


def run_meta(steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev) -> dict:
    """The device-side metadata of one decode forward (ops.block_table, then ops.window_table for a 128-key window)
    for a serving batch: 256 rows of U[1, 8192] tokens, page 16, req_to_token [1024, 8192] int32, rotated over copies
    past the Infinity Cache. The roofline figure is the block-table kernel's algorithmic bytes (4 B read + 4 B
    written per entry, 16 B per row) over its time; its req_to_token reads are strided (one 4-byte entry per page),
    so HBM moves a whole sector for each."""
    import numpy as np
    import torch

    from sglang_neuron_amd import ops

    B, P, ctx, nrows, window = 256, 16, 8192, 1024, 128
    g = np.random.default_rng(7)
    r2t_host = g.integers(0, 1 << 22, size=(nrows, ctx), dtype=np.int32)
    rows = g.permutation(nrows)[:B].astype(np.int64)
    lens = g.integers(1, ctx + 1, size=B).astype(np.int64)
    width = -(-int(lens.max()) // P)
    nb = ops.window_blocks(window, P, width)
    copies = _copies(B * width * 64, r2t_host.nbytes, 16)
    r2ts = [torch.from_numpy(r2t_host).to(dev) for _ in range(copies)]
    rows_d, lens_d = torch.from_numpy(rows).to(dev), torch.from_numpy(lens).to(dev)
    lens32 = torch.empty(B, dtype=torch.int32, device=dev)
    tables = [ops.block_table(r, rows_d, lens_d, P, width, seq_lens_i32=lens32) for r in r2ts]
    log(f"meta: B={B} page={P} width={width} window={window} ({nb} blocks), req_to_token {nrows}x{ctx} x {copies}")

    def device_us(fn):
        """Device time per launch of fn's kernels: a few eager calls, then steps_n calls captured in one HIP graph and
        replayed (one event pair around the replay), so the host's launch rate (Python, ctypes, ~10 µs a call) does
        not count: these kernels take a few µs."""
        time_us(fn, min(warmup, 5), 0)
        return time_us_graph(fn, steps_n)

    def both(i):
        ops.window_table(ops.block_table(r2ts[i % copies], rows_d, lens_d, P, width, seq_lens_i32=lens32), lens_d, P,
                         nb)

    torch.cuda.synchronize()
    with torch.cuda.stream(torch.cuda.Stream()):  # a side stream: a graph captures it
        bt_us = device_us(lambda i: ops.block_table(r2ts[i % copies], rows_d, lens_d, P, width, seq_lens_i32=lens32))
        wt_us = device_us(lambda i: ops.window_table(tables[i % copies], lens_d, P, nb))
        step_us = device_us(both)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for i in range(steps_n):
        both(i)
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t) / steps_n * 1e6
    bt_bytes = B * width * 8 + B * 16
    achieved = bt_bytes / (bt_us * 1e-6) / 1e9
    log(f"block_table {bt_us:.2f} us ({achieved:.0f} GB/s algorithmic), window_table {wt_us:.2f} us, both back to back "
        f"{step_us:.2f} us; {host_us:.2f} us per build by the host clock (Python + launches)")
    line = {
        "metric": META_METRIC, "value": round(step_us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps_n,
        "warmup": warmup, "ms_per_step": round(step_us * 1e-3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "int32", "data": "synthetic: random slots (numpy seed 7), U[1, 8192] lengths",
        "config": {"workload": "meta: decode metadata of a 256-row batch", "batch": B, "page_size": P,
                   "table_width": width, "window": window, "window_blocks": nb, "req_to_token": [nrows, ctx],
                   "copies": copies},
        "block_table_us": round(bt_us, 3), "window_table_us": round(wt_us, 3), "host_clock_us_per_build": round(host_us, 3),
        "roofline": {"bound": "hbm", "kernel": "block_table_kernel", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": _traffic("meta")[0], "traffic_source": _traffic("meta")[1], "alg_bytes_per_launch": bt_bytes, "avg_launch_us": round(bt_us, 3)},
        "cpu_baseline": None,
    }
    if cpu:
        from oracle import metadata as omd

        lens_t = torch.from_numpy(lens)

        def run():
            tb = omd.block_table(r2t_host, rows, lens, P)
            omd.swa_trimmed_table(tb, lens_t, window, P, nb)

        line["cpu_baseline"] = {"value": cpu_median_s(run) * 1e6, "unit": "us/step",
                                "cores": torch.get_num_threads(), "kind": "port",
                                "sample": "the whole batch (2 warm-ups, median of 5 runs): numpy block table + torch window trim, "
                                          "as the reference's host builders", "cpu": cpu_model()}
        log(f"CPU baseline: {line['cpu_baseline']['value']:.0f} us/step")
    return line


INDEXER_METRIC = "DSA indexer µs/step (scores of every cached key + top-k), FP8 index keys, 1 MI355X"


QKV_METRIC = "QKV writer µs/step (QK RMSNorm + RoPE + FP8 K/V store of a prefill chunk), 1 MI355X"


def run_qkv(steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev) -> dict:
    """The writer after the QKV projection for a Qwen3-8B-shaped prefill chunk: 8192 tokens (4 x 2048), 32 query and
    8 KV heads of 128, QK RMSNorm, RoPE, K/V stored into an FP8 pool (page 16, per-KV-head scales) at permuted slots.
    The projection output is rotated over copies past the Infinity Cache. The roofline figure is the kernel's
    algorithmic bytes (qkv, cos/sin, slots and gammas read; Q and the FP8 K/V written) over its time; it is HBM-bound.
    Its time comes from torch events on the stream the kernel launches on (torch's current stream)."""
    import torch

    from sglang_neuron_amd import ops

    T, Hq, Hkv, d, P = 8192, 32, 8, 128, 16
    g = torch.Generator().manual_seed(1400)
    width = (Hq + 2 * Hkv) * d
    qkv_host = (torch.randn(T, width, generator=g) * 2.0).to(torch.bfloat16)
    pos = torch.arange(T, dtype=torch.float64)[:, None] % 2048
    inv = 1.0 / (1.0e6 ** (torch.arange(d // 2, dtype=torch.float64) * 2 / d))
    ang = torch.cat([pos * inv, pos * inv], dim=-1)
    cos, sin = ang.cos().to(torch.bfloat16).to(dev), ang.sin().to(torch.bfloat16).to(dev)
    nb = T // P + 1
    slots = (torch.randperm(T, generator=g) + P).to(dev)
    qn = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev)
    kn = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(dev)
    ks = ((0.5 + torch.rand(Hkv, generator=g)) * 0.02).to(dev)
    vs = ((0.5 + torch.rand(Hkv, generator=g)) * 0.02).to(dev)
    kc = torch.zeros(nb, Hkv, P, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(T, Hq, d, dtype=torch.bfloat16, device=dev)
    alg = T * width * 2 + 2 * T * d * 2 + T * 8 + 2 * d * 2 + T * Hq * d * 2 + 2 * T * Hkv * d
    n = _copies(alg, qkv_host.numel() * 2, 16)
    inputs = [qkv_host.to(dev) for _ in range(n)]
    log(f"qkv: T={T} Hq={Hq} Hkv={Hkv} d={d} FP8 pool page {P}, {alg / 1e6:.1f} MB per step, {n} input copies")

    def step(i):
        ops.qkv_norm_rope_store(inputs[i % n], cos=cos, sin=sin, num_q_heads=Hq, num_kv_heads=Hkv, d_head=d,
                                k_cache=kc, v_cache=vc, slot_mapping=slots, q_norm=qn, k_norm=kn, norm_eps=1e-6,
                                k_scale=ks, v_scale=vs, q_out=q_out)

    us = time_us(step, steps_n, warmup)
    achieved = alg / (us * 1e-6) / 1e9
    log(f"qkv_norm_rope_store: {us:.2f} us/step ({achieved:.0f} GB/s)")
    line = {
        "metric": QKV_METRIC, "value": round(us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps_n,
        "warmup": warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 in, fp8_e4m3fn K/V out",
        "data": "synthetic: seeded N(0,1) projection output (torch.Generator seed 1400), permuted slots",
        "config": {"workload": "qkv: qwen3-8b prefill chunk writer", "tokens": T, "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": d, "page_size": P, "qk_norm": True, "kv_dtype": "fp8_e4m3fn per-KV-head scale",
                   "input_copies": n},
        "roofline": {"bound": "hbm", "kernel": "qkv_norm_rope_store_kernel", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": _traffic("qkv")[0], "traffic_source": _traffic("qkv")[1], "alg_bytes_per_launch": alg, "avg_launch_us": round(us, 3)},
        "cpu_baseline": None,
    }
    if cpu:
        from oracle import qkv as oqkv

        log("CPU baseline (oracle on the host cores)")
        qkv_c, cos_c, sin_c, slots_c = qkv_host, cos.cpu(), sin.cpu(), slots.cpu()
        qn_c, kn_c, ks_c, vs_c = qn.cpu(), kn.cpu(), ks.cpu(), vs.cpu()
        kc_c = torch.zeros(nb, Hkv, P, d, dtype=torch.uint8)
        vc_c = torch.zeros_like(kc_c)

        def run(rows):
            oqkv.qkv_norm_rope_store(qkv_c[:rows], cos_c[:rows], sin_c[:rows], Hq, Hkv, d, kc_c, vc_c, slots_c[:rows],
                                     qn_c, kn_c, 1e-6, ks_c, vs_c)

        line["cpu_baseline"] = _time_rows(run, T, cpu_budget)
        log(f"CPU baseline: {line['cpu_baseline']['value']:.0f} us/step")
    return line


def run_indexer(steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev) -> dict:
    """The DSA indexer's decode step at cfg5's scale: 16 rows, each scoring 131072 cached fp8 index keys (page 64,
    128 dims) with 64 index heads, then the top-2048 positions. The roofline figure is the score kernel's algorithmic
    bytes (128 per key read + 2 per score written) over its time; it is HBM-bound."""
    import torch

    from sglang_neuron_amd import ops

    B, N, H, P, k = 16, 131072, 64, 64, 2048
    g = torch.Generator(device="cpu").manual_seed(1200)
    pages = N // P
    nb = B * pages + 1
    copies = 2
    caches, tables = [], []
    for c in range(copies):
        perm = (torch.randperm(nb - 1, generator=g) + 1).to(torch.int32)
        tables.append(perm.reshape(B, pages).to(dev))
        cache = torch.empty(nb * P, 128, dtype=torch.uint8, device=dev)
        rows = torch.randn(nb * P, 128, generator=g).to(torch.bfloat16).to(dev)
        ops.index_key_store(rows, torch.arange(nb * P, dtype=torch.int64, device=dev), cache)
        caches.append(cache.reshape(nb, P, 128))
        del rows
    q = torch.randn(B, H, 128, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.rand(B, H, generator=g) * H ** -0.5).to(dev)
    limits = torch.full((B,), N, dtype=torch.int32, device=dev)
    scores = torch.empty(B, N, dtype=torch.bfloat16, device=dev)
    log(f"indexer: B={B} keys={N} heads={H} page={P} k={k}, {copies} key caches of {caches[0].numel() / 1e6:.0f} MB")

    def step(i):
        ops.indexer_scores(q, w, caches[i % copies], tables[i % copies], limits, N, out=scores)
        return ops.topk_positions(scores, k)

    step_us = time_us(step, steps_n, warmup)
    times = {"score": time_us(lambda i: ops.indexer_scores(q, w, caches[i % copies], tables[i % copies], limits, N,
                                                           out=scores), steps_n, warmup),
             "topk": time_us(lambda i: ops.topk_positions(scores, k), steps_n, warmup)}
    score_bytes = B * N * (128 + 2)
    achieved = score_bytes / (times["score"] * 1e-6) / 1e9
    log(f"indexer_score_kernel {times['score']:.1f} us ({achieved:.0f} GB/s), topk {times['topk']:.1f} us, "
        f"step {step_us:.1f} us")
    line = {
        "metric": INDEXER_METRIC, "value": round(step_us, 3), "unit": "us/step", "n_gpus": 1, "steps": steps_n,
        "warmup": warmup, "ms_per_step": round(step_us * 1e-3, 6), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8_e4m3fn keys, bf16 scores",
        "data": "synthetic: seeded N(0,1) keys and queries (torch.Generator seed 1200), random page permutation",
        "config": {"workload": "indexer: cfg5-scale DSA indexer, 16 rows x 131072 keys, 64 heads, top-2048",
                   "batch": B, "keys_per_row": N, "index_heads": H, "head_dim": 128, "page_size": P, "topk": k,
                   "key_copies": copies},
        "score_us": round(times["score"], 3), "topk_us": round(times["topk"], 3),
        "roofline": {"bound": "hbm", "kernel": "indexer_score_kernel", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": _traffic("indexer")[0], "traffic_source": _traffic("indexer")[1], "alg_bytes_per_launch": score_bytes,
                     "avg_launch_us": round(times["score"], 3)},
        "cpu_baseline": None,
    }
    if cpu:
        from oracle import indexer as oix

        c0, t0 = caches[0].cpu(), tables[0].cpu()
        qc, wc = q.cpu(), w.cpu()

        def run(n_keys):  # one row, its first n_keys keys, then its top-k
            sc = oix.indexer_scores(qc[:1], wc[:1], c0, t0[:1], torch.tensor([n_keys]), n_keys)
            oix.topk_positions(sc, min(k, n_keys))

        t = time.perf_counter()
        run(4096)
        t1 = time.perf_counter() - t
        n_keys = max(4096, min(N, int(4096 * cpu_budget / 7 / max(t1, 1e-6))))
        med = cpu_median_s(lambda: run(n_keys))
        line["cpu_baseline"] = {"value": round(med * (B * N / n_keys) * 1e6, 1), "unit": "us/step",
                                "cores": torch.get_num_threads(), "kind": "port",
                                "sample": f"row 0's first {n_keys} keys (2 warm-ups, median of 5 runs, scaled "
                                          f"x{B * N / n_keys:.1f}"
                                          " to the step)", "cpu": cpu_model()}
        log(f"CPU baseline: {line['cpu_baseline']['value']:.0f} us/step")
    return line


WIRE_METRIC = "PD page-item transfer GB/s (one request's KV pages moved pool to pool), Qwen3-8B FP8 pool, 1 MI355X"


def run_wire(steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev) -> dict:
    """One request's KV pages moved between two pools, the transfer's WRITE list on one GPU (ops.copy_page_items over
    get_contiguous_buf_infos): Qwen3-8B's FP8 pool (36 layers x K and V = 72 regions, items of 8 heads x 16 tokens x
    128 dims = 16 KB), a 4096-token request (256 pages, 302 MB). Four page sets rotate over pools of 2048 pages, so
    each step moves pages no earlier step touched. Pack (into a wire buffer) and unpack (out of it) are timed beside
    it. HBM-bound: every byte moved is read once and written once."""
    import torch

    from sglang_neuron_amd import ops
    from sglang_neuron_amd.mem_cache.memory_pool import NeuronMHATokenToKVPool

    layers, G, d, P, n_pages, pool_pages, sets = 36, 8, 128, 16, 256, 2048, 4
    pools = [NeuronMHATokenToKVPool(pool_pages * P, P, torch.float8_e4m3fn, G, d, layers, dev) for _ in range(2)]
    g = torch.Generator(device=dev).manual_seed(1300)
    for pool in pools:
        for t in pool.k_buffer + pool.v_buffer:
            t.view(torch.uint8).random_(0, 256, generator=g)  # in place: no copy dispatch beside the calibration's
    src_inf, dst_inf = pools[0].get_contiguous_buf_infos(), pools[1].get_contiguous_buf_infos()
    gc = torch.Generator().manual_seed(1301)
    src_sets = [(torch.randperm(pool_pages, generator=gc)[:n_pages] + 1).to(torch.int32).to(dev) for _ in range(sets)]
    dst_sets = [(torch.randperm(pool_pages, generator=gc)[:n_pages] + 1).to(torch.int32).to(dev) for _ in range(sets)]
    moved = ops.page_items_wire_bytes(src_inf, n_pages)
    wire = torch.empty(moved, dtype=torch.uint8, device=dev)
    log(f"wire: {len(src_inf[0])} regions, items of {src_inf[2][0]} B, {n_pages} pages per step: {moved / 1e6:.0f} MB")

    def step(i):
        ops.copy_page_items(src_inf, dst_inf, src_sets[i % sets], dst_sets[i % sets])

    step_us = time_us(step, steps_n, warmup)
    times = {"copy": step_us,
             "pack": time_us(lambda i: ops.pack_page_items(src_inf, src_sets[i % sets], wire), steps_n, warmup),
             "unpack": time_us(lambda i: ops.unpack_page_items(wire, dst_inf, dst_sets[i % sets]), steps_n, warmup)}
    # a plain device copy of as many bytes, for the practical ceiling
    flat = torch.empty(moved, dtype=torch.uint8, device=dev)
    dcopy_us = time_us(lambda i: flat.copy_(wire), 20, 3)
    del flat
    hbm = 2 * moved
    achieved = hbm / (times["copy"] * 1e-6) / 1e9
    log(f"page_items_kernel copy {times['copy']:.1f} us ({achieved:.0f} GB/s of HBM traffic), pack "
        f"{times['pack']:.1f} us, unpack {times['unpack']:.1f} us; step {step_us:.1f} us; a contiguous device copy "
        f"of as many bytes (torch copy_) {dcopy_us:.1f} us ({hbm / (dcopy_us * 1e-6) / 1e9:.0f} GB/s)")
    line = {
        "metric": WIRE_METRIC, "value": round(moved / (step_us * 1e-6) / 1e9, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps_n, "warmup": warmup, "ms_per_step": round(step_us * 1e-3, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u8 (fp8_e4m3fn pages)",
        "data": "synthetic: seeded random pool bytes (torch.Generator seed 1300), random page sets (seed 1301)",
        "config": {"workload": "wire: one 4096-token request of a Qwen3-8B FP8 pool (36 layers, K and V) moved "
                               "between two pools", "regions": len(src_inf[0]), "item_bytes": src_inf[2][0],
                   "pages": n_pages, "pool_pages": pool_pages, "page_sets": sets},
        "copy_us": round(times["copy"], 3), "pack_us": round(times["pack"], 3), "unpack_us": round(times["unpack"], 3),
        "device_copy_us": round(dcopy_us, 3),
        "roofline": {"bound": "hbm", "kernel": "page_items_kernel", "achieved": round(achieved, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": _traffic("wire")[0], "traffic_source": _traffic("wire")[1], "alg_bytes_per_launch": hbm,
                     "avg_launch_us": round(times["copy"], 3)},
        "cpu_baseline": None,
    }
    if cpu:
        from oracle import page_items as opi

        n_reg = 8  # a sample: 4 layers' K and V, every page of the request
        il = src_inf[2][0]
        src_host = [pools[0].k_buffer[j // 2].view(torch.uint8).reshape(-1).cpu() if j % 2 == 0 else
                    pools[0].v_buffer[j // 2].view(torch.uint8).reshape(-1).cpu() for j in range(n_reg)]
        dst_host = [torch.empty_like(t) for t in src_host]
        sp, dp = src_sets[0].tolist(), dst_sets[0].tolist()
        med = cpu_median_s(lambda: opi.copy(src_host, dst_host, [il] * n_reg, sp, dp))
        line["cpu_baseline"] = {"value": round(n_reg * n_pages * il / med / 1e9, 2), "unit": "GB/s", "cores": 1,
                                "kind": "port", "sample": f"{n_reg} of the {len(src_inf[0])} regions, every page of "
                                                          "the request (2 warm-ups, median of 5 runs; a scalar loop)",
                                "cpu": cpu_model()}
        log(f"CPU baseline: {line['cpu_baseline']['value']:.2f} GB/s")
    return line


PREFILL_METRIC = "prefill attention TFLOP/s over the FP8 pool (segmented, causal), 1 MI355X"


def run_prefill(steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev) -> dict:
    """Segmented prefill attention (ops.prefill_attention) on Qwen3-8B's shape: 4 requests, each a 2048-token chunk
    after a 2048-token prior, H 32 / G 8 / d 128, FP8 pool (page 16) written by the store kernel. The algorithmic work
    is 4 d flops per (query, head, visible key) (QK and PV); MFMA-bound, so the roofline is TFLOP/s against the bf16
    dense peak."""
    import torch

    from sglang_neuron_amd import ops

    R, S, prior, H, G, d, P = 4, 2048, 2048, 32, 8, 128, 16
    g = torch.Generator(device="cpu").manual_seed(1100)
    span = prior + S
    pages = span // P
    nb = R * pages + 1
    table = (torch.randperm(nb - 1, generator=g) + 1).to(torch.int32).reshape(R, pages)
    kc = torch.empty(nb, G, P, d, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.full((G,), 4.0 / 448, device=dev)
    vs = torch.full((G,), 4.0 / 448, device=dev)
    for r in range(R):
        k = torch.randn(span, G, d, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(span, G, d, generator=g).to(torch.bfloat16).to(dev)
        slots = table[r, torch.arange(span) // P].to(torch.int64) * P + torch.arange(span) % P
        ops.kv_store_mha(k, v, slots.to(dev), kc, vc, ks, vs)
    q = torch.randn(R * S, H, d, generator=g).to(torch.bfloat16).to(dev)
    q_start = torch.arange(0, R * S + 1, S, dtype=torch.int32, device=dev)
    priors = torch.full((R,), prior, dtype=torch.int32, device=dev)
    table_d = table.to(dev)
    out = torch.empty_like(q)
    scale = d ** -0.5
    flops = 4 * d * H * R * sum(prior + i + 1 for i in range(S))
    log(f"prefill: R={R} chunk={S} prior={prior} H={H} G={G} d={d} page={P}, {flops / 1e12:.2f} TFLOP per step")

    def step():
        ops.prefill_attention(q, kc, vc, table_d, q_start, priors, max_q_len=S, sm_scale=scale, k_scale=ks,
                              v_scale=vs, out=out)

    step_ms = time_us(lambda i: step(), steps_n, warmup) * 1e-3
    kernel_ms = step_ms  # the step is the one prefill kernel
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    log(f"prefill_gqa_kernel {kernel_ms * 1e3:.1f} us/step ({tflops:.0f} TFLOP/s)")
    line = {
        "metric": PREFILL_METRIC, "value": round(flops / (step_ms * 1e-3) / 1e12, 1), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": steps_n, "warmup": warmup, "ms_per_step": round(step_ms, 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 MFMA over fp8_e4m3fn K/V",
        "data": "synthetic: seeded N(0,1) K/V/Q (torch.Generator seed 1100), random page permutation",
        "config": {"workload": "prefill: qwen3-8b-gqa-fp8, 4 x (2048-token chunk after a 2048-token prior)",
                   "requests": R, "chunk": S, "prior": prior, "q_heads": H, "kv_heads": G, "head_dim": d,
                   "page_size": P, "kv_dtype": "fp8_e4m3fn per-KV-head scale"},
        "roofline": {"bound": "mfma", "kernel": "prefill_gqa_kernel", "achieved": round(tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": _traffic("prefill")[0], "traffic_source": _traffic("prefill")[1], "alg_flops_per_launch": flops,
                     "avg_launch_us": round(kernel_ms * 1e3, 3)},
        "cpu_baseline": None,
    }
    if cpu:
        from oracle import attention as oatt

        kc8, vc8 = kc.cpu().view(torch.uint8), vc.cpu().view(torch.uint8)
        qs, tb = q.cpu(), table.cpu()
        ksc, vsc = ks.cpu(), vs.cpu()

        def run(nq):  # the first nq queries of request 0
            oatt.segmented_prefill(qs[:nq], kc8, vc8, tb[:1], torch.tensor([0, nq]), torch.tensor([prior]),
                                   sm_scale=scale, k_scale=ksc, v_scale=vsc)

        t = time.perf_counter()
        run(16)
        t16 = time.perf_counter() - t
        nq = max(16, min(S, int(16 * cpu_budget / 7 / max(t16, 1e-6))))
        med = cpu_median_s(lambda: run(nq))
        sample_flops = 4 * d * H * sum(prior + i + 1 for i in range(nq))
        line["cpu_baseline"] = {"value": round(sample_flops / med / 1e12, 4), "unit": "TFLOP/s",
                                "cores": torch.get_num_threads(), "kind": "port",
                                "sample": f"the first {nq} queries of request 0 (2 warm-ups, median of 5 runs, "
                                          f"{sample_flops / 1e9:.0f} GFLOP)", "cpu": cpu_model(),
                                "us_per_step_scaled": round(med * flops / sample_flops * 1e6, 1)}
        log(f"CPU baseline: {line['cpu_baseline']['value']} TFLOP/s")
    return line


DECODE_CONFIGS = ("2", "1", "3", "4", "4swa", "5", "3bf16", "5mtp")


def setup(key: str, dev):
    if key in ("1", "2", "4"):
        return setup_gqa(int(key), 0, dev)
    if key == "4swa":
        from sglang_neuron_amd import workloads

        return setup_gqa(4, workloads.SWA_WINDOW, dev)
    if key in ("3", "3bf16"):
        return setup_mla(dev, key == "3bf16")
    if key == "5":
        return setup_dsa(dev)
    if key == "5mtp":
        from sglang_neuron_amd import workloads

        return setup_dsa(dev, workloads.DSA_MTP_SPEC)
    raise SystemExit(f"unknown config {key}")


def measure_decode(key: str, steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev,
                   graph_only: bool = False) -> dict:
    """One decode config: its step time, the roofline of the step's kernels, and (cpu) the CPU baseline. The step time
    is the steps_n steps captured in one HIP graph and replayed (one event pair around the replay); the same steps
    launched one by one from the host (one event pair around steps_n back-to-back calls, after warmup calls) are
    reported beside it: for the small steps that number is the host's launch rate, not the GPU's. ``graph_only``
    (a profiling run): the graph replays alone, so a kernel trace of the run holds the step's kernels from the two
    replays only (no launches one by one, no halves apart, no bound-plan leg). The pools are freed before
    returning."""
    import torch

    stream = torch.cuda.Stream()  # a side stream: the steps are bound to it, and a graph captures it
    with torch.cuda.stream(stream):
        steps, desc, step_bytes, kernels, mfma_flops, cpu_fn, legs = setup(key, dev)
        n = len(steps)
        us_eager, wall = None, 0.0
        if not graph_only:
            wall = time.perf_counter()
            us_eager = time_us(lambda i: steps[i % n](), steps_n, warmup)
            wall = time.perf_counter() - wall
        us = time_us_graph(lambda i: steps[i % n](), steps_n)
        # the step's halves apart, the same way (the decode without its store, and the store kernel alone)
        apart = {}
        for leg, fns in ({} if graph_only else legs).items():
            time_us(lambda i: fns[i % n](), min(warmup, 5), 0)
            apart[f"{leg}_us"] = round(time_us_graph(lambda i: fns[i % n](), steps_n), 3)
    gbs = step_bytes / (us * 1e-6) / 1e9
    wl = desc["workload"].split(":")[0]
    traffic, traffic_source = _traffic(wl)
    # MFMA work the kernels issue, bf16 and FP8 (a dict when both): total TFLOP/s and the fraction of the pipe's dense
    # peak time they fill (bf16 work over the bf16 peak plus FP8 work over the FP8 peak)
    mf = mfma_flops if isinstance(mfma_flops, dict) else {"bf16": mfma_flops, "fp8": 0}
    mfma_tflops = (mf["bf16"] + mf["fp8"]) / (us * 1e-6) / 1e12
    mfma_frac = (mf["bf16"] / PEAK_BF16_TFLOPS + mf["fp8"] / PEAK_FP8_TFLOPS) / (us * 1e-6) / 1e12
    if graph_only:
        log(f"{wl}: {us:.2f} us/step over {steps_n} steps replayed from a HIP graph ({gbs:.0f} GB/s, "
            f"{gbs / PEAK_HBM_GBS:.1%} of HBM peak); graph replays only; kernels {kernels}")
    else:
        log(f"{wl}: {us:.2f} us/step over {steps_n} steps replayed from a HIP graph ({gbs:.0f} GB/s, "
            f"{gbs / PEAK_HBM_GBS:.1%} of HBM peak); {us_eager:.2f} us/step launched one by one "
            f"({wall * 1e6 / (steps_n + warmup):.1f} us/step by the host clock); kernels {kernels}; apart: store "
            f"{apart['store_us']:.2f} us, decode without it {apart['decode_us']:.2f} us" +
            (f"; the step under a plan from a bound {apart['bound_plan_us']:.2f} us" if "bound_plan_us" in apart else ""))
    out = {
        "config": desc,
        "us_per_step": round(us, 3),
        "us_per_step_launched": None if us_eager is None else round(us_eager, 3),
        "apart": dict(apart, note="the step's store kernel alone and its decode without the fused store, each replayed "
                                  "from a HIP graph of the same steps; us_per_step is both together (fused); "
                                  "bound_plan_us: the whole step under a plan from a bound (the block table's width), "
                                  "which locates (GQA) or cuts (MLA) its work from the device's seq_lens, as a serving "
                                  "graph captured once for growing lengths runs it"),
        "step_alg_bytes": step_bytes,
        "roofline": {
            "bound": "hbm",
            "kernels": kernels,
            "scope": "the whole step (its kernels back to back)" if len(kernels) > 1 else "the step's one kernel",
            "achieved": round(gbs, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "alg_bytes_per_step": step_bytes,
            "us_per_step": round(us, 3),
            "timing": f"one HIP event pair (torch events, the launch stream) around one replay of a HIP graph of "
                      f"{steps_n} steps; us_per_step_launched: the same steps launched one by one from the host",
        },
        "mfma": {"alg_tflops": round(mfma_tflops, 2), "frac_of_dense_peak": round(mfma_frac, 4),
                 "fp8_share": round(mf["fp8"] / max(mf["bf16"] + mf["fp8"], 1), 4),
                 "source": "algorithmic: MFMA instructions the kernel issues (16x16 key tiles x shapes) / step time, "
                           "not a hardware counter"},
        "cpu_baseline": None,
    }
    mc = _mfma_counters(wl)
    if mc:
        out["mfma"]["counter_busy_pct"] = mc["mfma_busy_pct"]
        out["mfma"]["counter_flops_per_step"] = mc["mfma_flops_per_step"]
        if "mfma_f8_flops_per_step" in mc:
            out["mfma"]["counter_f8_flops_per_step"] = mc["mfma_f8_flops_per_step"]
        out["mfma"]["counter_source"] = (f"committed rocprofv3 pass of MfmaUtil, MfmaFlopsBF16 and "
                                         f"SQ_INSTS_VALU_MFMA_MOPS_F8 (profiles/mfma_{wl}.json), not this run")
    if cpu:
        log(f"{wl}: CPU baseline (oracle on {cpu_threads()} host threads)")
        cb = cpu_fn(cpu_budget)
        cb["alg_gbs"] = round(step_bytes / (cb["value"] * 1e-6) / 1e9, 3)
        out["cpu_baseline"] = cb
        log(f"{wl}: CPU baseline {cb['value']:.0f} us/step on {cb['cores']} threads")
    del steps
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def run_one(key: str, steps_n: int, warmup: int, cpu: bool, cpu_budget: float, dev, per_config=(),
            graph_only: bool = False) -> dict:
    m = measure_decode(key, steps_n, warmup, cpu, cpu_budget, dev, graph_only)
    us = m["us_per_step"]
    desc = m.pop("config")
    line = {
        "metric": METRIC,
        "value": m["roofline"]["achieved"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_n,
        "warmup": warmup,
        "ms_per_step": round(us * 1e-3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn" if "fp8" in desc.get("kv_dtype", "") else "bf16",
        "data": "synthetic: seeded N(0,1) values (torch.Generator seed 1000+cfg), random page permutation",
        "config": desc,
        **m,
    }
    if per_config:
        line["per_config"] = {}
        for k in per_config:
            pm = measure_decode(k, steps_n, warmup, cpu, cpu_budget * 2 / 3, dev, graph_only)
            name = "cfg" + k.replace("swa", "-swa128").replace("bf16", "-bf16").replace("mtp", "-mtp8")
            pm["workload"] = pm["config"]["workload"]
            line["per_config"][name] = pm
    return line


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="2",
                    help="1, 2, 3, 4, 4swa, 5, 5mtp or 3bf16 (default 2, the metric's workload); meta: the device-side metadata; "
                         "prefill: the segmented prefill attention; indexer: the DSA indexer; wire: the PD page-item "
                         "transfer")
    ap.add_argument("--all", action="store_true", help="one line per workload")
    ap.add_argument("--no-per-config", action="store_true",
                    help="the cfg2 line without the other decode configs under per_config")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU work for the baseline sample")
    ap.add_argument("--graph-only", action="store_true",
                    help="decode configs: time the graph replays alone (a profiling run: no launches one by one, no "
                         "halves apart), so a kernel trace holds the step's kernels from the replays only")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one plain device copy of 1 GiB (the reference dispatch for HBM counter scaling)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this build runs no collectives (asked for {max(args.gpus, world)} GPUs). "
              "The single-GPU number is the per-GPU share (GQA would shard by KV head, MLA and DSA by context).", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.empty(COPY_CALIBRATION_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"copy calibration: one copy of {COPY_CALIBRATION_BYTES} bytes (read) into as many (written)")
    keys = ["1", "2", "3", "4", "4swa", "5", "3bf16", "meta", "prefill", "indexer", "wire", "qkv"] if args.all \
        else [args.config]
    for k in keys:
        if k == "meta":
            line = run_meta(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev)
        elif k == "prefill":
            line = run_prefill(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev)
        elif k == "indexer":
            line = run_indexer(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev)
        elif k == "wire":
            line = run_wire(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev)
        elif k == "qkv":
            line = run_qkv(args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev)
        else:
            extra = () if (args.all or args.no_per_config or k != "2") else DECODE_CONFIGS[1:]
            line = run_one(k, args.steps, args.warmup, not args.no_cpu_baseline, args.cpu_budget, dev, extra,
                           args.graph_only)
        print(json.dumps(line), flush=True)
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
