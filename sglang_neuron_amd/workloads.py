"""Seeded synthetic inputs of the five decode configurations the path is measured on (BASELINE.json ``configs``).

Each builder draws lengths, page permutations and values from ``torch.Generator().manual_seed(1000 + cfg)``, so the
same case can be built on the CPU (to feed the oracle) and on the GPU (to feed the kernels). Values are drawn on
``gen_device`` and the pool is filled through a caller-supplied store function. The HIP store fills it on the GPU,
and a CPU restatement fills it in tests.

Layouts follow the reference: page 0 is reserved and the pool has one more page than it hands out
(mem_cache/memory_pool.py:20-21); block tables are int32 with -1 past a row's pages (attention/backend.py:114-130);
seq_lens count the new token (attention/backend.py:36).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable, Optional

import torch
from torch import Tensor

# ---- configuration table (BASELINE.json configs[0..4]) ----
GQA_CONFIGS = {
    1: dict(name="qwen3-0.6b-gqa-bf16", B=8, H=16, G=8, d=128, P=16, fp8=False, lens=(128, 1024), window=0,
            sinks=False),
    2: dict(name="qwen3-8b-gqa-fp8", B=64, H=32, G=8, d=128, P=16, fp8=True, lens=(4096, 4096), window=0,
            sinks=False),
    4: dict(name="gpt-oss-120b-share-fp8", B=128, H=8, G=1, d=64, P=16, fp8=True, lens=(2048, 8192), window=0,
            sinks=True, scales_multiply=True),
}
# cfg4's FP8 write is the GPT-OSS decode's own: k * k_scale with the bf16 inverted checkpoint scale, rounded to bf16
# before the cast (ops/attention/attention_decode.py:259-260; models/gpt_oss/mxfp4/common.py:481-485). Its
# "checkpoint" scale is the absmax / 448 of the case's tokens. cfg2's per-KV-head scales are this path's extension
# and divide (qkv.py:69-70).
MLA_CONFIG = dict(name="deepseek-v2-lite-mla-fp8", B=32, H=16, P=64, lens=(1024, 16384), latent_scale=0.5,
                  sm_scale=1.0 / math.sqrt(192.0))
DSA_CONFIG = dict(name="glm5-dsa-mla-fp8", B=16, H=16, P=64, pool_positions=131072, n_indices=2048, recent=128,
                  kv_scale=2.0 ** -6, sm_scale=0.0625, short_rows=(1000, 2000), spec=1)
# GLM-5.2's MTP verify decodes 8 query tokens per sequence (the token and 7 drafts; docs/model-recipes/glm52.md)
DSA_MTP_SPEC = 8
SWA_WINDOW = 128  # GPT-OSS sliding layers (models/gpt_oss/config.py)


def gen(cfg: int, device: str | torch.device = "cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(1000 + cfg)
    return g


def _randn_bf16(shape, g: torch.Generator, device, scale: float = 1.0) -> Tensor:
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if scale != 1.0:
        x = x * scale
    return x.to(torch.bfloat16)


def _page_layout(lens: list[int], P: int, g: torch.Generator, extra_pages: int = 0):
    """Block table [B, max_pages] int32 over a random permutation of pages 1..N (page 0 reserved), and the pool's
    page count N + 1."""
    pages_per = [(L + P - 1) // P for L in lens]
    n = sum(pages_per) + extra_pages
    perm = torch.randperm(n, generator=g) + 1
    width = max(pages_per)
    table = torch.full((len(lens), width), -1, dtype=torch.int32)
    off = 0
    for b, k in enumerate(pages_per):
        table[b, :k] = perm[off:off + k].to(torch.int32)
        off += k
    return table, n + 1


def _slots_of(table: Tensor, positions: Tensor, rows: Tensor, P: int) -> Tensor:
    return table[rows, positions // P].to(torch.int64) * P + positions % P


@dataclass
class GqaCase:
    cfg: int
    B: int
    H: int
    G: int
    d: int
    P: int
    fp8: bool
    window: int
    sm_scale: float
    seq_lens: Tensor          # [B] int64 (host)
    block_table: Tensor       # [B, W] int32 (host)
    num_blocks: int
    q: Tensor                 # [B, H, d] bf16
    k_prior: Tensor           # [T, G, d] bf16, the prefill tokens of all rows
    v_prior: Tensor
    prior_slots: Tensor       # [T] int64
    k_new: Tensor             # [B, G, d] bf16
    v_new: Tensor
    new_slots: Tensor         # [B] int64
    sinks: Optional[Tensor]   # [H] fp32
    extra: dict = field(default_factory=dict)
    scales_multiply: bool = False  # FP8 scales are GPT-OSS multipliers (SNA_DTYPE_FP8_E4M3FN_MUL), not divisors

    def to(self, device) -> "GqaCase":
        out = GqaCase(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        for k in ("q", "k_prior", "v_prior", "prior_slots", "k_new", "v_new", "new_slots", "sinks"):
            t = getattr(self, k)
            if t is not None:
                setattr(out, k, t.to(device))
        return out

    def kv_bytes_per_step(self) -> int:
        """Algorithmic HBM bytes of one decode step: prior K+V actually read (with the window), the new token's bf16
        read and cache write, Q, O, table entries and scales."""
        esz = 1 if self.fp8 else 2
        keys = 0
        for L in self.seq_lens.tolist():
            n = L - 1
            if self.window > 0:
                n = min(n, self.window - 1)
            keys += n
        b = keys * self.G * self.d * esz * 2
        b += self.B * self.G * self.d * (2 + esz) * 2       # new K,V: bf16 in + cache write
        b += self.B * self.H * self.d * 2 * 2                # q in, out
        pages = 0
        for L in self.seq_lens.tolist():
            n = L - 1 if self.window <= 0 else min(L - 1, self.window - 1)
            pages += (n + self.P - 1) // self.P
        b += pages * 4 + self.B * 4 * 2                      # table entries read, seq_lens, slots
        if self.fp8:
            b += self.G * 4 * 2
        return int(b)


def gqa_case(cfg: int, *, gen_device="cpu", overrides: Optional[dict] = None) -> GqaCase:
    """The cfg1 / cfg2 / cfg4 GQA case (cfg4 with overrides {'window': 128} for its sliding layer)."""
    spec = dict(GQA_CONFIGS[cfg])
    spec.update(overrides or {})
    B, H, G, d, P = spec["B"], spec["H"], spec["G"], spec["d"], spec["P"]
    g_cpu = gen(cfg)
    lo, hi = spec["lens"]
    lens = torch.randint(lo, hi + 1, (B,), generator=g_cpu) if hi > lo else torch.full((B,), lo)
    if "fixed_lens" in spec:
        lens = torch.as_tensor(spec["fixed_lens"], dtype=torch.int64)
    table, nb = _page_layout(lens.tolist(), P, g_cpu)
    sinks = torch.randn(H, generator=g_cpu) if spec["sinks"] else None
    g = gen(cfg, gen_device)
    q = _randn_bf16((B, H, d), g, gen_device)
    # prior tokens: positions 0 .. L-2 of each row
    rows = torch.cat([torch.full((int(L) - 1,), b, dtype=torch.int64) for b, L in enumerate(lens.tolist())])
    pos = torch.cat([torch.arange(int(L) - 1) for L in lens.tolist()])
    prior_slots = _slots_of(table, pos, rows, P)
    T = prior_slots.numel()
    k_prior = _randn_bf16((T, G, d), g, gen_device)
    v_prior = _randn_bf16((T, G, d), g, gen_device)
    k_new = _randn_bf16((B, G, d), g, gen_device)
    v_new = _randn_bf16((B, G, d), g, gen_device)
    new_slots = _slots_of(table, lens - 1, torch.arange(B), P)
    return GqaCase(cfg=cfg, B=B, H=H, G=G, d=d, P=P, fp8=spec["fp8"], window=spec["window"],
                   sm_scale=1.0 / math.sqrt(d), seq_lens=lens.to(torch.int64), block_table=table, num_blocks=nb,
                   q=q, k_prior=k_prior, v_prior=v_prior, prior_slots=prior_slots, k_new=k_new, v_new=v_new,
                   new_slots=new_slots, sinks=sinks, extra={"name": spec["name"]},
                   scales_multiply=bool(spec["fp8"] and spec.get("scales_multiply", False)))


@dataclass
class MlaCase:
    B: int
    H: int
    P: int
    sm_scale: float
    seq_lens: Tensor       # [B] int64
    block_table: Tensor    # [B, W] int32
    num_blocks: int
    ql_nope: Tensor        # [B, H, 512]
    q_pe: Tensor           # [B, H, 64]
    prior_rows: Tensor     # [T, 576] bf16 [latent | rope]
    prior_slots: Tensor    # [T]
    compact_new: Tensor    # [B, 576]
    new_slots: Tensor      # [B]

    def to(self, device) -> "MlaCase":
        out = MlaCase(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        for k in ("ql_nope", "q_pe", "prior_rows", "prior_slots", "compact_new", "new_slots"):
            setattr(out, k, getattr(self, k).to(device))
        return out

    def kv_bytes_per_step(self, bf16: bool = False) -> int:
        keys = int((self.seq_lens - 1).sum())
        row = 1152 if bf16 else 576 + 4                    # bf16 row, or fp8 row + per-token scale
        b = keys * row
        b += self.B * (576 * 2 + row)                      # own row: bf16 in, row (+ scale) out
        b += self.B * self.H * (512 + 64) * 2 + self.B * self.H * 512 * 2
        pages = int(((self.seq_lens - 1 + self.P - 1) // self.P).sum())
        b += pages * 4 + self.B * 4 * 2
        return int(b)


def mla_case(*, gen_device="cpu", overrides: Optional[dict] = None) -> MlaCase:
    spec = dict(MLA_CONFIG)
    spec.update(overrides or {})
    B, H, P = spec["B"], spec["H"], spec["P"]
    g_cpu = gen(3)
    lo, hi = spec["lens"]
    lens = torch.randint(lo, hi + 1, (B,), generator=g_cpu)
    if "fixed_lens" in spec:
        lens = torch.as_tensor(spec["fixed_lens"], dtype=torch.int64)
    table, nb = _page_layout(lens.tolist(), P, g_cpu)
    g = gen(3, gen_device)
    ql = _randn_bf16((B, H, 512), g, gen_device)
    qpe = _randn_bf16((B, H, 64), g, gen_device)
    rows_idx = torch.cat([torch.full((int(L) - 1,), b, dtype=torch.int64) for b, L in enumerate(lens.tolist())])
    pos = torch.cat([torch.arange(int(L) - 1) for L in lens.tolist()])
    prior_slots = _slots_of(table, pos, rows_idx, P)

    def rows(n):
        lat = _randn_bf16((n, 512), g, gen_device, spec["latent_scale"])
        rope = _randn_bf16((n, 64), g, gen_device)
        return torch.cat([lat, rope], dim=1)

    prior = rows(prior_slots.numel())
    new = rows(B)
    new_slots = _slots_of(table, lens - 1, torch.arange(B), P)
    return MlaCase(B=B, H=H, P=P, sm_scale=spec["sm_scale"], seq_lens=lens.to(torch.int64), block_table=table,
                   num_blocks=nb, ql_nope=ql, q_pe=qpe, prior_rows=prior, prior_slots=prior_slots, compact_new=new,
                   new_slots=new_slots)


@dataclass
class DsaCase:
    B: int                # sequences
    H: int
    P: int
    kv_scale: float
    sm_scale: float
    positions: Tensor     # [B * spec] int32: each query token's position (the last is its sequence's live length - 1)
    block_table: Tensor   # [B, W] int32, one row per sequence
    num_blocks: int
    indices: Tensor       # [B * spec, K] int32, -1 padded
    q_absorbed: Tensor    # [B * spec, H, 512]
    q_pe: Tensor          # [B * spec, H, 64]
    own_rows: Tensor      # [B * spec, 576] [k_pe | latent]
    new_slots: Tensor     # [B * spec]
    pool_positions: int
    spec: int = 1         # query tokens per sequence (sequence s owns tokens s * spec .. s * spec + spec - 1)

    def to(self, device) -> "DsaCase":
        out = DsaCase(**{k: getattr(self, k) for k in self.__dataclass_fields__})
        for k in ("q_absorbed", "q_pe", "own_rows", "new_slots"):
            setattr(out, k, getattr(self, k).to(device))
        return out

    def kv_bytes_per_step(self) -> int:
        T = self.B * self.spec
        valid = int((self.indices >= 0).sum())
        b = valid * (640 + 4)                              # gathered rows + their index
        b += (self.indices < 0).sum().item() * 4
        b += T * (576 * 2 + 640)                            # own rows: bf16 in, packed row out
        b += T * self.H * (512 + 64) * 2 + T * self.H * (512 * 2 + 4)
        b += valid * 4                                      # table entries
        return int(b)

    def fill_rows(self, store: Callable[[Tensor, Tensor], None], gen_device="cpu", chunk: int = 1 << 18) -> None:
        """Fill every prior position of every row (positions < the pool's per-sequence size, except each row's own
        position) through ``store(rows [n, 576] bf16, slots [n])``, in chunks."""
        g = torch.Generator(device=gen_device)
        g.manual_seed(2005)
        B, P = self.B, self.P
        per = self.pool_positions
        for b in range(B):
            for s0 in range(0, per, chunk):
                n = min(chunk, per - s0)
                pos = torch.arange(s0, s0 + n)
                slots = _slots_of(self.block_table, pos, torch.full((n,), b, dtype=torch.int64), P)
                vals = _randn_bf16((n, 576), g, gen_device)
                store(vals, slots.to(gen_device))


def dsa_case(*, gen_device="cpu", overrides: Optional[dict] = None) -> DsaCase:
    """cfg5. Every row's pool holds ``pool_positions`` positions; most rows decode at the pool's last position, and
    the rows named by ``short_rows`` (a builder choice) decode at those shorter lengths, so their index lists are all
    their prior positions padded with -1. Indices: the last ``recent`` prior positions + uniform draws without
    replacement from the rest. With ``spec`` > 1 a sequence decodes spec query tokens at its last spec positions
    (MTP verify); each token draws its own index list over the sequence's prior (the positions before its first
    token)."""
    cfg = dict(DSA_CONFIG)
    cfg.update(overrides or {})
    B, H, P, K, spec = cfg["B"], cfg["H"], cfg["P"], cfg["n_indices"], cfg["spec"]
    per = cfg["pool_positions"]
    g_cpu = gen(5)
    lens = [per] * B
    for i, L in enumerate(cfg["short_rows"]):
        if i < B:
            lens[B - 1 - i] = min(L, per)
    # extra_pages: unused pages mixed into the permutation (a larger pool, e.g. one past 4 GiB)
    table, nb = _page_layout([per] * B, P, g_cpu, cfg.get("extra_pages", 0))
    T = B * spec
    idx = torch.full((T, K), -1, dtype=torch.int32)
    for b, L in enumerate(lens):
        prior = L - spec
        for j in range(spec):
            if prior <= K:
                sel = torch.arange(prior)
            else:
                recent = torch.arange(prior - cfg["recent"], prior)
                rest = torch.randperm(prior - cfg["recent"], generator=g_cpu)[: K - cfg["recent"]]
                sel = torch.cat([recent, torch.sort(rest).values])
            idx[b * spec + j, : sel.numel()] = sel.to(torch.int32)
    g = gen(5, gen_device)
    qa = _randn_bf16((T, H, 512), g, gen_device)
    qpe = _randn_bf16((T, H, 64), g, gen_device)
    own = _randn_bf16((T, 576), g, gen_device)
    positions = torch.tensor([L - spec + j for L in lens for j in range(spec)], dtype=torch.int32)
    new_slots = _slots_of(table, positions.to(torch.int64), torch.arange(T) // spec, P)
    return DsaCase(B=B, H=H, P=P, kv_scale=cfg["kv_scale"], sm_scale=cfg["sm_scale"], positions=positions,
                   block_table=table, num_blocks=nb, indices=idx, q_absorbed=qa, q_pe=qpe, own_rows=own,
                   new_slots=new_slots, pool_positions=per, spec=spec)


# ---- pools on the GPU, filled through the HIP store kernels ----

def gqa_pool(case: GqaCase, device="cuda"):
    """(k_cache, v_cache, k_scale, v_scale) of one layer on ``device``: per-KV-head scales calibrated over every K (V)
    token of the case (prior and new) by the HIP absmax kernel (for a GPT-OSS case, inverted on the host as the
    reference's loader inverts its checkpoint scale), then the prior tokens stored by the HIP store."""
    from . import ops

    dt = torch.float8_e4m3fn if case.fp8 else torch.bfloat16
    kc = torch.zeros(case.num_blocks, case.G, case.P, case.d, dtype=dt, device=device)
    vc = torch.zeros_like(kc)
    ks = vs = None
    kp, vp = case.k_prior.to(device), case.v_prior.to(device)
    if case.fp8:
        ks = ops.kv_absmax_scale(torch.cat([kp, case.k_new.to(device)], dim=0))
        vs = ops.kv_absmax_scale(torch.cat([vp, case.v_new.to(device)], dim=0))
        if case.scales_multiply:
            ks, vs = ops.inverted_kv_scale(ks).to(device), ops.inverted_kv_scale(vs).to(device)
    if kp.shape[0]:
        ops.kv_store_mha(kp, vp, case.prior_slots.to(device), kc, vc, ks, vs, scales_multiply=case.scales_multiply)
    return kc, vc, ks, vs


def mla_pool(case: MlaCase, device="cuda", bf16: bool = False):
    """(rows [slots, 576] uint8, row_scale [slots]) of one layer on ``device``, the prior rows stored by the HIP
    per-token FP8 store; with ``bf16``, (rows [slots, 576] bf16, None) stored as they are."""
    from . import ops

    n = case.num_blocks * case.P
    cache = torch.zeros(n, 576, dtype=torch.bfloat16 if bf16 else torch.uint8, device=device)
    scale = None if bf16 else torch.zeros(n, dtype=torch.float32, device=device)
    if case.prior_slots.numel():
        ops.kv_store_mla(case.prior_rows.to(device), case.prior_slots.to(device), cache, scale)
    return cache, scale


def dsa_pool(case: DsaCase, device="cuda", gen_device="cpu"):
    """The 640-byte row cache of one layer on ``device``, every prior position filled by the HIP DSA store."""
    from . import ops

    cache = torch.zeros(case.num_blocks * case.P, 640, dtype=torch.uint8, device=device)
    case.fill_rows(lambda v, s: ops.kv_store_dsa(v.to(device), s.to(device), cache, case.kv_scale),
                   gen_device=gen_device)
    return cache
