"""ctypes binding of libsglang_neuron_amd.so (the C ABI declared in include/sglang_neuron_amd.h).

torch is imported first on purpose: the library links libamdhip64.so.7, and with torch's copy of that runtime already
loaded under the same soname, the dynamic loader binds the library to it, so torch's streams and allocations are valid
in the library's calls. There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (see the module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libsglang_neuron_amd.so"

SNA_OK = 0
SNA_ERR_INVALID_ARGUMENT = -1
SNA_ERR_WORKSPACE = -2
SNA_ERR_LAUNCH = -3
SNA_ERR_UNSUPPORTED = -4

NOALLOC_SCRATCH_BYTES = 16 << 20  # SNA_NOALLOC_SCRATCH_BYTES

DTYPE_BF16 = 0
DTYPE_FP8_E4M3FN = 1
DTYPE_FP8_E4M3FN_MUL = 2  # FP8 bytes; the scales are the GPT-OSS quantization multipliers (SNA_DTYPE_FP8_E4M3FN_MUL)

MAX_CTAS = 256       # SNA_MAX_CTAS
MAX_PLAN_ROWS = 256  # SNA_MAX_PLAN_ROWS
STREAM_MAX_COUNTERS = 2047  # (row, head group) merge counters of one MLA / DSA launch
WS_DIRTY_ARRIVAL = 1  # SNA_WS_DIRTY_ARRIVAL: a launch found a row's arrival count past its workgroups
WS_DIRTY_DONE = 2     # SNA_WS_DIRTY_DONE: a launch found the finished-workgroups count past its grid
SPARSE_MAX_RANGE_KEYS = 2048  # indices one DSA workgroup resolves

KIND_GQA = 0
KIND_MLA = 1
KIND_DSA = 2


class SplitPlan(ctypes.Structure):
    """sna_split_plan."""

    _fields_ = [("split_tiles", ctypes.c_int32), ("n_work", ctypes.c_int32), ("tile", ctypes.c_int32),
                ("target_ctas", ctypes.c_int32), ("max_splits", ctypes.c_int32), ("batch", ctypes.c_int32),
                ("empty_rows", ctypes.c_int32), ("depth", ctypes.c_int32), ("work_n", ctypes.c_int32),
                ("work", ctypes.c_uint32 * 512), ("n_ctas", ctypes.c_int32), ("total_tiles", ctypes.c_int32),
                ("wait_polls", ctypes.c_int32), ("cta_start", ctypes.c_uint32 * (MAX_CTAS + 1)),
                ("cta_row", ctypes.c_uint16 * MAX_CTAS), ("cta_off", ctypes.c_uint16 * MAX_CTAS),
                ("row_keys", ctypes.c_int32 * MAX_PLAN_ROWS), ("device_split", ctypes.c_int32)]

    def __repr__(self) -> str:
        return (f"SplitPlan(split_tiles={self.split_tiles}, n_work={self.n_work}, tile={self.tile}, "
                f"target_ctas={self.target_ctas}, max_splits={self.max_splits}, batch={self.batch}, "
                f"empty_rows={self.empty_rows}, depth={self.depth}, n_ctas={self.n_ctas})")


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

# name -> (restype, argtypes); the exact declarations of include/sglang_neuron_amd.h
SIGNATURES = {
    "sna_version": (_I32, []),
    "sna_last_error": (ctypes.c_char_p, []),
    "sna_kv_store_mha": (_I32, [_P, _P, _P, _I64, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "sna_qkv_norm_rope_store": (_I32, [_P, _I64, _I64, _I32, _I32, _I32, _P, _P, ctypes.c_float, _P, _P, _I64, _P, _P,
                                        _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "sna_absmax_workspace_bytes": (_I64, [_I64, _I32]),
    "sna_kv_absmax_scale": (_I32, [_P, _I64, _I32, _I32, _P, _P, _I64, _P]),
    "sna_kv_store_mla": (_I32, [_P, _P, _I64, _I32, _P, _P, _I64, _I32, _P]),
    "sna_kv_store_dsa": (_I32, [_P, _P, _I64, _F32, _P, _I64, _P]),
    "sna_plan_decode": (_I32, [_I32, _P, _I32, _I32, _I32, _I32, _I32, _I32, ctypes.POINTER(SplitPlan)]),
    "sna_decode_workspace_bytes": (_I64, [ctypes.POINTER(SplitPlan), _I32, _I32]),
    "sna_check_decode_operands": (_I32, [_P, _P, _I64, _I32, _P, _P, _I32, _I32, _I64]),
    "sna_stream_workspace_status": (_I32, [_P, _I64, _P, _P]),
    "sna_stream_workspace_reset": (_I32, [_P, _I64, _P]),
    "sna_paged_decode_gqa": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _I32, _F32, _P, _I32,
                                    _I32, _I32, _I32, _I32, _I64, _I32, ctypes.POINTER(SplitPlan), _P, _I64, _P]),
    "sna_paged_decode_gqa_noalloc": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _I32, _F32, _P,
                                            _I32, _I32, _I32, _I32, _I32, _I64, _I32, ctypes.POINTER(SplitPlan), _P]),
    "sna_mla_decode": (_I32, [_P, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _F32, _P, _I32, _I32, _I32, _I64, _I32,
                              ctypes.POINTER(SplitPlan), _P, _I64, _P]),
    "sna_mla_decode_sparse": (_I32, [_P, _P, _P, _F32, _P, _I32, _P, _I64, _I32, _P, _P, _P, _F32, _P, _P, _I32,
                                     _I32, _I32, _I32, _I64, ctypes.POINTER(SplitPlan), _P, _I64, _P]),
    "sna_lse_combine": (_I32, [_P, _P, _I32, _I64, _I32, _P, _P, _P]),
    "sna_prefill_attention": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I32, _P, _P, _I32, _I32, _P, _F32, _I32, _P,
                                     _I32, _I32, _I32, _I32, _I64, _I32, _P]),
    "sna_index_key_store": (_I32, [_P, _P, _I64, _I32, _P, _I64, _P]),
    "sna_indexer_scores": (_I32, [_P, _P, _P, _P, _I64, _I32, _P, _I32, _I32, _I32, _I32, _I64, _I32, _P, _I64, _P]),
    "sna_page_items_wire_bytes": (_I64, [_P, _I32, _I64]),
    "sna_page_items_pack": (_I32, [_P, _P, _P, _I32, _P, _I64, _P, _I64, _P]),
    "sna_page_items_unpack": (_I32, [_P, _I64, _P, _P, _P, _I32, _P, _I64, _P]),
    "sna_page_items_copy": (_I32, [_P, _P, _P, _P, _P, _I32, _P, _P, _I64, _P]),
    "sna_topk_workspace_bytes": (_I64, [_I32, _I32]),
    "sna_topk_positions": (_I32, [_P, _I64, _I32, _I32, _I32, _P, _I64, _P, _I64, _P]),
    "sna_block_table": (_I32, [_P, _I64, _I64, _I64, _P, _P, _I32, _I32, _I32, _P, _P, _P]),
    "sna_window_table": (_I32, [_P, _I64, _I32, _P, _I32, _I32, _I32, _P, _P, _P]),
    "sna_diag_fp8_to_bf16": (_I32, [_P, _P, _I64, _P]),
}

_lib = None


class SnaError(RuntimeError):
    """A launch the HIP runtime refused."""


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """The loaded library, with every declared symbol typed. Raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built: run `python -m sglang_neuron_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error() -> str:
    msg = load().sna_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Map a status code to the exception the reference raises for the same condition (ValueError for bad inputs,
    RuntimeError for launch failures)."""
    if rc == SNA_OK:
        return
    msg = last_error() or f"{what} failed with status {rc}"
    if rc in (SNA_ERR_INVALID_ARGUMENT, SNA_ERR_WORKSPACE, SNA_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise SnaError(msg)
