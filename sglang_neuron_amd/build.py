"""Build recipe of libsglang_neuron_amd.so: hipcc for gfx950, one object per source, then one shared library.

Run as ``python -m sglang_neuron_amd.build`` (or through ``__graft_entry__.build()``). The library lands next to this
file, in the package, where the loader looks for it. No GPU is needed: hipcc cross-compiles for gfx950.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB_NAME = "libsglang_neuron_amd.so"
LIB_PATH = PKG / LIB_NAME
ARCH = "gfx950"

# Packed-FP32 instructions are kept out of the code objects (hipcc's host pass warns that it does not know the
# feature; that is harmless). No fast-math: the FP8 store relies on IEEE-correct fp32 division.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-source additions: MFMA accumulators in VGPRs for the split-K decode kernels. They rescale their accumulators in
# the online softmax; with the accumulators in AGPRs the compiler copies them between the register files around that
# (rare) rescale branch on every tile. The indexer's score products feed VALU work (ReLU, the weighted head sum)
# straight away: in VGPRs they need no read back from AGPRs (16 moves a tile; 57.1 -> 56.6 us on the benchmark).
_MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA_FLAGS = {"decode_mla.hip": _MFMA_VGPR, "decode_gqa.hip": _MFMA_VGPR, "prefill_gqa.hip": _MFMA_VGPR,
               "indexer.hip": _MFMA_VGPR}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
