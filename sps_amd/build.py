"""Builds libsps_attn.so (gfx950) in-tree with hipcc.

Every HIP translation unit under ``sps_amd/csrc`` is compiled to an object in ``sps_amd/_build`` and
linked into ``sps_amd/libsps_attn.so``. Run ``python -m sps_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libsps_attn.so"
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Keep the compiler from emitting packed-fp32 VALU ops: some of their forms have given wrong
    # results on this hardware without any error.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA results in VGPRs (gfx950's unified register file): without it the backend routes every
    # accumulator through one AGPR tile with v_accvgpr copies around each MFMA.
    "-mllvm",
    "-amdgpu-mfma-vgpr-form=1",
]

SOURCES = ["attn_prep.hip", "attn_fwd.hip", "attn_bwd.hip", "decode.hip", "kv_update.hip", "rope.hip", "prefill_state.hip", "doc_ids.hip", "capi.cpp"]

# Per-source flags. The attention kernels are scheduled with LLVM's iterative ILP strategy, which
# interleaves their MFMA, exponential and LDS work more densely than the default occupancy-driven
# scheduler at the same register budget (measured on MI355X: C4 (D = 128) fwd+bwd -15 %, C3 (D = 64)
# unchanged).
SOURCE_FLAGS = {
    "attn_fwd.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "attn_bwd.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        futs = {}
        for name in SOURCES:
            src = CSRC / name
            obj = BUILD_DIR / (src.stem + ".o")
            objs.append(obj)
            futs[ex.submit(_compile, hipcc, src, obj)] = name
        for fut in cf.as_completed(futs):
            fut.result()
            if verbose:
                print(f"[sps_amd.build] compiled {futs[fut]}", flush=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[sps_amd.build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
