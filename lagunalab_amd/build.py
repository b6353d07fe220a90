"""Builds liblaguna_hip.so in-tree with hipcc for gfx950 (MI355X).

    python -m lagunalab_amd.build          # or __graft_entry__.build()

One shared library from every ``csrc/*.hip``; C ABI in ``include/laguna_hip.h``. No rpath is
embedded: at run time the library binds to the HIP runtime that PyTorch has already loaded
(same soname, ``libamdhip64.so.7``), so one HIP runtime serves the process.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "liblaguna_hip.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # never emit packed fp32 VALU ops (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the attention loops rescale their output accumulators on the
    # VALU, which with AGPR accumulators costs a copy of every accumulator per key tile
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, *FLAGS, "-o", str(tmp), *map(str, sources())]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
