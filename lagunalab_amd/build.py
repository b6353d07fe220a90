"""Builds liblaguna_hip.so in-tree with hipcc for gfx950 (MI355X).

    python -m lagunalab_amd.build          # or __graft_entry__.build()

One shared library from every ``csrc/*.hip`` (one object per source, compiled in parallel, then
linked); C ABI in ``include/laguna_hip.h``. No rpath is
embedded: at run time the library binds to the HIP runtime that PyTorch has already loaded
(same soname, ``libamdhip64.so.7``), so one HIP runtime serves the process.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "liblaguna_hip.so"
OBJ = PKG / "_build"  # one object per source (kept out of git and off the GPU box)
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # never emit packed fp32 VALU ops (v_pk_fma_f32 and friends)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the attention loops rescale their output accumulators on the
    # VALU, which with AGPR accumulators costs a copy of every accumulator per key tile
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


# Per-source extra flags. layer.hip: the decode-step kernels take plain pointer and scalar
# arguments, and gfx950's dispatch preloads the leading ones (up to 14 dwords: a GEMV's five
# pointers and N, K, eps) into SGPRs, so their first loads wait for no argument round trip.
EXTRA_FLAGS = {"layer.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=8"]}


def sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(hipcc, src, obj):
    cmd = [hipcc, *FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", "-o", str(obj), str(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    return cmd, r


def build(verbose: bool = False, incremental: bool = False) -> Path:
    """Compiles every source to an object (in parallel, one hipcc per file) and links the
    library. ``incremental`` recompiles only sources whose object is older than the source or
    than any header in ``csrc/``."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    newest_hdr = max((h.stat().st_mtime for h in CSRC.glob("*.h")), default=0.0)
    todo = []
    for src in srcs:
        obj = OBJ / (src.stem + ".o")
        if (not incremental or not obj.exists()
                or obj.stat().st_mtime < max(src.stat().st_mtime, newest_hdr)):
            todo.append((src, obj))
    noise = "is not a recognized feature for this target"
    jobs = min(len(todo), os.cpu_count() or 1, 16) or 1
    with ThreadPoolExecutor(jobs) as ex:
        for cmd, r in ex.map(lambda t: _compile(hipcc, *t), todo):
            err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
            if verbose:
                print(" ".join(cmd), flush=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
            if verbose and err.strip():
                print(err, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *(str(OBJ / (s.stem + ".o")) for s in srcs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed ({r.returncode}):\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
