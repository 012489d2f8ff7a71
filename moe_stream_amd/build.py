"""Build the gfx950 shared library of the expert hot path in-tree.

    python -m moe_stream_amd.build

writes moe_stream_amd/lib/libmoe_stream.so with hipcc.  The library links the
HIP runtime by soname (libamdhip64.so.7); loaded after `import torch` it binds
to the runtime torch already holds, so one HIP runtime is in the process.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libmoe_stream.so"
ARCH = os.environ.get("MOE_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed fp32 instructions anywhere in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs (no accumulator-register copies).
    # Under this flag the compiler can hand an MFMA's accumulator-input
    # registers to a VALU result a few instructions after the MFMA issues,
    # before the MFMA has read them (chained MFMAs whose destination differs
    # from their accumulator input).  grouped.hip keeps each chain's first
    # result alive with an empty asm use until the fold has read the chain's
    # output; the ragged-tile cases of tests/test_gpu_grouped.py returned
    # wrong outputs without it.  Changing this flag or the compiler calls for
    # those tests and a scan of the built assembly for such a write.
    "-Xarch_device", "-mllvm=-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def build(verbose: bool = True) -> Path:
    LIBDIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(PKG.parent / "include"),
           str(CSRC / "libmoe_stream.hip"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
