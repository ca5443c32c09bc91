"""In-tree build of ``libe4b_amd.so`` for gfx950 with ``hipcc`` (no cmake, no JIT cache).

``python -m experts4bit_qlora_amd._build`` (or ``__graft_entry__.build()``) compiles
``csrc/e4b_amd.hip`` into ``experts4bit_qlora_amd/libe4b_amd.so``. The output is written to a
temporary name and renamed, so a failed build never leaves a half-written library behind.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(_HERE, "csrc", "e4b_amd.hip")
OUT = os.path.join(_HERE, "libe4b_amd.so")
ARCH = os.environ.get("E4B_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no silent a*b+c contraction: FMAs are written explicitly where they are wanted, and the
    # dequant / combine products must round exactly once
    "-ffp-contract=off",
    # packed fp32 (v_pk_*_f32) is not generated
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False) -> str:
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *FLAGS, "-o", tmp, SRC]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{errs}")
    if verbose and errs.strip():
        print(errs, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
