"""In-tree build of ``libe4b_amd.so`` for gfx950 with ``hipcc`` (no cmake, no JIT cache).

``python -m experts4bit_qlora_amd._build`` (or ``__graft_entry__.build()``) compiles
``csrc/e4b_amd.hip`` (entry points and the routing / dequant / GEMV / LoRA / training kernels),
and ``csrc/decode_inst.hip`` and ``csrc/gemm_inst.hip`` once per (activation dtype, weight format)
pair, all in parallel, then links them into ``experts4bit_qlora_amd/libe4b_amd.so``. The output is written to a temporary
name and renamed, so a failed build never leaves a half-written library behind.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")
SRC = os.path.join(CSRC, "e4b_amd.hip")
DECODE_SRC = os.path.join(CSRC, "decode_inst.hip")
GEMM_SRC = os.path.join(CSRC, "gemm_inst.hip")
INCLUDE = os.path.join(os.path.dirname(_HERE), "include")
# (E4B_INST_DT, E4B_INST_FMT): bf16/fp16 x NF4/NF4_DQ/MXFP4
DECODE_PAIRS = [(dt, fmt) for dt in (0, 1) for fmt in (0, 1, 2)]
OUT = os.path.join(_HERE, "libe4b_amd.so")
ARCH = os.environ.get("E4B_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
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


def _run_all(cmds):
    procs = [(cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)) for cmd in cmds]
    noise = "is not a recognized feature for this target"
    msgs, failed = [], []
    for cmd, p in procs:
        _, err = p.communicate()
        err = "\n".join(l for l in err.splitlines() if noise not in l)
        if p.returncode != 0:
            failed.append(f"hipcc failed ({p.returncode}):\n{' '.join(cmd)}\n{err}")
        elif err.strip():
            msgs.append(err)
    if failed:
        raise RuntimeError("\n\n".join(failed))
    return msgs


def build(verbose: bool = False) -> str:
    cc = hipcc()
    inc = [f"-I{CSRC}", f"-I{INCLUDE}"]
    with tempfile.TemporaryDirectory(prefix="e4b_build_") as tmpdir:
        objs, cmds = [], []
        obj = os.path.join(tmpdir, "e4b_amd.o")
        cmds.append([cc, *FLAGS, *inc, "-c", "-o", obj, SRC])
        objs.append(obj)
        for dt, fmt in DECODE_PAIRS:
            obj = os.path.join(tmpdir, f"decode_{dt}_{fmt}.o")
            cmds.append([cc, *FLAGS, *inc, f"-DE4B_INST_DT={dt}", f"-DE4B_INST_FMT={fmt}", "-c", "-o", obj,
                         DECODE_SRC])
            objs.append(obj)
            obj = os.path.join(tmpdir, f"gemm_{dt}_{fmt}.o")
            cmds.append([cc, *FLAGS, *inc, f"-DE4B_INST_DT={dt}", f"-DE4B_INST_FMT={fmt}", "-c", "-o", obj,
                         GEMM_SRC])
            objs.append(obj)
        msgs = _run_all(cmds)
        tmp = OUT + ".tmp"
        msgs += _run_all([[cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]])
    if verbose and msgs:
        print("\n".join(msgs), file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
