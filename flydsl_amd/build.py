"""Build the gfx950 HIP library in-tree: ``flydsl_amd/_flygemm.so``.

``python -m flydsl_amd.build`` (or ``__graft_entry__.build()``) always recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SOURCES = [os.path.join(PKG_DIR, "csrc", f) for f in ("flygemm.hip", "moe.hip", "moe_stage2.hip", "moe_stream.hip", "moe_stream2.hip")]
OUT = os.path.join(PKG_DIR, "_flygemm.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed-fp32 VALU instructions (v_pk_*_f32) in device code: some of their forms
    # have produced silently wrong results on MI355X
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the epilogue rounds (acc * sa) * sb to fp32 before the output cast, as the
    # reference does; contraction would fuse the multiply into the cast (one rounding)
    "-ffp-contract=off",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build flydsl_amd")
    return path


# measurement aid for bench.py (shader clock under load), a library of its own so the GEMM
# ABI stays as declared in include/flygemm.h
PROBE_SRC = os.path.join(PKG_DIR, "csrc", "clock_probe.hip")
PROBE_OUT = os.path.join(PKG_DIR, "_clockprobe.so")


def build(verbose: bool = False) -> str:
    """Compile each source to an object in parallel, then link the shared library (and the
    clock probe next to it)."""
    objs, procs = [], []
    probe = [hipcc(), *HIPCC_FLAGS, "-o", PROBE_OUT + ".tmp", PROBE_SRC]
    if verbose:
        print(" ".join(probe), flush=True)
    procs.append((PROBE_SRC, subprocess.Popen(probe, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    for src in SOURCES:
        obj = os.path.splitext(OUT)[0] + "_" + os.path.splitext(os.path.basename(src))[0] + ".o"
        cmd = [hipcc(), *[f for f in HIPCC_FLAGS if f != "-shared"], "-c", "-o", obj, src]
        if verbose:
            print(" ".join(cmd), flush=True)
        objs.append(obj)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    errors = []
    for src, proc in procs:
        _, err = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"hipcc failed on {os.path.basename(src)} ({proc.returncode}):\n{err[-8000:]}")
    if errors:
        raise RuntimeError("\n".join(errors))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, OUT)
    os.replace(PROBE_OUT + ".tmp", PROBE_OUT)
    for obj in objs:
        os.remove(obj)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
