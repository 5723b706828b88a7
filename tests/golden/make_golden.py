"""Regenerate the committed fixtures under tests/golden/.

* ``small_<kind>.npz``: a small seeded case per path (inputs as the kernel receives them,
  plus the oracle's expected output) -- GPU tests run the kernels on exactly these bytes.
* ``workload_sha256.json``: SHA-256 of the operand bytes of every full-size workload, so a
  machine whose torch RNG or quantizer drifted is caught before parity is judged.

The reference ships no golden vectors for this path (its GEMM tests draw unseeded
``torch.rand``), so the expected outputs come from the oracle, whose own pins live in
``tests/test_oracle.py``.

Usage: python tests/golden/make_golden.py [--hashes]
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from flydsl_amd import workloads  # noqa: E402
from oracle import gemm as og  # noqa: E402

SMALL = {
    "fp8": workloads.custom("fp8", 20, 64, 256, seed=100),
    "int8": workloads.custom("int8", 20, 64, 256, seed=101),
    "int4": workloads.custom("int4", 20, 64, 256, seed=102, b_std=0.02),
    "fp8_block": workloads.custom("fp8_block", 20, 144, 256, seed=103),
}


def expected(ops):
    w = ops["workload"]
    a = ops["a"].view(__import__("torch").int8).numpy() if w.kind != "int8" and w.kind != "int4" else ops["a"].numpy()
    b = ops["b"].view(__import__("torch").int8).numpy() if w.kind in ("fp8", "fp8_block") else ops["b"].numpy()
    if w.kind == "fp8":
        return og.run_torch(a.view(np.uint8), b.view(np.uint8), ops["sa"].numpy(), ops["sb"].numpy(), "fp8", "f64")
    if w.kind == "fp8_block":
        return og.run_torch_blockscale(a.view(np.uint8), b.view(np.uint8), ops["sa"].numpy(), ops["sb"].numpy(), "f64")
    acc = og.acc_int(a, b)
    return acc


def operand_arrays(ops):
    import torch
    w = ops["workload"]
    out = {
        "a": ops["a"].view(torch.uint8).numpy() if ops["a"].dtype != torch.int8 else ops["a"].numpy().view(np.uint8),
        "b_dev": ops["b_dev"].contiguous().view(torch.uint8).numpy().reshape(-1)
        if ops["b_dev"].dtype != torch.int8 else ops["b_dev"].numpy().view(np.uint8).reshape(-1),
        "sa": (ops["sa_t"] if w.kind == "fp8_block" else ops["sa"]).numpy().reshape(-1),
        "sb": ops["sb"].numpy().reshape(-1),
    }
    return out


def write_small():
    for name, w in SMALL.items():
        ops = workloads.make_operands(w)
        arrs = operand_arrays(ops)
        exp = expected(ops)
        np.savez(os.path.join(HERE, f"small_{name}.npz"), M=w.M, N=w.N, K=w.K, kind=w.kind, expected=exp, **arrs)
        print("wrote", name, {k: v.shape for k, v in arrs.items()}, exp.dtype)


def workload_hashes():
    res = {}
    for name, w in workloads.WORKLOADS.items():
        ops = workloads.make_operands(w)
        arrs = operand_arrays(ops)
        res[name] = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() for k, v in arrs.items()}
        print(name, res[name]["b_dev"][:16], flush=True)
        del ops, arrs
    with open(os.path.join(HERE, "workload_sha256.json"), "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    write_small()
    if "--hashes" in sys.argv:
        workload_hashes()
