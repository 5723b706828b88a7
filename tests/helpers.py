"""Shared test plumbing: run the product launchers on workload operands and judge the
result against the oracle (numpy, CPU)."""
from __future__ import annotations

import numpy as np
import torch

from flydsl_amd.kernels.blockscale_preshuffle_gemm import compile_blockscale_preshuffle_gemm
from flydsl_amd.kernels.preshuffle_gemm import accumulators, compile_preshuffle_gemm_a8
from oracle import gemm as og
from oracle import numerics as on

OUT_TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16}


def variant_names() -> list[str]:
    """The library's kernel variant names, for parametrizing GPU tests at collection time; an
    empty list when the library is not built (then those tests collect as skipped, and CPU-only
    runs, which deselect them, still collect)."""
    from flydsl_amd import _lib

    try:
        return _lib.variants()
    except RuntimeError:
        return []


def u8(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous().cpu()
    return t.view(torch.uint8).numpy() if t.dtype != torch.uint8 else t.numpy()


def dev_flat(t: torch.Tensor, device) -> torch.Tensor:
    """Flat device view the launchers take: 1-byte types as int8 (fp8 is passed as int8, as
    in the reference harness), 2-byte types unchanged."""
    t = t.to(device)
    return (t.view(torch.int8) if t.element_size() == 1 else t).view(-1)


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def launch(ops, device, variant=-1, out_dtype="bf16", stream=None, tile_k=None):
    """Run the drop-in launcher for ``ops`` (from ``flydsl_amd.workloads.make_operands``);
    ``tile_k`` defaults to 128 bytes of K."""
    w = ops["workload"]
    M, N, K = w.M, w.N, w.K
    a = dev_flat(ops["a"], device)
    b = dev_flat(ops["b_dev"], device)
    c = torch.empty(M, N, dtype=OUT_TORCH[out_dtype], device=device)
    if w.kind == "fp8_block":
        fn = compile_blockscale_preshuffle_gemm(M=M, N=N, K=K, tile_m=64, tile_n=64, tile_k=128,
                                                out_dtype=out_dtype, variant=variant)
        fn(c.view(-1), a, b, ops["sa_t"].to(device).view(-1), ops["sb"].to(device).view(-1), M, N, stream)
    else:
        tk = tile_k or (64 if w.kind in ("bf16", "fp16") else 128)  # 128 bytes of K either way
        fn = compile_preshuffle_gemm_a8(K=K, tile_m=64, tile_n=128, tile_k=tk, in_dtype=w.kind,
                                        out_dtype=out_dtype, variant=variant)
        fn(c.view(-1), a, b, ops["sa"].to(device).view(-1), ops["sb"].to(device).view(-1), M, N, stream)
    return c


def raw_acc(ops, device, variant=-1):
    w = ops["workload"]
    kind = "fp8" if w.kind == "fp8_block" else w.kind
    acc = torch.empty(w.M, w.N, dtype=torch.int32 if kind in ("int8", "int4") else torch.float32, device=device)
    accumulators(acc, dev_flat(ops["a"], device), dev_flat(ops["b_dev"], device), w.M, w.N, w.K, kind,
                 variant=variant)
    return acc


def reference(ops, rows=None):
    """Oracle output: float64 [M, N] (fp8 paths) or exact int32 accumulators (int paths)."""
    w = ops["workload"]
    if w.kind in ("bf16", "fp16"):
        a = bits16(ops["a"])
        if rows is not None:
            a = a[rows]
        return og.run_torch(a, bits16(ops["b"]), None, None, w.kind, "f64")
    a = u8(ops["a"])
    b = u8(ops["b"])
    if rows is not None:
        a = a[rows]
    if w.kind == "fp8":
        sa = ops["sa"].numpy().reshape(-1)
        return og.run_torch(a, b, sa if rows is None else sa[rows], ops["sb"].numpy().reshape(-1), "fp8", "f64")
    if w.kind == "fp8_block":
        sa = ops["sa"].numpy()
        return og.run_torch_blockscale(a, b, sa if rows is None else sa[rows], ops["sb"].numpy(), "f64")
    return og.acc_int(a.view(np.int8), b.view(np.int8))


def check(ops, out: torch.Tensor, ref=None, rows=None, out_dtype="bf16"):
    """Assert the bar: int paths bit-exact against the oracle epilogue (bf16), fp8 paths
    |out - ref| <= 1e-2 |ref| + 1e-2 RMS(ref)."""
    w = ops["workload"]
    ref = reference(ops, rows) if ref is None else ref
    o = out.float().cpu().numpy()
    if rows is not None:
        o = o[rows]
    if w.kind in ("int8", "int4"):
        sa = ops["sa"].numpy().reshape(-1)
        if rows is not None:
            sa = sa[rows]
        if out_dtype == "bf16":
            exp = on.bf16_to_f32(og.epilogue_int_bf16(ref, sa, ops["sb"].numpy().reshape(-1)))
        else:
            v = (ref.astype(np.float32) * sa[:, None]).astype(np.float32) * ops["sb"].numpy().reshape(1, -1)
            exp = v.astype(np.float32).astype(np.float16).astype(np.float32)
        bad = np.flatnonzero(o.view(np.uint32) != exp.view(np.uint32))
        assert bad.size == 0, f"{w.name}: {bad.size} mismatches, first at {np.unravel_index(bad[0], o.shape)}: " \
                              f"got {o.flat[bad[0]]} want {exp.flat[bad[0]]}"
    else:
        ok, worst = og.within_bar(o, ref)
        assert ok, f"{w.name}: worst |err|/bound = {worst:.3g}"
    return ref
