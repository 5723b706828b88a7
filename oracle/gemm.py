"""Dequantize-then-matmul oracles and the fused epilogue (test infrastructure only).

* ``run_torch``            restates ``tests/kernels/test_preshuffle_gemm.py:55-65``:
                           ``mm(a.float() * sa[:, None], (b.float() * sb[:, None]).T)``;
                           for bf16/fp16 inputs (bit patterns, uint16) there are no scales
                           (``:146-151``): ``mm(a.float(), b.float().T)``.
* ``run_torch_blockscale`` restates ``tests/kernels/test_blockscale_preshuffle_gemm.py:86-109``:
                           A scales expanded over 1x128 blocks, B scales over 128x128 blocks
                           (``w_scale.view(-1,1).repeat(...).permute(0,2,1,3)``), then
                           ``F.linear`` in float32.
* ``acc_int``              the exact int32 accumulator ``sum_k a[m,k] * b[n,k]`` the int8/int4
                           kernels form before scaling (``kernels/preshuffle_gemm.py:764-797``).
* ``epilogue_int_bf16``    ``bf16(rne((float(acc) * sa[m]) * sb[n]))``: int->float, then the two
                           float32 multiplies in that order, then round to bf16
                           (``kernels/preshuffle_gemm.py:873-883``).

``dtype="f64"`` evaluates the same expressions in float64 (used as the accuracy
reference; the float32 form is what the reference itself computes).

Pins (``tests/test_oracle.py``): brute-force triple loops on small shapes; ``acc_int``
against ``torch._int_mm``/int64 ``torch.mm``; ``run_torch`` float32 path against the
float64 path within float32 accumulation error; ``run_torch_blockscale`` against an
independent per-block formulation ``sum_kb (A_kb B_kb^T) * sa[:,kb] * sb[n//128,kb]``, and
its reduction to ``run_torch`` when every block scale of a row/column is equal.
"""
from __future__ import annotations

import numpy as np

from .numerics import bf16_rne, bf16_to_f32, e4m3fn_decode, f16_to_f32


def dequant_rows(q: np.ndarray, scale, kind: str, dtype=np.float32) -> np.ndarray:
    if kind == "bf16":
        return bf16_to_f32(q).astype(dtype)
    if kind == "fp16":
        return f16_to_f32(q).astype(dtype)
    v = e4m3fn_decode(q) if kind == "fp8" else np.asarray(q).view(np.int8).astype(np.float32)
    out = (v * np.asarray(scale, dtype=np.float32).reshape(-1, 1)).astype(np.float32)
    return out.astype(dtype)


def run_torch(a_q, b_q, sa, sb, kind: str, dtype: str = "f32") -> np.ndarray:
    """C[M, N] = (A * sa) @ (B * sb)^T with A [M, K], B [N, K] in row-major (unshuffled)."""
    np_dt = np.float64 if dtype == "f64" else np.float32
    a = dequant_rows(a_q, sa, kind, np_dt)
    b = dequant_rows(b_q, sb, kind, np_dt)
    return a @ b.T


def acc_int(a_q, b_q) -> np.ndarray:
    """Exact int32 accumulator of int8 x int8 over K (float64 BLAS is exact below 2^53)."""
    a = np.asarray(a_q).view(np.int8).astype(np.float64)
    b = np.asarray(b_q).view(np.int8).astype(np.float64)
    assert a.shape[1] * 128 * 128 < 2 ** 31
    return (a @ b.T).astype(np.int64).astype(np.int32)


def epilogue_int_bf16(acc: np.ndarray, sa, sb) -> np.ndarray:
    """bf16 bit patterns of ``(float32(acc) * sa[m]) * sb[n]``."""
    v = acc.astype(np.float32) * np.asarray(sa, dtype=np.float32).reshape(-1, 1)
    v = v.astype(np.float32) * np.asarray(sb, dtype=np.float32).reshape(1, -1)
    return bf16_rne(v.astype(np.float32))


def _expand_blockscale(x_scale, w_scale, M, N, K, bn=128, bk=128):
    sk = (K + bk - 1) // bk
    sn = (N + bn - 1) // bn
    xs = np.asarray(x_scale, dtype=np.float32).reshape(M, sk)
    ws = np.asarray(w_scale, dtype=np.float32).reshape(sn, sk)
    xs_e = np.repeat(xs, bk, axis=1)[:, :K]
    ws_e = np.repeat(np.repeat(ws, bn, axis=0), bk, axis=1)[:N, :K]
    return xs_e, ws_e


def run_torch_blockscale(x_q, w_q, x_scale, w_scale, dtype: str = "f32") -> np.ndarray:
    """x_q fp8 [M, K], w_q fp8 [N, K] (unshuffled), x_scale [M, K/128], w_scale [N/128, K/128]."""
    np_dt = np.float64 if dtype == "f64" else np.float32
    M, K = x_q.shape
    N = w_q.shape[0]
    xs_e, ws_e = _expand_blockscale(x_scale, w_scale, M, N, K)
    x = (e4m3fn_decode(x_q) * xs_e).astype(np.float32).astype(np_dt)
    w = (e4m3fn_decode(w_q) * ws_e).astype(np.float32).astype(np_dt)
    return x @ w.T


def blockscale_per_block(x_q, w_q, x_scale, w_scale, bn=128, bk=128) -> np.ndarray:
    """Independent formulation: sum over K blocks of exact partial dots times both scales."""
    M, K = x_q.shape
    N = w_q.shape[0]
    sk = K // bk
    xs = np.asarray(x_scale, dtype=np.float64).reshape(M, sk)
    ws = np.asarray(w_scale, dtype=np.float64).reshape(-1, sk)
    a = e4m3fn_decode(x_q).astype(np.float64)
    b = e4m3fn_decode(w_q).astype(np.float64)
    out = np.zeros((M, N), dtype=np.float64)
    nb = np.arange(N) // bn
    for kb in range(sk):
        part = a[:, kb * bk:(kb + 1) * bk] @ b[:, kb * bk:(kb + 1) * bk].T
        out += part * xs[:, kb:kb + 1] * ws[nb, kb][None, :]
    return out


def within_bar(out: np.ndarray, ref: np.ndarray, rtol: float = 1e-2, atol_rms: float = 1e-2):
    """The bf16 acceptance bar: |out - ref| <= rtol*|ref| + atol_rms*RMS(ref), elementwise.

    Returns (ok, worst_ratio) where worst_ratio = max |out-ref| / bound (<= 1 passes).
    """
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) if ref.size else 0.0
    bound = rtol * np.abs(ref) + atol_rms * rms
    if out.size == 0:
        return True, 0.0
    ratio = np.abs(out - ref) / np.maximum(bound, 1e-30)
    worst = float(np.nanmax(ratio)) if np.isfinite(ratio).all() else float("inf")
    return bool(worst <= 1.0), worst
