"""Quantizers that prepare A, B and their scales (test infrastructure only).

Restates ``pertoken_quant`` (reference ``tests/utils.py:29-73``):
``x -> nan_to_num -> amax = max(max(x), -min(x)) per row -> scale = amax / dtypeMax
-> scale[scale == 0] = 1 -> q = cast(x / scale)``, all in float32.

The reference's cast for int8 is ``.to(torch.int8)``, which truncates toward zero
(``tests/utils.py:71``); the workloads this build is measured on specify
round-to-nearest for int8/int4, so ``quant_rows`` rounds half-to-even and clamps.
fp8 uses the e4m3fn round-to-nearest-even cast, as the reference does.

``quant_rows_recip`` restates the reference's device quant kernel
(``tests/kernels/test_quant.py:81-265``): no NaN/inf scrubbing, ``scale = amax/127`` (0 -> 1,
``:193-198``), then ``fptosi(x * (1/scale))`` -- a float32 reciprocal, a float32 product,
truncation toward zero (``:208-238``).

Pins (``tests/test_oracle.py``): smooth-quant and given-scale known answers; invariants ``|q| <= qmax``, ``|q*scale - x| <=
scale/2`` (int) or half an fp8 ulp (fp8), all-zero rows get scale 1, the row amax
maps to exactly +-qmax; agreement with the product's torch quantizer; the block
quantizer reduces to the row quantizer when the block covers the whole row.
"""
from __future__ import annotations

import numpy as np

from .numerics import E4M3FN_MAX, e4m3fn_encode

QMAX = {"fp8": E4M3FN_MAX, "int8": 127.0, "int4": 7.0}


def _row_scale(x32: np.ndarray, qmax: float) -> np.ndarray:
    amax = np.maximum(x32.max(axis=-1, keepdims=True), -x32.min(axis=-1, keepdims=True))
    scale = (amax / np.float32(qmax)).astype(np.float32)
    scale[scale == 0] = np.float32(1.0)
    scale[~np.isfinite(scale)] = np.float32(1.0)
    return scale


def _cast(y: np.ndarray, kind: str, rounding: str = "nearest") -> np.ndarray:
    if kind == "fp8":
        return e4m3fn_encode(y)
    qmax = QMAX[kind]
    if rounding == "truncate":
        return np.clip(np.trunc(y), -qmax, qmax).astype(np.int8)
    return np.clip(np.rint(y), -qmax, qmax).astype(np.int8)


def quant_rows(x: np.ndarray, kind: str, rounding: str = "nearest", x_scale=None, scale=None):
    """Per-row quantization: returns (q, scale[rows]) with q uint8 codes (fp8) or int8.
    ``rounding`` ("nearest" or "truncate") applies to the integer kinds; fp8 always rounds
    to nearest even.  ``x_scale`` (smooth quant) multiplies the rows first, in float32
    (``tests/utils.py:41-44``); ``scale`` replaces the computed per-row scales (non-finite ones
    become 1, ``:66-68``)."""
    qmax = QMAX[kind]
    x32 = np.asarray(x, dtype=np.float32)
    if x_scale is not None:
        x32 = (x32 * np.asarray(x_scale, dtype=np.float32)).astype(np.float32)
    x32 = np.nan_to_num(x32, nan=0.0, posinf=qmax, neginf=-qmax)
    if scale is None:
        sc = _row_scale(x32, qmax)
    else:
        sc = np.array(scale, dtype=np.float32).reshape(-1, 1)
        sc[~np.isfinite(sc)] = np.float32(1.0)
    q = _cast((x32 / sc).astype(np.float32), kind, rounding)
    return q, sc.reshape(-1)


def quant_rows_recip(x: np.ndarray):
    """The reference device kernel's int8 quantization: (q int8, scale[rows]) with
    ``q = trunc(float32(x * float32(1 / scale)))`` and no scrubbing (finite inputs)."""
    x32 = np.asarray(x, dtype=np.float32)
    amax = np.abs(x32).max(axis=-1, keepdims=True)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    scale[scale == 0] = np.float32(1.0)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    y = (x32 * inv).astype(np.float32)
    return np.trunc(y).astype(np.int8), scale.reshape(-1)


def quant_blocks(x: np.ndarray, block_rows: int, block_cols: int, kind: str = "fp8"):
    """Block quantization over (block_rows x block_cols) tiles: returns (q, scale[R/br, C/bc])."""
    x32 = np.asarray(x, dtype=np.float32)
    R, C = x32.shape
    assert R % block_rows == 0 and C % block_cols == 0
    qmax = QMAX[kind]
    t = x32.reshape(R // block_rows, block_rows, C // block_cols, block_cols).transpose(0, 2, 1, 3)
    t = t.reshape(R // block_rows, C // block_cols, block_rows * block_cols)
    scale = _row_scale(t, qmax)                     # [R/br, C/bc, 1]
    y = (t / scale).astype(np.float32)
    y = y.reshape(R // block_rows, C // block_cols, block_rows, block_cols).transpose(0, 2, 1, 3)
    q = _cast(y.reshape(R, C), kind)
    return q, scale.reshape(R // block_rows, C // block_cols)
