"""MXFP4 oracle (test infrastructure only): e2m1 values, E8M0 scales, the reference's 1x32
quantizer, its two shuffles and its dequantize-then-matmul.

Restates, in numpy:
* ``e2m1_decode``      ``mxfp4_to_f32`` (``tests/kernels/utils/fp4_utils.py:22-49``), here from
                       the bit fields: sign, 2 exponent bits (bias 1), 1 mantissa bit.
* ``e8m0_decode``      ``e8m0_to_f32`` (``:64-72``): 2**(s - 127), 0 -> 2**-127, 0xFF -> NaN.
* ``e8m0_encode``      ``f32_to_e8m0`` (``:52-61``): biased exponent, +1 when bit 22 is set and
                       (any of bits 0..21 is set or the exponent is nonzero).
* ``e2m1_encode``      ``_f32_to_floatx_unpacked(x, 2, 1)`` (``:123-239``): round to nearest
                       even on the e2m1 grid, saturate at 6.
* ``quant_1x32``       ``per_1x32_f4_quant`` (``:656-687``): scale = e8m0(amax / 4) per 32
                       elements, q = e2m1(x / scale), element 2j in the low nibble.
* ``shuffle_weight_w4`` / ``shuffle_scale_w4``  (``:578-653``, dense GEMM form).
* ``run_torch_w4``     ``tests/kernels/test_preshuffle_gemm.py:328-333``.

Pins (``tests/test_oracle.py``): the OCP MX e2m1 value table; exhaustive code round trips,
midpoint ties and saturation; E8M0 against floor(log2 x) + [significand >= 1.5] computed with
``math.frexp`` plus bit-pattern edge cases; quantizer error bounds and equality with the
product's torch quantizer; element-by-element loops for both shuffles; a brute-force matmul.
"""
from __future__ import annotations

import numpy as np


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes).astype(np.int64) & 0xF
    sign = np.where(c & 8, -1.0, 1.0)
    e = (c >> 1) & 3
    m = c & 1
    mag = np.where(e == 0, 0.5 * m, (1.0 + 0.5 * m) * np.exp2(e - 1.0))
    return (sign * mag).astype(np.float32)


def unpack(packed: np.ndarray) -> np.ndarray:
    """[..., n] bytes -> [..., 2n] codes, low nibble first."""
    b = np.asarray(packed).view(np.uint8)
    return np.stack([b & 0xF, b >> 4], axis=-1).reshape(*b.shape[:-1], -1)


def e8m0_decode(s: np.ndarray) -> np.ndarray:
    b = np.asarray(s).view(np.uint8).astype(np.int64)
    out = np.exp2(b - 127.0)
    out = np.where(b == 0, 2.0 ** -127, out)
    out = np.where(b == 0xFF, np.nan, out)
    return out.astype(np.float32)


def e8m0_encode(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    e = (u >> 23) & 0xFF
    up = ((u & 0x400000) != 0) & (((u & 0x3FFFFF) != 0) | (e > 0))
    out = np.where(e == 0xFF, 0xFF, e + up)
    return (out & 0xFF).astype(np.uint8)


def e2m1_encode(y: np.ndarray) -> np.ndarray:
    y = np.asarray(y, dtype=np.float32)
    a = np.abs(y).astype(np.float64)
    step = np.where(a < 2.0, 0.5, np.where(a < 4.0, 1.0, 2.0))
    q = np.minimum(np.rint(a / step) * step, 6.0)          # rint: half to even
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    mag = np.searchsorted(grid, q)
    sign = np.signbit(y).astype(np.int64) << 3
    return (mag | sign).astype(np.uint8)


def quant_1x32(x: np.ndarray):
    """x [R, K] (K % 32 == 0) -> (packed [R, K/2] uint8, scales [R, K/32] uint8)."""
    x = np.asarray(x, dtype=np.float32)
    R, K = x.shape
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    s = e8m0_encode((amax / np.float32(4.0)).astype(np.float32))
    y = (xb / e8m0_decode(s)[:, None]).astype(np.float32)
    codes = e2m1_encode(y).reshape(R, K)
    packed = (codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)
    return packed.astype(np.uint8), s.reshape(R, K // 32)


def dequant(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[R, K/2] packed codes and [R', K/32] scales (R' >= R) -> float64 [R, K]."""
    v = e2m1_decode(unpack(packed)).astype(np.float64)
    R, K = v.shape
    s = e8m0_decode(np.asarray(scales)[:R]).astype(np.float64)
    return v * np.repeat(s, 32, axis=1)[:, :K]


def run_torch_w4(a_packed, b_packed, a_scales, b_scales, dtype: str = "f32") -> np.ndarray:
    np_dt = np.float64 if dtype == "f64" else np.float32
    a = dequant(a_packed, a_scales).astype(np.float32).astype(np_dt)
    b = dequant(b_packed, b_scales).astype(np.float32).astype(np_dt)
    return a @ b.T


def shuffle_weight_w4(packed: np.ndarray) -> np.ndarray:
    """[N, K/2] bytes -> [N/16][K/128][4][16][16] bytes (flat)."""
    u = np.ascontiguousarray(np.asarray(packed).view(np.uint8))
    N, kb = u.shape
    return np.ascontiguousarray(u.reshape(N // 16, 16, kb // 64, 4, 16).transpose(0, 2, 3, 1, 4)).reshape(-1)


def shuffle_scale_w4(scales: np.ndarray) -> np.ndarray:
    """[R, K/32] bytes -> [R/32][K/256][4 (kl)][16 (rl)][2 (kp)][2 (rp)] bytes (flat)."""
    u = np.ascontiguousarray(np.asarray(scales).view(np.uint8))
    R, ks = u.shape
    t = u.reshape(R // 32, 2, 16, ks // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1)
    return np.ascontiguousarray(t).reshape(-1)
