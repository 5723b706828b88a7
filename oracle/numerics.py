"""Scalar formats used on the path: OCP fp8 e4m3fn and bf16 (test infrastructure only).

Pins (``tests/test_oracle.py``):
* ``e4m3fn_decode``  known values from the OCP FP8 spec (0x7E = 448, 0x08 = 2^-6,
  0x01 = 2^-9, 0x38 = 1.0, 0x7F/0xFF = NaN) and all 256 codes against torch's
  ``float8_e4m3fn -> float32`` conversion (the library routine the reference uses).
* ``e4m3fn_encode``  round trip ``encode(decode(c)) == c`` for every finite code,
  ties at exact midpoints resolved to the even mantissa, and agreement with torch's
  ``float32 -> float8_e4m3fn`` cast (``tests/utils.py:71`` uses that cast) on
  1e6 random values plus all midpoints.
* ``bf16_rne``       against torch's ``float32 -> bfloat16`` cast, and exact on values
  already representable in bf16.
"""
from __future__ import annotations

import numpy as np

E4M3FN_MAX = 448.0


def _decode_table() -> np.ndarray:
    """Value of every e4m3fn code: 1 sign, 4 exponent (bias 7), 3 mantissa bits.

    No infinities; exponent field 15 with mantissa 7 is NaN (OCP 8-bit FP spec, E4M3).
    """
    tab = np.empty(256, dtype=np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            v = np.nan
        elif e == 0:
            v = s * (m / 8.0) * 2.0 ** -6
        else:
            v = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
        tab[code] = v
    return tab


E4M3FN_TABLE = _decode_table()


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """uint8/int8 codes -> float32 values."""
    return E4M3FN_TABLE[np.asarray(codes).view(np.uint8)]


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes (uint8), round to nearest, ties to even.

    Magnitudes that round to 480 or above become NaN (0x7F | sign), matching the
    non-saturating cast the reference uses (``(x / scale).to(float8_e4m3fn)``,
    ``tests/utils.py:71``).  Quantized data never gets there: ``|x/scale| <= 448``.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.uint16) << 7
    _, E = np.frexp(a)                       # a = f * 2^E, f in [0.5, 1)
    e = np.maximum(E.astype(np.int64) - 1, -6)  # unbiased exponent, clamped to subnormal range
    q = np.ldexp(1.0, (e - 3).astype(np.int32))  # quantum: 3 mantissa bits
    with np.errstate(invalid="ignore", over="ignore"):
        r = np.rint(a / q)                   # exact division; rint is ties-to-even
        r = np.where(np.isfinite(r), r, 0.0)
    code = ((e + 7) << 3) + r.astype(np.int64) - 8
    code = np.where(a == 0, 0, code)
    bad = np.isnan(x) | np.isinf(x) | (code >= 0x7F)
    code = np.where(bad, 0x7F, code)
    return (code.astype(np.uint16) | sign).astype(np.uint8)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even; NaN kept quiet."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    out = np.where(nan, (b >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def bf16_trunc(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16) by truncation: the upper 16 bits, the
    conversion of the reference's int8/int4 -> bf16 weight path
    (``kernels/mfma_preshuffle_pipeline.py:111-141``, ``bits >> 16``)."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32."""
    return (np.asarray(bits).view(np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    """IEEE binary16 bit patterns (uint16) -> float32 (exact)."""
    return np.asarray(bits).view(np.uint16).view(np.float16).astype(np.float32)


def round_half_even(x: np.ndarray) -> np.ndarray:
    return np.rint(x)
