"""Epilogue contract of the MI355X kernels (counterpart of the reference's
``kernels/mfma_epilogues.py``).

In the reference, ``mfma_epilog`` (``kernels/mfma_epilogues.py:242-309``) is a trace-time
helper that emits either the direct row epilogue (``default_epilog``, ``:52-84``) or the
LDS "CShuffle" epilogue (``c_shuffle_epilog``, ``:87-239``).  Here the epilogue is fused
into the HIP kernels; this module states its contract so host code and tests share it:

* accumulator layout of one 16x16 MFMA tile (CDNA 16x16 output layout): lane ``l`` holds
  rows ``4*(l//16) + i`` (``i`` = 0..3) of column ``l % 16`` (reference ``default_epilog``
  row formula ``bx_m + mi*16 + lane_div_16*4 + ii``);
* ``rowcol``: ``out = cvt((float(acc) * scale_a[row]) * scale_b[col])`` -- int32 is converted
  to fp32 first, the two fp32 multiplies happen in that order, ``cvt`` rounds to nearest
  even (reference ``kernels/preshuffle_gemm.py:873-883``);
* ``block``: per 128-deep K block, ``acc = fma(partial, scale_a[kb][row] * scale_b[col//128][kb], acc)``,
  then ``cvt(acc)`` (``kernels/moe_blockscale_2stage.py:748-766``);
* ``raw``: the unscaled accumulator (int32 / fp32), for bit-exact checks.
"""
from __future__ import annotations

EPILOGUES = ("rowcol", "block", "raw")


def tile_coords(lane: int, mi: int = 0, ni: int = 0, ii: int = 0):
    """(row, col) inside a wave tile of the accumulator element ``acc[mi][ni][ii]`` of ``lane``."""
    if not (0 <= lane < 64 and 0 <= ii < 4):
        raise ValueError("lane must be in [0, 64) and ii in [0, 4)")
    return mi * 16 + (lane // 16) * 4 + ii, ni * 16 + lane % 16


def mfma_epilog(use_cshuffle: bool = False, **_):
    """Name of the fused epilogue a launcher uses; both reference modes map to the same
    fused store (the choice is a kernel-internal detail on MI355X)."""
    return "rowcol"
