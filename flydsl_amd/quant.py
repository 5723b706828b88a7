"""Host-side operand preparation in torch (runs on CPU or GPU tensors).

Mirrors the reference's helpers in ``tests/utils.py``:

* ``pertoken_quant``  (``tests/utils.py:29-73``, same arguments): per-row symmetric
  quantization of ``x * x_scale`` (smooth quant), ``scale = amax / dtypeMax`` (zero rows -> 1)
  unless given, ``q = cast(x / scale)``.  The reference's int8 cast truncates toward zero
  (``.to(torch.int8)``); here int8/int4 round half to even and clamp (``rounding="nearest"``,
  the rule the measured workloads specify); ``rounding="trunc"`` reproduces the reference's cast.
* ``shuffle_weight``  (``tests/utils.py:76-96``, 1-byte elements, ``layout=(16, 16)``):
  the B preshuffle, byte (n, k) -> ``[n//16][k//16][n%16][k%16]``.
* ``pack_int4``       (``tests/kernels/test_preshuffle_gemm.py:165-174``): two int4 per byte
  from the shuffled int8 values, ``out[j] = u[j] | u[j+4] << 4`` per 8 values.
* ``blockscale_quant``: per-block (1x128 for activations, 128x128 for weights) fp8 scales
  as the blockscale GEMM consumes them (``test_blockscale_preshuffle_gemm.py:86-109``).
"""
from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn  # OCP e4m3: the gfx950 MFMA fp8 format
_QMAX = {torch.int8: 127.0, FP8: 448.0}


def pertoken_quant(x: torch.Tensor, scale=None, x_scale=None, scale_dtype=torch.float32, quant_dtype=torch.int8,
                   dtypeMax=None, *, rounding: str = "nearest"):
    """Per-row quantization with the reference's arguments (``tests/utils.py:29-73``).

    ``x_scale`` (smooth quant): the rows are multiplied by it first (broadcast, e.g. a per-column
    ``[1, cols]`` smoothing factor).  ``scale``: use these per-row scales instead of
    ``amax / dtypeMax``.  Non-finite inputs are scrubbed (NaN -> 0, +-inf -> +-dtypeMax) and
    non-finite scales become 1, as in the reference.  ``scale_dtype``: dtype of the returned
    scales.  Returns (q [rows, cols] of quant_dtype, scale [rows, 1])."""
    x = x.to(torch.float32)
    hidden = x if x_scale is None else x * torch.as_tensor(x_scale, dtype=torch.float32, device=x.device)
    if dtypeMax is None:
        dtypeMax = _QMAX[quant_dtype]
    hidden = torch.nan_to_num(hidden, nan=0.0, posinf=float(dtypeMax), neginf=-float(dtypeMax))
    if scale is None:
        amax = torch.maximum(torch.amax(hidden, dim=-1, keepdim=True), -torch.amin(hidden, dim=-1, keepdim=True))
        per_row = amax / dtypeMax
        per_row[per_row == 0] = 1
    else:
        per_row = torch.as_tensor(scale, device=x.device).to(torch.float32)
    per_row = torch.nan_to_num(per_row, nan=1.0, posinf=1.0, neginf=1.0)
    y = hidden / per_row
    if quant_dtype == torch.int8:
        if rounding == "nearest":
            y = torch.round(y).clamp_(-dtypeMax, dtypeMax)
        elif rounding != "trunc":
            raise ValueError(f"rounding must be 'nearest' or 'trunc', got {rounding!r}")
    return y.to(quant_dtype), per_row.to(scale_dtype)


def blockscale_quant(x: torch.Tensor, block_rows: int, block_cols: int = 128, dtypeMax: float = 448.0):
    """fp8 quantization with one fp32 scale per (block_rows x block_cols) block.

    Returns (q [R, C] fp8, scale [R/block_rows, C/block_cols] fp32)."""
    x = x.to(torch.float32)
    R, C = x.shape
    if R % block_rows or C % block_cols:
        raise ValueError(f"shape {tuple(x.shape)} not divisible by block {block_rows}x{block_cols}")
    t = x.view(R // block_rows, block_rows, C // block_cols, block_cols).permute(0, 2, 1, 3)
    amax = torch.maximum(t.amax(dim=(-1, -2), keepdim=True), -t.amin(dim=(-1, -2), keepdim=True))
    scale = amax / dtypeMax
    scale[scale == 0] = 1
    q = (t / scale).permute(0, 2, 1, 3).reshape(R, C).to(FP8)
    return q, scale.reshape(R // block_rows, C // block_cols).contiguous()


def shuffle_weight(x: torch.Tensor, layout=(16, 16)) -> torch.Tensor:
    """Preshuffle a [N, K] weight of 1- or 2-byte elements; returns a tensor of the same shape
    and dtype.  Each 16-column block is laid out as 16-byte K chunks, column-interleaved
    (reference ``tests/utils.py:76-96``: 16 elements per chunk for 1-byte types, 8 for
    2-byte ones) -- the same permutation of each row's bytes in both cases."""
    if tuple(layout) != (16, 16):
        raise ValueError(f"only layout=(16, 16) is supported, got {layout!r}")
    es = x.element_size()
    if es not in (1, 2):
        raise ValueError(f"shuffle_weight expects 1- or 2-byte elements, got {x.dtype}")
    N, K = x.shape[-2], x.shape[-1]
    if N % 16 or K % 32:
        raise ValueError(f"B shape [{N}, {K}] must have N % 16 == 0 and K % 32 == 0")
    kb = K * es
    u = x.contiguous().view(torch.uint8).reshape(-1, N, kb)
    t = u.view(-1, N // 16, 16, kb // 32, 2, 16).permute(0, 1, 3, 4, 2, 5).contiguous()
    return t.view(torch.uint8).reshape(x.shape[:-1] + (kb,)).view(x.dtype).reshape(x.shape)


def pack_int4(x_shuffled: torch.Tensor) -> torch.Tensor:
    """Pack shuffled int8 values in [-8, 7] two per byte; returns flat int8 of half the size."""
    flat = x_shuffled.contiguous().view(-1).view(torch.int8).to(torch.int16)
    if flat.numel() % 8:
        raise ValueError("int4 packing needs a multiple of 8 values")
    u = (flat & 0xF).to(torch.uint8).view(-1, 8)
    out = u[:, 0:4] | (u[:, 4:8] << 4)
    return out.contiguous().view(-1).view(torch.int8)
