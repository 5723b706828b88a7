"""Device per-token quantization: the producer of a GEMM's A operand and ``scale_a``.

Two interfaces over ``flygemm_quant_rows`` (``include/flygemm.h``):

* ``build_quant_module(N)`` -> ``(launch_quant, config)`` -- the reference's quant kernel
  builder (``tests/kernels/test_quant.py:81-265``): ``launch_quant(Input, Output, Scales, m_in,
  stream=None)`` with fp16 ``Input[M, N]``, int8 ``Output[M, N]``, fp32 ``Scales[M]``;
  ``Scales = amax / 127`` (0 -> 1) and ``Output = fptosi(Input * (1 / Scales))``.  ``config``
  has the reference's keys.
* ``per_token_quant(x, quant_dtype, rounding)`` -- the reference's ``pertoken_quant``
  (``tests/utils.py:29-73``) on the device: NaN/inf scrubbing, ``scale = amax / dtypeMax``,
  ``q = (x / scale).to(quant_dtype)``; returns ``(q, scale[M, 1])``.  int8 rounds half to
  even by default (the benchmark workloads' rule) or truncates (``rounding="trunc"``, the
  reference's ``.to(torch.int8)``); fp8 (``torch.float8_e4m3fn``) rounds to nearest even.

* ``quant_gemm(x, b, scale_b, N, in_dtype=...)`` -- the GEMM of activations quantized on the
  way in (``flygemm_preshuffle_quant_a``): ``per_token_quant`` (or the reference kernel's
  mode) followed by the preshuffle GEMM launcher, in one call.

All fail loudly if the HIP library is missing; there is no host fallback.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._launch import device_ptr, stream_handle

BLOCK_THREADS = 256
WARP_SIZE = 64
VEC_WIDTH = 8
WIDE_N = 8192

_QIN = {torch.float16: _lib.QUANT_IN["fp16"], torch.bfloat16: _lib.QUANT_IN["bf16"],
        torch.float32: _lib.QUANT_IN["fp32"]}


def _launch(out_ptr, scale_ptr, in_ptr, M, N, in_code, out_code, mode, stream):
    rc = _lib.load().flygemm_quant_rows(out_ptr, scale_ptr, in_ptr, int(M), int(N), in_code, out_code, mode,
                                        stream_handle(stream))
    _lib.check(rc, "flygemm_quant_rows")


def build_quant_module(N: int):
    """Quant launcher for hidden size ``N`` (reference ``test_quant.py:81``)."""
    N = int(N)
    if N <= 0 or N % VEC_WIDTH:
        raise ValueError(f"N={N} must be a positive multiple of {VEC_WIDTH}")
    # the library runs rows of WIDE_N or more elements with twice the threads (kQuantWideN in
    # csrc/quant_rows.h): each thread still owns VEC_WIDTH consecutive elements per slice
    threads = 2 * BLOCK_THREADS if N >= WIDE_N else BLOCK_THREADS
    tile_cols = threads * VEC_WIDTH

    def launch_quant(Input, Output, Scales, m_in, stream=None):
        M = int(m_in)
        if M < 0:
            raise ValueError(f"invalid M={M}")
        i = device_ptr(Input, "Input", M * N, dtypes=(torch.float16,))
        o = device_ptr(Output, "Output", M * N, elem_bytes=1)
        s = device_ptr(Scales, "Scales", M, dtypes=(torch.float32,))
        _launch(o, s, i, M, N, _lib.QUANT_IN["fp16"], _lib.QUANT_OUT["int8"], _lib.QUANT_MODE["recip_trunc"], stream)

    config = {
        "N": N,
        "BLOCK_THREADS": threads,
        "VEC_WIDTH": VEC_WIDTH,
        "ELEMS_PER_BLOCK_ITER": tile_cols,
        "ITERS": (N + tile_cols - 1) // tile_cols,
    }
    return launch_quant, config


def per_token_quant(x: torch.Tensor, quant_dtype=torch.int8, rounding: str = "nearest", out=None, scale=None,
                    stream=None):
    """Per-row quantization of a 2-D fp16/bf16/fp32 GPU tensor; returns ``(q, scale[M, 1])``."""
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, N], got shape {tuple(x.shape)}")
    if x.dtype not in _QIN:
        raise TypeError(f"x dtype {x.dtype} not supported (fp16, bf16, fp32)")
    if quant_dtype == torch.int8:
        out_code = _lib.QUANT_OUT["int8"]
        if rounding == "nearest":
            mode = _lib.QUANT_MODE["div_nearest"]
        elif rounding == "trunc":
            mode = _lib.QUANT_MODE["div_trunc"]
        else:
            raise ValueError(f"rounding must be 'nearest' or 'trunc', got {rounding!r}")
    elif quant_dtype == torch.float8_e4m3fn:
        if rounding != "nearest":
            raise ValueError("fp8 quantization rounds to nearest")
        out_code, mode = _lib.QUANT_OUT["fp8"], _lib.QUANT_MODE["div_nearest"]
    else:
        raise TypeError(f"quant_dtype must be torch.int8 or torch.float8_e4m3fn, got {quant_dtype}")
    M, N = x.shape
    if out is None:
        out = torch.empty(M, N, dtype=quant_dtype, device=x.device)
    if scale is None:
        scale = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    i = device_ptr(x, "x", M * N, dtypes=(x.dtype,))
    o = device_ptr(out, "out", M * N, elem_bytes=1)
    s = device_ptr(scale, "scale", M, dtypes=(torch.float32,))
    _launch(o, s, i, M, N, _QIN[x.dtype], out_code, mode, stream)
    return out, scale


_GEMM_IN = {"fp8": 0, "int8": 1, "int4": 2}
_GEMM_OUT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def quant_gemm(x: torch.Tensor, b, scale_b, N: int, *, in_dtype: str = "fp8", out_dtype: str = "bf16",
               mode: str = "div_nearest", out=None, a_q=None, scale_a=None, variant: int = -1, stream=None):
    """``C[M, N] = GEMM(quant(x), B)`` with ``x`` [M, K] fp16 / bf16 / fp32 quantized per row to
    fp8 (``in_dtype="fp8"``) or int8 codes (``"int8"``, or ``"int4"`` for packed int4 weights),
    ``b`` the preshuffled weight bytes and ``scale_b`` [N] fp32: ``per_token_quant`` (mode
    ``"div_nearest"`` / ``"div_trunc"``) or the reference's quant kernel (``"recip_trunc"``)
    followed by ``compile_preshuffle_gemm_a8``'s launcher, in one call to the library (two
    launches on ``stream``).  ``a_q`` [M, K] and ``scale_a`` [M, 1] receive the codes and the
    row scales; they are allocated when not given.  Returns ``(out, a_q, scale_a)``."""
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [M, K], got shape {tuple(x.shape)}")
    if x.dtype not in _QIN:
        raise TypeError(f"x dtype {x.dtype} not supported (fp16, bf16, fp32)")
    if in_dtype not in _GEMM_IN:
        raise ValueError(f"in_dtype must be one of {sorted(_GEMM_IN)}, got {in_dtype!r}")
    if out_dtype not in _GEMM_OUT:
        raise ValueError(f"out_dtype must be 'bf16' or 'fp16', got {out_dtype!r}")
    if mode not in _lib.QUANT_MODE:
        raise ValueError(f"mode must be one of {sorted(_lib.QUANT_MODE)}, got {mode!r}")
    M, K = x.shape
    N = int(N)
    qdt = torch.float8_e4m3fn if in_dtype == "fp8" else torch.int8
    if out is None:
        out = torch.empty(M, N, dtype=_GEMM_OUT[out_dtype], device=x.device)
    if a_q is None:
        a_q = torch.empty(M, K, dtype=qdt, device=x.device)
    if scale_a is None:
        scale_a = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    b_elems = N * K // 2 if in_dtype == "int4" else N * K
    c = device_ptr(out, "out", M * N, dtypes=(_GEMM_OUT[out_dtype],))
    q = device_ptr(a_q, "a_q", M * K, elem_bytes=1)
    sa = device_ptr(scale_a, "scale_a", M, dtypes=(torch.float32,))
    xi = device_ptr(x, "x", M * K, dtypes=(x.dtype,))
    bp = device_ptr(b, "b", b_elems, elem_bytes=1)
    sb = device_ptr(scale_b, "scale_b", N, dtypes=(torch.float32,))
    rc = _lib.load().flygemm_preshuffle_quant_a(c, q, sa, xi, bp, sb, int(M), N, int(K), _QIN[x.dtype],
                                                _GEMM_IN[in_dtype], _lib.QUANT_MODE[mode],
                                                _lib.FLYGEMM_OUT[out_dtype], int(variant), stream_handle(stream))
    _lib.check(rc, "flygemm_preshuffle_quant_a")
    return out, a_q, scale_a
