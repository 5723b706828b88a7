"""MI355X preshuffle GEMM: the drop-in for the reference's ``kernels/preshuffle_gemm.py``.

``compile_preshuffle_gemm_a8`` keeps the reference's name, keyword arguments, argument
checks and launcher signature (reference ``kernels/preshuffle_gemm.py:39-202`` and
``:1268-1303``)::

    launch = compile_preshuffle_gemm_a8(K=K, tile_m=..., tile_n=..., tile_k=..., in_dtype="fp8",
                                        out_dtype="bf16")
    launch(c, a, b_preshuffled, scale_a, scale_b, M, N, stream)

computes ``c[m, n] = out_dtype((acc[m, n] * scale_a[m]) * scale_b[n])`` with
``acc = sum_k a[m, k] * b[n, k]`` (fp32 for fp8, exact int32 for int8/int4); bf16/fp16 inputs
are not scaled, ``c = out_dtype(acc)`` with fp32 ``acc``, and their scale arguments may be
empty tensors, as the reference's harness passes them (``tests/kernels/
test_preshuffle_gemm.py:183-188``).  Behind the
launcher there is no JIT: a ctypes call into the hand-written gfx950 kernels of
``flydsl_amd/csrc`` (``flygemm_preshuffle`` in ``include/flygemm.h``).

Differences from the reference, all on purpose:
* ``tile_m/tile_n/tile_k``, ``lds_stage``, ``use_cshuffle_epilog``, ``waves_per_eu`` and
  ``use_async_copy`` are validated exactly as the reference validates them and then serve
  as hints only: the kernel variant comes from the library's MI355X table, keyed on the
  run-time M, N, K.  ``variant=`` forces one (tests, tuning).
* Any ``N % 16 == 0`` is computed in full (the reference's grid silently skips a tail
  when ``N % tile_n != 0``); K must be a multiple of 64 (32 for bf16/fp16): 64-byte K tiles, as the reference's
  ``tile_k * elem_bytes % 64 == 0``.
* GPU errors raise ``RuntimeError`` (the reference prints them).
* ``in_dtype="fp4"`` (MXFP4, what ``compile_preshuffle_gemm_w4`` builds) takes packed e2m1
  bytes and shuffled E8M0 scale bytes (``flydsl_amd.fp4``); N % 32 == 0 and K % 256 == 0.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _lib
from ._launch import device_ptr, stream_handle

_IN_DTYPES = ("fp8", "int8", "int4", "fp16", "bf16", "fp4")
_OUT_TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16}
_IN_TORCH16 = {"bf16": torch.bfloat16, "fp16": torch.float16}


class PreshuffleGemm:
    """Launcher returned by :func:`compile_preshuffle_gemm_a8`.

    ``__call__(arg_c, arg_a, arg_b, arg_scale_a, arg_scale_b, M, N, stream=None)``.
    """

    def __init__(self, *, K, tile_m, tile_n, tile_k, in_dtype, out_dtype, variant=-1, **hints):
        self.K = int(K)
        self.tile_m, self.tile_n, self.tile_k = int(tile_m), int(tile_n), int(tile_k)
        self.in_dtype = in_dtype
        self.out_dtype = out_dtype
        self.variant = int(variant)
        self.hints = hints

    def __call__(self, arg_c, arg_a, arg_b, arg_scale_a, arg_scale_b, M, N, stream=None):
        if self.in_dtype == "fp4":
            return self._call_fp4(arg_c, arg_a, arg_b, arg_scale_a, arg_scale_b, M, N, stream)
        if self.in_dtype not in _lib.FLYGEMM_IN:
            raise NotImplementedError(f"in_dtype={self.in_dtype!r} has no MI355X kernel in this build")
        M, N, K = int(M), int(N), self.K
        h_stream = stream_handle(stream)
        if M < 0 or N <= 0:
            raise ValueError(f"invalid M={M}, N={N}")
        if N % 16:
            raise ValueError(f"N={N} must be a multiple of 16 (preshuffle block)")
        if K % self.tile_k:
            raise ValueError(f"K={K} must be divisible by tile_k={self.tile_k}")
        is16 = self.in_dtype in ("bf16", "fp16")
        if K % (32 if is16 else 64):
            raise ValueError(f"K={K} must be a multiple of {32 if is16 else 64} (64-byte K tile)")
        c = device_ptr(arg_c, "arg_c", M * N, dtypes=(_OUT_TORCH[self.out_dtype],))
        if is16:
            t = _IN_TORCH16[self.in_dtype]
            a = device_ptr(arg_a, "arg_a", M * K, dtypes=(t,))
            b = device_ptr(arg_b, "arg_b", N * K, dtypes=(t,))
            sa = sb = 0  # not scaled; the reference passes empty tensors here
        else:
            b_elems = N * K // 2 if self.in_dtype == "int4" else N * K
            a = device_ptr(arg_a, "arg_a", M * K, elem_bytes=1)
            b = device_ptr(arg_b, "arg_b", b_elems, elem_bytes=1)
            sa = device_ptr(arg_scale_a, "arg_scale_a", M, dtypes=(torch.float32,))
            sb = device_ptr(arg_scale_b, "arg_scale_b", N, dtypes=(torch.float32,))
        lib = _lib.load()
        rc = lib.flygemm_preshuffle(c, a, b, sa, sb, M, N, K, _lib.FLYGEMM_IN[self.in_dtype],
                                    _lib.FLYGEMM_OUT[self.out_dtype], self.variant, h_stream)
        _lib.check(rc, "flygemm_preshuffle")

    def _bind(self):
        """The launch with only the checks that keep it in bounds, for ``flydsl_amd.compile``:
        tensor data pointers, M, N and the stream are read per call and go straight to the C
        entry point (which checks the sizes), after one comparison of each tensor's element
        count with what M, N and K need (skipped when the same tensor objects and sizes come
        again); dtypes and contiguity are the caller's, as in the reference's
        ``CompiledFunction`` (python/flydsl/compiler/jit_function.py:895-915)."""
        lib = _lib.load()
        K, var, out = self.K, self.variant, _lib.FLYGEMM_OUT[self.out_dtype]
        check = _lib.check
        fp4 = self.in_dtype == "fp4"
        scaled = self.in_dtype not in _IN_TORCH16
        fn = lib.flygemm_mxfp4 if fp4 else lib.flygemm_preshuffle
        what = "flygemm_mxfp4" if fp4 else "flygemm_preshuffle"
        ind = None if fp4 else _lib.FLYGEMM_IN[self.in_dtype]
        # elements per row of A and B, and scale elements per row of A / of B, as the launcher
        # checks them (MXFP4 scales: bytes over rows padded to 32)
        ka = K // 2 if fp4 else K
        kb = K // 2 if fp4 or self.in_dtype == "int4" else K
        ks = K // 32 if fp4 else 1

        last = [None] * 7   # the tensors and sizes of the last call that passed the checks

        def call(c, a, b, sa, sb, M, N, stream=None):
            s = 0 if stream is None else (stream if type(stream) is int else stream.cuda_stream)
            if not (c is last[0] and a is last[1] and b is last[2] and sa is last[3] and sb is last[4]
                    and M == last[5] and N == last[6]):
                if (c.numel() < M * N or a.numel() < M * ka or b.numel() < N * kb
                        or (scaled and (sa.numel() < ((M + 31) // 32 * 32 if fp4 else M) * ks
                                        or sb.numel() < N * ks))):
                    raise ValueError(f"a tensor is too small for M={M}, N={N}, K={K}")
                last[:] = (c, a, b, sa, sb, M, N)
            if fp4:
                rc = fn(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), M, N, K, out, var, s)
            else:
                rc = fn(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr() if scaled else None,
                        sb.data_ptr() if scaled else None, M, N, K, ind, out, var, s)
            if rc:
                check(rc, what)
        return call

    def _call_fp4(self, arg_c, arg_a, arg_b, arg_scale_a, arg_scale_b, M, N, stream=None):
        """MXFP4: packed e2m1 A [M, K/2] and preshuffled B [N, K/2] bytes, shuffled E8M0 scales
        [round_up(M, 32), K/32] and [N, K/32] bytes (``flydsl_amd.fp4``; reference harness
        ``tests/kernels/test_preshuffle_gemm.py:315-358``)."""
        M, N, K = int(M), int(N), self.K
        h_stream = stream_handle(stream)
        if M < 0 or N <= 0:
            raise ValueError(f"invalid M={M}, N={N}")
        if N % 32:
            raise ValueError(f"N={N} must be a multiple of 32 for MXFP4 (scale groups)")
        if K % 256:
            raise ValueError(f"K={K} must be a multiple of 256 for MXFP4")
        if K % self.tile_k:
            raise ValueError(f"K={K} must be divisible by tile_k={self.tile_k}")
        c = device_ptr(arg_c, "arg_c", M * N, dtypes=(_OUT_TORCH[self.out_dtype],))
        a = device_ptr(arg_a, "arg_a", M * K // 2, elem_bytes=1)
        b = device_ptr(arg_b, "arg_b", N * K // 2, elem_bytes=1)
        sa = device_ptr(arg_scale_a, "arg_scale_a", (M + 31) // 32 * 32 * (K // 32), elem_bytes=1)
        sb = device_ptr(arg_scale_b, "arg_scale_b", N * (K // 32), elem_bytes=1)
        rc = _lib.load().flygemm_mxfp4(c, a, b, sa, sb, M, N, K, _lib.FLYGEMM_OUT[self.out_dtype], self.variant, h_stream)
        _lib.check(rc, "flygemm_mxfp4")


def compile_preshuffle_gemm_a8(
    *,
    M: int = 0,
    N: int = 0,
    K: int,
    tile_m: int,
    tile_n: int,
    tile_k: int,
    in_dtype: str = "fp8",
    out_dtype: str = "fp16",
    lds_stage: int = 2,
    use_cshuffle_epilog: bool = False,
    waves_per_eu: Optional[int] = None,
    use_async_copy: bool = False,
    variant: int = -1,
):
    """Validate like the reference (``kernels/preshuffle_gemm.py:67-134,670-673``) and return
    a launcher ``(c, a, b, scale_a, scale_b, M, N, stream)``."""
    if in_dtype not in _IN_DTYPES:
        raise ValueError(
            "in_dtype must be one of ('fp8','int8','int4','fp16','bf16','fp4'), " f"got {in_dtype!r}"
        )
    if out_dtype not in ("fp16", "bf16"):
        raise ValueError(f"out_dtype must be 'fp16' or 'bf16', got {out_dtype!r}")
    is_fp4 = in_dtype == "fp4"
    elem_bytes = 1 if in_dtype in ("fp8", "int8", "int4", "fp4") else 2
    pack = 2 if is_fp4 else 1
    tile_k_bytes = int(tile_k) * elem_bytes
    if tile_k_bytes % 64 != 0:
        raise ValueError(
            f"tile_k_bytes must be divisible by 64, got tile_k_bytes={tile_k_bytes} "
            f"(tile_k={tile_k}, elem_bytes={elem_bytes})"
        )
    if is_fp4 and tile_k_bytes // pack // 64 < 2 and int(tile_k) != 128:
        raise ValueError(f"FP4 requires tile_k=128 or tile_k >= {64 * 2 * pack}, got tile_k={tile_k}")
    if is_fp4 and int(tile_k) == 128 and lds_stage != 2:
        raise NotImplementedError("FP4 tile_k=128 currently only supports lds_stage=2")
    if int(lds_stage) not in (1, 2):
        raise ValueError(f"lds_stage must be 1 or 2, got {lds_stage!r}")
    bytes_a_per_tile = int(tile_m) * int(tile_k) * elem_bytes // pack
    if bytes_a_per_tile % 256 != 0:
        raise ValueError(
            "tile_m*tile_k*elem_bytes/a_elem_vec_pack must be divisible by 256: "
            f"tile_m={tile_m}, tile_k={tile_k}, elem_bytes={elem_bytes}, pack={pack}"
        )
    if (bytes_a_per_tile // 256) % 16 != 0:
        raise ValueError(f"bytes_per_thread_a ({bytes_a_per_tile // 256}) must be divisible by 16")
    if int(tile_n) % 64 != 0 or int(tile_m) % 16 != 0:
        raise ValueError(f"tile_n must be a multiple of 64 and tile_m of 16, got {tile_m}x{tile_n}")
    if in_dtype == "fp8" and int(tile_k) % 128 != 0:
        raise ValueError(f"tile_k must be divisible by 128 for mfma_scale_x128, got tile_k={tile_k}")
    return PreshuffleGemm(
        K=K, tile_m=tile_m, tile_n=tile_n, tile_k=tile_k, in_dtype=in_dtype, out_dtype=out_dtype,
        variant=variant, M=M, N=N, lds_stage=lds_stage, use_cshuffle_epilog=use_cshuffle_epilog,
        waves_per_eu=waves_per_eu, use_async_copy=use_async_copy,
    )


def compile_preshuffle_gemm_w4(*, M: int = 0, N: int = 0, K: int, tile_m: int, tile_n: int, tile_k: int,
                               a_dtype: str = "fp4", b_dtype: str = "fp4", out_dtype: str = "bf16",
                               lds_stage: int = 2, use_cshuffle_epilog: bool = False,
                               waves_per_eu: Optional[int] = None, use_async_copy: bool = False):
    """MXFP4 entry (reference ``kernels/preshuffle_gemm.py:1306-1337``): fp4 A and B with 1x32
    E8M0 block scales, applied inside the gfx950 scaled MFMA.  fp8 A is rejected as the
    reference rejects it."""
    if a_dtype == "fp8":
        raise NotImplementedError("fp8-A not yet supported with MXFP4 kernel (op_sel_a overflow)")
    return compile_preshuffle_gemm_a8(
        M=M, N=N, K=K, tile_m=tile_m, tile_n=tile_n, tile_k=tile_k, in_dtype="fp4",
        out_dtype=out_dtype, lds_stage=lds_stage, use_cshuffle_epilog=use_cshuffle_epilog,
        waves_per_eu=waves_per_eu, use_async_copy=use_async_copy,
    )


def accumulators(acc, a, b, M, N, K, in_dtype, variant=-1, stream=None):
    """Raw accumulators of ``sum_k a[m,k] b[n,k]`` (int32 for int8/int4, fp32 for fp8, bf16
    and fp16), no scaling: the value the kernels hold before the epilogue."""
    if in_dtype not in _lib.FLYGEMM_IN or in_dtype == "fp4":
        raise ValueError(f"in_dtype must be one of fp8, int8, int4, bf16, fp16 (MXFP4 accumulators: the fp4 "
                         f"launcher with out_dtype fp32 through flygemm_mxfp4), got {in_dtype!r}")
    b_elems = N * K // 2 if in_dtype == "int4" else N * K
    want = torch.int32 if in_dtype in ("int8", "int4") else torch.float32
    eb = 2 if in_dtype in ("bf16", "fp16") else 1
    p_acc = device_ptr(acc, "acc", M * N, dtypes=(want,))
    p_a = device_ptr(a, "a", M * K, elem_bytes=eb)
    p_b = device_ptr(b, "b", b_elems, elem_bytes=eb)
    lib = _lib.load()
    rc = lib.flygemm_accumulators(p_acc, p_a, p_b, int(M), int(N), int(K), _lib.FLYGEMM_IN[in_dtype],
                                  int(variant), stream_handle(stream))
    _lib.check(rc, "flygemm_accumulators")


__all__ = ["compile_preshuffle_gemm_a8", "compile_preshuffle_gemm_w4", "accumulators", "PreshuffleGemm"]
