"""MI355X FP8 blockscale preshuffle GEMM: drop-in for the reference's
``kernels/blockscale_preshuffle_gemm.py``.

The reference snapshot lacks that file; its contract is the call site
``tests/kernels/test_blockscale_preshuffle_gemm.py:173-204`` and the torch oracle
``:86-109`` (the block-scale compute pattern also appears in
``kernels/moe_blockscale_2stage.py:677-777``)::

    exe = compile_blockscale_preshuffle_gemm(M=M, N=N, K=K, tile_m=.., tile_n=.., tile_k=..,
                                             scale_block_k=128, out_dtype="bf16")
    exe(c, x_fp8, b_preshuffled, x_scale_t, w_scale, M, N, stream)

computes ``c[m, n] = sum_kb (sum_{k in kb} x[m,k] w[n,k]) * x_scale[m, kb] * w_scale[n//128, kb]``
with ``x_scale_t`` = ``x_scale.T`` flattened ([K/128, M], K-block major) and ``w_scale``
[ceil(N/128), K/128] row-major.  Per 128-deep K block the kernel forms the fp32 MFMA partial
and folds it into the accumulator with one fused multiply-add by ``sa * sb``.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._launch import device_ptr, stream_handle

_OUT_TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16}


class BlockscaleGemm:
    def __init__(self, *, K, tile_m, tile_n, tile_k, scale_block_k, out_dtype, variant=-1, **hints):
        self.K = int(K)
        self.tile_m, self.tile_n, self.tile_k = int(tile_m), int(tile_n), int(tile_k)
        self.scale_block_k = int(scale_block_k)
        self.out_dtype = out_dtype
        self.variant = int(variant)
        self.hints = hints

    def __call__(self, arg_c, arg_a, arg_b, arg_scale_a, arg_scale_b, M, N, stream=None):
        M, N, K = int(M), int(N), self.K
        h_stream = stream_handle(stream)
        if M < 0 or N <= 0 or N % 16:
            raise ValueError(f"invalid M={M}, N={N} (N must be a positive multiple of 16)")
        sk = K // self.scale_block_k
        sn = (N + 127) // 128
        c = device_ptr(arg_c, "arg_c", M * N, dtypes=(_OUT_TORCH[self.out_dtype],))
        a = device_ptr(arg_a, "arg_a", M * K, elem_bytes=1)
        b = device_ptr(arg_b, "arg_b", N * K, elem_bytes=1)
        sa = device_ptr(arg_scale_a, "arg_scale_a", M * sk, dtypes=(torch.float32,))
        sb = device_ptr(arg_scale_b, "arg_scale_b", sn * sk, dtypes=(torch.float32,))
        lib = _lib.load()
        rc = lib.flygemm_blockscale(c, a, b, sa, sb, M, N, K, self.scale_block_k,
                                    _lib.FLYGEMM_OUT[self.out_dtype], self.variant, h_stream)
        _lib.check(rc, "flygemm_blockscale")

    def _bind(self):
        """The launch with only its bounds checks, for ``flydsl_amd.compile`` (as
        ``PreshuffleGemm._bind``)."""
        fn = _lib.load().flygemm_blockscale
        K, sbk, out, var = self.K, self.scale_block_k, _lib.FLYGEMM_OUT[self.out_dtype], self.variant
        sk = K // sbk
        check = _lib.check

        last = [None] * 7

        def call(c, a, b, sa, sb, M, N, stream=None):
            s = 0 if stream is None else (stream if type(stream) is int else stream.cuda_stream)
            if not (c is last[0] and a is last[1] and b is last[2] and sa is last[3] and sb is last[4]
                    and M == last[5] and N == last[6]):
                if (c.numel() < M * N or a.numel() < M * K or b.numel() < N * K or sa.numel() < M * sk
                        or sb.numel() < (N + 127) // 128 * sk):
                    raise ValueError(f"a tensor is too small for M={M}, N={N}, K={K}")
                last[:] = (c, a, b, sa, sb, M, N)
            rc = fn(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(), M, N, K, sbk, out, var, s)
            if rc:
                check(rc, "flygemm_blockscale")
        return call


def compile_blockscale_preshuffle_gemm(*, M: int = 0, N: int = 0, K: int, tile_m: int = 64, tile_n: int = 128,
                                       tile_k: int = 128, scale_block_k: int = 128, out_dtype: str = "bf16",
                                       use_async_copy: bool = False, variant: int = -1):
    if out_dtype not in _OUT_TORCH:
        raise ValueError(f"out_dtype must be 'fp16' or 'bf16', got {out_dtype!r}")
    if int(scale_block_k) != 128:
        raise ValueError(f"scale_block_k must be 128, got {scale_block_k}")
    if int(tile_k) % int(scale_block_k) != 0:
        raise ValueError(f"tile_k={tile_k} must be a multiple of scale_block_k={scale_block_k}")
    if int(K) % int(tile_k) != 0:
        raise ValueError(f"K={K} must be divisible by tile_k={tile_k}")
    if int(tile_m) * int(tile_k) // 256 < 16:
        raise ValueError(f"tile_m*tile_k/256 must be >= 16, got tile {tile_m}x{tile_k}")
    return BlockscaleGemm(K=K, tile_m=tile_m, tile_n=tile_n, tile_k=tile_k, scale_block_k=scale_block_k,
                          out_dtype=out_dtype, variant=variant, M=M, N=N, use_async_copy=use_async_copy)


__all__ = ["compile_blockscale_preshuffle_gemm", "BlockscaleGemm"]
