"""ctypes binding of ``include/flygemm.h`` (the library built by ``flydsl_amd.build``).

There is no fallback: if the HIP library is missing or fails to load, every GEMM entry
point raises.  Only ``load()`` touches the file system; nothing here initializes the GPU.
"""
from __future__ import annotations

import ctypes
import os

from .build import OUT as LIB_PATH

FLYGEMM_IN = {"fp8": 0, "int8": 1, "int4": 2, "bf16": 3, "fp16": 4, "fp4": 5, "int4_bf16": 6, "int8smooth": 7}
FLYGEMM_OUT = {"bf16": 0, "fp16": 1, "fp32": 2}
QUANT_IN = {"fp16": 0, "bf16": 1, "fp32": 2}
QUANT_OUT = {"fp8": 0, "int8": 1}
QUANT_MODE = {"recip_trunc": 0, "div_trunc": 1, "div_nearest": 2}

# (name, restype, argtypes) for every symbol include/flygemm.h declares
_P = ctypes.c_void_p
_I = ctypes.c_int32
_F = ctypes.c_void_p  # const float*
SIGNATURES = [
    ("flygemm_preshuffle", ctypes.c_int, [_P, _P, _P, _F, _F, _I, _I, _I, _I, _I, _I, _P]),
    ("flygemm_blockscale", ctypes.c_int, [_P, _P, _P, _F, _F, _I, _I, _I, _I, _I, _I, _P]),
    ("flygemm_accumulators", ctypes.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    ("flygemm_quant_rows", ctypes.c_int, [_P, _F, _P, _I, _I, _I, _I, _I, _P]),
    ("flygemm_preshuffle_quant_a", ctypes.c_int, [_P] * 5 + [_F] + [_I] * 8 + [_P]),
    ("flygemm_mxfp4", ctypes.c_int, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    ("flygemm_moe_gemm1", ctypes.c_int, [_P, _P, _P, _F, _F, _P, _P, _F, _P] + [_I] * 12 + [_P]),
    ("flygemm_moe_gemm2", ctypes.c_int, [_P, _P, _P, _F, _F, _P, _P, _F, _P] + [_I] * 13 + [_P]),
    ("flygemm_moe_reduce", ctypes.c_int, [_P, _P, _P, _I, _I, _I, _I, _P]),
    ("flygemm_moe_select_tile", ctypes.c_int, [_I] * 10 + [_P, _P]),
    ("flygemm_moe_gemm2_reduce_noalloc", ctypes.c_int,
     [_P, _P, _P, _F, _F, _P, _P, _F, _P] + [_I] * 12 + [_P, _I, _P]),
    ("flygemm_moe_blockscale_gemm1", ctypes.c_int, [_P, _P, _P, _F, _F, _P, _P, _F, _P] + [_I] * 11 + [_P]),
    ("flygemm_moe_blockscale_gemm2", ctypes.c_int, [_P, _P, _P, _F, _F, _P, _P, _F, _P] + [_I] * 12 + [_P]),
    ("flygemm_num_variants", ctypes.c_int32, []),
    ("flygemm_variant_name", ctypes.c_char_p, [_I]),
    ("flygemm_select_variant", ctypes.c_int32, [_I, _I, _I, _I, _I]),
    ("flygemm_launch_shape", ctypes.c_int, [_I] * 6 + [_P] * 4),
    ("flygemm_last_error", ctypes.c_char_p, []),
]

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"flydsl_amd HIP library not built ({path} missing); run `python -m flydsl_amd.build`"
        )
    lib = ctypes.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().flygemm_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def variants() -> list[str]:
    lib = load()
    return [lib.flygemm_variant_name(i).decode() for i in range(lib.flygemm_num_variants())]
