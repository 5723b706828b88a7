"""Argument plumbing shared by the launchers: tensors -> device pointers, stream -> handle.

Follows the reference's calling convention (``tests/kernels/test_preshuffle_gemm.py:193-207``,
``python/flydsl/compiler/jit_argument.py:145-156``, ``python/flydsl/expr/typing.py:302-338``):
flat contiguous tensors whose data pointer is passed bare (fp8 may be passed as int8 views),
a stream given as ``torch.cuda.Stream``, a raw integer handle, or ``None`` (default stream).
"""
from __future__ import annotations

import torch


def stream_handle(stream) -> int:
    if stream is None:
        return 0
    if isinstance(stream, int):
        return stream
    handle = getattr(stream, "cuda_stream", None)
    if handle is None:
        raise TypeError(f"stream must be a torch.cuda.Stream, an int handle or None, got {type(stream).__name__}")
    return int(handle)


def device_ptr(t, name: str, min_elems: int, elem_bytes: int | None = None, dtypes=None) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor, got device {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtypes is not None and t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {[str(d) for d in dtypes]}")
    if elem_bytes is not None and t.element_size() != elem_bytes:
        raise TypeError(f"{name} must have {elem_bytes}-byte elements, got {t.dtype}")
    if t.numel() < min_elems:
        raise ValueError(f"{name} has {t.numel()} elements, needs at least {min_elems}")
    return t.data_ptr()
