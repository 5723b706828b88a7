"""B-operand byte layouts (test infrastructure only).

* ``shuffle_weight`` restates reference ``tests/utils.py:76-96`` for 1-byte elements and
  ``layout=(16, 16)``: ``view(N/16, 16, K/32, 2, 16).permute(0, 1, 3, 4, 2, 5)`` of the
  [N, K] bytes, i.e. byte (n, k) moves to ``[n//16][k//16][n%16][k%16]``.  The device view
  the reference builds on it is ``(N/16, K/64, 4, 16, 16)`` with strides
  ``(16K, 1024, 256, 16, 1)`` (``kernels/preshuffle_gemm.py:226-241``).
* ``pack_int4`` restates ``_pack_shuffled_int8_to_packed_int4_no_perm``
  (``tests/kernels/test_preshuffle_gemm.py:165-174``): every 8 shuffled int8 values
  u0..u7 become 4 bytes ``(u_j & 0xF) | (u_{j+4} & 0xF) << 4``.
* ``unpack_int4`` restates the in-register unpack of
  ``kernels/mfma_preshuffle_pipeline.py:277-291``.

Pins (``tests/test_oracle.py``): brute-force index loop on small shapes, invertibility of
the shuffle, exhaustive pack/unpack round trip over all 16 nibble values in every position.
"""
from __future__ import annotations

import numpy as np


def shuffle_weight(b: np.ndarray) -> np.ndarray:
    """[N, K] 1- or 2-byte elements -> the preshuffled bytes (returned flat, uint8 for 2-byte
    input).  For 2-byte elements the reference groups 8 elements per 16-byte chunk
    (``tests/utils.py:83-90``), which is the 1-byte rule applied to each row's 2K bytes."""
    b = np.ascontiguousarray(b)
    N, K = b.shape
    assert N % 16 == 0 and K % 32 == 0
    if b.dtype.itemsize == 2:
        b = b.view(np.uint8).reshape(N, 2 * K)
        K = 2 * K
    assert b.dtype.itemsize == 1
    t = b.reshape(N // 16, 16, K // 32, 2, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(t).reshape(-1)


def unshuffle_weight(flat: np.ndarray, N: int, K: int) -> np.ndarray:
    t = np.asarray(flat).reshape(N // 16, K // 32, 2, 16, 16).transpose(0, 3, 1, 2, 4)
    return np.ascontiguousarray(t).reshape(N, K)


def shuffle_index(n: int, k: int, K: int) -> int:
    """Flat byte offset of B[n, k] in the preshuffled buffer."""
    return (n // 16) * 16 * K + (k // 16) * 256 + (n % 16) * 16 + (k % 16)


def pack_int4(shuffled_i8: np.ndarray) -> np.ndarray:
    u = (np.asarray(shuffled_i8).view(np.int8).astype(np.int16) & 0xF).astype(np.uint8).reshape(-1, 8)
    out = u[:, 0:4] | (u[:, 4:8] << 4)
    return np.ascontiguousarray(out).reshape(-1).view(np.int8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of ``pack_int4`` using the device bit trick on little-endian int32 words."""
    p = np.asarray(packed).view(np.int8).view(np.uint32).astype(np.uint64)
    even = (p & 0x0F0F0F0F) | (((p & 0x08080808) * 0x1E) & 0xFFFFFFFF)
    t = p >> 4
    odd = (t & 0x0F0F0F0F) | (((t & 0x08080808) * 0x1E) & 0xFFFFFFFF)
    words = np.stack([even, odd], axis=1).astype(np.uint32)   # per packed word: 8 int8
    return words.reshape(-1).view(np.int8)
