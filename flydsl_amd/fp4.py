"""MXFP4 wire format: e2m1 values two per byte, one E8M0 scale per 32 elements of K.

Host (torch) helpers that produce exactly the bytes the reference's harness feeds its MXFP4
GEMM (``tests/kernels/utils/fp4_utils.py``), so weights and activations prepared for the
reference work unchanged:

* ``per_1x32_f4_quant(x)`` (reference ``:656-687``): per 32-element block,
  ``scale = e8m0(amax / 4)`` where 4 = 2**floor(log2(6)) and the E8M0 conversion rounds the
  fp32 exponent up when the significand is >= 1.5 (``f32_to_e8m0``, ``:52-61``); then
  ``q = e2m1(x / 2**(scale - 127))`` rounded to nearest even and saturated at 6
  (``_f32_to_floatx_unpacked``, ``:123-239``); element 2j in the low nibble (``:103-108``).
* ``mxfp4_to_f32`` / ``e8m0_to_f32`` (``:22-49``, ``:64-72``): E8M0 0 decodes to 2**-127 and
  0xFF to NaN.
* ``shuffle_weight_w4(b, 16, False, False)`` (``:578-621``): the packed [N, K/2] bytes viewed
  as ``(N/16, 16, K/128, 4, 16)`` and permuted to ``[n/16][kb/64][(kb/16)%4][n%16][kb%16]`` --
  the same permutation ``shuffle_weight`` applies to 1-byte elements.
* ``shuffle_scale_w4(s, 1, False)`` (``:624-653``): the [R, K/32] scale bytes viewed as
  ``(R/32, 2, 16, K/256, 2, 4)`` = (r1, rp, rl, k1, kp, kl) and permuted to
  ``[r1][k1][kl][rl][kp][rp]``: one 32-bit word per MFMA lane (kl*16 + rl) holding the scales
  of row blocks rp = 0/1 for K halves kp = 0/1 at byte ``2*kp + rp``.
"""
from __future__ import annotations

import torch

F4_MAX = 6.0
_E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def e8m0_from_f32(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> E8M0 byte: the biased exponent, plus one when the significand is >= 1.5
    (normal numbers) or when bit 22 and any lower bit are set (subnormals); NaN/inf -> 0xFF."""
    u = x.float().contiguous().view(torch.int32)
    e = (u >> 23) & 0xFF
    up = ((u & 0x400000) != 0) & (((u & 0x3FFFFF) != 0) | (e > 0))
    out = torch.where(e == 0xFF, torch.full_like(e, 0xFF), e + up.to(torch.int32))
    return out.to(torch.uint8)


def e8m0_to_f32(s: torch.Tensor) -> torch.Tensor:
    b = s.contiguous().view(torch.uint8).to(torch.int32)
    bits = b << 23
    bits = torch.where(b == 0, torch.full_like(bits, 0x00400000), bits)
    bits = torch.where(b == 0xFF, torch.full_like(bits, 0x7F800001), bits)
    return bits.view(torch.float32)


def e2m1_encode(y: torch.Tensor) -> torch.Tensor:
    """fp32 -> e2m1 code (uint8, low 4 bits), round to nearest even, saturating at +-6."""
    y = y.float()
    a = y.abs()
    step = torch.where(a < 2.0, torch.full_like(a, 0.5), torch.where(a < 4.0, torch.ones_like(a), torch.full_like(a, 2.0)))
    q = torch.clamp(torch.round(a / step) * step, max=F4_MAX)   # torch.round is half-to-even
    # magnitude -> 3-bit code
    mag = torch.zeros_like(q, dtype=torch.int32)
    for code, v in enumerate(_E2M1_VALUES):
        mag = torch.where(q == v, torch.full_like(mag, code), mag)
    sign = (y.view(torch.int32) < 0).to(torch.int32) << 3
    return (mag | sign).to(torch.uint8)


def pack_fp4(codes: torch.Tensor) -> torch.Tensor:
    """[..., 2n] e2m1 codes -> [..., n] bytes, element 2j in the low nibble."""
    c = codes.to(torch.uint8)
    return (c[..., 0::2] & 0xF) | ((c[..., 1::2] & 0xF) << 4)


def mxfp4_to_f32(x: torch.Tensor) -> torch.Tensor:
    """[..., n] packed bytes -> [..., 2n] fp32 values."""
    b = x.contiguous().view(torch.uint8)
    codes = torch.stack([b & 0xF, b >> 4], dim=-1).reshape(*b.shape[:-1], -1).long()
    table = torch.tensor(list(_E2M1_VALUES) + [-v for v in _E2M1_VALUES], dtype=torch.float32, device=b.device)
    return table[codes]


def per_1x32_f4_quant(x: torch.Tensor):
    """MXFP4 quantization of the last dimension (a multiple of 32): returns (packed bytes
    [..., K/2] uint8, E8M0 scales [rows, K/32] uint8, the scaled values before rounding)."""
    shape = x.shape
    xb = x.float().reshape(-1, 32)
    amax = xb.abs().amax(dim=1)
    scale = e8m0_from_f32(amax / 4.0)
    y = xb / e8m0_to_f32(scale).view(-1, 1)
    q = pack_fp4(e2m1_encode(y)).reshape(*shape[:-1], shape[-1] // 2)
    rows = xb.shape[0] * 32 // shape[-1]
    return q, scale.view(rows, shape[-1] // 32), y.reshape(shape)


def shuffle_weight_w4(src: torch.Tensor, NLane: int = 16, gate_up: bool = False, moe_gemm: bool = False):
    """Preshuffle packed MXFP4 weights [N, K/2] (dense GEMM form of the reference function)."""
    if moe_gemm or gate_up or NLane != 16:
        raise NotImplementedError("only the dense GEMM layout (NLane=16, gate_up=False, moe_gemm=False) is built")
    u = src.contiguous().view(torch.uint8)
    N, kb = u.shape
    if N % 16 or kb % 64:
        raise ValueError(f"packed weight shape [{N}, {kb}] needs N % 16 == 0 and (K/2) % 64 == 0")
    t = u.view(N // 16, 16, kb // 64, 4, 16).permute(0, 2, 3, 1, 4).contiguous()
    return t.view(N, kb).view(src.dtype)


def shuffle_scale_w4(src: torch.Tensor, experts_cnt: int = 1, gate_up: bool = False):
    """Shuffle E8M0 scales [R, K/32] (R % 32 == 0, K % 256 == 0) into per-lane 32-bit words."""
    if experts_cnt != 1 or gate_up:
        raise NotImplementedError("only experts_cnt=1, gate_up=False is built")
    u = src.contiguous().view(torch.uint8)
    R, ks = u.shape
    if R % 32 or ks % 8:
        raise ValueError(f"scale shape [{R}, {ks}] needs rows % 32 == 0 and (K/32) % 8 == 0")
    t = u.view(R // 32, 2, 16, ks // 8, 2, 4).permute(0, 3, 5, 2, 4, 1).contiguous()
    return t.view(R, ks).view(src.dtype)
