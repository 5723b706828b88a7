"""CPU-only tests of the host side: the C-ABI library loads and exports every declared
symbol, the drop-in entry points validate arguments like the reference, the variant
table and workload arithmetic are what the kernels and the measurements assume.  No
GPU compute is launched here."""
import ctypes
import os
import re

import pytest
import torch

from flydsl_amd import _lib, workloads
from flydsl_amd.kernels.blockscale_preshuffle_gemm import compile_blockscale_preshuffle_gemm
from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8, compile_preshuffle_gemm_w4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "flygemm.h")).read()
    return sorted(set(re.findall(r"\b(flygemm_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_symbols()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert bound == set(names)


def test_variant_table():
    names = _lib.variants()
    assert any(n.startswith("main_") for n in names) and any(n.startswith("decode_") for n in names)
    lib = _lib.load()
    assert names[lib.flygemm_select_variant(16, 28672, 8192, 0, 0)].startswith("decode_m1")
    assert names[lib.flygemm_select_variant(4096, 4096, 4096, 1, 0)].startswith("main_")
    # every shape gets a variant, and the five configurations get the tiles measured fastest
    expect = {(128, 4096, 4096, 0, 0): "rows_m2_nb4_w8_u3", (16, 28672, 8192, 0, 0): "decode_m1_nb7_w4_u2",
              (4096, 4096, 4096, 1, 0): "main_256x256_w2x4", (1024, 7168, 7168, 0, 1): "main_128x256_w2x4",
              (256, 14336, 4096, 2, 0): "main_64x128_w1x4", (8192, 8192, 8192, 0, 0): "main_256x256_w2x4"}
    for args, want in expect.items():
        assert names[lib.flygemm_select_variant(*args)] == want, args
    # 17-64 rows: decode only up to 32 rows (16 for blockscale with 32+ column tiles); the
    # 64x128 tile above, or the row-blocked kernel when that gives few tiles
    assert names[lib.flygemm_select_variant(64, 28672, 8192, 0, 0)] == "main_64x128_w1x4"
    # 17-32 rows: the decode family's 4-wave 32-row forms, whatever N (not blockscale)
    assert names[lib.flygemm_select_variant(32, 28672, 8192, 0, 0)] == "decode_m2_nb4_w4_u2"
    assert names[lib.flygemm_select_variant(20, 40960, 5120, 0, 0)] == "decode_m2_nb4_w4_u2"
    assert names[lib.flygemm_select_variant(32, 28672, 8192, 2, 0)] == "decode_m2_nb4_w4_u2"
    assert names[lib.flygemm_select_variant(32, 18432, 7168, 3, 0)] == "decode_m2_nb2_w4_u4"
    assert names[lib.flygemm_select_variant(32, 4096, 4096, 1, 0)] == "decode_m2_nb1_w8_u4"
    assert names[lib.flygemm_select_variant(32, 8192, 8192, 1, 0)].startswith("decode_m2")
    assert names[lib.flygemm_select_variant(48, 8192, 8192, 1, 0)] == "rows_m2_nb4_w8_u3"   # 256 against 384
    assert names[lib.flygemm_select_variant(48, 4096, 4096, 0, 0)] == "rows_m1_nb4_w8_u3"   # 192 against 128
    assert names[lib.flygemm_select_variant(48, 7168, 2048, 0, 0)] == "rows_m2_nb4_w8_u3"   # 224 against 336
    assert names[lib.flygemm_select_variant(64, 7168, 2048, 2, 0)] == "rows_m2_nb4_w8_u3"  # 56 tiles
    assert names[lib.flygemm_select_variant(64, 8192, 8192, 3, 0)] == "rows_m2_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(32, 7168, 7168, 0, 1)] == "rows_m1_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(32, 2112, 7168, 0, 1)].startswith("decode_m2")
    assert names[lib.flygemm_select_variant(16, 7168, 7168, 0, 1)].startswith("decode_m1")
    # 65-144 tiles of 64x128: 64x64 tiles (twice the workgroups); at most 64: the row-blocked
    # kernel; above 144: 64x128; never 64x64 for MXFP4
    for args in [(256, 4096, 4096, 0, 0), (128, 8192, 8192, 0, 0), (192, 4096, 4096, 0, 0), (128, 7168, 2048, 1, 0),
                 (256, 4096, 4096, 3, 0), (128, 7168, 7168, 0, 1), (96, 8192, 8192, 0, 0)]:
        assert names[lib.flygemm_select_variant(*args)] == "main_64x64_w1x4", args
    assert names[lib.flygemm_select_variant(128, 4096, 4096, 1, 0)] == "rows_m2_nb4_w8_u3"    # 64 tiles
    assert names[lib.flygemm_select_variant(320, 4096, 4096, 0, 0)] == "main_64x128_w1x4"     # 160 tiles
    assert names[lib.flygemm_select_variant(256, 7168, 7168, 0, 0)] == "main_64x128_w1x4"     # 224 tiles
    assert names[lib.flygemm_select_variant(256, 4096, 4096, 5, 0)] == "main_64x128_w1x4"     # MXFP4
    # blockscale: 256x256 from 200 tiles, 256x128 from 160
    assert names[lib.flygemm_select_variant(2048, 7168, 7168, 0, 1)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(2048, 3072, 1536, 0, 1)] == "main_128x256_w2x4"
    assert names[lib.flygemm_select_variant(1024, 2112, 7168, 0, 1)] == "main_64x64_w1x4"   # 272 64x128 tiles
    assert names[lib.flygemm_select_variant(512, 4096, 7168, 0, 1)] == "main_64x64_w1x4"
    assert names[lib.flygemm_select_variant(512, 7168, 2304, 0, 1)] == "main_64x128_w1x4"   # 448 tiles
    # not 256x256 between one and two tiles per CU
    assert names[lib.flygemm_select_variant(1024, 24576, 1536, 0, 1)] == "main_128x256_w2x4"  # K < 4096
    assert names[lib.flygemm_select_variant(2048, 24576, 1536, 0, 1)] == "main_128x256_w2x4"  # K < 4096
    assert names[lib.flygemm_select_variant(1536, 7168, 7168, 0, 1)] == "main_256x256_w2x4"  # 168 tiles
    # 256x256 from about 160 tiles, then 128x128 from 272
    assert names[lib.flygemm_select_variant(1536, 8192, 8192, 0, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(512, 28672, 8192, 0, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(1024, 8192, 8192, 0, 0)] == "main_128x256_w2x4"
    # 128x128 once it gives more than one tile per CU, or for K below 4096 bytes (not MXFP4)
    assert names[lib.flygemm_select_variant(1024, 7168, 7168, 0, 0)] == "main_128x256_w2x4"
    assert names[lib.flygemm_select_variant(1024, 7168, 4096, 0, 0)] == "main_128x256_w2x4"
    assert names[lib.flygemm_select_variant(1024, 7168, 2048, 0, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(1024, 7168, 3072, 1, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(1024, 7168, 2048, 3, 0)] == "main_128x256_w2x4"   # 4096 bytes
    assert names[lib.flygemm_select_variant(1024, 7168, 1024, 3, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(1024, 7168, 7168, 5, 0)] == "main_128x256_w2x4"   # MXFP4
    assert names[lib.flygemm_select_variant(1024, 7168, 7168, 2, 0)] == "main_128x128_w2x2"  # int4: no 128x256
    # int4: 256x256 only from 600 such tiles
    assert names[lib.flygemm_select_variant(1536, 28672, 8192, 2, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(4096, 4096, 4096, 2, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(8192, 8192, 8192, 2, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(9728, 8192, 8320, 2, 0)] == "main_256x256_w2x4"
    # ... and with one round of them where N >= 16M; 64x128 for 129-192 rows
    assert names[lib.flygemm_select_variant(512, 28672, 8192, 2, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(384, 28672, 8192, 2, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(768, 28672, 8192, 2, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(1024, 14336, 4096, 2, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(192, 28672, 8192, 2, 0)] == "main_64x128_w1x4"
    assert names[lib.flygemm_select_variant(256, 28672, 8192, 2, 0)] == "main_128x128_w2x2"
    assert names[lib.flygemm_select_variant(1280, 7168, 7168, 0, 0)] == "main_128x128_w2x2"  # 280 tiles of 128x256
    assert names[lib.flygemm_select_variant(1024, 4096, 4096, 0, 0)] == "main_64x128_w1x4"
    # 145-256 tiles of 64x128 and at least 384 rows: 128x64 tiles (not int4, MXFP4, blockscale)
    assert names[lib.flygemm_select_variant(512, 4096, 7168, 0, 0)] == "main_128x64_w2x2"
    assert names[lib.flygemm_select_variant(384, 5120, 7168, 1, 0)] == "main_128x64_w2x2"
    assert names[lib.flygemm_select_variant(512, 4096, 4096, 3, 0)] == "main_128x64_w2x2"
    # 129-192 rows, or 65-128 rows with at least 96 MB of B: 128x64 rather than 64x128 (not int4,
    # MXFP4, blockscale)
    for args, want in {(144, 14336, 4096, 0, 0): "main_128x64_w2x2", (192, 14336, 4096, 1, 0): "main_128x64_w2x2",
                       (160, 14336, 4096, 3, 0): "main_128x64_w2x2", (192, 8192, 8192, 4, 0): "main_128x64_w2x2",
                       (96, 28672, 8192, 0, 0): "main_128x64_w2x2", (112, 14336, 4096, 3, 0): "main_128x64_w2x2",
                       (96, 14336, 4096, 0, 0): "main_64x128_w1x4", (224, 14336, 4096, 0, 0): "main_64x128_w1x4",
                       (192, 14336, 4096, 5, 0): "main_64x128_w1x4", (192, 14336, 4096, 2, 0): "main_64x64_w1x4_k2",
                       (192, 14336, 7168, 0, 1): "main_64x128_w1x4"}.items():
        assert names[lib.flygemm_select_variant(*args)] == want, args
    # 129-256 rows: 256x128 where the list gives 128x256 (B read by one row block, not two)
    for args in [(144, 28672, 8192, 0, 0), (256, 28672, 8192, 1, 0), (192, 28672, 8192, 3, 0),
                 (160, 28672, 8192, 5, 0)]:
        assert names[lib.flygemm_select_variant(*args)] == "main_256x128_w2x4", args
    assert names[lib.flygemm_select_variant(384, 28672, 8192, 0, 0)] == "main_256x256_w2x4"
    assert names[lib.flygemm_select_variant(512, 14336, 4096, 0, 0)] == "main_256x128_w2x4"
    assert names[lib.flygemm_select_variant(512, 14336, 4096, 3, 0)] == "main_256x128_w2x4"
    assert names[lib.flygemm_select_variant(1024, 8192, 8192, 0, 0)] == "main_128x256_w2x4"
    # above 192 rows with K of at least 8192 bytes: 128x64 rather than 64x128
    for args, want in {(384, 8192, 8192, 0, 0): "main_128x64_w2x2", (640, 4096, 4096, 3, 0): "main_128x64_w2x2",
                       (640, 4096, 4096, 0, 0): "main_64x128_w1x4", (512, 7168, 2048, 3, 0): "main_64x128_w1x4",
                       (256, 7168, 7168, 0, 0): "main_64x128_w1x4", (1536, 2112, 7168, 3, 0): "main_64x128_w1x4",
                       (1024, 4096, 4096, 3, 0): "main_128x64_w2x2"}.items():
        assert names[lib.flygemm_select_variant(*args)] == want, args
    # int4 with 65-512 tiles of 64x128: two K tiles per step -- 64x64 tiles up to 352, 64x128
    # tiles above with K of at least 8192 (the one-K-tile 64x128 below that)
    for args, want in {(256, 4096, 4096, 2, 0): "main_64x64_w1x4_k2", (512, 4096, 4096, 2, 0): "main_64x64_w1x4_k2",
                       (64, 14336, 4096, 2, 0): "main_64x64_w1x4_k2", (320, 8192, 8192, 2, 0): "main_64x64_w1x4_k2",
                       (256, 14336, 8192, 2, 0): "main_64x128_w1x4_k2", (256, 14336, 4096, 2, 0): "main_64x128_w1x4",
                       (128, 4096, 4096, 2, 0): "rows_m2_nb4_w8_u3", (512, 14336, 8192, 2, 0): "main_128x128_w2x2",
                       (256, 4096, 4096, 0, 0): "main_64x64_w1x4"}.items():
        assert names[lib.flygemm_select_variant(*args)] == want, args
    assert names[lib.flygemm_select_variant(320, 4096, 4096, 0, 0)] == "main_64x128_w1x4"   # ragged 128-row tiles
    assert names[lib.flygemm_select_variant(768, 4096, 4096, 0, 0)] == "main_64x128_w1x4"   # 384 tiles
    # the row-blocked kernel where the 64x128 tiles leave CUs idle (at most 64 tiles; 96 with
    # the 16-row blocks of blockscale and MXFP4)
    assert names[lib.flygemm_select_variant(128, 4096, 4096, 0, 0)] == "rows_m2_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(128, 4096, 1024, 1, 0)] == "rows_m2_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(256, 8192, 4096, 0, 0)] == "main_64x128_w1x4"
    assert names[lib.flygemm_select_variant(128, 4096, 4096, 0, 1)] == "rows_m1_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(256, 2112, 7168, 0, 1)] == "rows_m1_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(33, 2112, 7168, 0, 1)] == "rows_m1_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(128, 4096, 4096, 5, 0)] == "rows_m1_nb4_w8_u3"
    assert names[lib.flygemm_select_variant(128, 4096, 2048, 3, 0)] == "rows_m2_nb4_w8_u3"  # 2 bytes/elt
    # decode of one 16-row block (fp8 / int8 / int4 codes): the most column blocks per workgroup
    # whose workgroups fill their last round over 256 CUs to at least 75%; 4-wave workgroups for
    # fp8 / int8 with 2+ blocks, ten blocks only for int4 (half-size blocks)
    dec = {(16, 14336, 4096, 2): "nb4_w8_u3", (16, 14336, 4096, 1): "nb4_w4_u4", (16, 40960, 5120, 0): "nb5_w4_u3",
           (16, 40960, 5120, 1): "nb5_w4_u3", (16, 40960, 5120, 2): "nb10_w8_u2", (16, 77824, 5120, 0): "nb7_w4_u2",
           (16, 77824, 5120, 2): "nb10_w8_u2", (16, 24576, 8192, 0): "nb7_w4_u2", (16, 7168, 2048, 0): "nb2_w4_u4",
           (16, 4096, 4096, 1): "nb1_w8_u4", (1, 57344, 8192, 0): "nb7_w4_u2", (16, 28672, 8192, 2): "nb7_w8_u2",
           (16, 12288, 4096, 0): "nb4_w4_u4", (16, 12288, 4096, 2): "nb4_w8_u3", (16, 28672, 8192, 1): "nb7_w4_u2"}
    for (m, n, k, ind), want in dec.items():
        assert names[lib.flygemm_select_variant(m, n, k, ind, 0)] == f"decode_m1_{want}", (m, n, k, ind)
    # the same rule for 16-bit inputs and blockscale; MXFP4 at most two blocks, on 4 waves only
    # above 256 workgroups
    more = {(16, 40960, 5120, 3, 0): "nb5_w4_u3", (16, 18432, 7168, 4, 0): "nb5_w4_u3",
            (16, 36864, 7168, 0, 1): "nb5_w4_u3", (16, 7168, 7168, 0, 1): "nb2_w4_u4",
            (16, 28672, 8192, 5, 0): "nb2_w4_u4", (16, 8192, 8192, 5, 0): "nb2_w8_u4",
            (16, 4096, 4096, 5, 0): "nb1_w8_u4"}
    for (m, n, k, ind, bs), want in more.items():
        assert names[lib.flygemm_select_variant(m, n, k, ind, bs)] == f"decode_m1_{want}", (m, n, k, ind, bs)
    # without a choice that fills 75% of the last round: the most blocks leaving 240 workgroups
    # (blockscale 16x2112x7168: 132 blocks)
    assert names[lib.flygemm_select_variant(16, 2112, 7168, 0, 1)] == "decode_m1_nb1_w8_u4"
    for m in (1, 17, 64, 65, 100, 1000, 5000):
        for n in (16, 128, 2048, 30000):
            for bs in (0, 1):
                assert 0 <= lib.flygemm_select_variant(m, n, 1024, 0, bs) < len(names)
    assert lib.flygemm_variant_name(-1) is None and lib.flygemm_variant_name(len(names)) is None


def test_abi_rejects_bad_arguments_before_launch():
    """Validation returns an error code and message without touching the GPU."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 16, 100, 256, 0, 0, -1, None)
    assert rc != 0 and b"multiple of 16" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 16, 128, 200, 0, 0, -1, None)
    assert rc != 0 and b"multiple of 64" in lib.flygemm_last_error()
    # K = 64 (mod 128) is accepted for 1-byte inputs (a last half K tile); blockscale keeps 128
    assert lib.flygemm_preshuffle(p, p, p, p, p, 0, 128, 192, 1, 0, -1, None) == 0
    rc = lib.flygemm_blockscale(p, p, p, p, p, 16, 128, 192, 128, 0, -1, None)
    assert rc != 0 and b"multiple of scale_block_k" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle(None, p, p, p, p, 16, 128, 256, 0, 0, -1, None)
    assert rc != 0 and b"null" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 16, 128, 256, 7, 0, -1, None)
    assert rc != 0 and b"in_dtype" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 16, 128, 256, 0, 0, 99, None)
    assert rc != 0 and b"variant" in lib.flygemm_last_error()
    # a variant index past the table (including the old split-count bits) is rejected
    names = _lib.variants()
    plain = names.index("main_64x128_w1x4")
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 100, 128, 1024, 0, 0, plain | (2 << 16), None)
    assert rc != 0 and b"unknown variant" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 100, 128, 1024, 0, 0, -2, None)
    assert rc != 0 and b"unknown variant" in lib.flygemm_last_error()
    rc = lib.flygemm_blockscale(p, p, p, p, p, 16, 128, 256, 64, 0, -1, None)
    assert rc != 0 and b"scale_block_k" in lib.flygemm_last_error()
    rc = lib.flygemm_accumulators(p, p, p, -1, 128, 256, 0, -1, None)
    assert rc != 0 and b"invalid sizes" in lib.flygemm_last_error()
    # M == 0 is a no-op that succeeds without launching
    assert lib.flygemm_preshuffle(p, p, p, p, p, 0, 128, 256, 0, 0, -1, None) == 0
    # int4 weights take K < 131072: their int32 accumulators hold 16x the dot product, and
    # 16 * 1024 * 131072 (every product (-128) * (-8)) would reach 2^31
    rc = lib.flygemm_preshuffle(p, p, p, p, p, 16, 16, 131072, 2, 0, -1, None)
    assert rc != 0 and b"int4 weights take K < 131072" in lib.flygemm_last_error()
    rc = lib.flygemm_accumulators(p, p, p, 16, 16, 131072, 2, -1, None)
    assert rc != 0 and b"int4 weights take K < 131072" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle_quant_a(p, p, p, p, p, p, 16, 16, 131072, 0, 2, 0, 0, -1, None)
    assert rc != 0 and b"int4 weights take K < 131072" in lib.flygemm_last_error()
    assert lib.flygemm_preshuffle(p, p, p, p, p, 0, 16, 131072 - 64, 2, 0, -1, None) == 0
    # per-row quantization
    rc = lib.flygemm_quant_rows(p, p, p, 4, 12, 0, 1, 0, None)
    assert rc != 0 and b"multiple of 8" in lib.flygemm_last_error()
    rc = lib.flygemm_quant_rows(p, p, p, 4, 64, 0, 0, 1, None)
    assert rc != 0 and b"fp8 output rounds to nearest" in lib.flygemm_last_error()
    rc = lib.flygemm_quant_rows(p, p, p, 4, 64, 3, 1, 0, None)
    assert rc != 0 and b"in_dtype" in lib.flygemm_last_error()
    rc = lib.flygemm_quant_rows(ctypes.c_void_p(17), p, p, 4, 64, 0, 1, 0, None)
    assert rc != 0 and b"misaligned" in lib.flygemm_last_error()
    # the GEMM that quantizes its activations checks its buffers and their alignment before its
    # first launch: x 16 bytes, a_q 8, scale_a 4; the code and scale buffers are required
    for x, aq, sa in [(ctypes.c_void_p(24), p, p), (p, ctypes.c_void_p(20), p), (p, p, ctypes.c_void_p(18))]:
        rc = lib.flygemm_preshuffle_quant_a(p, aq, sa, x, p, p, 16, 128, 256, 0, 1, 0, 0, -1, None)
        assert rc != 0 and b"misaligned" in lib.flygemm_last_error()
    rc = lib.flygemm_preshuffle_quant_a(p, None, None, p, p, p, 16, 128, 256, 0, 1, 0, 0, -1, None)
    assert rc != 0 and b"required" in lib.flygemm_last_error()
    assert lib.flygemm_quant_rows(p, p, p, 0, 64, 0, 1, 0, None) == 0
    # 16-bit inputs: K counts elements and must be a multiple of 32; scales are not needed
    rc = lib.flygemm_preshuffle(p, p, p, None, None, 16, 128, 80, 3, 0, -1, None)
    assert rc != 0 and b"multiple of 32" in lib.flygemm_last_error()
    assert lib.flygemm_preshuffle(p, p, p, None, None, 0, 128, 96, 4, 0, -1, None) == 0
    # MXFP4
    rc = lib.flygemm_mxfp4(p, p, p, p, p, 16, 128, 384, 0, -1, None)
    assert rc != 0 and b"multiple of 256" in lib.flygemm_last_error()
    rc = lib.flygemm_mxfp4(p, p, p, p, p, 16, 48, 512, 0, -1, None)
    assert rc != 0 and b"multiple of 32" in lib.flygemm_last_error()
    rc = lib.flygemm_mxfp4(p, p, p, None, p, 16, 128, 512, 0, -1, None)
    assert rc != 0 and b"null scale" in lib.flygemm_last_error()
    assert lib.flygemm_mxfp4(p, p, p, p, p, 0, 128, 512, 2, -1, None) == 0


@pytest.mark.parametrize("kw, exc", [
    (dict(in_dtype="fp32"), ValueError),
    (dict(out_dtype="fp32"), ValueError),
    (dict(tile_k=17), ValueError),          # the reference AOT example's bad tile (aot_example.py:226-240)
    (dict(tile_k=32), ValueError),          # tile_k bytes not a multiple of 64
    (dict(tile_m=8), ValueError),           # tile_m*tile_k not a multiple of 256
    (dict(in_dtype="fp8", tile_k=64), ValueError),  # gfx950 fp8 needs tile_k % 128 == 0
    (dict(lds_stage=3), ValueError),
])
def test_compile_validation_matches_reference(kw, exc):
    args = dict(K=4096, tile_m=64, tile_n=128, tile_k=128, in_dtype="int8", out_dtype="bf16")
    args.update(kw)
    with pytest.raises(exc):
        compile_preshuffle_gemm_a8(**args)


def test_w4_entry_and_unbuilt_dtypes():
    with pytest.raises(NotImplementedError):
        compile_preshuffle_gemm_w4(K=256, tile_m=64, tile_n=128, tile_k=128, a_dtype="fp8")
    fn = compile_preshuffle_gemm_w4(K=256, tile_m=64, tile_n=128, tile_k=128)
    with pytest.raises(ValueError, match="GPU tensor"):
        fn(torch.empty(16 * 128, dtype=torch.bfloat16), torch.empty(16 * 128, dtype=torch.uint8),
           torch.empty(128 * 128, dtype=torch.uint8), torch.empty(32 * 8, dtype=torch.uint8),
           torch.empty(128 * 8, dtype=torch.uint8), 16, 128, None)
    with pytest.raises(ValueError, match="multiple of 32"):
        fn(None, None, None, None, None, 16, 112, None)
    fn = compile_preshuffle_gemm_a8(K=256, tile_m=64, tile_n=128, tile_k=128, in_dtype="fp16")
    with pytest.raises(ValueError, match="GPU tensor"):
        fn(torch.empty(16 * 128, dtype=torch.float16), torch.empty(16 * 256, dtype=torch.float16),
           torch.empty(128 * 256, dtype=torch.float16), None, None, 16, 128, None)
    # bf16 is built: host tensors are rejected by the argument checks, before any launch
    fn = compile_preshuffle_gemm_a8(K=256, tile_m=64, tile_n=128, tile_k=128, in_dtype="bf16")
    x = torch.empty(16 * 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        fn(torch.empty(16 * 128, dtype=torch.bfloat16), x, x, None, None, 16, 128, None)


def test_launcher_rejects_host_tensors_and_bad_shapes():
    fn = compile_preshuffle_gemm_a8(K=256, tile_m=64, tile_n=128, tile_k=128, in_dtype="fp8", out_dtype="bf16")
    c = torch.empty(16 * 128, dtype=torch.bfloat16)
    a = torch.empty(16 * 256, dtype=torch.int8)
    b = torch.empty(128 * 256, dtype=torch.int8)
    s = torch.empty(128, dtype=torch.float32)
    with pytest.raises(ValueError, match="GPU tensor"):
        fn(c, a, b, s, s, 16, 128, None)
    with pytest.raises(ValueError, match="multiple of 16"):
        fn(c, a, b, s, s, 16, 120, None)
    with pytest.raises(TypeError):
        fn(c, a, b, s, s, 16, 128, "stream")


def test_blockscale_compile_validation():
    with pytest.raises(ValueError):
        compile_blockscale_preshuffle_gemm(K=7168, tile_m=64, tile_n=128, tile_k=128, scale_block_k=64)
    with pytest.raises(ValueError):
        compile_blockscale_preshuffle_gemm(K=7168, tile_m=64, tile_n=128, tile_k=192)
    compile_blockscale_preshuffle_gemm(K=7168, tile_m=64, tile_n=128, tile_k=128)


def test_workload_arithmetic_matches_baseline():
    W = workloads.WORKLOADS
    assert round(W["C2"].bytes / 1e6, 3) == 236.044
    assert round(W["C1"].bytes / 1e6, 3) == 18.367
    assert round(W["C4"].bytes / 1e6, 3) == 73.642
    assert round(W["C5"].bytes / 1e6, 3) == 37.807
    assert W["T"].flops == 2 * 8192 ** 3


def test_small_operands_roundtrip_through_oracle():
    """Product preparation (quantize, shuffle, pack) agrees with the oracle's restatement."""
    import numpy as np
    from oracle import layout as ol, quant as oq
    w = workloads.custom("int4", 32, 64, 256, seed=11, b_std=0.02)
    ops = workloads.make_operands(w)
    b = ops["b"].numpy()
    assert np.array_equal(ops["b_dev"].numpy(), ol.pack_int4(ol.shuffle_weight(b)))
    assert np.array_equal(ol.unpack_int4(ops["b_dev"].numpy()), ol.shuffle_weight(b))
    g = torch.Generator().manual_seed(11)
    a32 = torch.randn(32, 256, generator=g)
    q, s = oq.quant_rows(a32.numpy(), "int8")
    assert np.array_equal(ops["a"].numpy(), q)


def test_moe_abi_rejects_bad_arguments_before_launch():
    lib = _lib.load()
    p = ctypes.c_void_p(256)

    def s1(**kw):
        a = dict(tokens=64, inter=128, model=256, blocks=12, experts=4, topk=2, tile_m=16, tile_n=64, in_dtype=0,
                 out_dtype=1, doweight=0, group=-1, sw=p)
        a.update(kw)
        return lib.flygemm_moe_gemm1(p, p, p, p, a["sw"], p, p, p, p, a["tokens"], a["inter"], a["model"], a["blocks"],
                                     a["experts"], a["topk"], a["tile_m"], a["tile_n"], a["in_dtype"], a["out_dtype"],
                                     a["doweight"], a["group"], None)

    def err():
        return lib.flygemm_last_error()

    assert s1(tile_m=48) != 0 and b"tile_m" in err()
    assert s1(tile_n=96) != 0 and b"tile_n" in err()
    assert s1(inter=192, tile_n=128) != 0 and b"multiple of tile_n" in err()
    assert s1(model=200) != 0 and b"128-byte K tile" in err()
    assert s1(in_dtype=3, model=96) != 0 and b"multiple of 64" in err()
    assert s1(in_dtype=9) != 0 and b"in_dtype" in err()
    # group scales: int4_bf16 (W4A16) with 32-element groups only; W4A16 needs its weight scales
    assert s1(group=32) != 0 and b"group" in err()
    assert s1(in_dtype=6, group=64) != 0 and b"group" in err()
    assert s1(in_dtype=6, sw=None) != 0 and b"null scale" in err()
    assert s1(in_dtype=6, model=96) != 0 and b"multiple of 64" in err()
    assert s1(out_dtype=2) != 0 and b"out_dtype" in err()       # stage 1 has no fp32 output
    assert s1(topk=0) != 0 and b"topk" in err()
    assert s1(tokens=1 << 24) != 0 and b"2^24" in err()
    assert s1(tokens=0) == 0 and s1(blocks=0) == 0                # nothing to do
    assert s1(in_dtype=2, model=131072) != 0 and b"int4 weights take K < 131072" in err()
    rc = lib.flygemm_moe_gemm2(p, p, p, None, p, p, p, p, p, 64, 256, 128, 12, 4, 2, 16, 64, 0, 2, 1, 1, -1, None)
    assert rc != 0 and b"null scale" in err()
    rc = lib.flygemm_moe_gemm2(p, p, p, None, None, p, p, None, p, 64, 256, 128, 12, 4, 2, 16, 64, 3, 2, 1, 1, -1,
                               None)
    assert rc != 0 and b"sorted_weights" in err()
    # reduce mode (accumulate == 0) writes fp16/bf16 rows only
    rc = lib.flygemm_moe_gemm2(p, p, p, p, p, p, p, p, p, 64, 256, 128, 12, 4, 2, 16, 64, 0, 2, 1, 0, -1, None)
    assert rc != 0 and b"without accumulation" in err()
    # a per-expert weight slab above 2^31 bytes is refused
    rc = lib.flygemm_moe_gemm2(p, p, p, p, p, p, p, p, p, 8, 65536, 65536, 12, 4, 2, 16, 256, 0, 2, 0, 1, -1, None)
    assert rc != 0 and b"2^31" in err()
    # the reduction
    assert lib.flygemm_moe_reduce(p, p, None, 4, 2, 100, 1, None) != 0 and b"multiple of 8" in err()
    assert lib.flygemm_moe_reduce(p, p, None, 4, 0, 128, 1, None) != 0 and b"invalid sizes" in err()
    assert lib.flygemm_moe_reduce(p, p, None, 4, 2, 128, 7, None) != 0 and b"dtype" in err()
    assert lib.flygemm_moe_reduce(ctypes.c_void_p(8), p, None, 4, 2, 128, 1, None) != 0 and b"misaligned" in err()
    assert lib.flygemm_moe_reduce(p, p, None, 0, 2, 128, 1, None) == 0
    # the no-alloc stage 2 + reduction checks everything before its first launch and before it
    # looks up its scratch (which needs a device): here, without one, the argument errors come back

    def noalloc(out=p, tile_n=64, tokens=64):
        return lib.flygemm_moe_gemm2_reduce_noalloc(out, p, p, p, p, p, p, p, p, tokens, 256, 128, 12, 4, 2, 16,
                                                    tile_n, 0, 1, 0, -1, None, 1, None)
    assert noalloc(tile_n=96) != 0 and b"tile_n" in err()
    assert noalloc(out=ctypes.c_void_p(264)) != 0 and b"misaligned output" in err()
    assert noalloc(out=None) != 0 and b"null output" in err()
    assert noalloc(tokens=0) == 0


def test_moe_launchers_validate_like_reference():
    from flydsl_amd.kernels.moe_gemm_2stage import compile_moe_gemm1, compile_moe_gemm2
    kw = dict(model_dim=256, inter_dim=128, experts=4, topk=2, tile_m=16, tile_n=64, tile_k=128)
    with pytest.raises(ValueError):
        compile_moe_gemm1(**kw, doweight_stage1=False, in_dtype="fp32")
    with pytest.raises(ValueError):
        compile_moe_gemm1(**kw, doweight_stage1=False, out_dtype="f32")
    with pytest.raises(ValueError):
        compile_moe_gemm1(**{**kw, "tile_k": 32}, doweight_stage1=False)       # 32 bytes per K tile
    # every reference in_dtype compiles; group scales only for int4_bf16 with 32-element groups
    for dt in ("fp8", "fp16", "bf16", "int8", "int8smooth", "int4", "int4_bf16"):
        assert compile_moe_gemm1(**kw, doweight_stage1=False, in_dtype=dt).in_dtype == dt
    assert compile_moe_gemm2(**kw, doweight_stage2=True, in_dtype="int4_bf16", group_size=32).group_size == 32
    with pytest.raises(ValueError, match="group"):
        compile_moe_gemm1(**kw, doweight_stage1=False, in_dtype="bf16", group_size=32)
    with pytest.raises(ValueError):
        compile_moe_gemm2(**kw, doweight_stage2=True, out_dtype="f32", accumulate=False)
    from flydsl_amd.kernels.moe_gemm_2stage import MoeGemm2Mode, compile_moe_gemm2_ex, compile_moe_reduction
    assert compile_moe_gemm2_ex(**kw, doweight_stage2=True, mode=MoeGemm2Mode.REDUCE).mode == "reduce"
    assert not compile_moe_gemm2(**kw, doweight_stage2=True, accumulate=False).accumulate
    with pytest.raises(ValueError):
        compile_moe_reduction(topk=2, model_dim=100)
    with pytest.raises(ValueError):
        compile_moe_reduction(topk=2, model_dim=128, dtype_str="fp8")
    fn = compile_moe_gemm2(**kw, doweight_stage2=True, out_dtype="float")
    assert fn.out_dtype == "f32"
    c = torch.empty(64 * 256, dtype=torch.float32)
    b = torch.empty(4 * 256 * 128, dtype=torch.int8)
    s = torch.empty(4 * 256, dtype=torch.float32)
    i = torch.empty(200, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU tensor"):
        fn(c, b, b, s, s, i, i, s, i, 64, 256, 128, 12)


def test_moe_blockscale_validation():
    from flydsl_amd.kernels.moe_blockscale_2stage import (compile_moe_blockscale_gemm1, compile_moe_blockscale_gemm2,
                                                          compile_moe_blockscale_gemm2_ex)
    kw = dict(model_dim=512, inter_dim=128, experts=4, topk=2, tile_m=16, tile_n=64, tile_k=128)
    with pytest.raises(ValueError):
        compile_moe_blockscale_gemm1(**kw, doweight_stage1=False, scale_block_k=64)
    with pytest.raises(ValueError):
        compile_moe_blockscale_gemm1(**{**kw, "inter_dim": 96}, doweight_stage1=False)   # 2I % 128
    with pytest.raises(ValueError):
        compile_moe_blockscale_gemm2(**{**kw, "model_dim": 320}, doweight_stage2=True)  # model_dim % 128
    with pytest.raises(ValueError):
        compile_moe_blockscale_gemm2(**kw, doweight_stage2=True, out_dtype="f32", accumulate=False)
    with pytest.raises(ValueError):
        compile_moe_blockscale_gemm2_ex(**kw, doweight_stage2=True, in_dtype="int8")
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    rc = lib.flygemm_moe_blockscale_gemm1(p, p, p, p, p, p, p, p, p, 16, 128, 512, 6, 4, 2, 16, 64, 64, 1, 0, None)
    assert rc != 0 and b"scale_block_k" in lib.flygemm_last_error()
    rc = lib.flygemm_moe_blockscale_gemm2(p, p, p, p, p, p, p, p, p, 16, 320, 128, 6, 4, 2, 16, 64, 128, 1, 1, 1,
                                          None)
    assert rc != 0 and b"multiple of 128" in lib.flygemm_last_error()


def test_moe_tile_choice_pinned():
    """flygemm_moe_select_tile gives the launchers' tile choice without a device: stage 1 of
    1-byte, 16-bit and W4A8 weights runs the stream kernel (runs of 128 rows, 64 columns) but
    for large experts; W4A16 and blockscale stage 1 keep single-block tiles but blockscale's
    large experts of 16-row blocks; stage 2 takes runs for
    16-row blocks of prefill routings, 64 columns for decode-sized ones, wide single-block tiles
    in between (the reachable kernel set the GPU tests cover), and the launchers' validation."""
    import ctypes
    lib = _lib.load()

    def sel(stage, tokens, n, experts, topk, tile_m, tile_n, kind="fp8", bs=0, k=None):
        # k: the GEMM's depth, DS-TP8's by default (model_dim 7168 in stage 1, inter_dim 256 in 2)
        k = (7168 if stage == 1 else 256) if k is None else k
        r, tn = ctypes.c_int32(), ctypes.c_int32()
        rc = lib.flygemm_moe_select_tile(stage, tokens, n, k, experts, topk, tile_m, tile_n, _lib.FLYGEMM_IN[kind],
                                         bs, ctypes.byref(r), ctypes.byref(tn))
        return (r.value, tn.value) if rc == 0 else rc

    # stage 1 stream kernel: 128 / tile_m blocks per run, 64 columns, whatever the routing and the
    # caller's tile_n
    for kind in ("fp8", "int8", "bf16", "fp16", "int8smooth", "int4"):
        for tokens, n, experts, topk in ((8192, 256, 128, 8), (8, 256, 256, 8), (160, 1024, 64, 4), (64, 256, 4, 2)):
            for tm in (16, 32, 64):
                assert sel(1, tokens, n, experts, topk, tm, 256, kind) == (128 // tm, 64), (kind, tokens, tm)
    # stage 2 (accumulating calls) on DS-TP8 prefill: 64-column single-block tiles for 32- and
    # 64-row blocks (16+ routes per expert), runs of 256 rows and 256 columns for 16-row blocks
    assert sel(2, 8192, 7168, 128, 8, 64, 256) == (1, 64)
    assert sel(2, 8192, 7168, 128, 8, 32, 256) == (1, 64)
    assert sel(2, 8192, 7168, 128, 8, 64, 128) == (1, 64)
    assert sel(2, 1024, 7168, 128, 8, 64, 256) == (1, 64)     # 64 routes per expert
    assert sel(2, 160, 7168, 128, 8, 64, 256) == (1, 128)     # 10 routes per expert
    assert sel(2, 8192, 7168, 128, 8, 16, 256) == (16, 256)
    assert sel(2, 8192, 7168, 128, 8, 16, 256, "int4") == (16, 256)
    # decode: 64-column single-block tiles whatever the caller asked
    assert sel(1, 8, 256, 256, 8, 32, 256, "int4_bf16") == (1, 64)
    assert sel(2, 8, 7168, 256, 8, 32, 256) == (1, 64)
    # in between: stage 1 of W4A16 and blockscale 128 columns from about three workgroups per CU
    # (runs x inter_dim / 128 >= 768), else 64; stage 2 never keeps 256 single-block columns
    assert sel(1, 160, 1024, 64, 4, 32, 256, "int4_bf16") == (1, 64)      # 84 runs x 8 = 672
    assert sel(1, 512, 1024, 64, 4, 32, 256, "int4_bf16") == (1, 128)     # 128 runs x 8
    assert sel(1, 512, 1024, 64, 4, 32, 128, "fp8", 1) == (1, 128)
    assert sel(1, 160, 1024, 64, 4, 32, 256, "fp8", 1) == (1, 64)
    for kind in ("fp8", "int8", "bf16", "fp16", "int4", "int8smooth", "int4_bf16"):
        assert sel(2, 160, 512, 64, 4, 32, 256, kind) == (1, 128), kind
    assert sel(2, 128, 7168, 256, 8, 32, 0) == (1, 128)
    # fp8 routings with large experts (64-row blocks, inter_dim >= 1024, >= 512 routes per expert;
    # stage 1 with model_dim >= 4096): runs of 256 rows, 128 columns in stage 1, 256 in stage 2
    assert sel(1, 32768, 8192, 16, 4, 64, 128, k=8192) == (4, 128)      # the reference's benchmark shape
    assert sel(2, 32768, 8192, 16, 4, 64, 256, k=8192) == (4, 256)
    assert sel(1, 2048, 14336, 8, 2, 64, 128, k=4096) == (4, 128)       # 512 routes per expert
    assert sel(2, 2048, 4096, 8, 2, 64, 256, k=14336) == (4, 256)
    assert sel(1, 2048, 14336, 8, 2, 64, 128, k=2048) == (2, 64)        # model_dim below 4096
    assert sel(2, 8192, 2048, 128, 8, 64, 256, k=768) == (1, 64)        # inter_dim below 1024
    assert sel(1, 1024, 14336, 8, 2, 64, 128, k=4096) == (4, 128)       # 256 routes per expert, inter_dim
    assert sel(2, 1024, 4096, 8, 2, 64, 256, k=14336) == (4, 256)       # of 4096 or more
    assert sel(2, 2048, 4096, 64, 8, 64, 256, k=1536)[0] == 1           # 256 per expert, inter_dim 1536
    assert sel(2, 1024, 4096, 8, 2, 64, 256, "int4", k=14336)[0] == 1   # int4: 512 per expert
    assert sel(2, 960, 8192, 16, 4, 64, 256, k=8192)[0] == 1            # 240 routes per expert
    assert sel(1, 32768, 8192, 16, 4, 32, 128, k=8192) == (8, 128)      # 32- and 16-row blocks alike
    assert sel(2, 32768, 8192, 16, 4, 32, 256, k=8192) == (8, 256)
    assert sel(1, 32768, 8192, 16, 4, 16, 128, k=8192) == (16, 128)
    assert sel(1, 32768, 8192, 16, 4, 32, 128, k=2048) == (4, 64)       # model_dim below 4096: the stream kernel
    for kind in ("int8", "int8smooth", "bf16", "fp16"):
        assert sel(1, 32768, 8192, 16, 4, 64, 128, kind, k=8192) == (4, 128), kind
        assert sel(2, 32768, 8192, 16, 4, 64, 256, kind, k=8192) == (4, 256), kind
    assert sel(2, 32768, 8192, 16, 4, 64, 256, "int4_bf16", k=8192) == (4, 256)    # W4A16, per-row scales
    assert sel(1, 32768, 8192, 16, 4, 32, 128, "int4_bf16", k=8192) == (8, 128)
    assert sel(1, 32768, 8192, 16, 4, 16, 128, "int4_bf16", k=8192)[0] == 1     # not for 16-row blocks
    assert sel(1, 32768, 8192, 16, 4, 64, 128, "int4", k=8192) == (4, 128)    # int4 from inter_dim 4096
    assert sel(2, 32768, 8192, 16, 4, 64, 256, "int4", k=8192) == (4, 256)
    assert sel(1, 32768, 2048, 16, 4, 64, 128, "int4", k=8192) == (2, 64)
    assert sel(2, 32768, 8192, 16, 4, 64, 256, "int4", k=2048)[0] == 1
    # blockscale on large experts (inter_dim >= 1024): stage 2 runs of 256 rows x 128 columns for
    # 16-row blocks from 128 routes per expert and 64-row blocks from 512; stage 1 runs of 256 rows
    # x 64 columns for 16-row blocks only
    assert sel(2, 32768, 8192, 16, 4, 64, 256, "fp8", 1, k=8192) == (4, 128)
    assert sel(2, 16384, 7168, 256, 8, 16, 256, "fp8", 1, k=2048) == (16, 128)
    assert sel(2, 4096, 7168, 256, 8, 16, 256, "fp8", 1, k=2048) == (16, 128)      # 128 routes per expert
    assert sel(2, 4096, 7168, 256, 8, 64, 256, "fp8", 1, k=2048)[0] == 1           # 64-row blocks: 512
    assert sel(2, 4096, 7168, 256, 8, 32, 256, "fp8", 1, k=2048) == (8, 128)       # 32-row blocks: 128
    assert sel(2, 2048, 7168, 256, 8, 32, 256, "fp8", 1, k=2048)[0] == 1
    assert sel(1, 16384, 2048, 256, 8, 32, 256, "fp8", 1, k=7168)[0] == 1
    assert sel(1, 16384, 2048, 256, 8, 16, 256, "fp8", 1, k=7168) == (16, 64)
    assert sel(1, 16384, 2048, 256, 8, 64, 256, "fp8", 1, k=7168)[0] == 1
    assert sel(2, 8192, 7168, 256, 8, 16, 256, "fp8", 1, k=256)[0] == 1            # inter_dim 256
    assert lib.flygemm_moe_select_tile(1, 64, 256, 0, 4, 2, 64, 0, 0, 0, ctypes.byref(ctypes.c_int32()),
                                       ctypes.byref(ctypes.c_int32())) != 0   # k = 0
    # blockscale (inter_dim 256) and W4A16 take no run tiles
    assert sel(2, 8192, 7168, 128, 8, 16, 256, "fp8", 1)[0] == 1
    assert sel(2, 8192, 7168, 128, 8, 16, 256, "int4_bf16")[0] == 1
    assert sel(1, 8192, 256, 128, 8, 16, 256, "fp8", 1)[0] == 1
    assert sel(1, 8192, 256, 128, 8, 16, 256, "int4_bf16")[0] == 1
    # validation
    assert sel(3, 16, 256, 4, 2, 16, 64) != 0 and b"stage" in lib.flygemm_last_error()
    assert sel(1, 16, 256, 4, 2, 48, 64) != 0 and b"tile_m" in lib.flygemm_last_error()
    assert sel(1, 16, 320, 4, 2, 16, 256) != 0 and b"tile_n" in lib.flygemm_last_error()
    assert sel(1, 16, 256, 4, 2, 16, 64, "fp4") != 0 and b"in_dtype" in lib.flygemm_last_error()


def test_compile_validates_on_first_call():
    """``flydsl_amd.compile`` runs the launch once with every check (host tensors are refused
    before anything reaches the library); a callable that is not one of this package's
    launchers comes back as it is, after its first call."""
    import flydsl_amd
    fn = compile_preshuffle_gemm_a8(K=256, tile_m=64, tile_n=128, tile_k=128, in_dtype="fp8", out_dtype="bf16")
    x = torch.zeros(64 * 256, dtype=torch.int8)
    with pytest.raises(ValueError, match="GPU tensor"):
        flydsl_amd.compile(fn, torch.zeros(64 * 128, dtype=torch.bfloat16), x, x, torch.ones(64), torch.ones(128),
                           64, 128, None)
    seen = []
    plain = lambda *a: seen.append(a)   # noqa: E731
    assert flydsl_amd.compile(plain, 1, 2) is plain and seen == [(1, 2)]


def test_cpu_baseline_dispatches_on_the_kind():
    """bench.py's CPU baseline runs the reference's CPU path for each kind: per-row scales
    (fp8, int8, int4), the 1x128 / 128x128 block expansion (blockscale), no scales (bf16), and
    refuses MXFP4 with a clear error instead of timing wrong math."""
    import bench
    for kind in ("fp8", "int8", "int4", "fp8_block", "bf16"):
        r = bench.cpu_baseline(workloads.custom(kind, 32, 256, 256, seed=1, b_std=0.02 if kind == "int4" else 1.0))
        assert r["value"] > 0 and r["kind"] == "port" and r["cores"] >= 1, kind
    with pytest.raises(ValueError, match="no CPU baseline"):
        bench.cpu_baseline(workloads.custom("mxfp4", 32, 256, 256, seed=1))
