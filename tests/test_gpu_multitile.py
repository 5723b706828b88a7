"""GPU parity where the large-M kernel's persistent workgroups walk several output tiles, and on
the reference's own large test shapes.

The large-M kernel launches one workgroup per resident slot (CUs x workgroups per CU) and each
walks tiles w, w + grid, ...; the LDS ring carries the next tile's first K tiles across the tile
boundary and the staged epilogue reuses the stage the last step read.  Every main variant is
forced here onto shapes with more than twice as many tiles as slots (the launch is queried
through ``flygemm_launch_shape``), with ragged M and N edges, tile counts that are and are not
multiples of 8 (the XCD remap applies only to the former) and K of two and three K tiles
(a half last K tile where the kind allows one), for every kind.

Checked rows: two per tile row (at offsets that move through the tile's wave rows) and the last
row, with every column, so every output tile has checked rows.  Bars: int8/int4 raw int32
accumulators and bf16 outputs bit-exact against the oracle; fp8, blockscale, bf16 and MXFP4
within ``1e-2 |ref| + 1e-2 RMS(ref)`` of the float64 dequantize-then-matmul.
"""
import ctypes

import numpy as np
import pytest
import torch

from flydsl_amd import _lib, workloads
from oracle import gemm as og
from oracle import mxfp4 as om
from oracle import numerics as on
from tests import helpers as H

pytestmark = pytest.mark.gpu
VARIANTS = H.variant_names()
MAIN = [i for i, n in enumerate(VARIANTS) if n.startswith("main_")]
KINDS = ["fp8", "int8", "int4", "bf16", "fp8_block", "mxfp4"]


def _say(msg):
    print(msg, flush=True)


def _in_dtype(kind):
    return {"fp8_block": _lib.FLYGEMM_IN["fp8"], "mxfp4": _lib.FLYGEMM_IN["fp4"]}.get(kind, _lib.FLYGEMM_IN.get(kind))


def launch_shape(kind, M, N, K, variant):
    """(variant, grid, threads, items) of the launch the entry point would make."""
    out = [ctypes.c_int32(0) for _ in range(4)]
    rc = _lib.load().flygemm_launch_shape(M, N, K, _in_dtype(kind), int(kind == "fp8_block"), variant,
                                          *[ctypes.byref(o) for o in out])
    _lib.check(rc, "flygemm_launch_shape")
    return tuple(o.value for o in out)


def _tile(variant):
    bm, bn = VARIANTS[variant].split("_")[1].split("x")
    return int(bm), int(bn)


def multi_tile_shape(kind, variant, K, mult8):
    """M, N with ragged edges and more than 2.5x as many tiles as the variant has resident
    workgroups; the tile count a multiple of 8 or not (mult8)."""
    bm, bn = _tile(variant)
    slots = launch_shape(kind, 16384, 16384, K, variant)[1]   # grid of a shape with far more tiles
    need = slots * 5 // 2 + 1
    tr = int(np.ceil(np.sqrt(need)))
    tc = (need + tr - 1) // tr
    if not mult8 and tr % 8 == 0:
        tr += 1
    while ((tr * tc) % 8 == 0) != mult8:
        tc += 1
    n_align = 32 if kind == "mxfp4" else 16
    M = (tr - 1) * bm + 37
    N = (tc - 1) * bn + max(n_align, (bn // 3) // n_align * n_align)
    return M, N, tr, tc


def sample_rows(M, bm):
    rows = set()
    for r in range((M + bm - 1) // bm):
        for off in ((r * 37) % bm, (r * 37 + bm // 2) % bm):
            if r * bm + off < M:
                rows.add(r * bm + off)
    rows.add(M - 1)
    return np.array(sorted(rows))


def run_direct(ops, gpu, variant, raw=False):
    """One call through the C ABI (the fp8 launcher would reject a 64-byte tile_k)."""
    w = ops["workload"]
    lib = _lib.load()
    a, b = H.dev_flat(ops["a"], gpu), H.dev_flat(ops["b_dev"], gpu)
    if raw:
        dt = torch.int32 if w.kind in ("int8", "int4") else torch.float32
        acc = torch.empty(w.M, w.N, dtype=dt, device=gpu)
        _lib.check(lib.flygemm_accumulators(acc.data_ptr(), a.data_ptr(), b.data_ptr(), w.M, w.N, w.K,
                                            _in_dtype(w.kind), variant, None), "flygemm_accumulators")
        return acc
    c = torch.empty(w.M, w.N, dtype=torch.bfloat16, device=gpu)
    if w.kind == "fp8_block":
        sa, sb = ops["sa_t"].to(gpu).contiguous(), ops["sb"].to(gpu).contiguous()
        rc = lib.flygemm_blockscale(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                                    w.M, w.N, w.K, 128, 0, variant, None)
    elif w.kind == "mxfp4":
        sa, sb = ops["sa"].to(gpu).contiguous(), ops["sb"].to(gpu).contiguous()
        rc = lib.flygemm_mxfp4(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                               w.M, w.N, w.K, 0, variant, None)
    else:
        scaled = w.kind in ("fp8", "int8", "int4")
        sa = ops["sa"].to(gpu).contiguous() if scaled else None
        sb = ops["sb"].to(gpu).contiguous() if scaled else None
        rc = lib.flygemm_preshuffle(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr() if scaled else None,
                                    sb.data_ptr() if scaled else None, w.M, w.N, w.K, _in_dtype(w.kind), 0,
                                    variant, None)
    _lib.check(rc, "entry point")
    return c


def check_rows(ops, gpu, variant, rows):
    w = ops["workload"]
    out = run_direct(ops, gpu, variant)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()[rows]
    if w.kind == "mxfp4":
        ref = om.run_torch_w4(ops["a"].numpy()[rows], ops["b"].numpy(), ops["sa_raw"].numpy()[rows],
                              ops["sb_raw"].numpy(), "f64")
        ok, worst = og.within_bar(o, ref)
        assert ok, f"worst |err|/bound = {worst:.3g}"
        return
    ref = H.reference(ops, rows)
    if w.kind in ("int8", "int4"):
        acc = run_direct(ops, gpu, variant, raw=True)
        torch.cuda.synchronize()
        bad = np.flatnonzero(acc.cpu().numpy()[rows] != ref)
        assert bad.size == 0, f"{bad.size} accumulators differ, first at row {rows[bad[0] // w.N]} col {bad[0] % w.N}"
        want = on.bf16_to_f32(og.epilogue_int_bf16(ref, ops["sa"].numpy().reshape(-1)[rows],
                                                   ops["sb"].numpy().reshape(-1)))
        bad = np.flatnonzero(o.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"{bad.size} outputs differ, first at row {rows[bad[0] // w.N]} col {bad[0] % w.N}"
    else:
        ok, worst = og.within_bar(o, ref)
        assert ok, f"worst |err|/bound = {worst:.3g}"


def _ks(kind):
    """K values (elements): two and three K tiles; the second a half last K tile where allowed."""
    return {"fp8": (256, 320), "int8": (256, 320), "int4": (256, 320), "bf16": (128, 160),
            "fp8_block": (256, 384), "mxfp4": (512, 768)}[kind]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("variant", MAIN)
def test_multi_tile_walk(gpu, kind, variant):
    if kind == "mxfp4" and _tile(variant) == (64, 64):
        pytest.skip("64x64 is rejected for MXFP4 (its 16-column wave tiles split a scale group)")
    for i, K in enumerate(_ks(kind)):
        M, N, tr, tc = multi_tile_shape(kind, variant, K, mult8=(i == 0))
        v, grid, threads, items = launch_shape(kind, M, N, K, variant)
        assert v == variant and items == tr * tc
        assert items > 2 * grid, f"{VARIANTS[variant]}: {items} tiles on {grid} workgroups is not a multi-tile walk"
        _say(f"multi-tile {VARIANTS[variant]} {kind} {M}x{N}x{K}: {items} tiles on {grid} workgroups x {threads}")
        w = workloads.custom(kind, M, N, K, seed=M + 3 * N + K, b_std=0.02 if kind == "int4" else 1.0)
        ops = workloads.make_operands(w)
        check_rows(ops, gpu, variant, sample_rows(M, _tile(variant)[0]))


# ---------------------------------------------------------------- the reference's large shapes
@pytest.mark.parametrize("kind", ["fp8", "int8", "int4"])
@pytest.mark.parametrize("M,N,K", [(5120, 5120, 8320), (5120, 2048, 8320), (9728, 8192, 8320), (5133, 5120, 8320)])
def test_reference_preshuffle_shapes(gpu, kind, M, N, K):
    """tests/kernels/test_preshuffle_gemm.py:68-77 (the 1-byte kinds), the library's own variant,
    sampled rows: 64 spread over M plus the last."""
    v, grid, threads, items = launch_shape(kind, M, N, K, -1)
    _say(f"reference shape {kind} {M}x{N}x{K}: {VARIANTS[v]}, {items} tiles on {grid} workgroups")
    w = workloads.custom(kind, M, N, K, seed=M + N + K, b_std=0.02 if kind == "int4" else 1.0)
    ops = workloads.make_operands(w)
    rows = np.unique(np.r_[np.linspace(0, M - 1, 64).astype(int), M - 1])
    check_rows(ops, gpu, -1, rows)


@pytest.mark.parametrize("M", [256, 1024])
@pytest.mark.parametrize("N,K", [(7168, 2304), (2112, 7168), (3072, 1536)])
def test_blockscale_reference_shapes_large_m(gpu, M, N, K):
    """The reference's DeepSeek-V3 blockscale shapes at M = 256 and 1024
    (tests/kernels/test_blockscale_preshuffle_gemm.py:111-146), every row."""
    v, grid, _, items = launch_shape("fp8_block", M, N, K, -1)
    _say(f"blockscale {M}x{N}x{K}: {VARIANTS[v]}, {items} tiles on {grid} workgroups")
    ops = workloads.make_operands(workloads.custom("fp8_block", M, N, K, seed=M * 7 + N))
    check_rows(ops, gpu, -1, np.arange(M))


def test_blockscale_three_stage_multi_tile_selected(gpu):
    """4096x2112x7168: the table picks a three-stage 8-wave tile with more tiles than workgroups,
    so the staged blockscale epilogue runs between tiles of one workgroup."""
    M, N, K = 4096, 2112, 7168
    v, grid, _, items = launch_shape("fp8_block", M, N, K, -1)
    _say(f"blockscale {M}x{N}x{K}: {VARIANTS[v]}, {items} tiles on {grid} workgroups")
    assert items > grid
    ops = workloads.make_operands(workloads.custom("fp8_block", M, N, K, seed=11))
    check_rows(ops, gpu, -1, sample_rows(M, _tile(v)[0]))
