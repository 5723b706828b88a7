"""GPU parity of the MXFP4 path (``compile_preshuffle_gemm_w4`` / ``flygemm_mxfp4``) against the
oracle's ``run_torch_w4`` (float64) on operands prepared as the reference harness prepares them.

Bars: bf16/fp16 outputs within ``1e-2 |ref| + 1e-2 RMS(ref)``; fp32 outputs (the accumulators,
block scales applied by the MFMA) within ``1e-4 |ref| + 1e-4 RMS(ref)``."""
import numpy as np
import pytest
import torch

from flydsl_amd import _lib, workloads
from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8, compile_preshuffle_gemm_w4
from oracle import gemm as og
from oracle import mxfp4 as om
from tests import helpers as H

pytestmark = pytest.mark.gpu
VARIANTS = H.variant_names()
OUT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _say(msg):
    print(msg, flush=True)


def _run(ops, gpu, out_dtype="bf16", variant=-1):
    w = ops["workload"]
    c = torch.empty(w.M, w.N, dtype=OUT[out_dtype], device=gpu)
    if out_dtype == "fp32":
        lib = _lib.load()
        a, b = ops["a"].to(gpu), ops["b_dev"].to(gpu)
        sa, sb = ops["sa"].to(gpu), ops["sb"].to(gpu)
        rc = lib.flygemm_mxfp4(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr(),
                               w.M, w.N, w.K, 2, variant, None)
        _lib.check(rc, "flygemm_mxfp4")
        torch.cuda.synchronize()
        return c
    if variant < 0:
        fn = compile_preshuffle_gemm_w4(M=w.M, N=w.N, K=w.K, tile_m=64, tile_n=256, tile_k=256, out_dtype=out_dtype)
    else:
        fn = compile_preshuffle_gemm_a8(K=w.K, tile_m=64, tile_n=256, tile_k=256, in_dtype="fp4",
                                        out_dtype=out_dtype, variant=variant)
    fn(c.view(-1), ops["a"].to(gpu).view(-1), ops["b_dev"].to(gpu).view(-1), ops["sa"].to(gpu).view(-1),
       ops["sb"].to(gpu).view(-1), w.M, w.N, torch.cuda.current_stream())
    torch.cuda.synchronize()
    return c


def _ref(ops, rows=None):
    a = ops["a"].numpy()
    sa = ops["sa_raw"].numpy()
    if rows is not None:
        a, sa = a[rows], sa[rows]
    return om.run_torch_w4(a, ops["b"].numpy(), sa, ops["sb_raw"].numpy(), "f64")


_CACHE = {}


def _shape_case(M):
    """Operands and the sampled-row reference of one reference shape (kept for both out dtypes)."""
    if M not in _CACHE:
        _CACHE.clear()
        ops = workloads.make_operands(workloads.custom("mxfp4", M, 8192, 8192, seed=M))
        rows = np.arange(M) if M <= 128 else np.unique(np.r_[np.linspace(0, M - 1, 48).astype(int), M - 1])
        _CACHE[M] = (ops, rows, _ref(ops, rows))
    return _CACHE[M]


@pytest.mark.parametrize("M", [64, 32, 128, 1024, 5133])
@pytest.mark.parametrize("out_dtype", ["bf16", "fp16"])
def test_reference_shapes(gpu, M, out_dtype):
    """The reference test's shapes (test_preshuffle_gemm.py:264-273), N = K = 8192."""
    ops, rows, ref = _shape_case(M)
    _say(f"mxfp4 {M}x8192x8192 {out_dtype}")
    c = _run(ops, gpu, out_dtype)
    ok, worst = og.within_bar(c.float().cpu().numpy()[rows], ref)
    assert ok, f"worst |err|/bound = {worst:.3g}"


@pytest.mark.parametrize("variant", list(range(len(VARIANTS))))
def test_variants_ragged_fp32(gpu, variant):
    if VARIANTS[variant].startswith("main_64x64_w1x4"):   # also its two-K-tile form
        # its 16-column wave tiles would split a 32-column scale group: rejected before launch
        ops = workloads.make_operands(workloads.custom("mxfp4", 64, 64, 256, seed=1))
        with pytest.raises(RuntimeError, match="not available for MXFP4"):
            _run(ops, gpu, "fp32", variant)
        return
    for (M, N, K) in [(1, 64, 256), (7, 2080, 512), (16, 1024, 768), (33, 1056, 256), (100, 288, 512),
                      (300, 544, 768)]:
        _say(f"variant {VARIANTS[variant]} mxfp4 {M}x{N}x{K}")
        ops = workloads.make_operands(workloads.custom("mxfp4", M, N, K, seed=M + N + K))
        ref = _ref(ops)
        acc = _run(ops, gpu, "fp32", variant).cpu().numpy()
        ok, worst = og.within_bar(acc, ref, rtol=1e-4, atol_rms=1e-4)
        assert ok, f"fp32: worst |err|/bound = {worst:.3g}"
        out = _run(ops, gpu, "bf16", variant).float().cpu().numpy()
        ok, worst = og.within_bar(out, ref)
        assert ok, f"bf16: worst |err|/bound = {worst:.3g}"


def test_fp8_a_rejected_like_the_reference():
    with pytest.raises(NotImplementedError):
        compile_preshuffle_gemm_w4(K=8192, tile_m=64, tile_n=128, tile_k=128, a_dtype="fp8")
