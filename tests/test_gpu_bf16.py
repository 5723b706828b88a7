"""GPU parity of ``in_dtype="bf16"/"fp16"`` (unscaled 16-bit GEMM through the same preshuffle
entry point) against the oracle's float64 ``mm(a.float(), b.float().T)``.

Bars: bf16/fp16 outputs within ``1e-2 |ref| + 1e-2 RMS(ref)``; raw fp32 accumulators within
``1e-4 |ref| + 1e-4 RMS(ref)`` (fp32 accumulation error over K).  Data as the reference test
draws it (``torch.rand`` in [0, 1), ``tests/kernels/test_preshuffle_gemm.py:141-151``) and
N(0, 1) for the ragged variant sweep."""
import numpy as np
import pytest
import torch

from flydsl_amd import _lib, quant, workloads
from flydsl_amd.kernels.preshuffle_gemm import accumulators, compile_preshuffle_gemm_a8
from oracle import gemm as og
from tests import helpers as H

pytestmark = pytest.mark.gpu
VARIANTS = H.variant_names()
DT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _say(msg):
    print(msg, flush=True)


def _rand_ops(kind, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(M, K, generator=g).to(DT[kind])
    b = torch.rand(N, K, generator=g).to(DT[kind])
    return a, b, quant.shuffle_weight(b)


def _run(kind, a, b_shuf, M, N, K, gpu, variant=-1, out_dtype="bf16"):
    fn = compile_preshuffle_gemm_a8(K=K, tile_m=64, tile_n=128, tile_k=64, in_dtype=kind, out_dtype=out_dtype,
                                    variant=variant)
    c = torch.empty(M, N, dtype=DT[out_dtype], device=gpu)
    empty = torch.empty(0, dtype=torch.float32, device=gpu)
    fn(c.view(-1), a.to(gpu).view(-1), b_shuf.to(gpu).view(-1), empty, empty, M, N, torch.cuda.current_stream())
    return c


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("M,N,K", [(16, 5120, 8192), (33, 1024, 2048), (5120, 5120, 8320), (5120, 2048, 8320),
                                   (9728, 8192, 8320), (5133, 5120, 8320)])
def test_reference_shapes(gpu, kind, M, N, K):
    """The reference test's shapes (test_preshuffle_gemm.py:70-79), sampled rows above 1024."""
    _say(f"16-bit {kind} {M}x{N}x{K}")
    a, b, b_shuf = _rand_ops(kind, M, N, K, seed=M + N + K)
    c = _run(kind, a, b_shuf, M, N, K, gpu)
    torch.cuda.synchronize()
    rows = np.arange(M) if M <= 1024 else np.unique(np.r_[np.linspace(0, M - 1, 64).astype(int), M - 1])
    ref = og.run_torch(H.bits16(a)[rows], H.bits16(b), None, None, kind, "f64")
    ok, worst = og.within_bar(c.float().cpu().numpy()[rows], ref)
    assert ok, f"worst |err|/bound = {worst:.3g}"


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("variant", list(range(len(VARIANTS))))
def test_variants_ragged(gpu, kind, variant):
    for (M, N, K) in [(1, 64, 64), (7, 2112, 256), (16, 1024, 2048), (33, 1040, 384), (100, 272, 192),
                      (300, 528, 640)]:
        _say(f"variant {VARIANTS[variant]} {kind} {M}x{N}x{K}")
        ops = workloads.make_operands(workloads.custom(kind, M, N, K, seed=M * 3 + N + K))
        out = H.launch(ops, gpu, variant=variant)
        torch.cuda.synchronize()
        ref = H.check(ops, out)
        acc = H.raw_acc(ops, gpu, variant).cpu().numpy()
        ok, worst = og.within_bar(acc, ref, rtol=1e-4, atol_rms=1e-4)
        assert ok, f"accumulators: worst |err|/bound = {worst:.3g}"


def test_fp16_output_and_errors(gpu):
    ops = workloads.make_operands(workloads.custom("fp16", 160, 512, 1088, seed=3))
    out = H.launch(ops, gpu, out_dtype="fp16")
    torch.cuda.synchronize()
    H.check(ops, out)
    fn = compile_preshuffle_gemm_a8(K=1056, tile_m=64, tile_n=128, tile_k=32, in_dtype="bf16", out_dtype="bf16")
    x = torch.empty(64 * 1056, dtype=torch.bfloat16, device=gpu)
    c = torch.empty(64 * 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):   # K % 64 != 0
        fn(c, x, x, torch.empty(0, device=gpu), torch.empty(0, device=gpu), 64, 128)
    fn = compile_preshuffle_gemm_a8(K=1088, tile_m=64, tile_n=128, tile_k=64, in_dtype="bf16", out_dtype="bf16")
    with pytest.raises(TypeError):    # fp16 tensor for a bf16 GEMM
        fn(c, x.view(torch.float16), x, torch.empty(0, device=gpu), torch.empty(0, device=gpu), 64, 128)
    acc = torch.empty(4, 4, dtype=torch.int32, device=gpu)
    with pytest.raises(TypeError):    # bf16 accumulators are fp32
        accumulators(acc, x, x, 4, 4, 1088, "bf16")
