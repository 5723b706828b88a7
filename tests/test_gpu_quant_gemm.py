"""GPU check of ``flygemm_preshuffle_quant_a`` (``flydsl_amd.kernels.quant.quant_gemm``), the GEMM
of activations quantized on the way in, in one call.

Its output, codes and scales must equal, bit for bit, those of the two entry points it stands
for on the same inputs: ``flygemm_quant_rows`` (the reference's quant kernel,
tests/kernels/test_quant.py:81-265, or pertoken_quant, tests/utils.py:29-73) followed by
``flygemm_preshuffle``.  Covered: fp8, int8 and int4 weights, fp16 / bf16 / fp32 activations,
every quantization mode, all-zero rows and NaN / inf rows (the host quantizer's modes), a half
last K tile, decode and larger M, forced variants; and the argument checks (buffers required,
alignment, modes), all made before any launch.  The parity of the two underlying entry points
with the oracle is covered by test_gpu_quant.py and test_gpu_parity.py."""
import numpy as np
import pytest
import torch

from flydsl_amd import _lib, quant
from flydsl_amd.kernels.quant import quant_gemm
from tests import helpers as H

pytestmark = pytest.mark.gpu
VARIANTS = H.variant_names()
DECODE = [i for i, n in enumerate(VARIANTS) if n.startswith("decode_m1_")]
OUT_T = {"bf16": torch.bfloat16, "fp16": torch.float16}
QIN = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
KINDS = [("fp8", "div_nearest"), ("int8", "recip_trunc"), ("int8", "div_trunc"), ("int8", "div_nearest"),
         ("int4", "recip_trunc")]


def _say(msg):
    print(msg, flush=True)


def _weights(in_dtype, N, K, dev, seed):
    g = torch.Generator().manual_seed(seed)
    b32 = torch.randn(N, K, generator=g) * (0.02 if in_dtype == "int4" else 1.0)
    if in_dtype == "fp8":
        b, sb = quant.pertoken_quant(b32, quant_dtype=quant.FP8)
    else:
        b, sb = quant.pertoken_quant(b32, quant_dtype=torch.int8, dtypeMax=7 if in_dtype == "int4" else None)
    shuf = quant.shuffle_weight(b)
    b_dev = quant.pack_int4(shuf) if in_dtype == "int4" else shuf
    return b_dev.contiguous().view(torch.int8).view(-1).to(dev), sb.contiguous().view(-1).to(dev)


def _activations(M, K, dtype, dev, seed, specials):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g) * 3.0
    if M > 2:
        x[1] = 0.0                                     # an all-zero row: scale 1
        x[2, :K // 3] *= 1e-3                          # a row of very different magnitudes
    if specials and M > 4:
        x[3, 5] = float("nan")                          # scrubbed to 0 by the host quantizer's modes
        x[4, 7] = float("inf")
        x[4, 9] = float("-inf")
    return x.to(dtype).to(dev)


def _two_steps(x, b, sb, M, N, K, in_dtype, mode, out_dtype, variant):
    lib = _lib.load()
    qdt = torch.float8_e4m3fn if in_dtype == "fp8" else torch.int8
    q = torch.empty(M, K, dtype=qdt, device=x.device)
    s = torch.empty(M, 1, dtype=torch.float32, device=x.device)
    c = torch.full((M, N), float("nan"), dtype=OUT_T[out_dtype], device=x.device)
    _lib.check(lib.flygemm_quant_rows(q.data_ptr(), s.data_ptr(), x.data_ptr(), M, K, QIN[x.dtype],
                                      0 if in_dtype == "fp8" else 1, _lib.QUANT_MODE[mode], None),
               "flygemm_quant_rows")
    _lib.check(lib.flygemm_preshuffle(c.data_ptr(), q.data_ptr(), b.data_ptr(), s.data_ptr(), sb.data_ptr(), M, N, K,
                                      _lib.FLYGEMM_IN[in_dtype], _lib.FLYGEMM_OUT[out_dtype], variant, None),
               "flygemm_preshuffle")
    return c, q, s


def _same(got, want, what):
    torch.cuda.synchronize()
    a = got.contiguous().view(torch.uint8).cpu().numpy()
    b = want.contiguous().view(torch.uint8).cpu().numpy()
    bad = np.flatnonzero(a != b)
    assert bad.size == 0, f"{what}: {bad.size} bytes differ, first at byte {bad[0]}"


def _check(x, b, sb, M, N, K, in_dtype, mode, out_dtype="bf16", variant=-1, what=""):
    """The one-call entry against the two entry points it stands for."""
    c, q, s = quant_gemm(x, b, sb, N, in_dtype=in_dtype, out_dtype=out_dtype, mode=mode, variant=variant)
    c_ref, q_ref, s_ref = _two_steps(x, b, sb, M, N, K, in_dtype, mode, out_dtype, variant)
    _same(s, s_ref, f"{what} scales")
    _same(q, q_ref, f"{what} codes")
    _same(c, c_ref, f"{what} output")
    assert torch.isfinite(c.float()).all(), f"{what}: non-finite output"


@pytest.mark.parametrize("in_dtype,mode", KINDS, ids=[f"{k}-{m}" for k, m in KINDS])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_every_decode_variant(gpu, in_dtype, mode, xdt):
    """Every one-row-block decode variant forced, ragged N, K with a half last K tile and without."""
    for (M, N, K) in [(13, 528, 640), (7, 2112, 192)]:
        b, sb = _weights(in_dtype, N, K, gpu, seed=N + K)
        x = _activations(M, K, xdt, gpu, seed=M + K, specials=mode != "recip_trunc")
        for v in DECODE:
            _say(f"quant gemm {VARIANTS[v]} {in_dtype} {mode} {xdt} {M}x{N}x{K}")
            _check(x, b, sb, M, N, K, in_dtype, mode, variant=v, what=f"{VARIANTS[v]} {M}x{N}x{K}")


@pytest.mark.parametrize("in_dtype,mode", KINDS, ids=[f"{k}-{m}" for k, m in KINDS])
def test_library_choice_shapes(gpu, in_dtype, mode):
    """The library's own variant on decode shapes up to C2's 16x28672x8192 and on larger M, fp16
    output too."""
    for (M, N, K, out) in [(1, 4096, 4096, "bf16"), (16, 28672, 8192, "bf16"), (16, 7168, 2048, "fp16"),
                           (20, 1024, 1024, "bf16"), (300, 2112, 1024, "bf16")]:
        b, sb = _weights(in_dtype, N, K, gpu, seed=N)
        x = _activations(M, K, torch.bfloat16, gpu, seed=M, specials=mode != "recip_trunc")
        _say(f"quant gemm {in_dtype} {mode} {M}x{N}x{K} {out}")
        _check(x, b, sb, M, N, K, in_dtype, mode, out_dtype=out, what=f"{M}x{N}x{K}")


def test_fp32_activations_and_errors(gpu):
    """fp32 activations and larger M; the C ABI needs a_q and scale_a; invalid combinations and
    misaligned buffers are rejected before any launch."""
    b, sb = _weights("int8", 528, 1024, gpu, seed=1)
    for (M, xdt, mode) in [(8, torch.float32, "div_trunc"), (40, torch.float32, "div_nearest"),
                           (300, torch.float16, "div_trunc")]:
        x = _activations(M, 1024, xdt, gpu, seed=M, specials=mode != "recip_trunc")
        _say(f"quant gemm int8 {M} {xdt} {mode}")
        _check(x, b, sb, M, 528, 1024, "int8", mode, what=f"{M} {mode}")
    lib = _lib.load()
    x = _activations(40, 1024, torch.bfloat16, gpu, seed=3, specials=False)
    c = torch.empty(40, 528, dtype=torch.bfloat16, device=gpu)
    q = torch.empty(40 * 1024 + 16, dtype=torch.int8, device=gpu)
    s = torch.empty(64, dtype=torch.float32, device=gpu)

    def call(qp, sp, M=40, in_dtype=1, mode=2, xp=None):
        return lib.flygemm_preshuffle_quant_a(c.data_ptr(), qp, sp, xp or x.data_ptr(), b.data_ptr(), sb.data_ptr(), M,
                                              528, 1024, 1, in_dtype, mode, 0, -1, None)
    assert call(None, None) != 0 and b"a_q" in lib.flygemm_last_error()
    assert call(q.data_ptr(), None) != 0 and b"scale_a" in lib.flygemm_last_error()
    assert call(q.data_ptr() + 4, s.data_ptr()) != 0 and b"misaligned" in lib.flygemm_last_error()
    assert call(q.data_ptr(), s.data_ptr(), xp=x.data_ptr() + 8) != 0 and b"misaligned" in lib.flygemm_last_error()
    assert call(q.data_ptr(), s.data_ptr(), in_dtype=0, mode=0) != 0 and b"DIV_NEAREST" in lib.flygemm_last_error()
    assert call(q.data_ptr(), s.data_ptr(), in_dtype=3) != 0 and b"in_dtype" in lib.flygemm_last_error()
    assert call(None, None, M=0) == 0   # nothing to do
    torch.cuda.synchronize()
