"""GPU parity of the per-token quant kernel (``flygemm_quant_rows``) against the CPU oracle.

Bar: bit-exact codes and bit-exact fp32 scales.  Cases: the reference test's own data
(np.random.seed(42), uniform(-5, 5) fp16, tests/kernels/test_quant.py:306-307) at its shapes,
every input dtype and rounding mode, rows held in registers (1/2/4/8 slices of 2048) and the
streaming variant, ragged N, zero rows, NaN/inf scrubbing, M = 0, a side stream."""
import numpy as np
import pytest
import torch

from flydsl_amd.kernels.quant import build_quant_module, per_token_quant
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _ref_data(M, N, seed=42):
    np.random.seed(seed)
    return np.random.uniform(-5.0, 5.0, size=(M, N)).astype(np.float16)


@pytest.mark.parametrize("M,N", [(2048, 8192), (4096, 8192), (7, 2056), (1, 8), (33, 16384), (5, 20480)])
def test_reference_kernel_semantics(gpu, M, N):
    _say(f"quant recip_trunc fp16->int8 M={M} N={N}")
    x = _ref_data(M, N)
    launch, cfg = build_quant_module(N)
    threads = 512 if N >= 8192 else 256   # rows of 8192+ elements run 512 threads
    assert cfg["BLOCK_THREADS"] == threads and cfg["ITERS"] == (N + threads * 8 - 1) // (threads * 8)
    xi = torch.from_numpy(x).to(gpu)
    out = torch.empty(M, N, dtype=torch.int8, device=gpu)
    sc = torch.empty(M, dtype=torch.float32, device=gpu)
    launch(xi, out, sc, M)
    torch.cuda.synchronize()
    q_ref, s_ref = oq.quant_rows_recip(x)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(out.cpu().numpy(), q_ref)
    # the reference test's own acceptance: within 1 of (x / scale).astype(int8)
    xf = x.astype(np.float32)
    amax = np.abs(xf).max(axis=1)
    rs = amax / 127.0
    rs[rs == 0] = 1.0
    assert np.max(np.abs(out.cpu().numpy().astype(np.int32) - (xf / rs[:, None]).astype(np.int8))) <= 1


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("qd,rounding", [(torch.int8, "nearest"), (torch.int8, "trunc"),
                                         (torch.float8_e4m3fn, "nearest")])
@pytest.mark.parametrize("N", [8, 2048, 4104, 8192, 16384, 24576])
def test_pertoken_quant_modes(gpu, dtype, qd, rounding, N):
    M = 37
    _say(f"quant {dtype} -> {qd} rounding={rounding} M={M} N={N}")
    g = torch.Generator().manual_seed(N + M)
    x = torch.randn(M, N, generator=g) * 4
    x[3] = 0.0                      # zero row -> scale 1
    x[5, N // 2] = 1e4              # one large value dominates the row
    x[6] = x[6] * 1e-3              # small-magnitude row (fp8 subnormals)
    xh = x.to(dtype)
    q, s = per_token_quant(xh.to(gpu), quant_dtype=qd, rounding=rounding)
    torch.cuda.synchronize()
    kind = "fp8" if qd == torch.float8_e4m3fn else "int8"
    q_ref, s_ref = oq.quant_rows(xh.float().numpy(), kind, rounding="truncate" if rounding == "trunc" else "nearest")
    assert s.shape == (M, 1)
    assert np.array_equal(s.cpu().view(-1).numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().view(torch.uint8).numpy(), q_ref.view(np.uint8))


@pytest.mark.parametrize("qd", [torch.int8, torch.float8_e4m3fn])
def test_nonfinite_scrubbing(gpu, qd):
    """pertoken_quant's nan_to_num before the amax (tests/utils.py:50-55)."""
    x = torch.randn(6, 64) * 2
    x[0, 3] = float("nan")
    x[1, 5] = float("inf")
    x[2, 7] = float("-inf")
    x[3, :] = float("nan")
    q, s = per_token_quant(x.to(gpu), quant_dtype=qd)
    kind = "fp8" if qd == torch.float8_e4m3fn else "int8"
    q_ref, s_ref = oq.quant_rows(x.numpy(), kind)
    assert np.array_equal(s.cpu().view(-1).numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().view(torch.uint8).numpy(), q_ref.view(np.uint8))


def test_quant_feeds_gemm_bit_exact(gpu):
    """A produced on the device by the quant kernel equals the host quantizer's A, so the
    GEMM that consumes it sees identical operands (int8 per-token, round to nearest)."""
    from flydsl_amd import quant as pq
    g = torch.Generator().manual_seed(5)
    x = torch.randn(128, 4096, generator=g)
    q_d, s_d = per_token_quant(x.to(gpu), quant_dtype=torch.int8)
    q_h, s_h = pq.pertoken_quant(x, quant_dtype=torch.int8)
    assert torch.equal(q_d.cpu(), q_h) and torch.equal(s_d.cpu().view(-1), s_h.view(-1))
    q_d8, s_d8 = per_token_quant(x.to(gpu), quant_dtype=torch.float8_e4m3fn)
    q_h8, s_h8 = pq.pertoken_quant(x, quant_dtype=pq.FP8)
    assert torch.equal(q_d8.cpu().view(torch.uint8), q_h8.view(torch.uint8))
    assert torch.equal(s_d8.cpu().view(-1), s_h8.view(-1))


def test_zero_rows_side_stream_and_errors(gpu):
    launch, _ = build_quant_module(64)
    x = torch.empty(0, 64, dtype=torch.float16, device=gpu)
    launch(x, torch.empty(0, 64, dtype=torch.int8, device=gpu), torch.empty(0, device=gpu), 0)
    s = torch.cuda.Stream()
    xh = _ref_data(16, 64, seed=3)
    xi = torch.from_numpy(xh).to(gpu)
    out = torch.empty(16, 64, dtype=torch.int8, device=gpu)
    sc = torch.empty(16, dtype=torch.float32, device=gpu)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launch(xi, out, sc, 16, stream=s)
    s.synchronize()
    q_ref, s_ref = oq.quant_rows_recip(xh)
    assert np.array_equal(out.cpu().numpy(), q_ref) and np.array_equal(sc.cpu().numpy(), s_ref)
    with pytest.raises(TypeError):
        launch(xi.float(), out, sc, 16)
    with pytest.raises(ValueError):
        build_quant_module(12)
