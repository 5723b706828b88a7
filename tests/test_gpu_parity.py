"""GPU parity: the gfx950 kernels, called through the drop-in launchers / C ABI, against the
CPU oracle on the same seeded operands.

Bars: int8/int4 -- raw int32 accumulators and bf16 outputs bit-exact; fp8 paths --
|out - ref| <= 1e-2 |ref| + 1e-2 RMS(ref) with ref the float64 dequantize-then-matmul."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from flydsl_amd import _lib, workloads
from tests import helpers as H

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
VARIANTS = H.variant_names()
MAIN = [i for i, n in enumerate(VARIANTS) if n.startswith("main_")]


def _say(msg):
    print(msg, flush=True)


_OPS = {}


def _ops(name):
    if name not in _OPS:
        _OPS.clear()
        _OPS[name] = workloads.make_operands(workloads.WORKLOADS[name])
    return _OPS[name]


# ---------------------------------------------------------------- committed fixtures
@pytest.mark.parametrize("kind", ["fp8", "int8", "int4", "fp8_block"])
def test_golden_fixture(gpu, kind):
    z = np.load(os.path.join(GOLDEN, f"small_{kind}.npz"), allow_pickle=False)
    M, N, K = int(z["M"]), int(z["N"]), int(z["K"])
    _say(f"golden {kind} {M}x{N}x{K}")
    a = torch.from_numpy(z["a"]).to(gpu).view(torch.int8).view(-1)
    b = torch.from_numpy(z["b_dev"]).to(gpu).view(torch.int8)
    sa = torch.from_numpy(z["sa"]).to(gpu)
    sb = torch.from_numpy(z["sb"]).to(gpu)
    from oracle import gemm as og, numerics as on
    for v in [-1] + list(range(len(VARIANTS))):
        c = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        if kind == "fp8_block":
            rc = _lib.load().flygemm_blockscale(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(),
                                                sb.data_ptr(), M, N, K, 128, 0, v, None)
        else:
            rc = _lib.load().flygemm_preshuffle(c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(),
                                                sb.data_ptr(), M, N, K, _lib.FLYGEMM_IN[kind], 0, v, None)
        _lib.check(rc, "golden")
        torch.cuda.synchronize()
        out = c.float().cpu().numpy()
        exp = z["expected"]
        if kind in ("int8", "int4"):
            want = on.bf16_to_f32(og.epilogue_int_bf16(exp, z["sa"], z["sb"]))
            assert np.array_equal(out, want), f"variant {v}"
        else:
            assert og.within_bar(out, exp)[0], f"variant {v}"


def test_workload_operands_match_committed_hashes(gpu):
    """The box generates the same operand bytes as the machine that wrote the fixtures."""
    with open(os.path.join(GOLDEN, "workload_sha256.json")) as f:
        want = json.load(f)
    for name in ["C1", "C3", "C5"]:
        ops = workloads.make_operands(workloads.WORKLOADS[name])
        got = hashlib.sha256(H.u8(ops["b_dev"]).tobytes()).hexdigest()
        assert got == want[name]["b_dev"], name


# ---------------------------------------------------------------- full-size configurations
@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_config_parity(gpu, name):
    ops = _ops(name)
    w = ops["workload"]
    _say(f"config {name} {w.kind} {w.M}x{w.N}x{w.K} variant={VARIANTS[_lib.load().flygemm_select_variant(w.M, w.N, w.K, 0, 0)]}")
    out = H.launch(ops, gpu)
    torch.cuda.synchronize()
    ref = H.check(ops, out)
    if w.kind in ("int8", "int4"):
        acc = H.raw_acc(ops, gpu).cpu().numpy()
        assert np.array_equal(acc, ref), f"{name}: int32 accumulators differ"


def test_config_T_sampled_rows(gpu):
    ops = _ops("T")
    _say("config T fp8 8192^3 (sampled rows)")
    out = H.launch(ops, gpu)
    torch.cuda.synchronize()
    rows = np.random.default_rng(0).choice(8192, 96, replace=False)
    rows.sort()
    H.check(ops, out, rows=rows)


# ---------------------------------------------------------------- every variant, ragged shapes
SHAPES = [(1, 64, 128), (7, 2112, 256), (16, 1024, 2048), (33, 1040, 384), (100, 272, 384), (300, 528, 640)]
# every variant handles any M: the decode and rows variants add row blocks past 16*MR rows


@pytest.mark.parametrize("kind", ["fp8", "int8", "int4", "fp8_block"])
@pytest.mark.parametrize("variant", list(range(len(VARIANTS))))
def test_variants_ragged(gpu, kind, variant):
    for (M, N, K) in SHAPES:
        w = workloads.custom(kind, M, N, K, seed=M + N + K, b_std=0.02 if kind == "int4" else 1.0)
        ops = workloads.make_operands(w)
        _say(f"variant {VARIANTS[variant]} {kind} {M}x{N}x{K}")
        out = H.launch(ops, gpu, variant=variant)
        torch.cuda.synchronize()
        ref = H.check(ops, out)
        if kind in ("int8", "int4"):
            assert np.array_equal(H.raw_acc(ops, gpu, variant).cpu().numpy(), ref)


# ---------------------------------------------------------------- int4 accumulators at the K bound
@pytest.mark.parametrize("bval, byte", [(-8, 0x88), (7, 0x77)])
def test_int4_accumulators_exact_at_the_k_bound(gpu, bval, byte):
    """The int4 unpack leaves each nibble in the high half of its byte, so the int32 accumulators
    hold 16x the dot product until an exact shift.  At the largest accepted K (131008, a half
    last K tile) with every activation -128 and every weight -8 (16 * 1024 * K, the largest
    positive sum, just below 2^31) or 7 (the most negative one with this activation), every raw
    accumulator of every variant equals the closed form K * (-128) * bval."""
    lib = _lib.load()
    M, N, K = 16, 32, 131008
    a = torch.full((M * K,), -128, dtype=torch.int8, device=gpu)
    b = torch.full((N * K // 2,), byte, dtype=torch.uint8, device=gpu)   # two equal nibbles a byte
    acc = torch.empty(M, N, dtype=torch.int32, device=gpu)
    for v in [-1] + list(range(len(VARIANTS))):
        _say(f"int4 K bound {VARIANTS[v] if v >= 0 else 'auto'} b={bval} {M}x{N}x{K}")
        acc.fill_(0)
        _lib.check(lib.flygemm_accumulators(acc.data_ptr(), a.data_ptr(), b.data_ptr(), M, N, K,
                                            _lib.FLYGEMM_IN["int4"], v, None), "flygemm_accumulators")
        torch.cuda.synchronize()
        assert bool((acc == K * (-128) * bval).all()), (v, acc.min().item(), acc.max().item())


# ---------------------------------------------------------------- row-blocked streaming kernel
ROWS = [i for i, n in enumerate(VARIANTS) if n.startswith("rows_")]


@pytest.mark.parametrize("kind", ["fp8", "int8", "int4", "fp8_block", "bf16"])
@pytest.mark.parametrize("variant", ROWS)
def test_rows_variants(gpu, kind, variant):
    """The row-blocked kernel (several row blocks per column group, K split over the waves
    and summed in LDS) on ragged shapes: a partial last row block, N not a multiple of the
    column group, K tiles not a multiple of the wave count.  Int paths bit-exact (raw
    accumulators and bf16 output), the rest within the bar; a repeated call gives the same
    bits (the LDS sum has a fixed order)."""
    for (M, N, K) in [(100, 272, 1024), (130, 528, 2176), (300, 96, 640)]:
        w = workloads.custom(kind, M, N, K, seed=M + N + K, b_std=0.02 if kind == "int4" else 1.0)
        ops = workloads.make_operands(w)
        _say(f"rows {VARIANTS[variant]} {kind} {M}x{N}x{K}")
        out = H.launch(ops, gpu, variant=variant)
        again = H.launch(ops, gpu, variant=variant)
        torch.cuda.synchronize()
        assert torch.equal(out, again)
        ref = H.check(ops, out)
        if kind in ("int8", "int4"):
            assert np.array_equal(H.raw_acc(ops, gpu, variant).cpu().numpy(), ref)


@pytest.mark.parametrize("kind", ["fp8", "int8", "int4", "bf16", "fp16"])
def test_k_half_tile_every_variant(gpu, kind):
    """K with a last K tile of 64 bytes (K = 64 mod 128 for 1-byte inputs, 32 mod 64 for 16-bit
    ones: the reference's tile_k * elem_bytes % 64 == 0, e.g. int8 K = 192), through every
    variant of all three families, on ragged M/N.  int8/int4/bf16/fp16 go through the launcher
    with the 64-byte tile_k the reference harness would pass; fp8, whose reference launcher
    wants tile_k % 128 == 0 on gfx950 (kernels/preshuffle_gemm.py:665-673), through the C ABI.
    The half tile's upper 64 bytes (the next row's or block's bytes, or past the buffer) must
    not enter the sums: int8/int4 raw accumulators and outputs bit-exact, the others within the
    bar, and every output finite."""
    eb = 2 if kind in ("bf16", "fp16") else 1
    lib = _lib.load()
    for (M, N, Kb) in [(5, 80, 64), (37, 272, 192), (130, 160, 320), (300, 96, 576)]:
        K = Kb // eb
        w = workloads.custom(kind, M, N, K, seed=M + N + K, b_std=0.02 if kind == "int4" else 1.0)
        ops = workloads.make_operands(w)
        for variant in range(len(VARIANTS)):
            _say(f"half K tile {VARIANTS[variant]} {kind} {M}x{N}x{K}")
            if kind == "fp8":
                out = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
                a, b = H.dev_flat(ops["a"], gpu), H.dev_flat(ops["b_dev"], gpu)
                sa, sb = ops["sa"].to(gpu).contiguous(), ops["sb"].to(gpu).contiguous()
                _lib.check(lib.flygemm_preshuffle(out.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(),
                                                  sb.data_ptr(), M, N, K, _lib.FLYGEMM_IN["fp8"], 0, variant, None),
                           "flygemm_preshuffle")
            else:
                out = H.launch(ops, gpu, variant=variant, tile_k=64 // eb)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all(), f"{VARIANTS[variant]} {kind} {M}x{N}x{K}: non-finite output"
            ref = H.check(ops, out)
            if kind in ("int8", "int4"):
                assert np.array_equal(H.raw_acc(ops, gpu, variant).cpu().numpy(), ref)


@pytest.mark.parametrize("kind,M,N,K", [("fp8", 128, 4096, 4096), ("fp8_block", 33, 2112, 7168),
                                        ("fp8_block", 64, 2112, 7168), ("fp8_block", 256, 2112, 7168),
                                        ("int8", 128, 2048, 4096)])
def test_graph_capture_reference_pattern(gpu, kind, M, N, K):
    """The reference harness's graph path (tests/test_common.py:79-89 with the launcher of
    test_blockscale_preshuffle_gemm.py:199-213): eager launches on the current stream, then
    ``torch.cuda.graph(g)`` on torch's own capture stream, which has never run the shape.
    Every replay, with eager work of the same shape in between, equals the eager result."""
    ops = workloads.make_operands(workloads.custom(kind, M, N, K, seed=M + N))
    _say(f"graph capture {kind} {M}x{N}x{K} variant="
          f"{VARIANTS[_lib.load().flygemm_select_variant(M, N, K, 0 if kind == 'fp8_block' else _lib.FLYGEMM_IN[kind], int(kind == 'fp8_block'))]}")
    a = H.dev_flat(ops["a"], gpu)
    b = H.dev_flat(ops["b_dev"], gpu)
    sa = (ops["sa_t"] if kind == "fp8_block" else ops["sa"]).to(gpu).contiguous().view(-1)
    sb = ops["sb"].to(gpu).contiguous().view(-1)
    c = torch.zeros(M, N, dtype=torch.bfloat16, device=gpu)
    if kind == "fp8_block":
        from flydsl_amd.kernels.blockscale_preshuffle_gemm import compile_blockscale_preshuffle_gemm
        fn = compile_blockscale_preshuffle_gemm(M=M, N=N, K=K, tile_m=64, tile_n=128, tile_k=128, out_dtype="bf16")
    else:
        from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8
        fn = compile_preshuffle_gemm_a8(K=K, tile_m=64, tile_n=128, tile_k=128, in_dtype=kind, out_dtype="bf16")

    def launch_kernel():
        fn(c.view(-1), a, b, sa, sb, M, N, torch.cuda.current_stream())

    for _ in range(3):
        launch_kernel()
    torch.cuda.synchronize()
    eager = c.clone()
    H.check(ops, eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch_kernel()
    for i in range(3):
        c.zero_()
        other = H.launch(ops, gpu)  # eager work of the same shape between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, eager), f"replay {i}"
        assert torch.equal(other, eager)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_odd_k_tile_count_and_fp16_out(gpu, kind):
    """K = 8320 = 65 K tiles (reference test shape), fp16 output."""
    w = workloads.custom(kind, 160, 512, 8320, seed=9)
    ops = workloads.make_operands(w)
    _say(f"odd-k {kind} fp16")
    out = H.launch(ops, gpu, out_dtype="fp16")
    torch.cuda.synchronize()
    H.check(ops, out, out_dtype="fp16")


@pytest.mark.parametrize("M", [1, 7, 16, 33, 64])
@pytest.mark.parametrize("N,K", [(7168, 2304), (2112, 7168), (3072, 1536)])
def test_blockscale_reference_shapes(gpu, M, N, K):
    """The reference's DeepSeek-V3 blockscale shapes (test_blockscale_preshuffle_gemm.py:111-149)."""
    ops = workloads.make_operands(workloads.custom("fp8_block", M, N, K, seed=M * 7 + N))
    _say(f"blockscale {M}x{N}x{K}")
    out = H.launch(ops, gpu)
    torch.cuda.synchronize()
    H.check(ops, out)


# ---------------------------------------------------------------- streams, graphs, no-ops
def test_side_stream_and_zero_m(gpu):
    ops = workloads.make_operands(workloads.custom("int8", 48, 256, 512, seed=21))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = H.launch(ops, gpu, stream=s)
    s.synchronize()
    H.check(ops, out)
    c = torch.full((4,), 7.0, dtype=torch.bfloat16, device=gpu)
    lib = _lib.load()
    assert lib.flygemm_preshuffle(c.data_ptr(), c.data_ptr(), c.data_ptr(), c.data_ptr(), c.data_ptr(),
                                  0, 64, 128, 0, 0, -1, None) == 0
    torch.cuda.synchronize()
    assert (c.float() == 7.0).all()


def test_graph_replay(gpu):
    """Capture the launcher in a HIP graph; every replay (with eager work in between) must
    equal the eager result."""
    ops = workloads.make_operands(workloads.custom("fp8", 64, 1024, 1024, seed=31))
    eager = H.launch(ops, gpu)
    torch.cuda.synchronize()
    a = ops["a"].to(gpu).view(torch.int8).view(-1)
    b = ops["b_dev"].to(gpu).view(torch.int8).view(-1)
    sa, sb = ops["sa"].to(gpu).view(-1), ops["sb"].to(gpu).view(-1)
    c = torch.empty(64, 1024, dtype=torch.bfloat16, device=gpu)
    from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8
    fn = compile_preshuffle_gemm_a8(K=1024, tile_m=64, tile_n=128, tile_k=128, in_dtype="fp8", out_dtype="bf16")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(c.view(-1), a, b, sa, sb, 64, 1024, s)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn(c.view(-1), a, b, sa, sb, 64, 1024, torch.cuda.current_stream())
    for i in range(3):
        c.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, eager), f"replay {i}"


def test_compiled_fast_path_matches_launcher(gpu):
    """``flydsl_amd.compile(launcher, *args)`` (the reference's ``flyc.compile``) runs the launch
    once with its checks, then repeats it for new tensors, M and stream without them: the same
    bits as the launcher, for fp8, int8, blockscale and bf16, on the default and a side stream."""
    import flydsl_amd
    from flydsl_amd.kernels.blockscale_preshuffle_gemm import compile_blockscale_preshuffle_gemm
    from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8

    side = torch.cuda.Stream()
    for kind in ("fp8", "int8", "fp8_block", "bf16"):
        N, K = 512, 1024
        first, second = [workloads.make_operands(workloads.custom(kind, M, N, K, seed=M + 5)) for M in (64, 200)]
        if kind == "fp8_block":
            fn = compile_blockscale_preshuffle_gemm(M=64, N=N, K=K, tile_m=64, tile_n=128, tile_k=128, out_dtype="bf16")
        else:
            fn = compile_preshuffle_gemm_a8(K=K, tile_m=64, tile_n=128, tile_k=64 if kind == "bf16" else 128,
                                            in_dtype=kind, out_dtype="bf16")

        def args(ops, c):
            sa = ops["sa_t"] if kind == "fp8_block" else ops["sa"]
            return (c.view(-1), H.dev_flat(ops["a"], gpu), H.dev_flat(ops["b_dev"], gpu),
                    sa.to(gpu).contiguous().view(-1), ops["sb"].to(gpu).contiguous().view(-1))

        _say(f"compiled fast path {kind}")
        c1 = torch.empty(64, N, dtype=torch.bfloat16, device=gpu)
        cf = flydsl_amd.compile(fn, *args(first, c1), 64, N, torch.cuda.current_stream())
        torch.cuda.synchronize()
        want1 = H.launch(first, gpu)
        torch.cuda.synchronize()
        assert torch.equal(c1, want1)
        c2 = torch.zeros(200, N, dtype=torch.bfloat16, device=gpu)
        with torch.cuda.stream(side):
            cf(*args(second, c2), 200, N, side)
        side.synchronize()
        want2 = H.launch(second, gpu)
        torch.cuda.synchronize()
        assert torch.equal(c2, want2)
        H.check(second, c2)
        c1.zero_()
        cf(*args(first, c1), 64, N, torch.cuda.current_stream().cuda_stream)   # a raw stream handle
        torch.cuda.synchronize()
        assert torch.equal(c1, want1)
    with pytest.raises(RuntimeError, match="multiple of 16"):   # the C entry still checks sizes
        cf(*args(first, c1), 64, 100, None)
    with pytest.raises(ValueError, match="too small"):          # and every tensor's capacity
        cf(*args(first, c1), 65, N, None)
