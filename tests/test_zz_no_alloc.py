"""GPU check of ``flygemm_moe_gemm2_reduce_noalloc``, MoE stage 2 in reduce mode in one call that
allocates nothing (its per-route rows live in the library's static device array).

Its output must equal, bit for bit, what the entry points it stands in for give on the same
inputs: ``flygemm_moe_gemm2`` with ``accumulate = 0`` into a caller-allocated (zeroed)
intermediate, then ``flygemm_moe_reduce`` (the same kernels in the same order).  Covered: two
calls in a row with the second smaller (the array keeps the first call's rows), fp16 and bf16,
fp8 / bf16 / int4_bf16 (group scales) inputs, a valid mask, ``zero_intermediate = 0`` with every
route written, graph capture with replays, and the size limit (rejected before any launch, the
output left untouched).  Every case calls through the C-ABI with ctypes."""
import numpy as np
import pytest
import torch

from flydsl_amd import _lib
from flydsl_amd import workloads as W

pytestmark = pytest.mark.gpu
OUT_T = {"fp16": torch.float16, "bf16": torch.bfloat16}
SCRATCH_BYTES = 64 << 20       # FLYGEMM_MOE_NOALLOC_SCRATCH_BYTES in include/flygemm.h


def _say(msg):
    print(msg, flush=True)


def _ptr(t):
    return 0 if t is None else t.data_ptr()


def _problem(shape, kind, dev, tokens=None, group_size=-1, seed=0):
    b = W.MOE_WORKLOADS[shape] if isinstance(shape, str) else shape
    w = W.MoeWorkload(b.name, tokens or b.tokens, b.model_dim, b.inter_dim, b.experts, b.topk, b.tile_m, b.tile_n1,
                      b.tile_n2, kind, seed)
    return W.moe_problem(w, dev, group_size=group_size)


def _args(p, out_dtype, doweight, group_size):
    w = p["workload"]
    return ([p["a2"].data_ptr(), p["w2_shuf"].data_ptr(), _ptr(p["sa2"]), _ptr(p["sw2"]), p["sorted_ids"].data_ptr(),
             p["sorted_expert_ids"].data_ptr(), p["sorted_weights"].data_ptr(), p["num_valid_ids"].data_ptr(),
             w.tokens, w.model_dim, w.inter_dim, p["blocks"], w.experts, w.topk, w.tile_m, 0,
             _lib.FLYGEMM_IN[w.kind], _lib.FLYGEMM_OUT[out_dtype], int(doweight)])


def two_calls(p, out_dtype, doweight=True, group_size=-1, mask=None):
    """The existing entry points: per-route rows into a zeroed torch buffer, then the reduction."""
    w = p["workload"]
    lib = _lib.load()
    s = torch.cuda.current_stream().cuda_stream
    inter = torch.zeros(w.tokens * w.topk, w.model_dim, dtype=OUT_T[out_dtype], device=p["a2"].device)
    out = torch.full((w.tokens, w.model_dim), float("nan"), dtype=OUT_T[out_dtype], device=p["a2"].device)
    rc = lib.flygemm_moe_gemm2(inter.data_ptr(), *_args(p, out_dtype, doweight, group_size), 0, group_size, s)
    _lib.check(rc, "flygemm_moe_gemm2")
    rc = lib.flygemm_moe_reduce(out.data_ptr(), inter.data_ptr(), _ptr(mask), w.tokens, w.topk, w.model_dim,
                                _lib.FLYGEMM_OUT[out_dtype], s)
    _lib.check(rc, "flygemm_moe_reduce")
    return out


def noalloc(p, out_dtype, doweight=True, group_size=-1, mask=None, zero=1, out=None):
    w = p["workload"]
    if out is None:
        out = torch.full((w.tokens, w.model_dim), float("nan"), dtype=OUT_T[out_dtype], device=p["a2"].device)
    rc = _lib.load().flygemm_moe_gemm2_reduce_noalloc(out.data_ptr(), *_args(p, out_dtype, doweight, group_size),
                                                      group_size, _ptr(mask), zero,
                                                      torch.cuda.current_stream().cuda_stream)
    return rc, out


def _same(a, b, what):
    torch.cuda.synchronize()
    x = a.view(torch.int16).cpu().numpy()
    y = b.view(torch.int16).cpu().numpy()
    bad = np.argwhere(x != y)
    assert bad.size == 0, f"{what}: {len(bad)} outputs differ, first at {tuple(bad[0])}"
    assert torch.isfinite(a.float()).all(), f"{what}: non-finite output"


def test_first_call_under_capture_is_refused(gpu):
    """The scratch address is resolved on a device's first call, which must not run under graph
    capture: such a call returns an error naming the rule and launches nothing (the capture ends
    empty, the output untouched); an eager call then resolves the address, and a captured call
    replays to the two-call result.  (Kept first in this file: it needs the process's first call.)"""
    p = _problem("MS", "fp8", gpu, seed=5)
    w = p["workload"]
    lib = _lib.load()
    out = torch.full((w.tokens, w.model_dim), float("nan"), dtype=torch.float16, device=gpu)
    torch.cuda.synchronize()
    _say("no-alloc: first call under capture")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.flygemm_moe_gemm2_reduce_noalloc(out.data_ptr(), *_args(p, "fp16", True, -1), -1, None, 1,
                                                  torch.cuda.current_stream().cuda_stream)
    if rc == 0:
        pytest.skip("the scratch address was already resolved in this process (not its first call)")
    assert b"graph capture" in lib.flygemm_last_error()
    g.replay()
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all(), "the refused call wrote the output"
    want = two_calls(p, "fp16")
    rc, eager = noalloc(p, "fp16")      # resolves the address
    _lib.check(rc, "flygemm_moe_gemm2_reduce_noalloc")
    _same(eager, want, "eager after the refused capture")
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        rc = lib.flygemm_moe_gemm2_reduce_noalloc(out.data_ptr(), *_args(p, "fp16", True, -1), -1, None, 1,
                                                  torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.flygemm_last_error()
    for i in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g2.replay()
        _same(out, want, f"captured replay {i}")


CASES = [  # (shape, kind, group, out dtype, first tokens (None: the shape's), second (smaller) tokens)
    ("MM", "fp8", -1, "fp16", None, 40),
    ("MM", "bf16", -1, "bf16", None, 17),
    ("MM", "int4_bf16", 32, "bf16", None, 64),
    ("DSD", "fp8", -1, "bf16", None, 3),
    # 600 tokens top-2 of 8 experts: a full 128-row run per expert, so the GEMM runs the
    # stage-2 stream kernel; the second call (100 tokens) the single-block kernel
    ("MM", "fp8", -1, "bf16", 600, 100),
]


@pytest.mark.parametrize("shape,kind,group,out_dtype,tokens1,tokens2", CASES)
def test_noalloc_matches_two_calls_twice(gpu, shape, kind, group, out_dtype, tokens1, tokens2):
    """Two calls in a row, the second with fewer tokens (and other data), each equal to the
    existing two-call reduce mode bit for bit."""
    for tokens, seed in ((tokens1, 0), (tokens2, 7)):
        p = _problem(shape, kind, gpu, tokens=tokens, group_size=group, seed=seed)
        w = p["workload"]
        _say(f"noalloc {shape} {kind} g={group} {out_dtype} tokens={w.tokens}")
        rc, got = noalloc(p, out_dtype, group_size=group)
        _lib.check(rc, "flygemm_moe_gemm2_reduce_noalloc")
        _same(got, two_calls(p, out_dtype, group_size=group), f"{shape} {kind} tokens={w.tokens}")


def test_noalloc_mask_and_no_zeroing(gpu):
    """A valid mask (the rows it skips are never read) and zero_intermediate = 0 with every route
    written: both equal the two-call path, after a larger call has left other rows behind."""
    big = _problem("MM", "fp8", gpu, seed=3)
    _lib.check(noalloc(big, "fp16")[0], "noalloc (fill)")
    p = _problem("MM", "fp8", gpu, tokens=50, seed=4)
    w = p["workload"]
    g = torch.Generator().manual_seed(11)
    mask = (torch.rand(w.tokens, w.topk, generator=g) < 0.7).to(torch.int8).to(gpu)
    _say("noalloc mask")
    rc, got = noalloc(p, "fp16", mask=mask.view(-1))
    _lib.check(rc, "noalloc mask")
    _same(got, two_calls(p, "fp16", mask=mask.view(-1)), "mask")
    _say("noalloc zero_intermediate=0")
    rc, got = noalloc(p, "fp16", zero=0)
    _lib.check(rc, "noalloc no zeroing")
    _same(got, two_calls(p, "fp16"), "zero_intermediate=0")


def test_noalloc_graph_capture(gpu):
    """Captured once (after an eager call resolved the array's address), replayed three times
    with eager work in between; every replay equals the two-call path."""
    p = _problem("MM", "fp8", gpu, seed=5)
    w = p["workload"]
    ref = two_calls(p, "bf16")
    _lib.check(noalloc(p, "bf16")[0], "noalloc eager")
    out = torch.full((w.tokens, w.model_dim), float("nan"), dtype=torch.bfloat16, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        rc, _ = noalloc(p, "bf16", out=out)
    torch.cuda.current_stream().wait_stream(side)
    _lib.check(rc, "noalloc under capture")
    for i in range(3):
        out.fill_(float("nan"))
        other = _problem("MM", "fp8", gpu, tokens=20, seed=20 + i)     # eager use of the array between replays
        _lib.check(noalloc(other, "bf16")[0], "noalloc between replays")
        _say(f"noalloc replay {i}")
        g.replay()
        _same(out, ref, f"replay {i}")


def test_noalloc_rejects_above_the_scratch(gpu):
    """tokens*topk*model_dim*2 above the array: an error before any launch, output untouched."""
    p = _problem("DSD", "fp8", gpu)
    w = p["workload"]
    tokens = SCRATCH_BYTES // (w.topk * w.model_dim * 2) + 1
    out = torch.full((w.tokens, w.model_dim), 3.0, dtype=torch.bfloat16, device=gpu)
    args = _args(p, "bf16", True, -1)
    args[8] = tokens          # more tokens than the array holds rows for
    rc = _lib.load().flygemm_moe_gemm2_reduce_noalloc(out.data_ptr(), *args, -1, 0, 1,
                                                      torch.cuda.current_stream().cuda_stream)
    assert rc != 0
    assert "static scratch" in _lib.load().flygemm_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
    rc, _ = noalloc(p, "bf16")
    _lib.check(rc, "noalloc after a rejected call")
