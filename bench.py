"""Benchmark of the MI355X quantized preshuffle GEMM (one GPU).

    python bench.py [--steps K] [--warmup W] [--workload C2] [--secondary C1,C3,C4,C5,T,Q] [--no-cpu]

A step is one GEMM launch over the workload's operands, already resident in HBM.  The
headline workload is C2 (FP8 decode 16x28672x8192, HBM-bound): ``value`` is achieved GB/s
of algorithmic traffic (A + B + C + scales), timed with HIP events on the launch stream
around exactly K launches after W warm-up launches.  The other BASELINE configurations (C1,
C3, C4, C5), the FP8 8192^3 north-star shape T and the per-token quant kernel Q are measured
in the same run under ``secondary``: each is captured as a HIP graph of 50 launches and
timed over replays, so short kernels are timed at their own rate rather than at the host's
launch rate and MFMA-bound ones at the clock they hold under sustained load.  B (and A) are
rotated over several copies whose total exceeds the 256 MB last-level cache, so every
launch streams its operands from HBM.  The CPU baseline times the reference's CPU path
(dequantize, fp32 ``torch.mm``) on the host cores.

Profiling helpers (used by the commands recorded under profiles/):
    python bench.py --launches-only C2 --n 20   # only the GEMM launches of one workload
    python bench.py --copy-bytes 268435456      # a device-to-device copy of known size,
                                                # to calibrate FETCH_SIZE / WRITE_SIZE
``roofline.traffic`` (HBM bytes per launch) is read from profiles/hbm_traffic.md, which
records those counter runs; it is null when that file has no entry for the workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

from flydsl_amd import _lib, workloads
from flydsl_amd.kernels.blockscale_preshuffle_gemm import compile_blockscale_preshuffle_gemm
from flydsl_amd.kernels.preshuffle_gemm import compile_preshuffle_gemm_a8

METRIC = "FP8 GEMM TFLOP/s + % MFMA peak (large M); achieved HBM GB/s (small M)"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"fp8": 5000.0, "fp8_block": 5000.0, "int8": 5000.0, "int4": 5000.0, "bf16": 2500.0,
                    "fp16": 2500.0, "mxfp4": 10100.0}
LLC_BYTES = 256 << 20


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def _dev_flat(t, dev):
    """Flat device operand: 1-byte types viewed as int8 (as the reference harness passes fp8),
    2-byte types unchanged."""
    t = t.to(dev)
    return (t.view(torch.int8) if t.element_size() == 1 else t).view(-1)


class Runner:
    """Device operands (rotated copies) and a launch closure for one workload."""

    def __init__(self, w: workloads.Workload, dev, min_rotation_bytes=3 * LLC_BYTES):
        self.w = w
        ops = workloads.make_operands(w)
        per_call = ops["a"].numel() + ops["b_dev"].numel()
        copies = max(1, min(8, -(-min_rotation_bytes // per_call)))
        self.copies = copies
        self.a = [_dev_flat(ops["a"], dev) for _ in range(copies)]
        self.b = [_dev_flat(ops["b_dev"], dev) for _ in range(copies)]
        sa = ops["sa_t"] if w.kind == "fp8_block" else ops["sa"]
        self.sa = sa.to(dev).contiguous().view(-1)
        self.sb = ops["sb"].to(dev).contiguous().view(-1)
        self.c = torch.empty(w.M, w.N, dtype=torch.bfloat16, device=dev)
        if w.kind == "fp8_block":
            self.fn = compile_blockscale_preshuffle_gemm(M=w.M, N=w.N, K=w.K, tile_m=64, tile_n=128, tile_k=128,
                                                         out_dtype="bf16")
        else:
            self.fn = compile_preshuffle_gemm_a8(M=w.M, N=w.N, K=w.K, tile_m=128, tile_n=128, tile_k=128,
                                                 in_dtype="fp4" if w.kind == "mxfp4" else w.kind, out_dtype="bf16")
        self.variant = _lib.variants()[_lib.load().flygemm_select_variant(
            w.M, w.N, w.K, _lib.FLYGEMM_IN.get("fp4" if w.kind == "mxfp4" else w.kind, 0),
            int(w.kind == "fp8_block"))]
        del ops

    def launch(self, i, stream):
        j = i % self.copies
        self.fn(self.c.view(-1), self.a[j], self.b[j], self.sa, self.sb, self.w.M, self.w.N, stream)

    def time(self, steps, warmup, graph=False, replays=3, warm_s=0.1):
        """Average milliseconds per launch over ``steps`` launches, timed with HIP events on
        the launch stream.  ``graph``: the launches are captured once into a HIP graph, the
        graph is replayed untimed for at least ``warm_s`` seconds of back-to-back work (at
        least twice; the GPU reaches the clock it holds under sustained load only after some
        tens of milliseconds, and two replays of 50 launches of a 25 us kernel last 2.5 ms),
        and the median of ``replays`` timed replays is reported; a kernel shorter than the
        host's per-call cost (about 9 us through the Python launcher) is then timed at its own
        rate rather than at the rate the host can issue calls."""
        stream = torch.cuda.current_stream()
        for i in range(warmup):
            self.launch(i, stream)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                cap = torch.cuda.current_stream()
                for i in range(steps):
                    self.launch(i, cap)
            t_warm, n_warm = time.perf_counter(), 0
            while n_warm < 2 or (time.perf_counter() - t_warm < warm_s and n_warm < 2000):
                for _ in range(4 if n_warm >= 2 else 2):
                    g.replay()
                n_warm += 4 if n_warm >= 2 else 2
                torch.cuda.synchronize()
            times, walls = [], []
            for _ in range(replays):
                t0 = time.perf_counter()
                start.record(stream)
                g.replay()
                end.record(stream)
                torch.cuda.synchronize()
                walls.append(time.perf_counter() - t0)
                times.append(start.elapsed_time(end))
            k = sorted(range(replays), key=lambda j: times[j])[replays // 2]
            return times[k] / steps, walls[k]
        t0 = time.perf_counter()
        start.record(stream)
        for i in range(steps):
            self.launch(i, stream)
        end.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = start.elapsed_time(end)
        return ms / steps, wall


class QuantWorkload:
    """The reference's per-token quant benchmark (tests/kernels/test_quant.py:277-297):
    fp16 [M, N] uniform(-5, 5) with np.random.seed(42) -> int8 [M, N] + fp32 scales [M];
    bytes = 2MN + MN + 4M."""
    name, kind, note = "Q", "fp16->int8", "per-token quant (reference kernel semantics)"

    def __init__(self, M=4096, N=8192):
        self.M, self.N, self.K, self.seed = M, N, 0, 42
        self.bytes = 2 * M * N + M * N + 4 * M
        self.flops = 0


class QuantRunner:
    def __init__(self, w: QuantWorkload, dev, min_rotation_bytes=3 * LLC_BYTES):
        import numpy as np

        from flydsl_amd.kernels.quant import build_quant_module
        self.w = w
        np.random.seed(w.seed)
        x = torch.from_numpy(np.random.uniform(-5.0, 5.0, size=(w.M, w.N)).astype(np.float16))
        per_call = w.bytes
        self.copies = max(1, min(8, -(-min_rotation_bytes // per_call)))
        self.x = [x.to(dev) for _ in range(self.copies)]
        self.out = [torch.empty(w.M, w.N, dtype=torch.int8, device=dev) for _ in range(self.copies)]
        self.sc = torch.empty(w.M, dtype=torch.float32, device=dev)
        self.fn, _ = build_quant_module(w.N)
        self.variant = "quant_rows_recip_trunc"

    def launch(self, i, stream):
        j = i % self.copies
        self.fn(self.x[j], self.out[j], self.sc, self.w.M, stream)

    time = Runner.time


class MoeStageWorkload:
    """One stage of an MoE layer (``workloads.MOE_WORKLOADS``): M = routes (tokens * topk),
    N = the stage's output width, K = its reduction width; bytes = the active experts' weights
    plus activations, scales, outputs and routing metadata once; flops = 2 * routes * N_total * K
    (stage 1 counts gate and up)."""

    def __init__(self, name: str, base: workloads.MoeWorkload, stage: int, active_experts: int):
        self.name, self.base, self.stage, self.kind = name, base, stage, base.kind
        self.M = base.routes
        self.N = 2 * base.inter_dim if stage == 1 else base.model_dim
        self.K = base.model_dim if stage == 1 else base.inter_dim
        self.seed = base.seed
        self.flops = base.flops1 if stage == 1 else base.flops2
        self.bytes = workloads.moe_bytes(base, stage, active_experts)
        self.note = f"MoE stage {stage}, {base.note}: {base.tokens} tokens, E={base.experts} top-{base.topk}, " \
                    f"model_dim {base.model_dim}, inter_dim {base.inter_dim}, {active_experts} experts active"


# bench name -> (MoE workload, stage)
# (the R variants run stage 2 in reduce mode: per-route rows, then the top-k reduction)
MOE_BENCH = {"MP1": ("DSP", 1), "MP2": ("DSP", 2), "MP2R": ("DSP", 2), "MD1": ("DSD", 1), "MD2": ("DSD", 2),
             "MD2R": ("DSD", 2), "MB1": ("DSB", 1), "MB2": ("DSB", 2),
             "MG1": ("RBL", 1), "MG2": ("RBL", 2), "MH1": ("RBS", 1), "MH2": ("RBS", 2)}


class MoeRunner:
    def __init__(self, name: str, dev, min_rotation_bytes=0):
        from flydsl_amd.kernels.moe_gemm_2stage import compile_moe_gemm1, compile_moe_gemm2

        key, stage = MOE_BENCH[name]
        base = workloads.MOE_WORKLOADS[key]
        p = workloads.moe_problem(base, dev, with_stage2_input=stage == 2)
        active = int(torch.unique(p["topk_ids"]).numel())
        self.w = MoeStageWorkload(name, base, stage, active)
        self.p, self.stage = p, stage
        kw = dict(model_dim=base.model_dim, inter_dim=base.inter_dim, experts=base.experts, topk=base.topk,
                  tile_m=base.tile_m, tile_k=128, in_dtype=base.kind)
        if base.kind == "fp8_block":
            from flydsl_amd.kernels.moe_blockscale_2stage import (compile_moe_blockscale_gemm1,
                                                                  compile_moe_blockscale_gemm2)
            kw.pop("in_dtype")
            compile_moe_gemm1 = lambda **k: compile_moe_blockscale_gemm1(**k)   # noqa: E731
            compile_moe_gemm2 = lambda **k: compile_moe_blockscale_gemm2(**k)   # noqa: E731
        if stage == 1:
            self.fn = compile_moe_gemm1(**kw, tile_n=base.tile_n1, doweight_stage1=False, out_dtype="f16")
            self.out = torch.empty(base.tokens, base.topk, base.inter_dim, dtype=torch.float16, device=dev)
            self.args = (_dev_flat(p["x"], dev), _dev_flat(p["w1_shuf"], dev), p["sx"], p["sw1"])
            self.nk = (base.inter_dim, base.model_dim)
        elif name.endswith("R"):
            from flydsl_amd.kernels.moe_gemm_2stage import MoeGemm2Mode, compile_moe_gemm2_ex
            # every route is written (no mask), so the intermediate needs no zeroing
            self.fn = compile_moe_gemm2_ex(**kw, tile_n=base.tile_n2, doweight_stage2=True, out_dtype="f16",
                                           mode=MoeGemm2Mode.REDUCE, zero_intermediate=False)
            self.out = torch.zeros(base.tokens, base.model_dim, dtype=torch.float16, device=dev)
            self.args = (_dev_flat(p["a2"], dev), _dev_flat(p["w2_shuf"], dev), p["sa2"], p["sw2"])
            self.nk = (base.model_dim, base.inter_dim)
        else:
            self.fn = compile_moe_gemm2(**kw, tile_n=base.tile_n2, doweight_stage2=True, out_dtype="f16")
            self.out = torch.zeros(base.tokens, base.model_dim, dtype=torch.float16, device=dev)
            self.args = (_dev_flat(p["a2"], dev), _dev_flat(p["w2_shuf"], dev), p["sa2"], p["sw2"])
            self.nk = (base.model_dim, base.inter_dim)
        self.copies = 1
        # the library picks the column tile and the rows per workgroup (profiles name the kernel)
        self.variant = f"moe_gemm{stage} tile_m={base.tile_m}" + (" +reduce" if name.endswith("R") else "")

    def launch(self, i, stream):
        p, b = self.p, self.w.base
        self.fn(self.out, *self.args, p["sorted_ids"], p["sorted_expert_ids"], p["sorted_weights"],
                p["num_valid_ids"], b.tokens, self.nk[0], self.nk[1], p["blocks"], stream)

    time = Runner.time


def make_runner(name, dev, **kw):
    if name == "Q":
        return QuantRunner(QuantWorkload(), dev, **kw)
    if name in MOE_BENCH:
        return MoeRunner(name, dev, **kw)
    return Runner(workloads.WORKLOADS[name], dev, **kw)


def roofline(w: workloads.Workload, ms_per_launch: float, bound: str, traffic=None):
    if bound == "hbm":
        achieved = w.bytes / (ms_per_launch * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic}
    achieved = w.flops / (ms_per_launch * 1e-3) / 1e12
    peak = MFMA_PEAK_TFLOPS[w.kind]
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic}


def cpu_baseline(w: workloads.Workload):
    """The reference's CPU path for this GEMM, timed on the host: dequantize A and B to fp32
    with their scales, ``torch.mm`` in fp32 on all host cores, cast to bf16 (``run_torch``,
    reference tests/kernels/test_preshuffle_gemm.py:55-65; blockscale: the 1x128 / 128x128
    scale expansion of ``run_torch_blockscale``, test_blockscale_preshuffle_gemm.py:86-109;
    bf16/fp16: no scales), on the full call of the workload's seeded operands; 1 warm-up,
    median of 3.  The oracle's numpy float32 restatement of the same
    path is timed once as a second figure.  MXFP4 has no CPU baseline here (its e2m1 bytes
    are not a torch dtype)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import gemm as og

    if w.kind not in ("fp8", "int8", "int4", "fp8_block", "bf16", "fp16"):
        raise ValueError(f"no CPU baseline for kind {w.kind!r}")
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ops = workloads.make_operands(w)
    a_q, b_q = ops["a"], ops["b"]
    if w.kind == "fp8_block":
        sa = ops["sa"].float().repeat_interleave(128, dim=1)[:, : w.K]
        sb = ops["sb"].float().repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)[: w.N, : w.K]
    elif w.kind in ("bf16", "fp16"):
        sa = sb = torch.ones(1, 1)
    else:
        sa, sb = ops["sa"].reshape(-1, 1).float(), ops["sb"].reshape(-1, 1).float()

    def run_torch():
        a = a_q.to(torch.float32) * sa
        b = b_q.to(torch.float32) * sb
        return torch.mm(a, b.t()).to(torch.bfloat16)

    run_torch()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run_torch()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]

    def raw(x):
        if x.dtype in (torch.bfloat16, torch.float16):
            return x.view(torch.int16).numpy().view(np.uint16)
        return x.view(torch.uint8).numpy() if x.dtype != torch.int8 else x.numpy()

    with threadpool_limits(limits=cores):
        t0 = time.perf_counter()
        if w.kind == "fp8_block":
            og.run_torch_blockscale(raw(a_q), raw(b_q), ops["sa"].numpy(), ops["sb"].numpy())
        elif w.kind in ("bf16", "fp16"):
            og.run_torch(raw(a_q), raw(b_q), None, None, w.kind)
        else:
            og.run_torch(raw(a_q), raw(b_q), ops["sa"].numpy().reshape(-1), ops["sb"].numpy().reshape(-1),
                         "fp8" if w.kind == "fp8" else "int8")
        t_np = time.perf_counter() - t0
    return {"value": round(w.bytes / t / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full {w.name} call ({w.M}x{w.N}x{w.K}): dequantize to fp32, torch.mm fp32 on {cores} threads, "
                      f"cast to bf16; median of 3 after 1 warm-up: {t * 1e3:.1f} ms = {w.flops / t / 1e12:.4f} TFLOP/s "
                      f"(oracle numpy float32 restatement, one run: {t_np * 1e3:.1f} ms)",
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def traffic_from_profile(name: str):
    """HBM bytes per launch recorded in profiles/hbm_traffic.md (line 'traffic <W> <bytes>')."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.strip().strip("`").split()
        if len(parts) == 3 and parts[0] == "traffic" and parts[1] == name:
            return int(parts[2])
    return None


def gfx_clock_under(work, dev, work_ms, seconds=0.5):
    """Median shader clock (MHz) while ``work`` (a graph replay on the current stream, about
    ``work_ms`` long) runs: a one-wave probe on a side stream counts core cycles (s_memtime)
    against the 100 MHz constant counter over half the replay, at most 2 ms, so each sample
    averages the clock over many launches (``flydsl_amd/_clockprobe.so``).  A sample counts
    only if the probe ended before the replay did (a second, one-tick probe queued behind the
    replay on its stream gives the replay's end), so the clock is the one under load.  None if
    the probe is not built or no sample overlapped."""
    import ctypes

    from flydsl_amd.build import PROBE_OUT
    if not os.path.exists(PROBE_OUT):
        log("[bench] no clock probe library: the line goes without a clock")
        return None
    probe = ctypes.CDLL(PROBE_OUT).flygemm_clock_probe
    probe.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_void_p]
    out = torch.zeros(4, dtype=torch.int64, device=dev)
    end = torch.zeros(4, dtype=torch.int64, device=dev)
    main, side = torch.cuda.current_stream(), torch.cuda.Stream()
    vals, tries = [], 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0 < seconds or len(vals) < 5) and tries < 200:
        tries += 1
        work()
        ticks = max(1000, min(200000, int(work_ms * 0.5 * 1e5)))   # 100 MHz ticks
        if probe(out.data_ptr(), ticks, side.cuda_stream) or probe(end.data_ptr(), 1, main.cuda_stream):
            return None
        torch.cuda.synchronize()
        cyc, ticks, _, r_end = out.tolist()
        if r_end + 100 < end.tolist()[2]:
            vals.append(cyc / (ticks / 100.0))
    log(f"[bench] clock probe: {len(vals)} of {tries} samples overlapped the work")
    if not vals:
        return None
    vals.sort()
    return round(vals[len(vals) // 2])


def dispatch_cost(dev, calls=1000):
    """Host cost of one eager call (microseconds), on a 1x64x128 fp8 GEMM: the validating
    launcher, the pre-bound callable of ``flydsl_amd.compile`` and the bare ctypes call; and C1
    timed eagerly through the pre-bound callable (HIP events around 200 back-to-back launches)
    against its graph-replay time."""
    import flydsl_amd

    def host_us(fn):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        t = time.perf_counter() - t0
        torch.cuda.synchronize()
        return round(t / calls * 1e6, 2)

    w = workloads.custom("fp8", 1, 64, 128, seed=0)
    ops = workloads.make_operands(w)
    a, b = _dev_flat(ops["a"], dev), _dev_flat(ops["b_dev"], dev)
    sa, sb = ops["sa"].to(dev).view(-1), ops["sb"].to(dev).view(-1)
    c = torch.empty(w.M * w.N, dtype=torch.bfloat16, device=dev)
    fn = compile_preshuffle_gemm_a8(K=w.K, tile_m=32, tile_n=128, tile_k=128, in_dtype="fp8", out_dtype="bf16")
    s = torch.cuda.current_stream()
    h = s.cuda_stream
    cf = flydsl_amd.compile(fn, c, a, b, sa, sb, w.M, w.N, h)
    lib = _lib.load()
    pc, pa, pb, psa, psb = c.data_ptr(), a.data_ptr(), b.data_ptr(), sa.data_ptr(), sb.data_ptr()
    out = {"shape": f"fp8 {w.M}x{w.N}x{w.K}", "calls": calls,
           "launcher_us": host_us(lambda: fn(c, a, b, sa, sb, w.M, w.N, s)),
           "compiled_us": host_us(lambda: cf(c, a, b, sa, sb, w.M, w.N, h)),
           "ctypes_us": host_us(lambda: lib.flygemm_preshuffle(pc, pa, pb, psa, psb, w.M, w.N, w.K, 0, 0, -1, h))}
    r = Runner(workloads.WORKLOADS["C1"], dev)
    cc = flydsl_amd.compile(r.fn, r.c.view(-1), r.a[0], r.b[0], r.sa, r.sb, r.w.M, r.w.N, h)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 200
    for i in range(20):
        cc(r.c.view(-1), r.a[i % r.copies], r.b[i % r.copies], r.sa, r.sb, r.w.M, r.w.N, h)
    torch.cuda.synchronize()
    ev0.record(s)
    for i in range(n):
        cc(r.c.view(-1), r.a[i % r.copies], r.b[i % r.copies], r.sa, r.sb, r.w.M, r.w.N, h)
    ev1.record(s)
    torch.cuda.synchronize()
    out["C1_eager_ms"] = round(ev0.elapsed_time(ev1) / n, 5)
    out["C1_graph_ms"] = round(r.time(50, 2, graph=True)[0], 5)
    return out


def launches_only(name: str, n: int):
    dev = torch.device("cuda:0")
    r = make_runner(name, dev, min_rotation_bytes=0)
    stream = torch.cuda.current_stream()
    for i in range(n):
        r.launch(i, stream)
    torch.cuda.synchronize()
    log(f"[bench] {n} launches of {name} ({r.variant}) done")


def copy_bytes(nbytes: int, n: int = 5):
    dev = torch.device("cuda:0")
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(n):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] {n} copies of {nbytes} bytes done")


def vs_library(n: int = 50):
    """Context for the roofline fractions: the same shapes through ROCm's own GEMM library
    (hipBLASLt via torch._scaled_mm / torch._int_mm / torch.mm), operands resident and reused,
    per-tensor and per-row scales.  Prints one JSON line; nothing here is the product path."""
    dev = torch.device("cuda:0")

    def timeit(fn):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    res = {}
    g = torch.Generator(device=dev).manual_seed(0)
    for name in ("T", "C1", "C2", "C4"):
        w = workloads.WORKLOADS[name]
        a = torch.randn(w.M, w.K, device=dev, generator=g).to(torch.float8_e4m3fn)
        b = torch.randn(w.N, w.K, device=dev, generator=g).to(torch.float8_e4m3fn)
        for mode in ("tensor", "rowwise"):
            sa = torch.ones((), device=dev) if mode == "tensor" else torch.ones(w.M, 1, device=dev)
            sb = torch.ones((), device=dev) if mode == "tensor" else torch.ones(1, w.N, device=dev)
            try:
                ms = timeit(lambda: torch._scaled_mm(a, b.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16))
                res[f"{name}_fp8_{mode}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(w.flops / ms / 1e9, 1)}
            except Exception as e:  # a scaling mode the library lacks
                res[f"{name}_fp8_{mode}"] = {"error": f"{type(e).__name__}: {str(e)[:120]}"}
        del a, b
    for name, dt in (("C3", torch.int8), ("T16", torch.bfloat16)):
        w = workloads.WORKLOADS[name]
        if dt == torch.int8:
            a = torch.randint(-127, 127, (w.M, w.K), device=dev, dtype=dt, generator=g)
            b = torch.randint(-127, 127, (w.N, w.K), device=dev, dtype=dt, generator=g)
            fn = lambda: torch._int_mm(a, b.t())
        else:
            a = torch.randn(w.M, w.K, device=dev, dtype=dt, generator=g)
            b = torch.randn(w.N, w.K, device=dev, dtype=dt, generator=g)
            fn = lambda: torch.mm(a, b.t())
        ms = timeit(fn)
        res[name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(w.flops / ms / 1e9, 1)}
        del a, b
    print(json.dumps({"library": "hipBLASLt (torch)", "results": res}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="C2")
    ap.add_argument("--secondary", default="C1,C3,C4,C5,T,Q,G1,G2,G3,G4,G5,G6,G7",
                    help="extra workloads, comma separated ('' to skip)")
    ap.add_argument("--secondary-launches", type=int, default=50,
                    help="launches per timed graph replay of each secondary workload")
    ap.add_argument("--all", action="store_true", help="also time every configuration")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-dispatch", action="store_true", help="skip the host dispatch-cost line")
    ap.add_argument("--launches-only", default="", help="profiling: only launch this workload --n times")
    ap.add_argument("--n", type=int, default=20)
    ap.add_argument("--copy-bytes", type=int, default=0, help="profiling: copy this many bytes on the GPU")
    ap.add_argument("--vs-library", action="store_true", help="time the same shapes through hipBLASLt (context)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path: run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    _lib.load()
    if args.launches_only:
        launches_only(args.launches_only, args.n)
        return
    if args.copy_bytes:
        copy_bytes(args.copy_bytes)
        return
    if args.vs_library:
        vs_library()
        return

    w = workloads.WORKLOADS[args.workload]
    log(f"[bench] preparing {w.name} {w.kind} {w.M}x{w.N}x{w.K}")
    r = Runner(w, dev)
    log(f"[bench] timing {w.name} variant={r.variant} copies={r.copies}")
    ms, wall = r.time(args.steps, args.warmup)
    bound = "hbm" if w.name in ("C1", "C2") else "mfma"
    gbs = w.bytes * args.steps / (ms * args.steps * 1e-3) / 1e9
    result = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8" if "fp8" in w.kind else ("int8" if w.kind == "int8" else "int4xint8"),
        "data": "synthetic (seeded N(0,1), quantized per BASELINE)",
        "config": {"workload": f"{w.name}: {w.note} {w.M}x{w.N}x{w.K} seed {w.seed}", "M": w.M, "N": w.N,
                   "K": w.K, "kernel": r.variant, "wall_s": round(wall, 4)},
        "roofline": roofline(w, ms, "hbm", traffic_from_profile(w.name)),
    }
    if bound == "mfma":
        result["roofline_mfma"] = roofline(w, ms, "mfma")
    del r
    torch.cuda.empty_cache()

    extra = [n for n in args.secondary.split(",") if n]
    if args.all:
        extra += [n for n in list(workloads.WORKLOADS) + ["Q"] + list(MOE_BENCH)
                  if n not in extra and n != args.workload]
    sec = {}
    for name in extra:
        r2 = make_runner(name, dev)
        w2 = r2.w
        log(f"[bench] preparing {name} {w2.kind} {w2.M}x{w2.N}x{w2.K}")
        log(f"[bench] timing {name} variant={r2.variant}")
        n2 = max(50, args.secondary_launches)
        ms2, _ = r2.time(n2, max(2, args.warmup // 2), graph=True)
        b2 = "hbm" if name in ("C1", "C2", "G1", "G2", "Q", "MD1", "MD2", "MD2R", "MB1", "MB2", "MH1", "MH2") else "mfma"
        sec[name] = {"ms": round(ms2, 5), "GB/s": round(w2.bytes / ms2 / 1e6, 1), "kernel": r2.variant,
                     "timing": f"HIP graph of {n2} launches, median of 3 timed replays after >= 0.1 s of untimed ones",
                     "roofline": roofline(w2, ms2, b2, traffic_from_profile(name))}
        if w2.flops:
            sec[name]["TFLOP/s"] = round(w2.flops / ms2 / 1e9, 1)
        if b2 == "mfma" and name not in MOE_BENCH:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                cap = torch.cuda.current_stream()
                for i in range(n2):
                    r2.launch(i, cap)
            clk = gfx_clock_under(g.replay, dev, ms2 * n2)
            del g
            if clk:
                # the dense peak assumes 2.4 GHz; under sustained MFMA load the chip holds less
                sec[name]["clock_mhz"] = clk
                sec[name]["frac_at_clock"] = round(sec[name]["roofline"]["frac"] * 2400.0 / clk, 4)
        del r2
        torch.cuda.empty_cache()
    if sec:
        result["secondary"] = sec
    if not args.no_dispatch:
        result["dispatch"] = dispatch_cost(dev)
    if not args.no_cpu:
        log("[bench] CPU baseline")
        result["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
