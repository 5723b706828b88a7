"""The measured workloads and their seeded synthetic operands.

Five configurations plus the large square FP8 shape used for the MFMA-throughput target.
Operands are drawn on the CPU from ``torch.Generator().manual_seed(seed)`` (A first,
then B), quantized with ``flydsl_amd.quant`` and preshuffled, so every process that asks
for a configuration sees the same bytes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import fp4, quant


@dataclass(frozen=True)
class Workload:
    name: str
    kind: str          # "fp8" | "int8" | "int4" | "fp8_block" | "bf16" | "fp16" | "mxfp4"
    M: int
    N: int
    K: int
    seed: int
    b_std: float = 1.0
    note: str = ""

    @property
    def flops(self) -> int:
        return 2 * self.M * self.N * self.K

    @property
    def bytes(self) -> int:
        """Algorithmic bytes: A + B + C(bf16) + fp32 scales (reference test_preshuffle_gemm.py:254,
        test_blockscale_preshuffle_gemm.py:222)."""
        M, N, K = self.M, self.N, self.K
        if self.kind in ("bf16", "fp16"):
            return 2 * (M * K + N * K + M * N)   # no scales
        if self.kind == "mxfp4":   # reference test_preshuffle_gemm.py:371-374
            return M * K // 2 + N * K // 2 + 2 * M * N + (M + N) * (K // 32)
        b = N * K // 2 if self.kind == "int4" else N * K
        base = M * K + b + 2 * M * N
        if self.kind == "fp8_block":
            return base + 4 * (M * (K // 128) + ((N + 127) // 128) * (K // 128))
        return base + 4 * (M + N)


WORKLOADS = {
    "C1": Workload("C1", "fp8", 128, 4096, 4096, 0, note="FP8 per-token/per-channel"),
    "C2": Workload("C2", "fp8", 16, 28672, 8192, 1, note="FP8 decode, HBM-bound"),
    "C3": Workload("C3", "int8", 4096, 4096, 4096, 2, note="INT8 W8A8"),
    "C4": Workload("C4", "fp8_block", 1024, 7168, 7168, 3, note="FP8 1x128/128x128 blockscale"),
    "C5": Workload("C5", "int4", 256, 14336, 4096, 4, b_std=0.02, note="W4A8"),
    "T": Workload("T", "fp8", 8192, 8192, 8192, 5, note="FP8 8192^3, MFMA-bound target"),
    "T16": Workload("T16", "bf16", 8192, 8192, 8192, 6, note="BF16 8192^3 (in_dtype='bf16', unscaled)"),
    "F4": Workload("F4", "mxfp4", 8192, 8192, 8192, 7, note="MXFP4 8192^3 (1x32 E8M0 block scales)"),
    # the reference's GEMM benchmark list (scripts/run_benchmark.sh:71-79) beyond T
    "G1": Workload("G1", "fp8", 16, 40960, 5120, 8, note="FP8 decode (reference benchmark list)"),
    "G2": Workload("G2", "fp8", 16, 77824, 5120, 9, note="FP8 decode (reference benchmark list)"),
    "G3": Workload("G3", "fp8", 5120, 5120, 8320, 10, note="FP8 (reference benchmark list)"),
    "G4": Workload("G4", "fp8", 9728, 8192, 8320, 11, note="FP8 (reference benchmark list)"),
    "G5": Workload("G5", "int8", 9728, 8192, 8320, 12, note="INT8 W8A8 (reference benchmark list)"),
    "G6": Workload("G6", "int4", 9728, 8192, 8320, 13, b_std=0.02, note="W4A8 (reference benchmark list)"),
    "G7": Workload("G7", "bf16", 5120, 5120, 8320, 14, note="BF16 (reference benchmark list)"),
}


def custom(kind: str, M: int, N: int, K: int, seed: int, b_std: float = 1.0) -> Workload:
    return Workload(f"{kind}_{M}x{N}x{K}_s{seed}", kind, M, N, K, seed, b_std)


def make_operands(w: Workload) -> dict:
    """CPU operands for workload ``w``.

    Keys: ``a`` (A quantized, [M, K]), ``b`` (B quantized, unshuffled [N, K], int8 values for
    int4), ``b_dev`` (the B buffer the kernel reads: shuffled, int4 packed), ``sa``, ``sb``
    (fp32 scales; blockscale: ``sa`` is [M, K/128] and ``sa_t`` its [K/128, M] transpose,
    ``sb`` is [N/128, K/128]; bf16/fp16: A and B are the inputs cast to that type and the
    scales are empty).
    """
    g = torch.Generator().manual_seed(w.seed)
    a32 = torch.randn(w.M, w.K, generator=g, dtype=torch.float32)
    b32 = torch.randn(w.N, w.K, generator=g, dtype=torch.float32) * w.b_std
    out = {"workload": w}
    if w.kind == "fp8":
        a, sa = quant.pertoken_quant(a32, quant_dtype=quant.FP8)
        b, sb = quant.pertoken_quant(b32, quant_dtype=quant.FP8)
    elif w.kind == "int8":
        a, sa = quant.pertoken_quant(a32, quant_dtype=torch.int8)
        b, sb = quant.pertoken_quant(b32, quant_dtype=torch.int8)
    elif w.kind == "int4":
        a, sa = quant.pertoken_quant(a32, quant_dtype=torch.int8)
        b, sb = quant.pertoken_quant(b32, quant_dtype=torch.int8, dtypeMax=7)
    elif w.kind == "fp8_block":
        a, sa = quant.blockscale_quant(a32, 1, 128)
        pad = (-w.N) % 128
        b32p = torch.cat([b32, torch.zeros(pad, w.K)]) if pad else b32
        b, sb = quant.blockscale_quant(b32p, 128, 128)
        b = b[: w.N].contiguous()
        out["sa_t"] = sa.t().contiguous()
    elif w.kind == "mxfp4":
        # as the reference harness prepares them (test_preshuffle_gemm.py:304-336): A quantized
        # on rows padded to a multiple of 32, both scale arrays shuffled for the MFMA lanes
        m32 = (w.M + 31) // 32 * 32
        a_pad = torch.zeros(m32, w.K)
        a_pad[: w.M] = a32
        a_q, sa_raw, _ = fp4.per_1x32_f4_quant(a_pad)
        b_q, sb_raw, _ = fp4.per_1x32_f4_quant(b32)
        del a32, b32, a_pad
        out.update(a=a_q[: w.M].contiguous(), b=b_q, b_dev=fp4.shuffle_weight_w4(b_q),
                   sa=fp4.shuffle_scale_w4(sa_raw), sb=fp4.shuffle_scale_w4(sb_raw), sa_raw=sa_raw, sb_raw=sb_raw)
        return out
    elif w.kind in ("bf16", "fp16"):
        dt = torch.bfloat16 if w.kind == "bf16" else torch.float16
        a, b = a32.to(dt), b32.to(dt)
        sa = sb = torch.empty(0, dtype=torch.float32)
    else:
        raise ValueError(f"unknown kind {w.kind!r}")
    del a32, b32
    b_shuf = quant.shuffle_weight(b)
    out["b_dev"] = quant.pack_int4(b_shuf) if w.kind == "int4" else b_shuf
    out.update(a=a.contiguous(), b=b.contiguous(), sa=sa.contiguous(), sb=sb.contiguous())
    return out


# ---- MoE 2-stage ------------------------------------------------------------------------
@dataclass(frozen=True)
class MoeWorkload:
    """One MoE layer: ``tokens`` routed to ``topk`` of ``experts`` experts, each expert a gate/up
    projection [2*inter_dim, model_dim] (stage 1) and a down projection [model_dim, inter_dim]
    (stage 2).  Shapes follow the reference's tests (``tests/kernels/test_moe_gemm.py:1173-1182,
    1477-1489``)."""
    name: str
    tokens: int
    model_dim: int
    inter_dim: int
    experts: int
    topk: int
    tile_m: int
    tile_n1: int
    tile_n2: int
    kind: str = "fp8"     # "fp8" | "int8" | "int8smooth" | "int4" | "int4_bf16" | "bf16" | "fp16" | "fp8_block"
    seed: int = 0
    note: str = ""

    @property
    def routes(self) -> int:
        return self.tokens * self.topk

    @property
    def flops1(self) -> int:
        return 2 * self.routes * 2 * self.inter_dim * self.model_dim

    @property
    def flops2(self) -> int:
        return 2 * self.routes * self.model_dim * self.inter_dim


MOE_WORKLOADS = {
    "MS": MoeWorkload("MS", 64, 256, 128, 4, 2, 16, 64, 64, note="reference test shape S"),
    "MM": MoeWorkload("MM", 129, 1024, 256, 8, 2, 32, 128, 128, note="reference test shape M"),
    "ML": MoeWorkload("ML", 333, 4096, 2048, 17, 9, 64, 128, 256, note="reference test shape L"),
    "DSP": MoeWorkload("DSP", 8192, 7168, 256, 128, 8, 64, 256, 256, seed=1, note="DS-TP8-prefill-S"),
    "DSD": MoeWorkload("DSD", 8, 7168, 256, 256, 8, 32, 256, 256, seed=2, note="DS-TP8-decode-bs8"),
    "DSB": MoeWorkload("DSB", 128, 7168, 256, 256, 8, 16, 256, 256, "fp8_block", seed=3,
                       note="DS-V3-M128 blockscale (test_moe_blockscale.py:201)"),
    # the reference's MoE benchmark list (scripts/run_benchmark.sh:100-104): tokens, model_dim,
    # inter_dim, experts, topk, tile_m, tile_n, tile_n2
    "RBL": MoeWorkload("RBL", 32768, 8192, 8192, 16, 4, 64, 128, 256, seed=4, note="reference MoE benchmark, large"),
    "RBS": MoeWorkload("RBS", 64, 6144, 1024, 128, 8, 16, 64, 64, seed=5, note="reference MoE benchmark, small"),
}


def moe_custom(tokens, model_dim, inter_dim, experts, topk, tile_m, tile_n1, tile_n2, kind="fp8", seed=0):
    return MoeWorkload("custom", tokens, model_dim, inter_dim, experts, topk, tile_m, tile_n1, tile_n2, kind, seed)


_MOE_T16 = {"bf16": torch.bfloat16, "fp16": torch.float16}


def _moe_quant(x: torch.Tensor, kind: str, weight: bool = False):
    """-> (q, scale) : per-row fp32 scales [rows] (fp8 / int8), None (16-bit), or for "fp8_block"
    block scales [rows/128, K/128] (weights) or [rows, K/128] (activations)."""
    if kind in _MOE_T16:
        return x.to(_MOE_T16[kind]), None
    if kind == "fp8_block":
        return quant.blockscale_quant(x, 128 if weight else 1, 128)
    q, s = quant.pertoken_quant(x.reshape(-1, x.shape[-1]), quant_dtype=quant.FP8 if kind == "fp8" else torch.int8)
    return q.reshape(x.shape), s.reshape(-1)


def moe_problem(w: MoeWorkload, device, with_stage2_input: bool = True, group_size: int = -1) -> dict:
    """Synthetic operands drawn as the reference's 2-stage test draws them
    (``test_moe_gemm.py:1236-1262``: x ~ 0.2 N(0,1), W1 ~ 0.2 N(0,1), W2 ~ 0.2/sqrt(I) N(0,1),
    routing = softmax over the top-k of uniform scores), generated on ``device`` from
    ``torch.Generator(device).manual_seed(seed)``, quantized per row and preshuffled; routing
    metadata from ``flydsl_amd.moe.moe_sorting`` with ``block_size = tile_m``.

    The stage-2 input ``a2`` [tokens*topk, inter_dim] is drawn directly (0.2 N(0,1), quantized
    per row) so stage 2 can be measured and tested on its own.

    Kinds beyond fp8/int8/bf16/fp16/fp8_block follow the reference harness's preparation
    (``test_moe_gemm.py:414-450,471-491``): ``int8smooth`` -- a per-expert smoothing factor
    0.75 + 0.5 U(0,1) per column, x expanded per route and quantized per route, passed
    slot-major (``x`` [topk*tokens, D], ``sx`` [topk*tokens]; ``x_route`` / ``sx_route`` keep
    [tokens, topk, ...]); ``int4`` -- int8 x, weights quantized per row to [-7, 7] and packed two
    per byte after the shuffle; ``int4_bf16`` -- bf16 x and the same int4 weights, with
    ``group_size = 32`` group scales 0.005 + 0.05 U(0,1) of shape [E, K/32, rows] (``w1_groups``,
    ``w2_groups``; ``sw1`` / ``sw2`` then hold them flat) in place of the per-row scales."""
    from .moe import moe_sorting

    g = torch.Generator(device=device).manual_seed(w.seed)
    T, D, I, E, k, s = w.tokens, w.model_dim, w.inter_dim, w.experts, w.topk, 0.2
    x = torch.randn(T, D, generator=g, device=device) * s
    w1 = torch.randn(E * 2 * I, D, generator=g, device=device) * s
    w2 = torch.randn(E * D, I, generator=g, device=device) * (s / I ** 0.5)
    score = torch.rand(T, E, generator=g, device=device)
    vals, topk_ids = torch.topk(score, k=k, dim=1)
    topk_w = torch.softmax(vals, dim=1).float()
    kind = w.kind
    extra = {}
    if kind in ("int4", "int4_bf16"):
        xq, sx = _moe_quant(x, "int8" if kind == "int4" else "bf16")
        w1q, sw1 = quant.pertoken_quant(w1, quant_dtype=torch.int8, dtypeMax=7)
        w2q, sw2 = quant.pertoken_quant(w2, quant_dtype=torch.int8, dtypeMax=7)
        sw1, sw2 = sw1.reshape(-1), sw2.reshape(-1)
        if kind == "int4_bf16" and group_size > 0:
            w1g = torch.rand(E, D // group_size, 2 * I, generator=g, device=device) * 0.05 + 0.005
            w2g = torch.rand(E, I // group_size, D, generator=g, device=device) * 0.05 + 0.005
            extra.update(w1_groups=w1g, w2_groups=w2g)
            sw1, sw2 = w1g.contiguous().view(-1), w2g.contiguous().view(-1)
        w1_dev = quant.pack_int4(quant.shuffle_weight(w1q))
        w2_dev = quant.pack_int4(quant.shuffle_weight(w2q))
    else:
        if kind == "int8smooth":
            smooth = 0.75 + 0.5 * torch.rand(E, D, generator=g, device=device)
            x_route = x[:, None, :] * smooth[topk_ids.long()]               # [T, k, D]
            q, sr = quant.pertoken_quant(x_route.reshape(T * k, D), quant_dtype=torch.int8)
            q, sr = q.view(T, k, D), sr.view(T, k)
            extra.update(x_route=q, sx_route=sr, smooth=smooth)
            xq = q.permute(1, 0, 2).contiguous().view(k * T, D)          # slot-major rows s*T + t
            sx = sr.t().contiguous().view(-1)
            wk = "int8"
        else:
            xq, sx = _moe_quant(x, kind)
            wk = kind
        w1q, sw1 = _moe_quant(w1, wk, weight=True)
        w2q, sw2 = _moe_quant(w2, wk, weight=True)
        w1_dev, w2_dev = quant.shuffle_weight(w1q), quant.shuffle_weight(w2q)
    del w1, w2
    sid, sw, eid, post = moe_sorting(topk_ids.to(torch.int32), topk_w, E, w.tile_m)
    out = dict(workload=w, x=xq, sx=sx, w1=w1q, sw1=sw1, w1_shuf=w1_dev, w2=w2q, sw2=sw2,
               w2_shuf=w2_dev, topk_ids=topk_ids.to(torch.int32), topk_weights=topk_w,
               sorted_ids=sid, sorted_weights=sw, sorted_expert_ids=eid, num_valid_ids=post[:1].contiguous(),
               blocks=int(eid.numel()), group_size=group_size, **extra)
    if with_stage2_input:
        a2 = torch.randn(T * k, I, generator=g, device=device) * s
        a2_kind = {"int8smooth": "int8", "int4": "int8", "int4_bf16": "bf16"}.get(kind, kind)
        out["a2"], out["sa2"] = _moe_quant(a2, a2_kind)
    if kind == "fp8_block":
        # the kernels take activation block scales K-block major ([K/128, rows], the reference's
        # transpose_scale layout) and weight block scales flat; *_blocks keep [rows, K/128]
        out["sx_blocks"], out["sx"] = sx, sx.t().contiguous().view(-1)
        out["sw1"], out["sw2"] = sw1.contiguous().view(-1), sw2.contiguous().view(-1)
        out["sw1_blocks"], out["sw2_blocks"] = sw1, sw2
        if with_stage2_input:
            out["sa2_blocks"], out["sa2"] = out["sa2"], out["sa2"].t().contiguous().view(-1)
    return out


def moe_bytes(w: MoeWorkload, stage: int, active_experts: int, group_size: int = -1) -> float:
    """Algorithmic HBM bytes of one stage: each active expert's weights and every activation,
    scale and output element once (index/weight metadata included).  Packed int4 weights count
    half a byte; ``int8smooth`` reads stage-1 activations per route; group scales (int4_bf16,
    ``group_size`` > 0) are one float per weight row and K group."""
    eb = 2 if w.kind in _MOE_T16 or w.kind == "int4_bf16" else 1     # activation bytes
    wb = 0.5 if w.kind in ("int4", "int4_bf16") else eb               # weight bytes
    T, D, I, k = w.tokens, w.model_dim, w.inter_dim, w.topk
    meta = 4 * (T * k + w.experts * w.tile_m) * 2
    bs = w.kind == "fp8_block"   # block scales: per (row, 128 K) for activations, 128 x 128 for weights
    a_scaled = w.kind != "int4_bf16" and w.kind not in _MOE_T16
    if stage == 1:
        x_rows = T * k if w.kind == "int8smooth" else T
        if bs:
            sc = T * (D // 128) + active_experts * (2 * I // 128) * (D // 128)
        else:
            wsc = active_experts * 2 * I * (D // group_size if group_size > 0 else 1)
            sc = (x_rows if a_scaled else 0) + wsc
        return active_experts * 2 * I * D * wb + x_rows * D * eb + T * k * I * 2 + sc * 4 + meta
    if bs:
        sc = T * k * (I // 128) + active_experts * (D // 128) * (I // 128)
    else:
        sc = (T * k if a_scaled else 0) + active_experts * D * (I // group_size if group_size > 0 else 1)
    return active_experts * D * I * wb + T * k * I * eb + T * D * 2 + sc * 4 + meta
