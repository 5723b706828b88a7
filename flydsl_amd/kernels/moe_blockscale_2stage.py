"""MI355X blockscale MoE 2-stage GEMM: the drop-in for the reference's
``kernels/moe_blockscale_2stage.py`` (fp8 only; ScaleBlockM = 1, ScaleBlockN = ScaleBlockK = 128).

``compile_moe_blockscale_gemm1`` / ``compile_moe_blockscale_gemm2`` keep the reference's names,
keyword arguments, checks and launcher signatures (``:75-1217``, ``:1220-2445``; harness
``tests/kernels/test_moe_blockscale.py:204-400``)::

    s1 = compile_moe_blockscale_gemm1(model_dim=D, inter_dim=I, experts=E, topk=k, tile_m=16,
                                      tile_n=256, tile_k=128, doweight_stage1=False)
    s1(out1, x_q, w1_shuffled, x_scale_t, w1_scale, sorted_token_ids, sorted_expert_ids,
       sorted_weights, num_valid_ids, tokens, I, D, blocks, stream)

``x_scale_t`` fp32 ``[D/128, tokens]`` (K-block major, as the reference's quant kernel writes
it with ``transpose_scale=True``), ``w1_scale`` fp32 ``[E, (2I/128)*(D/128)]`` flat (one per
128x128 block of each expert's ``[2I, D]`` weight); stage 2 takes ``a2_scale_t``
``[I/128, tokens*topk]`` and ``w2_scale`` ``[E, (D/128)*(I/128)]``.  Each 128-deep K block's
partial product is scaled by both block scales before it is accumulated.  Behind the
launchers: ``flygemm_moe_blockscale_gemm1/2`` of ``include/flygemm.h``.
"""
from __future__ import annotations

from .moe_gemm_2stage import (_OUT_ALIAS, MoeGemm2Mode, _MoeGemm2ReduceWrapper, _MoeStage, _check_common,
                              compile_moe_reduction)


def _check_bs(scale_block_k, tile_m, tile_n, tile_k):
    if int(scale_block_k) != 128:
        raise ValueError(f"scale_block_k={scale_block_k}: only 128 is supported")
    return _check_common("fp8", -1, tile_m, tile_n, tile_k)


def compile_moe_blockscale_gemm1(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int,
                                 tile_n: int, tile_k: int, doweight_stage1: bool, scale_block_k: int = 128,
                                 out_dtype: str = "f16", use_cshuffle_epilog=None, waves_per_eu=None):
    """Stage 1 (validates like reference ``moe_blockscale_2stage.py:108-140``)."""
    if out_dtype not in ("f16", "bf16"):
        raise ValueError(f"out_dtype must be 'f16' or 'bf16', got {out_dtype!r}")
    elem = _check_bs(scale_block_k, tile_m, tile_n, tile_k)
    if int(model_dim) % int(scale_block_k):
        raise ValueError(f"model_dim ({model_dim}) must be divisible by scale_block_k ({scale_block_k})")
    if (2 * int(inter_dim)) % 128:
        raise ValueError(f"2*inter_dim ({2 * int(inter_dim)}) must be divisible by 128 (ScaleBlockN)")
    if int(inter_dim) % int(tile_n):
        raise ValueError(f"inter_dim={inter_dim} must be divisible by tile_n={tile_n}")
    return _MoeStage(1, model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m,
                     tile_n=tile_n, tile_k=tile_k, doweight=doweight_stage1, in_dtype="fp8", out_dtype=out_dtype,
                     elem=elem, blockscale=True)


def compile_moe_blockscale_gemm2(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int,
                                 tile_n: int, tile_k: int, doweight_stage2: bool, scale_block_k: int = 128,
                                 out_dtype: str = "f16", use_cshuffle_epilog=None, accumulate: bool = True,
                                 waves_per_eu=None):
    """Stage 2 (validates like reference ``moe_blockscale_2stage.py:1262-1330``); ``accumulate=False``
    writes per-route rows for ``compile_moe_reduction``."""
    out_dtype = _OUT_ALIAS.get(str(out_dtype).strip().lower(), out_dtype)
    if out_dtype not in ("f16", "bf16", "f32"):
        raise ValueError(f"out_dtype must be 'f16', 'bf16', or 'f32', got {out_dtype!r}")
    if not accumulate and out_dtype == "f32":
        raise ValueError("compile_moe_blockscale_gemm2(accumulate=False) only supports out_dtype in {'f16','bf16'}")
    elem = _check_bs(scale_block_k, tile_m, tile_n, tile_k)
    if int(inter_dim) % int(scale_block_k):
        raise ValueError(f"inter_dim ({inter_dim}) must be divisible by scale_block_k ({scale_block_k})")
    if int(model_dim) % 128:
        raise ValueError(f"model_dim ({model_dim}) must be divisible by 128 (ScaleBlockN)")
    if int(model_dim) % int(tile_n):
        raise ValueError(f"model_dim={model_dim} must be divisible by tile_n={tile_n}")
    return _MoeStage(2, model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m,
                     tile_n=tile_n, tile_k=tile_k, doweight=doweight_stage2, in_dtype="fp8", out_dtype=out_dtype,
                     elem=elem, accumulate=accumulate, blockscale=True)


def compile_moe_blockscale_gemm2_ex(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int,
                                    tile_n: int, tile_k: int, doweight_stage2: bool, in_dtype: str = "fp8",
                                    out_dtype: str = "f16", use_cshuffle_epilog=None,
                                    mode: str = MoeGemm2Mode.ATOMIC, valid_mask=None):
    """Stage 2 with the execution mode chosen explicitly (reference ``moe_blockscale_2stage.py:2740-2820``)."""
    if in_dtype != "fp8":
        raise ValueError(f"blockscale MoE is fp8 only, got in_dtype={in_dtype!r}")
    kw = dict(model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m, tile_n=tile_n,
              tile_k=tile_k, doweight_stage2=doweight_stage2, out_dtype=out_dtype,
              use_cshuffle_epilog=use_cshuffle_epilog)
    if mode != MoeGemm2Mode.REDUCE:
        return compile_moe_blockscale_gemm2(**kw, accumulate=True)
    gemm2 = compile_moe_blockscale_gemm2(**kw, accumulate=False)
    use_mask = valid_mask is not None
    return _MoeGemm2ReduceWrapper(gemm2, compile_moe_reduction(topk=topk, model_dim=model_dim,
                                                               dtype_str=gemm2.out_dtype, use_mask=use_mask),
                                  topk, model_dim, gemm2.out_dtype, use_mask)
