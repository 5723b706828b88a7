"""MI355X MoE 2-stage GEMM: the drop-in for the reference's ``kernels/moe_gemm_2stage.py``.

``compile_moe_gemm1`` / ``compile_moe_gemm2`` keep the reference's names, keyword arguments,
argument checks and launcher signatures (reference ``kernels/moe_gemm_2stage.py:93-1264`` and
``:1267-2481``; harness ``tests/kernels/test_moe_gemm.py:299-1170``)::

    s1 = compile_moe_gemm1(model_dim=D, inter_dim=I, experts=E, topk=k, tile_m=32, tile_n=128,
                           tile_k=128, doweight_stage1=False, in_dtype="fp8", out_dtype="f16")
    s1(out1, x, w1, scale_x, scale_w1, sorted_token_ids, sorted_expert_ids, sorted_weights,
       num_valid_ids, tokens, I, D, blocks, stream)
    s2 = compile_moe_gemm2(..., doweight_stage2=True, out_dtype="f16")
    s2(out2, a2, w2, scale_a2, scale_w2, sorted_token_ids, sorted_expert_ids, sorted_weights,
       num_valid_ids, tokens, D, I, blocks, stream)

Stage 1 writes ``out1[t, s, :] = silu(gate) * up`` for every route (token t, slot s) of the
sorted metadata; stage 2 adds ``a2[t, s] @ W2[e]^T`` (scaled, optionally weighted) into
``out2[t]`` with device atomics, so ``out2`` must be zeroed first, as in the reference harness.
The metadata is what ``flydsl_amd.moe.moe_sorting`` (or the reference's ``moe_sorting``)
produces with ``block_size == tile_m``.

Behind the launchers: ``flygemm_moe_gemm1`` / ``flygemm_moe_gemm2`` of ``include/flygemm.h``,
hand-written gfx950 kernels; no JIT and no host fallback.

Built: every ``in_dtype`` of the reference -- fp8, int8 (per-token x scale, per-row weight scale),
fp16, bf16 (unscaled), ``int8smooth`` (stage-1 x given per route, slot-major rows
``s*tokens + t`` with their own scales; stage 2 as int8), ``int4`` (W4A8: int8 x, packed int4
weights), ``int4_bf16`` (W4A16: bf16 x, packed int4 weights with per-row scales, or with
``group_size=32`` group scales ``[E, K/32, rows]``, reference ``tests/utils.py:99-120``);
``tile_m`` 16/32/64; ``tile_n`` 64/128/256.  ``group_size > 0`` with another in_dtype raises
``ValueError`` (the reference accepts and ignores it; its harness skips those cases,
``tests/kernels/test_moe_gemm.py:1230-1231``).  Stage 2 also has the
reference's reduce mode (``accumulate=False`` + ``compile_moe_reduction``, or
``compile_moe_gemm2_ex(mode=MoeGemm2Mode.REDUCE)``): per-route rows with plain stores, then a
reduction over the top-k slots -- about three times faster than atomics on MI355X, whose atomic
units take ~1.3 TB/s of fp16 payload against ~7 TB/s for plain stores.  ``tile_k`` is validated as the
reference validates it and otherwise a hint (the kernels' K tile is 128 bytes).
"""
from __future__ import annotations

import torch

from .. import _lib
from ._launch import device_ptr, stream_handle

_ALL_IN = ("fp8", "fp16", "bf16", "int8", "int8smooth", "int4", "int4_bf16")
_T16 = {"bf16": torch.bfloat16, "fp16": torch.float16, "int4_bf16": torch.bfloat16}   # 2-byte activations
_W4 = ("int4", "int4_bf16")   # packed int4 weights
_OUT = {"f16": ("fp16", torch.float16), "bf16": ("bf16", torch.bfloat16), "f32": ("fp32", torch.float32)}
# stage 2 spellings the reference accepts (moe_gemm_2stage.py:1315-1316)
_OUT_ALIAS = {"fp16": "f16", "half": "f16", "bfloat16": "bf16", "fp32": "f32", "float": "f32"}


def _check_common(in_dtype, group_size, tile_m, tile_n, tile_k):
    if in_dtype not in _ALL_IN:
        raise ValueError(f"in_dtype must be one of {_ALL_IN}, got {in_dtype!r}")
    elem = 2 if in_dtype in ("fp16", "bf16", "int4_bf16") else 1
    if (int(tile_k) * elem) % 64:
        raise ValueError(f"tile_k_bytes must be divisible by 64, got tile_k={tile_k} (elem_bytes={elem})")
    if (int(tile_m) * int(tile_k) * elem) % 256:
        raise ValueError(f"tile_m*tile_k*elem_bytes must be divisible by 256: tile_m={tile_m}, tile_k={tile_k}")
    if int(group_size) > 0 and (in_dtype != "int4_bf16" or int(group_size) != 32):
        raise ValueError(f"group_size={group_size}: group-wise weight scales are built for in_dtype='int4_bf16' "
                         f"with group_size=32")
    if int(tile_m) not in (16, 32, 64):
        raise ValueError(f"tile_m={tile_m}: the MI355X kernels take routing blocks of 16, 32 or 64 rows")
    if int(tile_n) not in (64, 128, 256):
        raise ValueError(f"tile_n={tile_n} must be 64, 128 or 256")
    return elem


class _MoeStage:
    def __init__(self, stage, *, model_dim, inter_dim, experts, topk, tile_m, tile_n, tile_k, doweight, in_dtype,
                 out_dtype, elem, accumulate=True, blockscale=False, group_size=-1):
        self.stage = stage
        self.model_dim, self.inter_dim = int(model_dim), int(inter_dim)
        self.experts, self.topk = int(experts), int(topk)
        self.tile_m, self.tile_n, self.tile_k = int(tile_m), int(tile_n), int(tile_k)
        self.doweight = bool(doweight)
        self.in_dtype, self.out_dtype = in_dtype, out_dtype
        self.elem = elem
        self.accumulate = bool(accumulate)
        self.blockscale = bool(blockscale)   # fp8 with 1x128 / 128x128 block scales
        self.group_size = int(group_size) if int(group_size) > 0 else -1

    def __call__(self, arg_out, arg_x, arg_w, arg_scale_x, arg_scale_w, arg_sorted_token_ids, arg_expert_ids,
                 arg_sorted_weights, arg_num_valid_ids, tokens, n_in, k_in, size_expert_ids, stream=None):
        tokens, N, K, blocks = int(tokens), int(n_in), int(k_in), int(size_expert_ids)
        h_stream = stream_handle(stream)
        if tokens < 0 or blocks < 0:
            raise ValueError(f"invalid tokens={tokens} / size_expert_ids={blocks}")
        want_n, want_k = (self.inter_dim, self.model_dim) if self.stage == 1 else (self.model_dim, self.inter_dim)
        if N != want_n or K != want_k:
            raise ValueError(f"stage {self.stage} was compiled for N={want_n}, K={want_k}; got N={N}, K={K}")
        if N % self.tile_n:
            raise ValueError(f"N={N} must be divisible by tile_n={self.tile_n}")
        if K % self.tile_k:
            raise ValueError(f"K={K} must be divisible by tile_k={self.tile_k}")
        E, topk = self.experts, self.topk
        # int8smooth stage 1 takes x per route (slot-major rows s*tokens + t)
        per_route = self.stage == 2 or self.in_dtype == "int8smooth"
        a_rows = tokens * topk if per_route else tokens
        w_rows = E * 2 * N if self.stage == 1 else E * N
        w_bytes = w_rows * K // 2 if self.in_dtype in _W4 else w_rows * K
        out_name, out_t = _OUT[self.out_dtype]
        out_elems = tokens * topk * N if (self.stage == 1 or not self.accumulate) else tokens * N
        o = device_ptr(arg_out, "arg_out", out_elems, dtypes=(out_t,))
        if self.in_dtype in _T16:
            x = device_ptr(arg_x, "arg_x", a_rows * K, dtypes=(_T16[self.in_dtype],))
            sx = 0  # unscaled activations; the reference passes empty tensors
            if self.in_dtype == "int4_bf16":
                w = device_ptr(arg_w, "arg_w", w_bytes, elem_bytes=1)
                nsw = w_rows * (K // self.group_size) if self.group_size > 0 else w_rows
                sw = device_ptr(arg_scale_w, "arg_scale_w", nsw, dtypes=(torch.float32,))
            else:
                w = device_ptr(arg_w, "arg_w", w_rows * K, dtypes=(_T16[self.in_dtype],))
                sw = 0
        else:
            x = device_ptr(arg_x, "arg_x", a_rows * K, elem_bytes=1)
            w = device_ptr(arg_w, "arg_w", w_bytes, elem_bytes=1)
            nsx, nsw = (a_rows * (K // 128), w_rows // 128 * (K // 128)) if self.blockscale else (a_rows, w_rows)
            sx = device_ptr(arg_scale_x, "arg_scale_x", nsx, dtypes=(torch.float32,))
            sw = device_ptr(arg_scale_w, "arg_scale_w", nsw, dtypes=(torch.float32,))
        # moe_sorting allocates tokens*topk + E*tile_m - topk entries, which need not fill the
        # last block; the kernels read entries only below num_valid_ids[0]
        n_sorted = min(blocks * self.tile_m, max(tokens * topk + E * self.tile_m - topk, 0))
        ids = device_ptr(arg_sorted_token_ids, "arg_sorted_token_ids", n_sorted, dtypes=(torch.int32,))
        eids = device_ptr(arg_expert_ids, "arg_expert_ids", blocks, dtypes=(torch.int32,))
        sws = (device_ptr(arg_sorted_weights, "arg_sorted_weights", n_sorted, dtypes=(torch.float32,))
               if self.doweight else 0)
        nv = device_ptr(arg_num_valid_ids, "arg_num_valid_ids", 1, dtypes=(torch.int32,))
        lib = _lib.load()
        dt = 128 if self.blockscale else _lib.FLYGEMM_IN[self.in_dtype]   # scale_block_k / in_dtype
        args = (o, x, w, sx, sw, ids, eids, sws, nv, tokens, N, K, blocks, E, topk, self.tile_m, self.tile_n, dt,
                _lib.FLYGEMM_OUT[out_name], int(self.doweight))
        name = f"flygemm_moe_{'blockscale_' if self.blockscale else ''}gemm{self.stage}"
        fn = getattr(lib, name)
        tail = () if self.blockscale else (self.group_size,)
        if self.stage == 1:
            rc = fn(*args, *tail, h_stream)
        else:
            rc = fn(*args, int(self.accumulate), *tail, h_stream)
        _lib.check(rc, name)


def compile_moe_gemm1(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int, tile_n: int,
                      tile_k: int, doweight_stage1: bool, in_dtype: str = "fp8", group_size: int = -1,
                      out_dtype: str = "f16", use_cshuffle_epilog=None):
    """Stage 1 (gate/up GEMM + silu(gate) * up); validates like reference ``moe_gemm_2stage.py:126-200``."""
    elem = _check_common(in_dtype, group_size, tile_m, tile_n, tile_k)
    if out_dtype not in ("f16", "bf16"):
        raise ValueError(f"out_dtype must be 'f16' or 'bf16', got {out_dtype!r}")
    if int(inter_dim) % int(tile_n) or int(model_dim) % int(tile_k):
        raise ValueError(f"inter_dim={inter_dim} % tile_n={tile_n} and model_dim={model_dim} % tile_k={tile_k} must be 0")
    return _MoeStage(1, model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m,
                     tile_n=tile_n, tile_k=tile_k, doweight=doweight_stage1, in_dtype=in_dtype, out_dtype=out_dtype,
                     elem=elem, group_size=group_size)


def compile_moe_gemm2(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int, tile_n: int,
                      tile_k: int, doweight_stage2: bool, in_dtype: str = "fp8", group_size: int = -1,
                      out_dtype: str = "f16", use_cshuffle_epilog=None, accumulate: bool = True):
    """Stage 2 (down GEMM accumulated over the top-k slots); validates like reference
    ``moe_gemm_2stage.py:1300-1430``.  ``accumulate=False`` writes per-route rows (reduce mode)."""
    elem = _check_common(in_dtype, group_size, tile_m, tile_n, tile_k)
    out_dtype = _OUT_ALIAS.get(str(out_dtype).strip().lower(), out_dtype)
    if out_dtype not in ("f16", "bf16", "f32"):
        raise ValueError(f"out_dtype must be 'f16', 'bf16', or 'f32', got {out_dtype!r}")
    if not accumulate and out_dtype == "f32":
        raise ValueError("compile_moe_gemm2(accumulate=False) only supports out_dtype in {'f16','bf16'}")
    if int(model_dim) % int(tile_n) or int(inter_dim) % int(tile_k):
        raise ValueError(f"model_dim={model_dim} % tile_n={tile_n} and inter_dim={inter_dim} % tile_k={tile_k} must be 0")
    return _MoeStage(2, model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m,
                     tile_n=tile_n, tile_k=tile_k, doweight=doweight_stage2, in_dtype=in_dtype, out_dtype=out_dtype,
                     elem=elem, accumulate=accumulate, group_size=group_size)


_RED_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
_RED_CODE = {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}


def compile_moe_reduction(*, topk: int, model_dim: int, dtype_str: str = "f16", use_mask: bool = False):
    """Reduce mode, second step (reference ``moe_gemm_2stage.py:2484-2604``): returns
    ``launch(X, Y, valid_mask, m_tokens, stream=None)`` computing ``Y[t, d] = sum_k X[t, k, d]``
    over ``k < topk`` (slots with ``valid_mask[t, k] == 0`` skipped when ``use_mask``)."""
    if dtype_str not in _RED_DT:
        raise ValueError(f"Unsupported dtype: {dtype_str}")
    topk, model_dim = int(topk), int(model_dim)
    ve = 4 if dtype_str == "f32" else 8
    if model_dim % ve:
        raise ValueError(f"model_dim={model_dim} must be a multiple of {ve}")
    dt = _RED_DT[dtype_str]

    def launch_moe_reduction(X, Y, valid_mask, i32_m_tokens, stream=None):
        m = int(i32_m_tokens)
        if m < 0:
            raise ValueError(f"invalid m_tokens={m}")
        h = stream_handle(stream)
        x = device_ptr(X, "X", m * topk * model_dim, dtypes=(dt,))
        y = device_ptr(Y, "Y", m * model_dim, dtypes=(dt,))
        mk = device_ptr(valid_mask, "valid_mask", m * topk, elem_bytes=1) if use_mask else 0
        rc = _lib.load().flygemm_moe_reduce(y, x, mk, m, topk, model_dim, _lib.FLYGEMM_OUT[_RED_CODE[dtype_str]], h)
        _lib.check(rc, "flygemm_moe_reduce")

    return launch_moe_reduction


class MoeGemm2Mode:
    """Execution mode of MoE stage 2 (reference ``moe_gemm_2stage.py:2682-2686``)."""
    ATOMIC = "atomic"       # atomic accumulation into [tokens, model_dim]
    REDUCE = "reduce"       # per-route rows [tokens*topk, model_dim], then a reduction over topk


class _MoeGemm2ReduceWrapper:
    """Stage 2 in reduce mode (reference ``moe_gemm_2stage.py:2689-2774``): the GEMM writes
    every route's row of an intermediate [tokens*topk, model_dim] with plain stores, then the
    reduction sums the top-k rows of each token into ``arg_out``.  The intermediate comes from
    torch's caching allocator (zeroed unless a valid mask says which rows to read, or
    ``zero_intermediate=False`` promises every route is written)."""

    def __init__(self, gemm2_exe, reduce_exe, topk, model_dim, out_dtype_str="f16", use_mask=False,
                 zero_intermediate=True):
        self._gemm2_exe, self._reduce_exe = gemm2_exe, reduce_exe
        self._topk, self._model_dim = int(topk), int(model_dim)
        self._out_dtype_str = out_dtype_str
        self._use_mask = bool(use_mask)
        self._zero_intermediate = bool(zero_intermediate)

    def __call__(self, arg_out, arg_x, arg_w, arg_scale_x, arg_scale_w, arg_sorted_token_ids, arg_expert_ids,
                 arg_sorted_weights, arg_num_valid_ids, tokens_in, n_in, k_in, size_expert_ids_in, valid_mask=None,
                 stream=None):
        tokens = int(tokens_in)
        if stream is None:
            stream = torch.cuda.current_stream()
        inter = torch.empty(tokens * self._topk, self._model_dim, device=arg_out.device,
                            dtype=_RED_DT[self._out_dtype_str])
        if self._zero_intermediate and not self._use_mask:
            inter.zero_()
        self._gemm2_exe(inter.view(-1), arg_x, arg_w, arg_scale_x, arg_scale_w, arg_sorted_token_ids, arg_expert_ids,
                        arg_sorted_weights, arg_num_valid_ids, tokens, n_in, k_in, size_expert_ids_in, stream)
        if self._use_mask and valid_mask is None:
            raise ValueError("this reduce-mode stage 2 was compiled with a valid mask; pass valid_mask")
        mask = valid_mask.contiguous().view(-1) if self._use_mask else None
        self._reduce_exe(inter.view(-1), arg_out.view(-1), mask, tokens, stream)

    @property
    def mode(self) -> str:
        return MoeGemm2Mode.REDUCE


def compile_moe_gemm2_ex(*, model_dim: int, inter_dim: int, experts: int, topk: int, tile_m: int, tile_n: int,
                         tile_k: int, doweight_stage2: bool, in_dtype: str = "fp8", group_size: int = -1,
                         out_dtype: str = "f16", use_cshuffle_epilog=None, mode: str = MoeGemm2Mode.ATOMIC,
                         valid_mask=None, zero_intermediate: bool = True):
    """Stage 2 with the execution mode chosen explicitly (reference ``moe_gemm_2stage.py:2777-2877``)."""
    kw = dict(model_dim=model_dim, inter_dim=inter_dim, experts=experts, topk=topk, tile_m=tile_m, tile_n=tile_n,
              tile_k=tile_k, doweight_stage2=doweight_stage2, in_dtype=in_dtype, group_size=group_size,
              out_dtype=out_dtype, use_cshuffle_epilog=use_cshuffle_epilog)
    if mode != MoeGemm2Mode.REDUCE:
        return compile_moe_gemm2(**kw, accumulate=True)
    gemm2 = compile_moe_gemm2(**kw, accumulate=False)
    dt = gemm2.out_dtype
    use_mask = valid_mask is not None
    return _MoeGemm2ReduceWrapper(gemm2, compile_moe_reduction(topk=topk, model_dim=model_dim, dtype_str=dt,
                                                               use_mask=use_mask),
                                  topk, model_dim, dt, use_mask, zero_intermediate)
