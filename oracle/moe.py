"""MoE 2-stage oracle (test infrastructure only): routing metadata sorted by expert and the two
grouped GEMMs, restated in numpy.

* ``moe_sorting``   ``moe_sorting_torch_native`` (``tests/kernels/test_moe_gemm.py:97-160``):
                    for each expert in order, its routes (token, slot) in row-major order of
                    ``topk_ids``, written as ``(slot << 24) | token`` and padded to a multiple of
                    ``block_size`` with ``(topk << 24) | tokens``; one expert id per block (-1
                    past the last); ``num_tokens_post_pad = [padded total, tokens]``.  Buffer
                    sizes as the reference allocates them: ``tokens*topk + E*block - topk``
                    entries and ``ceil(that / block)`` blocks.  Padding weights, which the
                    reference leaves uninitialised, are 0 here.
* ``gemm1``         ``torch_moe_gemm1`` (``tests/kernels/test_ref.py:7-75``), per-row scales:
                    ``y = x[t] @ (W1[e] * sw)^T`` split into gate (first ``inter_dim``) and up,
                    ``out[t, s] = silu(gate) * up`` (times ``topk_weights[t, s]`` if doweight).
* ``gemm2``         ``torch_moe_gemm2`` (``:78-141``): ``out[t] += a2[t, s] @ (W2[e] * sw)^T``
                    (times the weight if doweight), summed over the slots.
* ``gemm1_sorted`` / ``gemm2_sorted``  the same results reached by walking the sorted metadata
                    block by block, as the kernels do; their agreement with ``gemm1`` / ``gemm2``
                    pins the metadata interpretation (slot/token packing, padding, expert per block).

Activations and weights arrive as quantized bytes (fp8 e4m3fn, int8) with fp32 per-row scales,
or as bf16/fp16 bit patterns without scales; the products are evaluated in float64.  The
reference's other input kinds map onto these: ``int4`` (W4A8) is int8 activations with int4
weight values (kind "int8", values in [-7, 7]); ``int4_bf16`` (W4A16) is bf16 activations
(``kind="bf16"``) with int4 weight values (``w_kind="int8"``), scaled per row or, with
``w_groups`` [E, K/g, rows], per (K group, row): ``w[e,n,k] * w_groups[e, k // g, n]``
(``tests/kernels/test_ref.py:44-50,117-123``); ``int8smooth`` gives stage 1 its activations
per route, ``x_q`` [tokens, topk, K] with ``sx`` [tokens, topk] (the reference oracle's 3-D
``x_fp8``, ``:26-34``).

* ``gemm1_blockscale`` / ``gemm2_blockscale``  ``torch_stage1_blockscale_ref`` /
                    ``torch_stage2_blockscale_ref`` (``tests/kernels/test_moe_blockscale.py:64-133``):
                    fp8 activations scaled per (row, 128-wide K block), weights per 128 x 128
                    block, then the route loops above.

Pins (``tests/test_oracle.py``): a hand-worked sorting example; sorting invariants on random
routings (every route exactly once, runs padded and expert-homogeneous, the padded total);
silu's closed-form values and the identity ``silu(x) - silu(-x) = x``; gate/up order through
weights that zero one half; ``gemm2`` against one dense matmul when all experts are equal and the
routing weights sum to one; sorted-walk forms against the route forms; the blockscale forms
against the dense blockscale oracle (``gemm.run_torch_blockscale``, itself pinned) with every
token routed to one expert, and against the per-row forms when every block scale of a row is
equal.
"""
from __future__ import annotations

import numpy as np

from .gemm import dequant_rows


def moe_sorting(topk_ids: np.ndarray, topk_weights: np.ndarray, num_experts: int, block_size: int,
                expert_mask: np.ndarray | None = None):
    """-> (sorted_ids int32, sorted_weights f32, sorted_expert_ids int32, num_tokens_post_pad int32[2])."""
    ids = np.asarray(topk_ids).astype(np.int64)
    w = np.asarray(topk_weights, dtype=np.float32)
    M, topk = ids.shape
    max_pad = M * topk + num_experts * block_size - topk
    max_blocks = (max_pad + block_size - 1) // block_size
    sorted_ids = np.full(max_pad, (topk << 24) | M, dtype=np.int64)
    sorted_w = np.zeros(max_pad, dtype=np.float32)
    sorted_eid = np.full(max_blocks, -1, dtype=np.int64)
    pos = blk = skipped = 0
    for e in range(num_experts):
        if expert_mask is not None and int(expert_mask[e]) == 0:
            skipped += 1
            continue
        t_idx, s_idx = np.nonzero(ids == e)            # row-major order, as torch.where
        n = len(t_idx)
        nblk = (n + block_size - 1) // block_size
        sorted_ids[pos:pos + n] = (s_idx << 24) | t_idx
        sorted_w[pos:pos + n] = w[t_idx, s_idx]
        sorted_eid[blk:blk + nblk] = e - skipped
        pos += nblk * block_size
        blk += nblk
    post = np.array([pos, M], dtype=np.int32)
    return sorted_ids.astype(np.int32), sorted_w, sorted_eid.astype(np.int32), post


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def _expert_w(wq, sw, kind, rows: int, e: int, w_groups=None, w_round=None) -> np.ndarray:
    """Dequantized float64 weight rows [e*rows, (e+1)*rows) (one expert, on demand); with
    ``w_groups`` [E, K/g, rows] each (row, K group) has its own scale instead of ``sw``;
    ``w_round="bf16_trunc"`` turns those dequantized weights into bf16 by truncation, the bf16
    matrix-instruction operand the reference's kernel forms from them
    (``kernels/mfma_preshuffle_pipeline.py:111-141``); ``w_round="bf16"`` rounds to nearest
    even instead."""
    lo, hi = e * rows, (e + 1) * rows
    if w_groups is not None:
        # the reference multiplies in float32 (an fp32 weight tensor scaled in place)
        v = np.asarray(wq)[lo:hi].view(np.int8).astype(np.float32)
        gs = np.asarray(w_groups, dtype=np.float32)[e]            # [K/g, rows]
        g = v.shape[1] // gs.shape[0]
        wd = (v * np.repeat(gs.T, g, axis=1)).astype(np.float32)
        if w_round in ("bf16", "bf16_trunc"):
            from .numerics import bf16_rne, bf16_to_f32, bf16_trunc
            wd = bf16_to_f32(bf16_rne(wd) if w_round == "bf16" else bf16_trunc(wd))
        return wd.astype(np.float64)
    return dequant_rows(np.asarray(wq)[lo:hi], None if sw is None else np.asarray(sw).reshape(-1)[lo:hi], kind,
                        np.float64)


def _selected(T, tokens_subset):
    sel = np.zeros(T, bool)
    sel[np.arange(T) if tokens_subset is None else np.asarray(tokens_subset)] = True
    return sel


def _act(x_q, sx, kind):
    """Dequantized float64 activations: [tokens, K], or [tokens, topk, K] given per route."""
    q = np.asarray(x_q)
    flat = q.reshape(-1, q.shape[-1])
    x = dequant_rows(flat, None if sx is None else np.asarray(sx).reshape(-1), kind, np.float64)
    return x.reshape(q.shape)


def gemm1(x_q, w1_q, sx, sw1, topk_ids, topk_weights, inter_dim: int, doweight: bool, kind: str,
          tokens_subset=None, w_kind=None, w_groups=None, w_round=None) -> np.ndarray:
    """[tokens, topk, inter_dim] float64 (rows of tokens outside ``tokens_subset`` are 0).
    x_q [tokens, K] (or [tokens, topk, K] per route, sx then [tokens, topk]); w1_q [E*2I, K]
    unshuffled; sx [tokens]; sw1 [E*2I]; ``w_kind`` the weights' kind when it differs from the
    activations'; ``w_groups`` [E, K/g, 2I] group scales in place of sw1."""
    ids = np.asarray(topk_ids).astype(np.int64)
    T, topk = ids.shape
    E = np.asarray(w1_q).shape[0] // (2 * inter_dim)
    x = _act(x_q, sx, kind)
    out = np.zeros((T, topk, inter_dim))
    sel = _selected(T, tokens_subset)
    for e in range(E):
        t_idx, s_idx = np.nonzero((ids == e) & sel[:, None])
        if len(t_idx) == 0:
            continue
        x_in = x[t_idx, s_idx] if x.ndim == 3 else x[t_idx]
        y = x_in @ _expert_w(w1_q, sw1, w_kind or kind, 2 * inter_dim, e, w_groups, w_round).T
        v = silu(y[:, :inter_dim]) * y[:, inter_dim:]
        if doweight:
            v = v * np.asarray(topk_weights, np.float64)[t_idx, s_idx][:, None]
        out[t_idx, s_idx] = v
    return out


def gemm2(a2_q, w2_q, sa2, sw2, topk_ids, topk_weights, model_dim: int, doweight: bool, kind: str,
          tokens_subset=None, w_kind=None, w_groups=None, w_round=None, route_round=None) -> np.ndarray:
    """[tokens, model_dim] float64.  a2_q [tokens*topk, K] (row t*topk + s); w2_q [E*D, K]
    unshuffled; sa2 [tokens*topk]; sw2 [E*D]; ``w_kind`` / ``w_groups`` [E, K/g, D] as in gemm1.
    ``route_round`` ("bf16" / "f16"): the reduce mode -- each route's (weighted) row is written in
    that type before the top-k sum (reference ``compile_moe_gemm2`` with ``accumulate=False``,
    ``kernels/moe_gemm_2stage.py:1267-2481``, then ``compile_moe_reduction``, ``:2484-2604``,
    which sums the rows in fp32)."""
    ids = np.asarray(topk_ids).astype(np.int64)
    T, topk = ids.shape
    E = np.asarray(w2_q).shape[0] // model_dim
    sel = _selected(T, tokens_subset)
    rows = np.nonzero(np.repeat(sel, topk))[0]
    a2 = np.zeros((T * topk, np.asarray(a2_q).shape[1]))
    a2[rows] = dequant_rows(np.asarray(a2_q)[rows], None if sa2 is None else np.asarray(sa2).reshape(-1)[rows], kind,
                            np.float64)
    out = np.zeros((T, model_dim))
    for e in range(E):
        t_idx, s_idx = np.nonzero((ids == e) & sel[:, None])
        if len(t_idx) == 0:
            continue
        y = a2[t_idx * topk + s_idx] @ _expert_w(w2_q, sw2, w_kind or kind, model_dim, e, w_groups, w_round).T
        if doweight:
            y = y * np.asarray(topk_weights, np.float64)[t_idx, s_idx][:, None]
        if route_round is not None:
            y = _round_rows(y, route_round)
        np.add.at(out, t_idx, y)
    return out


def _round_rows(y: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 rows as the kernel holds them, rounded to bf16 / fp16 (nearest even)."""
    from .numerics import bf16_rne, bf16_to_f32
    y32 = np.asarray(y, dtype=np.float32)
    if dtype == "bf16":
        return bf16_to_f32(bf16_rne(y32)).astype(np.float64)
    if dtype == "f16":
        return y32.astype(np.float16).astype(np.float64)
    raise ValueError(f"route_round {dtype!r}")


def _sorted_routes(sorted_ids, sorted_eids, num_valid, block_size, tokens, topk):
    """(entry index i, token, slot, expert) of every valid entry, walking blocks as the kernels do."""
    sid = np.asarray(sorted_ids).astype(np.int64)
    for b, e in enumerate(np.asarray(sorted_eids)):
        if b * block_size >= int(num_valid) or e < 0:
            continue
        for i in range(b * block_size, (b + 1) * block_size):
            t, s = sid[i] & 0xFFFFFF, sid[i] >> 24
            if t < tokens and s < topk:
                yield i, int(t), int(s), int(e)


def gemm1_sorted(x_q, w1_q, sx, sw1, sorted_ids, sorted_w, sorted_eids, num_valid, block_size, tokens, topk,
                 inter_dim, doweight, kind):
    x = dequant_rows(x_q, None if sx is None else np.asarray(sx).reshape(-1), kind, np.float64)
    out = np.zeros((tokens, topk, inter_dim))
    for i, t, s, e in _sorted_routes(sorted_ids, sorted_eids, num_valid, block_size, tokens, topk):
        y = _expert_w(w1_q, sw1, kind, 2 * inter_dim, e) @ x[t]
        v = silu(y[:inter_dim]) * y[inter_dim:]
        out[t, s] = v * float(sorted_w[i]) if doweight else v
    return out


def gemm2_sorted(a2_q, w2_q, sa2, sw2, sorted_ids, sorted_w, sorted_eids, num_valid, block_size, tokens, topk,
                 model_dim, doweight, kind):
    a2 = dequant_rows(a2_q, None if sa2 is None else np.asarray(sa2).reshape(-1), kind, np.float64)
    out = np.zeros((tokens, model_dim))
    for i, t, s, e in _sorted_routes(sorted_ids, sorted_eids, num_valid, block_size, tokens, topk):
        y = _expert_w(w2_q, sw2, kind, model_dim, e) @ a2[t * topk + s]
        out[t] += y * float(sorted_w[i]) if doweight else y
    return out


# ---- blockscale (fp8, 1 x 128 activation blocks, 128 x 128 weight blocks) -----------------
# Restates torch_stage1_blockscale_ref / torch_stage2_blockscale_ref
# (tests/kernels/test_moe_blockscale.py:64-133): activations dequantized per (row, 128-wide K
# block), weights per 128 x 128 block of the flattened [E*rows, K] array, then the same route
# loops as gemm1 / gemm2.

def _dequant_blocks(q, scale, row0: int = 0, blk: int = 128) -> np.ndarray:
    """fp8 bytes [R, K] times scale [R / rb, K / blk] expanded (rb = blk for weights, 1 for
    activations -- told apart by the scale's row count)."""
    from .numerics import e4m3fn_decode
    v = e4m3fn_decode(np.asarray(q)).astype(np.float64)
    s = np.asarray(scale, dtype=np.float64)
    rb = v.shape[0] // s.shape[0] if s.shape[0] != v.shape[0] else 1
    return v * np.repeat(np.repeat(s, rb, axis=0), blk, axis=1)[:, :v.shape[1]]


def gemm1_blockscale(x_q, w1_q, x_scale, w1_scale, topk_ids, topk_weights, inter_dim: int, doweight: bool,
                     tokens_subset=None) -> np.ndarray:
    """x_q [T, D] fp8; x_scale [T, D/128]; w1_q [E*2I, D] fp8 unshuffled; w1_scale [E*2I/128, D/128]."""
    ids = np.asarray(topk_ids).astype(np.int64)
    T, topk = ids.shape
    rows = 2 * inter_dim
    E = np.asarray(w1_q).shape[0] // rows
    x = _dequant_blocks(x_q, x_scale)
    out = np.zeros((T, topk, inter_dim))
    sel = _selected(T, tokens_subset)
    for e in range(E):
        t_idx, s_idx = np.nonzero((ids == e) & sel[:, None])
        if len(t_idx) == 0:
            continue
        w = _dequant_blocks(np.asarray(w1_q)[e * rows:(e + 1) * rows],
                            np.asarray(w1_scale)[e * rows // 128:(e + 1) * rows // 128])
        y = x[t_idx] @ w.T
        v = silu(y[:, :inter_dim]) * y[:, inter_dim:]
        if doweight:
            v = v * np.asarray(topk_weights, np.float64)[t_idx, s_idx][:, None]
        out[t_idx, s_idx] = v
    return out


def gemm2_blockscale(a2_q, w2_q, a2_scale, w2_scale, topk_ids, topk_weights, model_dim: int, doweight: bool,
                     tokens_subset=None) -> np.ndarray:
    """a2_q [T*topk, I] fp8; a2_scale [T*topk, I/128]; w2_q [E*D, I]; w2_scale [E*D/128, I/128]."""
    ids = np.asarray(topk_ids).astype(np.int64)
    T, topk = ids.shape
    E = np.asarray(w2_q).shape[0] // model_dim
    sel = _selected(T, tokens_subset)
    a2 = _dequant_blocks(a2_q, a2_scale)
    out = np.zeros((T, model_dim))
    for e in range(E):
        t_idx, s_idx = np.nonzero((ids == e) & sel[:, None])
        if len(t_idx) == 0:
            continue
        w = _dequant_blocks(np.asarray(w2_q)[e * model_dim:(e + 1) * model_dim],
                            np.asarray(w2_scale)[e * model_dim // 128:(e + 1) * model_dim // 128])
        y = a2[t_idx * topk + s_idx] @ w.T
        if doweight:
            y = y * np.asarray(topk_weights, np.float64)[t_idx, s_idx][:, None]
        np.add.at(out, t_idx, y)
    return out
