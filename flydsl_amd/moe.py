"""Routing metadata for the MoE 2-stage GEMM: ``moe_sorting`` groups the routes of a top-k
routing by expert and pads each expert's run to the GEMM's row block.

Same outputs as the reference harness's ``moe_sorting_torch_native``
(``tests/kernels/test_moe_gemm.py:97-160``), computed without a per-expert loop or a host
synchronisation, so it runs on the device tensors it is given:

* ``sorted_ids`` int32 ``[tokens*topk + E*block - topk]``: per expert in order, its routes in
  row-major order of ``topk_ids`` as ``(slot << 24) | token``, padded to a multiple of ``block``
  with ``(topk << 24) | tokens``;
* ``sorted_weights`` fp32, aligned with ``sorted_ids`` (0 in the padding);
* ``sorted_expert_ids`` int32 ``[ceil(len(sorted_ids) / block)]``: the expert of each block,
  -1 past the last;
* ``num_tokens_post_pad`` int32 ``[2]``: the padded row count and ``tokens``.

With ``expert_mask`` (0/1 per expert), routes to masked experts are dropped and the remaining
experts are renumbered consecutively, as in the reference.
"""
from __future__ import annotations

import torch


def moe_sorting(topk_ids: torch.Tensor, topk_weights: torch.Tensor, num_experts: int, block_size: int,
                expert_mask: torch.Tensor | None = None):
    if topk_ids.dim() != 2 or topk_weights.shape != topk_ids.shape:
        raise ValueError(f"topk_ids / topk_weights must both be [tokens, topk], got {tuple(topk_ids.shape)} "
                         f"and {tuple(topk_weights.shape)}")
    E, bs = int(num_experts), int(block_size)
    if E <= 0 or bs <= 0:
        raise ValueError(f"num_experts={E} and block_size={bs} must be positive")
    dev = topk_ids.device
    M, topk = topk_ids.shape
    max_pad = M * topk + E * bs - topk
    max_blocks = (max_pad + bs - 1) // bs

    flat = topk_ids.reshape(-1).to(torch.int64)
    route = torch.arange(M * topk, device=dev, dtype=torch.int64)     # t * topk + s
    keep = (flat >= 0) & (flat < E)
    local = torch.arange(E, device=dev, dtype=torch.int64)
    if expert_mask is not None:
        m = expert_mask.to(device=dev).reshape(-1)[:E].to(torch.int64) != 0
        keep = keep & m[flat.clamp(0, E - 1)]
        local = torch.cumsum(m.to(torch.int64), 0) - 1                # renumbered id of kept experts
    key = torch.where(keep, flat, torch.full_like(flat, E))           # dropped routes sort last
    key_sorted, order = torch.sort(key, stable=True)
    counts = torch.bincount(key, minlength=E + 1)[:E]
    padded = (counts + bs - 1) // bs * bs
    start = torch.cumsum(padded, 0) - padded                          # first row of each expert
    first = torch.cumsum(counts, 0) - counts                          # first sorted route of each expert

    n_keep = M * topk  # routes past the kept ones carry key E and are discarded below
    j = torch.arange(n_keep, device=dev, dtype=torch.int64)
    valid = key_sorted < E
    e_of = key_sorted.clamp(max=E - 1)
    dest = torch.where(valid, start[e_of] + (j - first[e_of]), torch.full_like(j, max_pad))

    t = order // topk
    s = order % topk
    sorted_ids = torch.full((max_pad + 1,), (topk << 24) | M, device=dev, dtype=torch.int64)
    sorted_ids[dest] = (s << 24) | t
    sorted_w = torch.zeros(max_pad + 1, device=dev, dtype=torch.float32)
    sorted_w[dest] = topk_weights.reshape(-1).to(torch.float32)[order]

    # expert of each block: blocks [start_e / bs, (start_e + padded_e) / bs) belong to expert e
    blk_end = torch.cumsum(padded // bs, 0)                           # exclusive end block per expert
    b = torch.arange(max_blocks, device=dev, dtype=torch.int64)
    e_blk = torch.searchsorted(blk_end, b, right=True)
    sorted_eids = torch.where(e_blk < E, local[e_blk.clamp(max=E - 1)], torch.full_like(b, -1))

    post = torch.stack([padded.sum(), torch.tensor(M, device=dev, dtype=torch.int64)]).to(torch.int32)
    return sorted_ids[:max_pad].to(torch.int32), sorted_w[:max_pad], sorted_eids.to(torch.int32), post
