"""Learned block selection: the drop-in for sparse/ops/block_score.py:16-98.

get_block_score keeps the reference signature and output layout
([num_kv_heads, total_q, topk] int32, batch-local compressed-key ids
ascending, -1 padded) and runs on the gfx950 kernel lsrm_block_score (one
launch through the operator torch.ops.lsrm_hip.block_score, no host
synchronisation; the reference loops over batch elements and
kv heads with .item() calls and a dense [q_len, n_compressed] score matrix
per head).  seqlens_q / compressed_seqlens are accepted and unused, as the
lengths follow from the cumulative arrays.
"""

from __future__ import annotations

import math

import torch

import lsrm_hip  # noqa: F401  (registers torch.ops.lsrm_hip)


def get_block_score(
    q: torch.Tensor,
    compressed_k: torch.Tensor,
    lse: torch.Tensor,
    topk: int,
    cu_seqlens_q: torch.Tensor,
    compressed_cu_seqlens: torch.Tensor,
    seqlens_q: torch.Tensor,
    compressed_seqlens: torch.Tensor,
    sm_scale: float = None,
) -> torch.Tensor:
    """q [total_q, Hq, D], compressed_k [total_compressed, Hkv, D], lse
    [Hq, total_q] (natural log, as flash-attn / compressed_attention return
    it) -> block_topk [Hkv, total_q, topk] int32.

    Score of compressed key c for token i and kv head h: the sum over h's
    query heads g of exp2(q[i,g].ck[c,h] * sm_scale * 1.44269504 -
    lse[g,i] * 1.44269504); the min(topk, n_compressed) best keys, ascending.
    Among equal scores the lower id is chosen (torch.topk leaves that order
    unspecified in the reference).
    """
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    return torch.ops.lsrm_hip.block_score(q, compressed_k, lse, int(topk), cu_seqlens_q,
                                          compressed_cu_seqlens, float(sm_scale))
