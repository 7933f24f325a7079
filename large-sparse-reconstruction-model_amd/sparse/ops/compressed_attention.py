"""Attention of every query against the compressed (block-pooled) keys of its
batch element: the drop-in for the flash_attn_varlen_func call of
SpatialSparseAttentionMid.forward (sparse/module/spatial_sparse_attention.py:
121-145, causal=False, return_attn_probs=True -> (out, softmax_lse, _)).

The compressed keys of batch element b are one contiguous run of rows, so
this is selected attention with a single selected "block" per batch element:
the gfx950 selected-attention kernels run it (forward and, through the same
autograd Function, backward for q, compressed_k and compressed_v).  The LSE
is returned in natural-log units [Hq, total_q], as flash-attn returns it and
as get_block_score expects.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .native_sparse_attention import native_sparse_attend

LN2 = math.log(2.0)


def compressed_attention(q: torch.Tensor, compressed_k: torch.Tensor,
                         compressed_v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                         compressed_cu_seqlens: torch.Tensor,
                         softmax_scale: Optional[float] = None, return_lse: bool = True):
    """q [total_q, Hq, D], compressed_k / compressed_v [total_compressed, Hkv, D],
    cu_seqlens_q / compressed_cu_seqlens [batch + 1] int32 -> out
    [total_q, Hq, D] (and lse [Hq, total_q] fp32, natural log, when
    return_lse).  A batch element without compressed keys gives out = 0 and
    lse = -inf."""
    hkv = compressed_k.shape[1]
    batch = cu_seqlens_q.numel() - 1
    dev = q.device
    # one selected block (batch-local id 0) per query: all compressed keys
    topk_idx = torch.zeros((hkv, q.shape[0], 1), dtype=torch.int32, device=dev)
    cu_seqblocks = torch.arange(batch + 1, dtype=torch.int32, device=dev)
    cu_c = compressed_cu_seqlens.to(torch.int32)
    out, lse2 = native_sparse_attend(q, compressed_k, compressed_v, topk_idx, cu_seqblocks,
                                     cu_c, cu_seqlens_q.to(torch.int32), cu_c,
                                     softmax_scale=softmax_scale, return_lse=True)
    if not return_lse:
        return out
    return out, lse2 * LN2
