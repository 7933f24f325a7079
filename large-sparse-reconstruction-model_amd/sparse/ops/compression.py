"""Key/value block compression: per-block mean over variable-length blocks.

Replaces SpatialSparseAttentionIn.sparse3d_compression
(sparse/module/spatial_sparse_attention.py:27-37), which calls
torch.segment_reduce(data=x, reduce="mean", lengths=..., axis=0) on a 2-D
[N, H*D] tensor; here the reduction is the lsrm_block_mean_pool HIP kernel
(operator torch.ops.lsrm_hip.block_mean_pool).
"""

from __future__ import annotations

from typing import Optional

import torch

import lsrm_hip  # noqa: F401  (registers torch.ops.lsrm_hip)


def sparse3d_compression(x: torch.Tensor, cu_block_include_tokens: torch.Tensor) -> torch.Tensor:
    """[N, C] -> [n_blocks, C] block means in x's dtype (an empty block gives
    NaN, as torch.segment_reduce does)."""
    return torch.ops.lsrm_hip.block_mean_pool(x, cu_block_include_tokens)


def block_mean_pool(x: torch.Tensor, cu_block_include_tokens: torch.Tensor,
                    out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Like sparse3d_compression; accepts [N, H, D] (pooled per head) and an
    output dtype (fp32 keeps the unrounded means used by select_blocks)."""
    if x.dim() == 3:
        n, h, d = x.shape
        return torch.ops.lsrm_hip.block_mean_pool(x.reshape(n, h * d), cu_block_include_tokens,
                                                  out_dtype).view(-1, h, d)
    return torch.ops.lsrm_hip.block_mean_pool(x, cu_block_include_tokens, out_dtype)
