"""Per-block ("window") attention: every block attends only to itself.

Replaces sparse/ops/block_window_attention.py:14-31, which runs
flash_attn_varlen_func with the block offsets as cu_seqlens for q and k
(non-causal, scale 1/sqrt(D)).  Here the self-block selection is built on
the device (lsrm_block_ids) and fed to the selected-attention kernels, so
forward and backward both run on gfx950 HIP kernels.
"""

from __future__ import annotations

import torch

import lsrm_hip as _hip

from .native_sparse_attention import native_sparse_attend


def sparse_window_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            cu_block_include_tokens: torch.Tensor) -> torch.Tensor:
    """q [N, Hq, D], k/v [N, Hkv, D] -> [N, Hq, D]; block-diagonal attention."""
    if q.shape[0] != k.shape[0]:
        raise ValueError("window attention needs as many query tokens as key tokens")
    dev = q.device
    cu = _hip._i32(cu_block_include_tokens)
    nb = cu.numel() - 1
    n = q.shape[0]
    cu_seqblocks = torch.tensor([0, nb], dtype=torch.int32, device=dev)
    cu_seqlens = torch.tensor([0, n], dtype=torch.int32, device=dev)
    ids = torch.ops.lsrm_hip.block_ids(cu_seqblocks, cu, n, k.shape[1])
    return native_sparse_attend(q, k, v, ids, cu_seqblocks, cu, cu_seqlens, cu_seqlens)
