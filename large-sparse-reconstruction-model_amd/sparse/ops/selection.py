"""Per-query-block top-k block selection (self attention).

Rule: mean-pool Q and K per block (fp32), score each (query block, key
block) pair of a batch element by the fp64 dot product of the pooled means
summed over the query heads of a kv head, force the query's own block (and
an optional list of batch-local blocks, e.g. the image blocks of a mixed
image/voxel sequence) and fill the remaining slots by (score descending,
block id ascending).  Output rows are ascending, -1 padded, in the
[num_kv_heads, total_tokens, topk] layout spatial_selection_attention reads
(the layout sparse/ops/block_score.py:16-98 produces in the reference).
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

import lsrm_hip  # noqa: F401  (registers torch.ops.lsrm_hip)


def select_blocks(q: torch.Tensor, k: torch.Tensor, cu_seqblocks: torch.Tensor,
                  cu_block_include_tokens: torch.Tensor, topk: int,
                  forced_blocks: Optional[Sequence[int]] = None, force_self: bool = True,
                  return_compact: bool = False):
    """q [N, Hq, D], k [N, Hkv, D] -> block_topk [Hkv, N, topk] int32
    (and the per-block rows [Hkv, n_blocks, topk] when return_compact)."""
    topk_idx, compact = torch.ops.lsrm_hip.select_blocks(
        q, k, cu_seqblocks, cu_block_include_tokens, int(topk),
        [int(b) for b in (forced_blocks or [])], bool(force_self), None)
    if return_compact:
        return topk_idx, compact
    return topk_idx
