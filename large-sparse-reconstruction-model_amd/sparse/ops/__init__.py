"""gfx950 HIP replacement of LSRM's sparse/ops (same public names and
signatures as sparse/ops/__init__.py:7-9, plus the compression, selection,
learned-selection (get_block_score, sparse/ops/block_score.py:16-98),
compressed-attention and gated branch merge
(sparse/module/spatial_sparse_attention.py:256-269) operators)."""

from .block_score import get_block_score
from .block_window_attention import sparse_window_attention
from .compressed_attention import compressed_attention
from .compression import block_mean_pool, sparse3d_compression
from .gate_merge import GateMerge, gate_merge
from .native_sparse_attention import (
    NSA,
    native_sparse_attend,
    set_key_centric,
    set_validation,
    set_variant,
    spatial_selection_attention,
)
from .selection import select_blocks

__all__ = [
    "GateMerge",
    "NSA",
    "block_mean_pool",
    "compressed_attention",
    "gate_merge",
    "get_block_score",
    "native_sparse_attend",
    "select_blocks",
    "set_key_centric",
    "set_validation",
    "set_variant",
    "sparse3d_compression",
    "sparse_window_attention",
    "spatial_selection_attention",
]
