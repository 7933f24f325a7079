"""MI355X-native replacement of LSRM's ``sparse`` package hot path.

``sparse.ops`` keeps the call signatures and tensor layouts of the
reference's ``sparse/ops`` (spatial_selection_attention, native_sparse_attend,
sparse_window_attention, get_block_score) and adds the block compression,
per-query-block selection, compressed attention and gated branch merge
operators.  Every operator runs on gfx950 HIP kernels from liblsrm_hip.so,
reached through the registered PyTorch operators torch.ops.lsrm_hip.*
(lsrm_hip.torch_ops).
"""
