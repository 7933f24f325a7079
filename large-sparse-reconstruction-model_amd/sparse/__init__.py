"""MI355X-native replacement of LSRM's ``sparse`` package hot path.

``sparse.ops`` keeps the call signatures and tensor layouts of the
reference's ``sparse/ops`` (spatial_selection_attention, native_sparse_attend,
sparse_window_attention) and adds the block compression and per-query-block
selection operators; every operator runs on gfx950 HIP kernels from
liblsrm_hip.so.  The reference's learned selection (get_block_score) is not
provided.
"""
