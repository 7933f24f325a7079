"""Reverse (CSR) query map oracle.

Restates _build_reverse_query_mapping
(sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:575-684): for
each kv head and global block c = cu_seqblocks[b] + v (v a valid batch-local
id of query i, kvcentric:525-529), the ascending list of query ids that
selected c, one entry per selection (a repeated id appears twice);
cu_reverse_count is the exclusive prefix of the per-block counts.
Pins: a dict-of-lists build in pure Python on tiny inputs; counts sum to the
number of valid entries; every (block, query) pair appears with its
multiplicity (tests/test_oracle_revmap.py).
"""

from __future__ import annotations

import numpy as np


def reverse_query_map_ref(topk_idx: np.ndarray, cu_seqlens_q: np.ndarray,
                          cu_seqblocks: np.ndarray, total_blocks: int):
    """-> (cu_reverse_count [Hkv, nb+1] int32, list of per-head int32 arrays)."""
    hkv, nq, k = topk_idx.shape
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_sb = np.asarray(cu_seqblocks, dtype=np.int64)
    nbb = np.zeros(nq, dtype=np.int64)
    base = np.zeros(nq, dtype=np.int64)
    for b in range(cu_q.shape[0] - 1):
        nbb[cu_q[b]:cu_q[b + 1]] = cu_sb[b + 1] - cu_sb[b]
        base[cu_q[b]:cu_q[b + 1]] = cu_sb[b]
    cu_rev = np.zeros((hkv, total_blocks + 1), dtype=np.int32)
    lists = []
    for h in range(hkv):
        t = topk_idx[h].astype(np.int64)
        valid = (t >= 0) & (t < nbb[:, None])
        qi = np.repeat(np.arange(nq), k).reshape(nq, k)[valid]
        blk = (t + base[:, None])[valid]
        order = np.argsort(blk, kind="stable")   # entries are (query, slot) ordered
        counts = np.bincount(blk, minlength=total_blocks)[:total_blocks]
        cu_rev[h, 1:] = np.cumsum(counts)
        lists.append(qi[order].astype(np.int32))
    return cu_rev, lists
