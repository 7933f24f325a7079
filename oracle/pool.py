"""Block mean pooling oracle.

Restates SpatialSparseAttentionIn.sparse3d_compression
(sparse/module/spatial_sparse_attention.py:27-37): torch.segment_reduce
(reduce="mean") over the rows of each block.  The summation order is the
library's and unspecified there; this build fixes it (the contract the HIP
kernel implements bit for bit):
  * rows are cut into pieces at every multiple of 64 of the global row index
    and at block boundaries;
  * each piece is summed in fp32 in row order, starting from +0.0;
  * a block's piece sums are added in order, starting from +0.0;
  * mean = IEEE fp32 quotient sum / length (0/0 = NaN for an empty block),
    then rounded to the output type to nearest even.
Pins: torch.segment_reduce (the reference's own call) within fp32 rounding;
exact results on integer-valued inputs (every partial sum representable);
hand-computed cancellation cases that distinguish the piece order from a
plain sequential or pairwise sum (tests/test_oracle_pool.py).
"""

from __future__ import annotations

import numpy as np

CHUNK = 64


def block_mean_pool_ref(x: np.ndarray, cu: np.ndarray) -> np.ndarray:
    """x [N, C] float32, cu [nb + 1] ints -> [nb, C] float32 means."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cu = np.asarray(cu, dtype=np.int64)
    n, c = x.shape
    nb = cu.shape[0] - 1
    out = np.empty((nb, c), dtype=np.float32)
    zero = np.float32(0.0)
    for b in range(nb):
        s = int(min(max(cu[b], 0), n))
        e = int(min(max(cu[b + 1], 0), n))
        acc = np.zeros(c, dtype=np.float32)
        if e > s:
            for j in range(s // CHUNK, (e - 1) // CHUNK + 1):
                lo, hi = max(s, CHUNK * j), min(e, CHUNK * j + CHUNK)
                # accumulate() is a running sequential sum; adding it to +0.0
                # reproduces a sum started from +0.0 (they differ only in the
                # sign of an all-negative-zero piece).
                piece = zero + np.add.accumulate(x[lo:hi], axis=0, dtype=np.float32)[-1]
                acc = acc + piece
            out[b] = acc / np.float32(e - s)
        else:
            out[b] = np.float32(np.nan)
    return out
