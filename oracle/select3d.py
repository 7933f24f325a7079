"""3D-aware per-token block selection oracle (volume to volume).

Restates the use_3d_aware_attn branch of build_volume_to_volume_attn
(misc/sparse_utils.py:1203-1280) for one kv head (the reference stacks the
same rows for its two kv heads, line 1273):
  * token points from integer volume coordinates (from_volcoords_to_points,
    misc/sparse_utils.py:644-650): radius = bbox_radius * 1.05,
    z = 2 (c1 / (R - 1) - 0.5) radius, y from c2, x from c3, point (x, y, z),
    in fp32;
  * block centroids: the mean of the block's token points
    (torch.segment_reduce mean, line 1237), here under the pooling contract
    of oracle/pool.py (fp32, bit-exact with lsrm_block_mean_pool);
  * per token, the min(topk, blocks of its batch element) blocks nearest to
    its point, listed ascending, -1 padded (lines 1244-1268).
Distances rank by the exact squared distance: fp32 differences, squares and
their three-term sum are all exact in float64, so the ranking is a fixed
function of the fp32 points and centroids; among equal distances the lower
block id wins.  (The reference ranks fp32 sqrt values with torch.topk; it can
differ only among points that are at equal distance up to fp32 rounding.)
Pins (tests/test_oracle_select3d.py): a brute force over Python floats with
the distance itself (math.dist); a regular grid whose nearest blocks are
known by construction; topk >= blocks selects all; ties to the lowest id.
"""

from __future__ import annotations

import numpy as np

from oracle.pool import block_mean_pool_ref


def volume_points_ref(coords: np.ndarray, volume_res: int, bbox_radius: float) -> np.ndarray:
    """coords [N, 4] ints (batch, c1, c2, c3) -> points [N, 3] fp32 (x, y, z)."""
    c = np.asarray(coords)
    radius = np.float32(bbox_radius * 1.05)
    den = np.float32(volume_res - 1)
    half = np.float32(0.5)
    two = np.float32(2.0)
    z = two * (c[:, 1].astype(np.float32) / den - half) * radius
    y = two * (c[:, 2].astype(np.float32) / den - half) * radius
    x = two * (c[:, 3].astype(np.float32) / den - half) * radius
    return np.stack([x, y, z], axis=1).astype(np.float32)


def nearest_blocks_ref(points: np.ndarray, cu_block_tokens: np.ndarray,
                       cu_seqblocks: np.ndarray, cu_seqlens: np.ndarray, topk: int,
                       chunk: int = 4096) -> np.ndarray:
    """points [N, 3] fp32 -> [N, topk] int32 batch-local block ids."""
    return nearest_blocks_to_ref(points, points, cu_block_tokens, cu_seqblocks, cu_seqlens, topk,
                                 chunk)


def nearest_blocks_to_ref(qpoints: np.ndarray, key_points: np.ndarray,
                          cu_block_tokens: np.ndarray, cu_seqblocks: np.ndarray,
                          cu_seqlens_q: np.ndarray, topk: int, chunk: int = 4096) -> np.ndarray:
    """Query points [Nq, 3] against the block centroids of other key points
    (build_image_to_volume_attn, misc/sparse_utils.py:960-980: image token
    points against volume-block centroids) -> [Nq, topk] int32."""
    pts = np.asarray(qpoints, dtype=np.float32)
    cu_blk = np.asarray(cu_block_tokens, dtype=np.int64)
    cen = block_mean_pool_ref(np.asarray(key_points, dtype=np.float32), cu_blk)  # [nb, 3]
    cu_sb = np.asarray(cu_seqblocks, dtype=np.int64)
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    out = np.full((pts.shape[0], topk), -1, dtype=np.int32)
    for b in range(cu_q.shape[0] - 1):
        qs, qe = int(cu_q[b]), int(cu_q[b + 1])
        bs, be = int(cu_sb[b]), int(cu_sb[b + 1])
        nbb = be - bs
        if nbb <= 0:
            continue
        kk = min(topk, nbb)
        c64 = cen[bs:be].astype(np.float64)
        ids = np.arange(nbb)
        for r0 in range(qs, qe, chunk):
            r1 = min(qe, r0 + chunk)
            p64 = pts[r0:r1].astype(np.float64)
            d2 = np.zeros((r1 - r0, nbb), dtype=np.float64)
            for a in range(3):
                diff = p64[:, a, None] - c64[None, :, a]
                d2 = d2 + diff * diff
            d2 = np.where(np.isnan(d2), np.inf, d2)
            # (distance, id) lexicographic: stable argsort on distance keeps ids ascending
            order = np.argsort(d2, axis=1, kind="stable")[:, :kk]
            out[r0:r1, :kk] = np.sort(ids[order], axis=1)
    return out
