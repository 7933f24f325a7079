"""3D-aware per-token selection oracles on the image side (test infrastructure).

Restates, in numpy on the CPU, the use_3d_aware_attn branches of
  build_image_to_image_attn   misc/sparse_utils.py:690-898
  build_image_to_volume_attn  misc/sparse_utils.py:901-988
  build_volume_to_image_attn  misc/sparse_utils.py:991-1200
and their helpers from_imcoords_to_points (653-688) and
compute_block_topk_dist_chunked (16-57).  The HIP path must match these
bit for bit (indices are integers); they fix the arithmetic the reference
leaves to its libraries:
  * image token point (653-688): the dense surface point of the token's
    patch whose mask value is largest, the first one in (row, column) order
    among equal maxima (torch.max(dim).indices returns the first);
  * image blocks (the per-image loop, 733-792 / 1034-1091): block (by, bx)
    of block_pixel_size = patch_size * block_size pixels is kept when its
    mask pixels sum to non-zero (the mask is non-negative, so: any pixel
    non-zero), kept blocks numbered in row-major order; its dense points are
    the impoints_block_size^2 points under it (impoints_block_size =
    dense_res // blocks per column), valid where masks_input > 0.2; its
    centre is (bx + 0.5, by + 0.5);
  * projection (795-840 / 1093-1138) in fp32 with every product and sum
    rounded separately, in this order: p_c = ((x w_c0 + y w_c1) + z w_c2) +
    w_c3 for the rows c = 0..2 of the world-to-camera matrix (the inverse
    of the camera's extrinsic, as the caller computes it), u = p_0 /
    max(-p_2, 1e-6), v = -p_1 / max(-p_2, 1e-6), u' = 0.5 (u / t + 1),
    v' = 0.5 (v / t + 1) with t = tan(fov / 2) as the caller computes it;
    pixel = u' (S - 1), or with a crop ((u' (o - 1) - c) / (s - 1)) (S - 1);
    block coordinate = pixel / impoints_block_size (the reference's matmul
    and tan are library routines; this order is the build's);
  * window candidates (842-845): per image, the min(win, kept blocks)
    blocks nearest in block coordinates, by the fp32 value
    (bx - cx)^2 + (by - cy)^2, the lower block number among equal values
    (torch.topk leaves ties unspecified);
  * 3D distance of a candidate (16-57): the smallest distance from the
    token's point to the block's dense points, a masked point counting
    max_dist = fp32(2 * bbox_radius); ranked by the exact squared distance
    (fp32 differences, squares and the three-term sum are exact in float64;
    the reference ranks fp32 square roots);
  * final row (858-890): the candidates of all images concatenated (image
    order, then window rank), the min(topk_num, total) nearest kept, the
    lower position among equal distances, written in position order, block
    ids offset by the kept blocks of the earlier images, -1 padded;
  * image to volume (901-988): the nearest volume-block centroids to the
    image token points, the rule of oracle/select3d.nearest_blocks_ref.
Pins: tests/test_oracle_select3d_image.py (Python-float brute force of every
step, a camera with a known projection, hand-built masks and tie cases).
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import numpy as np

F32 = np.float32


def imcoords_points_ref(imcoords: np.ndarray, surface_points: np.ndarray, masks: np.ndarray,
                        patch_res: int) -> np.ndarray:
    """imcoords [N, 4] (batch, image, patch row, patch column); surface_points
    [B, M, S, S, 3] fp32; masks with B*M*S*S values -> points [N, 3] fp32."""
    sp = np.asarray(surface_points, dtype=np.float32)
    b_n, m_n, s = sp.shape[0], sp.shape[1], sp.shape[2]
    mk = np.asarray(masks, dtype=np.float32).reshape(b_n, m_n, s, s)
    ps = s // patch_res
    c = np.asarray(imcoords, dtype=np.int64)
    out = np.empty((c.shape[0], 3), dtype=np.float32)
    for t in range(c.shape[0]):
        b, m, r, col = (int(x) for x in c[t])
        vals = mk[b, m, r * ps:(r + 1) * ps, col * ps:(col + 1) * ps].reshape(-1)
        k = int(np.argmax(vals))  # first maximum (NaN counts as the maximum)
        i, j = divmod(k, ps)
        out[t] = sp[b, m, r * ps + i, col * ps + j]
    return out


class ImageBlocks:
    """Kept blocks of one image: ids (row-major block numbers), centres,
    dense points [n, ibs*ibs, 3] and validity [n, ibs*ibs]."""

    def __init__(self, mask_img, sp_m, mk_m, patch_size: int, block_size: int):
        mask = np.asarray(mask_img, dtype=np.float32)
        bps = patch_size * block_size
        h, w = mask.shape
        self.bh, self.bw = h // bps, w // bps
        blocks = mask[: self.bh * bps, : self.bw * bps].reshape(self.bh, bps, self.bw, bps)
        any_px = (blocks != 0).any(axis=(1, 3)).reshape(-1)
        self.sel = np.nonzero(any_px)[0]
        sp_m = np.asarray(sp_m, dtype=np.float32)
        self.s = sp_m.shape[0]
        self.ibs = self.s // self.bh
        ibs = self.ibs
        pts = sp_m[: self.bh * ibs, : self.bw * ibs].reshape(self.bh, ibs, self.bw, ibs, 3)
        pts = pts.transpose(0, 2, 1, 3, 4).reshape(self.bh * self.bw, ibs * ibs, 3)
        valid = np.asarray(mk_m, dtype=np.float32).reshape(self.s, self.s)
        valid = (valid[: self.bh * ibs, : self.bw * ibs] > F32(0.2)).reshape(
            self.bh, ibs, self.bw, ibs).transpose(0, 2, 1, 3).reshape(self.bh * self.bw, -1)
        self.pts = pts[self.sel]
        self.valid = valid[self.sel]
        self.cx = (self.sel % self.bw).astype(np.float32) + F32(0.5)
        self.cy = (self.sel // self.bw).astype(np.float32) + F32(0.5)


def project_ref(points: np.ndarray, w2c: np.ndarray, tan_half: float, s: int, ibs: int,
                crop: Optional[Sequence[float]] = None):
    """-> (bx, by) fp32 block coordinates of the points in one image.  crop
    = (origin_size - 1, crop x0, crop y0, crop_size - 1) as fp32 values."""
    p = np.asarray(points, dtype=np.float32)
    wm = np.asarray(w2c, dtype=np.float32)
    x, y, z = p[:, 0], p[:, 1], p[:, 2]
    pc = [((x * wm[c, 0] + y * wm[c, 1]) + z * wm[c, 2]) + wm[c, 3] for c in range(3)]
    den = np.maximum(-pc[2], F32(1e-6))
    u = pc[0] / den
    v = -pc[1] / den
    t = F32(tan_half)
    u = F32(0.5) * (u / t + F32(1.0))
    v = F32(0.5) * (v / t + F32(1.0))
    sm1 = F32(s - 1)
    if crop is not None:
        om1, cx0, cy0, csm1 = (F32(c) for c in crop)
        px = ((u * om1 - cx0) / csm1) * sm1
        py = ((v * om1 - cy0) / csm1) * sm1
    else:
        px = u * sm1
        py = v * sm1
    return px / F32(ibs), py / F32(ibs)


def window_candidates_ref(bx: np.ndarray, by: np.ndarray, blocks: ImageBlocks, win: int):
    """-> [N, min(win, kept)] kept-block numbers, nearest first."""
    d2 = (bx[:, None] - blocks.cx[None, :]) ** 2 + (by[:, None] - blocks.cy[None, :]) ** 2
    d2 = d2.astype(np.float32)
    k = min(win, blocks.sel.shape[0])
    ids = np.arange(blocks.sel.shape[0])
    out = np.empty((bx.shape[0], k), dtype=np.int64)
    for t in range(bx.shape[0]):
        order = np.lexsort((ids, d2[t]))
        out[t] = order[:k]
    return out


def block_min_dist2_ref(points: np.ndarray, cand: np.ndarray, blocks: ImageBlocks,
                        max_dist: float) -> np.ndarray:
    """Exact squared 3D distance from each point to each candidate block
    (min over the block's dense points; invalid points count max_dist)."""
    p64 = np.asarray(points, dtype=np.float32).astype(np.float64)
    md = float(F32(max_dist))
    out = np.empty(cand.shape, dtype=np.float64)
    for t in range(cand.shape[0]):
        for j in range(cand.shape[1]):
            q = blocks.pts[cand[t, j]].astype(np.float64)
            d = q - p64[t][None, :]
            d2 = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
            d2 = np.where(blocks.valid[cand[t, j]], d2, md * md)
            d2 = np.where(np.isnan(d2), np.inf, d2)
            out[t, j] = d2.min() if d2.shape[0] else np.inf
    return out


def image_rank_rows_ref(points: np.ndarray, images: List[dict], patch_size: int,
                        block_size: int, win: int, topk_num: int, max_dist: float) -> np.ndarray:
    """The per-token rows of one batch element.  points [N, 3] fp32 (the
    query points); images: one dict per image with keys mask [H, W],
    surface [S, S, 3], dense_mask [S, S], w2c [4, 4], tan_half, crop (None
    or the 4 fp32 values of project_ref) -> [N, topk_num] int32."""
    n = points.shape[0]
    cands, dists = [], []
    offset = 0
    for im in images:
        blocks = ImageBlocks(im["mask"], im["surface"], im["dense_mask"], patch_size, block_size)
        if blocks.sel.shape[0] == 0:
            continue
        bx, by = project_ref(points, im["w2c"], im["tan_half"], blocks.s, blocks.ibs,
                             im.get("crop"))
        cand = window_candidates_ref(bx, by, blocks, win)
        cands.append(cand + offset)
        dists.append(block_min_dist2_ref(points, cand, blocks, max_dist))
        offset += blocks.sel.shape[0]
    out = np.full((n, topk_num), -1, dtype=np.int32)
    if not cands:
        return out
    cand = np.concatenate(cands, axis=1)
    dist = np.concatenate(dists, axis=1)
    k = min(topk_num, cand.shape[1])
    pos = np.arange(cand.shape[1])
    for t in range(n):
        keep = np.sort(np.lexsort((pos, dist[t]))[:k])
        out[t, :k] = cand[t, keep]
    return out
