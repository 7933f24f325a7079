"""CPU pins of the image-side 3D-aware selection oracle
(oracle/select3d_image.py): each step against a Python-float brute force or
a closed form, on inputs built so that a dropped term, a swapped axis or a
wrong tie order gives a different answer."""

import math

import numpy as np
import pytest

from oracle.select3d import nearest_blocks_ref, nearest_blocks_to_ref
from oracle.select3d_image import (ImageBlocks, block_min_dist2_ref, image_rank_rows_ref,
                                   imcoords_points_ref, project_ref, window_candidates_ref)


def test_imcoords_points_brute_force_and_first_maximum():
    rng = np.random.default_rng(0)
    b_n, m_n, s, pr = 2, 2, 8, 4          # 2x2 dense points per patch
    sp = rng.standard_normal((b_n, m_n, s, s, 3)).astype(np.float32)
    mk = rng.random((b_n, m_n, s, s)).astype(np.float32)
    mk[1, 0, 2:4, 6:8] = 0.75             # patch (1, 3) of image 0: all four tie
    coords = np.array([[b, m, r, c] for b in range(b_n) for m in range(m_n)
                       for r in range(pr) for c in range(pr)])
    out = imcoords_points_ref(coords, sp, mk, pr)
    for t, (b, m, r, c) in enumerate(coords):
        best, arg = None, None
        for i in range(2):
            for j in range(2):
                v = float(mk[b, m, 2 * r + i, 2 * c + j])
                if best is None or v > best:
                    best, arg = v, (2 * r + i, 2 * c + j)
        assert out[t].tolist() == sp[b, m, arg[0], arg[1]].tolist()
    t = int(np.nonzero((coords == [1, 0, 1, 3]).all(1))[0][0])
    assert out[t].tolist() == sp[1, 0, 2, 6].tolist()  # the first of the tied maxima


def test_projection_closed_form():
    # camera at (0, 0, d) looking down -z: world-to-camera = translation by -d
    d, s, ibs, t = 2.0, 33, 4, 0.5
    w2c = np.eye(4, dtype=np.float32)
    w2c[2, 3] = -d
    pts = np.array([[0.0, 0.0, 0.0], [0.5, -0.25, 0.0], [1.0, 1.0, -1.0]], dtype=np.float32)
    bx, by = project_ref(pts, w2c, t, s, ibs)
    # point 0 projects to the image centre
    assert bx[0] == np.float32(0.5 * (s - 1) / ibs) and by[0] == bx[0]
    for k in range(3):
        zc = float(pts[k, 2]) - d
        u = 0.5 * (float(pts[k, 0]) / -zc / t + 1.0) * (s - 1) / ibs
        v = 0.5 * (-float(pts[k, 1]) / -zc / t + 1.0) * (s - 1) / ibs
        assert abs(float(bx[k]) - u) < 1e-5 and abs(float(by[k]) - v) < 1e-5
    # crop: ((u' (o - 1) - x0) / (c - 1)) (S - 1)
    crop = (99.0, 10.0, 20.0, 49.0)
    cx, cy = project_ref(pts, w2c, t, s, ibs, crop)
    for k in range(3):
        zc = float(pts[k, 2]) - d
        u = 0.5 * (float(pts[k, 0]) / -zc / t + 1.0)
        v = 0.5 * (-float(pts[k, 1]) / -zc / t + 1.0)
        assert abs(float(cx[k]) - (u * 99.0 - 10.0) / 49.0 * (s - 1) / ibs) < 1e-4
        assert abs(float(cy[k]) - (v * 99.0 - 20.0) / 49.0 * (s - 1) / ibs) < 1e-4
    # behind the camera: the depth clamps to 1e-6
    bz, _ = project_ref(np.array([[0.1, 0.0, 5.0]], dtype=np.float32), w2c, t, s, ibs)
    assert bz[0] > 1e4


def _blocks(mask, sp, dm, patch_size=2, block_size=2):
    return ImageBlocks(mask, sp, dm, patch_size, block_size)


def test_kept_blocks_and_centres():
    mask = np.zeros((16, 16), dtype=np.float32)   # 4x4 blocks of 4x4 pixels
    mask[5, 6] = 1.0                              # block (1, 1)
    mask[15, 0] = 0.3                             # block (3, 0)
    sp = np.zeros((8, 8, 3), dtype=np.float32)    # 2x2 dense points per block
    sp[2:4, 2:4] = 7.0
    dm = np.ones((8, 8), dtype=np.float32)
    dm[2, 2] = 0.1                                # below 0.2: invalid
    blk = _blocks(mask, sp, dm)
    assert blk.sel.tolist() == [5, 12]
    assert blk.cx.tolist() == [1.5, 0.5] and blk.cy.tolist() == [1.5, 3.5]
    assert blk.ibs == 2 and (blk.pts[0] == 7.0).all()
    assert blk.valid[0].tolist() == [False, True, True, True]


def test_window_candidates_ties_to_lower_block():
    mask = np.ones((16, 16), dtype=np.float32)
    blk = _blocks(mask, np.zeros((8, 8, 3), np.float32), np.ones((8, 8), np.float32))
    # a point at the corner shared by blocks 5, 6, 9, 10 (centres 1.5/2.5)
    bx = np.array([2.0, 0.5], dtype=np.float32)
    by = np.array([2.0, 0.5], dtype=np.float32)
    cand = window_candidates_ref(bx, by, blk, 5)
    assert cand[0, :4].tolist() == [5, 6, 9, 10]
    for t in range(2):
        d = [((float(bx[t]) - (j % 4 + 0.5)) ** 2 + (float(by[t]) - (j // 4 + 0.5)) ** 2, j)
             for j in range(16)]
        assert cand[t].tolist() == [j for _, j in sorted(d)[:5]]


def test_block_min_distance_brute_force():
    rng = np.random.default_rng(3)
    mask = np.ones((16, 16), dtype=np.float32)
    sp = rng.standard_normal((8, 8, 3)).astype(np.float32)
    dm = rng.random((8, 8)).astype(np.float32)
    blk = _blocks(mask, sp, dm)
    pts = rng.standard_normal((5, 3)).astype(np.float32)
    cand = np.array([[0, 3, 15]] * 5)
    max_dist = 0.9
    got = block_min_dist2_ref(pts, cand, blk, max_dist)
    for t in range(5):
        for j, c in enumerate(cand[t]):
            best = math.inf
            for k in range(4):
                if blk.valid[c, k]:
                    d = math.dist([float(v) for v in pts[t]], [float(v) for v in blk.pts[c, k]])
                else:
                    d = float(np.float32(max_dist))
                best = min(best, d)
            assert abs(math.sqrt(got[t, j]) - best) < 1e-12


def _scene(seed, crop=False):
    rng = np.random.default_rng(seed)
    images = []
    for m in range(3):
        mask = (rng.random((16, 16)) < 0.25).astype(np.float32)
        if m == 1:
            mask[:] = 0.0                 # an image with no kept block
        ang = 0.6 * m
        c, s_ = math.cos(ang), math.sin(ang)
        pos = np.array([3.0 * s_, 0.3, 3.0 * c])
        back = pos / np.linalg.norm(pos)
        right = np.cross([0.0, 1.0, 0.0], back)
        right /= np.linalg.norm(right)
        up = np.cross(back, right)
        ext = np.eye(4)
        ext[:3, 0], ext[:3, 1], ext[:3, 2], ext[:3, 3] = right, up, back, pos
        images.append({
            "mask": mask,
            "surface": (0.5 * rng.standard_normal((8, 8, 3))).astype(np.float32),
            "dense_mask": rng.random((8, 8)).astype(np.float32),
            "w2c": np.linalg.inv(ext).astype(np.float32),
            "tan_half": float(np.float32(math.tan(0.45))),
            "crop": (99.0, 10.0, 20.0, 59.0) if crop else None,
        })
    return images


@pytest.mark.parametrize("crop", [False, True])
def test_image_rows_brute_force(crop):
    images = _scene(7, crop)
    rng = np.random.default_rng(8)
    pts = (0.4 * rng.standard_normal((12, 3))).astype(np.float32)
    win, topk, max_dist = 3, 5, 1.0
    rows = image_rank_rows_ref(pts, images, 2, 2, win, topk, max_dist)
    for t in range(pts.shape[0]):
        cands, offset = [], 0
        for im in images:
            blk = _blocks(im["mask"], im["surface"], im["dense_mask"])
            n = blk.sel.shape[0]
            if n == 0:
                continue
            bx, by = project_ref(pts[t:t + 1], im["w2c"], im["tan_half"], blk.s, blk.ibs,
                                 im["crop"])
            d2 = [(float(np.float32(np.float32(bx[0] - blk.cx[j]) ** 2 +
                                    np.float32(by[0] - blk.cy[j]) ** 2)), j) for j in range(n)]
            for _, j in sorted(d2)[:win]:
                dist = math.inf
                for k in range(4):
                    if blk.valid[j, k]:
                        dk = math.dist([float(v) for v in pts[t]],
                                       [float(v) for v in blk.pts[j, k]])
                    else:
                        dk = float(np.float32(max_dist))
                    dist = min(dist, dk)
                cands.append((dist, len(cands), offset + j))
            offset += n
        keep = sorted(sorted(cands)[:topk], key=lambda c: c[1])
        expect = [c[2] for c in keep] + [-1] * (topk - len(keep))
        assert rows[t].tolist() == expect


def test_nearest_blocks_to_matches_self_form():
    rng = np.random.default_rng(9)
    pts = rng.standard_normal((60, 3)).astype(np.float32)
    cu = np.array([0, 10, 25, 40, 60])
    a = nearest_blocks_ref(pts, cu, np.array([0, 4]), np.array([0, 60]), 3)
    b = nearest_blocks_to_ref(pts, pts, cu, np.array([0, 4]), np.array([0, 60]), 3)
    assert (a == b).all()
    # image points against volume-block centroids: brute force
    q = rng.standard_normal((7, 3)).astype(np.float32)
    got = nearest_blocks_to_ref(q, pts, cu, np.array([0, 4]), np.array([0, 7]), 2)
    cen = [pts[cu[i]:cu[i + 1]].astype(np.float64).mean(0) for i in range(4)]
    for t in range(7):
        d = sorted((math.dist(q[t].tolist(), c.tolist()), i) for i, c in enumerate(cen))
        assert got[t].tolist() == sorted(i for _, i in d[:2])
