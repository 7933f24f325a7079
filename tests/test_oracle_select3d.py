"""Pins of the 3D-aware selection oracle (oracle/select3d.py): brute force
with the Euclidean distance itself, a layout whose nearest blocks are known
by construction, the point formula on known coordinates, and the layout
rules (topk >= blocks, ties to the lowest id, batch-local ids)."""

import math

import numpy as np

from oracle.pool import block_mean_pool_ref
from oracle.select3d import nearest_blocks_ref, volume_points_ref


def test_points_follow_the_reference_formula():
    # R = 65: c = 0 -> -radius, c = 64 -> +radius, c = 32 -> 0 (radius = 1.05 r)
    coords = np.array([[0, 0, 32, 64], [0, 64, 0, 32]])
    p = volume_points_ref(coords, 65, 2.0)
    r = np.float32(2.0 * 1.05)
    np.testing.assert_allclose(p, [[r, 0.0, -r], [0.0, -r, r]], rtol=1e-6, atol=1e-6)


def test_matches_brute_force_with_math_dist():
    rng = np.random.default_rng(0)
    pts = rng.standard_normal((60, 3)).astype(np.float32)
    sizes = [7, 3, 12, 9, 5, 10, 8, 6]
    cu = np.concatenate([[0], np.cumsum(sizes)])
    cu_sb = np.array([0, 3, 8])
    cu_q = np.array([0, 22, 60])
    got = nearest_blocks_ref(pts, cu, cu_sb, cu_q, 3)
    cen = block_mean_pool_ref(pts, cu)
    for b in range(2):
        for i in range(cu_q[b], cu_q[b + 1]):
            cand = [(math.dist(pts[i].tolist(), cen[c].tolist()), c - cu_sb[b])
                    for c in range(cu_sb[b], cu_sb[b + 1])]
            best = sorted(cand)[:min(3, len(cand))]
            expect = sorted(c for _, c in best)
            assert got[i, :len(expect)].tolist() == expect
            assert (got[i, len(expect):] == -1).all()


def test_line_of_blocks_nearest_by_construction():
    # 10 blocks of 4 points each along x, block c centred at x = 10 c: a
    # point at x = 10 c + 1 has nearest blocks c, c + 1, c - 1 (distances 1,
    # 9, 11), so topk = 2 picks {c, c + 1} and topk = 3 adds c - 1.
    xs = np.concatenate([10.0 * c + np.array([-1.5, -0.5, 0.5, 1.5]) for c in range(10)])
    pts = np.stack([xs, np.zeros_like(xs), np.zeros_like(xs)], 1).astype(np.float32)
    cu = np.arange(0, 41, 4)
    probe = np.array([[10.0 * c + 1.0, 0.0, 0.0] for c in range(1, 9)], dtype=np.float32)
    allp = np.concatenate([pts, probe])
    cu_all = np.concatenate([cu, [40 + 8]])  # probes form an 11th block (ignored by the check)
    got = nearest_blocks_ref(allp, cu_all, np.array([0, 10]), np.array([0, 48]), 3)
    for j, c in enumerate(range(1, 9)):
        assert got[40 + j].tolist() == sorted([c - 1, c, c + 1])


def test_topk_at_least_blocks_and_ties_lowest_id():
    pts = np.zeros((6, 3), dtype=np.float32)        # every centroid at the origin
    cu = np.array([0, 2, 4, 6])
    got = nearest_blocks_ref(pts, cu, np.array([0, 3]), np.array([0, 6]), 2)
    assert (got == [0, 1]).all()                     # all distances tie -> lowest ids
    got5 = nearest_blocks_ref(pts, cu, np.array([0, 3]), np.array([0, 6]), 5)
    assert (got5[:, :3] == [0, 1, 2]).all() and (got5[:, 3:] == -1).all()
