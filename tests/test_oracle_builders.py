"""Pins of the block-metadata builder oracle (oracle/builders.py)."""

import itertools
from collections import Counter

import numpy as np

from oracle.builders import (block_sort_keys_ref, block_sort_perm_ref,
                             compute_block_separation_ref)


def test_separation_matches_counting_brute_force():
    rng = np.random.default_rng(0)
    coords = np.concatenate([np.sort(rng.integers(0, 3, 300))[:, None],
                             rng.integers(0, 16, (300, 3))], axis=1)
    cu_sb, cu_blk = compute_block_separation_ref(coords, 3, [4, 4, 4], 3, [16, 16, 16])
    pos = 0
    for b in range(3):
        cnt = Counter((x // 4) * 16 + (y // 4) * 4 + z // 4
                      for bb, x, y, z in coords.tolist() if bb == b)
        sizes = [cnt[k] for k in sorted(cnt)]
        assert cu_sb[b + 1] - cu_sb[b] == len(sizes)
        got = np.diff(cu_blk[cu_sb[b]:cu_sb[b + 1] + 1]).tolist()
        assert got == sizes
        pos += len(sizes)
    assert cu_blk[-1] == 300


def test_separation_full_grid_and_outside_points():
    cells = np.array(list(itertools.product(range(8), range(8))))
    coords = np.concatenate([np.zeros((64, 1), np.int64), cells], axis=1)
    extra = np.array([[0, 8, 0], [0, -1, 3], [1, 0, 0]])   # outside grid / batch
    cu_sb, cu_blk = compute_block_separation_ref(np.concatenate([coords, extra]), 2, [2, 4], 1,
                                                 [8, 8])
    assert cu_sb.tolist() == [0, 8]                    # 4 x 2 blocks
    assert np.diff(cu_blk).tolist() == [8] * 8         # 2 x 4 tokens each


def test_volume_keys_order_blocks_before_positions():
    # block (0,0,1) precedes block (0,1,0); inside a block, row-major positions
    coords = np.array([[0, 0, 4, 0], [0, 0, 0, 4], [0, 3, 3, 3], [0, 0, 0, 1], [1, 0, 0, 0]])
    keys = block_sort_keys_ref(coords, 0, 4, (8,))
    assert block_sort_perm_ref(coords, 0, 4, (8,)).tolist() == [3, 2, 1, 0, 4]
    assert len(set(keys.tolist())) == 5


def test_image_keys_order_images_then_blocks():
    coords = np.array([[0, 1, 0, 0], [0, 0, 2, 2], [0, 0, 0, 3], [0, 0, 1, 0]])
    perm = block_sort_perm_ref(coords, 1, 2, (2, 4))
    # image 0: block (0,1) holds (0,3); block (0,0) holds (1,0); block (1,1) holds (2,2)
    assert perm.tolist() == [3, 2, 1, 0]
