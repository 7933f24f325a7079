"""CPU pins of the per-query-block selection oracle (oracle/select.py).

Pinned by a brute force that uses only Python floats (exact products of
fp32 values summed in double precision in the contract's order) and Python's
own sort, by constructed inputs with a known ranking, and by the special
cases the rule fixes: topk >= blocks selects everything, identical pooled
keys tie to the lowest ids, forced blocks are always present.  Output layout
and -1 padding follow sparse/ops/block_score.py:61-63, 94-96.
"""

import numpy as np
import pytest

from oracle.pool import block_mean_pool_ref
from oracle.select import block_scores_ref, expand_per_token, select_blocks_ref


def _brute(pq, pk, cu_sb, topk, forced, force_self):
    nb, hq, d = pq.shape
    hkv = pk.shape[1]
    g = hq // hkv
    out = np.full((hkv, nb, topk), -1, dtype=np.int32)
    for e in range(len(cu_sb) - 1):
        cs, ce = int(cu_sb[e]), int(cu_sb[e + 1])
        nbb = ce - cs
        kmax = min(topk, nbb)
        for h in range(hkv):
            for b in range(nbb):
                scores = []
                for c in range(nbb):
                    s = 0.0
                    for gg in range(g):
                        for dd in range(d):
                            s += float(pq[cs + b, h * g + gg, dd]) * float(pk[cs + c, h, dd])
                    scores.append(s)
                chosen = []
                for f in ([b] if force_self else []) + list(forced):
                    if 0 <= f < nbb and f not in chosen and len(chosen) < kmax:
                        chosen.append(f)
                rest = sorted((c for c in range(nbb) if c not in chosen),
                              key=lambda c: (-scores[c], c))
                chosen += rest[: kmax - len(chosen)]
                out[h, cs + b, :kmax] = sorted(chosen)
    return out


@pytest.mark.parametrize("seed,hq,hkv,topk,forced", [
    (0, 2, 2, 3, []), (1, 4, 2, 4, [5, 1]), (2, 3, 1, 6, [0]), (3, 2, 2, 20, [])])
def test_brute_force_tiny(seed, hq, hkv, topk, forced):
    rng = np.random.default_rng(seed)
    nb, d = 9, 8
    pq = rng.standard_normal((nb, hq, d)).astype(np.float32)
    pk = rng.standard_normal((nb, hkv, d)).astype(np.float32)
    cu_sb = np.array([0, 4, nb])          # two batch elements
    out = select_blocks_ref(pq, pk, cu_sb, topk, forced, True)
    np.testing.assert_array_equal(out, _brute(pq, pk, cu_sb, topk, forced, True))


def test_no_self_forcing():
    rng = np.random.default_rng(7)
    pq = rng.standard_normal((6, 2, 4)).astype(np.float32)
    pk = rng.standard_normal((6, 2, 4)).astype(np.float32)
    out = select_blocks_ref(pq, pk, np.array([0, 6]), 2, [], False)
    np.testing.assert_array_equal(out, _brute(pq, pk, [0, 6], 2, [], False))


def test_known_ranking():
    # pk[c] = c * e0 and pq = e0 -> score(b, c) = c: top-3 are the last ids.
    nb = 8
    pk = np.zeros((nb, 1, 4), dtype=np.float32)
    pk[:, 0, 0] = np.arange(nb)
    pq = np.zeros((nb, 1, 4), dtype=np.float32)
    pq[:, 0, 0] = 1.0
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 3, [], False)
    assert (out[0] == np.array([5, 6, 7])).all()
    # with self forced, block 0 keeps itself plus the two best
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 3, [], True)
    assert out[0, 0].tolist() == [0, 6, 7]
    assert out[0, 7].tolist() == [5, 6, 7]


def test_ties_lowest_index_and_nan():
    nb = 6
    pq = np.ones((nb, 1, 2), dtype=np.float32)
    pk = np.ones((nb, 1, 2), dtype=np.float32)
    pk[2] = np.nan                          # NaN scores rank lowest
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 3, [], False)
    assert (out[0] == np.array([0, 1, 3])).all()


def test_topk_ge_blocks_and_forced_present():
    rng = np.random.default_rng(3)
    nb = 7
    pq = rng.standard_normal((nb, 2, 4)).astype(np.float32)
    pk = rng.standard_normal((nb, 2, 4)).astype(np.float32)
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 10, [], True)
    assert (out[..., :nb] == np.arange(nb)).all() and (out[..., nb:] == -1).all()
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 3, [4, 4, 99, 2], True)
    for b in range(nb):
        row = set(out[0, b].tolist())
        assert b in row and 4 in row and (2 in row or b in (2, 4) or len(row) == 3)


def test_forced_truncates_to_topk():
    pq = np.ones((5, 1, 2), dtype=np.float32)
    pk = np.ones((5, 1, 2), dtype=np.float32)
    out = select_blocks_ref(pq, pk, np.array([0, 5]), 2, [4, 3, 2], True)
    assert out[0, 0].tolist() == [0, 4]       # self, then the first forced id


def test_fp64_order_is_sequential_over_heads_then_dims():
    rng = np.random.default_rng(11)
    pq = rng.standard_normal((5, 4, 16)).astype(np.float32)
    pk = rng.standard_normal((5, 2, 16)).astype(np.float32)
    s = block_scores_ref(pq, pk, 1)
    for b in range(5):
        for c in range(5):
            acc = 0.0
            for g in range(2):
                for dd in range(16):
                    acc += float(pq[b, 2 + g, dd]) * float(pk[c, 1, dd])
            assert s[b, c] == acc


def test_expand_per_token_layout():
    compact = np.array([[[1, -1], [0, 1]]], dtype=np.int32)
    out = expand_per_token(compact, np.array([0, 3, 5]), 5)
    assert out.shape == (1, 5, 2)
    assert out[0, :3].tolist() == [[1, -1]] * 3 and out[0, 3:].tolist() == [[0, 1]] * 2


def test_selection_from_pooled_tokens_end_to_end():
    # pooled means from the pool oracle feed the selection, as select_blocks does
    rng = np.random.default_rng(5)
    sizes = rng.integers(3, 20, size=10)
    cu = np.concatenate([[0], np.cumsum(sizes)])
    n = int(cu[-1])
    q = rng.standard_normal((n, 2 * 4)).astype(np.float32)
    k = rng.standard_normal((n, 2 * 4)).astype(np.float32)
    pq = block_mean_pool_ref(q, cu).reshape(-1, 2, 4)
    pk = block_mean_pool_ref(k, cu).reshape(-1, 2, 4)
    out = select_blocks_ref(pq, pk, np.array([0, 10]), 4, [9], True)
    np.testing.assert_array_equal(out, _brute(pq, pk, [0, 10], 4, [9], True))


@pytest.mark.parametrize("seed,topk,forced", [(0, 3, []), (1, 5, [2]), (2, 4, [7, 0])])
def test_brute_force_many_ties(seed, topk, forced):
    # Small-integer pooled values make many scores equal, so the top-k cut
    # falls inside groups of tied scores (lowest ids must win) and forced ids
    # can sit inside or outside a tied group.
    rng = np.random.default_rng(100 + seed)
    nb, d = 11, 3
    pq = rng.integers(-1, 2, size=(nb, 2, d)).astype(np.float32)
    pk = rng.integers(-1, 2, size=(nb, 1, d)).astype(np.float32)
    cu_sb = np.array([0, nb])
    out = select_blocks_ref(pq, pk, cu_sb, topk, forced, True)
    np.testing.assert_array_equal(out, _brute(pq, pk, cu_sb, topk, forced, True))
    out = select_blocks_ref(pq, pk, cu_sb, topk, forced, False)
    np.testing.assert_array_equal(out, _brute(pq, pk, cu_sb, topk, forced, False))


def test_brute_force_nan_scores():
    # NaN pooled keys rank below every finite score; among themselves by id:
    # 5 finite ids fill five of six slots, the sixth goes to NaN id 1.
    rng = np.random.default_rng(5)
    nb = 8
    pq = rng.standard_normal((nb, 1, 4)).astype(np.float32)
    pk = rng.standard_normal((nb, 1, 4)).astype(np.float32)
    pk[[1, 4, 6], 0, 2] = np.nan
    out = select_blocks_ref(pq, pk, np.array([0, nb]), 6, [], False)
    for b in range(nb):
        assert out[0, b].tolist() == [0, 1, 2, 3, 5, 7]
