"""CPU pins of the block mean pooling oracle (oracle/pool.py).

The oracle fixes the summation order of torch.segment_reduce(mean)
(reference: sparse/module/spatial_sparse_attention.py:27-37).  It is pinned
here by (1) the reference's own library call within fp32 rounding, (2) exact
rational arithmetic on integer-valued inputs, where every partial sum is
representable and the only rounding is the final divide, and (3) hand-built
cancellation cases whose result is different under a plain sequential sum,
a pairwise sum, or pieces cut anywhere but at multiples of 64.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle.pool import CHUNK, block_mean_pool_ref


def _cu(sizes):
    return np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)


def test_matches_segment_reduce_within_fp32():
    rng = np.random.default_rng(0)
    sizes = rng.integers(1, 300, size=40)
    x = rng.standard_normal((int(sizes.sum()), 33)).astype(np.float32)
    out = block_mean_pool_ref(x, _cu(sizes))
    ref = torch.segment_reduce(torch.from_numpy(x).double(), "mean",
                               lengths=torch.from_numpy(sizes), axis=0).numpy()
    np.testing.assert_allclose(out, ref, rtol=2e-6, atol=2e-6)


def test_integer_inputs_exact_mean():
    # |x| <= 1000 and blocks <= 700 rows: every partial sum is an integer
    # below 2^24, so the only rounding is the final quotient.
    rng = np.random.default_rng(1)
    sizes = rng.integers(1, 700, size=25)
    x = rng.integers(-1000, 1001, size=(int(sizes.sum()), 5)).astype(np.float32)
    cu = _cu(sizes)
    out = block_mean_pool_ref(x, cu)
    for b in range(len(sizes)):
        for c in range(5):
            exact = Fraction(int(x[cu[b]:cu[b + 1], c].astype(np.int64).sum()), int(sizes[b]))
            assert out[b, c] == np.float32(float(exact)), (b, c)


def test_piece_order_cancellation():
    # Block covers rows 62..65, crossing the row-64 piece boundary.
    # pieces: [1 + 1e8] = 1e8 and [-1e8 + 1] = -1e8 -> total 0 -> mean 0.
    # A plain sequential sum gives ((1 + 1e8) - 1e8) + 1 = 1 -> mean 0.25.
    x = np.zeros((70, 1), dtype=np.float32)
    x[62:66, 0] = [1.0, 1e8, -1e8, 1.0]
    out = block_mean_pool_ref(x, np.array([0, 62, 66, 70]))
    assert out[1, 0] == np.float32(0.0)
    seq = np.float32(0.0)
    for r in range(62, 66):
        seq = np.float32(seq + x[r, 0])
    assert seq / np.float32(4) == np.float32(0.25)  # the sum this contract excludes


def test_piece_cut_is_global_row_index():
    # Same four values at rows 60..63 lie in ONE piece: sequential inside it.
    x = np.zeros((70, 1), dtype=np.float32)
    x[60:64, 0] = [1.0, 1e8, -1e8, 1.0]
    out = block_mean_pool_ref(x, np.array([0, 60, 64, 70]))
    assert out[1, 0] == np.float32(0.25)


def test_pairwise_sum_excluded():
    # 64 rows in one piece: sequential fp32 accumulation of 2^24 + many 1.0
    # drops every 1.0; a pairwise sum would keep them.
    x = np.ones((64, 1), dtype=np.float32)
    x[0, 0] = 2.0 ** 24
    out = block_mean_pool_ref(x, np.array([0, 64]))
    assert out[0, 0] == np.float32(2.0 ** 24) / np.float32(64)
    pairwise = np.float32(x[:, 0].astype(np.float64).sum() / 64)
    assert pairwise != out[0, 0]


def test_empty_block_nan_and_bounds():
    x = np.ones((10, 3), dtype=np.float32)
    out = block_mean_pool_ref(x, np.array([0, 4, 4, 10]))
    assert np.isnan(out[1]).all()
    assert (out[0] == 1).all() and (out[2] == 1).all()


@pytest.mark.parametrize("start", [0, 63, 64, 65, 127])
def test_chunk_boundaries_single_block(start):
    rng = np.random.default_rng(start)
    n = start + 3 * CHUNK + 7
    x = rng.standard_normal((n, 4)).astype(np.float32)
    out = block_mean_pool_ref(x, np.array([0, start, n]) if start else np.array([0, n]))
    b = 1 if start else 0
    # reassemble with explicit piece sums
    acc = np.zeros(4, dtype=np.float32)
    r = start
    while r < n:
        e = min(n, (r // CHUNK + 1) * CHUNK)
        piece = np.float32(0) + np.zeros(4, dtype=np.float32)
        for t in range(r, e):
            piece = (piece + x[t]).astype(np.float32)
        acc = (acc + piece).astype(np.float32)
        r = e
    np.testing.assert_array_equal(out[b], acc / np.float32(n - start))
