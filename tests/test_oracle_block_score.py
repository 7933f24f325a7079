"""Pins of the learned-selection oracle (oracle/block_score.py): brute force,
reductions to known rankings, constructed cases that fail if a term of the
score is dropped or mis-scaled, and the compressed-attention restatement
against torch's own attention routines."""

import math

import numpy as np
import torch

from oracle.block_score import (LOG2E_REF, compressed_attention_ref, get_block_score_ref,
                                topk_rows_ref)


def _brute(q, ck, lse, topk, cu_q, cu_c, sm_scale):
    """Pure-Python restatement with math.pow and sorted()."""
    nq, hq, d = q.shape
    hkv = ck.shape[1]
    g_n = hq // hkv
    out = np.full((hkv, nq, topk), -1, dtype=np.int32)
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_c[b], cu_c[b + 1]
        nc = ke - ks
        if nc <= 0:
            continue
        for h in range(hkv):
            for i in range(qs, qe):
                sc = []
                for c in range(nc):
                    tot = 0.0
                    for g in range(g_n):
                        hh = h * g_n + g
                        dot = sum(float(q[i, hh, x]) * float(ck[ks + c, h, x]) for x in range(d))
                        tot += math.pow(2.0, dot * sm_scale * LOG2E_REF
                                        - float(lse[hh, i]) * LOG2E_REF)
                    sc.append((-tot, c))
                best = sorted(sc)[:min(topk, nc)]
                out[h, i, :len(best)] = sorted(c for _, c in best)
    return out


def _rand_case(seed, nq_per=(5, 7), nc_per=(6, 9), hq=4, hkv=2, d=8):
    rng = np.random.default_rng(seed)
    cu_q = [0]
    cu_c = [0]
    for a, b in zip(nq_per, nc_per):
        cu_q.append(cu_q[-1] + a)
        cu_c.append(cu_c[-1] + b)
    q = rng.standard_normal((cu_q[-1], hq, d)).astype(np.float32)
    ck = rng.standard_normal((cu_c[-1], hkv, d)).astype(np.float32)
    lse = rng.uniform(1.0, 4.0, size=(hq, cu_q[-1])).astype(np.float32)
    return q, ck, lse, cu_q, cu_c


def test_matches_brute_force():
    for seed in range(3):
        q, ck, lse, cu_q, cu_c = _rand_case(seed)
        got = get_block_score_ref(q, ck, lse, 4, cu_q, cu_c, 0.35)
        np.testing.assert_array_equal(got, _brute(q, ck, lse, 4, cu_q, cu_c, 0.35))


def test_single_head_group_is_top_k_by_dot_product():
    q, ck, lse, cu_q, cu_c = _rand_case(5, hq=2, hkv=2)
    got = get_block_score_ref(q, ck, lse, 3, cu_q, cu_c, None)
    for b in range(2):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_c[b], cu_c[b + 1]
        for h in range(2):
            dots = q[qs:qe, h].astype(np.float64) @ ck[ks:ke, h].astype(np.float64).T
            expect = topk_rows_ref(dots, 3)
            np.testing.assert_array_equal(got[h, qs:qe, :3], expect)


def test_group_sum_picks_a_block_no_single_head_ranks_first():
    # Two query heads share one kv head, 3 blocks, d = 2.  Head 0's logits
    # are (10, 0, 7), head 1's are (0, 10, 7): alone they rank block 0 and
    # block 1 first.  With x = 2^(0.05 * 1.44269504) the group sums are
    # x^10 + 1 for blocks 0 and 1 and 2 x^7 for block 2, and 2 x^7 is larger,
    # so topk = 1 must pick block 2.
    ck = np.array([[[10.0, 0.0]], [[0.0, 10.0]], [[7.0, 7.0]]], dtype=np.float32)
    q = np.array([[[1.0, 0.0], [0.0, 1.0]]], dtype=np.float32)
    lse = np.zeros((2, 1), dtype=np.float32)
    x = 2.0 ** (0.05 * LOG2E_REF)
    assert 2 * x ** 7 > x ** 10 + 1
    assert get_block_score_ref(q, ck, lse, 1, [0, 1], [0, 3], 0.05)[0, 0, 0] == 2
    # each head alone (one query head per kv head) ranks its own block first
    for h, best in ((0, 0), (1, 1)):
        q1 = q[:, h:h + 1]
        l1 = lse[h:h + 1]
        assert get_block_score_ref(q1, ck, l1, 1, [0, 1], [0, 3], 0.05)[0, 0, 0] == best


def test_lse_term_and_its_units_change_the_ranking():
    # Two heads, two blocks.  Head 0 prefers block 0, head 1 block 1 by a
    # larger margin; head 1's lse is large, which shrinks its weight.
    ck = np.array([[[1.0]], [[-1.0]]], dtype=np.float32)
    q = np.array([[[2.0], [-3.0]]], dtype=np.float32)
    def pick(lse1, scale=1.0):
        lse = np.array([[0.0], [lse1]], dtype=np.float32)
        return int(get_block_score_ref(q, ck, lse, 1, [0, 1], [0, 2], scale)[0, 0, 0])
    assert pick(0.0) == 1            # without the lse shift head 1 wins
    assert pick(3.0) == 0            # the natural-log lse of head 1 flips it
    # With c = 1.44269504 block 1 wins iff 2^-L (e^3 - e^-3) > e^2 - e^-2,
    # i.e. L < 1.466.  lse = 1.2 in natural-log units is L = 1.2 c = 1.73
    # (block 0); misread as log2 units it would be L = 1.2 (block 1).
    def sums(l2):
        s0 = 2 ** (2 * LOG2E_REF) + 2 ** (-3 * LOG2E_REF - l2)
        s1 = 2 ** (-2 * LOG2E_REF) + 2 ** (3 * LOG2E_REF - l2)
        return s0, s1
    nat0, nat1 = sums(1.2 * LOG2E_REF)
    mis0, mis1 = sums(1.2)
    assert nat0 > nat1 and mis1 > mis0
    assert pick(1.2) == 0


def test_topk_at_least_blocks_and_padding():
    q, ck, lse, cu_q, cu_c = _rand_case(7, nq_per=(3, 4), nc_per=(2, 5))
    got = get_block_score_ref(q, ck, lse, 6, cu_q, cu_c, None)
    np.testing.assert_array_equal(got[:, 0:3, :2], np.broadcast_to([0, 1], (2, 3, 2)))
    assert (got[:, 0:3, 2:] == -1).all()
    np.testing.assert_array_equal(got[:, 3:7, :5], np.broadcast_to(np.arange(5), (2, 4, 5)))
    assert (got[:, 3:7, 5:] == -1).all()


def test_empty_batch_element_and_batch_local_ids():
    q, ck, lse, cu_q, cu_c = _rand_case(9, nq_per=(3, 4, 2), nc_per=(4, 0, 5))
    got = get_block_score_ref(q, ck, lse, 2, cu_q, cu_c, None)
    assert (got[:, 3:7] == -1).all()          # no compressed keys
    assert got[:, 7:9].max() < 5 and got[:, 7:9].min() >= 0  # local ids of element 2


def test_ties_take_the_lowest_index_and_nan_ranks_last():
    s = np.array([[1.0, 3.0, 3.0, np.nan, 3.0, 0.5]])
    np.testing.assert_array_equal(topk_rows_ref(s, 2), [[1, 2]])
    np.testing.assert_array_equal(topk_rows_ref(s, 5), [[0, 1, 2, 4, 5]])


def test_compressed_attention_matches_sdpa_and_logsumexp():
    g = torch.Generator().manual_seed(3)
    cu_q = torch.tensor([0, 9, 20], dtype=torch.int32)
    cu_c = torch.tensor([0, 5, 12], dtype=torch.int32)
    q = torch.randn(20, 4, 16, generator=g)
    ck = torch.randn(12, 2, 16, generator=g)
    cv = torch.randn(12, 2, 16, generator=g)
    o, lse = compressed_attention_ref(q, ck, cv, cu_q, cu_c, 0.3)
    for b in range(2):
        qs, qe, ks, ke = cu_q[b].item(), cu_q[b + 1].item(), cu_c[b].item(), cu_c[b + 1].item()
        qb = q[qs:qe].permute(1, 0, 2)
        kb = ck[ks:ke].permute(1, 0, 2).repeat_interleave(2, 0)
        vb = cv[ks:ke].permute(1, 0, 2).repeat_interleave(2, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, scale=0.3)
        torch.testing.assert_close(o[qs:qe], ref.permute(1, 0, 2), rtol=1e-5, atol=1e-5)
        logits = torch.einsum("hld,hcd->hlc", qb, kb) * 0.3
        torch.testing.assert_close(lse[:, qs:qe], torch.logsumexp(logits, -1),
                                   rtol=1e-5, atol=1e-5)
