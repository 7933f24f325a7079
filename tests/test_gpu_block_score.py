"""GPU parity of the learned-selection path: compressed attention (output,
natural-log LSE and gradients) against the fp32 CPU oracle, and
get_block_score against the float64 oracle of sparse/ops/block_score.py:16-98.

The GPU scores are fp32 (bf16 x bf16 products summed by the MFMA, hardware
exp2), the oracle's float64, so a row may choose differently only between
keys whose oracle scores lie within a relative 1e-4 of the row's
real_topk-th best score (near-ties); every other row must match exactly, and
every row must be ascending, -1 padded and of length min(topk, keys)."""

import numpy as np
import pytest
import torch

import sparse.ops as ops
from oracle.block_score import compressed_attention_ref, get_block_score_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL_MAX, TOL_MEAN = 2e-2, 2e-3   # attention outputs / gradients vs fp32
NEAR_TIE = 1e-4


def _case(seed, q_lens, c_lens, hq, hkv, d, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    cu_c = torch.tensor(np.concatenate([[0], np.cumsum(c_lens)]), dtype=torch.int32)
    q = (0.5 * torch.randn(int(cu_q[-1]), hq, d, generator=g)).to(dtype)
    ck = (0.5 * torch.randn(int(cu_c[-1]), hkv, d, generator=g)).to(dtype)
    cv = (0.5 * torch.randn(int(cu_c[-1]), hkv, d, generator=g)).to(dtype)
    return q, ck, cv, cu_q, cu_c


def _check_selection(got, ref, scores, topk, cu_q, cu_c):
    """Exact match except between near-tied keys; layout rules everywhere."""
    got = got.cpu().numpy()
    hkv, nq, _ = got.shape
    mismatched = 0
    for b in range(cu_q.numel() - 1):
        qs, qe = int(cu_q[b]), int(cu_q[b + 1])
        nc = int(cu_c[b + 1] - cu_c[b])
        kk = min(topk, max(nc, 0))
        rows = got[:, qs:qe]
        assert (rows[..., kk:] == -1).all()
        if kk == 0:
            continue
        assert (np.diff(rows[..., :kk], axis=-1) > 0).all()   # ascending, distinct
        assert rows[..., :kk].min() >= 0 and rows[..., :kk].max() < nc
    for h, qs, qe, s in scores:
        kk = min(topk, s.shape[1])
        for r in range(qe - qs):
            a = set(got[h, qs + r, :kk].tolist())
            e = set(ref[h, qs + r, :kk].tolist())
            if a == e:
                continue
            mismatched += 1
            kth = np.sort(s[r])[::-1][kk - 1]
            for c in a ^ e:
                assert abs(s[r, c] - kth) <= NEAR_TIE * max(abs(kth), 1e-30), \
                    (h, qs + r, c, s[r, c], kth)
    return mismatched


@pytest.mark.parametrize("hq,hkv,d,topk", [
    (4, 4, 64, 16),      # MHA, the BASELINE head_dim
    (8, 4, 64, 24),      # G = 2, topk not a power of two
    (8, 2, 64, 32),      # G = 4
    (32, 2, 32, 16),     # the product's GQA shape: G = 16, D = 32
    (2, 2, 128, 8),      # D = 128
    (4, 4, 64, 64),      # largest single-launch topk
    (4, 4, 64, 72),      # two launches: the product's topk_multiimage * 18 images
    (8, 2, 64, 65),      # two launches, the first selecting 63
    (4, 4, 64, 128),     # largest topk
])
def test_block_score_matches_oracle(hq, hkv, d, topk):
    q_lens, c_lens = [157, 300, 45], [90, 61, 40]
    if topk > 64:
        c_lens = [150, 61, 200]          # one element with fewer keys than topk
    q, ck, cv, cu_q, cu_c = _case(1, q_lens, c_lens, hq, hkv, d)
    _, lse = compressed_attention_ref(q, ck, cv, cu_q, cu_c)      # natural log
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), topk, cu_q.to(DEV),
                              cu_c.to(DEV), None, None)
    ref, scores = get_block_score_ref(q.float().numpy(), ck.float().numpy(), lse.numpy(),
                                      topk, cu_q.numpy(), cu_c.numpy(), return_scores=True)
    mism = _check_selection(got, ref, scores, topk, cu_q, cu_c)
    assert mism <= 0.01 * q.shape[0] * hkv + 2


def test_block_score_fewer_keys_than_topk_and_empty_element():
    q, ck, cv, cu_q, cu_c = _case(2, [33, 70, 31], [5, 0, 9], 4, 2, 64)
    lse = torch.randn(4, q.shape[0]).abs() + 1.0
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), 8, cu_q.to(DEV),
                              cu_c.to(DEV), None, None, 0.2)
    ref, scores = get_block_score_ref(q.float().numpy(), ck.float().numpy(), lse.numpy(), 8,
                                      cu_q.numpy(), cu_c.numpy(), 0.2, return_scores=True)
    _check_selection(got, ref, scores, 8, cu_q, cu_c)
    g = got.cpu()
    assert (g[:, 33:103] == -1).all()                 # no compressed keys
    assert (g[:, :33, :5] == torch.arange(5)).all()   # 5 keys < topk: all chosen


def test_block_score_ties_take_the_lowest_id():
    # every compressed key identical -> all scores tie -> ids 0..topk-1
    q, ck, cv, cu_q, cu_c = _case(3, [64], [40], 2, 2, 64)
    ck = ck[:1].expand(40, 2, 64).contiguous()
    lse = torch.zeros(2, 64)
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), 8, cu_q.to(DEV),
                              cu_c.to(DEV), None, None)
    assert (got.cpu() == torch.arange(8)).all()


def test_compressed_attention_forward_backward():
    q, ck, cv, cu_q, cu_c = _case(4, [200, 77], [60, 23], 8, 4, 64)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(9))
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, ck, cv))
    out, lse = ops.compressed_attention(qd, kd, vd, cu_q.to(DEV), cu_c.to(DEV))
    out.backward(do.to(DEV).to(q.dtype))
    qf, kf, vf = (t.float().requires_grad_() for t in (q, ck, cv))
    ref, ref_lse = compressed_attention_ref(qf, kf, vf, cu_q, cu_c)
    ref.backward(do)
    for name, a, b in (("out", out, ref), ("dq", qd.grad, qf.grad), ("dk", kd.grad, kf.grad),
                       ("dv", vd.grad, vf.grad)):
        err = (a.detach().float().cpu() - b.detach()).abs()
        assert float(err.max()) <= TOL_MAX and float(err.mean()) <= TOL_MEAN, name
    torch.testing.assert_close(lse.cpu(), ref_lse.detach(), rtol=0, atol=1e-2)


def test_learned_selection_path_end_to_end():
    """compressed attention -> LSE -> get_block_score -> selected attention,
    the composition of SpatialSparseAttentionMid.forward
    (spatial_sparse_attention.py:121-184) when block_topk is None."""
    from lsrm_hip import workloads as W
    from oracle.attention import sel_attn_ref
    from oracle.pool import block_mean_pool_ref
    w = W.config(2, n=4096, heads=4)
    q, k, v = W.tensors(w, "cpu")
    cu_blk = w.cu_block_tokens
    ck = torch.from_numpy(block_mean_pool_ref(k.float().reshape(w.n, -1).numpy(),
                                              cu_blk.numpy())).reshape(-1, w.hkv, w.d)
    cv = torch.from_numpy(block_mean_pool_ref(v.float().reshape(w.n, -1).numpy(),
                                              cu_blk.numpy())).reshape(-1, w.hkv, w.d)
    ck, cv = ck.to(q.dtype), cv.to(q.dtype)
    cu_sb = w.cu_seqblocks
    _, lse = ops.compressed_attention(q.to(DEV), ck.to(DEV), cv.to(DEV), w.cu_seqlens.to(DEV),
                                      cu_sb.to(DEV))
    topk_idx = ops.get_block_score(q.to(DEV), ck.to(DEV), lse, 8, w.cu_seqlens.to(DEV),
                                   cu_sb.to(DEV), None, None)
    out = ops.spatial_selection_attention(q.to(DEV), k.to(DEV), v.to(DEV), topk_idx,
                                          cu_sb.to(DEV), cu_blk.to(DEV), w.cu_seqlens.to(DEV),
                                          w.cu_seqlens.to(DEV), None, None)
    ref, _ = sel_attn_ref(q.float(), k.float(), v.float(), topk_idx.cpu(), cu_sb, cu_blk,
                          w.cu_seqlens, w.scale)
    err = (out.float().cpu() - ref).abs()
    assert float(err.max()) <= TOL_MAX and float(err.mean()) <= TOL_MEAN
    # the selection itself against the oracle, from the same (GPU) lse
    ref_sel, scores = get_block_score_ref(q.float().numpy(), ck.float().numpy(),
                                          lse.cpu().numpy(), 8, w.cu_seqlens.numpy(),
                                          cu_sb.numpy(), return_scores=True)
    _check_selection(topk_idx, ref_sel, scores, 8, w.cu_seqlens, cu_sb)


@pytest.mark.parametrize("hq,hkv,d,topk", [
    (4, 4, 64, 16),      # MHA, the BASELINE head_dim
    (8, 4, 64, 24),      # G = 2, topk not a power of two
    (8, 2, 64, 32),      # G = 4
    (2, 2, 128, 8),      # D = 128
])
def test_block_score_many_keys(hq, hkv, d, topk):
    """Elements with at least 8 topk keys take the two-pass selection (a
    lower bound on the row's topk-th score from block maxima, then a
    filtered buffer); the last element stays on the one-pass merge."""
    q_lens, c_lens = [157, 300, 45, 70], [462, 300, 1030, 100]
    q, ck, cv, cu_q, cu_c = _case(4, q_lens, c_lens, hq, hkv, d)
    _, lse = compressed_attention_ref(q, ck, cv, cu_q, cu_c)
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), topk, cu_q.to(DEV),
                              cu_c.to(DEV), None, None)
    ref, scores = get_block_score_ref(q.float().numpy(), ck.float().numpy(), lse.numpy(),
                                      topk, cu_q.numpy(), cu_c.numpy(), return_scores=True)
    mism = _check_selection(got, ref, scores, topk, cu_q, cu_c)
    assert mism <= 0.01 * q.shape[0] * hkv + 2


def test_block_score_many_keys_all_tied():
    # 300 identical compressed keys: every key reaches the two-pass bound, the
    # buffer fills and is merged repeatedly; ties still take the lowest ids
    q, ck, cv, cu_q, cu_c = _case(5, [96], [300], 2, 2, 64)
    ck = ck[:1].expand(300, 2, 64).contiguous()
    lse = torch.zeros(2, 96)
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), 16, cu_q.to(DEV),
                              cu_c.to(DEV), None, None)
    assert (got.cpu() == torch.arange(16)).all()


def test_block_score_tokens_outside_every_element():
    # cu_seqlens_q starts at 10 and ends at 100 of 130 tokens: rows 0-9 and
    # 100-129 belong to no batch element and come back as -1 rows
    q, ck, cv, cu_q, cu_c = _case(6, [130], [70], 4, 2, 64)
    cu_q = torch.tensor([10, 60, 100], dtype=torch.int32)
    cu_c = torch.tensor([0, 40, 70], dtype=torch.int32)
    lse = torch.randn(4, 130).abs() + 1.0
    got = ops.get_block_score(q.to(DEV), ck.to(DEV), lse.to(DEV), 8, cu_q.to(DEV),
                              cu_c.to(DEV), None, None).cpu()
    assert (got[:, :10] == -1).all() and (got[:, 100:] == -1).all()
    ref, scores = get_block_score_ref(q.float().numpy(), ck.float().numpy(), lse.numpy(), 8,
                                      cu_q.numpy(), cu_c.numpy(), return_scores=True)
    _check_selection(got, ref, scores, 8, cu_q, cu_c)
