"""CPU pins of the selected-attention oracle (oracle/attention.py).

The oracle restates forward_kernel_varblock
(sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:55-247); these
tests pin it against routines it does not share code with:
  * topk = every block  ->  full softmax attention
    (torch.nn.functional.scaled_dot_product_attention);
  * topk = own block    ->  block-diagonal attention;
  * a repeated block    ->  SDPA over the key list with that block's keys
    listed twice;
  * lse in log2 units   ->  the softmax weights exp2(scale*log2e*q.k - lse)
    sum to one;
  * out rows are convex combinations of the attended V rows;
  * the backward (kvcentric:262-478, 687-923) -> fp64 finite differences
    (torch.autograd.gradcheck);
  * batch-local ids, -1 padding, out-of-range ids and empty rows.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.attention import LOG2E, attended_pairs, sel_attn_bwd_ref, sel_attn_ref


def _problem(n=96, hq=4, hkv=2, d=16, sizes=(10, 30, 5, 21, 30), seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, hq, d, generator=g, dtype=dtype)
    k = torch.randn(n, hkv, d, generator=g, dtype=dtype)
    v = torch.randn(n, hkv, d, generator=g, dtype=dtype)
    cu = torch.tensor([0] + list(np.cumsum(sizes)), dtype=torch.int32)
    assert int(cu[-1]) == n
    return q, k, v, cu


def _sdpa(q, k, v, g):
    # q [L, Hq, D], k/v [S, Hkv, D] -> [L, Hq, D]
    kk = k.repeat_interleave(g, 1).transpose(0, 1)
    vv = v.repeat_interleave(g, 1).transpose(0, 1)
    return F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv).transpose(0, 1)


def test_all_blocks_equals_full_attention():
    q, k, v, cu = _problem()
    nb = cu.numel() - 1
    topk = torch.arange(nb, dtype=torch.int32).view(1, 1, nb).expand(2, 96, nb).contiguous()
    o, lse = sel_attn_ref(q, k, v, topk, torch.tensor([0, nb]), cu, torch.tensor([0, 96]),
                          1 / math.sqrt(16))
    torch.testing.assert_close(o, _sdpa(q, k, v, 2), rtol=1e-10, atol=1e-10)


def test_self_block_equals_block_diagonal():
    q, k, v, cu = _problem(seed=1)
    nb = cu.numel() - 1
    ids = torch.repeat_interleave(torch.arange(nb), (cu[1:] - cu[:-1]).long())
    topk = ids.view(1, -1, 1).expand(2, -1, 1).to(torch.int32).contiguous()
    o, _ = sel_attn_ref(q, k, v, topk, torch.tensor([0, nb]), cu, torch.tensor([0, 96]),
                        1 / math.sqrt(16))
    for b in range(nb):
        s, e = int(cu[b]), int(cu[b + 1])
        torch.testing.assert_close(o[s:e], _sdpa(q[s:e], k[s:e], v[s:e], 2), rtol=1e-10,
                                   atol=1e-10)


def test_repeated_block_counts_twice():
    q, k, v, cu = _problem(seed=2)
    topk = torch.tensor([1, 1, 3], dtype=torch.int32).view(1, 1, 3).expand(2, 96, 3).contiguous()
    o, _ = sel_attn_ref(q, k, v, topk, torch.tensor([0, 5]), cu, torch.tensor([0, 96]), 0.25)
    keys = torch.cat([torch.arange(cu[1], cu[2])] * 2 + [torch.arange(cu[3], cu[4])])
    kk, vv = k[keys], v[keys]
    ref = _sdpa(q * 1.0, kk, vv, 2)  # sdpa's default scale is 1/sqrt(16) = 0.25
    torch.testing.assert_close(o, ref, rtol=1e-10, atol=1e-10)


def test_lse_log2_normalises_weights_and_convexity():
    q, k, v, cu = _problem(seed=3)
    g = torch.Generator().manual_seed(3)
    topk = torch.stack([torch.randperm(5, generator=g)[:3] for _ in range(2 * 96)]).view(2, 96, 3)
    topk = topk.to(torch.int32)
    scale = 0.3
    o, lse = sel_attn_ref(q, k, v, topk, torch.tensor([0, 5]), cu, torch.tensor([0, 96]), scale)
    for h in range(4):
        hk = h // 2
        for i in range(0, 96, 7):
            keys = torch.cat([torch.arange(cu[c], cu[c + 1]) for c in topk[hk, i].tolist()])
            w = torch.exp2(scale * LOG2E * (k[keys, hk] @ q[i, h]) - lse[h, i])
            assert abs(float(w.sum()) - 1.0) < 1e-12
            vv = v[keys, hk]
            assert (o[i, h] <= vv.max(0).values + 1e-12).all()
            assert (o[i, h] >= vv.min(0).values - 1e-12).all()


def test_padding_out_of_range_empty_rows_and_batch_local_ids():
    q, k, v, cu = _problem(seed=4)
    cu_sb = torch.tensor([0, 2, 5])       # batch 0: blocks 0,1 (40 tokens); batch 1: 2..4
    cu_q = torch.tensor([0, 40, 96])
    topk = torch.full((2, 96, 3), -1, dtype=torch.int32)
    topk[:, :, 0] = 1
    topk[:, 50:60, 1] = 7                 # out of range for batch 1 (3 blocks) -> ignored
    topk[:, 10:12, 0] = -1                # empty rows
    o, lse = sel_attn_ref(q, k, v, topk, cu_sb, cu, cu_q, 0.25)
    assert (o[10:12] == 0).all() and torch.isinf(lse[:, 10:12]).all()
    # batch 0 query attends global block 1, batch 1 query attends global block 3
    torch.testing.assert_close(o[0:1], _sdpa(q[0:1], k[10:40], v[10:40], 2))
    torch.testing.assert_close(o[50:51], _sdpa(q[50:51], k[45:66], v[45:66], 2))
    assert attended_pairs(topk, cu_sb, cu, cu_q) == 2 * (38 * 30 + 56 * 21)


def test_backward_gradcheck_fp64():
    q, k, v, cu = _problem(n=40, hq=2, hkv=1, d=4, sizes=(7, 13, 20), seed=5)
    topk = torch.tensor([[2, 0], [1, -1]], dtype=torch.int32)
    rows = torch.cat([topk[0].view(1, 2).expand(20, 2), topk[1].view(1, 2).expand(20, 2)])
    rows = rows.view(1, 40, 2).contiguous()
    meta = (torch.tensor([0, 3]), cu, torch.tensor([0, 40]))

    def fn(q, k, v):
        return sel_attn_ref(q, k, v, rows, *meta, 0.7)[0]

    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()
    assert torch.autograd.gradcheck(fn, (q, k, v), eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("case", ["gqa_batches", "duplicates_empty", "per_token"])
def test_explicit_backward_equals_autograd(case):
    # sel_attn_bwd_ref (run by run, no graph) against torch.autograd through
    # sel_attn_ref, in fp64: GQA over two batch elements with padding and
    # out-of-range ids; a block listed twice plus empty rows; and per-token
    # rows (every query its own run).
    q, k, v, cu = _problem(seed=11)
    g = torch.Generator().manual_seed(12)
    do = torch.randn(q.shape, generator=g, dtype=q.dtype)
    cu_sb = torch.tensor([0, 2, 5])
    cu_q = torch.tensor([0, 40, 96])
    topk = torch.full((2, 96, 4), -1, dtype=torch.int32)
    if case == "gqa_batches":
        topk[:, :40, 0], topk[:, :40, 1] = 0, 1
        topk[:, 40:, 0], topk[:, 40:, 1], topk[:, 40:, 2] = 2, 0, 1
        topk[1, 60:70, 3] = 9              # out of range for batch 1 -> ignored
    elif case == "duplicates_empty":
        topk[:, :, 0], topk[:, :, 1] = 1, 1
        topk[:, 20:25] = -1
        topk[:, 50:80, 2] = 2
    else:
        topk = torch.stack([torch.stack([torch.randperm(2, generator=g) if i < 40 else
                                         torch.randperm(3, generator=g)[:2]
                                         for i in range(96)]) for _ in range(2)]).to(torch.int32)
    meta = (topk, cu_sb, cu, cu_q)
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    o, _ = sel_attn_ref(qa, ka, va, *meta, 0.3)
    o.backward(do)
    dq, dk, dv, delta = sel_attn_bwd_ref(q, k, v, do, *meta, 0.3)
    torch.testing.assert_close(dq, qa.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dk, ka.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dv, va.grad, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(delta, (o.detach() * do).sum(-1).transpose(0, 1),
                               rtol=1e-10, atol=1e-12)
