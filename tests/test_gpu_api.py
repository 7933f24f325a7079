"""GPU tests of the reference-compatible API (sparse.ops): autograd through
spatial_selection_attention / native_sparse_attend, window attention,
compression, validation errors."""

import math

import numpy as np
import pytest
import torch

import lsrm_hip as H
import sparse.ops as ops
from helpers import assert_attn_close, random_topk
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _meta(w):
    return [t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.cu_seqlens)]


def test_spatial_selection_attention_autograd():
    w = W.config(2, n=2048, heads=2)
    q, k, v, do = W.tensors(w, "cpu", with_grad_out=True)
    gen = torch.Generator().manual_seed(2)
    topk = random_topk(w.hkv, w.n, w.n_blocks, w.topk, gen, per_block_cu=w.cu_block_tokens)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    cu_sb, cu_blk, cu_q, cu_k = _meta(w)
    seqlens = cu_q[1:] - cu_q[:-1]
    out = ops.spatial_selection_attention(qd, kd, vd, topk.to(DEV), cu_sb, cu_blk, cu_q, cu_k,
                                          seqlens, seqlens)
    out.backward(do.to(DEV))
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    ref, _ = sel_attn_ref(qf, kf, vf, topk, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens,
                          w.scale)
    ref.backward(do.float())
    assert_attn_close(out, ref, "out")
    assert_attn_close(qd.grad, qf.grad, "dq")
    assert_attn_close(kd.grad, kf.grad, "dk")
    assert_attn_close(vd.grad, vf.grad, "dv")


def test_native_sparse_attend_return_lse_and_asserts():
    w = W.config(2, n=1024, heads=2)
    q, k, v = (t.to(DEV) for t in W.tensors(w, "cpu"))
    gen = torch.Generator().manual_seed(3)
    topk = random_topk(w.hkv, w.n, w.n_blocks, 4, gen).to(DEV)
    out, lse = ops.native_sparse_attend(q, k, v, topk, *_meta(w), return_lse=True)
    assert out.shape == q.shape and lse.shape == (w.hq, w.n) and lse.dtype == torch.float32
    with pytest.raises(AssertionError):
        ops.native_sparse_attend(q.float(), k.float(), v.float(), topk, *_meta(w))
    with pytest.raises(AssertionError):
        ops.native_sparse_attend(q, k, v, topk.long(), *_meta(w))


def test_validation_rejects_bad_metadata():
    w = W.config(2, n=1024, heads=2)
    q, k, v = (t.to(DEV) for t in W.tensors(w, "cpu"))
    topk = torch.full((w.hkv, w.n, 3), -1, dtype=torch.int32, device=DEV)
    topk[:, :, 0] = 0
    topk[:, 7, 2] = 1   # valid id after a -1: not a prefix
    with pytest.raises(ValueError, match="valid block id after an invalid"):
        ops.native_sparse_attend(q, k, v, topk, *_meta(w))
    cu_sb, cu_blk, cu_q, cu_k = _meta(w)
    bad = cu_blk.clone()
    bad[3] = bad[5]
    topk[:, 7, 2] = -1
    with pytest.raises(ValueError, match="not monotone"):
        ops.native_sparse_attend(q, k, v, topk, cu_sb, bad, cu_q, cu_k)


def test_sparse_window_attention_block_diagonal():
    n, hq, hkv, d = 2000, 4, 2, 64
    rng = np.random.default_rng(1)
    sizes = W.uniform_partition(n, 16, 200, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(n, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    out = ops.sparse_window_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV))
    # block-diagonal SDPA per block in fp32
    ref = torch.empty(n, hq, d)
    g = hq // hkv
    for b in range(len(sizes)):
        s, e = int(cu[b]), int(cu[b + 1])
        qq = q[s:e].float().transpose(0, 1)
        kk = k[s:e].float().repeat_interleave(g, 1).transpose(0, 1)
        vv = v[s:e].float().repeat_interleave(g, 1).transpose(0, 1)
        ref[s:e] = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv).transpose(0, 1)
    assert_attn_close(out, ref, "window")


def test_sparse3d_compression_matches_segment_reduce():
    w = W.config(3, n=8192)
    x = torch.randn(w.n, 3 * 64, device=DEV).to(torch.bfloat16)
    out = ops.sparse3d_compression(x, w.cu_block_tokens.to(DEV))
    lens = (w.cu_block_tokens[1:] - w.cu_block_tokens[:-1]).to(DEV)
    ref = torch.segment_reduce(x.float(), "mean", lengths=lens, axis=0)
    assert out.dtype == torch.bfloat16 and out.shape == ref.shape
    torch.testing.assert_close(out.float(), ref, rtol=1e-2, atol=1e-2)


def test_select_blocks_feeds_attention():
    w = W.config(3, n=8192, heads=2)
    q, k, v = (t.to(DEV) for t in W.tensors(w, "cpu"))
    cu_sb, cu_blk, cu_q, cu_k = _meta(w)
    topk = ops.select_blocks(q, k, cu_sb, cu_blk, w.topk, w.forced_blocks)
    assert topk.shape == (w.hkv, w.n, w.topk)
    out = ops.spatial_selection_attention(q, k, v, topk, cu_sb, cu_blk, cu_q, cu_k, None, None)
    ref, _ = sel_attn_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), topk.cpu(),
                          w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale)
    assert_attn_close(out, ref, "out")
