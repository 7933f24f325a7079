"""One device plan per selection through autograd, and the one-shot C entry
points.

sparse.ops builds the selection's plan once, with its backward part, in the
forward; the forward, an activation-checkpoint recompute of it and the
backward all run on that plan (lsrm_hip.plan_builds counts the plans built).
The one-shot entry points lsrm_sel_attn_fwd / lsrm_sel_attn_bwd (plan and
run in one call), which the Python layer no longer calls, are checked through
the C ABI against the plan path bit for bit."""

import ctypes

import pytest
import torch
import torch.utils.checkpoint as cp

import lsrm_hip as H
import sparse.ops as ops
from helpers import assert_attn_close, random_topk
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(per_token, seed=3):
    w = W.config(2, n=4096, heads=4)
    gen = torch.Generator().manual_seed(seed)
    q, k, v = ((0.5 * torch.randn(w.n, w.hq, w.d, generator=gen)).to(torch.bfloat16)
               for _ in range(3))
    rows = random_topk(w.hkv, w.n, w.n_blocks, 8, gen,
                       per_block_cu=None if per_token else w.cu_block_tokens)
    meta = [t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens)]
    return w, q, k, v, rows, meta


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("checkpoint", [False, True])
def test_one_plan_per_selection_through_autograd(per_token, checkpoint):
    w, q, k, v, rows, (cu_sb, cu_blk, cu_q) = _case(per_token)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    rd = rows.to(DEV)
    H.clear_plan_cache()
    before = H.plan_builds

    def attend(a, b, c):
        return ops.native_sparse_attend(a, b, c, rd, cu_sb, cu_blk, cu_q, cu_q, w.scale)

    out = cp.checkpoint(attend, qd, kd, vd, use_reentrant=False) if checkpoint else \
        attend(qd, kd, vd)
    g = torch.Generator().manual_seed(5)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    out.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert H.plan_builds - before == 1
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    o_ref, _ = sel_attn_ref(qf, kf, vf, rows, w.cu_seqblocks, w.cu_block_tokens,
                            w.cu_seqlens, w.scale)
    o_ref.backward(do.float())
    assert_attn_close(out, o_ref, "out")
    assert_attn_close(qd.grad, qf.grad, "dq")
    assert_attn_close(kd.grad, kf.grad, "dk")
    assert_attn_close(vd.grad, vf.grad, "dv")


def test_in_place_change_of_the_selection_builds_a_new_plan():
    w, q, k, v, rows, (cu_sb, cu_blk, cu_q) = _case(False)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    rd = rows.to(DEV)
    H.clear_plan_cache()
    before = H.plan_builds
    a, _ = H.sel_attn_fwd(qd, kd, vd, rd, cu_sb, cu_blk, cu_q, w.scale)
    b, _ = H.sel_attn_fwd(qd, kd, vd, rd, cu_sb, cu_blk, cu_q, w.scale)
    assert H.plan_builds - before == 1 and torch.equal(a, b)
    rd[:, :, 0] = rd[:, :, 1]  # same tensor, new contents: the version moves
    c, _ = H.sel_attn_fwd(qd, kd, vd, rd, cu_sb, cu_blk, cu_q, w.scale)
    assert H.plan_builds - before == 2
    o_ref, _ = sel_attn_ref(q.float(), k.float(), v.float(), rd.cpu(), w.cu_seqblocks,
                            w.cu_block_tokens, w.cu_seqlens, w.scale)
    assert_attn_close(c, o_ref, "out after the change")


def test_one_shot_entry_points_match_the_plan_path():
    w, q, k, v, rows, (cu_sb, cu_blk, cu_q) = _case(True, seed=9)
    qd, kd, vd, rd = (t.to(DEV) for t in (q, k, v, rows))
    nq, hq, d = qd.shape
    nk, hkv, _ = kd.shape
    nb = cu_blk.numel() - 1
    lib = H.lib()
    st = torch.cuda.current_stream().cuda_stream
    o_p, lse_p = H.sel_attn_fwd(qd, kd, vd, rd, cu_sb, cu_blk, cu_q, w.scale)
    ws = torch.empty(lib.lsrm_sel_attn_workspace_size(nq, nk, hq, hkv, 8, nb, 1),
                     dtype=torch.uint8, device=DEV)
    o = torch.empty_like(qd)
    lse = torch.empty(hq, nq, dtype=torch.float32, device=DEV)
    assert lib.lsrm_sel_attn_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), H.BF16, nq, nk,
                                 hq, hkv, d, rd.data_ptr(), 8, cu_sb.data_ptr(),
                                 cu_blk.data_ptr(), nb, cu_q.data_ptr(), 1, w.scale,
                                 o.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(),
                                 st) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o_p) and torch.equal(lse, lse_p)
    g = torch.Generator().manual_seed(8)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype).to(DEV)
    ref = H.sel_attn_bwd(do, qd, kd, vd, o, lse, rd, cu_sb, cu_blk, cu_q, w.scale)
    dq, dk, dv = torch.empty_like(qd), torch.zeros_like(kd), torch.zeros_like(vd)
    delta = torch.empty(hq, nq, dtype=torch.float32, device=DEV)
    assert lib.lsrm_sel_attn_bwd(do.data_ptr(), qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                 o.data_ptr(), lse.data_ptr(), H.BF16, nq, nk, hq, hkv, d,
                                 rd.data_ptr(), 8, cu_sb.data_ptr(), cu_blk.data_ptr(), nb,
                                 cu_q.data_ptr(), 1, w.scale, dq.data_ptr(), dk.data_ptr(),
                                 dv.data_ptr(), delta.data_ptr(), ws.data_ptr(), ws.numel(),
                                 st) == 0
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip((dq, dk, dv, delta), ref))
