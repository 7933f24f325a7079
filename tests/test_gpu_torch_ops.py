"""GPU checks of the registered operators (torch.ops.lsrm_hip.*): results
against the oracle, torch.library.opcheck (schema, fake implementation,
autograd registration, AOT dispatch with dynamic shapes) and a whole
sparse-attention step under torch.compile(fullgraph=True) with no graph
break, equal to eager."""

import math

import numpy as np
import pytest
import torch

import lsrm_hip  # noqa: F401
import sparse.ops as ops
from helpers import assert_attn_close, random_topk
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_ref
from oracle.pool import block_mean_pool_ref
from oracle.select import select_blocks_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(n=2048, heads=4, seed=0):
    w = W.config(2, n=n, heads=heads)
    q, k, v = (t.to(DEV) for t in W.tensors(w, "cpu"))
    gen = torch.Generator().manual_seed(seed)
    topk = random_topk(w.hkv, w.n, w.n_blocks, w.topk, gen,
                       per_block_cu=w.cu_block_tokens).to(DEV)
    meta = [t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens)]
    return w, q, k, v, topk, meta


def test_sel_attn_fwd_operator_matches_oracle():
    w, q, k, v, topk, meta = _case()
    o, lse = torch.ops.lsrm_hip.sel_attn_fwd(q, k, v, topk, *meta, w.scale)
    o_ref, lse_ref = sel_attn_ref(q.float().cpu(), k.float().cpu(), v.float().cpu(), topk.cpu(),
                                  w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale)
    assert_attn_close(o, o_ref, "out")
    assert float((lse.cpu() - lse_ref).abs().max()) <= 2e-2


def test_sel_attn_operator_autograd_matches_oracle():
    w, q, k, v, topk, meta = _case(n=1024, heads=2, seed=1)
    do = torch.randn_like(q)
    qd, kd, vd = (t.clone().requires_grad_() for t in (q, k, v))
    o, _ = torch.ops.lsrm_hip.sel_attn_fwd(qd, kd, vd, topk, *meta, w.scale)
    o.backward(do)
    qf, kf, vf = (t.float().cpu().requires_grad_() for t in (q, k, v))
    o_ref, _ = sel_attn_ref(qf, kf, vf, topk.cpu(), w.cu_seqblocks, w.cu_block_tokens,
                            w.cu_seqlens, w.scale)
    o_ref.backward(do.float().cpu())
    for nm, a, b in (("dq", qd.grad, qf.grad), ("dk", kd.grad, kf.grad), ("dv", vd.grad, vf.grad)):
        assert_attn_close(a, b, nm)


def test_pool_and_select_operators_bitexact():
    w, q, k, _, _, meta = _case(n=4096, heads=2)
    pk = torch.ops.lsrm_hip.block_mean_pool(k.view(w.n, -1), meta[1], torch.float32)
    cu = w.cu_block_tokens.numpy()
    ref_pk = block_mean_pool_ref(k.float().cpu().view(w.n, -1).numpy(), cu)
    assert np.array_equal(pk.cpu().numpy().view(np.int32), ref_pk.view(np.int32))
    t, c = torch.ops.lsrm_hip.select_blocks(q, k, meta[0], meta[1], w.topk, [0, 3], True, pk)
    ref_pq = block_mean_pool_ref(q.float().cpu().view(w.n, -1).numpy(), cu)
    ref = select_blocks_ref(ref_pq.reshape(-1, w.hq, w.d), ref_pk.reshape(-1, w.hkv, w.d),
                            w.cu_seqblocks.numpy(), w.topk, [0, 3], True)
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


def test_opcheck_operators():
    w, q, k, v, topk, meta = _case(n=1024, heads=2, seed=2)
    qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
    torch.library.opcheck(torch.ops.lsrm_hip.sel_attn_fwd.default,
                          (qg, kg, vg, topk, *meta, w.scale))
    torch.library.opcheck(torch.ops.lsrm_hip.block_mean_pool.default,
                          (k.view(w.n, -1), meta[1], torch.float32))
    torch.library.opcheck(torch.ops.lsrm_hip.block_mean_pool2.default,
                          (k.view(w.n, -1), v.view(w.n, -1), meta[1], torch.float32, None))
    torch.library.opcheck(torch.ops.lsrm_hip.select_blocks.default,
                          (q, k, meta[0], meta[1], 8, [1], True, None))
    torch.library.opcheck(torch.ops.lsrm_hip.block_ids.default, (meta[0], meta[1], w.n, w.hkv))
    ck = torch.ops.lsrm_hip.block_mean_pool(k.view(w.n, -1), meta[1], None).view(-1, w.hkv, w.d)
    lse = torch.randn(w.hq, w.n, device=DEV)
    cu_c = torch.tensor([0, ck.shape[0]], dtype=torch.int32, device=DEV)
    torch.library.opcheck(torch.ops.lsrm_hip.block_score.default,
                          (q, ck, lse, 6, meta[2], cu_c, w.scale))
    hid = w.hq * w.d
    gate = torch.rand(w.n, 3 * hid, device=DEV).to(q.dtype).requires_grad_()
    brs = [torch.randn(w.n, hid, device=DEV).to(q.dtype).requires_grad_() for _ in range(3)]
    torch.library.opcheck(torch.ops.lsrm_hip.gate_merge.default, (gate, *brs))


def test_compiled_layer_equals_eager():
    # pool K -> select -> selected attention -> gated merge, compiled whole
    # (fullgraph: any graph break raises) with the AOT-autograd eager
    # backend, forward and backward; results equal the eager ones bitwise.
    w, q, k, v, _, meta = _case(n=2048, heads=4, seed=3)
    hid = w.hq * w.d
    gate = torch.rand(w.n, 2 * hid, device=DEV).to(q.dtype)
    other = torch.randn(w.n, hid, device=DEV).to(q.dtype)

    def layer(q, k, v, gate, other):
        topk = ops.select_blocks(q, k, meta[0], meta[1], w.topk, [0], True)
        o = ops.spatial_selection_attention(q, k, v, topk, meta[0], meta[1], meta[2], meta[2],
                                            None, None)
        return ops.gate_merge(gate, other, o.reshape(w.n, hid))

    ops.set_validation(False)
    try:
        compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
        results = []
        for fn in (layer, compiled):
            ins = [t.clone().requires_grad_() for t in (q, k, v, gate, other)]
            out = fn(*ins)
            out.backward(torch.ones_like(out))
            results.append([out.detach()] + [t.grad for t in ins])
    finally:
        ops.set_validation(True)
    for a, b in zip(*results):
        assert torch.equal(a, b)
