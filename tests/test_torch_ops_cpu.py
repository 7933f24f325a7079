"""CPU checks of the torch operator registration (lsrm_hip.torch_ops): every
operator is registered under torch.ops.lsrm_hip, its fake implementation
gives the output shapes and dtypes the HIP path returns (checked here on
meta tensors, which dispatch to it), and CPU tensors raise instead of
falling back."""

import pytest
import torch

import lsrm_hip
import sparse.ops as ops
from lsrm_hip.torch_ops import OPS

META = "meta"


def test_every_operator_registered():
    for name in OPS:
        op = getattr(torch.ops.lsrm_hip, name)
        assert op.default._schema.name == f"lsrm_hip::{name}"


def _attn_inputs(n=300, hq=8, hkv=2, d=64, topk=5, nb=7, dtype=torch.bfloat16, dev=META):
    q = torch.empty(n, hq, d, dtype=dtype, device=dev)
    k = torch.empty(n, hkv, d, dtype=dtype, device=dev)
    v = torch.empty(n, hkv, d, dtype=dtype, device=dev)
    topk_idx = torch.empty(hkv, n, topk, dtype=torch.int32, device=dev)
    cu_sb = torch.empty(2, dtype=torch.int32, device=dev)
    cu_blk = torch.empty(nb + 1, dtype=torch.int32, device=dev)
    cu_q = torch.empty(2, dtype=torch.int32, device=dev)
    return q, k, v, topk_idx, cu_sb, cu_blk, cu_q


def test_fake_attention_shapes():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _attn_inputs()
    o, lse = torch.ops.lsrm_hip.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, 0.125)
    assert o.shape == q.shape and o.dtype == q.dtype and o.device.type == META
    assert lse.shape == (8, 300) and lse.dtype == torch.float32
    dq, dk, dv, delta = torch.ops.lsrm_hip.sel_attn_bwd(q, q, k, v, o, lse, topk_idx, cu_sb,
                                                        cu_blk, cu_q, 0.125)
    assert (dq.shape, dk.shape, dv.shape, delta.shape) == (q.shape, k.shape, v.shape, (8, 300))
    assert dq.dtype == dk.dtype == dv.dtype == torch.bfloat16 and delta.dtype == torch.float32


def test_fake_autograd_through_forward_operator():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _attn_inputs(dtype=torch.float16)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    o, _ = torch.ops.lsrm_hip.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, 0.125)
    gq, gk, gv = torch.autograd.grad(o.sum(), (q, k, v))
    assert (gq.shape, gk.shape, gv.shape) == (q.shape, k.shape, v.shape)
    assert gq.dtype == torch.float16


def test_fake_pool_selection_score_shapes():
    q, k, _, _, cu_sb, cu_blk, _ = _attn_inputs()
    x = torch.empty(300, 128, dtype=torch.bfloat16, device=META)
    p = torch.ops.lsrm_hip.block_mean_pool(x, cu_blk, None)
    assert p.shape == (7, 128) and p.dtype == torch.bfloat16
    p32 = torch.ops.lsrm_hip.block_mean_pool(x, cu_blk, torch.float32)
    assert p32.dtype == torch.float32
    pa, pb = torch.ops.lsrm_hip.block_mean_pool2(x, x, cu_blk, torch.float32, None)
    assert pa.shape == pb.shape == (7, 128)
    assert pa.dtype == torch.float32 and pb.dtype == torch.bfloat16
    t, c = torch.ops.lsrm_hip.select_blocks(q, k, cu_sb, cu_blk, 4, [0, 1], True, None)
    assert t.shape == (2, 300, 4) and c.shape == (2, 7, 4) and t.dtype == torch.int32
    ck = torch.empty(7, 2, 64, dtype=torch.bfloat16, device=META)
    lse = torch.empty(8, 300, dtype=torch.float32, device=META)
    s = torch.ops.lsrm_hip.block_score(q, ck, lse, 3, cu_sb, cu_sb, 0.125)
    assert s.shape == (2, 300, 3) and s.dtype == torch.int32
    ids = torch.ops.lsrm_hip.block_ids(cu_sb, cu_blk, 300, 2)
    assert ids.shape == (2, 300, 1) and ids.dtype == torch.int32


@pytest.mark.parametrize("win", [False, True])
def test_fake_gate_merge_shapes(win):
    h = 64
    gate = torch.empty(10, (3 if win else 2) * h, dtype=torch.bfloat16, device=META,
                       requires_grad=True)
    br = [torch.empty(10, h, dtype=torch.bfloat16, device=META, requires_grad=True)
          for _ in range(3 if win else 2)]
    out = torch.ops.lsrm_hip.gate_merge(gate, br[0], br[1], br[2] if win else None)
    assert out.shape == (10, h)
    grads = torch.autograd.grad(out.sum(), [gate] + br)
    assert [g.shape for g in grads] == [gate.shape] + [b.shape for b in br]


def test_cpu_tensors_raise_no_fallback():
    q, k, v, topk_idx, cu_sb, cu_blk, cu_q = _attn_inputs(dev="cpu", n=8, nb=2)
    with pytest.raises(RuntimeError):
        torch.ops.lsrm_hip.sel_attn_fwd(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, 0.125)
    with pytest.raises(RuntimeError):
        ops.sparse3d_compression(torch.zeros(8, 16), torch.tensor([0, 8], dtype=torch.int32))
