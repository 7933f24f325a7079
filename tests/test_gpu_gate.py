"""GPU parity of the gated branch merge (sparse.ops.gate_merge, HIP
lsrm_gate_merge / _bwd) against the oracle, bit for bit: both dtypes of the
attention path and fp32, two and three branches, the 16-byte vector path and
the element path (hidden not a multiple of 8), forward and autograd; at the
cfg3 layer shape through one-hot gates and a sampled oracle check."""

import numpy as np
import pytest
import torch

import sparse.ops as ops
from oracle.gate import gate_merge_bwd_ref, gate_merge_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("win", [False, True])
@pytest.mark.parametrize("hidden", [64, 50])
def test_gate_merge_fwd_bwd_bitexact(dtype, win, hidden):
    n = 300
    g = torch.Generator().manual_seed(hidden + 7 * win)
    k = 3 if win else 2
    gate = torch.sigmoid(torch.randn(n, k * hidden, generator=g)).to(DT[dtype])
    br = [torch.randn(n, hidden, generator=g).to(DT[dtype]) for _ in range(k)]
    dout = torch.randn(n, hidden, generator=g).to(DT[dtype])
    gd = gate.to(DEV).requires_grad_(True)
    bd = [b.to(DEV).requires_grad_(True) for b in br]
    out = ops.gate_merge(gd, bd[0], bd[1], bd[2] if win else None)
    ref = gate_merge_ref(_np(gate), _np(br[0]), _np(br[1]), _np(br[2]) if win else None, dtype)
    np.testing.assert_array_equal(_np(out), ref)
    out.backward(dout.to(DEV))
    d_gate, d_c, d_s, d_w = gate_merge_bwd_ref(_np(dout), _np(gate), _np(br[0]), _np(br[1]),
                                               _np(br[2]) if win else None, dtype)
    np.testing.assert_array_equal(_np(gd.grad), d_gate)
    np.testing.assert_array_equal(_np(bd[0].grad), d_c)
    np.testing.assert_array_equal(_np(bd[1].grad), d_s)
    if win:
        np.testing.assert_array_equal(_np(bd[2].grad), d_w)


def test_gate_merge_matches_torch_on_device():
    n, h = 1000, 96
    g = torch.Generator(device=DEV).manual_seed(3)
    gate = torch.sigmoid(torch.randn(n, 3 * h, generator=g, device=DEV)).bfloat16()
    c, s, w = (torch.randn(n, h, generator=g, device=DEV).bfloat16() for _ in range(3))
    ref = gate[:, 0:h] * c + gate[:, h:2 * h] * s + gate[:, 2 * h:] * w
    assert torch.equal(ops.gate_merge(gate, c, s, w), ref)


def test_gate_merge_layer_shape_one_hot_and_sampled():
    # cfg3 layer: 131072 tokens, hidden 1536, three branches
    n, h = 131072, 1536
    g = torch.Generator(device=DEV).manual_seed(5)
    br = [torch.randn(n, h, generator=g, device=DEV).bfloat16() for _ in range(3)]
    for i in range(3):
        gate = torch.zeros(n, 3 * h, device=DEV, dtype=torch.bfloat16)
        gate[:, i * h:(i + 1) * h] = 1.0
        assert torch.equal(ops.gate_merge(gate, *br), br[i])
    gate = torch.sigmoid(torch.randn(n, 3 * h, generator=g, device=DEV)).bfloat16()
    out = ops.gate_merge(gate, *br)
    rows = torch.randint(0, n, (64,), generator=g, device=DEV)
    ref = gate_merge_ref(_np(gate[rows]), *(_np(b[rows]) for b in br), "bf16")
    np.testing.assert_array_equal(_np(out[rows]), ref)
