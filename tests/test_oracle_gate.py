"""Pins of the gated branch merge oracle (oracle/gate.py) against PyTorch's
own CPU evaluation of the reference expression
(sparse/module/spatial_sparse_attention.py:256-269) and its autograd, plus
closed forms that a wrong rounding order would fail."""

import numpy as np
import pytest
import torch

from oracle.gate import gate_merge_bwd_ref, gate_merge_ref, round_to

DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _case(n, h, win, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    k = 3 if win else 2
    gate = torch.sigmoid(torch.randn(n, k * h, generator=g)).to(DT[dtype])
    br = [torch.randn(n, h, generator=g).to(DT[dtype]) for _ in range(k)]
    return gate, br


def _np(t):
    return t.detach().float().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("win", [False, True])
def test_matches_torch_expression_and_autograd(dtype, win):
    gate, br = _case(64, 48, win, dtype, 1 + win)
    gate.requires_grad_(True)
    for b in br:
        b.requires_grad_(True)
    h = br[0].shape[1]
    # the reference's expression, evaluated by PyTorch on the CPU
    out = gate[:, 0:h] * br[0] + gate[:, h:2 * h] * br[1]
    if win:
        out = out + gate[:, 2 * h:] * br[2]
    ref = gate_merge_ref(_np(gate), _np(br[0]), _np(br[1]), _np(br[2]) if win else None, dtype)
    np.testing.assert_array_equal(_np(out), ref)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(9)).to(out.dtype)
    out.backward(dout)
    d_gate, d_c, d_s, d_w = gate_merge_bwd_ref(_np(dout), _np(gate), _np(br[0]), _np(br[1]),
                                               _np(br[2]) if win else None, dtype)
    np.testing.assert_array_equal(_np(gate.grad), d_gate)
    np.testing.assert_array_equal(_np(br[0].grad), d_c)
    np.testing.assert_array_equal(_np(br[1].grad), d_s)
    if win:
        np.testing.assert_array_equal(_np(br[2].grad), d_w)


def test_one_hot_gates_select_a_branch():
    _, br = _case(16, 8, True, "bf16", 3)
    x = [_np(b) for b in br]
    for i in range(3):
        gate = np.zeros((16, 24), np.float32)
        gate[:, i * 8:(i + 1) * 8] = 1.0
        np.testing.assert_array_equal(gate_merge_ref(gate, x[0], x[1], x[2], "bf16"), x[i])


def test_rounding_after_each_op_and_left_to_right():
    # bf16 has 8 significant bits: 256 + 1 rounds to 256 (ties to even), so
    # (256 + 1) + 1 = 256 while a fused fp32 sum gives 258 -> 258 in bf16.
    one = np.ones((1, 1), np.float32)
    out = gate_merge_ref(np.ones((1, 3), np.float32), 256 * one, one, one, "bf16")
    assert out[0, 0] == 256.0
    assert round_to(np.float32(258.0), "bf16") == 258.0
    # products are rounded before the sum: 1.00390625 = 1 + 2^-8 is not a
    # bf16 value; g * x rounds it to 1 before adding 1.
    g = np.array([[1.00390625, 1.0]], np.float32)
    out2 = gate_merge_ref(g, one, one, None, "fp32")
    assert out2[0, 0] == np.float32(2.00390625)
    out3 = gate_merge_ref(round_to(g, "bf16"), one, one, None, "bf16")
    assert out3[0, 0] == 2.0
