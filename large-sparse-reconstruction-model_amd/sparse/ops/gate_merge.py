"""Gated merge of the sparse-attention branches.

Replaces the expression of sparse/module/spatial_sparse_attention.py:256-269
(SpatialSparseAttentionOut.forward):

    gate = self.gate(x)
    attn_output = gate[:, 0:H] * compressed + gate[:, H:2H] * selection
                  (+ gate[:, 2H:] * window)

with one streaming HIP kernel each way (lsrm_gate_merge / _bwd, operators
torch.ops.lsrm_hip.gate_merge / gate_merge_bwd) instead of
five or eight PyTorch elementwise kernels and their intermediates.  Results
are bit-identical to PyTorch's evaluation of the expression in the tensors'
dtype (every product and sum rounded to the dtype, left to right).
"""

from __future__ import annotations

from typing import Optional

import torch

import lsrm_hip  # noqa: F401  (registers torch.ops.lsrm_hip)


class GateMerge(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, o_cmp, o_slc, o_win):
        ctx.save_for_backward(gate, o_cmp, o_slc, o_win)
        ctx.has_win = o_win is not None
        return torch.ops.lsrm_hip.gate_merge(gate, o_cmp, o_slc, o_win)

    @staticmethod
    def backward(ctx, dout):
        gate, o_cmp, o_slc, o_win = ctx.saved_tensors
        grads = torch.ops.lsrm_hip.gate_merge_bwd(
            dout.contiguous(), gate, o_cmp, o_slc, o_win if ctx.has_win else None)
        return grads[0], grads[1], grads[2], (grads[3] if ctx.has_win else None)


def gate_merge(gate: torch.Tensor, compressed_attn_output: torch.Tensor,
               selection_attn_output: torch.Tensor,
               window_attn_output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gate [N, 2H or 3H], branch outputs [N, H] -> [N, H] (differentiable)."""
    return GateMerge.apply(gate, compressed_attn_output, selection_attn_output,
                           window_attn_output)
