"""Gated branch merge oracle (test infrastructure only).

Restates the expression of SpatialSparseAttentionOut.forward
(sparse/module/spatial_sparse_attention.py:256-269)

    out = gate[:, 0:H] * o_cmp + gate[:, H:2H] * o_slc (+ gate[:, 2H:] * o_win)

as PyTorch evaluates it on tensors of one dtype: every product and every sum
is a separate elementwise op computed in fp32 and rounded to the dtype
(round to nearest even), left to right.  The backward is autograd of the
expression: d_o_x = rnd(dout * g_x), d_g_x = rnd(dout * o_x).
Pins (tests/test_oracle_gate.py): PyTorch's own CPU evaluation of the
reference expression and of its autograd, bit for bit, in bf16 / fp16 / fp32;
one-hot gates return a branch exactly; a case where the reference's
left-to-right order and rounding after each op give a different result from
an fp32 fused sum.
"""

from __future__ import annotations

from typing import Optional

import numpy as np


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """fp32 -> dtype ('bf16', 'fp16', 'fp32') with round to nearest even,
    returned as fp32 values."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "fp32":
        return x
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    if dtype != "bf16":
        raise ValueError(dtype)
    bits = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    lsb = (bits >> 16) & 1
    r = ((bits + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def gate_merge_ref(gate: np.ndarray, o_cmp: np.ndarray, o_slc: np.ndarray,
                   o_win: Optional[np.ndarray], dtype: str) -> np.ndarray:
    """Inputs hold dtype values (as fp32 arrays); returns out as fp32 values."""
    h = o_cmp.shape[1]
    r = lambda v: round_to(v, dtype)
    g = np.asarray(gate, dtype=np.float32)
    t = r(r(g[:, 0:h] * o_cmp) + r(g[:, h:2 * h] * o_slc))
    if o_win is not None:
        t = r(t + r(g[:, 2 * h:3 * h] * o_win))
    return t


def gate_merge_bwd_ref(dout: np.ndarray, gate: np.ndarray, o_cmp: np.ndarray,
                       o_slc: np.ndarray, o_win: Optional[np.ndarray], dtype: str):
    """-> (d_gate, d_cmp, d_slc, d_win or None), fp32 arrays of dtype values."""
    h = o_cmp.shape[1]
    r = lambda v: round_to(v, dtype)
    branches = [o_cmp, o_slc] + ([o_win] if o_win is not None else [])
    g = np.asarray(gate, dtype=np.float32)
    d_gate = np.concatenate([r(dout * b) for b in branches], axis=1)
    d_br = [r(dout * g[:, i * h:(i + 1) * h]) for i in range(len(branches))]
    return d_gate, d_br[0], d_br[1], (d_br[2] if o_win is not None else None)
