"""Variable-block selected attention (forward + backward) on gfx950.

Public API and autograd mirror
sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:1272-1435
(set_variant, NSA, native_sparse_attend) and
sparse/ops/triton_native_sparse_attention.py:17-41
(spatial_selection_attention); the kernels behind them are the HIP kernels of
liblsrm_hip.so (lsrm_sel_attn_fwd / lsrm_sel_attn_bwd), reached through the
registered operators torch.ops.lsrm_hip.sel_attn_fwd / sel_attn_bwd.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

import lsrm_hip as _hip

_default_variant = "a"
_validate = True
_key_centric = "auto"


def set_variant(variant: str) -> None:
    """Kept for API compatibility (kvcentric:1275-1278).  The reference picks
    Triton pipeline depths for its dK/dV kernel; the HIP kernels have one
    tuned configuration, so the value is recorded and otherwise unused."""
    global _default_variant
    _default_variant = variant


def set_validation(enabled: bool) -> None:
    """Enables/disables the device-side metadata check (one host sync per
    forward call).  On by default; turn off for graph capture or timing."""
    global _validate
    _validate = bool(enabled)


def set_key_centric(enabled) -> None:
    """Plans the forward and dQ with the key-centric pass for per-token rows
    (learned selections, 3D-aware maps): the grouped tiles (consecutive
    queries whose rows differ) are taken out of the grouped-tile passes,
    each block's selecting queries are gathered into full tiles and the
    per-block partial results merged in row order, one range of queries at
    a time so that the partial results stay within 1 GiB.  True, False, or
    "auto" (the default): per selection, on when its runs of identical rows
    are short enough for the plan to form grouped tiles (one device
    reduction and one host read per selection)."""
    global _key_centric
    _key_centric = enabled if enabled == "auto" else bool(enabled)


def _use_key_centric(q, k, topk_idx) -> bool:
    """The key-centric choice for this selection (see set_key_centric)."""
    if _key_centric != "auto":
        return bool(_key_centric)
    # Under graph capture or compilation the count cannot be read back (and a
    # key-centric plan is not built under capture): the grouped-tile plan.
    if topk_idx.shape[1] < 2 or torch.compiler.is_compiling() or \
            (topk_idx.is_cuda and torch.cuda.is_current_stream_capturing()):
        return False
    # The plan groups runs shorter than a quarter of a 128-row tile's
    # queries; the key-centric part pays off when such runs dominate.
    short = max(1, (128 // (q.shape[1] // k.shape[1])) // 4)
    changes = int((topk_idx[:, 1:] != topk_idx[:, :-1]).any(-1).sum())
    runs = changes + topk_idx.shape[0]
    return runs * short > topk_idx.shape[0] * topk_idx.shape[1]


def _check_meta(q, k, topk_idx, cu_seqblocks, cu_block_include_tokens, cu_seqlens_q,
                cu_seqlens_k) -> None:
    if topk_idx.dim() != 3 or topk_idx.shape[0] != k.shape[1] or topk_idx.shape[1] != q.shape[0]:
        raise ValueError(
            f"topk_idx must be [num_kv_heads, total_q, topk]; got {tuple(topk_idx.shape)} for "
            f"q {tuple(q.shape)} and k {tuple(k.shape)}")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError("num_q_heads must be a multiple of num_kv_heads")
    if cu_seqlens_q.numel() != cu_seqblocks.numel():
        raise ValueError("cu_seqlens_q and cu_seqblocks must both have batch_size + 1 entries")
    if not _validate:
        return
    bits = _hip.validate(topk_idx, cu_seqblocks, cu_block_include_tokens, cu_seqlens_q,
                         cu_seqlens_k, k.shape[0])
    bits &= ~_hip.META_TOPK_EMPTY_ROW   # empty rows are defined: output 0
    if bits:
        raise ValueError(f"invalid sparse-attention metadata: {_hip.describe_meta_error(bits)}")


class NSA(torch.autograd.Function):
    """Autograd wrapper (kvcentric:1281-1371): forward returns (o, lse);
    backward returns grads for q, k, v only."""

    @staticmethod
    def forward(ctx, q, k, v, topk_idx, cu_seqblocks, cu_block_include_tokens,
                cu_seqlens_q, cu_seqlens_k, softmax_scale=None):
        assert q.dtype in [torch.float16, torch.bfloat16], "Only fp16/bf16 supported"
        assert q.dtype == k.dtype == v.dtype
        assert topk_idx.dtype == torch.int32
        assert cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32

        q = q.contiguous()
        k = k.contiguous()
        v = v.contiguous()
        topk_idx = topk_idx.contiguous()
        cu_seqblocks = _hip._i32(cu_seqblocks)
        cu_block_include_tokens = _hip._i32(cu_block_include_tokens)
        cu_seqlens_q = cu_seqlens_q.contiguous()
        cu_seqlens_k = cu_seqlens_k.contiguous()

        if softmax_scale is None:
            softmax_scale = 1.0 / math.sqrt(q.shape[-1])

        _check_meta(q, k, topk_idx, cu_seqblocks, cu_block_include_tokens, cu_seqlens_q,
                    cu_seqlens_k)
        key_centric = _use_key_centric(q, k, topk_idx)
        if any(t.requires_grad for t in (q, k, v)) and q.is_cuda and q.shape[0] > 0 and \
                not torch.compiler.is_compiling():
            # One plan per selection: built here with its backward part, it
            # serves this forward, a checkpoint recompute and the backward.
            _hip.plan_for(q.shape, k.shape, topk_idx, cu_seqblocks, cu_block_include_tokens,
                          cu_seqlens_q, backward=True, key_centric=key_centric)
        o, lse = torch.ops.lsrm_hip.sel_attn_fwd(q, k, v, topk_idx, cu_seqblocks,
                                                 cu_block_include_tokens, cu_seqlens_q,
                                                 float(softmax_scale), key_centric)
        ctx.save_for_backward(q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, topk_idx,
                              cu_seqblocks, cu_block_include_tokens)
        ctx.softmax_scale = softmax_scale
        ctx.key_centric = key_centric
        ctx.mark_non_differentiable(lse)
        return o, lse

    @staticmethod
    def backward(ctx, do, _dlse):
        (q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, topk_idx, cu_seqblocks,
         cu_block_include_tokens) = ctx.saved_tensors
        do = do.contiguous()
        if do.dtype != q.dtype:
            do = do.to(q.dtype)
        dq, dk, dv, _delta = torch.ops.lsrm_hip.sel_attn_bwd(
            do, q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_include_tokens,
            cu_seqlens_q, float(ctx.softmax_scale), ctx.key_centric)
        return dq, dk, dv, None, None, None, None, None, None


_native_sparse_attend = NSA.apply


def native_sparse_attend(
    q,  # [total_tokens, num_q_heads, dim]
    k,  # [total_tokens, num_kv_heads, dim]
    v,  # [total_tokens, num_kv_heads, dim]
    topk_idx,  # [num_kv_heads, total_tokens, topk]
    cu_seqblocks,  # [batch_size + 1]
    cu_block_include_tokens,  # [total_blocks + 1]
    cu_seqlens_q,  # [batch_size + 1]
    cu_seqlens_k,  # [batch_size + 1]
    softmax_scale: Optional[float] = None,
    return_lse: bool = False,
):
    """Variable-block-size native sparse attention (kvcentric:1382-1435).

    Every query attends to the tokens of its valid selected blocks (batch-local
    ids in [0, blocks of its batch element)); repeated ids count twice.
    Returns out [total_q, num_q_heads, dim] (and lse [num_q_heads, total_q],
    fp32, log2 units, when return_lse).
    """
    out, lse = _native_sparse_attend(q, k, v, topk_idx, cu_seqblocks, cu_block_include_tokens,
                                     cu_seqlens_q, cu_seqlens_k, softmax_scale)
    if not return_lse:
        return out
    return out, lse


def spatial_selection_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    block_topk: torch.Tensor,
    cu_seqblocks: torch.Tensor,
    cu_block_include_tokens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    seqlens_q: torch.Tensor,
    seqlens_k: torch.Tensor,
    softmax_scale: Optional[float] = None,
) -> torch.Tensor:
    """Drop-in for sparse/ops/triton_native_sparse_attention.py:17-41
    (seqlens_q / seqlens_k are accepted and unused, as there)."""
    return native_sparse_attend(q, k, v, block_topk, cu_seqblocks, cu_block_include_tokens,
                                cu_seqlens_q, cu_seqlens_k, softmax_scale=softmax_scale)
