"""The C ABI registered as PyTorch operators (namespace ``lsrm_hip``).

Each operator wraps one lsrm_hip call (which goes through liblsrm_hip.so):
the dispatcher sees it as an opaque kernel with a schema, a fake (meta)
implementation for shape propagation (torch.compile, FakeTensor, meta
tensors) and, for the two differentiable ones, an autograd formula.  The
sparse.ops front end routes every call through ``torch.ops.lsrm_hip.*``.

Operators (the reference interface each one stands in for):
  sel_attn_fwd     kvcentric:931-1010   native_sparse_attn_forward -> (o, lse)
  sel_attn_bwd     kvcentric:1018-1263  native_sparse_attn_backward -> (dq, dk, dv, delta)
  block_mean_pool  spatial_sparse_attention.py:27-37  sparse3d_compression
  block_mean_pool2 spatial_sparse_attention.py:49-66  the key and value pair
  select_blocks    the benchmark's per-query-block selection -> (topk_idx, compact)
  block_score      block_score.py:16-98  get_block_score
  gate_merge       spatial_sparse_attention.py:256-269 (the gated branch sum)
  gate_merge_bwd   its gradients -> [d_gate, d_cmp, d_slc(, d_win)]
  block_ids        the self-block rows of sparse_window_attention
                   (block_window_attention.py:14-31)
Tensors on the CPU raise (there is no CPU implementation).
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import (
    block_ids as _block_ids,
    block_mean_pool as _block_mean_pool,
    block_mean_pool2 as _block_mean_pool2,
    block_score as _block_score,
    gate_merge as _gate_merge,
    gate_merge_bwd as _gate_merge_bwd,
    sel_attn_bwd as _sel_attn_bwd,
    sel_attn_fwd as _sel_attn_fwd,
    select_blocks as _select_blocks,
)

NS = "lsrm_hip"


# ------------------------------------------------------------- attention --

@torch.library.custom_op(f"{NS}::sel_attn_fwd", mutates_args=())
def sel_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk_idx: torch.Tensor,
                 cu_seqblocks: torch.Tensor, cu_block_tokens: torch.Tensor,
                 cu_seqlens_q: torch.Tensor, softmax_scale: float, key_centric: bool = False
                 ) -> Tuple[torch.Tensor, torch.Tensor]:
    """out [Nq, Hq, D] (q's dtype), lse [Hq, Nq] fp32 in log2 units
    (key_centric: the key-centric plan for per-token rows without locality)."""
    return _sel_attn_fwd(q, k, v, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
                         softmax_scale, key_centric)


@sel_attn_fwd.register_fake
def _(q, k, v, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q, softmax_scale,
      key_centric=False):
    return torch.empty_like(q), q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32)


@torch.library.custom_op(f"{NS}::sel_attn_bwd", mutates_args=())
def sel_attn_bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 o: torch.Tensor, lse: torch.Tensor, topk_idx: torch.Tensor,
                 cu_seqblocks: torch.Tensor, cu_block_tokens: torch.Tensor,
                 cu_seqlens_q: torch.Tensor, softmax_scale: float, key_centric: bool = False
                 ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv, delta [Hq, Nq] fp32 = rowsum(o * do))."""
    return _sel_attn_bwd(do, q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens,
                         cu_seqlens_q, softmax_scale, key_centric)


@sel_attn_bwd.register_fake
def _(do, q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
      softmax_scale, key_centric=False):
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32))


def _fwd_setup(ctx, inputs, output):
    q, k, v, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q, scale = inputs[:8]
    o, lse = output
    ctx.save_for_backward(q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens,
                          cu_seqlens_q)
    ctx.scale = scale
    ctx.key_centric = bool(inputs[8]) if len(inputs) > 8 else False


def _fwd_backward(ctx, do, _dlse):
    q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q = ctx.saved_tensors
    dq, dk, dv, _ = torch.ops.lsrm_hip.sel_attn_bwd(
        do.contiguous().to(q.dtype), q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens,
        cu_seqlens_q, ctx.scale, ctx.key_centric)
    return dq, dk, dv, None, None, None, None, None, None


sel_attn_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup)


# --------------------------------------------------- pooling, selection --

@torch.library.custom_op(f"{NS}::block_mean_pool", mutates_args=())
def block_mean_pool(x: torch.Tensor, cu_block_tokens: torch.Tensor,
                    out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """[N, C] -> [n_blocks, C] block means (bit-exact contract of
    lsrm_block_mean_pool)."""
    return _block_mean_pool(x, cu_block_tokens, out_dtype)


@block_mean_pool.register_fake
def _(x, cu_block_tokens, out_dtype=None):
    return x.new_empty((cu_block_tokens.shape[0] - 1, x.shape[1]), dtype=out_dtype or x.dtype)


@torch.library.custom_op(f"{NS}::block_mean_pool2", mutates_args=())
def block_mean_pool2(x_a: torch.Tensor, x_b: torch.Tensor, cu_block_tokens: torch.Tensor,
                     out_a_dtype: Optional[torch.dtype] = None,
                     out_b_dtype: Optional[torch.dtype] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Keys and values of one block partition in one launch pair (each
    output equals block_mean_pool of its input)."""
    return _block_mean_pool2(x_a, x_b, cu_block_tokens, out_a_dtype, out_b_dtype)


@block_mean_pool2.register_fake
def _(x_a, x_b, cu_block_tokens, out_a_dtype=None, out_b_dtype=None):
    nb = cu_block_tokens.shape[0] - 1
    return (x_a.new_empty((nb, x_a.shape[1]), dtype=out_a_dtype or x_a.dtype),
            x_b.new_empty((nb, x_b.shape[1]), dtype=out_b_dtype or x_b.dtype))


@torch.library.custom_op(f"{NS}::select_blocks", mutates_args=())
def select_blocks(q: torch.Tensor, k: torch.Tensor, cu_seqblocks: torch.Tensor,
                  cu_block_tokens: torch.Tensor, topk: int, forced_blocks: List[int],
                  force_self: bool, pooled_k: Optional[torch.Tensor] = None
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
    """(topk_idx [Hkv, N, topk], compact [Hkv, n_blocks, topk]) int32."""
    return _select_blocks(q, k, cu_seqblocks, cu_block_tokens, topk, forced_blocks,
                          force_self, pooled_k)


@select_blocks.register_fake
def _(q, k, cu_seqblocks, cu_block_tokens, topk, forced_blocks, force_self, pooled_k=None):
    hkv, n, nb = k.shape[1], q.shape[0], cu_block_tokens.shape[0] - 1
    return (q.new_empty((hkv, n, topk), dtype=torch.int32),
            q.new_empty((hkv, nb, topk), dtype=torch.int32))


@torch.library.custom_op(f"{NS}::block_score", mutates_args=())
def block_score(q: torch.Tensor, compressed_k: torch.Tensor, lse: torch.Tensor, topk: int,
                cu_seqlens_q: torch.Tensor, compressed_cu_seqlens: torch.Tensor,
                sm_scale: float) -> torch.Tensor:
    """get_block_score -> [Hkv, Nq, topk] int32."""
    return _block_score(q, compressed_k, lse, topk, cu_seqlens_q, compressed_cu_seqlens,
                        sm_scale)


@block_score.register_fake
def _(q, compressed_k, lse, topk, cu_seqlens_q, compressed_cu_seqlens, sm_scale):
    return q.new_empty((compressed_k.shape[1], q.shape[0], topk), dtype=torch.int32)


@torch.library.custom_op(f"{NS}::block_ids", mutates_args=())
def block_ids(cu_seqblocks: torch.Tensor, cu_block_tokens: torch.Tensor, n_tokens: int,
              hkv: int) -> torch.Tensor:
    """Batch-local block id of every token, [hkv, n_tokens, 1] int32."""
    return _block_ids(cu_seqblocks, cu_block_tokens, n_tokens, hkv)


@block_ids.register_fake
def _(cu_seqblocks, cu_block_tokens, n_tokens, hkv):
    return cu_block_tokens.new_empty((hkv, n_tokens, 1), dtype=torch.int32)


# ------------------------------------------------------------ gate merge --

@torch.library.custom_op(f"{NS}::gate_merge", mutates_args=())
def gate_merge(gate: torch.Tensor, o_cmp: torch.Tensor, o_slc: torch.Tensor,
               o_win: Optional[torch.Tensor] = None) -> torch.Tensor:
    return _gate_merge(gate, o_cmp, o_slc, o_win)


@gate_merge.register_fake
def _(gate, o_cmp, o_slc, o_win=None):
    return torch.empty_like(o_cmp)


@torch.library.custom_op(f"{NS}::gate_merge_bwd", mutates_args=())
def gate_merge_bwd(dout: torch.Tensor, gate: torch.Tensor, o_cmp: torch.Tensor,
                   o_slc: torch.Tensor, o_win: Optional[torch.Tensor] = None
                   ) -> List[torch.Tensor]:
    """[d_gate, d_cmp, d_slc] (+ [d_win] when o_win is given)."""
    out = _gate_merge_bwd(dout, gate, o_cmp, o_slc, o_win)
    return [t for t in out if t is not None]


@gate_merge_bwd.register_fake
def _(dout, gate, o_cmp, o_slc, o_win=None):
    out = [torch.empty_like(gate), torch.empty_like(o_cmp), torch.empty_like(o_slc)]
    if o_win is not None:
        out.append(torch.empty_like(o_win))
    return out


def _gm_setup(ctx, inputs, output):
    gate, o_cmp, o_slc, o_win = inputs
    ctx.has_win = o_win is not None
    ctx.save_for_backward(gate, o_cmp, o_slc, *([o_win] if ctx.has_win else []))


def _gm_backward(ctx, dout):
    saved = ctx.saved_tensors
    grads = torch.ops.lsrm_hip.gate_merge_bwd(dout.contiguous(), *saved)
    return grads[0], grads[1], grads[2], (grads[3] if ctx.has_win else None)


gate_merge.register_autograd(_gm_backward, setup_context=_gm_setup)

OPS = ("sel_attn_fwd", "sel_attn_bwd", "block_mean_pool", "block_mean_pool2", "select_blocks",
       "block_score",
       "block_ids", "gate_merge", "gate_merge_bwd")
