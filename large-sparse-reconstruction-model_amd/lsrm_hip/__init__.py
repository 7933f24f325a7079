"""Python binding of liblsrm_hip.so (the C ABI in include/lsrm_hip.h).

PyTorch supplies device memory and the current HIP stream; every compute call
goes to a gfx950 kernel in liblsrm_hip.so through ctypes.  There is no CPU or
PyTorch fallback: a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import collections
import ctypes
import math
from pathlib import Path
from typing import Optional, Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblsrm_hip.so"

F32, F16, BF16 = 0, 1, 2
PLAN_BACKWARD, PLAN_KEY_CENTRIC = 1, 2  # lsrm_sel_attn_plan2 flags
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# lsrm_meta_error bits (include/lsrm_hip.h)
META_ERRORS = {
    1: "cu_block_include_tokens is not monotone",
    2: "a block's token range lies outside [0, n_k)",
    4: "cu_seqblocks is not monotone or exceeds the block count",
    8: "cu_seqlens_q / cu_seqlens_k are not valid offsets",
    16: "a top-k row has a valid block id after an invalid entry",
    32: "a top-k row selects no valid block",
    64: "a batch element's blocks leave its key range",
}
META_TOPK_EMPTY_ROW = 32

_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "lsrm_status_string": (ctypes.c_char_p, [_I]),
    "lsrm_version": (_I, []),
    "lsrm_block_mean_pool_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lsrm_block_mean_pool": (_I, [_P, _I, _I64, _I64, _P, _I64, _P, _I, _P, _SZ, _P]),
    "lsrm_block_mean_pool_noalloc": (_I, [_P, _I, _I64, _I64, _P, _I64, _P, _I, _P]),
    "lsrm_block_mean_pool2_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "lsrm_block_mean_pool2": (
        _I, [_P, _P, _I, _I64, _I64, _P, _I64, _P, _I, _P, _I, _P, _SZ, _P]),
    "lsrm_select_blocks_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "lsrm_select_blocks": (
        _I,
        [_P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I,
         _P, _P, _P, _SZ, _P],
    ),
    "lsrm_select_blocks_pooled": (
        _I,
        [_P, _P, _I, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I,
         _P, _P, _P, _SZ, _P],
    ),
    "lsrm_sel_attn_validate": (
        _I, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _I64, _P, _P]),
    "lsrm_sel_attn_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I]),
    "lsrm_sel_attn_fwd": (
        _I,
        [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P,
         _I64, _F, _P, _P, _P, _SZ, _P],
    ),
    "lsrm_sel_attn_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P,
         _I64, _P, _I64, _F, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "lsrm_sel_attn_plan": (
        _I, [_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I, _P, _SZ, _P]),
    "lsrm_sel_attn_fwd_run": (
        _I,
        [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P,
         _I64, _F, _P, _P, _P, _SZ, _P],
    ),
    "lsrm_sel_attn_workspace_size2": (
        _SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I]),
    "lsrm_sel_attn_plan2": (
        _I, [_P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I, _P, _SZ,
             _P]),
    "lsrm_sel_attn_fwd_run2": (
        _I,
        [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P,
         _I64, _F, _P, _P, _P, _SZ, _I, _P],
    ),
    "lsrm_sel_attn_bwd_run2": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P,
         _I64, _P, _I64, _F, _P, _P, _P, _P, _P, _SZ, _I, _P],
    ),
    "lsrm_sel_attn_bwd_run": (
        _I,
        [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _P,
         _I64, _P, _I64, _F, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "lsrm_reverse_query_map_workspace_size": (_SZ, [_I64, _I64, _I64, _I64]),
    "lsrm_reverse_query_map": (
        _I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _SZ, _P]),
    "lsrm_block_ids": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "lsrm_block_score": (
        _I, [_P, _P, _I, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _F, _P, _P]),
    "lsrm_volume_points": (_I, [_P, _I64, _I64, _F, _P, _P]),
    "lsrm_nearest_blocks": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "lsrm_image_points": (_I, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "lsrm_image_block_rank_workspace_size": (_SZ, [_I64, _I64]),
    "lsrm_image_block_rank": (
        _I, [_P, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64,
             _I64, _F, _I64, _P, _P, _SZ, _P]),
    "lsrm_block_separation_workspace_size": (_SZ, [_I64, _I, _P, _P]),
    "lsrm_block_separation": (_I, [_P, _I64, _I, _P, _P, _I64, _P, _P, _P, _P, _SZ, _P]),
    "lsrm_block_sort_workspace_size": (_SZ, [_I64]),
    "lsrm_block_sort": (_I, [_P, _I64, _I, _I64, _P, _P, _P, _SZ, _P]),
    "lsrm_gate_merge": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _P, _P]),
    "lsrm_gate_merge_bwd": (_I, [_P, _P, _P, _P, _P, _I, _I64, _I64, _P, _P, _P, _P, _P]),
}


def lib() -> ctypes.CDLL:
    """Loads liblsrm_hip.so (built in-tree by lsrm_hip.build)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m lsrm_hip.build` "
                "(there is no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols() -> list:
    return list(_SIGNATURES)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().lsrm_status_string(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {rc})")


def _dev_check(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "lsrm_hip kernels need ROCm device tensors; got a tensor on "
                f"{t.device} (there is no CPU fallback)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("all tensors must live on the same device")
    return dev


def _attn_check(q, k, v, topk_idx, do=None, o=None, lse=None) -> torch.device:
    """Device, dtype, shape and layout checks shared by every attention entry
    (the C ABI takes raw pointers: a CPU tensor or a mis-shaped buffer must
    stop here, before any kernel sees its address)."""
    dev = _dev_check(q, k, v, topk_idx, do, o, lse)
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError("q [Nq, Hq, D], k and v [Nk, Hkv, D] expected")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k must share the head dim")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or \
            v.dtype != q.dtype:
        raise TypeError("q, k and v must share dtype float16 or bfloat16")
    if topk_idx.dim() != 3 or topk_idx.dtype != torch.int32 or \
            topk_idx.shape[0] != k.shape[1] or topk_idx.shape[1] != q.shape[0]:
        raise ValueError("topk_idx must be int32 [Hkv, Nq, topk]")
    for name, t in (("do", do), ("o", o)):
        if t is not None and (t.shape != q.shape or t.dtype != q.dtype):
            raise ValueError(f"{name} must match q in shape and dtype")
    if lse is not None and (tuple(lse.shape) != (q.shape[1], q.shape[0]) or
                            lse.dtype != torch.float32):
        raise ValueError("lse must be float32 [Hq, Nq]")
    for t in (q, k, v, topk_idx, do, o, lse):
        if t is not None and not t.is_contiguous():
            raise ValueError("attention tensors must be contiguous")
    return dev


def _no_capture(what: str) -> None:
    """Backward and key-centric plans sort with rocPRIM, whose radix sort
    clears its state with hipMemsetAsync: such plans are not built under HIP
    graph capture (a memset node has given wrong results on graph replays)."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(f"{what} cannot be built under HIP graph capture (its sort "
                           "issues memsets); build the plan before capturing")


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


# --------------------------------------------------------------- pooling --

def block_mean_pool(x: torch.Tensor, cu_block_tokens: torch.Tensor,
                    out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Mean of each block's rows of a 2-D [N, C] tensor -> [n_blocks, C].

    Bit-exact contract: fp32 sums over pieces cut at multiples of 64 rows and
    at block boundaries, sequential within and across pieces, IEEE divide,
    round-to-nearest-even to out_dtype (default: x's dtype).
    """
    if x.dim() != 2:
        raise ValueError("x must be 2-D [n_tokens, channels]")
    if x.dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported dtype {x.dtype}")
    out_dtype = out_dtype or x.dtype
    if out_dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported output dtype {out_dtype}")
    dev = _dev_check(x, cu_block_tokens)
    x = x.contiguous()
    cu = _i32(cu_block_tokens)
    n, c = x.shape
    nb = cu.numel() - 1
    out = torch.empty(nb, c, dtype=out_dtype, device=dev)
    if nb == 0:
        return out
    with torch.cuda.device(dev):
        ws_n = lib().lsrm_block_mean_pool_workspace_size(n, c, nb)
        ws = _workspace(ws_n, dev)
        _check(lib().lsrm_block_mean_pool(
            _ptr(x), _DTYPE_CODE[x.dtype], n, c, _ptr(cu), nb, _ptr(out),
            _DTYPE_CODE[out_dtype], _ptr(ws), ws.numel(), _stream(dev)),
            "lsrm_block_mean_pool")
    return out


def block_mean_pool2(x_a: torch.Tensor, x_b: torch.Tensor, cu_block_tokens: torch.Tensor,
                     out_a_dtype: Optional[torch.dtype] = None,
                     out_b_dtype: Optional[torch.dtype] = None):
    """block_mean_pool of two [N, C] tensors of one dtype over one block
    partition (keys and values) in one pair of launches -> (out_a, out_b),
    each bit for bit equal to block_mean_pool of its input."""
    if x_a.dim() != 2 or x_a.shape != x_b.shape:
        raise ValueError("x_a and x_b must be 2-D [n_tokens, channels] of one shape")
    if x_a.dtype not in _DTYPE_CODE or x_b.dtype != x_a.dtype:
        raise TypeError(f"unsupported or mismatched dtypes {x_a.dtype}, {x_b.dtype}")
    out_a_dtype = out_a_dtype or x_a.dtype
    out_b_dtype = out_b_dtype or x_a.dtype
    if out_a_dtype not in _DTYPE_CODE or out_b_dtype not in _DTYPE_CODE:
        raise TypeError(f"unsupported output dtypes {out_a_dtype}, {out_b_dtype}")
    dev = _dev_check(x_a, x_b, cu_block_tokens)
    x_a, x_b = x_a.contiguous(), x_b.contiguous()
    cu = _i32(cu_block_tokens)
    n, c = x_a.shape
    nb = cu.numel() - 1
    out_a = torch.empty(nb, c, dtype=out_a_dtype, device=dev)
    out_b = torch.empty(nb, c, dtype=out_b_dtype, device=dev)
    if nb == 0:
        return out_a, out_b
    with torch.cuda.device(dev):
        ws = _workspace(lib().lsrm_block_mean_pool2_workspace_size(n, c, nb), dev)
        _check(lib().lsrm_block_mean_pool2(
            _ptr(x_a), _ptr(x_b), _DTYPE_CODE[x_a.dtype], n, c, _ptr(cu), nb, _ptr(out_a),
            _DTYPE_CODE[out_a_dtype], _ptr(out_b), _DTYPE_CODE[out_b_dtype], _ptr(ws),
            ws.numel(), _stream(dev)), "lsrm_block_mean_pool2")
    return out_a, out_b


# ------------------------------------------------------------- selection --

def select_blocks(q: torch.Tensor, k: torch.Tensor, cu_seqblocks: torch.Tensor,
                  cu_block_tokens: torch.Tensor, topk: int,
                  forced_blocks=None,  # sequence of ints, or a device int32 tensor
                  force_self: bool = True,
                  pooled_k: Optional[torch.Tensor] = None):
    """Per-query-block top-k selection (self attention).

    q [N, Hq, D], k [N, Hkv, D].  Returns (topk_idx [Hkv, N, topk],
    topk_compact [Hkv, n_blocks, topk]) int32, ids batch-local, ascending,
    -1 padded.  pooled_k, when given, is block_mean_pool(k.view(N, -1),
    cu_block_tokens, torch.float32): the selection then skips pooling k.
    """
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q [N, Hq, D] and k [N, Hkv, D] must share N and D")
    if q.dtype != k.dtype or q.dtype not in _DTYPE_CODE:
        raise TypeError("q and k must share a float dtype")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError("Hq must be a multiple of Hkv")
    if topk <= 0:
        raise ValueError("topk must be positive")
    dev = _dev_check(q, k, cu_seqblocks, cu_block_tokens,
                     *([] if pooled_k is None else [pooled_k]))
    q = q.contiguous()
    k = k.contiguous()
    cu_sb = _i32(cu_seqblocks)
    cu = _i32(cu_block_tokens)
    n, hq, d = q.shape
    hkv = k.shape[1]
    nb = cu.numel() - 1
    batch = cu_sb.numel() - 1
    forced = None
    if isinstance(forced_blocks, torch.Tensor):
        # a device int32 tensor is used as is (no host-to-device copy per call)
        if forced_blocks.numel() > 0:
            forced = forced_blocks.to(device=dev, dtype=torch.int32).contiguous()
    elif forced_blocks is not None and len(forced_blocks) > 0:
        forced = torch.as_tensor(list(forced_blocks), dtype=torch.int32, device=dev)
    if nb == 0 or n == 0:
        return (torch.full((hkv, n, topk), -1, dtype=torch.int32, device=dev),
                torch.full((hkv, max(nb, 0), topk), -1, dtype=torch.int32, device=dev))
    # every row is written by the kernels (uncovered tokens get -1 rows)
    topk_idx = torch.empty((hkv, n, topk), dtype=torch.int32, device=dev)
    compact = torch.empty((hkv, nb, topk), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        ws_n = lib().lsrm_select_blocks_workspace_size(n, nb, hq, hkv, d)
        ws = _workspace(ws_n, dev)
        if pooled_k is not None:
            if pooled_k.dtype != torch.float32 or tuple(pooled_k.shape) != (nb, hkv * d):
                raise ValueError(f"pooled_k must be float32 [{nb}, {hkv * d}]")
            pooled_k = pooled_k.contiguous()
        entry = lib().lsrm_select_blocks if pooled_k is None else lib().lsrm_select_blocks_pooled
        _check(entry(
            _ptr(q), _ptr(k if pooled_k is None else pooled_k), _DTYPE_CODE[q.dtype], n, hq,
            hkv, d, _ptr(cu_sb), batch,
            _ptr(cu), nb, topk, _ptr(forced), 0 if forced is None else forced.numel(),
            1 if force_self else 0, _ptr(topk_idx), _ptr(compact), _ptr(ws), ws.numel(),
            _stream(dev)), "lsrm_select_blocks" if pooled_k is None else "lsrm_select_blocks_pooled")
    return topk_idx, compact


# ------------------------------------------------------------- attention --

def validate(topk_idx: torch.Tensor, cu_seqblocks: torch.Tensor,
             cu_block_tokens: torch.Tensor, cu_seqlens_q: torch.Tensor,
             cu_seqlens_k: torch.Tensor, n_k: int) -> int:
    """Device-side metadata check; returns the lsrm_meta_error bits (syncs)."""
    dev = _dev_check(topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q, cu_seqlens_k)
    topk_idx = _i32(topk_idx)
    hkv, nq, k = topk_idx.shape
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _check(lib().lsrm_sel_attn_validate(
            _ptr(topk_idx), hkv, nq, k, _ptr(_i32(cu_seqblocks)),
            _ptr(_i32(cu_block_tokens)), cu_block_tokens.numel() - 1,
            _ptr(_i32(cu_seqlens_q)), _ptr(_i32(cu_seqlens_k)), cu_seqlens_q.numel() - 1,
            n_k, _ptr(flags), _stream(dev)), "lsrm_sel_attn_validate")
    return int(flags.item())


def describe_meta_error(bits: int) -> str:
    return "; ".join(msg for b, msg in META_ERRORS.items() if bits & b)


def sel_attn_fwd(q, k, v, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
                 softmax_scale: float, key_centric: bool = False):
    """Selected-block attention forward -> (out [Nq, Hq, D], lse [Hq, Nq] log2).

    The device plan comes from plan_for (one plan per selection, shared with
    a later backward of the same selection).  key_centric: plan with
    LSRM_PLAN_KEY_CENTRIC (per-token rows without locality run as per-block
    gathered tiles plus a merge, over query ranges whose partial results
    stay within 1 GiB)."""
    dev = _attn_check(q, k, v, topk_idx)
    _dev_check(q, cu_seqblocks, cu_block_tokens, cu_seqlens_q)
    out = torch.empty_like(q)
    lse = torch.empty(q.shape[1], q.shape[0], dtype=torch.float32, device=dev)
    if q.shape[0] == 0:
        return out, lse
    plan = plan_for(q.shape, k.shape, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
                    backward=False, key_centric=key_centric)
    return plan.fwd(q, k, v, softmax_scale, out, lse)


def sel_attn_bwd(do, q, k, v, o, lse, topk_idx, cu_seqblocks, cu_block_tokens,
                 cu_seqlens_q, softmax_scale: float, key_centric: bool = False):
    """Selected-block attention backward -> (dq, dk, dv, delta) on the plan
    of the selection (plan_for: the forward's plan when it was built with
    its backward part, otherwise a new backward plan).  key_centric: dQ of
    per-token rows without locality on gathered tiles."""
    dev = _attn_check(q, k, v, topk_idx, do=do, o=o, lse=lse)
    _dev_check(q, cu_seqblocks, cu_block_tokens, cu_seqlens_q)
    if q.shape[0] == 0:
        return (torch.empty_like(q), torch.zeros_like(k), torch.zeros_like(v),
                torch.empty(q.shape[1], 0, dtype=torch.float32, device=dev))
    plan = plan_for(q.shape, k.shape, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
                    backward=True, key_centric=key_centric)
    return plan.bwd(do, q, k, v, o, lse, softmax_scale)


# Plans of the most recent selections, keyed by the selection's tensors
# (address, version counter, shape) and the plan flags: the forward, an
# activation-checkpoint recompute and the backward of one selection share one
# plan.  A cached plan holds its selection tensors, so their memory cannot be
# handed to another tensor while the entry lives; an in-place change of a
# tensor bumps its version and misses.
_PLAN_CACHE_SIZE = 2
_plan_cache: "collections.OrderedDict" = collections.OrderedDict()
plan_builds = 0  # plans built through plan_for (a counter for tests)


def _plan_key(q_shape, k_shape, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
              key_centric):
    ts = (topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q)
    return (tuple(q_shape), tuple(k_shape[:2]), bool(key_centric), str(topk_idx.device),
            tuple(topk_idx.shape)) + tuple((t.data_ptr(), t._version, t.numel()) for t in ts)


def plan_for(q_shape, k_shape, topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q,
             backward: bool = False, key_centric: bool = False) -> "SelAttnPlan":
    """The SelAttnPlan of a selection, built once and reused: a cached plan
    with the backward part also serves forwards; a forward-only plan is
    replaced by one with the backward part when a backward asks.  Under HIP
    graph capture the plan is always built inside the capture (a replay then
    rebuilds it from the replayed selection)."""
    global plan_builds
    capturing = torch.cuda.is_current_stream_capturing()
    if capturing and not backward:
        # the key-centric part sorts with rocPRIM (memsets): a captured
        # forward takes the grouped-tile plan, which captures
        key_centric = False
    key = None if capturing else _plan_key(q_shape, k_shape, topk_idx, cu_seqblocks,
                                           cu_block_tokens, cu_seqlens_q, key_centric)
    if key is not None:
        hit = _plan_cache.get(key)
        if hit is not None and (hit.backward or not backward):
            _plan_cache.move_to_end(key)
            return hit
    plan = SelAttnPlan(q_shape, k_shape, topk_idx, cu_seqblocks, cu_block_tokens,
                       cu_seqlens_q, backward=backward, key_centric=key_centric)
    plan_builds += 1
    if key is not None:
        _plan_cache[key] = plan
        _plan_cache.move_to_end(key)
        while len(_plan_cache) > _PLAN_CACHE_SIZE:
            _plan_cache.popitem(last=False)
    return plan


def clear_plan_cache() -> None:
    """Drops the cached plans (and the workspace memory they hold)."""
    _plan_cache.clear()


class SelAttnPlan:
    """Device plan of one selection (lsrm_sel_attn_plan), replayable by
    fwd()/bwd() any number of times on the current stream.  The tensors given
    here must stay alive and unchanged while the plan is used."""

    def __init__(self, q_shape, k_shape, topk_idx, cu_seqblocks, cu_block_tokens,
                 cu_seqlens_q, backward: bool = False, key_centric: bool = False):
        dev = _dev_check(topk_idx, cu_seqblocks, cu_block_tokens, cu_seqlens_q)
        self.dev = dev
        self.nq, self.hq, self.d = q_shape
        self.nk, self.hkv = k_shape[0], k_shape[1]
        self.topk_idx = topk_idx
        self.cu_seqblocks = cu_seqblocks
        self.cu_block_tokens = cu_block_tokens
        self.cu_seqlens_q = cu_seqlens_q
        self.topk = topk_idx.shape[-1]
        self.nb = cu_block_tokens.numel() - 1
        self.batch = cu_seqlens_q.numel() - 1
        self.backward = backward
        self.flags = (PLAN_BACKWARD if backward else 0) | (PLAN_KEY_CENTRIC if key_centric else 0)
        if self.flags:
            _no_capture("a backward or key-centric plan")
        with torch.cuda.device(dev):
            n = lib().lsrm_sel_attn_workspace_size2(self.nq, self.nk, self.hq, self.hkv,
                                                    self.d, self.topk, self.nb, self.flags)
            if n == 0:
                raise ValueError("unsupported attention plan sizes or flags")
            self.ws = _workspace(n, dev)
            _check(lib().lsrm_sel_attn_plan2(
                _ptr(topk_idx), self.nq, self.nk, self.hq, self.hkv, self.d, self.topk,
                _ptr(cu_seqblocks), _ptr(cu_block_tokens), self.nb, _ptr(cu_seqlens_q),
                self.batch, self.flags, _ptr(self.ws), self.ws.numel(), _stream(dev)),
                "lsrm_sel_attn_plan2")

    def _check_shapes(self, q, k, v, do=None, o=None, lse=None):
        dev = _attn_check(q, k, v, self.topk_idx, do=do, o=o, lse=lse)
        if dev != self.dev or tuple(q.shape) != (self.nq, self.hq, self.d) or \
                tuple(k.shape[:2]) != (self.nk, self.hkv):
            raise ValueError("q / k / v do not match the shapes or device the plan was built for")

    def fwd(self, q, k, v, softmax_scale: float, out=None, lse=None):
        out = torch.empty_like(q) if out is None else out
        lse = torch.empty(self.hq, self.nq, dtype=torch.float32, device=self.dev) \
            if lse is None else lse
        self._check_shapes(q, k, v, o=out, lse=lse)
        with torch.cuda.device(self.dev):
            _check(lib().lsrm_sel_attn_fwd_run2(
                _ptr(q), _ptr(k), _ptr(v), _DTYPE_CODE[q.dtype], self.nq, self.nk, self.hq,
                self.hkv, self.d, _ptr(self.topk_idx), self.topk, _ptr(self.cu_seqblocks),
                _ptr(self.cu_block_tokens), self.nb, _ptr(self.cu_seqlens_q), self.batch,
                float(softmax_scale), _ptr(out), _ptr(lse), _ptr(self.ws), self.ws.numel(),
                self.flags, _stream(self.dev)), "lsrm_sel_attn_fwd_run2")
        return out, lse

    def bwd(self, do, q, k, v, o, lse, softmax_scale: float):
        if not self.backward:
            raise RuntimeError("plan was built without backward=True")
        self._check_shapes(q, k, v, do=do, o=o, lse=lse)
        dq = torch.empty_like(q)
        dk = torch.zeros_like(k)
        dv = torch.zeros_like(v)
        delta = torch.empty(self.hq, self.nq, dtype=torch.float32, device=self.dev)
        with torch.cuda.device(self.dev):
            _check(lib().lsrm_sel_attn_bwd_run2(
                _ptr(do), _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _DTYPE_CODE[q.dtype],
                self.nq, self.nk, self.hq, self.hkv, self.d, _ptr(self.topk_idx), self.topk,
                _ptr(self.cu_seqblocks), _ptr(self.cu_block_tokens), self.nb,
                _ptr(self.cu_seqlens_q), self.batch, float(softmax_scale), _ptr(dq), _ptr(dk),
                _ptr(dv), _ptr(delta), _ptr(self.ws), self.ws.numel(), self.flags,
                _stream(self.dev)), "lsrm_sel_attn_bwd_run2")
        return dq, dk, dv, delta


def reverse_query_map(topk_idx: torch.Tensor, cu_seqlens_q: torch.Tensor,
                      cu_seqblocks: torch.Tensor, total_blocks: int):
    """CSR inverse of a top-k selection (the reference's
    _build_reverse_query_mapping): returns (cu_reverse_count [Hkv, nb+1],
    reverse_query_indices [Hkv, max_entries]) int32, segments ascending.
    Synchronises once to size the output, as the reference does."""
    dev = _dev_check(topk_idx, cu_seqlens_q, cu_seqblocks)
    topk_idx = _i32(topk_idx)
    hkv, nq, k = topk_idx.shape
    cap = max(nq * k, 1)
    cu_rev = torch.empty(hkv, total_blocks + 1, dtype=torch.int32, device=dev)
    rev = torch.empty(hkv, cap, dtype=torch.int32, device=dev)
    totals = torch.empty(hkv, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        ws_n = lib().lsrm_reverse_query_map_workspace_size(nq, hkv, k, total_blocks)
        ws = _workspace(ws_n, dev)
        _check(lib().lsrm_reverse_query_map(
            _ptr(topk_idx), hkv, nq, k, _ptr(_i32(cu_seqlens_q)), _ptr(_i32(cu_seqblocks)),
            cu_seqblocks.numel() - 1, total_blocks, _ptr(cu_rev), _ptr(rev), cap,
            _ptr(totals), _ptr(ws), ws.numel(), _stream(dev)), "lsrm_reverse_query_map")
    max_entries = int(totals.max().item()) if hkv > 0 else 0
    max_entries = max(max_entries, 1)
    return cu_rev, rev[:, :max_entries].contiguous()


def block_ids(cu_seqblocks: torch.Tensor, cu_block_tokens: torch.Tensor, n_tokens: int,
              hkv: int) -> torch.Tensor:
    """Batch-local block id of every token, [hkv, n_tokens, 1] int32."""
    dev = _dev_check(cu_seqblocks, cu_block_tokens)
    ids = torch.empty(hkv, n_tokens, 1, dtype=torch.int32, device=dev)
    if n_tokens == 0:
        return ids
    with torch.cuda.device(dev):
        _check(lib().lsrm_block_ids(
            _ptr(_i32(cu_seqblocks)), cu_seqblocks.numel() - 1, _ptr(_i32(cu_block_tokens)),
            cu_block_tokens.numel() - 1, n_tokens, hkv, _ptr(ids), _stream(dev)),
            "lsrm_block_ids")
    return ids


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


# ------------------------------------------------------ learned selection --

def block_score(q: torch.Tensor, compressed_k: torch.Tensor, lse: torch.Tensor, topk: int,
                cu_seqlens_q: torch.Tensor, compressed_cu_seqlens: torch.Tensor,
                sm_scale: float) -> torch.Tensor:
    """get_block_score on the GPU -> block_topk [Hkv, Nq, topk] int32
    (batch-local compressed-key ids ascending, -1 padded)."""
    if q.dim() != 3 or compressed_k.dim() != 3 or q.shape[2] != compressed_k.shape[2]:
        raise ValueError("q [Nq, Hq, D] and compressed_k [Nc, Hkv, D] must share D")
    if q.dtype != compressed_k.dtype or q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("q and compressed_k must share dtype float16 or bfloat16")
    if q.shape[1] % compressed_k.shape[1] != 0:
        raise ValueError("Hq must be a multiple of Hkv")
    if topk <= 0:
        raise ValueError("topk must be positive")
    dev = _dev_check(q, compressed_k, lse, cu_seqlens_q, compressed_cu_seqlens)
    nq, hq, d = q.shape
    hkv = compressed_k.shape[1]
    if tuple(lse.shape) != (hq, nq):
        raise ValueError(f"lse must be [Hq, Nq] = [{hq}, {nq}]; got {tuple(lse.shape)}")
    q = q.contiguous()
    ck = compressed_k.contiguous()
    lse = lse.contiguous().float()
    cu_q = _i32(cu_seqlens_q)
    cu_c = _i32(compressed_cu_seqlens)
    batch = cu_q.numel() - 1
    if nq == 0 or batch <= 0:
        return torch.full((hkv, nq, topk), -1, dtype=torch.int32, device=dev)
    out = torch.empty((hkv, nq, topk), dtype=torch.int32, device=dev)  # the kernel writes every row
    with torch.cuda.device(dev):
        _check(lib().lsrm_block_score(
            _ptr(q), _ptr(ck), _DTYPE_CODE[q.dtype], _ptr(lse), nq, hq, hkv, d, _ptr(cu_q),
            _ptr(cu_c), batch, topk, float(sm_scale), _ptr(out), _stream(dev)),
            "lsrm_block_score")
    return out


# ------------------------------------------------------------ 3D-aware --

def volume_points(coords: torch.Tensor, volume_res: int, bbox_radius: float) -> torch.Tensor:
    """coords [N, 4] ints (batch, c1, c2, c3) -> points [N, 3] fp32 (x, y, z)."""
    if coords.dim() != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be [N, 4] (batch, c1, c2, c3)")
    dev = _dev_check(coords)
    c = _i32(coords)
    n = c.shape[0]
    pts = torch.empty(n, 3, dtype=torch.float32, device=dev)
    radius = float(torch.tensor(bbox_radius * 1.05, dtype=torch.float32))
    with torch.cuda.device(dev):
        _check(lib().lsrm_volume_points(_ptr(c), n, int(volume_res), radius, _ptr(pts),
                                        _stream(dev)), "lsrm_volume_points")
    return pts


def nearest_blocks(points: torch.Tensor, cu_block_tokens: torch.Tensor,
                   cu_seqblocks: torch.Tensor, cu_seqlens: torch.Tensor, topk: int,
                   num_kv_heads: int = 2) -> torch.Tensor:
    """Per-token nearest block centroids -> block_topk [num_kv_heads, N, topk]
    int32 (batch-local ids ascending, -1 padded)."""
    if points.dim() != 2 or points.shape[1] != 3 or points.dtype != torch.float32:
        raise ValueError("points must be [N, 3] float32")
    if topk <= 0:
        raise ValueError("topk must be positive")
    dev = _dev_check(points, cu_block_tokens, cu_seqblocks, cu_seqlens)
    points = points.contiguous()
    n = points.shape[0]
    cu_q = _i32(cu_seqlens)
    cu_sb = _i32(cu_seqblocks)
    centroids = block_mean_pool(points, cu_block_tokens, torch.float32)
    out = torch.full((num_kv_heads, n, topk), -1, dtype=torch.int32, device=dev)
    batch = cu_q.numel() - 1
    if n == 0 or batch <= 0:
        return out
    with torch.cuda.device(dev):
        _check(lib().lsrm_nearest_blocks(_ptr(points), _ptr(centroids), _ptr(cu_q),
                                         _ptr(cu_sb), batch, n, topk, num_kv_heads,
                                         _ptr(out), _stream(dev)), "lsrm_nearest_blocks")
    return out


def nearest_blocks_to(qpoints: torch.Tensor, key_points: torch.Tensor,
                      cu_block_tokens: torch.Tensor, cu_seqblocks: torch.Tensor,
                      cu_seqlens_q: torch.Tensor, topk: int,
                      num_kv_heads: int = 2) -> torch.Tensor:
    """Per query point, the nearest block centroids of another token set
    (centroid = block mean of key_points) -> [num_kv_heads, Nq, topk] int32
    (batch-local ids ascending, -1 padded)."""
    for t in (qpoints, key_points):
        if t.dim() != 2 or t.shape[1] != 3 or t.dtype != torch.float32:
            raise ValueError("points must be [N, 3] float32")
    if topk <= 0:
        raise ValueError("topk must be positive")
    dev = _dev_check(qpoints, key_points, cu_block_tokens, cu_seqblocks, cu_seqlens_q)
    qpoints = qpoints.contiguous()
    n = qpoints.shape[0]
    cu_q = _i32(cu_seqlens_q)
    cu_sb = _i32(cu_seqblocks)
    centroids = block_mean_pool(key_points.contiguous(), cu_block_tokens, torch.float32)
    out = torch.full((num_kv_heads, n, topk), -1, dtype=torch.int32, device=dev)
    batch = cu_q.numel() - 1
    if n == 0 or batch <= 0:
        return out
    with torch.cuda.device(dev):
        _check(lib().lsrm_nearest_blocks(_ptr(qpoints), _ptr(centroids), _ptr(cu_q), _ptr(cu_sb),
                                         batch, n, topk, num_kv_heads, _ptr(out), _stream(dev)),
               "lsrm_nearest_blocks")
    return out


def image_points(imcoords: torch.Tensor, surface_points: torch.Tensor, masks: torch.Tensor,
                 patch_res: int) -> torch.Tensor:
    """from_imcoords_to_points: imcoords [N, 4] (batch, image, patch row,
    patch column), surface_points [B, M, S, S, 3] fp32, masks B*M*S*S values
    -> [N, 3] fp32 points (NaN for coordinates outside the arrays)."""
    if imcoords.dim() != 2 or imcoords.shape[1] != 4:
        raise ValueError("imcoords must be [N, 4]")
    if surface_points.dim() != 5 or surface_points.shape[-1] != 3 or \
            surface_points.shape[2] != surface_points.shape[3]:
        raise ValueError("surface_points must be [B, M, S, S, 3]")
    b, m, s = surface_points.shape[:3]
    if masks.numel() != b * m * s * s:
        raise ValueError("masks must hold B * M * S * S values")
    dev = _dev_check(imcoords, surface_points, masks)
    c = _i32(imcoords)
    sp = surface_points.contiguous().float()
    mk = masks.contiguous().float()
    out = torch.empty(c.shape[0], 3, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _check(lib().lsrm_image_points(_ptr(c), c.shape[0], _ptr(sp), _ptr(mk), b, m, s,
                                       int(patch_res), _ptr(out), _stream(dev)),
               "lsrm_image_points")
    return out


def image_block_rank(qpoints: torch.Tensor, cu_seqlens_q: torch.Tensor, cameras: torch.Tensor,
                     image_meta: torch.Tensor, kept_blocks: torch.Tensor,
                     cols_per_batch: torch.Tensor, cols: int, blocks_w: int, ibs: int,
                     surface_points: torch.Tensor, dense_masks: torch.Tensor, win: int,
                     topk: int, max_dist: float, num_kv_heads: int = 2) -> torch.Tensor:
    """The per-token image-block rows of build_image_to_image_attn /
    build_volume_to_image_attn from the per-image records the sparse.builders
    host code prepares (cameras [B, M, 18] fp32, image_meta [B, M, 4] int32)
    -> [num_kv_heads, Nq, topk] int32 (position order, -1 padded)."""
    dev = _dev_check(qpoints, cu_seqlens_q, cameras, image_meta, cols_per_batch,
                     surface_points, dense_masks)
    b, m, s = surface_points.shape[:3]
    n = qpoints.shape[0]
    out = torch.full((num_kv_heads, n, topk), -1, dtype=torch.int32, device=dev)
    if n == 0:
        return out
    kept = _i32(kept_blocks) if kept_blocks.numel() else torch.zeros(1, dtype=torch.int32,
                                                                       device=dev)
    qp = qpoints.contiguous().float()
    sp = surface_points.contiguous().float()
    dm = dense_masks.contiguous().float()
    cam = cameras.contiguous().float()
    meta = _i32(image_meta)
    cpb = _i32(cols_per_batch)
    cu_q = _i32(cu_seqlens_q)
    with torch.cuda.device(dev):
        ws_n = lib().lsrm_image_block_rank_workspace_size(n, int(cols))
        ws = _workspace(ws_n, dev)
        _check(lib().lsrm_image_block_rank(
            _ptr(qp), n, _ptr(cu_q), cu_q.numel() - 1, m, _ptr(cam), _ptr(meta), _ptr(kept),
            _ptr(cpb), int(cols), int(blocks_w), s, int(ibs), _ptr(sp), _ptr(dm), int(win),
            int(topk), float(max_dist), num_kv_heads, _ptr(out), _ptr(ws), ws.numel(),
            _stream(dev)), "lsrm_image_block_rank")
    return out


# ------------------------------------------------------- metadata builders --

def block_separation(coords: torch.Tensor, dim: int, block_size, resolution,
                     batch: int):
    """compute_block_separation on the GPU -> (cu_seqblocks [batch + 1],
    cu_block_tokens [n_blocks + 1]) int32 (one host synchronisation, to
    size the second output)."""
    if coords.dim() != 2 or coords.shape[1] != 1 + dim:
        raise ValueError(f"coords must be [N, {1 + dim}] (batch, then {dim} coordinates)")
    dev = _dev_check(coords)
    c = _i32(coords)
    bs = (ctypes.c_int32 * dim)(*[int(x) for x in block_size][:dim])
    res = (ctypes.c_int32 * dim)(*[int(x) for x in resolution][:dim])
    bs_p, res_p = ctypes.addressof(bs), ctypes.addressof(res)
    ws_n = lib().lsrm_block_separation_workspace_size(batch, dim, bs_p, res_p)
    if ws_n == 0:
        raise ValueError("unsupported block_size / resolution / batch")
    nbins = 1
    for d in range(dim):
        nbins *= int(resolution[d]) // int(block_size[d])
    cu_sb = torch.empty(batch + 1, dtype=torch.int32, device=dev)
    cu_blk = torch.empty(batch * nbins + 1, dtype=torch.int32, device=dev)
    n_blocks = torch.empty(1, dtype=torch.int32, device=dev)
    ws = _workspace(ws_n, dev)
    with torch.cuda.device(dev):
        _check(lib().lsrm_block_separation(
            _ptr(c), c.shape[0], dim, bs_p, res_p, batch, _ptr(cu_sb), _ptr(cu_blk),
            _ptr(n_blocks), _ptr(ws), ws.numel(), _stream(dev)), "lsrm_block_separation")
    nb = int(n_blocks.item())
    return cu_sb, cu_blk[:nb + 1]


def block_sort_permutation(coords: torch.Tensor, layout: int, block_size: int, dims) -> torch.Tensor:
    """Sort permutation of sort_volume_blocks (layout 0, dims = (volume_res,))
    or sort_image_blocks (layout 1, dims = (n_images, patch_res)) -> int64 [N]."""
    if coords.dim() != 2 or coords.shape[1] != 4:
        raise ValueError("coords must be [N, 4]")
    dev = _dev_check(coords)
    c = _i32(coords)
    n = c.shape[0]
    perm = torch.empty(n, dtype=torch.int32, device=dev)
    if n == 0:
        return perm.long()
    dd = (ctypes.c_int64 * len(dims))(*[int(x) for x in dims])
    ws = _workspace(lib().lsrm_block_sort_workspace_size(n), dev)
    with torch.cuda.device(dev):
        _check(lib().lsrm_block_sort(_ptr(c), n, layout, int(block_size), ctypes.addressof(dd),
                                     _ptr(perm),
                                     _ptr(ws), ws.numel(), _stream(dev)), "lsrm_block_sort")
    return perm.long()


def _gate_args(gate, branches):
    """Shared checks of gate_merge / gate_merge_bwd: one dtype and device,
    gate [N, k*H] for k branches [N, H]."""
    for t in branches:
        if t.dim() != 2 or t.shape != branches[0].shape:
            raise ValueError("branch outputs must all be [n_tokens, hidden]")
    n, hid = branches[0].shape
    if gate.dim() != 2 or gate.shape[0] != n or gate.shape[1] != len(branches) * hid:
        raise ValueError(f"gate must be [n_tokens, {len(branches)} * hidden]")
    if any(t.dtype != gate.dtype for t in branches) or gate.dtype not in _DTYPE_CODE:
        raise TypeError("gate and branch outputs must share one of bf16 / fp16 / fp32")
    _dev_check(gate, *branches)
    return n, hid


def gate_merge(gate: torch.Tensor, o_cmp: torch.Tensor, o_slc: torch.Tensor,
               o_win: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gate[:, :H] * o_cmp + gate[:, H:2H] * o_slc (+ gate[:, 2H:] * o_win),
    each op rounded to the dtype as PyTorch evaluates the expression."""
    branches = [o_cmp, o_slc] + ([o_win] if o_win is not None else [])
    gate = gate.contiguous()
    branches = [b.contiguous() for b in branches]
    n, hid = _gate_args(gate, branches)
    out = torch.empty_like(branches[0])
    dev = gate.device
    with torch.cuda.device(dev):
        _check(lib().lsrm_gate_merge(
            _ptr(gate), _ptr(branches[0]), _ptr(branches[1]),
            _ptr(branches[2]) if o_win is not None else None, _DTYPE_CODE[gate.dtype], n, hid,
            _ptr(out), _stream(dev)), "lsrm_gate_merge")
    return out


def gate_merge_bwd(dout: torch.Tensor, gate: torch.Tensor, o_cmp: torch.Tensor,
                   o_slc: torch.Tensor, o_win: Optional[torch.Tensor] = None):
    """Gradients of gate_merge: (d_gate, d_cmp, d_slc, d_win or None)."""
    branches = [o_cmp, o_slc] + ([o_win] if o_win is not None else [])
    gate = gate.contiguous()
    branches = [b.contiguous() for b in branches]
    dout = dout.contiguous()
    n, hid = _gate_args(gate, branches)
    if dout.shape != branches[0].shape or dout.dtype != gate.dtype:
        raise ValueError("dout must match the branch outputs")
    d_gate = torch.empty_like(gate)
    d_br = [torch.empty_like(b) for b in branches]
    dev = gate.device
    with torch.cuda.device(dev):
        _check(lib().lsrm_gate_merge_bwd(
            _ptr(dout), _ptr(gate), _ptr(branches[0]), _ptr(branches[1]),
            _ptr(branches[2]) if o_win is not None else None, _DTYPE_CODE[gate.dtype], n, hid,
            _ptr(d_gate), _ptr(d_br[0]), _ptr(d_br[1]),
            _ptr(d_br[2]) if o_win is not None else None, _stream(dev)), "lsrm_gate_merge_bwd")
    return d_gate, d_br[0], d_br[1], (d_br[2] if o_win is not None else None)


# The functions above registered as torch operators (torch.ops.lsrm_hip.*).
from . import torch_ops  # noqa: E402,F401
