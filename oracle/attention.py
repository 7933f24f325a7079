"""Selected-block attention oracle (PyTorch fp32 on the CPU).

Restates forward_kernel_varblock
(sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:55-247) as dense
math: for kv head h and query i, the attended keys are the tokens of the
valid entries of topk_idx[h, i] (batch-local ids v with 0 <= v < blocks of
i's batch element, block cu_seqblocks[b] + v, list order, repeats count
twice, kvcentric:143-178); every query head of h's group uses them;
o = softmax(scale * q k^T) v and lse = log2(sum exp2(scale * log2(e) * q.k))
(log2 units, kvcentric:204-229).  A row with no valid entry gives o = 0,
lse = -inf (the reference divides 0 by 0 there).  Queries are grouped into
runs of identical rows so each run is one dense softmax.  The backward
(kvcentric:262-478, 687-923) is torch.autograd through this function, or
sel_attn_bwd_ref, the same gradients written out run by run so that memory
stays bounded at the benchmark sizes.
Pins: topk = every block reduces to full softmax attention
(torch.nn.functional.scaled_dot_product_attention); topk = own block reduces
to block-diagonal attention; a repeated block equals doubling its weight;
outputs are convex combinations of V; fp64 finite differences for the
backward; sel_attn_bwd_ref equals torch.autograd of sel_attn_ref
(tests/test_oracle_attention.py).
"""

from __future__ import annotations

import math
from typing import List, Tuple

import torch

LOG2E = 1.4426950408889634


def _row_runs(rows: torch.Tensor, starts: torch.Tensor) -> List[Tuple[int, int]]:
    """Runs of identical consecutive rows; `starts` marks forced run starts."""
    n = rows.shape[0]
    if n == 0:
        return []
    brk = torch.zeros(n, dtype=torch.bool)
    brk[0] = True
    if n > 1:
        brk[1:] = (rows[1:] != rows[:-1]).any(dim=1)
    brk |= starts
    idx = torch.nonzero(brk).flatten().tolist() + [n]
    return [(idx[j], idx[j + 1]) for j in range(len(idx) - 1)]


def normalized_rows(topk_idx: torch.Tensor, cu_seqblocks: torch.Tensor,
                    cu_seqlens_q: torch.Tensor):
    """Per-query batch-local validity: returns (rows with invalid -> -1,
    per-query block base, seq-start mask)."""
    hkv, nq, k = topk_idx.shape
    cu_q = cu_seqlens_q.to(torch.int64)
    cu_sb = cu_seqblocks.to(torch.int64)
    nbb = torch.zeros(nq, dtype=torch.int64)
    base = torch.zeros(nq, dtype=torch.int64)
    starts = torch.zeros(nq, dtype=torch.bool)
    for b in range(cu_q.numel() - 1):
        s, e = int(cu_q[b]), int(cu_q[b + 1])
        nbb[s:e] = int(cu_sb[b + 1] - cu_sb[b])
        base[s:e] = int(cu_sb[b])
        if e > s:
            starts[s] = True
    t = topk_idx.to(torch.int64)
    valid = (t >= 0) & (t < nbb.view(1, nq, 1))
    rows = torch.where(valid, t, torch.full_like(t, -1))
    return rows, base, starts


def sel_attn_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk_idx: torch.Tensor,
                 cu_seqblocks: torch.Tensor, cu_block_tokens: torch.Tensor,
                 cu_seqlens_q: torch.Tensor, scale: float):
    """q [Nq, Hq, D], k/v [Nk, Hkv, D] (fp32 or fp64, CPU; may require grad) ->
    (o [Nq, Hq, D], lse [Hq, Nq] log2 units), both in q's dtype."""
    nq, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    cu = cu_block_tokens.to(torch.int64)
    rows, base, starts = normalized_rows(topk_idx, cu_seqblocks, cu_seqlens_q)
    lse = torch.full((hq, nq), -math.inf, dtype=q.dtype)
    o = torch.zeros(nq, hq, d, dtype=q.dtype)
    pieces = []  # (h, a, b, o_run [L, G, D])
    for h in range(hkv):
        for a, b in _row_runs(rows[h], starts):
            sel = [int(x) for x in rows[h, a].tolist() if x >= 0]
            bb = int(base[a])
            spans = [torch.arange(int(cu[bb + c]), int(cu[bb + c + 1])) for c in sel]
            spans = [s for s in spans if s.numel() > 0]
            if not spans:
                continue
            kidx = torch.cat(spans)
            qr = q[a:b, h * g:(h + 1) * g, :].reshape(-1, d)
            kk = k.index_select(0, kidx)[:, h, :]
            vv = v.index_select(0, kidx)[:, h, :]
            s = (qr @ kk.transpose(0, 1)) * scale
            p = torch.softmax(s, dim=-1)
            orun = (p @ vv).view(b - a, g, d)
            pieces.append((h, a, b, orun))
            lse[h * g:(h + 1) * g, a:b] = (torch.logsumexp(s.detach(), dim=-1) * LOG2E).view(
                b - a, g).transpose(0, 1)
    # Slice assignment into a fresh tensor is differentiable (copy_ into views).
    for h, a, b, orun in pieces:
        o[a:b, h * g:(h + 1) * g, :] = orun
    return o, lse


def sel_attn_bwd_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor,
                     topk_idx: torch.Tensor, cu_seqblocks: torch.Tensor,
                     cu_block_tokens: torch.Tensor, cu_seqlens_q: torch.Tensor, scale: float):
    """Gradients of sel_attn_ref without an autograd graph -> (dq, dk, dv,
    delta [Hq, Nq]), all in q's dtype.

    Follows the reference's backward (kvcentric:263-478 for dQ with the fused
    Delta = sum_d O * dO at 387-404; kvcentric:688-923 for dK / dV): per run
    of identical rows, P = softmax(scale * q k^T), dP = dO v^T,
    dS = P * (dP - Delta) (kvcentric:462-463, 892-893), dQ = scale * dS k,
    dK += scale * dS^T q, dV += P^T dO, accumulated over every listing of a
    key (a repeated block contributes twice).  O here is the exact softmax
    output, not a rounded forward result."""
    nq, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    cu = cu_block_tokens.to(torch.int64)
    rows, base, starts = normalized_rows(topk_idx, cu_seqblocks, cu_seqlens_q)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    delta = torch.zeros(hq, nq, dtype=q.dtype)
    for h in range(hkv):
        dk_h = torch.zeros(k.shape[0], d, dtype=k.dtype)
        dv_h = torch.zeros(v.shape[0], d, dtype=v.dtype)
        for a, b in _row_runs(rows[h], starts):
            sel = [int(x) for x in rows[h, a].tolist() if x >= 0]
            bb = int(base[a])
            spans = [torch.arange(int(cu[bb + c]), int(cu[bb + c + 1])) for c in sel]
            spans = [s for s in spans if s.numel() > 0]
            if not spans:
                continue
            kidx = torch.cat(spans)
            qr = q[a:b, h * g:(h + 1) * g, :].reshape(-1, d)
            dor = do[a:b, h * g:(h + 1) * g, :].reshape(-1, d).to(q.dtype)
            kk = k.index_select(0, kidx)[:, h, :]
            vv = v.index_select(0, kidx)[:, h, :]
            p = torch.softmax((qr @ kk.transpose(0, 1)) * scale, dim=-1)
            dl = ((p @ vv) * dor).sum(-1)
            ds = p * (dor @ vv.transpose(0, 1) - dl[:, None])
            dq[a:b, h * g:(h + 1) * g, :] = (scale * (ds @ kk)).view(b - a, g, d)
            dk_h.index_add_(0, kidx, scale * (ds.transpose(0, 1) @ qr))
            dv_h.index_add_(0, kidx, p.transpose(0, 1) @ dor)
            delta[h * g:(h + 1) * g, a:b] = dl.view(b - a, g).transpose(0, 1)
        dk[:, h, :] = dk_h
        dv[:, h, :] = dv_h
    return dq, dk, dv, delta


def attended_pairs(topk_idx: torch.Tensor, cu_seqblocks: torch.Tensor,
                   cu_block_tokens: torch.Tensor, cu_seqlens_q: torch.Tensor) -> int:
    """Sum over kv heads and queries of the attended key count."""
    rows, base, _ = normalized_rows(topk_idx, cu_seqblocks, cu_seqlens_q)
    cu = cu_block_tokens.to(torch.int64)
    lens = cu[1:] - cu[:-1]
    gl = torch.where(rows >= 0, rows + base.view(1, -1, 1), torch.zeros_like(rows))
    a = torch.where(rows >= 0, lens[gl], torch.zeros_like(gl))
    return int(a.sum())
