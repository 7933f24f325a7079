"""Learned block selection oracle (get_block_score) and compressed attention.

Restates get_block_score (sparse/ops/block_score.py:16-98): for every query
token i of batch element b and kv head h, over the compressed keys c of b
(compressed_cu_seqlens[b] .. compressed_cu_seqlens[b+1], batch-local index
c - compressed_cu_seqlens[b]),
    score(i, c) = sum over the G = Hq/Hkv query heads g of h of
                  2 ** (q[i, hG+g] . ck[c, h] * qk_scale - lse[hG+g, i] * 1.44269504)
with qk_scale = sm_scale * 1.44269504 (lines 53-56, 87-92; the constant
1.44269504 is the reference's, not log2(e) to full precision);
real_topk = min(topk, n_compressed) best blocks (line 76, 94), listed
ascending (line 95), the row padded with -1 (lines 61-63); a batch element
with no compressed keys gives all -1 (lines 73-74).

Evaluation here is in float64 with the dot product summed over d in order
(fp32 x fp32 products are exact in float64).  Ranking: score descending,
index ascending among equal scores; NaN scores rank below every number.
The reference ranks with torch.topk, whose order among equal scores is
unspecified; the GPU kernel evaluates in fp32, so the GPU tests accept a
different choice only between scores within a relative 1e-4 of the
real_topk-th best (near-ties).

compressed_attention_ref restates the dense flash_attn_varlen_func call of
SpatialSparseAttentionMid.forward (sparse/module/spatial_sparse_attention.py:
121-131, causal=False): every query attends to all compressed keys of its
batch element; the LSE is returned in natural-log units [Hq, Nq] as
flash-attn returns it.

Pins (tests/test_oracle_block_score.py): a pure-Python brute force with
math.pow on tiny inputs; G = 1 reduces to top-k by the dot product (exp2 and
the per-row lse shift are monotone); a constructed GQA case whose group sum
ranks a block that neither head ranks first alone (a dropped head term
fails); a constructed case where dropping the lse term or using natural-log
units changes the ranking; topk >= n_compressed selects every block;
batch-local ids and empty batch elements; compressed attention equals
torch.nn.functional.scaled_dot_product_attention per batch element and its
LSE equals torch.logsumexp of the scaled logits.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch

LOG2E_REF = 1.44269504  # the constant of sparse/ops/block_score.py:53-56


def block_score_matrix_ref(q: np.ndarray, ck: np.ndarray, lse: np.ndarray, h: int,
                           sm_scale: float) -> np.ndarray:
    """float64 scores [nq, nc] of kv head h: q [nq, Hq, D], ck [nc, Hkv, D],
    lse [Hq, nq] (natural log)."""
    hq, hkv = q.shape[1], ck.shape[1]
    g_n = hq // hkv
    qk_scale = float(sm_scale) * LOG2E_REF
    kk = ck[:, h, :].astype(np.float64)
    s = np.zeros((q.shape[0], ck.shape[0]), dtype=np.float64)
    for g in range(g_n):
        qq = q[:, h * g_n + g, :].astype(np.float64)
        dot = np.zeros_like(s)
        for dd in range(q.shape[2]):
            dot = dot + qq[:, dd, None] * kk[None, :, dd]
        l2 = lse[h * g_n + g, :].astype(np.float64) * LOG2E_REF
        s = s + np.exp2(dot * qk_scale - l2[:, None])
    return s


def topk_rows_ref(s: np.ndarray, k: int) -> np.ndarray:
    """Best k columns of every row of s under (score desc, index asc, NaN
    last), listed ascending -> [rows, k] int64."""
    key = np.where(np.isnan(s), -np.inf, s)
    nan_rank = np.isnan(s)
    out = np.empty((s.shape[0], k), dtype=np.int64)
    cols = np.arange(s.shape[1])
    for r in range(s.shape[0]):
        order = np.lexsort((cols, -key[r], nan_rank[r]))
        out[r] = np.sort(order[:k])
    return out


def get_block_score_ref(q: np.ndarray, compressed_k: np.ndarray, lse: np.ndarray, topk: int,
                        cu_seqlens_q: np.ndarray, compressed_cu_seqlens: np.ndarray,
                        sm_scale: Optional[float] = None,
                        return_scores: bool = False):
    """-> block_topk [Hkv, Nq, topk] int32 (and, with return_scores, a list
    of (kv head, q_s, q_e, scores [q_len, n_compressed] float64) per batch
    element)."""
    q = np.asarray(q, dtype=np.float32)
    ck = np.asarray(compressed_k, dtype=np.float32)
    lse = np.asarray(lse, dtype=np.float32)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    hkv = ck.shape[1]
    nq = q.shape[0]
    out = np.full((hkv, nq, topk), -1, dtype=np.int32)
    cu_q = np.asarray(cu_seqlens_q, dtype=np.int64)
    cu_c = np.asarray(compressed_cu_seqlens, dtype=np.int64)
    scores = []
    for b in range(cu_q.shape[0] - 1):
        qs, qe = int(cu_q[b]), int(cu_q[b + 1])
        ks, ke = int(cu_c[b]), int(cu_c[b + 1])
        nc = ke - ks
        if nc <= 0 or qe <= qs:
            continue
        kk = min(topk, nc)
        for h in range(hkv):
            s = block_score_matrix_ref(q[qs:qe], ck[ks:ke], lse[:, qs:qe], h, sm_scale)
            out[h, qs:qe, :kk] = topk_rows_ref(s, kk).astype(np.int32)
            if return_scores:
                scores.append((h, qs, qe, s))
    if return_scores:
        return out, scores
    return out


def compressed_attention_ref(q: torch.Tensor, ck: torch.Tensor, cv: torch.Tensor,
                             cu_seqlens_q: torch.Tensor, compressed_cu_seqlens: torch.Tensor,
                             sm_scale: Optional[float] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dense non-causal varlen attention in fp32 on the CPU -> (o [Nq, Hq, D],
    lse [Hq, Nq] natural log).  A batch element without compressed keys
    gives o = 0 and lse = -inf.  Differentiable through torch autograd."""
    q, ck, cv = q.float(), ck.float(), cv.float()
    nq, hq, d = q.shape
    hkv = ck.shape[1]
    g_n = hq // hkv
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    outs, lses = [], []
    cu_q = cu_seqlens_q.tolist()
    cu_c = compressed_cu_seqlens.tolist()
    for b in range(len(cu_q) - 1):
        qs, qe, ks, ke = cu_q[b], cu_q[b + 1], cu_c[b], cu_c[b + 1]
        qb = q[qs:qe].permute(1, 0, 2)                                # [Hq, L, D]
        if ke <= ks:
            outs.append(torch.zeros(qe - qs, hq, d))
            lses.append(torch.full((hq, qe - qs), -math.inf))
            continue
        kb = ck[ks:ke].permute(1, 0, 2).repeat_interleave(g_n, dim=0)  # [Hq, C, D]
        vb = cv[ks:ke].permute(1, 0, 2).repeat_interleave(g_n, dim=0)
        logits = torch.matmul(qb, kb.transpose(1, 2).contiguous()) * sm_scale
        lse_b = torch.logsumexp(logits, dim=-1)                          # [Hq, L]
        p = torch.exp(logits - lse_b[..., None])
        outs.append(torch.matmul(p, vb).permute(1, 0, 2))
        lses.append(lse_b)
    return torch.cat(outs, 0), torch.cat(lses, 1)
