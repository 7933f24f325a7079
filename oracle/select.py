"""Per-query-block top-k block selection oracle.

No reference function implements this rule (the benchmark defines it); the
nearest reference analogue is get_block_score (sparse/ops/block_score.py:16-98),
whose output layout ([Hkv, Nq, topk] int32, ascending, -1 padded, lines
61-63 and 94-96) is kept.  Rule:
  * pooled means pq [nb, Hq, D], pk [nb, Hkv, D] in fp32 (oracle/pool.py);
  * score(b, c) for kv head h = sum over the G = Hq/Hkv query heads g of h,
    then over d, of float64(pq[b, hG+g, d]) * float64(pk[c, h, d]),
    accumulated in that order (the products are exact in fp64);
  * candidates: the blocks of b's batch element; NaN scores rank lowest;
  * forced first: b itself (force_self), then forced ids in order, skipping
    duplicates and out-of-range ids, truncated to topk;
  * remaining slots: best (score descending, block id ascending);
  * the row lists the chosen batch-local ids ascending, -1 padded.
Pins: brute force with Python float arithmetic on tiny inputs; topk >= nb
selects everything; identical pooled keys tie to the lowest ids; forced ids
always present; constructed inputs with a known ranking
(tests/test_oracle_select.py).
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np


def block_scores_ref(pq: np.ndarray, pk: np.ndarray, h: int) -> np.ndarray:
    """fp64 score matrix [nbq, nbk] for kv head h (sequential over g, d).

    Rows are computed in chunks (cache-sized temporaries); every element is
    still the sum over g, then d, of exact fp64 products, in that order."""
    hq, hkv = pq.shape[1], pk.shape[1]
    g_n = hq // hkv
    d = pq.shape[2]
    nbq, nbk = pq.shape[0], pk.shape[0]
    kt = np.ascontiguousarray(pk[:, h, :].astype(np.float64).T)  # [d, nbk]
    s = np.empty((nbq, nbk), dtype=np.float64)
    chunk = max(1, (1 << 17) // max(nbk, 1))
    for r0 in range(0, nbq, chunk):
        r1 = min(nbq, r0 + chunk)
        acc = np.zeros((r1 - r0, nbk), dtype=np.float64)
        for g in range(g_n):
            a = pq[r0:r1, h * g_n + g, :].astype(np.float64)
            for dd in range(d):
                acc += a[:, dd, None] * kt[dd][None, :]
        s[r0:r1] = acc
    return s


def _best_remaining(row: np.ndarray, chosen: list, need: int) -> list:
    """The `need` best ids of `row` outside `chosen` by (score descending, id
    ascending): every id scoring above the need-th best remaining score,
    then the lowest ids among those equal to it."""
    nbb = row.shape[0]
    avail = np.ones(nbb, dtype=bool)
    avail[chosen] = False
    ids = np.nonzero(avail)[0]
    vals = row[ids]
    if need >= ids.shape[0]:
        return ids.tolist()
    thr = np.partition(vals, ids.shape[0] - need)[ids.shape[0] - need]
    above = ids[vals > thr]
    tied = ids[vals == thr]
    return above.tolist() + tied[: need - above.shape[0]].tolist()


def select_blocks_ref(pq: np.ndarray, pk: np.ndarray, cu_seqblocks: np.ndarray, topk: int,
                      forced: Optional[Sequence[int]] = None,
                      force_self: bool = True) -> np.ndarray:
    """-> compact selection [Hkv, nb, topk] int32 (batch-local ids)."""
    nb = pq.shape[0]
    hkv = pk.shape[1]
    forced = list(forced or [])
    out = np.full((hkv, nb, topk), -1, dtype=np.int32)
    cu_sb = np.asarray(cu_seqblocks, dtype=np.int64)
    for e in range(cu_sb.shape[0] - 1):
        cs, ce = int(cu_sb[e]), int(cu_sb[e + 1])
        nbb = ce - cs
        if nbb <= 0:
            continue
        kmax = min(topk, nbb)
        for h in range(hkv):
            s = block_scores_ref(pq[cs:ce], pk[cs:ce], h)
            s = np.where(np.isnan(s), -np.inf, s)
            for b in range(nbb):
                chosen = []
                cand_forced = ([b] if force_self else []) + forced
                for f in cand_forced:
                    if len(chosen) >= kmax:
                        break
                    if 0 <= f < nbb and f not in chosen:
                        chosen.append(f)
                if len(chosen) < kmax:
                    chosen += _best_remaining(s[b], chosen, kmax - len(chosen))
                out[h, cs + b, :kmax] = np.sort(np.asarray(chosen, dtype=np.int32))
    return out


def expand_per_token(compact: np.ndarray, cu_block_tokens: np.ndarray, n: int) -> np.ndarray:
    """[Hkv, nb, topk] per-block rows -> [Hkv, n, topk] per-token rows."""
    hkv, nb, topk = compact.shape
    out = np.full((hkv, n, topk), -1, dtype=np.int32)
    cu = np.asarray(cu_block_tokens, dtype=np.int64)
    for b in range(nb):
        s, e = max(int(cu[b]), 0), min(int(cu[b + 1]), n)
        if e > s:
            out[:, s:e, :] = compact[:, b:b + 1, :]
    return out
