"""CPU pins of the reverse (CSR) query map oracle (oracle/revmap.py), which
restates _build_reverse_query_mapping
(sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:575-684).
Pinned against a dict-of-lists build in pure Python and exact integer
invariants (counts sum to the valid entries; multiplicity preserved;
segments ascending)."""

from collections import defaultdict

import numpy as np
import pytest

from oracle.revmap import reverse_query_map_ref


def _dict_build(topk, cu_q, cu_sb, nb):
    hkv, nq, k = topk.shape
    out = []
    for h in range(hkv):
        d = defaultdict(list)
        for b in range(len(cu_q) - 1):
            nbb = cu_sb[b + 1] - cu_sb[b]
            for i in range(cu_q[b], cu_q[b + 1]):
                for j in range(k):
                    c = int(topk[h, i, j])
                    if 0 <= c < nbb:
                        d[cu_sb[b] + c].append(i)
        out.append({c: sorted(v) for c, v in d.items()})
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_matches_dict_build(seed):
    rng = np.random.default_rng(seed)
    nq, hkv, k = 60, 2, 4
    cu_q = [0, 25, 60]
    cu_sb = [0, 3, 8]
    topk = rng.integers(-1, 6, size=(hkv, nq, k)).astype(np.int32)
    topk[0, 3, :2] = 2                     # a query selecting one block twice
    cu_rev, lists = reverse_query_map_ref(topk, np.array(cu_q), np.array(cu_sb), 8)
    ref = _dict_build(topk, cu_q, cu_sb, 8)
    for h in range(hkv):
        for c in range(8):
            seg = lists[h][cu_rev[h, c]:cu_rev[h, c + 1]].tolist()
            assert seg == ref[h].get(c, []), (h, c)
            assert seg == sorted(seg)
        valid = sum(len(v) for v in ref[h].values())
        assert cu_rev[h, -1] == valid == len(lists[h])
    assert lists[0][cu_rev[0, 2]:cu_rev[0, 3]].tolist().count(3) == 2


def test_empty_selection():
    topk = np.full((1, 5, 3), -1, dtype=np.int32)
    cu_rev, lists = reverse_query_map_ref(topk, np.array([0, 5]), np.array([0, 2]), 2)
    assert (cu_rev == 0).all() and len(lists[0]) == 0
