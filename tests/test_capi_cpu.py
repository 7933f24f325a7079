"""CPU checks of the C-ABI boundary and the host layer: liblsrm_hip.so loads,
exports every entry point include/lsrm_hip.h declares, the ctypes binding
covers them, host-only queries answer, and the product path refuses CPU
tensors instead of falling back to a CPU implementation."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import lsrm_hip as H

HEADER = Path(__file__).resolve().parents[1] / "include" / "lsrm_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lsrm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    for must in ("lsrm_block_mean_pool", "lsrm_select_blocks", "lsrm_sel_attn_fwd",
                 "lsrm_sel_attn_bwd", "lsrm_reverse_query_map", "lsrm_sel_attn_plan"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not H.LIB_PATH.exists():
        pytest.skip("liblsrm_hip.so not built (run __graft_entry__.build())")
    raw = ctypes.CDLL(str(H.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(raw, n)]
    assert not missing, missing
    assert sorted(H.exported_symbols()) == _declared()


def test_host_queries():
    if not H.LIB_PATH.exists():
        pytest.skip("liblsrm_hip.so not built")
    lib = H.lib()
    assert lib.lsrm_version() >= 100
    assert lib.lsrm_status_string(0) == b"ok"
    assert b"workspace" in lib.lsrm_status_string(3)
    assert lib.lsrm_sel_attn_workspace_size(131072, 131072, 24, 24, 16, 462, 0) > 0
    bwd = lib.lsrm_sel_attn_workspace_size(4096, 4096, 4, 4, 16, 40, 1)
    fwd = lib.lsrm_sel_attn_workspace_size(4096, 4096, 4, 4, 16, 40, 0)
    assert bwd > fwd > 0
    assert lib.lsrm_sel_attn_workspace_size(10, 10, 3, 2, 4, 2, 0) == 0  # hq % hkv != 0
    assert lib.lsrm_block_mean_pool_workspace_size(1000, 64, 10) >= 0
    assert lib.lsrm_select_blocks_workspace_size(1000, 10, 4, 4, 64) > 0


def test_invalid_arguments_rejected_without_device():
    if not H.LIB_PATH.exists():
        pytest.skip("liblsrm_hip.so not built")
    lib = H.lib()
    # unsupported head_dim / dtype are refused before any device work
    rc = lib.lsrm_sel_attn_fwd(None, None, None, 2, 10, 10, 2, 2, 48, None, 4, None, None, 2,
                               None, 1, 0.1, None, None, None, 0, None)
    assert rc == 2
    rc = lib.lsrm_sel_attn_fwd(None, None, None, 0, 10, 10, 2, 2, 64, None, 4, None, None, 2,
                               None, 1, 0.1, None, None, None, 0, None)
    assert rc == 2
    rc = lib.lsrm_sel_attn_fwd(None, None, None, 2, 10, 10, 2, 2, 64, None, 4, None, None, 2,
                               None, 1, 0.1, None, None, None, 0, None)
    assert rc == 1   # null pointers


def test_no_cpu_fallback():
    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        H.block_mean_pool(q.view(8, -1), cu)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        H.sel_attn_fwd(q, q, q, torch.zeros(2, 8, 1, dtype=torch.int32), torch.tensor([0, 1]),
                       cu, cu, 0.125)


def test_reference_api_asserts_dtypes_on_cpu():
    import sparse.ops as ops

    q = torch.zeros(8, 2, 64)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(AssertionError):
        ops.native_sparse_attend(q, q, q, torch.zeros(2, 8, 1, dtype=torch.int32),
                                 torch.tensor([0, 1], dtype=torch.int32), cu, cu, cu)


def test_attention_entries_refuse_host_tensors_before_any_launch():
    # Every attention entry point checks devices, dtypes and shapes before a
    # pointer reaches the C ABI; a CPU dO on the key-centric backward path
    # raises like everywhere else.
    import lsrm_hip as H

    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    rows = torch.zeros(2, 8, 1, dtype=torch.int32)
    lse = torch.zeros(2, 8)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    cu_blk = torch.tensor([0, 8], dtype=torch.int32)
    cu_q = torch.tensor([0, 8], dtype=torch.int32)
    for kc in (True, False):
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            H.sel_attn_bwd(q, q, k, k, q, lse, rows, cu, cu_blk, cu_q, 0.125, key_centric=kc)
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            H.sel_attn_fwd(q, k, k, rows, cu, cu_blk, cu_q, 0.125, key_centric=kc)


def test_key_centric_partials_bounded_to_one_gib():
    # The key-centric plan's partial results (Hq * N * topk * (2D + 4) bytes
    # when all of them fit) stay within 1 GiB: beyond it the plan runs in
    # passes and holds one pass's partials.  The rest of the key-centric part
    # (block -> query map with slots, its sort buffers, per-pass item lists)
    # grows with Hkv * N * topk, not with D or the query heads.
    if not H.LIB_PATH.exists():
        pytest.skip("liblsrm_hip.so not built")
    lib = H.lib()
    gib = 1 << 30

    def extra(n, hq, hkv, d, topk, nb):
        kc = lib.lsrm_sel_attn_workspace_size2(n, n, hq, hkv, d, topk, nb, 2)
        plain = lib.lsrm_sel_attn_workspace_size2(n, n, hq, hkv, d, topk, nb, 0)
        assert kc > plain > 0
        return kc - plain

    # small: every partial fits, so the plan holds all of them
    n, hq, d, topk = 4096, 4, 64, 8
    assert extra(n, hq, hq, d, topk, 40) >= hq * n * topk * (2 * d + 4)
    # config 3 (6.6 GB unbounded) and LSRM's heads (Hq=32, Hkv=2, D=32: 4.6 GB)
    for args in ((131072, 24, 24, 64, 16, 462), (131072, 32, 2, 32, 16, 462)):
        n, hq, hkv, d, topk, nb = args
        assert hq * n * topk * (2 * d + 4) > 4 * gib
        e = extra(*args)
        maps = hkv * n * topk * 4 * 6  # the listing map, its sort keys and buffers (bound)
        assert gib <= e <= gib + maps + 64 * (1 << 20), (args, e / gib)
