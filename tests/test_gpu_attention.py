"""GPU parity: selected-block attention forward/backward against the fp32
CPU oracle (north_star tolerance: max-abs 2e-2, mean-abs 2e-3), the reverse
query map bit-exact, and the sparse.ops API surface."""

import math

import numpy as np
import pytest
import torch

import lsrm_hip as H
from helpers import assert_attn_close, random_topk
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_ref
from oracle.revmap import reverse_query_map_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _run_case(q, k, v, topk_idx, cu_sb, cu_blk, cu_q, scale, do=None):
    """HIP forward (and backward when do is given) vs the oracle."""
    dq_ = [t.to(DEV) for t in (q, k, v, topk_idx, cu_sb, cu_blk, cu_q)]
    o, lse = H.sel_attn_fwd(*dq_, scale)
    qf, kf, vf = (t.float().requires_grad_(do is not None) for t in (q, k, v))
    o_ref, lse_ref = sel_attn_ref(qf, kf, vf, topk_idx, cu_sb, cu_blk, cu_q, scale)
    assert_attn_close(o, o_ref, "out")
    lse_c = lse.cpu()
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse_c), fin)
    assert (lse_c[fin] - lse_ref[fin]).abs().max() <= 2e-2 if fin.any() else True
    if do is None:
        return o, lse
    dq, dk, dv, delta = H.sel_attn_bwd(do.to(DEV), *dq_[:3], o, lse, *dq_[3:], scale)
    o_ref.backward(do.float())
    assert_attn_close(dq, qf.grad, "dq")
    assert_attn_close(dk, kf.grad, "dk")
    assert_attn_close(dv, vf.grad, "dv")
    delta_ref = (o.float().cpu() * do.float()).sum(-1).transpose(0, 1)
    torch.testing.assert_close(delta.cpu(), delta_ref, rtol=1e-4, atol=1e-4)
    return o, lse, dq, dk, dv


def _blocks_topk(w, topk, gen):
    return random_topk(w.hkv, w.n, w.n_blocks, topk, gen, per_block_cu=w.cu_block_tokens)


def test_fwd_block_selection_cfg2_small():
    w = W.config(2, n=4096, heads=4)
    q, k, v = W.tensors(w, "cpu")
    gen = torch.Generator().manual_seed(11)
    topk = _blocks_topk(w, w.topk, gen)
    _run_case(q, k, v, topk, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale)


def test_fwd_from_select_blocks_cfg3_small():
    w = W.config(3, n=16384, heads=2)
    q, k, v = W.tensors(w, "cpu")
    topk_idx, _ = H.select_blocks(q.to(DEV), k.to(DEV), w.cu_seqblocks.to(DEV),
                                  w.cu_block_tokens.to(DEV), w.topk, w.forced_blocks, True)
    _run_case(q, k, v, topk_idx.cpu(), w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale)


@pytest.mark.parametrize("d,dtype", [(32, torch.bfloat16), (64, torch.float16), (128, torch.bfloat16)])
def test_fwd_gqa_per_token_rows(d, dtype):
    # Product shape family: Hq = 8 query heads over Hkv = 2 kv heads; every
    # token has its own selection row (the 3D-aware maps of the reference).
    n, hq, hkv = 1536, 8, 2
    rng = np.random.default_rng(5)
    sizes = W.uniform_partition(n, 8, 96, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    gen = torch.Generator().manual_seed(d)
    q = torch.randn(n, hq, d, generator=gen).to(dtype)
    k = torch.randn(n, hkv, d, generator=gen).to(dtype)
    v = torch.randn(n, hkv, d, generator=gen).to(dtype)
    topk = random_topk(hkv, n, len(sizes), 6, gen, pad_frac=0.5)
    cu_sb = torch.tensor([0, len(sizes)], dtype=torch.int32)
    cu_q = torch.tensor([0, n], dtype=torch.int32)
    _run_case(q, k, v, topk, cu_sb, cu, cu_q, 1.0 / math.sqrt(d))


def test_fwd_duplicates_empty_rows_and_batches():
    # Two batch elements; repeated ids, -1 padding, out-of-range ids and an
    # empty row (output 0, lse -inf).
    n0, n1, hq, d = 700, 500, 4, 64
    rng = np.random.default_rng(9)
    s0 = W.uniform_partition(n0, 16, 128, rng)
    s1 = W.uniform_partition(n1, 16, 128, rng)
    sizes = np.concatenate([s0, s1])
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    cu_sb = torch.tensor([0, len(s0), len(sizes)], dtype=torch.int32)
    cu_q = torch.tensor([0, n0, n0 + n1], dtype=torch.int32)
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(n0 + n1, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(n0 + n1, hq, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(n0 + n1, hq, d, generator=gen).to(torch.bfloat16)
    topk = torch.full((hq, n0 + n1, 5), -1, dtype=torch.int32)
    topk[:, :, 0] = 1
    topk[:, :, 1] = 1          # duplicate counts twice
    topk[:, :, 2] = 3
    topk[:, 10:20, :] = -1     # empty rows
    topk[:, n0 + 5, 0] = len(s1) + 7  # out of range for batch 1 -> ignored
    _run_case(q, k, v, topk, cu_sb, cu, cu_q, 0.125)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_fwd_token_map_boundary(d):
    # Run tiles whose key stream has at most 2048 positions read a position ->
    # token map; longer streams walk the segment list.  Block 0's queries
    # select 64 blocks of 32 keys (exactly 2048 positions), block 1's select
    # 63 of them and one of 33 in reverse order (2049), block 2's nothing,
    # block 3's three small blocks; the other rows list up to 64 blocks of
    # 1..40 keys (nearly every 8-key copy group crosses a block boundary),
    # with repeated ids and padding.
    hq, hkv, topk = 4, 2, 64
    rng = np.random.default_rng(d)
    sizes = np.concatenate([np.full(64, 32), [33], rng.integers(1, 41, size=235)])
    nb = len(sizes)
    n = int(sizes.sum())
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    rows = np.full((hkv, nb, topk), -1, dtype=np.int32)
    for h in range(hkv):
        for b in range(4, nb):
            m = int(rng.integers(1, topk + 1))
            ids = rng.integers(65, nb, size=m)
            if m > 3:
                ids[1] = ids[0]
            rows[h, b, :m] = ids
    rows[:, 0, :] = np.arange(64)
    rows[:, 1, :] = np.arange(64, 0, -1)
    rows[:, 3, :3] = [70, 65, 200]
    counts = np.diff(cu.numpy())
    topk_idx = torch.from_numpy(np.repeat(rows, counts, axis=1))
    keys = [int(sizes[r[r >= 0]].sum()) for r in rows[0, :4]]
    assert keys == [2048, 2049, 0, int(sizes[[70, 65, 200]].sum())]
    gen = torch.Generator().manual_seed(d + 1)
    q = torch.randn(n, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    cu_sb = torch.tensor([0, nb], dtype=torch.int32)
    cu_q = torch.tensor([0, n], dtype=torch.int32)
    # forward only: the map is the forward's (the backward walks the segments)
    _run_case(q, k, v, topk_idx, cu_sb, cu, cu_q, 1.0 / math.sqrt(d))


@pytest.mark.parametrize("topk", [32, 64])
def test_fwd_long_rows_runs_and_batch_boundary(topk):
    # Rows of 32 and more ids (the plan's row-comparison kernel reads them a
    # wave of lanes per few rows): identical rows either side of the batch
    # boundary still start a new run, rows that differ only in ids naming no
    # block of their batch element form one run, and other rows change every
    # few tokens.
    n0, n1, hq, d = 600, 520, 2, 64
    rng = np.random.default_rng(topk)
    s0 = W.uniform_partition(n0, 8, 64, rng)
    s1 = W.uniform_partition(n1, 8, 64, rng)
    sizes = np.concatenate([s0, s1])
    nb0, nb1 = len(s0), len(s1)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    cu_sb = torch.tensor([0, nb0, nb0 + nb1], dtype=torch.int32)
    cu_q = torch.tensor([0, n0, n0 + n1], dtype=torch.int32)
    n = n0 + n1
    m = min(nb0, nb1)
    rows = np.full((1, n, topk), -1, dtype=np.int32)
    t = 0
    while t < n:
        run = int(rng.integers(1, 9))
        ids = rng.integers(0, m, size=topk)
        ids[rng.random(topk) < 0.2] = -1
        rows[0, t:t + run] = ids
        t += run
    rows[0, n0 - 40:n0 + 40] = rows[0, n0 - 40]  # one row across the boundary
    rows[0, 100:140, topk - 1] = 10 ** 6          # out of range: same as -1
    rows[0, 100:140:2, topk - 1] = -1
    gen = torch.Generator().manual_seed(topk + 3)
    q = torch.randn(n, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(n, 1, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(n, 1, d, generator=gen).to(torch.bfloat16)
    _run_case(q, k, v, torch.from_numpy(rows), cu_sb, cu, cu_q, 0.125)


def test_bwd_cfg4_small():
    w = W.config(4, n=4096, heads=4)
    q, k, v, do = W.tensors(w, "cpu", with_grad_out=True)
    gen = torch.Generator().manual_seed(4)
    topk = _blocks_topk(w, w.topk, gen)
    _run_case(q, k, v, topk, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale, do=do)


def test_bwd_gqa_per_token_rows():
    n, hq, hkv, d = 1024, 8, 2, 32
    rng = np.random.default_rng(2)
    sizes = W.uniform_partition(n, 8, 80, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(n, hq, d, generator=gen).to(torch.bfloat16)
    k = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    v = torch.randn(n, hkv, d, generator=gen).to(torch.bfloat16)
    do = torch.randn(n, hq, d, generator=gen).to(torch.bfloat16)
    topk = random_topk(hkv, n, len(sizes), 5, gen, pad_frac=0.4)
    _run_case(q, k, v, topk, torch.tensor([0, len(sizes)], dtype=torch.int32), cu,
              torch.tensor([0, n], dtype=torch.int32), 1.0 / math.sqrt(d), do=do)


def test_deterministic_bitwise():
    w = W.config(4, n=4096, heads=2)
    q, k, v, do = (t.to(DEV) for t in W.tensors(w, "cpu", with_grad_out=True))
    gen = torch.Generator().manual_seed(8)
    topk = _blocks_topk(w, w.topk, gen).to(DEV)
    meta = [t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens)]
    runs = []
    for _ in range(2):
        o, lse = H.sel_attn_fwd(q, k, v, topk, *meta, w.scale)
        dq, dk, dv, _ = H.sel_attn_bwd(do, q, k, v, o, lse, topk, *meta, w.scale)
        runs.append([t.clone() for t in (o, lse, dq, dk, dv)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_reverse_query_map_bitexact():
    w = W.config(2, n=3000, heads=3)
    gen = torch.Generator().manual_seed(6)
    topk = random_topk(w.hkv, w.n, w.n_blocks, 7, gen, pad_frac=0.3)
    topk[:, 5, 1] = topk[:, 5, 0]  # a duplicate
    cu_rev, rev = H.reverse_query_map(topk.to(DEV), w.cu_seqlens.to(DEV), w.cu_seqblocks.to(DEV),
                                      w.n_blocks)
    ref_cu, ref_lists = reverse_query_map_ref(topk.numpy(), w.cu_seqlens.numpy(),
                                              w.cu_seqblocks.numpy(), w.n_blocks)
    np.testing.assert_array_equal(cu_rev.cpu().numpy(), ref_cu)
    for h in range(w.hkv):
        m = int(ref_cu[h, -1])
        np.testing.assert_array_equal(rev[h, :m].cpu().numpy(), ref_lists[h])


def test_reverse_query_map_long_segments():
    # One block selected by every query: a segment longer than the in-LDS
    # sort capacity exercises the windowed counting sort.
    n, nb = 12000, 4
    cu_q = torch.tensor([0, n], dtype=torch.int32)
    cu_sb = torch.tensor([0, nb], dtype=torch.int32)
    gen = torch.Generator().manual_seed(0)
    topk = torch.zeros(1, n, 2, dtype=torch.int32)
    topk[0, :, 1] = torch.randint(1, nb, (n,), generator=gen).to(torch.int32)
    cu_rev, rev = H.reverse_query_map(topk.to(DEV), cu_q.to(DEV), cu_sb.to(DEV), nb)
    ref_cu, ref_lists = reverse_query_map_ref(topk.numpy(), cu_q.numpy(), cu_sb.numpy(), nb)
    np.testing.assert_array_equal(cu_rev.cpu().numpy(), ref_cu)
    np.testing.assert_array_equal(rev[0, : int(ref_cu[0, -1])].cpu().numpy(), ref_lists[0])


@pytest.mark.parametrize("mode", ["large", "all_negative"])
def test_fwd_bwd_extreme_scores(mode):
    # Scores far outside the kernel's zero-reference window (|s| >> 64 in
    # log2 units) move the softmax reference; outputs must stay exact.
    w = W.config(2, n=2048, heads=2)
    gen = torch.Generator().manual_seed(21)
    if mode == "large":
        q = 4.0 * torch.randn(w.n, w.hq, w.d, generator=gen)
        k = 4.0 * torch.randn(w.n, w.hkv, w.d, generator=gen)
    else:
        u = torch.randn(1, 1, w.d, generator=gen)
        q = 4.0 * u + 0.05 * torch.randn(w.n, w.hq, w.d, generator=gen)
        k = -4.0 * u + 0.05 * torch.randn(w.n, w.hkv, w.d, generator=gen)
    v = torch.randn(w.n, w.hkv, w.d, generator=gen)
    do = torch.randn(w.n, w.hq, w.d, generator=gen)
    q, k, v, do = (t.to(torch.bfloat16) for t in (q, k, v, do))
    topk = _blocks_topk(w, 8, gen)
    if mode == "large":
        # only the forward: dS magnitudes make a fixed absolute tolerance
        # meaningless for the gradients at these logit scales
        _run_case(q, k, v, topk, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale)
    else:
        _run_case(q, k, v, topk, w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens, w.scale,
                  do=do)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fwd_later_blocks_dominate(dtype):
    # Every query lists a weak block first (K scaled down) and strong blocks
    # after it, so the row maxima of later key tiles exceed the first tile's
    # by ~17 log2 units: unnormalised probabilities reach 2^17, which bf16
    # holds and fp16 overflows (the kernel must then take its exact online
    # pass).  Outputs must match the oracle either way.
    n, bl, hkv, d, topk_n = 2048, 128, 2, 64, 4
    nb = n // bl
    gen = torch.Generator().manual_seed(31)
    cu_blk = torch.arange(0, n + 1, bl, dtype=torch.int32)
    cu_sb = torch.tensor([0, nb], dtype=torch.int32)
    cu_q = torch.tensor([0, n], dtype=torch.int32)
    q = 2.0 * torch.randn(n, hkv, d, generator=gen)
    k = 2.0 * torch.randn(n, hkv, d, generator=gen)
    k[:bl] *= 0.02
    v = torch.randn(n, hkv, d, generator=gen)
    topk = torch.randint(1, nb, (hkv, n, topk_n), generator=gen).to(torch.int32)
    topk[:, :, 0] = 0
    q, k, v = (t.to(dtype) for t in (q, k, v))
    _run_case(q, k, v, topk, cu_sb, cu_blk, cu_q, 1.0 / math.sqrt(d))


@pytest.mark.parametrize("per_token", [False, True])
def test_bwd_head_dim_128(per_token):
    # head dim 128 takes the dQ and dK/dV bodies sized for it (run tiles and
    # grouped per-token tiles alike)
    n, hq, hkv, d = 1536, 4, 2, 128
    rng = np.random.default_rng(12)
    sizes = W.uniform_partition(n, 16, 160, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    gen = torch.Generator().manual_seed(13)
    q = (0.5 * torch.randn(n, hq, d, generator=gen)).to(torch.bfloat16)
    k = (0.5 * torch.randn(n, hkv, d, generator=gen)).to(torch.bfloat16)
    v = (0.5 * torch.randn(n, hkv, d, generator=gen)).to(torch.bfloat16)
    do = (0.5 * torch.randn(n, hq, d, generator=gen)).to(torch.bfloat16)
    if per_token:
        topk = random_topk(hkv, n, len(sizes), 5, gen, pad_frac=0.3)
    else:
        topk = random_topk(hkv, n, len(sizes), 5, gen, per_block_cu=cu)
    _run_case(q, k, v, topk, torch.tensor([0, len(sizes)], dtype=torch.int32), cu,
              torch.tensor([0, n], dtype=torch.int32), 1.0 / math.sqrt(d), do=do)


def test_bwd_run_rejects_forward_only_plan():
    # A forward-only plan (no reverse maps) in a workspace sized for the
    # backward: lsrm_sel_attn_bwd_run's kernels see the missing backward
    # marker and leave every output untouched; the same workspace replanned
    # with backward=1 then gives the normal gradients.
    w = W.config(4, n=2048, heads=2)
    q, k, v, do = (t.to(DEV) for t in W.tensors(w, "cpu", with_grad_out=True))
    gen = torch.Generator().manual_seed(3)
    topk = _blocks_topk(w, w.topk, gen).to(DEV)
    cu_sb, cu_blk, cu_q = (t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens))
    o, lse = H.sel_attn_fwd(q, k, v, topk, cu_sb, cu_blk, cu_q, w.scale)
    lib = H.lib()
    nb, n = w.n_blocks, w.n
    ws_n = lib.lsrm_sel_attn_workspace_size(n, n, w.hq, w.hkv, w.topk, nb, 1)
    ws = torch.empty(ws_n, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    outs = [torch.full_like(q, 7.0), torch.full_like(k, 7.0), torch.full_like(v, 7.0),
            torch.full((w.hq, n), 7.0, device=DEV)]

    def bwd_run():
        return lib.lsrm_sel_attn_bwd_run(
            do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            lse.data_ptr(), H.BF16, n, n, w.hq, w.hkv, w.d, topk.data_ptr(), w.topk,
            cu_sb.data_ptr(), cu_blk.data_ptr(), nb, cu_q.data_ptr(), 1, w.scale,
            *[t.data_ptr() for t in outs], ws.data_ptr(), ws_n, stream)

    for backward in (1, 0):  # a backward plan first, then a forward-only one over it
        assert lib.lsrm_sel_attn_plan(topk.data_ptr(), n, n, w.hq, w.hkv, w.topk,
                                      cu_sb.data_ptr(), cu_blk.data_ptr(), nb, cu_q.data_ptr(),
                                      1, backward, ws.data_ptr(), ws_n, stream) == 0
    assert bwd_run() == 0
    torch.cuda.synchronize()
    for t in outs:
        assert (t == 7.0).all()
    assert lib.lsrm_sel_attn_plan(topk.data_ptr(), n, n, w.hq, w.hkv, w.topk, cu_sb.data_ptr(),
                                  cu_blk.data_ptr(), nb, cu_q.data_ptr(), 1, 1, ws.data_ptr(),
                                  ws_n, stream) == 0
    outs[1].zero_()
    outs[2].zero_()
    assert bwd_run() == 0
    dq, dk, dv, delta = H.sel_attn_bwd(do, q, k, v, o, lse, topk, cu_sb, cu_blk, cu_q, w.scale)
    for a, b in zip(outs, (dq, dk, dv, delta)):
        assert torch.equal(a, b)
