"""GPU parity of the key-centric forward (plan flag LSRM_PLAN_KEY_CENTRIC):
the queries of per-token rows (learned selections, 3D-aware maps) that fall
in grouped tiles run as per-block gathered tiles whose partial results are
merged in row order.  Checked
against the fp32 oracle at the attention tolerance (output and LSE), against
the grouped-tile path, for run-to-run bitwise repeatability, and together
with the backward on the same plan."""

import numpy as np
import pytest
import torch

import lsrm_hip as H
import sparse.ops as ops
from helpers import assert_attn_close
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_bwd_ref, sel_attn_ref
from oracle.select3d import nearest_blocks_ref, volume_points_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _random_rows(n=6000, hq=2, hkv=2, topk=12, seed=4, d=64, dtype=torch.bfloat16,
                 sizes=(4, 17)):
    """Blocks of 4..16 tokens (about n / 10 of them) with unrelated random rows
    per token, as learned selections on unstructured data: 96 consecutive
    queries list several hundred distinct blocks; the grouped tiles go to the
    key-centric pass.  -1 padding,
    out-of-range ids and empty rows included."""
    rng = np.random.default_rng(seed)
    sizes = rng.integers(sizes[0], sizes[1], size=n // sizes[0])
    cu = np.concatenate([[0], np.cumsum(sizes)])
    cu = cu[cu <= n]
    cu[-1] = n
    nb = len(cu) - 1
    g = torch.Generator().manual_seed(seed)
    q = (0.5 * torch.randn(n, hq, d, generator=g)).to(dtype)
    k = (0.5 * torch.randn(n, hkv, d, generator=g)).to(dtype)
    v = (0.5 * torch.randn(n, hkv, d, generator=g)).to(dtype)
    rows = torch.randint(0, nb, (hkv, n, topk), generator=g, dtype=torch.int32)
    rows[:, ::5, topk - 3:] = -1
    rows[:, 1::7, 3] = nb + 5
    rows[:, 2::11, :] = -1
    return (q, k, v, rows, torch.tensor([0, nb], dtype=torch.int32),
            torch.from_numpy(cu.astype(np.int32)), torch.tensor([0, n], dtype=torch.int32))


def _fwd(args, key_centric, scale=0.125):
    dev_args = [t.to(DEV) for t in args]
    return H.sel_attn_fwd(*dev_args, scale, key_centric=key_centric)


def _check_oracle(args, o, lse, scale=0.125):
    q, k, v, rows, cu_sb, cu_blk, cu_q = args
    o_ref, lse_ref = sel_attn_ref(q.float(), k.float(), v.float(), rows, cu_sb, cu_blk, cu_q,
                                  scale)
    assert_attn_close(o, o_ref, "out")
    lse_c = lse.cpu()
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse_c), fin)
    if fin.any():
        assert float((lse_c[fin] - lse_ref[fin]).abs().max()) <= 2e-2


def test_random_rows_match_oracle_and_grouped_path():
    args = _random_rows()
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)
    o2, lse2 = _fwd(args, False)
    assert_attn_close(o, o2.float().cpu(), "out vs grouped tiles")
    # the two paths round differently: equal bits would mean no tile was
    # gathered
    assert not torch.equal(o, o2)


def test_random_rows_bitwise_repeatable():
    args = _random_rows(seed=5)
    a = _fwd(args, True)
    b = _fwd(args, True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_duplicate_ids_count_twice():
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(seed=6)
    rows = rows.clone()
    rows[:, ::3, 1] = rows[:, ::3, 0]      # the same block listed twice
    rows[:, 1::4, 2] = rows[:, 1::4, 0]
    rows[:, 1::4, 5] = rows[:, 1::4, 0]    # three times
    args = (q, k, v, rows, cu_sb, cu_blk, cu_q)
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)


@pytest.mark.parametrize("hq,hkv,d,topk", [(8, 2, 64, 8), (32, 2, 32, 4), (2, 2, 128, 8)])
def test_gqa_and_head_dims(hq, hkv, d, topk):
    args = _random_rows(n=3000, hq=hq, hkv=hkv, d=d, topk=topk, seed=7)
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)


def test_fp16_and_empty_blocks():
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(n=3000, seed=8, dtype=torch.float16)
    # blocks 3 and 4 hold no tokens (block 5 takes theirs): their listings
    # contribute nothing
    cu = cu_blk.clone()
    cu[4] = cu[3]
    cu[5] = cu[3]
    rows = rows.clone()
    rows[:, ::2, 0] = 3
    rows[:, ::4, 1] = 4
    args = (q, k, v, rows, cu_sb, cu, cu_q)
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)


def test_two_batch_elements():
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(n=3000, seed=9)
    n = q.shape[0]
    nb = cu_blk.numel() - 1
    args = (torch.cat([q, q]), torch.cat([k, k]), torch.cat([v, v]),
            torch.cat([rows, rows.flip(1)], dim=1).contiguous(),
            torch.tensor([0, nb, 2 * nb], dtype=torch.int32),
            torch.cat([cu_blk, cu_blk[1:] + n]),
            torch.tensor([0, n, 2 * n], dtype=torch.int32))
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)


def test_block_rows_unchanged_by_the_flag():
    # Rows shared by the 128 queries of each block (block-level selection):
    # every tile is a full run tile, none is grouped, so the gathered pass
    # has no work and the result is the same bits.
    nb, blk, topk = 40, 128, 8
    n = nb * blk
    g = torch.Generator().manual_seed(12)
    per_block = torch.stack([torch.randperm(nb, generator=g)[:topk] for _ in range(nb)])
    rows = per_block.repeat_interleave(blk, dim=0).to(torch.int32)
    rows = torch.stack([rows, rows.flip(1)]).contiguous()
    q, k, v = ((0.5 * torch.randn(n, 2, 64, generator=g)).to(torch.bfloat16) for _ in range(3))
    args = (q, k, v, rows, torch.tensor([0, nb], dtype=torch.int32),
            torch.arange(0, n + 1, blk, dtype=torch.int32), torch.tensor([0, n], dtype=torch.int32))
    a = _fwd(args, True)
    b = _fwd(args, False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _aware_rows(heads=2, seed=12):
    # 3D-aware rows of cfg3-style voxel tokens (blocks of 32..512 Morton-
    # ordered voxels): each token's nearest 16 block centroids.
    w = W.config(3, n=16384, heads=heads)
    nv = w.voxel_coords.shape[0]
    cu_all = w.cu_block_tokens.numpy().astype(np.int64)
    cu_v = (cu_all[w.n_image_blocks:] - cu_all[w.n_image_blocks]).astype(np.int32)
    coords = np.concatenate([np.zeros((nv, 1), np.int64), w.voxel_coords], axis=1)
    pts = volume_points_ref(coords, 64, 1.0)
    sel = nearest_blocks_ref(pts, cu_v, np.array([0, len(cu_v) - 1]), np.array([0, nv]), 16)
    rows = torch.from_numpy(np.broadcast_to(sel, (heads, nv, 16)).copy())
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((0.5 * torch.randn(nv, heads, 64, generator=g)).to(torch.bfloat16)
               for _ in range(3))
    return (q, k, v, rows, torch.tensor([0, len(cu_v) - 1], dtype=torch.int32),
            torch.from_numpy(cu_v), torch.tensor([0, nv], dtype=torch.int32))


def test_3d_aware_rows_take_the_gathered_pass():
    # The grouped tiles of 3D-aware rows (runs of identical rows average ~1.3
    # queries) go to the gathered pass.  Forward and backward of the
    # key-centric plan against the oracle.
    args = _aware_rows()
    q, k, v, rows, cu_sb, cu_blk, cu_q = args
    dev = [t.to(DEV) for t in args]
    plan = H.SelAttnPlan(dev[0].shape, dev[1].shape, dev[3], dev[4], dev[5], dev[6],
                         backward=True, key_centric=True)
    o, lse = plan.fwd(dev[0], dev[1], dev[2], 0.125)
    _check_oracle(args, o, lse)
    o2, _ = _fwd(args, False)
    assert not torch.equal(o, o2)
    g = torch.Generator().manual_seed(113)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    dq, dk, dv, _ = plan.bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, 0.125)
    # the oracle's explicit backward (an autograd graph over runs of ~1.3
    # queries would hold every run's gathered keys)
    dq_r, dk_r, dv_r, _ = sel_attn_bwd_ref(q.float(), k.float(), v.float(), do.float(), rows,
                                           cu_sb, cu_blk, cu_q, 0.125)
    assert_attn_close(dq, dq_r, "dq")
    assert_attn_close(dk, dk_r, "dk")
    assert_attn_close(dv, dv_r, "dv")


def test_plan_with_backward_and_key_centric():
    # One plan carrying both parts: the key-centric forward, then the
    # backward on the same workspace.
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(n=3000, topk=6, seed=10)
    dev = [t.to(DEV) for t in (q, k, v, rows, cu_sb, cu_blk, cu_q)]
    plan = H.SelAttnPlan(dev[0].shape, dev[1].shape, dev[3], dev[4], dev[5], dev[6],
                         backward=True, key_centric=True)
    o, lse = plan.fwd(dev[0], dev[1], dev[2], 0.125)
    _check_oracle((q, k, v, rows, cu_sb, cu_blk, cu_q), o, lse)
    g = torch.Generator().manual_seed(110)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    dq, dk, dv, _ = plan.bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, 0.125)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    o_ref, _ = sel_attn_ref(qf, kf, vf, rows, cu_sb, cu_blk, cu_q, 0.125)
    o_ref.backward(do.float())
    assert_attn_close(dq, qf.grad, "dq")
    assert_attn_close(dk, kf.grad, "dk")
    assert_attn_close(dv, vf.grad, "dv")


def test_sparse_ops_knob_with_autograd():
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(n=2000, topk=6, seed=11)
    # sparse.ops validates the rows: -1 only as trailing padding
    rows = torch.where(rows >= cu_blk.numel() - 1, rows[..., :1], rows)
    rows = torch.where(rows[..., :1] < 0, torch.full_like(rows, -1), rows)
    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    ops.set_key_centric(True)
    try:
        out = ops.native_sparse_attend(qd, kd, vd, rows.to(DEV), cu_sb.to(DEV),
                                       cu_blk.to(DEV), cu_q.to(DEV), cu_q.to(DEV), 0.125)
    finally:
        ops.set_key_centric("auto")
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    o_ref, _ = sel_attn_ref(qf, kf, vf, rows, cu_sb, cu_blk, cu_q, 0.125)
    assert_attn_close(out, o_ref, "out")
    g = torch.Generator().manual_seed(111)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    out.backward(do.to(DEV))
    o_ref.backward(do.float())
    assert_attn_close(qd.grad, qf.grad, "dq")
    assert_attn_close(kd.grad, kf.grad, "dk")
    assert_attn_close(vd.grad, vf.grad, "dv")
    assert np.isfinite(out.detach().float().cpu().numpy()).all()


@pytest.mark.parametrize("hq,hkv,d", [(2, 2, 64), (32, 2, 32)])
def test_backward_gathered_dq_duplicates_empty_rows(hq, hkv, d):
    # dQ of the grouped queries on gathered tiles (slot shares added in row
    # order); repeated ids, rows without any block (dQ = 0, Delta still
    # rowsum(O dO)), GQA 16 at head dim 32.
    q, k, v, rows, cu_sb, cu_blk, cu_q = _random_rows(n=2400, hq=hq, hkv=hkv, d=d, topk=6,
                                                      seed=12)
    rows = rows.clone()
    rows[:, ::3, 1] = rows[:, ::3, 0]
    args = (q, k, v, rows, cu_sb, cu_blk, cu_q)
    o, lse = _fwd(args, True)
    g = torch.Generator().manual_seed(112)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    dev = [t.to(DEV) for t in args]
    dq, dk, dv, delta = H.sel_attn_bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, *dev[3:],
                                       0.125, key_centric=True)
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    o_ref, _ = sel_attn_ref(qf, kf, vf, rows, cu_sb, cu_blk, cu_q, 0.125)
    o_ref.backward(do.float())
    assert_attn_close(dq, qf.grad, "dq")
    assert_attn_close(dk, kf.grad, "dk")
    assert_attn_close(dv, vf.grad, "dv")
    delta_ref = (o.float().cpu() * do.float()).sum(-1).transpose(0, 1)
    torch.testing.assert_close(delta.cpu(), delta_ref, rtol=1e-4, atol=1e-4)
    again = H.sel_attn_bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, *dev[3:], 0.125,
                           key_centric=True)
    assert all(torch.equal(x, y) for x, y in zip((dq, dk, dv, delta), again))


@pytest.mark.parametrize("hq,hkv,d,topk", [(2, 2, 64, 8), (8, 2, 64, 20), (2, 2, 32, 8),
                                           (2, 2, 128, 8)])
def test_large_and_small_blocks_all_gathered_kernels(hq, hkv, d, topk):
    # Blocks of 4..700 keys: those of at most 256 keys run with the block
    # resident in LDS (four waves), those of 257..512 keys too at head dim
    # <= 64 (eight waves, two groups of four tiles with the softmax
    # reference raised between them), the rest through the streaming
    # gathered tiles.  topk 20: the merge takes the slots 16 at a time.
    args = _random_rows(n=20000, hq=hq, hkv=hkv, d=d, topk=topk, seed=13, sizes=(4, 700))
    cu = args[5]
    lens = cu[1:] - cu[:-1]
    assert (lens <= 256).any() and ((lens > 256) & (lens <= 512)).any() and (lens > 512).any()
    o, lse = _fwd(args, True)
    _check_oracle(args, o, lse)
    again = _fwd(args, True)
    assert torch.equal(o, again[0]) and torch.equal(lse, again[1])


@pytest.mark.parametrize("hq,hkv,d,topk", [(2, 2, 64, 8), (8, 2, 64, 20), (2, 2, 32, 8),
                                           (2, 2, 128, 8)])
def test_backward_all_gathered_dq_kernels(hq, hkv, d, topk):
    # dQ of blocks of 4..700 keys: the resident dQ kernels (four waves up to
    # 256 keys; eight waves for 257..512 keys at head dim <= 64) and the
    # streaming gathered dQ tiles for the rest, then the slot-order merge.
    args = _random_rows(n=8000, hq=hq, hkv=hkv, d=d, topk=topk, seed=14, sizes=(4, 700))
    q, k, v, rows, cu_sb, cu_blk, cu_q = args
    lens = cu_blk[1:] - cu_blk[:-1]
    assert (lens <= 256).any() and ((lens > 256) & (lens <= 512)).any() and (lens > 512).any()
    dev = [t.to(DEV) for t in args]
    plan = H.SelAttnPlan(dev[0].shape, dev[1].shape, dev[3], dev[4], dev[5], dev[6],
                         backward=True, key_centric=True)
    o, lse = plan.fwd(dev[0], dev[1], dev[2], 0.125)
    g = torch.Generator().manual_seed(114)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    dq, dk, dv, delta = plan.bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, 0.125)
    # the oracle's explicit backward (an autograd graph over one run per
    # query would hold every gathered key set)
    dq_r, dk_r, dv_r, _ = sel_attn_bwd_ref(q.float(), k.float(), v.float(), do.float(), rows,
                                           cu_sb, cu_blk, cu_q, 0.125)
    assert_attn_close(dq, dq_r, "dq")
    assert_attn_close(dk, dk_r, "dk")
    assert_attn_close(dv, dv_r, "dv")
    delta_ref = (o.float().cpu() * do.float()).sum(-1).transpose(0, 1)
    torch.testing.assert_close(delta.cpu(), delta_ref, rtol=1e-4, atol=1e-4)
    again = plan.bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, 0.125)
    assert all(torch.equal(x, y) for x, y in zip((dq, dk, dv, delta), again))


@pytest.mark.parametrize("hq,topk", [(2, 64), (16, 64), (2, 128), (16, 128)])
def test_long_rows_forward_and_backward(hq, topk):
    # get_block_score emits rows of up to 128 blocks: the forward merge
    # rescales its running maximum across up to 8 groups of 16 slots, the dQ
    # merge adds up to 128 slot shares, each already rounded to the input
    # type.
    args = _random_rows(n=3000, hq=hq, hkv=2, d=64, topk=topk,
                        seed=15 + topk, sizes=(4, 24))
    q, k, v, rows, cu_sb, cu_blk, cu_q = args
    dev = [t.to(DEV) for t in args]
    plan = H.SelAttnPlan(dev[0].shape, dev[1].shape, dev[3], dev[4], dev[5], dev[6],
                         backward=True, key_centric=True)
    o, lse = plan.fwd(dev[0], dev[1], dev[2], 0.125)
    _check_oracle(args, o, lse)
    g = torch.Generator().manual_seed(115)
    do = (0.5 * torch.randn(q.shape, generator=g)).to(q.dtype)
    dq, dk, dv, _ = plan.bwd(do.to(DEV), dev[0], dev[1], dev[2], o, lse, 0.125)
    dq_r, dk_r, dv_r, _ = sel_attn_bwd_ref(q.float(), k.float(), v.float(), do.float(), rows,
                                           cu_sb, cu_blk, cu_q, 0.125)
    assert_attn_close(dq, dq_r, "dq")
    assert_attn_close(dk, dk_r, "dk")
    assert_attn_close(dv, dv_r, "dv")


def _raw_plan(args, flags, head_dim, ws_flags, ws_head_dim):
    """A plan built through the C ABI with `flags` / `head_dim` in a
    workspace sized for `ws_flags` / `ws_head_dim`."""
    q, k, rows, cu_sb, cu_blk, cu_q = args
    nq, hq, _ = q.shape
    nk, hkv, _ = k.shape
    nb = cu_blk.numel() - 1
    lib = H.lib()
    n = max(lib.lsrm_sel_attn_workspace_size2(nq, nk, hq, hkv, ws_head_dim, rows.shape[-1], nb,
                                              ws_flags),
            lib.lsrm_sel_attn_workspace_size2(nq, nk, hq, hkv, head_dim, rows.shape[-1], nb,
                                              flags))
    ws = torch.empty(n, dtype=torch.uint8, device=DEV)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.lsrm_sel_attn_plan2(rows.data_ptr(), nq, nk, hq, hkv, head_dim, rows.shape[-1],
                                 cu_sb.data_ptr(), cu_blk.data_ptr(), nb, cu_q.data_ptr(), 1,
                                 flags, ws.data_ptr(), ws.numel(), st)
    assert rc == 0
    return ws


def _raw_fwd(q, k, v, rows, cu_sb, cu_blk, cu_q, ws, flags):
    nq, hq, d = q.shape
    nk, hkv, _ = k.shape
    out = torch.full_like(q, float("nan"))
    lse = torch.full((hq, nq), float("nan"), dtype=torch.float32, device=DEV)
    rc = H.lib().lsrm_sel_attn_fwd_run2(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), H.BF16, nq, nk, hq, hkv, d, rows.data_ptr(),
        rows.shape[-1], cu_sb.data_ptr(), cu_blk.data_ptr(), cu_blk.numel() - 1,
        cu_q.data_ptr(), 1, 0.125, out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(),
        flags, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out, lse


def test_key_centric_run_needs_a_key_centric_plan():
    # A forward-only plan run with the key-centric flag: the carving finds
    # item lists that were never built; the key-centric kernels read the
    # plan's marker and exit without touching memory, so the grouped
    # queries' rows stay as they were (NaN here) and nothing faults.  The
    # run-tile rows are still computed and correct.
    args = list(_random_rows(n=3000, seed=16))
    args[3] = args[3].clone()
    args[3][:, :1024] = args[3][:, :1]  # 1024 identical rows: run tiles
    q, k, v, rows, cu_sb, cu_blk, cu_q = (t.to(DEV) for t in args)
    ws = _raw_plan((q, k, rows, cu_sb, cu_blk, cu_q), 0, 64, H.PLAN_KEY_CENTRIC, 64)
    out, lse = _raw_fwd(q, k, v, rows, cu_sb, cu_blk, cu_q, ws, H.PLAN_KEY_CENTRIC)
    untouched = torch.isnan(lse)
    assert untouched.any()
    o_ref, lse_ref = sel_attn_ref(*(t.float() for t in args[:3]), *args[3:], 0.125)
    done = ~untouched.cpu()
    lr = lse_ref[done]
    fin = torch.isfinite(lr)
    assert float((lse.cpu()[done][fin] - lr[fin]).abs().max()) <= 2e-2
    rows_done = done.transpose(0, 1)  # [nq, hq]
    assert_attn_close(out.cpu()[rows_done], o_ref[rows_done], "run-tile rows")


def test_key_centric_plan_for_another_head_dim_is_refused():
    # A key-centric plan built for head dim 64 (blocks of 257..512 keys in
    # the eight-wave resident list) run at head dim 128, where that kernel
    # does not exist: the marker differs, the key-centric kernels exit, and
    # no partial is merged unwritten.
    args = _random_rows(n=3000, seed=17, d=128, sizes=(200, 400))
    q, k, v, rows, cu_sb, cu_blk, cu_q = (t.to(DEV) for t in args)
    ws = _raw_plan((q, k, rows, cu_sb, cu_blk, cu_q), H.PLAN_KEY_CENTRIC, 64,
                   H.PLAN_KEY_CENTRIC, 128)
    _, lse = _raw_fwd(q, k, v, rows, cu_sb, cu_blk, cu_q, ws, H.PLAN_KEY_CENTRIC)
    assert torch.isnan(lse).any()
    # the same plan built for head dim 128 gives the oracle's result
    ws = _raw_plan((q, k, rows, cu_sb, cu_blk, cu_q), H.PLAN_KEY_CENTRIC, 128,
                   H.PLAN_KEY_CENTRIC, 128)
    o, lse = _raw_fwd(q, k, v, rows, cu_sb, cu_blk, cu_q, ws, H.PLAN_KEY_CENTRIC)
    _check_oracle(args, o, lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sizes", [(65, 257), (257, 513)])
def test_resident_blocks_later_tiles_dominate(dtype, sizes):
    # Blocks of 65..256 keys (four-wave resident kernel) or 257..512 keys
    # (eight-wave) whose first 64-key tile is scaled down: the row maxima of
    # the later tiles exceed the first tile's by ~17 log2 units, so against
    # the first tile's maximum the probabilities reach 2^17 -- bf16 holds
    # them, fp16 overflows and the kernel must rerun those rows with the
    # exact online maximum.  Outputs must match the oracle either way.
    n, hkv, d, topk = 6000, 2, 64, 3
    rng = np.random.default_rng(41)
    lens = rng.integers(sizes[0], sizes[1], size=n // sizes[0] + 1)
    cu = np.concatenate([[0], np.cumsum(lens)])
    cu = cu[cu <= n]
    cu[-1] = n
    nb = len(cu) - 1
    g = torch.Generator().manual_seed(42)
    q = 2.0 * torch.randn(n, hkv, d, generator=g)
    k = 2.0 * torch.randn(n, hkv, d, generator=g)
    for c in range(nb):
        k[cu[c]:min(cu[c] + 64, cu[c + 1])] *= 0.02
    v = torch.randn(n, hkv, d, generator=g)
    rows = torch.randint(0, nb, (hkv, n, topk), generator=g, dtype=torch.int32)
    args = (q.to(dtype), k.to(dtype), v.to(dtype), rows, torch.tensor([0, nb], dtype=torch.int32),
            torch.from_numpy(cu.astype(np.int32)), torch.tensor([0, n], dtype=torch.int32))
    o, lse = _fwd(args, True)
    _check_oracle(args, o.cpu(), lse)
