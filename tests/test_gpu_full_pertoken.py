"""GPU parity of the per-token paths at the size the benchmark times them.

Config 3's full token layout (131072 tokens; the 122880 voxel tokens for the
3D-aware rows) with per-token selection rows:
  * 3D-aware rows (each voxel token's nearest 16 block centroids), H=24, D=64:
    the key-centric plan (forward and backward) and the grouped-tile plan
    (forward and backward);
  * learned rows (compressed attention + get_block_score, top-16 of all 462
    blocks for every token), H=24, D=64: the key-centric plan;
  * LSRM's own decoder head layout (32 query heads, 2 kv heads, head dim 32)
    on the 3D-aware rows: the key-centric plan.
The GPU runs the whole problem (every head, every query).  The oracle checks
sampled kv heads: the forward and dQ on a random sample of queries (a query's
output and dQ depend on its own row only), dK / dV on sampled blocks of
different sizes together with every query that lists them (then the keys of
those blocks receive every contribution), Delta on the sampled queries.
"""

import os
import time

import numpy as np
import pytest
import torch

import lsrm_hip as H
import sparse.ops as ops
from helpers import assert_attn_close
from lsrm_hip import workloads as W
from oracle.attention import sel_attn_bwd_ref, sel_attn_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(msg):
    print(f"[full-per-token] {msg}", flush=True)


def _cpu_threads():
    torch.set_num_threads(max(1, min(16, len(os.sched_getaffinity(0)))))


def _voxel_problem(w):
    """Device tensors of config 3's voxel tokens and their 3D-aware rows (the
    GPU builders, bit-exact against their oracles in test_gpu_builders)."""
    q, k, v, do = W.tensors(w, DEV, with_grad_out=True)
    n_img, nb_img = w.n_image_tokens, w.n_image_blocks
    nv = w.n - n_img
    coords = torch.zeros(nv, 4, dtype=torch.int32)
    coords[:, 1:] = torch.from_numpy(w.voxel_coords)
    cu_v = (w.cu_block_tokens[nb_img:] - w.cu_block_tokens[nb_img]).to(DEV)
    cu_sb = torch.tensor([0, cu_v.numel() - 1], dtype=torch.int32, device=DEV)
    cu_q = torch.tensor([0, nv], dtype=torch.int32, device=DEV)
    pts = H.volume_points(coords.to(DEV), 64, 1.0)
    rows = H.nearest_blocks(pts, cu_v, cu_sb, cu_q, 16, w.hkv)
    qv, kv, vv, dov = (t[n_img:].contiguous() for t in (q, k, v, do))
    del q, k, v, do
    return qv, kv, vv, dov, rows, cu_sb, cu_v, cu_q


def _learned_problem(w):
    """Config 3 with get_block_score rows: compressed attention over the
    block means, then the top-16 blocks of every token."""
    q, k, v, do = W.tensors(w, DEV, with_grad_out=True)
    cu_sb, cu_blk, cu_q = (t.to(DEV) for t in (w.cu_seqblocks, w.cu_block_tokens, w.cu_seqlens))
    ck = H.block_mean_pool(k.view(w.n, -1), cu_blk).view(-1, w.hkv, w.d)
    cv = H.block_mean_pool(v.view(w.n, -1), cu_blk).view(-1, w.hkv, w.d)
    ops.set_validation(False)
    try:
        _, lse = ops.compressed_attention(q, ck, cv, cu_q, cu_sb)
        rows = ops.get_block_score(q, ck, lse, 16, cu_q, cu_sb, None, None)
    finally:
        ops.set_validation(True)
    return q, k, v, do, rows, cu_sb, cu_blk, cu_q


def _check_head(h, g, scale, cpu, gpu, n_q_sample, blocks, seed):
    """Oracle checks of kv head h.  cpu = (q, k, v, do, rows, cu_blk) on the
    CPU; gpu = (o, lse, dq, dk, dv, delta) or (o, lse) from the device."""
    q, k, v, do, rows, cu_blk = cpu
    nq = q.shape[0]
    nb = cu_blk.numel() - 1
    hs = slice(h * g, (h + 1) * g)
    kh = k[:, h:h + 1].float()
    vh = v[:, h:h + 1].float()
    cu_sb = torch.tensor([0, nb], dtype=torch.int32)
    gen = torch.Generator().manual_seed(seed)
    qs = torch.randperm(nq, generator=gen)[:n_q_sample].sort().values
    rows_s = rows[h:h + 1, qs].contiguous()
    cu_s = torch.tensor([0, qs.numel()], dtype=torch.int32)
    t0 = time.time()
    o_ref, lse_ref = sel_attn_ref(q[qs][:, hs].float(), kh, vh, rows_s, cu_sb, cu_blk, cu_s,
                                  scale)
    o, lse = gpu[0], gpu[1]
    assert_attn_close(o[qs][:, hs], o_ref, f"head {h} out")
    lse_g = lse[hs][:, qs]
    fin = torch.isfinite(lse_ref)
    assert torch.equal(torch.isfinite(lse_g), fin)
    if fin.any():
        assert float((lse_g[fin] - lse_ref[fin]).abs().max()) <= 2e-2, f"head {h} lse"
    _say(f"head {h}: forward on {qs.numel()} sampled queries ({time.time() - t0:.1f} s)")
    if len(gpu) == 2:
        return
    dq, dk, dv, delta = gpu[2:]
    t0 = time.time()
    dq_r, _, _, dl_r = sel_attn_bwd_ref(q[qs][:, hs].float(), kh, vh, do[qs][:, hs].float(),
                                        rows_s, cu_sb, cu_blk, cu_s, scale)
    assert_attn_close(dq[qs][:, hs], dq_r, f"head {h} dq")
    # Delta = rowsum(O dO) with the kernel's own rounded O
    dl_own = (o[qs][:, hs].float() * do[qs][:, hs].float()).sum(-1).transpose(0, 1)
    torch.testing.assert_close(delta[hs][:, qs], dl_own, rtol=1e-4, atol=1e-4)
    _say(f"head {h}: dQ, Delta on the sampled queries ({time.time() - t0:.1f} s)")
    for c in blocks:
        t0 = time.time()
        lst = torch.nonzero((rows[h] == c).any(-1)).flatten()
        keys = slice(int(cu_blk[c]), int(cu_blk[c + 1]))
        rows_c = rows[h:h + 1, lst].contiguous()
        cu_c = torch.tensor([0, lst.numel()], dtype=torch.int32)
        _, dk_r, dv_r, _ = sel_attn_bwd_ref(q[lst][:, hs].float(), kh, vh,
                                            do[lst][:, hs].float(), rows_c, cu_sb, cu_blk,
                                            cu_c, scale)
        assert_attn_close(dk[keys, h], dk_r[keys, 0], f"head {h} block {c} dk")
        assert_attn_close(dv[keys, h], dv_r[keys, 0], f"head {h} block {c} dv")
        _say(f"head {h}: dK/dV of block {c} ({keys.stop - keys.start} keys, listed by "
             f"{lst.numel()} queries; {time.time() - t0:.1f} s)")


def _sample_blocks(rows_h, cu_blk, want=((1, 256), (257, 512), (513, 1 << 30)), cap=20000):
    """Per size class of `want` (the blocks the resident four-wave, resident
    eight-wave and streaming gathered kernels take), the block listed by the
    median number of queries of its class and the most listed one, among
    those listed at most `cap` times."""
    lens = (cu_blk[1:] - cu_blk[:-1]).long()
    ids = rows_h[rows_h >= 0].long()
    counts = torch.bincount(ids, minlength=lens.numel())[:lens.numel()]
    out = []
    for lo, hi in want:
        cand = torch.nonzero((lens >= lo) & (lens <= hi) & (counts > 0) &
                             (counts <= cap)).flatten()
        if cand.numel():
            order = cand[torch.argsort(counts[cand])]
            for c in (int(order[order.numel() // 2]), int(order[-1])):
                if c not in out:
                    out.append(c)
    return out


def _run_case(qd, kd, vd, dod, rows, cu_sb, cu_blk, cu_q, g, scale, key_centric, heads,
              n_q_sample, backward=True):
    plan = H.SelAttnPlan(qd.shape, kd.shape, rows, cu_sb, cu_blk, cu_q, backward=backward,
                         key_centric=key_centric)
    o, lse = plan.fwd(qd, kd, vd, scale)
    gpu = [o, lse]
    if backward:
        gpu += list(plan.bwd(dod, qd, kd, vd, o, lse, scale))
    torch.cuda.synchronize()
    del plan
    gpu = [t.cpu() for t in gpu]
    torch.cuda.empty_cache()
    cpu = (qd.cpu(), kd.cpu(), vd.cpu(), dod.cpu(), rows.cpu(), cu_blk.cpu())
    for i, h in enumerate(heads):
        blocks = _sample_blocks(cpu[4][h], cpu[5]) if backward else []
        _check_head(h, g, scale, cpu, gpu, n_q_sample, blocks, seed=100 + i)


@pytest.mark.parametrize("key_centric", [True, False])
def test_3d_aware_rows_cfg3_full(key_centric):
    _cpu_threads()
    w = W.config(3)
    _say(f"3D-aware rows, cfg3 full: N={w.n - w.n_image_tokens} voxel tokens, H={w.hq}, "
         f"key_centric={key_centric}")
    qv, kv, vv, dov, rows, cu_sb, cu_v, cu_q = _voxel_problem(w)
    _run_case(qv, kv, vv, dov, rows, cu_sb, cu_v, cu_q, w.hq // w.hkv, w.scale, key_centric,
              heads=(0, 17), n_q_sample=8192)


def test_learned_rows_cfg3_full_key_centric():
    _cpu_threads()
    w = W.config(3)
    _say(f"learned rows, cfg3 full: N={w.n}, H={w.hq}, key-centric plan")
    q, k, v, do, rows, cu_sb, cu_blk, cu_q = _learned_problem(w)
    _run_case(q, k, v, do, rows, cu_sb, cu_blk, cu_q, w.hq // w.hkv, w.scale, True,
              heads=(5, 22), n_q_sample=8192)


def test_product_head_layout_3d_aware_rows_full():
    # LSRM's decoder heads: 32 query heads over 2 kv heads (G = 16), head
    # dim 32, the 3D-aware rows of config 3's 122880 voxel tokens.
    _cpu_threads()
    w = W.product_shape()
    _say(f"product heads: N={w.n - w.n_image_tokens} voxel tokens, Hq={w.hq}, Hkv={w.hkv}, "
         f"D={w.d}, key-centric plan")
    qv, kv, vv, dov, rows, cu_sb, cu_v, cu_q = _voxel_problem(w)
    _run_case(qv, kv, vv, dov, rows, cu_sb, cu_v, cu_q, w.hq // w.hkv, w.scale, True,
              heads=(0, 1), n_q_sample=4096)
