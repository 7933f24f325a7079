"""GPU parity: block mean pooling and per-query-block selection, bit-exact
against the CPU oracle (through the C ABI via lsrm_hip)."""

import numpy as np
import pytest
import torch

import lsrm_hip as H
from lsrm_hip import workloads as W
from oracle.pool import block_mean_pool_ref
from oracle.select import expand_per_token, select_blocks_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _pool_case(n, c, dtype, out_dtype, lo=16, hi=300, seed=0):
    rng = np.random.default_rng(seed)
    sizes = W.uniform_partition(n, lo, hi, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32))
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, c, generator=g).to(dtype)
    out = H.block_mean_pool(x.to(DEV), cu.to(DEV), out_dtype)
    ref = block_mean_pool_ref(_f32(x), cu.numpy())
    ref_t = torch.from_numpy(ref).to(out_dtype or dtype)
    return out.cpu(), ref_t


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
def test_pool_bitexact(dtype, out_dtype):
    out, ref = _pool_case(5000, 256, dtype, out_dtype)
    assert torch.equal(out.view(torch.int16 if out.element_size() == 2 else torch.int32),
                       ref.view(torch.int16 if ref.element_size() == 2 else torch.int32))


def test_pool_scalar_path_and_long_blocks():
    # C not a multiple of 8 -> scalar path; blocks longer than several pieces.
    out, ref = _pool_case(3001, 12, torch.bfloat16, torch.float32, lo=100, hi=1000, seed=3)
    assert torch.equal(out, ref)


def test_pool_cfg3_shape_bitexact():
    w = W.config(3)
    g = torch.Generator(device=DEV).manual_seed(7)
    x = (0.5 * torch.randn(w.n, w.hkv * w.d, generator=g, device=DEV)).to(torch.bfloat16)
    out = H.block_mean_pool(x, w.cu_block_tokens.to(DEV))
    ref = block_mean_pool_ref(_f32(x), w.cu_block_tokens.numpy())
    ref = torch.from_numpy(ref).to(torch.bfloat16)
    assert torch.equal(out.cpu().view(torch.int16), ref.view(torch.int16))


def test_pool_matches_segment_reduce_and_empty_block():
    cu = torch.tensor([0, 5, 5, 70, 200], dtype=torch.int32)
    x = torch.randn(200, 64)
    out = H.block_mean_pool(x.to(DEV), cu.to(DEV)).cpu()
    ref = torch.segment_reduce(x, "mean", lengths=(cu[1:] - cu[:-1]).long(), axis=0)
    assert torch.isnan(out[1]).all() and torch.isnan(ref[1]).all()
    keep = torch.tensor([0, 2, 3])
    torch.testing.assert_close(out[keep], ref[keep], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("c", [256, 512, 1024, 1536, 3072])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
@pytest.mark.parametrize("n_blocks", [300, 800])
def test_pool_slab_path_small_and_empty_blocks(c, dtype, out_dtype, n_blocks):
    # 16-bit rows of 256 channels take two chunks per wave; multiples of 512
    # one 512-channel slab per wave (512), two (1024), three (1536: whole
    # rows; 3072: two waves per chunk), with the in-kernel block lookup below
    # 512 blocks and the lookup table above.
    # Blocks of length 0..40 put several block boundaries (and empty blocks,
    # whose mean is NaN) inside one 64-row piece; rows before the first and
    # after the last block are ignored.
    rng = np.random.default_rng(11)
    sizes = rng.integers(0, 41, size=n_blocks)
    sizes[[3, 4, 50, 299]] = 0
    sizes[[10, 11]] = 1
    cu_np = np.concatenate([[37], 37 + np.cumsum(sizes)]).astype(np.int32)
    n = int(cu_np[-1]) + 29
    g = torch.Generator().manual_seed(5)
    x = torch.randn(n, c, generator=g).to(dtype)
    cu = torch.from_numpy(cu_np)
    ref = torch.from_numpy(block_mean_pool_ref(_f32(x), cu_np)).to(out_dtype or dtype)
    for _ in range(2):
        out = H.block_mean_pool(x.to(DEV), cu.to(DEV), out_dtype).cpu()
        nan = torch.isnan(ref)
        assert torch.equal(torch.isnan(out), nan)
        ints = torch.int16 if out.element_size() == 2 else torch.int32
        assert torch.equal(out[~nan.all(1)].view(ints), ref[~nan.all(1)].view(ints))


@pytest.mark.parametrize("n_blocks", [512, 4881, 8191, 8192, 20000])
def test_pool_256_channels_block_lookup(n_blocks):
    # 256-channel 16-bit rows: up to 8191 blocks the kernel finds each
    # chunk's first block itself (32 sampled offsets, then up to 256 offsets
    # of the hit interval; 8191 blocks use the whole second round), beyond
    # that it reads the lookup table.  Empty blocks (runs of equal offsets,
    # one across a sampled offset), rows before the first and after the last
    # block.
    rng = np.random.default_rng(n_blocks)
    sizes = rng.integers(0, 21, size=n_blocks)
    s_rt = (n_blocks + 32) // 32
    sizes[[0, 1, s_rt - 1, s_rt, min(2 * s_rt, n_blocks - 1)]] = 0
    cu_np = np.concatenate([[45], 45 + np.cumsum(sizes)]).astype(np.int32)
    n = int(cu_np[-1]) + 70
    g = torch.Generator().manual_seed(n_blocks)
    x = torch.randn(n, 256, generator=g).to(torch.bfloat16)
    cu = torch.from_numpy(cu_np)
    ref = torch.from_numpy(block_mean_pool_ref(_f32(x), cu_np)).to(torch.bfloat16)
    out = H.block_mean_pool(x.to(DEV), cu.to(DEV), None).cpu()
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(out), nan)
    assert torch.equal(out[~nan.all(1)].view(torch.int16), ref[~nan.all(1)].view(torch.int16))


@pytest.mark.parametrize("c,n_blocks,out_a,out_b", [
    (512, 300, torch.float32, None),      # slab path, in-kernel block lookup
    (1024, 800, None, torch.float32),     # two slabs per wave, lookup table
    (1536, 300, torch.float32, None),     # whole rows per wave, in-kernel lookup
    (3072, 800, None, torch.float32),     # three slabs per wave, lookup table
    (256, 300, torch.float32, None),      # single-tensor fallback (C % 512 != 0)
])
def test_pool2_equals_oracle_and_single_calls(c, n_blocks, out_a, out_b):
    # keys and values pooled in one launch pair: each output bit for bit the
    # oracle and the single-tensor entry point, also with empty blocks and
    # rows outside every block.
    rng = np.random.default_rng(13)
    sizes = rng.integers(0, 41, size=n_blocks)
    sizes[[3, 4, 50]] = 0
    cu_np = np.concatenate([[19], 19 + np.cumsum(sizes)]).astype(np.int32)
    n = int(cu_np[-1]) + 7
    g = torch.Generator().manual_seed(2)
    xa = torch.randn(n, c, generator=g).to(torch.bfloat16)
    xb = (3.0 * torch.randn(n, c, generator=g)).to(torch.bfloat16)
    cu = torch.from_numpy(cu_np).to(DEV)
    pa, pb = H.block_mean_pool2(xa.to(DEV), xb.to(DEV), cu, out_a, out_b)
    sa = H.block_mean_pool(xa.to(DEV), cu, out_a)
    sb = H.block_mean_pool(xb.to(DEV), cu, out_b)
    for got, single, x, od in ((pa, sa, xa, out_a), (pb, sb, xb, out_b)):
        ref = torch.from_numpy(block_mean_pool_ref(_f32(x), cu_np)).to(od or torch.bfloat16)
        ints = torch.int16 if got.element_size() == 2 else torch.int32
        assert got.dtype == (od or torch.bfloat16)
        assert torch.equal(got.cpu().view(ints), single.cpu().view(ints))
        nan = torch.isnan(ref)
        assert torch.equal(torch.isnan(got.cpu()), nan)
        assert torch.equal(got.cpu()[~nan.all(1)].view(ints), ref[~nan.all(1)].view(ints))


def test_pool2_cfg3_shape_bitexact():
    w = W.config(3)
    g = torch.Generator(device=DEV).manual_seed(8)
    k = (0.5 * torch.randn(w.n, w.hkv * w.d, generator=g, device=DEV)).to(torch.bfloat16)
    v = torch.randn(w.n, w.hkv * w.d, generator=g, device=DEV).to(torch.bfloat16)
    cu = w.cu_block_tokens.to(DEV)
    pk, pv = H.block_mean_pool2(k, v, cu, torch.float32, None)
    assert torch.equal(pk, H.block_mean_pool(k, cu, torch.float32))
    assert torch.equal(pv.view(torch.int16), H.block_mean_pool(v, cu).view(torch.int16))
    ref = torch.from_numpy(block_mean_pool_ref(_f32(v), w.cu_block_tokens.numpy()))
    assert torch.equal(pv.cpu().view(torch.int16), ref.to(torch.bfloat16).view(torch.int16))


def _select_case(w, forced=None, hq=None, hkv=None, dtype=None):
    dtype = dtype or w.dtype
    g = torch.Generator().manual_seed(w.seed)
    hq = hq or w.hq
    hkv = hkv or w.hkv
    q = torch.randn(w.n, hq, w.d, generator=g).to(dtype)
    k = torch.randn(w.n, hkv, w.d, generator=g).to(dtype)
    if w.lowrank:
        u = torch.randn(w.n, 4, generator=g)
        q = (0.95 * q.float() + 0.3 * (u @ torch.randn(4, hq * w.d, generator=g)).view(q.shape)).to(dtype)
        k = (0.95 * k.float() + 0.3 * (u @ torch.randn(4, hkv * w.d, generator=g)).view(k.shape)).to(dtype)
    forced = w.forced_blocks if forced is None else forced
    topk_idx, compact = H.select_blocks(q.to(DEV), k.to(DEV), w.cu_seqblocks.to(DEV),
                                        w.cu_block_tokens.to(DEV), w.topk, forced, w.force_self)
    cu = w.cu_block_tokens.numpy()
    pq = block_mean_pool_ref(_f32(q).reshape(w.n, -1), cu).reshape(-1, hq, w.d)
    pk = block_mean_pool_ref(_f32(k).reshape(w.n, -1), cu).reshape(-1, hkv, w.d)
    ref = select_blocks_ref(pq, pk, w.cu_seqblocks.numpy(), w.topk, forced, w.force_self)
    return topk_idx.cpu().numpy(), compact.cpu().numpy(), ref


@pytest.mark.parametrize("cfg,n,heads", [(1, None, None), (2, 8192, 4), (3, 16384, 4), (5, 65536, 4)])
def test_select_bitexact(cfg, n, heads):
    w = W.config(cfg, n=n, heads=heads)
    topk_idx, compact, ref = _select_case(w)
    np.testing.assert_array_equal(compact, ref)
    np.testing.assert_array_equal(topk_idx, expand_per_token(ref, w.cu_block_tokens.numpy(), w.n))
    # forced blocks are always selected
    for f in w.forced_blocks:
        assert (compact == f).any(-1).all()
    # self block is always selected
    nb = w.n_blocks
    assert (compact == np.arange(nb)[None, :, None]).any(-1).all()



@pytest.mark.parametrize("cfg,n,heads,hq", [(3, 16384, 4, 4), (2, 8192, 2, 8)])
def test_select_with_pooled_keys_matches(cfg, n, heads, hq):
    """lsrm_select_blocks_pooled (keys pooled once in fp32 by the caller)
    selects exactly what lsrm_select_blocks does, and rounding those fp32
    means gives the bf16 compressed keys block_mean_pool returns."""
    w = W.config(cfg, n=n, heads=heads)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(w.n, hq, w.d, generator=g).bfloat16().to(DEV)
    k = torch.randn(w.n, w.hkv, w.d, generator=g).bfloat16().to(DEV)
    cu_sb, cu = w.cu_seqblocks.to(DEV), w.cu_block_tokens.to(DEV)
    a_idx, a_cmp = H.select_blocks(q, k, cu_sb, cu, w.topk, w.forced_blocks, w.force_self)
    pk = H.block_mean_pool(k.view(w.n, -1), cu, torch.float32)
    b_idx, b_cmp = H.select_blocks(q, k, cu_sb, cu, w.topk, w.forced_blocks, w.force_self,
                                   pooled_k=pk)
    assert torch.equal(a_idx, b_idx) and torch.equal(a_cmp, b_cmp)
    ck = H.block_mean_pool(k.view(w.n, -1), cu)
    assert torch.equal(pk.to(torch.bfloat16).view(torch.int16), ck.view(torch.int16))
    with pytest.raises(ValueError):
        H.select_blocks(q, k, cu_sb, cu, w.topk, w.forced_blocks, w.force_self,
                        pooled_k=pk.bfloat16())

def test_select_gqa_bitexact():
    w = W.config(2, n=4096)
    topk_idx, compact, ref = _select_case(w, hq=8, hkv=2)
    np.testing.assert_array_equal(compact, ref)


def test_select_topk_ge_blocks_selects_all():
    w = W.config(1, n=600, heads=2)
    w.topk = w.n_blocks + 3
    _, compact, ref = _select_case(w)
    np.testing.assert_array_equal(compact, ref)
    assert (compact[..., : w.n_blocks] == np.arange(w.n_blocks)).all()
    assert (compact[..., w.n_blocks:] == -1).all()


def test_select_ties_lowest_index():
    # Every block has the same pooled key -> all scores tie -> lowest ids win.
    n, d = 640, 64
    cu = torch.arange(0, n + 1, 64, dtype=torch.int32)
    q = torch.randn(n, 2, d).to(torch.bfloat16)
    k = torch.ones(n, 2, d, dtype=torch.bfloat16)
    _, compact = H.select_blocks(q.to(DEV), k.to(DEV), torch.tensor([0, 10], dtype=torch.int32, device=DEV),
                                 cu.to(DEV), 3, None, True)
    compact = compact.cpu()
    for b in range(10):
        expect = sorted(set([b] + [x for x in range(10) if x != b][:2]))
        assert compact[:, b].tolist() == [expect, expect]


def test_select_split_path_bitexact():
    # More than 2048 blocks per batch element: the four-wave split selection
    # (cfg5's heavy-tailed blocks with near-tie scores, forced ids).
    w = W.config(5, n=262144, heads=2)
    assert 2048 < w.n_blocks <= 8192
    topk_idx, compact, ref = _select_case(w, forced=[0, 5, 17])
    np.testing.assert_array_equal(compact, ref)
    np.testing.assert_array_equal(topk_idx, expand_per_token(ref, w.cu_block_tokens.numpy(), w.n))


def test_select_split_path_ties_and_nan():
    # 2200 one-token blocks whose keys are equal (every score ties: the
    # lowest ids win) except one NaN block (ranked last).
    n, d, topk = 2200, 64, 5
    cu = torch.arange(0, n + 1, dtype=torch.int32)
    q = torch.randn(n, 2, d).to(torch.bfloat16)
    k = torch.ones(n, 2, d, dtype=torch.bfloat16)
    k[1] = float("nan")
    _, compact = H.select_blocks(q.to(DEV), k.to(DEV), torch.tensor([0, n], dtype=torch.int32, device=DEV),
                                 cu.to(DEV), topk, [7], True)
    compact = compact.cpu().numpy()
    for b in (0, 1, 2, 7, 1000, n - 1):
        chosen = [b] + ([7] if b != 7 else [])
        rest = [x for x in range(n) if x not in chosen and x != 1]
        expect = sorted(chosen + rest[:topk - len(chosen)])
        if b == 1:  # the NaN block's own row: forced ids, then the lowest non-NaN ids
            expect = sorted([1, 7] + [x for x in range(n) if x not in (1, 7)][:topk - 2])
        assert compact[:, b].tolist() == [expect, expect], (b, compact[:, b].tolist(), expect)


@pytest.mark.parametrize("nb,topk", [(1500, 16), (1500, 64), (4881, 32), (4881, 64)])
@pytest.mark.parametrize("pattern", ["random", "lane_periodic", "sorted"])
def test_select_threshold_pass_and_fallback(nb, topk, pattern):
    # One-token blocks, so the pooled queries are the queries themselves, and
    # pooled keys given directly: 1500 blocks take the one-wave top-k, 4881
    # the four-wave split.  "lane_periodic" scores depend on id % 64 only
    # (eight tie classes), so each lane holds candidates of one score and the
    # threshold pass has far more than 64 survivors (the exact fallback runs);
    # "sorted" scores grow with the id; topk 64 leaves no lane-best threshold.
    d = 64
    g = torch.Generator().manual_seed(nb * 7 + topk)
    q = torch.randn(nb, 1, d, generator=g).to(torch.bfloat16)
    if pattern == "random":
        pk = torch.randn(nb, 1, d, generator=g)
    else:
        q[:, :, 1:] = 0
        q[:, :, 0] = 1
        ids = torch.arange(nb, dtype=torch.float32)
        pk = torch.zeros(nb, 1, d)
        pk[:, 0, 0] = (ids % 64) // 8 if pattern == "lane_periodic" else ids / nb
    cu = torch.arange(nb + 1, dtype=torch.int32)
    cu_sb = torch.tensor([0, nb], dtype=torch.int32)
    forced = [0, 5, 17]
    topk_idx, compact = H.select_blocks(q.to(DEV), q.to(DEV), cu_sb.to(DEV), cu.to(DEV), topk,
                                        forced, True, pooled_k=pk.reshape(nb, d).to(DEV))
    ref = select_blocks_ref(_f32(q), pk.numpy(), cu_sb.numpy(), topk, forced, True)
    np.testing.assert_array_equal(compact.cpu().numpy(), ref)
    np.testing.assert_array_equal(topk_idx.cpu().numpy(), ref)


def test_select_tokens_outside_blocks_get_empty_rows():
    # the blocks cover tokens [100, n - 50): the other tokens' rows are -1
    n, d, hq = 2000, 64, 2
    rng = np.random.default_rng(21)
    sizes = W.uniform_partition(n - 150, 16, 96, rng)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32) + 100)
    g = torch.Generator().manual_seed(22)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
    cu_sb = torch.tensor([0, len(sizes)], dtype=torch.int32)
    topk_idx, compact = H.select_blocks(q.to(DEV), k.to(DEV), cu_sb.to(DEV), cu.to(DEV), 4, None, True)
    pq = block_mean_pool_ref(_f32(q).reshape(n, -1), cu.numpy()).reshape(-1, hq, d)
    pk = block_mean_pool_ref(_f32(k).reshape(n, -1), cu.numpy()).reshape(-1, hq, d)
    ref = select_blocks_ref(pq, pk, cu_sb.numpy(), 4, None, True)
    np.testing.assert_array_equal(compact.cpu().numpy(), ref)
    ti = topk_idx.cpu().numpy()
    assert (ti[:, :100] == -1).all() and (ti[:, n - 50:] == -1).all()
    np.testing.assert_array_equal(ti, expand_per_token(ref, cu.numpy(), n))


@pytest.mark.parametrize("n_blocks,topk", [(300, 8), (2100, 16), (2100, 80)])
def test_select_blocks_outside_every_batch_element(n_blocks, topk):
    # cu_seqblocks[-1] < n_blocks: the trailing blocks belong to no batch
    # element, so their tokens' rows must be -1 (the output is allocated
    # uninitialised, over memory pre-filled with valid-looking ids).  The
    # three sizes take the wave, split and workgroup top-k kernels.
    rng = np.random.default_rng(n_blocks + topk)
    sizes = rng.integers(1, 6, size=n_blocks)
    cu_np = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    n = int(cu_np[-1])
    inside = (n_blocks * 2) // 3
    cu_sb = torch.tensor([0, inside // 2, inside], dtype=torch.int32)
    g = torch.Generator().manual_seed(3)
    hq, hkv, d = 4, 2, 64
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
    for _ in range(2):
        junk = torch.full((hkv, n, topk), 3, dtype=torch.int32, device=DEV)
        junk2 = torch.full((hkv, n_blocks, topk), 3, dtype=torch.int32, device=DEV)
        del junk, junk2
        topk_idx, compact = H.select_blocks(q.to(DEV), k.to(DEV), cu_sb.to(DEV),
                                            torch.from_numpy(cu_np).to(DEV), topk, [], True)
        pq = block_mean_pool_ref(_f32(q).reshape(n, -1), cu_np).reshape(-1, hq, d)
        pk = block_mean_pool_ref(_f32(k).reshape(n, -1), cu_np).reshape(-1, hkv, d)
        ref = select_blocks_ref(pq, pk, cu_sb.numpy(), topk, [], True)
        np.testing.assert_array_equal(compact.cpu().numpy(), ref)
        np.testing.assert_array_equal(topk_idx.cpu().numpy(), expand_per_token(ref, cu_np, n))
        assert (topk_idx[:, int(cu_np[inside]):].cpu() == -1).all()
