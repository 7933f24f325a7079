"""lsrm_block_mean_pool_noalloc (the allocation-free entry point) against
lsrm_block_mean_pool, both called through the C ABI: bit-identical outputs
on two calls in a row (the second on a smaller input, so stale scratch from
the first call is present), and inputs beyond the fixed scratch rejected
with LSRM_ERR_SCRATCH before anything is launched."""

import numpy as np
import pytest
import torch

import lsrm_hip as H
from lsrm_hip import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
LSRM_ERR_SCRATCH = 5


def _pool_both(x, cu, out_dtype):
    lib = H.lib()
    n, c = x.shape
    nb = cu.numel() - 1
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.full((nb, c), 3.0, dtype=out_dtype, device=DEV)
    ws_n = lib.lsrm_block_mean_pool_workspace_size(n, c, nb)
    ws = torch.empty(ws_n, dtype=torch.uint8, device=DEV)
    assert lib.lsrm_block_mean_pool(x.data_ptr(), H._DTYPE_CODE[x.dtype], n, c, cu.data_ptr(), nb,
                                    ref.data_ptr(), H._DTYPE_CODE[out_dtype], ws.data_ptr(), ws_n,
                                    stream) == 0
    out = torch.full((nb, c), 5.0, dtype=out_dtype, device=DEV)
    assert lib.lsrm_block_mean_pool_noalloc(x.data_ptr(), H._DTYPE_CODE[x.dtype], n, c,
                                            cu.data_ptr(), nb, out.data_ptr(),
                                            H._DTYPE_CODE[out_dtype], stream) == 0
    torch.cuda.synchronize()
    return out, ref


def _bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_twice(out_dtype):
    # call 1: the cfg3 key tensor (131072 x 1536 bf16, 462 blocks; the slab
    # path); call 2: 256 channels over 2000 blocks of 0-40 rows (the
    # two-chunk kernel with its in-kernel block lookup); call 3: a smaller,
    # ragged input (the scalar-channel path, blocks of 0-300 rows).  Each call
    # runs over the scratch the previous one left behind.
    w = W.config(3)
    g = torch.Generator(device=DEV).manual_seed(5)
    x1 = (0.5 * torch.randn(w.n, w.hkv * w.d, generator=g, device=DEV)).to(torch.bfloat16)
    cu1 = w.cu_block_tokens.to(DEV)
    rng = np.random.default_rng(2)
    sizes = rng.integers(0, 301, size=40)
    cu2 = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)).to(DEV)
    x2 = torch.randn(int(sizes.sum()), 12, generator=g, device=DEV).to(torch.float16)
    sizes3 = rng.integers(0, 41, size=2000)
    cu3 = torch.from_numpy(np.concatenate([[0], np.cumsum(sizes3)]).astype(np.int32)).to(DEV)
    x3 = torch.randn(int(sizes3.sum()), 256, generator=g, device=DEV).to(torch.bfloat16)
    for x, cu in ((x1, cu1), (x3, cu3), (x2, cu2)):
        out, ref = _pool_both(x, cu, out_dtype)
        nan = torch.isnan(ref)
        assert torch.equal(torch.isnan(out), nan)
        assert torch.equal(_bits(out)[~nan], _bits(ref)[~nan])


def test_noalloc_rejects_inputs_beyond_scratch():
    lib = H.lib()
    n, c, nb = 1 << 20, 4096, 100
    assert lib.lsrm_block_mean_pool_workspace_size(n, c, nb) > (64 << 20)
    dummy = torch.zeros(16, dtype=torch.int32, device=DEV)
    rc = lib.lsrm_block_mean_pool_noalloc(dummy.data_ptr(), H.BF16, n, c, dummy.data_ptr(), nb,
                                          dummy.data_ptr(), H.BF16,
                                          torch.cuda.current_stream().cuda_stream)
    assert rc == LSRM_ERR_SCRATCH
    assert "scratch" in lib.lsrm_status_string(rc).decode()
    torch.cuda.synchronize()
    assert (dummy == 0).all()
