// Block metadata builders on gfx950, the steps either side of the attention
// kernels in misc/sparse_utils.py.
//
// Block separation (compute_block_separation, lines 592-641).  Token i of
// batch element b = coords[i, 0] with integer coordinates c[0..dim) lies in
// block (c[0] / bs[0], ..., c[dim-1] / bs[dim-1]), flattened row-major
// (dimension 0 most significant) over res[d] / bs[d] blocks per dimension.
// The reference counts tokens per block with torch.histc for every batch
// element and keeps the non-empty blocks in block order; here one kernel
// builds the [batch, bins] histogram with integer atomics and two scans turn
// it into cu_seqblocks (non-empty blocks per batch element, prefix) and
// cu_block_include_tokens (prefix of the non-empty counts).  Tokens outside
// the grid are not counted (histc ignores values outside [min, max]).
//
// Block sorting (sort_volume_blocks / sort_image_blocks, lines 95-152): the
// reference's sort key for every token (batch, then block coordinates, then
// in-block coordinates, with its offsets) and a stable LSD radix sort of
// (key, token index) pairs (rocPRIM); the sorted indices are the
// permutation.  The reference sorts with torch.argsort, whose order among
// equal keys is unspecified; with distinct cells the keys are distinct.
#include <rocprim/device/device_radix_sort.hpp>

#include "common.h"

namespace lsrm {

int launch_zero_i32(int32_t* p, int64_t n, hipStream_t st);  // plan.hip

struct SepGeom {
  int dim;
  int bs[3];
  int nbd[3];  // blocks per dimension = res / bs
  int64_t nbins;
};

__global__ __launch_bounds__(256) void sep_hist_kernel(const int32_t* __restrict__ coords,
                                                       int64_t n, int64_t batch, SepGeom g,
                                                       int32_t* __restrict__ counts) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t* c = coords + i * (1 + g.dim);
  const int64_t b = c[0];
  if (b < 0 || b >= batch) return;
  int64_t flat = 0;
  for (int d = 0; d < g.dim; ++d) {
    const int v = c[1 + d];
    if (v < 0) return;
    const int bd = v / g.bs[d];
    if (bd >= g.nbd[d]) return;
    flat = flat * g.nbd[d] + bd;
  }
  atomicAdd(&counts[b * g.nbins + flat], 1);
}

// Exclusive scans over the [batch * nbins] histogram (chunked: per-chunk
// sums, a scan of the sums, then the apply pass).
constexpr int SEP_T = 256;
constexpr int SEP_PER = 16;
constexpr int SEP_CHUNK = SEP_T * SEP_PER;

__device__ inline void sep_block_scan(int v, int& ex, int& tot) {
  __shared__ int s_w[SEP_T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_w[w] = x;
  __syncthreads();
  int off = 0;
  tot = 0;
  for (int k = 0; k < SEP_T / 64; ++k) {
    if (k < w) off += s_w[k];
    tot += s_w[k];
  }
  __syncthreads();
  ex = off + x - v;
}

// mode 0: value = (count > 0); mode 1: value = count.
__global__ __launch_bounds__(SEP_T) void sep_chunk_sums(const int32_t* __restrict__ counts,
                                                        int64_t m, int mode,
                                                        int32_t* __restrict__ sums) {
  const int64_t base = (int64_t)blockIdx.x * SEP_CHUNK + threadIdx.x * SEP_PER;
  int s = 0;
  for (int k = 0; k < SEP_PER; ++k) {
    const int64_t i = base + k;
    if (i < m) s += mode ? counts[i] : (counts[i] > 0);
  }
  int ex, tot;
  sep_block_scan(s, ex, tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ __launch_bounds__(SEP_T) void sep_scan_sums(int32_t* __restrict__ sums, int nch,
                                                       int32_t* __restrict__ total) {
  int carry = 0;
  for (int base = 0; base < nch; base += SEP_T) {
    const int i = base + threadIdx.x;
    const int v = i < nch ? sums[i] : 0;
    int ex, tot;
    sep_block_scan(v, ex, tot);
    if (i < nch) sums[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) *total = carry;
}

// Writes, for every non-empty bin, its block's end offset (pos[i] from the
// flag scan, tok[i] from the count scan), and cu_seqblocks at the first bin
// of every batch element.
__global__ __launch_bounds__(SEP_T) void sep_emit(const int32_t* __restrict__ counts,
                                                  int64_t m, int64_t nbins, int64_t batch,
                                                  const int32_t* __restrict__ flag_sums,
                                                  const int32_t* __restrict__ count_sums,
                                                  const int32_t* __restrict__ n_nonempty,
                                                  int32_t* __restrict__ cu_seqblocks,
                                                  int32_t* __restrict__ cu_block_tokens) {
  const int64_t base = (int64_t)blockIdx.x * SEP_CHUNK + threadIdx.x * SEP_PER;
  int f[SEP_PER], cnt[SEP_PER];
  int sf = 0, sc = 0;
  for (int k = 0; k < SEP_PER; ++k) {
    const int64_t i = base + k;
    cnt[k] = i < m ? counts[i] : 0;
    f[k] = cnt[k] > 0;
    sf += f[k];
    sc += cnt[k];
  }
  int exf, exc, tf, tc;
  sep_block_scan(sf, exf, tf);
  sep_block_scan(sc, exc, tc);
  int pos = flag_sums[blockIdx.x] + exf;
  int tok = count_sums[blockIdx.x] + exc;
  for (int k = 0; k < SEP_PER; ++k) {
    const int64_t i = base + k;
    if (i >= m) break;
    if (i % nbins == 0) cu_seqblocks[i / nbins] = pos;
    tok += cnt[k];
    if (f[k]) cu_block_tokens[pos + 1] = tok;
    pos += f[k];
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    cu_block_tokens[0] = 0;
    cu_seqblocks[batch] = *n_nonempty;
  }
}

// ------------------------------------------------------------ sort keys --
// key = sum over fields f of coef[f] * value[f], the reference's offsets:
// volume (lines 131-148): batch, c // bs (3), c % bs (3);
// image (lines 97-115): batch, image, c // bs (2), c % bs (2).
struct SortKeyGeom {
  int ncols;    // coordinate columns per token (4 volume, 4 image)
  int image;    // 1: image layout (batch, image, row, col)
  int bs;
  int64_t coef[7];
};

__global__ __launch_bounds__(256) void sort_key_kernel(const int32_t* __restrict__ coords,
                                                       int64_t n, SortKeyGeom g,
                                                       int64_t* __restrict__ keys,
                                                       int32_t* __restrict__ idx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t* c = coords + i * g.ncols;
  int64_t k;
  if (g.image) {
    k = g.coef[0] * c[0] + g.coef[1] * c[1] + g.coef[2] * (c[2] / g.bs) +
        g.coef[3] * (c[3] / g.bs) + g.coef[4] * (c[2] % g.bs) + c[3] % g.bs;
  } else {
    k = g.coef[0] * c[0] + g.coef[1] * (c[1] / g.bs) + g.coef[2] * (c[2] / g.bs) +
        g.coef[3] * (c[3] / g.bs) + g.coef[4] * (c[1] % g.bs) + g.coef[5] * (c[2] % g.bs) +
        c[3] % g.bs;
  }
  keys[i] = k;
  idx[i] = (int32_t)i;
}

}  // namespace lsrm

using namespace lsrm;

namespace {
bool sep_geom(int dim, const int32_t* block_size, const int32_t* resolution, SepGeom& g) {
  if (dim < 1 || dim > 3 || !block_size || !resolution) return false;
  g.dim = dim;
  g.nbins = 1;
  for (int d = 0; d < 3; ++d) {
    g.bs[d] = 1;
    g.nbd[d] = 1;
  }
  for (int d = 0; d < dim; ++d) {
    if (block_size[d] <= 0 || resolution[d] <= 0) return false;
    g.bs[d] = block_size[d];
    g.nbd[d] = resolution[d] / block_size[d];
    if (g.nbd[d] <= 0) return false;
    g.nbins *= g.nbd[d];
  }
  return g.nbins < (1ll << 28);
}
}  // namespace

extern "C" size_t lsrm_block_separation_workspace_size(int64_t batch, int dim,
                                                       const int32_t* block_size,
                                                       const int32_t* resolution) {
  SepGeom g;
  if (batch <= 0 || !sep_geom(dim, block_size, resolution, g)) return 0;
  const int64_t m = batch * g.nbins;
  const int64_t nch = (m + SEP_CHUNK - 1) / SEP_CHUNK;
  return (size_t)(align_up((size_t)m * 4, 256) + 2 * align_up((size_t)nch * 4, 256) + 256 + 256);
}

extern "C" int lsrm_block_separation(const int32_t* coords, int64_t n_tokens, int dim,
                                     const int32_t* block_size, const int32_t* resolution,
                                     int64_t batch, int32_t* cu_seqblocks,
                                     int32_t* cu_block_tokens, int32_t* n_blocks,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  SepGeom g;
  if (n_tokens < 0 || batch <= 0 || !cu_seqblocks || !cu_block_tokens || !n_blocks ||
      (n_tokens > 0 && !coords))
    return LSRM_ERR_INVALID_ARG;
  if (!sep_geom(dim, block_size, resolution, g)) return LSRM_ERR_UNSUPPORTED;
  const size_t need = lsrm_block_separation_workspace_size(batch, dim, block_size, resolution);
  if (!workspace || workspace_bytes < need) return LSRM_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const int64_t m = batch * g.nbins;
  const int nch = (int)((m + SEP_CHUNK - 1) / SEP_CHUNK);
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0, workspace_bytes - 256};
  int32_t* counts = ws.take<int32_t>((size_t)m);
  int32_t* fsum = ws.take<int32_t>((size_t)nch);
  int32_t* csum = ws.take<int32_t>((size_t)nch);
  int32_t* ctot = ws.take<int32_t>(1);
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  int rc = launch_zero_i32(counts, m, st);
  if (rc) return rc;
  if (n_tokens > 0)
    hipLaunchKernelGGL(sep_hist_kernel, dim3((unsigned)((n_tokens + 255) / 256)), dim3(256), 0,
                       st, coords, n_tokens, batch, g, counts);
  hipLaunchKernelGGL(sep_chunk_sums, dim3(nch), dim3(SEP_T), 0, st, counts, m, 0, fsum);
  hipLaunchKernelGGL(sep_scan_sums, dim3(1), dim3(SEP_T), 0, st, fsum, nch, n_blocks);
  hipLaunchKernelGGL(sep_chunk_sums, dim3(nch), dim3(SEP_T), 0, st, counts, m, 1, csum);
  hipLaunchKernelGGL(sep_scan_sums, dim3(1), dim3(SEP_T), 0, st, csum, nch, ctot);
  hipLaunchKernelGGL(sep_emit, dim3(nch), dim3(SEP_T), 0, st, counts, m, g.nbins, batch, fsum,
                     csum, n_blocks, cu_seqblocks, cu_block_tokens);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

namespace {
bool sort_geom(int layout, int64_t block_size, const int64_t* dims, SortKeyGeom& g) {
  // layout 0: volume, dims = {volume_res}; layout 1: image,
  // dims = {n_images, patch_res}.
  if (block_size <= 0 || !dims) return false;
  g.bs = (int)block_size;
  g.ncols = 4;
  for (int f = 0; f < 7; ++f) g.coef[f] = 0;
  const int64_t b = block_size;
  if (layout == 0) {
    const int64_t r = dims[0];
    if (r <= 0) return false;
    g.image = 0;
    g.coef[0] = r * r * r;  // offset1..offset6 of sort_volume_blocks
    g.coef[1] = r * r * b;
    g.coef[2] = r * b * b;
    g.coef[3] = b * b * b;
    g.coef[4] = b * b;
    g.coef[5] = b;
    return true;
  }
  if (layout == 1) {
    const int64_t im = dims[0], pr = dims[1];
    if (im <= 0 || pr <= 0) return false;
    g.image = 1;
    g.coef[0] = im * pr * pr;  // offset1..offset5 of sort_image_blocks
    g.coef[1] = pr * pr;
    g.coef[2] = pr * b;
    g.coef[3] = b * b;
    g.coef[4] = b;
    return true;
  }
  return false;
}

size_t sort_temp_bytes(int64_t n) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, bytes, (const int64_t*)nullptr, (int64_t*)nullptr,
                                  (const int32_t*)nullptr, (int32_t*)nullptr, (unsigned)n, 0,
                                  63, (hipStream_t)0);
  return bytes;
}
}  // namespace

extern "C" size_t lsrm_block_sort_workspace_size(int64_t n_tokens) {
  if (n_tokens < 0 || n_tokens > INT32_MAX) return 0;
  const int64_t n = n_tokens > 0 ? n_tokens : 1;
  return align_up((size_t)n * 8, 256) * 2 + align_up((size_t)n * 4, 256) +
         align_up(sort_temp_bytes(n), 256) + 256;
}

extern "C" int lsrm_block_sort(const int32_t* coords, int64_t n_tokens, int layout,
                               int64_t block_size, const int64_t* dims, int32_t* perm,
                               void* workspace, size_t workspace_bytes, void* stream) {
  SortKeyGeom g;
  if (n_tokens < 0 || n_tokens > INT32_MAX || (n_tokens > 0 && (!coords || !perm)))
    return LSRM_ERR_INVALID_ARG;
  if (!sort_geom(layout, block_size, dims, g)) return LSRM_ERR_UNSUPPORTED;
  if (n_tokens == 0) return LSRM_OK;
  const size_t need = lsrm_block_sort_workspace_size(n_tokens);
  if (!workspace || workspace_bytes < need) return LSRM_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0, workspace_bytes - 256};
  int64_t* keys = ws.take<int64_t>((size_t)n_tokens);
  int64_t* keys_out = ws.take<int64_t>((size_t)n_tokens);
  int32_t* idx = ws.take<int32_t>((size_t)n_tokens);
  size_t tb = sort_temp_bytes(n_tokens);
  char* temp = ws.take<char>(tb);
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  hipLaunchKernelGGL(sort_key_kernel, dim3((unsigned)((n_tokens + 255) / 256)), dim3(256), 0,
                     st, coords, n_tokens, g, keys, idx);
  LSRM_CHECK_LAUNCH();
  // Keys are non-negative for in-range coordinates: 63 bits order them.
  if (rocprim::radix_sort_pairs(temp, tb, keys, keys_out, idx, perm, (unsigned)n_tokens, 0, 63,
                                st) != hipSuccess)
    return LSRM_ERR_LAUNCH;
  return LSRM_OK;
}
