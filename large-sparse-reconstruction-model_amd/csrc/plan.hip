// Planning kernels: batched exclusive scans, query-tile plans, reverse (CSR)
// maps with a deterministic per-segment sort, key-chunk items, metadata
// validation and per-token block ids.
//
// The reverse map replaces the reference's _count_queries_kernel /
// _scatter_queries_kernel / host-looped segmented sort
// (sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:494-684),
// all on the device and without host synchronisation: for rows that are
// queries, one stable radix sort of (head * n_blocks + block, listing) pairs
// generated in (head, query, slot) order; for rows that are run tiles,
// count -> scan -> atomic scatter -> per-segment sort.
#include <algorithm>
#include <rocprim/device/device_radix_sort.hpp>

#include "plan.h"

namespace lsrm {

constexpr int SCAN_T = 256;
constexpr int SCAN_PER = 16;
constexpr int SCAN_CHUNK = SCAN_T * SCAN_PER;

__device__ inline int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Exclusive scan of one value per thread over a 256-thread block; returns the
// exclusive prefix and writes the block total to *total.
__device__ inline int block_excl_scan(int v, int* total) {
  __shared__ int s_w[SCAN_T / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_w[w] = x;
  __syncthreads();
  int off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < SCAN_T / 64; ++i) {
    if (i < w) off += s_w[i];
    tot += s_w[i];
  }
  __syncthreads();
  *total = tot;
  return off + x - v;
}

template <class F>
__global__ __launch_bounds__(SCAN_T) void scan_reduce(F f, int64_t n,
                                                      int32_t* sums,
                                                      int nchunks) {
  const int seg = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * SCAN_CHUNK + threadIdx.x * SCAN_PER;
  const int64_t lim = f.limit(seg, n);
  int s = 0;
  for (int i = 0; i < SCAN_PER; ++i) {
    const int64_t idx = base + i;
    if (idx < lim) s += f(seg, idx);
  }
  int tot;
  block_excl_scan(s, &tot);
  if (threadIdx.x == 0) sums[(int64_t)seg * nchunks + blockIdx.x] = tot;
}

// In-place exclusive scan of each segment's chunk sums; totals[seg] = total.
__global__ __launch_bounds__(SCAN_T) void scan_chunks(int32_t* sums,
                                                      int nchunks,
                                                      int32_t* totals) {
  const int seg = blockIdx.x;
  int32_t* p = sums + (int64_t)seg * nchunks;
  int carry = 0;
  for (int base = 0; base < nchunks; base += SCAN_T) {
    const int i = base + threadIdx.x;
    const int v = i < nchunks ? p[i] : 0;
    int tot;
    const int ex = block_excl_scan(v, &tot);
    if (i < nchunks) p[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0) totals[seg] = carry;
}

template <class F, class W>
__global__ __launch_bounds__(SCAN_T) void scan_apply(F f, W w, int64_t n,
                                                     const int32_t* sums,
                                                     int nchunks) {
  const int seg = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * SCAN_CHUNK + threadIdx.x * SCAN_PER;
  const int64_t lim = f.limit(seg, n);
  int v[SCAN_PER];
  int s = 0;
#pragma unroll
  for (int i = 0; i < SCAN_PER; ++i) {
    const int64_t idx = base + i;
    v[i] = idx < lim ? f(seg, idx) : 0;
    s += v[i];
  }
  int tot;
  int ex = block_excl_scan(s, &tot) + sums[(int64_t)seg * nchunks + blockIdx.x];
#pragma unroll
  for (int i = 0; i < SCAN_PER; ++i) {
    const int64_t idx = base + i;
    if (idx < lim) w(seg, idx, ex, v[i], lim);
    ex += v[i];
  }
}

// Runs scan_reduce / scan_chunks / scan_apply over `nseg` segments of at
// most n elements; totals[seg] receives each segment's sum.
template <class F, class W>
int run_scan(F f, W w, int64_t n, int nseg, int32_t* chunk_sums,
             int32_t* totals, hipStream_t st) {
  if (n <= 0 || nseg <= 0) return LSRM_OK;
  const int nchunks = ceil_div(n, SCAN_CHUNK);
  dim3 grid(nchunks, nseg);
  hipLaunchKernelGGL((scan_reduce<F>), grid, dim3(SCAN_T), 0, st, f, n,
                     chunk_sums, nchunks);
  hipLaunchKernelGGL(scan_chunks, dim3(nseg), dim3(SCAN_T), 0, st, chunk_sums,
                     nchunks, totals);
  hipLaunchKernelGGL((scan_apply<F, W>), grid, dim3(SCAN_T), 0, st, f, w, n,
                     chunk_sums, nchunks);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

inline int64_t scan_sums_size(int64_t n, int64_t nseg) {
  return (int64_t)ceil_div(n > 0 ? n : 1, SCAN_CHUNK) * nseg;
}

// ------------------------------------------------------------- utilities --

__global__ void zero_i32_kernel(int32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

int launch_zero_i32(int32_t* p, int64_t n, hipStream_t st) {
  if (n <= 0) return LSRM_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     p, n);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

// Number of valid (batch-local id in [0, nbb)) entries in a selection row is
// not needed; rows compare by their sequence of normalised entries.
__device__ inline int norm_entry(int v, int nbb) {
  return (v >= 0 && v < nbb) ? v : -1;
}

// --------------------------------------------------------------- tiles --

// brk[h, i] = 1 where a new run of identical (normalised) rows starts.
__global__ __launch_bounds__(256) void breaks_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, uint8_t* __restrict__ brk) {
  const int h = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nq) return;
  int b, bs, nbb;
  bool start;
  query_batch(cu_q, batch, cu_sb, i, &b, &bs, &nbb, &start);
  bool br = (i == 0) || start;
  if (!br) {
    const int32_t* r1 = topk + ((int64_t)h * nq + i) * k;
    const int32_t* r0 = r1 - k;
    for (int j = 0; j < k; ++j) {
      if (norm_entry(r1[j], nbb) != norm_entry(r0[j], nbb)) {
        br = true;
        break;
      }
    }
  }
  brk[(int64_t)h * nq + i] = br ? 1 : 0;
}

// Same as breaks_kernel for k % 4 == 0 and 16-byte-aligned rows: each
// thread reads its row with 16-byte loads (a wave reads 64 consecutive rows
// contiguously) and takes the previous row from the neighbouring lane.
__global__ __launch_bounds__(256) void breaks_vec_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, uint8_t* __restrict__ brk) {
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = i < nq;
  int b = 0, bs = 0, nbb = 0;
  bool start = true;
  if (live) query_batch(cu_q, batch, cu_sb, i, &b, &bs, &nbb, &start);
  const int64_t ii = live ? i : nq - 1;
  const u32x4* r1 = reinterpret_cast<const u32x4*>(topk + ((int64_t)h * nq + ii) * k);
  const u32x4* r0 = reinterpret_cast<const u32x4*>(
      topk + ((int64_t)h * nq + (ii > 0 ? ii - 1 : 0)) * k);
  bool diff = false;
  for (int c = 0; c < k / 4; ++c) {
    const u32x4 cur = r1[c];
    u32x4 prev;
#pragma unroll
    for (int e = 0; e < 4; ++e) prev[e] = (uint32_t)__shfl_up((int)cur[e], 1);
    if (lane == 0) prev = r0[c];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      diff |= norm_entry((int)cur[e], nbb) != norm_entry((int)prev[e], nbb);
  }
  if (live) brk[(int64_t)h * nq + i] = (i == 0 || start || diff) ? 1 : 0;
}

// Same for rows of P 16-byte pieces (k = 4 P), P a power of two <= 64: lane
// (row i, piece p) holds piece p of row i, so a wave reads 64 / P whole rows
// as one contiguous run per load; piece p of row i - 1 is the lane P below
// (the last row of the previous group, or a load for the wave's first row),
// and the P lanes of a row OR their differences.  A wave covers BRK_G such
// groups with all their loads in flight, and looks its batch element up once
// when its rows lie inside one (else row by row).
constexpr int BRK_G = 8;
template <int P>
__global__ __launch_bounds__(256) void breaks_rows_kernel(
    const int32_t* __restrict__ topk, int64_t nq, const int32_t* __restrict__ cu_q,
    int64_t batch, const int32_t* __restrict__ cu_sb, uint8_t* __restrict__ brk) {
  static_assert(P >= 1 && P <= 64 && (P & (P - 1)) == 0, "rows must tile a wave");
  constexpr int RPW = 64 / P;  // rows per group
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t i0 =
      ((int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)) * (RPW * BRK_G);
  if (i0 >= nq) return;  // whole waves
  const int p = lane % P, rl = lane / P;
  const u32x4* rows = reinterpret_cast<const u32x4*>(topk + (int64_t)h * nq * (4 * P));
  u32x4 cur[BRK_G];
#pragma unroll
  for (int g = 0; g < BRK_G; ++g) {
    const int64_t i = i0 + g * RPW + rl;
    cur[g] = rows[(i < nq ? i : nq - 1) * P + p];
  }
  u32x4 first_prev = cur[0];
  if (lane < P && i0 > 0) first_prev = rows[(i0 - 1) * P + p];
  const int64_t i_last = i0 + RPW * BRK_G - 1 < nq ? i0 + RPW * BRK_G - 1 : nq - 1;
  int b0 = 0, bs0 = 0, nbb0 = 0;
  bool st0 = true;
  query_batch(cu_q, batch, cu_sb, i0, &b0, &bs0, &nbb0, &st0);
  const int64_t qs0 = b0 >= 0 ? cu_q[b0] : 0;
  const bool one = b0 >= 0 && i_last < (int64_t)cu_q[b0 + 1];
#pragma unroll
  for (int g = 0; g < BRK_G; ++g) {
    const int64_t i = i0 + g * RPW + rl;
    u32x4 prev;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int up = __shfl_up((int)cur[g][e], P);
      const int last = g > 0 ? __shfl((int)cur[g > 0 ? g - 1 : 0][e], (RPW - 1) * P + p)
                             : (int)first_prev[e];
      prev[e] = (uint32_t)(lane >= P ? up : last);
    }
    int nbb = nbb0;
    bool start = i == qs0;
    if (!one && i < nq) {
      int b, bs;
      query_batch(cu_q, batch, cu_sb, i, &b, &bs, &nbb, &start);
    }
    int diff = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      diff |= norm_entry((int)cur[g][e], nbb) != norm_entry((int)prev[e], nbb) ? 1 : 0;
#pragma unroll
    for (int o = 1; o < P; o <<= 1) diff |= __shfl_xor(diff, o);
    if (i < nq && p == 0) brk[(int64_t)h * nq + i] = (i == 0 || start || diff) ? 1 : 0;
  }
}

struct BrkF {
  const uint8_t* brk;
  int64_t nq;
  __device__ int64_t limit(int, int64_t n) const { return n; }
  __device__ int operator()(int h, int64_t i) const {
    return brk[(int64_t)h * nq + i];
  }
};
struct RunStartW {
  int32_t* run_start;  // [hkv, nq + 1]
  int64_t nq;
  __device__ void operator()(int h, int64_t i, int ex, int v,
                             int64_t lim) const {
    int32_t* rs = run_start + (int64_t)h * (nq + 1);
    if (v) rs[ex] = (int32_t)i;
    if (i == lim - 1) rs[ex + v] = (int32_t)nq;
  }
};

struct RunTilesF {
  const int32_t* run_start;
  const int32_t* n_runs;  // [hkv]
  int64_t nq;
  int tq;
  __device__ int64_t limit(int h, int64_t) const { return n_runs[h]; }
  __device__ int operator()(int h, int64_t r) const {
    const int32_t* rs = run_start + (int64_t)h * (nq + 1);
    const int len = rs[r + 1] - rs[r];
    return (len + tq - 1) / tq;
  }
};
struct EmitTilesW {
  const int32_t* run_start;
  int2* tiles;
  int64_t nq;
  int tq;
  __device__ void operator()(int h, int64_t r, int ex, int v, int64_t) const {
    const int32_t* rs = run_start + (int64_t)h * (nq + 1);
    const int s = rs[r];
    const int len = rs[r + 1] - s;
    int2* out = tiles + (int64_t)h * nq + ex;
    for (int t = 0; t < v; ++t) {
      const int q0 = s + t * tq;
      const int rem = len - t * tq;
      out[t] = make_int2(q0, rem < tq ? rem : tq);
    }
  }
};


// --------------------------------------------------------- union tiles --
// Consecutive short run tiles (fewer than tq / 4 queries) of one batch
// element whose first queries fall in the same window of 3 tq / 4 queries
// form a group of at most tq - 1 queries; two neighbours of which one has 8
// or more queries join only when their rows share at least half of the
// first one's valid ids.  Per-token rows change every few queries and share
// most blocks with their neighbours; a block-row selection's short runs are
// whole small blocks whose neighbours select other blocks (config 5: 0-6 of
// 32 shared), where the union only adds masked keys to a tile that already
// runs as a whole tile of its own.  Groups of two or more run tiles
// become grouped tiles (TilePlan::gtiles): the forward runs them over the
// union of their queries' selections with a per-query mask, or run by run
// when that is cheaper.  Every other run tile is kept as it is.
constexpr int GROUP_FEW_Q = 8;

// gbrk[h, t] = 1 where run tile t starts a new group.  One thread per tile
// decides the plain cases; the tiles that need the shared-ids count (at most
// a few hundred per head) are taken one at a time by their whole wave: lane
// j holds id j of both rows (one load round for rows of <= 64 ids) and the
// other row's ids are broadcast with readlane.
__global__ __launch_bounds__(256) void group_breaks_kernel(
    const int2* __restrict__ tiles, const int32_t* __restrict__ count,
    const int32_t* __restrict__ cu_q, int64_t batch, const int32_t* __restrict__ topk,
    int64_t nq, int k, int short_q, int window_q, uint8_t* __restrict__ gbrk) {
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t cnt = count[h];
  int brk = 1;
  bool check = false;
  int qa = 0, qb = 0;
  if (t > 0 && t < cnt) {
    const int2 a = tiles[(int64_t)h * nq + t - 1], b = tiles[(int64_t)h * nq + t];
    if (a.y < short_q && b.y < short_q && a.x / window_q == b.x / window_q &&
        batch_of(cu_q, batch, a.x) == batch_of(cu_q, batch, b.x)) {
      if (a.y < GROUP_FEW_Q && b.y < GROUP_FEW_Q) {
        brk = 0;
      } else {
        // a run's rows are identical: its first query's row stands for it
        check = true;
        qa = a.x;
        qb = b.x;
      }
    }
  }
  uint64_t pend = __ballot(check);
  while (pend) {
    const int l = __builtin_ctzll(pend);
    pend &= pend - 1;
    const int64_t ra = ((int64_t)h * nq + __builtin_amdgcn_readlane(qa, l)) * k;
    const int64_t rb = ((int64_t)h * nq + __builtin_amdgcn_readlane(qb, l)) * k;
    int valid = 0, shared = 0;
    for (int c0 = 0; c0 < k; c0 += 64) {
      const int x = c0 + lane < k ? topk[ra + c0 + lane] : -1;
      bool hit = false;
      for (int d0 = 0; d0 < k; d0 += 64) {
        const int y = d0 + lane < k ? topk[rb + d0 + lane] : -1;
        const int m_end = k - d0 < 64 ? k - d0 : 64;
        for (int m = 0; m < m_end; ++m) hit |= x == __builtin_amdgcn_readlane(y, m);
      }
      valid += __popcll(__ballot(x >= 0));
      shared += __popcll(__ballot(x >= 0 && hit));
    }
    if (lane == l) brk = 2 * shared >= valid ? 0 : 1;
  }
  if (t < cnt) gbrk[(int64_t)h * nq + t] = (uint8_t)brk;
}

struct GroupF {
  const uint8_t* gbrk;
  const int32_t* count;
  int64_t nq;
  __device__ int64_t limit(int h, int64_t) const { return count[h]; }
  __device__ int operator()(int h, int64_t t) const { return gbrk[(int64_t)h * nq + t]; }
};
struct GroupW {
  int32_t* gstart;  // [hkv, nq + 1]
  int64_t nq;
  __device__ void operator()(int h, int64_t t, int ex, int v, int64_t lim) const {
    int32_t* gs = gstart + (int64_t)h * (nq + 1);
    if (v) gs[ex] = (int32_t)t;
    if (t == lim - 1) gs[ex + v] = (int32_t)lim;
  }
};
// Second pass over the groups: grouped (>= 2 run tiles) or kept.
struct SplitF {
  const int32_t* gstart;
  const int32_t* n_groups;
  int64_t nq;
  __device__ int64_t limit(int h, int64_t) const { return n_groups[h]; }
  __device__ int operator()(int h, int64_t s) const {
    const int32_t* gs = gstart + (int64_t)h * (nq + 1);
    return gs[s + 1] - gs[s] > 1 ? 1 : 0;
  }
};
struct SplitW {
  const int2* run_tiles;
  const int32_t* gstart;
  int64_t nq;
  int2* tiles;
  int2* gtiles;
  __device__ void operator()(int h, int64_t s, int ex, int v, int64_t) const {
    const int32_t* gs = gstart + (int64_t)h * (nq + 1);
    const int t0 = gs[s], t1 = gs[s + 1];
    const int2 first = run_tiles[(int64_t)h * nq + t0];
    const int2 last = run_tiles[(int64_t)h * nq + t1 - 1];
    const int2 out = make_int2(first.x, last.x + last.y - first.x);
    if (v)
      gtiles[(int64_t)h * nq + ex] = out;
    else
      tiles[(int64_t)h * nq + (s - ex)] = out;
  }
};

// tile_count = groups - grouped tiles (grouping) or the run count.
__global__ void plan_offsets_kernel(const int32_t* n_groups, int32_t* tile_count,
                                    const int32_t* gtile_count, int hkv,
                                    int32_t* head_off, int32_t* ghead_off,
                                    int32_t* counter) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    int acc = 0, gacc = 0;
    head_off[0] = 0;
    ghead_off[0] = 0;
    for (int h = 0; h < hkv; ++h) {
      const int g = gtile_count[h];
      const int c = n_groups ? n_groups[h] - g : tile_count[h];
      tile_count[h] = c;
      acc += c;
      gacc += g;
      head_off[h + 1] = acc;
      ghead_off[h + 1] = gacc;
    }
    for (int i = 0; i < PLAN_BWD_SLOT; ++i) counter[i] = 0;
    counter[PLAN_BWD_SLOT] = 0;  // set again by mark_backward_plan
    counter[PLAN_KC_SLOT] = 0;   // set again by the key-centric part
  }
}

__global__ void mark_backward_plan_kernel(int32_t* counter) {
  if (threadIdx.x == 0 && blockIdx.x == 0) counter[PLAN_BWD_SLOT] = PLAN_BWD_MAGIC;
}

int mark_backward_plan(int32_t* counter, hipStream_t st) {
  hipLaunchKernelGGL(mark_backward_plan_kernel, dim3(1), dim3(64), 0, st, counter);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

int build_tile_plan(const int32_t* topk, int64_t hkv, int64_t nq,
                    int64_t topk_n, const int32_t* cu_q, int64_t batch,
                    const int32_t* cu_sb, int tq, Carver& ws, TilePlan& plan,
                    hipStream_t st, bool group_short) {
  uint8_t* brk = ws.take<uint8_t>((size_t)(hkv * nq));
  int32_t* run_start = ws.take<int32_t>((size_t)(hkv * (nq + 1)));
  int32_t* n_runs = ws.take<int32_t>((size_t)hkv);
  int32_t* sums = ws.take<int32_t>((size_t)scan_sums_size(nq, hkv));
  plan.tiles = ws.take<int2>((size_t)(hkv * (nq > 0 ? nq : 1)));
  plan.tile_count = ws.take<int32_t>((size_t)hkv);
  plan.head_off = ws.take<int32_t>((size_t)(hkv + 1));
  plan.counter = ws.take<int32_t>(64);
  plan.gtile_count = ws.take<int32_t>((size_t)hkv);
  plan.ghead_off = ws.take<int32_t>((size_t)(hkv + 1));
  plan.gtiles = nullptr;
  int2* run_tiles = plan.tiles;
  int32_t* run_count = plan.tile_count;
  int32_t* gstart = nullptr;
  int32_t* n_groups = nullptr;
  if (group_short) {
    plan.gtiles = ws.take<int2>((size_t)(hkv * (nq > 0 ? nq : 1)));
    run_tiles = ws.take<int2>((size_t)(hkv * (nq > 0 ? nq : 1)));
    run_count = ws.take<int32_t>((size_t)hkv);
    gstart = ws.take<int32_t>((size_t)(hkv * (nq + 1)));
    n_groups = ws.take<int32_t>((size_t)hkv);
  }
  if (!ws.base || ws.dry) return LSRM_OK;
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  int rc0 = launch_zero_i32(plan.gtile_count, hkv, st);
  if (rc0) return rc0;

  if (nq > 0) {
    dim3 grid(ceil_div(nq, 256), (unsigned)hkv);
    const int64_t pieces = topk_n / 4;
    const bool vec = topk_n % 4 == 0 && ((uintptr_t)topk % 16) == 0;
    // Rows of 4 or more pieces: one row per lane would read 64 rows' worth
    // of lines per load and lose them between the row's loads (config 5's
    // 128-byte rows fetched 6.9x their bytes); with eight row groups per wave
    // the piece-per-lane form also beats it on 64-byte rows (top-16: 42 -> 39
    // us on average over bench.py's plans).  Shorter rows keep one per lane.
    if (vec && pieces >= 4 && pieces <= 64 && (pieces & (pieces - 1)) == 0) {
      // one wave per BRK_G groups of 64 / pieces rows, four waves per block
      const dim3 grow(ceil_div(ceil_div(nq, (64 / pieces) * BRK_G), 4), (unsigned)hkv);
#define LSRM_BRK(P)                                                                  \
  case P:                                                                            \
    hipLaunchKernelGGL(breaks_rows_kernel<P>, grow, dim3(256), 0, st, topk, nq, cu_q, \
                       batch, cu_sb, brk);                                           \
    break;
      switch (pieces) {
        LSRM_BRK(4) LSRM_BRK(8) LSRM_BRK(16) LSRM_BRK(32) LSRM_BRK(64)
      }
#undef LSRM_BRK
    } else if (vec)
      hipLaunchKernelGGL(breaks_vec_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, brk);
    else
      hipLaunchKernelGGL(breaks_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, brk);
    LSRM_CHECK_LAUNCH();
    int rc = run_scan(BrkF{brk, nq}, RunStartW{run_start, nq}, nq, (int)hkv,
                      sums, n_runs, st);
    if (rc) return rc;
    rc = run_scan(RunTilesF{run_start, n_runs, nq, tq},
                  EmitTilesW{run_start, run_tiles, nq, tq}, nq, (int)hkv, sums,
                  run_count, st);
    if (rc) return rc;
    if (group_short) {
      const int short_q = tq / 4 > 1 ? tq / 4 : 1;
      const int window_q = (3 * tq) / 4 > 1 ? (3 * tq) / 4 : 1;
      // brk is free again: it takes the group starts
      hipLaunchKernelGGL(group_breaks_kernel, grid, dim3(256), 0, st, run_tiles, run_count,
                         cu_q, batch, topk, nq, (int)topk_n, short_q, window_q, brk);
      LSRM_CHECK_LAUNCH();
      rc = run_scan(GroupF{brk, run_count, nq},
                    GroupW{gstart, nq}, nq, (int)hkv, sums, n_groups, st);
      if (rc) return rc;
      rc = run_scan(SplitF{gstart, n_groups, nq},
                    SplitW{run_tiles, gstart, nq, plan.tiles, plan.gtiles}, nq, (int)hkv,
                    sums, plan.gtile_count, st);
      if (rc) return rc;
    }
  } else {
    int rc = launch_zero_i32(plan.tile_count, hkv, st);
    if (rc) return rc;
    n_groups = nullptr;
  }
  hipLaunchKernelGGL(plan_offsets_kernel, dim3(1), dim3(64), 0, st,
                     nq > 0 ? n_groups : nullptr, plan.tile_count, plan.gtile_count, (int)hkv,
                     plan.head_off, plan.ghead_off, plan.counter);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

// --------------------------------------------------------- reverse map --

// Row source: row r of head h reads the selection of query `query(h, r)`;
// rows that `skip` are not entered.
struct RowSrc {
  const int2* tiles;      // null: rows are queries
  const int32_t* count;   // rows per head (tiles) or null
  int64_t nq;
  const uint8_t* only;    // rows are queries: [hkv, nq] mask, or null (all)
  int enc;                // > 0: a listing stores row * enc + slot (enc = topk)
  __device__ int64_t n_rows(int h) const {
    return tiles ? (int64_t)count[h] : nq;
  }
  // Range of the stored values (the counting sort's key range).
  __device__ int64_t n_values(int h) const { return n_rows(h) * (enc > 0 ? enc : 1); }
  __device__ int64_t query(int h, int64_t r) const {
    return tiles ? (int64_t)tiles[(int64_t)h * nq + r].x : r;
  }
  __device__ bool skip(int h, int64_t r) const {
    return !tiles && only && !only[(int64_t)h * nq + r];
  }
};

__global__ __launch_bounds__(256) void rev_count_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, int64_t nb, RowSrc rows,
    int32_t* __restrict__ counts) {
  const int h = blockIdx.y;
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows.n_rows(h) || rows.skip(h, r)) return;
  const int64_t q = rows.query(h, r);
  int b, bs, nbb;
  bool start;
  query_batch(cu_q, batch, cu_sb, q, &b, &bs, &nbb, &start);
  const int32_t* row = topk + ((int64_t)h * nq + q) * k;
  for (int j = 0; j < k; ++j) {
    const int v = row[j];
    if (v >= 0 && v < nbb && (int64_t)bs + v < nb)
      atomicAdd(&counts[(int64_t)h * nb + bs + v], 1);
  }
}

__global__ __launch_bounds__(256) void rev_scatter_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, int64_t nb, RowSrc rows,
    const int32_t* __restrict__ cu_rev, int32_t* __restrict__ fill,
    int32_t* __restrict__ rev, int64_t cap) {
  const int h = blockIdx.y;
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows.n_rows(h) || rows.skip(h, r)) return;
  const int64_t q = rows.query(h, r);
  int b, bs, nbb;
  bool start;
  query_batch(cu_q, batch, cu_sb, q, &b, &bs, &nbb, &start);
  const int32_t* row = topk + ((int64_t)h * nq + q) * k;
  for (int j = 0; j < k; ++j) {
    const int v = row[j];
    if (v >= 0 && v < nbb && (int64_t)bs + v < nb) {
      const int64_t c = bs + v;
      const int64_t pos =
          cu_rev[(int64_t)h * (nb + 1) + c] +
          atomicAdd(&fill[(int64_t)h * nb + c], 1);
      if (pos < cap) rev[(int64_t)h * cap + pos] = (int32_t)(rows.enc > 0 ? r * rows.enc + j : r);
    }
  }
}

// rev_count_kernel / rev_scatter_kernel with the workgroup's listings first
// gathered in LDS (nb <= REV_LDS_BINS): a block listed by many rows (the
// forced blocks, listed by every tile) takes one global atomic per
// workgroup instead of one per listing.  The scatter reserves each block's
// range for the workgroup with one atomic and places its listings in that
// range through LDS counters; the segment sort that follows fixes the order.
constexpr int REV_LDS_BINS = 8192;

__global__ __launch_bounds__(256) void rev_count_lds_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, int64_t nb, RowSrc rows,
    int32_t* __restrict__ counts) {
  __shared__ int hist[REV_LDS_BINS];
  const int h = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * blockDim.x;
  if (r0 >= rows.n_rows(h)) return;  // whole workgroup
  for (int i = threadIdx.x; i < nb; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  const int64_t r = r0 + threadIdx.x;
  if (r < rows.n_rows(h) && !rows.skip(h, r)) {
    const int64_t q = rows.query(h, r);
    int b, bs, nbb;
    bool start;
    query_batch(cu_q, batch, cu_sb, q, &b, &bs, &nbb, &start);
    const int32_t* row = topk + ((int64_t)h * nq + q) * k;
    for (int j = 0; j < k; ++j) {
      const int v = row[j];
      if (v >= 0 && v < nbb && (int64_t)bs + v < nb) atomicAdd(&hist[bs + v], 1);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb; i += blockDim.x)
    if (hist[i]) atomicAdd(&counts[(int64_t)h * nb + i], hist[i]);
}

__global__ __launch_bounds__(256) void rev_scatter_lds_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, int64_t nb, RowSrc rows,
    const int32_t* __restrict__ cu_rev, int32_t* __restrict__ fill,
    int32_t* __restrict__ rev, int64_t cap) {
  __shared__ int cnt[REV_LDS_BINS];   // listings of the workgroup, then its base
  __shared__ int local[REV_LDS_BINS];  // placed so far
  const int h = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * blockDim.x;
  if (r0 >= rows.n_rows(h)) return;  // whole workgroup
  for (int i = threadIdx.x; i < nb; i += blockDim.x) {
    cnt[i] = 0;
    local[i] = 0;
  }
  __syncthreads();
  const int64_t r = r0 + threadIdx.x;
  const bool on = r < rows.n_rows(h) && !rows.skip(h, r);
  int bs = 0, nbb = 0;
  const int32_t* row = topk;
  if (on) {
    const int64_t q = rows.query(h, r);
    int b;
    bool start;
    query_batch(cu_q, batch, cu_sb, q, &b, &bs, &nbb, &start);
    row = topk + ((int64_t)h * nq + q) * k;
    for (int j = 0; j < k; ++j) {
      const int v = row[j];
      if (v >= 0 && v < nbb && (int64_t)bs + v < nb) atomicAdd(&cnt[bs + v], 1);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb; i += blockDim.x)
    if (cnt[i]) cnt[i] = atomicAdd(&fill[(int64_t)h * nb + i], cnt[i]);
  __syncthreads();
  if (on) {
    for (int j = 0; j < k; ++j) {
      const int v = row[j];
      if (v >= 0 && v < nbb && (int64_t)bs + v < nb) {
        const int64_t c = bs + v;
        const int64_t pos = cu_rev[(int64_t)h * (nb + 1) + c] + cnt[c] + atomicAdd(&local[c], 1);
        if (pos < cap) rev[(int64_t)h * cap + pos] = (int32_t)(rows.enc > 0 ? r * rows.enc + j : r);
      }
    }
  }
}

struct CountF {
  const int32_t* counts;
  int64_t nb;
  __device__ int64_t limit(int, int64_t n) const { return n; }
  __device__ int operator()(int h, int64_t c) const {
    return counts[(int64_t)h * nb + c];
  }
};
struct CuRevW {
  int32_t* cu_rev;
  int64_t nb;
  __device__ void operator()(int h, int64_t c, int ex, int v,
                             int64_t lim) const {
    int32_t* p = cu_rev + (int64_t)h * (nb + 1);
    p[c] = ex;
    if (c == lim - 1) p[c + 1] = ex + v;
  }
};

constexpr int SORT_CAP = 8192;  // segments sorted in LDS up to this length

// Sorts every segment rev[h, cu_rev[h,c] .. cu_rev[h,c+1]) ascending.  Short
// segments use an LDS bitonic sort; longer ones a windowed counting sort over
// the row-id range through `aux` (same shape as rev).
__global__ __launch_bounds__(256) void rev_sort_kernel(
    const int32_t* __restrict__ cu_rev, int32_t* __restrict__ rev,
    int32_t* __restrict__ aux, int64_t nb, int64_t cap, RowSrc rows) {
  __shared__ int s[SORT_CAP];
  const int h = blockIdx.y;
  const int64_t c = blockIdx.x;
  const int64_t s0 = cu_rev[(int64_t)h * (nb + 1) + c];
  int64_t s1 = cu_rev[(int64_t)h * (nb + 1) + c + 1];
  if (s1 > cap) s1 = cap;
  const int64_t len = s1 - s0;
  if (len <= 1) return;
  int32_t* seg = rev + (int64_t)h * cap + s0;
  if (len <= SORT_CAP) {
    int p = 1;
    while (p < len) p <<= 1;
    for (int i = threadIdx.x; i < p; i += blockDim.x)
      s[i] = i < len ? seg[i] : INT32_MAX;
    __syncthreads();
    for (int kk = 2; kk <= p; kk <<= 1) {
      for (int j = kk >> 1; j > 0; j >>= 1) {
        for (int i = threadIdx.x; i < p; i += blockDim.x) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const bool up = (i & kk) == 0;
            const int a = s[i], bb = s[ixj];
            if ((a > bb) == up) {
              s[i] = bb;
              s[ixj] = a;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int i = threadIdx.x; i < len; i += blockDim.x) seg[i] = s[i];
    return;
  }
  // Windowed counting sort: values are row ids in [0, n_rows) (or encoded
  // listings in [0, n_rows * enc)).
  int32_t* out = aux + (int64_t)h * cap + s0;
  const int64_t range = rows.n_values(h);
  __shared__ int s_base;
  if (threadIdx.x == 0) s_base = 0;
  __syncthreads();
  for (int64_t w0 = 0; w0 < range; w0 += SORT_CAP) {
    for (int i = threadIdx.x; i < SORT_CAP; i += blockDim.x) s[i] = 0;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) {
      const int64_t v = seg[i] - w0;
      if (v >= 0 && v < SORT_CAP) atomicAdd(&s[v], 1);
    }
    __syncthreads();
    // Exclusive scan of the window counts: 256 threads x 32 entries.
    constexpr int PER = SORT_CAP / 256;
    int loc[PER];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      loc[i] = s[threadIdx.x * PER + i];
      sum += loc[i];
    }
    int tot;
    int ex = block_excl_scan(sum, &tot) + s_base;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int n = loc[i];
      for (int m = 0; m < n; ++m)
        out[ex + m] = (int32_t)(w0 + threadIdx.x * PER + i);
      ex += n;
    }
    __syncthreads();
    if (threadIdx.x == 0) s_base += tot;
    __syncthreads();
  }
  for (int64_t i = threadIdx.x; i < len; i += blockDim.x) seg[i] = out[i];
}

// ------------------------------------- query rows: one stable radix sort --

// Pair i = (h * nq + q) * k + j: key h * nb + block for a valid slot of a
// marked query, else the sentinel hkv * nb; value the listing (q, or
// q * k + j when encoding the slot).  Generated in (h, q, j) order, so the
// stable sort leaves each block's listings ascending.  One thread per pair
// (n = hkv * nq * k < 2^31, checked by the caller): the row reads and the
// key / value writes are contiguous across the wave.
__global__ __launch_bounds__(256) void rev_pairs_kernel(
    const int32_t* __restrict__ topk, int64_t hkv, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch, const int32_t* __restrict__ cu_sb,
    int64_t nb, const uint8_t* __restrict__ only, bool encode, uint32_t* __restrict__ keys,
    int32_t* __restrict__ vals) {
  // 32-bit index arithmetic (every index here is below 2^31); a grid-stride
  // loop over a bounded grid
  const uint32_t n = (uint32_t)(hkv * nq * k);
  const uint32_t none = (uint32_t)(hkv * nb);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const uint32_t hq = i / (uint32_t)k;  // h * nq + q
    const int j = (int)(i - hq * (uint32_t)k);
    const int h = (int)(hq / (uint32_t)nq);
    const int64_t q = (int64_t)(hq - (uint32_t)h * (uint32_t)nq);
    const bool on = !only || only[hq];
    int b, bs, nbb;
    bool start;
    query_batch(cu_q, batch, cu_sb, q, &b, &bs, &nbb, &start);
    const int v = topk[i];
    const bool ok = on && v >= 0 && v < nbb && (int64_t)bs + v < nb;
    keys[i] = ok ? (uint32_t)(h * nb + bs + v) : none;
    vals[i] = encode ? (int32_t)(q * k + j) : (int32_t)q;
  }
}

// seg[s] = first sorted position whose key is >= s, for s = 0 .. hkv * nb:
// one thread per s, a binary search over the sorted keys (the work does not
// depend on how the keys are spread; with every key the sentinel, a walk
// between neighbouring keys would leave one thread writing all of seg).
__global__ __launch_bounds__(256) void rev_bounds_kernel(const uint32_t* __restrict__ keys,
                                                         int64_t n, int64_t n_seg,
                                                         int32_t* __restrict__ seg) {
  const int64_t sgi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (sgi > n_seg) return;
  int64_t lo = 0, hi = n;  // answer in [lo, hi]
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)keys[mid] < sgi)
      lo = mid + 1;
    else
      hi = mid;
  }
  seg[sgi] = (int32_t)lo;
}

// Per-head CSR offsets and totals from the segment starts.
__global__ __launch_bounds__(256) void rev_offsets_kernel(const int32_t* __restrict__ seg,
                                                          int64_t hkv, int64_t nb,
                                                          int32_t* __restrict__ cu_rev,
                                                          int32_t* __restrict__ totals) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= hkv * (nb + 1)) return;
  const int64_t h = t / (nb + 1), c = t - h * (nb + 1);
  const int32_t base = seg[h * nb];
  cu_rev[t] = seg[h * nb + c] - base;
  if (c == nb) totals[h] = seg[h * nb + nb] - base;
}

// rev[h * cap + pos] = the sorted listings of head h (the first seg[n_seg]
// sorted pairs are the valid ones).
__global__ __launch_bounds__(256) void rev_place_kernel(const uint32_t* __restrict__ keys,
                                                        const int32_t* __restrict__ vals,
                                                        const int32_t* __restrict__ seg,
                                                        int64_t nb, int64_t n_seg, int64_t cap,
                                                        int32_t* __restrict__ rev) {
  const int64_t n = seg[n_seg];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t h = keys[i] / (uint32_t)nb;  // keys and nb below 2^31: 32-bit divide
    rev[h * cap + (i - seg[h * nb])] = vals[i];
  }
}

size_t rev_sort_temp_bytes(int64_t n, unsigned bits) {
  size_t bytes = 0;
  (void)rocprim::radix_sort_pairs(nullptr, bytes, (const uint32_t*)nullptr,
                                  (uint32_t*)nullptr, (const int32_t*)nullptr,
                                  (int32_t*)nullptr, (unsigned)(n > 0 ? n : 1), 0, bits,
                                  (hipStream_t)0);
  return bytes;
}

int build_query_reverse_map(const int32_t* topk, int64_t hkv, int64_t nq, int64_t topk_n,
                            const int32_t* cu_q, int64_t batch, const int32_t* cu_sb,
                            int64_t nb, Carver& ws, RevMap& map, hipStream_t st,
                            const uint8_t* only, bool encode_slot) {
  const int64_t n = hkv * nq * topk_n;
  const int64_t n_seg = hkv * nb;
  uint32_t* keys = ws.take<uint32_t>((size_t)(n > 0 ? n : 1));
  uint32_t* keys_out = ws.take<uint32_t>((size_t)(n > 0 ? n : 1));
  int32_t* vals = ws.take<int32_t>((size_t)(n > 0 ? n : 1));
  int32_t* vals_out = ws.take<int32_t>((size_t)(n > 0 ? n : 1));
  int32_t* seg = ws.take<int32_t>((size_t)(n_seg + 1));
  unsigned bits = 1;  // key bits: keys are <= n_seg
  while (bits < 32 && (1ull << bits) <= (unsigned long long)n_seg) ++bits;
  const size_t tb = rev_sort_temp_bytes(n, bits);
  char* temp = ws.take<char>(tb);
  if (!map.cu_rev) map.cu_rev = ws.take<int32_t>((size_t)(hkv * (nb + 1)));
  if (!map.rev) map.rev = ws.take<int32_t>((size_t)(hkv * (map.cap > 0 ? map.cap : 1)));
  if (!map.totals) map.totals = ws.take<int32_t>((size_t)hkv);
  if (!ws.base || ws.dry) return LSRM_OK;
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  if (nb == 0 || n == 0) {
    int rc = launch_zero_i32(map.cu_rev, hkv * (nb + 1), st);
    if (rc) return rc;
    return launch_zero_i32(map.totals, hkv, st);
  }
  const int64_t grid = std::min<int64_t>(ceil_div(n + 1, 256), 16384);
  hipLaunchKernelGGL(rev_pairs_kernel, dim3(grid), dim3(256), 0, st, topk,
                     hkv, nq, (int)topk_n, cu_q, batch, cu_sb, nb, only, encode_slot, keys,
                     vals);
  LSRM_CHECK_LAUNCH();
  size_t tbv = tb;
  if (rocprim::radix_sort_pairs(temp, tbv, keys, keys_out, vals, vals_out, (unsigned)n, 0,
                                bits, st) != hipSuccess)
    return LSRM_ERR_LAUNCH;
  hipLaunchKernelGGL(rev_bounds_kernel, dim3(ceil_div(n_seg + 1, 256)), dim3(256), 0, st,
                     keys_out, n, n_seg, seg);
  LSRM_CHECK_LAUNCH();
  hipLaunchKernelGGL(rev_offsets_kernel, dim3(ceil_div(hkv * (nb + 1), 256)), dim3(256), 0, st,
                     seg, hkv, nb, map.cu_rev, map.totals);
  LSRM_CHECK_LAUNCH();
  hipLaunchKernelGGL(rev_place_kernel, dim3(grid), dim3(256), 0, st, keys_out,
                     vals_out, seg, nb, n_seg, map.cap, map.rev);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

int build_reverse_map(const int32_t* topk, int64_t hkv, int64_t nq,
                      int64_t topk_n, const int32_t* cu_q, int64_t batch,
                      const int32_t* cu_sb, int64_t nb, bool rows_are_tiles,
                      const TilePlan* plan, Carver& ws, RevMap& map,
                      hipStream_t st, const uint8_t* only, bool encode_slot) {
  if (!rows_are_tiles && hkv * nq * topk_n < (int64_t{1} << 31) &&
      hkv * nb < (int64_t{1} << 31))
    return build_query_reverse_map(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, nb, ws, map, st,
                                   only, encode_slot);
  int32_t* counts = ws.take<int32_t>((size_t)(hkv * (nb > 0 ? nb : 1)));
  int32_t* fill = ws.take<int32_t>((size_t)(hkv * (nb > 0 ? nb : 1)));
  int32_t* sums = ws.take<int32_t>((size_t)scan_sums_size(nb, hkv));
  int32_t* aux = ws.take<int32_t>((size_t)(hkv * (map.cap > 0 ? map.cap : 1)));
  if (!map.cu_rev) map.cu_rev = ws.take<int32_t>((size_t)(hkv * (nb + 1)));
  if (!map.rev) map.rev = ws.take<int32_t>((size_t)(hkv * (map.cap > 0 ? map.cap : 1)));
  if (!map.totals) map.totals = ws.take<int32_t>((size_t)hkv);
  if (!ws.base || ws.dry) return LSRM_OK;
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;

  RowSrc rows{rows_are_tiles ? plan->tiles : nullptr,
              rows_are_tiles ? plan->tile_count : nullptr, nq,
              rows_are_tiles ? nullptr : only,
              (!rows_are_tiles && encode_slot) ? (int)topk_n : 0};
  int rc = launch_zero_i32(counts, hkv * nb, st);
  if (rc) return rc;
  rc = launch_zero_i32(fill, hkv * nb, st);
  if (rc) return rc;
  if (nb == 0) {
    rc = launch_zero_i32(map.cu_rev, hkv, st);
    if (rc) return rc;
    return launch_zero_i32(map.totals, hkv, st);
  }
  const bool lds_bins = nb <= REV_LDS_BINS;
  if (nq > 0) {
    dim3 grid(ceil_div(nq, 256), (unsigned)hkv);
    if (lds_bins)
      hipLaunchKernelGGL(rev_count_lds_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, nb, rows, counts);
    else
      hipLaunchKernelGGL(rev_count_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, nb, rows, counts);
    LSRM_CHECK_LAUNCH();
  }
  rc = run_scan(CountF{counts, nb}, CuRevW{map.cu_rev, nb}, nb, (int)hkv, sums,
                map.totals, st);
  if (rc) return rc;
  if (nq > 0) {
    dim3 grid(ceil_div(nq, 256), (unsigned)hkv);
    if (lds_bins)
      hipLaunchKernelGGL(rev_scatter_lds_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, nb, rows, map.cu_rev,
                         fill, map.rev, map.cap);
    else
      hipLaunchKernelGGL(rev_scatter_kernel, grid, dim3(256), 0, st, topk, nq,
                         (int)topk_n, cu_q, batch, cu_sb, nb, rows, map.cu_rev,
                         fill, map.rev, map.cap);
    LSRM_CHECK_LAUNCH();
    dim3 sgrid((unsigned)nb, (unsigned)hkv);
    hipLaunchKernelGGL(rev_sort_kernel, sgrid, dim3(256), 0, st, map.cu_rev,
                       map.rev, aux, nb, map.cap, rows);
    LSRM_CHECK_LAUNCH();
  }
  return LSRM_OK;
}

__global__ __launch_bounds__(256) void mark_grouped_kernel(const int2* __restrict__ gtiles,
                                                           const int32_t* __restrict__ gcount,
                                                           int64_t nq,
                                                           uint8_t* __restrict__ flags) {
  const int h = blockIdx.y;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= gcount[h]) return;
  const int2 g = gtiles[(int64_t)h * nq + t];
  for (int i = 0; i < g.y; ++i) flags[(int64_t)h * nq + g.x + i] = 1;
}

int mark_grouped_queries(const TilePlan& plan, int64_t hkv, int64_t nq,
                         uint8_t* flags, hipStream_t st) {
  if (nq <= 0) return LSRM_OK;
  int rc = launch_zero_i32(reinterpret_cast<int32_t*>(flags), (hkv * nq + 3) / 4, st);
  if (rc) return rc;
  if (!plan.gtiles) return LSRM_OK;
  // Grouped tiles hold >= 2 queries, so at most nq / 2 per head.
  hipLaunchKernelGGL(mark_grouped_kernel, dim3(ceil_div(nq / 2 + 1, 256), (unsigned)hkv),
                     dim3(256), 0, st, plan.gtiles, plan.gtile_count, nq, flags);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

// -------------------------------------------------- key-centric part --

// Token count of block c, clamped as the attention kernels clamp it.
__device__ inline int64_t kc_block_len(const int32_t* cu_blk, int64_t nk, int64_t c) {
  int64_t s0 = cu_blk[c], s1 = cu_blk[c + 1];
  s0 = s0 < 0 ? 0 : (s0 > nk ? nk : s0);
  s1 = s1 < s0 ? s0 : (s1 > nk ? nk : s1);
  return s1 - s0;
}

// The listings of block c of grev's segment of kv head h that belong to
// queries [p * pq, (p + 1) * pq) (pass p of pq queries): [s, e) of the
// segment, found by binary search (listings q * topk + slot ascend).
struct KcPassRange {
  const int32_t* cu_rev;
  const int32_t* rev;
  int64_t nb, cap;
  int hkv;
  int64_t pass_listings;  // query passes: pq * topk; 0 = no query cut
  int pass_heads;         // head passes: kv heads per pass; 0 = none
  __device__ void operator()(int vs, int64_t c, int64_t& s, int64_t& e) const {
    const int p = vs / hkv, h = vs - p * hkv;
    const int32_t* cr = cu_rev + (int64_t)h * (nb + 1);
    s = cr[c];
    e = cr[c + 1];
    e = e < cap ? e : cap;
    if (pass_heads > 0 && h / pass_heads != p) e = s;  // another pass's head
    if (pass_listings == 0 || e <= s) return;
    const int32_t* r = rev + (int64_t)h * cap;
    auto first_at = [&](int64_t x) {  // first i in [s, e) with r[i] >= x
      int64_t lo = s, hi = e;
      while (lo < hi) {
        const int64_t m = (lo + hi) >> 1;
        if ((int64_t)r[m] < x) lo = m + 1; else hi = m;
      }
      return lo;
    };
    const int64_t a = first_at(p * pass_listings), b = first_at((p + 1) * pass_listings);
    s = a;
    e = b;
  }
};

// Gathered tiles of block c in the segment "vs" = (pass p, kv head h):
// ceil(listings / tq) pieces of the pass's listings of the block.  With
// cu_blk set, only blocks of lo + 1 .. hi keys count (the resident forwards'
// items, lo >= 0), or with `outside` only the other blocks (the streaming
// forward's); with cu_blk null, every block counts.
struct KcItemsF {
  KcPassRange rg;
  int tq;
  const int32_t* cu_blk;
  int64_t nk;
  int lo, hi;
  bool outside;
  __device__ int64_t limit(int, int64_t n) const { return n; }
  __device__ int operator()(int vs, int64_t c) const {
    if (cu_blk) {
      const int64_t len = kc_block_len(cu_blk, nk, c);
      const bool in = len > lo && len <= hi;
      if (in == outside) return 0;
    }
    int64_t s, e;
    rg(vs, c, s, e);
    return e > s ? (int)((e - s + tq - 1) / tq) : 0;
  }
};
struct KcItemsW {
  KcPassRange rg;
  int tq;
  int4* items;
  int64_t item_cap;
  __device__ void operator()(int vs, int64_t c, int ex, int v, int64_t) const {
    if (v == 0) return;
    int64_t s, e;
    rg(vs, c, s, e);
    for (int t = 0; t < v && ex + t < item_cap; ++t) {
      const int64_t e0 = s + (int64_t)tq * t;
      const int64_t n = e - e0 < tq ? e - e0 : tq;
      items[(int64_t)vs * item_cap + ex + t] = make_int4((int)c, (int)e0, (int)n, 0);
    }
  }
};

__global__ __launch_bounds__(256) void derive_offsets_kernel(RevMap enc, RevMap plain,
                                                             int64_t hkv, int64_t nb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < hkv * (nb + 1)) plain.cu_rev[i] = enc.cu_rev[i];
  if (i < hkv) plain.totals[i] = enc.totals[i];
}
__global__ __launch_bounds__(256) void derive_rev_kernel(RevMap enc, RevMap plain, int64_t hkv,
                                                         int k) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < hkv * enc.cap;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t h = i / enc.cap;
    if (i - h * enc.cap < enc.totals[h]) plain.rev[i] = enc.rev[i] / k;
  }
}

int derive_query_map(const RevMap& enc, const RevMap& plain, int64_t hkv, int64_t nb,
                     int64_t topk_n, hipStream_t st) {
  if (enc.cap != plain.cap || hkv <= 0 || topk_n <= 0) return LSRM_ERR_INVALID_ARG;
  hipLaunchKernelGGL(derive_offsets_kernel, dim3(ceil_div(hkv * (nb + 1) + hkv, 256)), dim3(256),
                     0, st, enc, plain, hkv, nb);
  LSRM_CHECK_LAUNCH();
  const int64_t grid = std::min<int64_t>(ceil_div(hkv * enc.cap, 256), 16384);
  hipLaunchKernelGGL(derive_rev_kernel, dim3(grid > 0 ? grid : 1), dim3(256), 0, st, enc, plain,
                     hkv, (int)topk_n);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

// Per-(pass, head) offsets of the item lists (resident, eight-wave
// resident, streaming) -- each pass's heads from 0 -- and their cleared work
// counters.
struct KcCounts {
  const int32_t* count[3];
  int32_t* off[3];
};
__global__ void kc_offsets_kernel(KcCounts c, int hkv, int n_pass, int32_t* counter,
                                  int32_t marker) {
  if (threadIdx.x < 3 && blockIdx.x == 0) {
    const int32_t* cnt = c.count[threadIdx.x];
    int32_t* off = c.off[threadIdx.x];
    for (int p = 0; p < n_pass; ++p) {
      int acc = 0;
      off[p * (hkv + 1)] = 0;
      for (int h = 0; h < hkv; ++h) {
        acc += cnt[p * hkv + h];
        off[p * (hkv + 1) + h + 1] = acc;
      }
    }
  }
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    counter[KC_QUEUE_SLOT] = 0;
    counter[KC_EXIT_SLOT] = 0;
    counter[KC_RQUEUE_SLOT] = 0;
    counter[KC_REXIT_SLOT] = 0;
    counter[KC_R2QUEUE_SLOT] = 0;
    counter[KC_R2EXIT_SLOT] = 0;
    counter[PLAN_KC_SLOT] = marker;
  }
}

void kc_passes(int64_t n_q, int64_t hkv, int64_t topk, int g, int64_t head_dim, int* n_pass,
               int* pass_heads, int64_t* q_span) {
  const int64_t nq = n_q > 0 ? n_q : 1;
  const int64_t per_row = topk * g * (2 * (head_dim > 0 ? head_dim : 1) + 4);
  const int64_t per_head = nq * per_row;
  if (per_head * hkv <= KC_PART_BUDGET || per_head <= KC_PART_BUDGET) {
    // whole kv heads per pass (one pass when everything fits)
    int64_t hp = KC_PART_BUDGET / per_head;
    hp = hp < 1 ? 1 : (hp > hkv ? hkv : hp);
    *pass_heads = hkv > 1 && hp < hkv ? (int)hp : 0;
    *q_span = nq;
    *n_pass = (int)((hkv + hp - 1) / hp);
    if (*pass_heads == 0) *n_pass = 1;
    return;
  }
  int64_t span = KC_PART_BUDGET / (hkv * per_row);
  if (span < 1) span = 1;
  if (span >= nq) span = nq;
  *pass_heads = 0;
  *q_span = span;
  *n_pass = (int)((nq + span - 1) / span);
}

int build_kc_items(const RevMap& grev, const int32_t* cu_blk, int64_t nk, int64_t hkv,
                   int64_t nb, int tq, int64_t head_dim, int64_t topk_n, Carver& ws,
                   KcPlan& kc, int32_t* counter, int32_t marker, hipStream_t st) {
  const int rq = tq * KC_RES_CHUNKS;
  const int res_max = kc_res_max((int)(head_dim > 0 ? head_dim : 1));
  const int np = kc.n_pass > 0 ? kc.n_pass : 1;
  // listings of one (pass, head): at most the pass's queries times topk
  const int64_t lst = (np > 1 && kc.pass_heads == 0) ? kc.q_span_max * topk_n : grev.cap;
  kc.ritem_cap = lst / (rq > 0 ? rq : 1) + nb + 1;
  kc.ritems = ws.take<int4>((size_t)(np * hkv * kc.ritem_cap));
  kc.ritem_count = ws.take<int32_t>((size_t)(np * hkv));
  kc.ritem_off = ws.take<int32_t>((size_t)(np * (hkv + 1)));
  kc.r2item_cap = kc.ritem_cap;
  kc.r2items = ws.take<int4>((size_t)(np * hkv * kc.r2item_cap));
  kc.r2item_count = ws.take<int32_t>((size_t)(np * hkv));
  kc.r2item_off = ws.take<int32_t>((size_t)(np * (hkv + 1)));
  kc.fitem_cap = lst / (tq > 0 ? tq : 1) + nb + 1;
  kc.fitems = ws.take<int4>((size_t)(np * hkv * kc.fitem_cap));
  kc.fitem_count = ws.take<int32_t>((size_t)(np * hkv));
  kc.fitem_off = ws.take<int32_t>((size_t)(np * (hkv + 1)));
  int32_t* sums = ws.take<int32_t>((size_t)scan_sums_size(nb, np * hkv));
  if (!ws.base || ws.dry) return LSRM_OK;
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  for (int32_t* cnt : {kc.ritem_count, kc.r2item_count, kc.fitem_count}) {
    const int rc = launch_zero_i32(cnt, np * hkv, st);
    if (rc) return rc;
  }
  const KcPassRange rg{grev.cu_rev, grev.rev, nb, grev.cap, (int)hkv,
                       (np > 1 && kc.pass_heads == 0) ? kc.q_span_max * topk_n : 0,
                       kc.pass_heads};
  const int nseg = (int)(np * hkv);
  int rc = run_scan(KcItemsF{rg, rq, cu_blk, nk, 0, KC_RES_KEYS, false},
                    KcItemsW{rg, rq, kc.ritems, kc.ritem_cap}, nb, nseg, sums, kc.ritem_count,
                    st);
  if (rc) return rc;
  if (res_max > KC_RES_KEYS) {
    rc = run_scan(KcItemsF{rg, rq, cu_blk, nk, KC_RES_KEYS, res_max, false},
                  KcItemsW{rg, rq, kc.r2items, kc.r2item_cap}, nb, nseg, sums, kc.r2item_count,
                  st);
    if (rc) return rc;
  }
  rc = run_scan(KcItemsF{rg, tq, cu_blk, nk, 0, res_max, true},
                KcItemsW{rg, tq, kc.fitems, kc.fitem_cap}, nb, nseg, sums, kc.fitem_count, st);
  if (rc) return rc;
  const KcCounts c{{kc.ritem_count, kc.r2item_count, kc.fitem_count},
                   {kc.ritem_off, kc.r2item_off, kc.fitem_off}};
  hipLaunchKernelGGL(kc_offsets_kernel, dim3(1), dim3(64), 0, st, c, (int)hkv, np, counter,
                     marker);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

// ----------------------------------------------------------- key items --

struct KeyChunksF {
  const int32_t* cu;
  int64_t nk;
  __device__ int64_t limit(int, int64_t n) const { return n; }
  __device__ int operator()(int, int64_t c) const {
    int64_t s = cu[c], e = cu[c + 1];
    s = s < 0 ? 0 : (s > nk ? nk : s);
    e = e < 0 ? 0 : (e > nk ? nk : e);
    return e > s ? (int)((e - s + KEY_CHUNK - 1) / KEY_CHUNK) : 0;
  }
};
struct KeyChunksW {
  const int32_t* cu;
  int64_t nk;
  int4* items;
  int64_t cap;
  __device__ void operator()(int, int64_t c, int ex, int v, int64_t) const {
    int64_t s = cu[c], e = cu[c + 1];
    s = s < 0 ? 0 : (s > nk ? nk : s);
    e = e < 0 ? 0 : (e > nk ? nk : e);
    for (int t = 0; t < v && ex + t < cap; ++t) {
      const int64_t t0 = s + (int64_t)KEY_CHUNK * t;
      const int64_t len = e - t0 < KEY_CHUNK ? e - t0 : KEY_CHUNK;
      items[ex + t] = make_int4((int)c, (int)t0, (int)len, 0);
    }
  }
};

int build_key_items(const int32_t* cu_blk, int64_t nb, int64_t nk, Carver& ws,
                    KeyItems& ki, hipStream_t st) {
  const int64_t cap = nb + nk / KEY_CHUNK + 2;
  ki.items = ws.take<int4>((size_t)cap);
  ki.n_items = ws.take<int32_t>(64);
  int32_t* sums = ws.take<int32_t>((size_t)scan_sums_size(nb, 1));
  if (!ws.base || ws.dry) return LSRM_OK;
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;
  int rc = launch_zero_i32(ki.n_items, 1, st);
  if (rc) return rc;
  return run_scan(KeyChunksF{cu_blk, nk}, KeyChunksW{cu_blk, nk, ki.items, cap}, nb,
                  1, sums, ki.n_items, st);
}

// ------------------------------------------------------------ validate --

__global__ __launch_bounds__(256) void validate_meta_kernel(
    const int32_t* __restrict__ cu_sb, const int32_t* __restrict__ cu_blk,
    int64_t nb, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, int64_t batch, int64_t nq, int64_t nk,
    int32_t* flags) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int f = 0;
  if (i < nb) {
    const int64_t s = cu_blk[i], e = cu_blk[i + 1];
    if (e < s) f |= LSRM_META_OFFSETS_NOT_MONOTONE;
    if (s < 0 || e > nk) f |= LSRM_META_BLOCK_OUT_OF_RANGE;
  }
  if (i < batch) {
    if (cu_sb[i + 1] < cu_sb[i] || cu_sb[i] < 0 || cu_sb[i + 1] > nb)
      f |= LSRM_META_SEQBLOCKS_BAD;
    if (cu_q[i + 1] < cu_q[i] || cu_k[i + 1] < cu_k[i] || cu_q[i] < 0 ||
        cu_k[i] < 0 || cu_k[i + 1] > nk)
      f |= LSRM_META_SEQLENS_BAD;
    if (i == 0 && (cu_q[0] != 0 || cu_q[batch] != nq))
      f |= LSRM_META_SEQLENS_BAD;
    const int64_t b0 = cu_sb[i], b1 = cu_sb[i + 1];
    if (b0 >= 0 && b1 <= nb && b1 > b0) {
      if (cu_blk[b0] < cu_k[i] || cu_blk[b1] > cu_k[i + 1])
        f |= LSRM_META_BLOCK_OUTSIDE_SEQ;
    }
  }
  if (f) atomicOr(flags, f);
}

__global__ __launch_bounds__(256) void validate_topk_kernel(
    const int32_t* __restrict__ topk, int64_t nq, int k,
    const int32_t* __restrict__ cu_q, int64_t batch,
    const int32_t* __restrict__ cu_sb, int32_t* flags) {
  const int h = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nq) return;
  int b, bs, nbb;
  bool start;
  query_batch(cu_q, batch, cu_sb, i, &b, &bs, &nbb, &start);
  const int32_t* row = topk + ((int64_t)h * nq + i) * k;
  bool seen_invalid = false, any = false;
  int f = 0;
  for (int j = 0; j < k; ++j) {
    const bool valid = norm_entry(row[j], nbb) >= 0;
    if (valid) {
      any = true;
      if (seen_invalid) f |= LSRM_META_TOPK_NOT_PREFIX;
    } else {
      seen_invalid = true;
    }
  }
  if (!any) f |= LSRM_META_TOPK_EMPTY_ROW;
  if (f) atomicOr(flags, f);
}

// ----------------------------------------------------------- block ids --

__global__ __launch_bounds__(256) void block_ids_kernel(
    const int32_t* __restrict__ cu_sb, int64_t batch,
    const int32_t* __restrict__ cu_blk, int64_t nb, int64_t n, int64_t hkv,
    int32_t* __restrict__ ids) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  int id = -1;
  const int64_t b = upper_index(cu_blk, 0, nb + 1, t);
  if (b >= 0 && b < nb && t < cu_blk[b + 1]) {
    const int64_t e = upper_index(cu_sb, 0, batch + 1, b);
    if (e >= 0 && e < batch) id = (int)(b - cu_sb[e]);
  }
  for (int64_t h = 0; h < hkv; ++h) ids[h * n + t] = id;
}

}  // namespace lsrm

using namespace lsrm;

extern "C" int lsrm_sel_attn_validate(
    const int32_t* topk_idx, int64_t hkv, int64_t n_q, int64_t topk,
    const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
    int64_t n_blocks, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
    int64_t batch, int64_t n_k, int32_t* flags, void* stream) {
  if (hkv <= 0 || n_q < 0 || topk <= 0 || n_blocks < 0 || batch <= 0 ||
      n_k < 0 || !flags || !cu_seqblocks || !cu_block_tokens || !cu_seqlens_q ||
      !cu_seqlens_k || (n_q > 0 && !topk_idx))
    return LSRM_ERR_INVALID_ARG;
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_zero_i32(flags, 1, st);
  if (rc) return rc;
  const int64_t m = n_blocks > batch ? n_blocks : batch;
  hipLaunchKernelGGL(validate_meta_kernel, dim3(ceil_div(m > 0 ? m : 1, 256)),
                     dim3(256), 0, st, cu_seqblocks, cu_block_tokens, n_blocks,
                     cu_seqlens_q, cu_seqlens_k, batch, n_q, n_k, flags);
  LSRM_CHECK_LAUNCH();
  if (n_q > 0) {
    dim3 grid(ceil_div(n_q, 256), (unsigned)hkv);
    hipLaunchKernelGGL(validate_topk_kernel, grid, dim3(256), 0, st, topk_idx,
                       n_q, (int)topk, cu_seqlens_q, batch, cu_seqblocks,
                       flags);
    LSRM_CHECK_LAUNCH();
  }
  return LSRM_OK;
}

extern "C" size_t lsrm_reverse_query_map_workspace_size(int64_t n_q,
                                                        int64_t hkv,
                                                        int64_t topk,
                                                        int64_t n_blocks) {
  if (n_q < 0 || hkv <= 0 || topk <= 0 || n_blocks < 0) return 0;
  Carver ws{nullptr, 0, 0};
  RevMap map{};
  map.cap = n_q * topk;
  // cu_rev / rev / totals are caller outputs: mark them present.
  map.cu_rev = reinterpret_cast<int32_t*>(1);
  map.rev = reinterpret_cast<int32_t*>(1);
  map.totals = reinterpret_cast<int32_t*>(1);
  build_reverse_map(nullptr, hkv, n_q, topk, nullptr, 1, nullptr, n_blocks,
                    false, nullptr, ws, map, nullptr);
  return ws.used + 256;
}

extern "C" int lsrm_reverse_query_map(
    const int32_t* topk_idx, int64_t hkv, int64_t n_q, int64_t topk,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqblocks, int64_t batch,
    int64_t n_blocks, int32_t* cu_reverse_count,
    int32_t* reverse_query_indices, int64_t capacity, int32_t* totals,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (hkv <= 0 || n_q < 0 || topk <= 0 || n_blocks < 0 || batch <= 0 ||
      capacity < 0 || !cu_reverse_count || !totals || !cu_seqlens_q ||
      !cu_seqblocks || (n_q > 0 && !topk_idx) ||
      (capacity > 0 && !reverse_query_indices))
    return LSRM_ERR_INVALID_ARG;
  const size_t need =
      lsrm_reverse_query_map_workspace_size(n_q, hkv, topk, n_blocks);
  if (workspace_bytes < need || !workspace) return LSRM_ERR_WORKSPACE;
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0,
            workspace_bytes - 256};
  RevMap map{cu_reverse_count, reverse_query_indices, totals, capacity};
  // The sort's aux buffer is sized by map.cap: keep it equal to capacity.
  return build_reverse_map(topk_idx, hkv, n_q, topk, cu_seqlens_q, batch,
                           cu_seqblocks, n_blocks, false, nullptr, ws, map,
                           (hipStream_t)stream);
}

extern "C" int lsrm_block_ids(const int32_t* cu_seqblocks, int64_t batch,
                              const int32_t* cu_block_tokens, int64_t n_blocks,
                              int64_t n_tokens, int64_t hkv, int32_t* ids,
                              void* stream) {
  if (batch <= 0 || n_blocks < 0 || n_tokens < 0 || hkv <= 0 || !cu_seqblocks ||
      !cu_block_tokens || (n_tokens > 0 && !ids))
    return LSRM_ERR_INVALID_ARG;
  if (n_tokens == 0) return LSRM_OK;
  hipLaunchKernelGGL(block_ids_kernel, dim3(ceil_div(n_tokens, 256)), dim3(256),
                     0, (hipStream_t)stream, cu_seqblocks, batch,
                     cu_block_tokens, n_blocks, n_tokens, hkv, ids);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}
