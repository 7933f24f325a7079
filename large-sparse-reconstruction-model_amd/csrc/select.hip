// Per-query-block top-k block selection.
//
// The rule (no reference function implements it; the reference's learned
// selection is sparse/ops/block_score.py:16-98): mean-pool Q and K per block
// (fp32, the lsrm_block_mean_pool contract), score every (query block b,
// key block c) pair of a batch element as
//     s(b, c) = sum_{g in group(h)} sum_d (double)pq[b,g,d] * (double)pk[c,h,d]
// accumulated in fp64 in that order (fp32 x fp32 products are exact in fp64,
// so the sum is a fixed function of the pooled means), then take the forced
// blocks followed by the best remaining blocks under (score descending,
// block id ascending).  Selected ids are written ascending, -1 padded.
#include "common.h"

namespace lsrm {

int launch_block_mean_pool(const void* x, int x_dtype, int64_t n, int64_t ch,
                           const int32_t* cu, int64_t nb, void* out,
                           int out_dtype, float* partial, int32_t* first,
                           hipStream_t st);
int64_t pool_partial_rows(int64_t n, int64_t nb);
int64_t pool_first_count(int64_t n);

constexpr int SEL_MAXD = 128;
constexpr int SEL_CAND_LDS = 8192;      // candidate scores cached in LDS
constexpr int SEL_MAX_CAND = 65536;     // bitmap capacity (blocks per batch)
constexpr int SEL_MAXK = 256;

// scores[h, b, c] for b, c in [0, nb): 128x128 tile per workgroup, 8x8 per
// thread (rows ty + 16 i, columns tx + 16 j), fp64 accumulation over (g, d)
// in order.  The pooled rows are staged in LDS as doubles, SCORE_DC head-dim
// columns at a time and transposed ([column][row]), so a thread's eight row
// operands are wave-broadcast reads and its eight column operands are
// conflict-free reads of consecutive doubles: 16 LDS reads per 64 fused
// multiply-adds (the kernel is bound by the fp64 FMA rate, not by LDS).
// Converting each element once and the order of the fused multiply-adds
// leave every score a fixed function of the pooled means.
constexpr int SCORE_TILE = 128;
constexpr int SCORE_DC = 16;
__global__ __launch_bounds__(256) void score_kernel(
    const float* __restrict__ pq, const float* __restrict__ pk, int64_t nb,
    int hq, int hkv, int d, double* __restrict__ scores) {
  __shared__ double sq[SCORE_DC][SCORE_TILE + 1];
  __shared__ double sk[SCORE_DC][SCORE_TILE + 1];
  const int h = blockIdx.z;
  const int64_t b0 = (int64_t)blockIdx.y * SCORE_TILE;
  const int64_t c0 = (int64_t)blockIdx.x * SCORE_TILE;
  const int g_n = hq / hkv;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  double acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.0;

  // Chunks (g, dc) in order; each thread stages SCORE_PER elements of the Q
  // rows and of the K rows per chunk.  The next chunk's global loads are
  // issued into registers before the current chunk's multiply-adds, so
  // their latency overlaps the arithmetic.
  constexpr int SCORE_PER = SCORE_TILE * SCORE_DC / 256;
  const int n_dc = (d + SCORE_DC - 1) / SCORE_DC;
  const int n_chunk = g_n * n_dc;
  float pq_r[SCORE_PER], pk_r[SCORE_PER];
  auto fetch = [&](int ci) __attribute__((always_inline)) {
    const int g = ci / n_dc, dc = (ci - g * n_dc) * SCORE_DC;
    const int hh = h * g_n + g;
    const int dn = d - dc < SCORE_DC ? d - dc : SCORE_DC;
#pragma unroll
    for (int u = 0; u < SCORE_PER; ++u) {
      const int i = (int)threadIdx.x + 256 * u;
      const int r = i / SCORE_DC, dd = i % SCORE_DC;
      const bool in_d = dd < dn;
      pq_r[u] = (in_d && b0 + r < nb)
                    ? pq[(b0 + r) * (int64_t)hq * d + (int64_t)hh * d + dc + dd]
                    : 0.0f;
      pk_r[u] = (in_d && c0 + r < nb)
                    ? pk[(c0 + r) * (int64_t)hkv * d + (int64_t)h * d + dc + dd]
                    : 0.0f;
    }
  };
  fetch(0);
  for (int ci = 0; ci < n_chunk; ++ci) {
    const int dc = (ci % n_dc) * SCORE_DC;
    const int dn = d - dc < SCORE_DC ? d - dc : SCORE_DC;
#pragma unroll
    for (int u = 0; u < SCORE_PER; ++u) {
      const int i = (int)threadIdx.x + 256 * u;
      const int r = i / SCORE_DC, dd = i % SCORE_DC;
      sq[dd][r] = (double)pq_r[u];
      sk[dd][r] = (double)pk_r[u];
    }
    __syncthreads();
    if (ci + 1 < n_chunk) fetch(ci + 1);
    for (int dd = 0; dd < dn; ++dd) {
      double a[8], bv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = sq[dd][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 8; ++j) bv[j] = sk[dd][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_fma(a[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t b = b0 + ty + 16 * i;
    if (b >= nb) continue;
    double* out = scores + ((int64_t)h * nb + b) * nb;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t c = c0 + tx + 16 * j;
      if (c < nb) out[c] = acc[i][j];
    }
  }
}

// dst[t * topk + j] = ord[j] for the `total` / topk token rows at dst, the
// stores spread over the calling threads (`first`, `step`).  When topk / 4
// divides `step`, a thread's 16-byte stores all carry the same four ids.
__device__ inline void fill_token_rows(int32_t* __restrict__ dst, int64_t total,
                                       const int* __restrict__ ord, int topk, int first,
                                       int step) {
  const int q4 = topk >> 2;
  if ((topk & 3) == 0 && step % q4 == 0 && ((uintptr_t)dst & 15) == 0) {
    const int j = (first % q4) * 4;
    const int4 val = make_int4(ord[j], ord[j + 1], ord[j + 2], ord[j + 3]);
    int4* d4 = reinterpret_cast<int4*>(dst);
    for (int64_t i = first; i < (total >> 2); i += step) d4[i] = val;
  } else {
    for (int64_t i = first; i < total; i += step) dst[i] = ord[i % topk];
  }
}

// A block outside every batch element selects nothing: its compact row and
// the per-token rows of its tokens (clamped to [0, n_tokens)) become -1.
// `first` / `step` spread the stores over the calling threads.
__device__ inline void clear_block_rows(const int32_t* __restrict__ cu_blk, int64_t b,
                                        int64_t n_tokens, int topk, int32_t* crow,
                                        int32_t* head_rows, int first, int step) {
  for (int j = first; j < topk; j += step) crow[j] = -1;
  int64_t t0 = cu_blk[b], t1 = cu_blk[b + 1];
  t0 = t0 < 0 ? 0 : (t0 > n_tokens ? n_tokens : t0);
  t1 = t1 < t0 ? t0 : (t1 > n_tokens ? n_tokens : t1);
  int32_t* dst = head_rows + t0 * topk;
  const int64_t total = (t1 - t0) * topk;
  for (int64_t i = first; i < total; i += step) dst[i] = -1;
}

__device__ inline bool sel_better(double s1, int i1, double s2, int i2) {
  return s1 > s2 || (s1 == s2 && i1 < i2);
}

__device__ inline double readlane_f64(double x, int j) {
  const uint64_t u = __builtin_bit_cast(uint64_t, x);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, j);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), j);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The best R candidates (score descending, id ascending) of those a wave
// holds -- M per lane: candidate (lane, m) has id q0 + lane + 64 m and score
// v[m], and bit m of `taken` marks it unavailable -- written to ls / li in
// that order (ls may be null: ids only); returns how many there are
// (min(R, available)).
// Threshold pass: each lane's best available candidate is its lane best;
// the lane bests of rank 0 .. R-1 are R distinct candidates no worse than
// the rank R-1 lane best T, so every member of the best R is no worse than
// T.  The candidates no worse than T (the survivors) are compacted through
// cs / ci (64 entries) and ranked among themselves.  Fallback (fewer than R
// lane bests, or more than 64 survivors): R rounds of lane-local scan plus
// wave butterfly.  Both give the same list, since the best R under a strict
// total order are unique.
template <int M>
__device__ int wave_best_r(const double (&v)[M], uint32_t taken, int q0, int R,
                           double* __restrict__ ls, int* __restrict__ li,
                           double* __restrict__ cs, int* __restrict__ ci) {
  const int lane = threadIdx.x & 63;
  if (R <= 0) return 0;
  double bs = -__builtin_inf();
  int bi = INT32_MAX;
#pragma unroll
  for (int m = 0; m < M; ++m)
    if (!((taken >> m) & 1u) && sel_better(v[m], q0 + lane + 64 * m, bs, bi)) {
      bs = v[m];
      bi = q0 + lane + 64 * m;
    }
  const int nv = __popcll(__ballot(bi != INT32_MAX));
  int S = 65;
  if (nv >= R) {
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 64; ++j)
      rank += sel_better(readlane_f64(bs, j), __builtin_amdgcn_readlane(bi, j), bs, bi) ? 1 : 0;
    const unsigned long long at = __ballot(bi != INT32_MAX && rank == R - 1);
    const int tl = __builtin_amdgcn_readfirstlane(__ffsll((long long)at) - 1);
    const double ts = readlane_f64(bs, tl);
    const int ti = __builtin_amdgcn_readlane(bi, tl);
    S = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int id = q0 + lane + 64 * m;
      const bool p = !((taken >> m) & 1u) && !sel_better(ts, ti, v[m], id);
      const unsigned long long bm = __ballot(p);
      const int pos = S + (int)__builtin_amdgcn_mbcnt_hi(
                              (uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
      if (p && pos < 64) {
        cs[pos] = v[m];
        ci[pos] = id;
      }
      S += __popcll(bm);
    }
  }
  if (S <= 64) {
    // One wave's LDS accesses complete in order; the clobber keeps the
    // compiler from moving the reads above the writes.
    asm volatile("" ::: "memory");
    const double xs = lane < S ? cs[lane] : -__builtin_inf();
    const int xi = lane < S ? ci[lane] : INT32_MAX;
    int rank = 0;
    for (int j = 0; j < S; ++j)
      rank += sel_better(readlane_f64(xs, j), __builtin_amdgcn_readlane(xi, j), xs, xi) ? 1 : 0;
    const int nw = S < R ? S : R;
    if (lane < S && rank < nw) {
      if (ls) ls[rank] = xs;
      li[rank] = xi;
    }
    return nw;
  }
  uint32_t tk = taken;
  int nw = 0;
  for (int n = 0; n < R; ++n) {
    double rs = -__builtin_inf();
    int ri = INT32_MAX;
#pragma unroll
    for (int m = 0; m < M; ++m)
      if (!((tk >> m) & 1u) && sel_better(v[m], q0 + lane + 64 * m, rs, ri)) {
        rs = v[m];
        ri = q0 + lane + 64 * m;
      }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const double os = __shfl_xor(rs, o);
      const int oi = __shfl_xor(ri, o);
      if (sel_better(os, oi, rs, ri)) {
        rs = os;
        ri = oi;
      }
    }
    ri = __builtin_amdgcn_readfirstlane(ri);
    if (ri == INT32_MAX) break;  // no candidate left
    const int lc = ri - q0;
    if ((lc & 63) == lane) tk |= 1u << (lc >> 6);
    if (lane == 0) {
      if (ls) ls[nw] = rs;
      li[nw] = ri;
    }
    ++nw;
  }
  return nw;
}

// One workgroup per (query block b, kv head h).
__global__ __launch_bounds__(256) void topk_kernel(
    const double* __restrict__ scores, int64_t nb,
    const int32_t* __restrict__ cu_sb, int64_t batch,
    const int32_t* __restrict__ cu_blk, int64_t n_tokens, int topk,
    const int32_t* __restrict__ forced, int n_forced, int force_self,
    int32_t* __restrict__ topk_idx, int32_t* __restrict__ compact) {
  __shared__ double s_sc[SEL_CAND_LDS];
  __shared__ uint32_t s_taken[SEL_MAX_CAND / 32];
  __shared__ int s_sel[SEL_MAXK];
  __shared__ int s_out[SEL_MAXK];
  __shared__ double s_ws[4];
  __shared__ int s_wi[4];
  __shared__ int s_nsel;

  const int h = blockIdx.y;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t e = upper_index(cu_sb, 0, batch + 1, b);
  int32_t* crow = compact + ((int64_t)h * nb + b) * topk;
  if (e < 0 || e >= batch || b >= cu_sb[e + 1]) {
    clear_block_rows(cu_blk, b, n_tokens, topk, crow, topk_idx + (int64_t)h * n_tokens * topk,
                     tid, 256);
    return;
  }
  const int64_t cs = cu_sb[e];
  const int nbb = (int)(cu_sb[e + 1] - cs);
  const bool cached = nbb <= SEL_CAND_LDS;
  const double* row = scores + ((int64_t)h * nb + b) * nb + cs;

  for (int i = tid; i < (nbb + 31) / 32; i += 256) s_taken[i] = 0u;
  if (cached) {
    for (int i = tid; i < nbb; i += 256) {
      const double v = row[i];
      s_sc[i] = (v != v) ? -__builtin_inf() : v;
    }
  }
  __syncthreads();
  const int kmax = topk < nbb ? topk : nbb;
  if (tid == 0) {
    int n = 0;
    auto add = [&](int id) {
      if (n >= kmax || id < 0 || id >= nbb) return;
      if (s_taken[id >> 5] & (1u << (id & 31))) return;
      s_taken[id >> 5] |= 1u << (id & 31);
      s_sel[n++] = id;
    };
    if (force_self) add((int)(b - cs));
    for (int f = 0; f < n_forced; ++f) add(forced[f]);
    s_nsel = n;
  }
  __syncthreads();

  for (int n = s_nsel; n < kmax; ++n) {
    double bs = -__builtin_inf();
    int bi = INT32_MAX;
    for (int i = tid; i < nbb; i += 256) {
      if (s_taken[i >> 5] & (1u << (i & 31))) continue;
      double v;
      if (cached) {
        v = s_sc[i];
      } else {
        v = row[i];
        if (v != v) v = -__builtin_inf();
      }
      if (sel_better(v, i, bs, bi)) {
        bs = v;
        bi = i;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const double os = __shfl_xor(bs, o);
      const int oi = __shfl_xor(bi, o);
      if (sel_better(os, oi, bs, bi)) {
        bs = os;
        bi = oi;
      }
    }
    if (lane == 0) {
      s_ws[w] = bs;
      s_wi[w] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      double fs = s_ws[0];
      int fi = s_wi[0];
      for (int i = 1; i < 4; ++i)
        if (sel_better(s_ws[i], s_wi[i], fs, fi)) {
          fs = s_ws[i];
          fi = s_wi[i];
        }
      s_sel[n] = fi;
      s_taken[fi >> 5] |= 1u << (fi & 31);
    }
    __syncthreads();
  }
  // Ascending order by rank (ids are distinct), -1 padding.
  for (int j = tid; j < topk; j += 256) s_out[j] = -1;
  __syncthreads();
  for (int j = tid; j < kmax; j += 256) {
    const int v = s_sel[j];
    int r = 0;
    for (int m = 0; m < kmax; ++m) r += s_sel[m] < v;
    s_out[r] = v;
  }
  __syncthreads();
  for (int j = tid; j < topk; j += 256) crow[j] = s_out[j];
  int64_t t0 = cu_blk[b], t1 = cu_blk[b + 1];
  t0 = t0 < 0 ? 0 : (t0 > n_tokens ? n_tokens : t0);
  t1 = t1 < t0 ? t0 : (t1 > n_tokens ? n_tokens : t1);
  int32_t* dst = topk_idx + ((int64_t)h * n_tokens + t0) * topk;
  const int64_t total = (t1 - t0) * topk;
  fill_token_rows(dst, total, s_out, topk, tid, 256);
}

// One wave per (kv head, query block) row when the candidates fit the
// registers (M per lane, blocks per batch <= 64 M): the row's scores stay in
// registers, forced blocks are taken first, then wave_best_r lists the best
// of the rest (score descending, id ascending).  No LDS candidate cache and
// no workgroup barriers.
template <int M>
__global__ __launch_bounds__(256) void topk_wave_kernel(
    const double* __restrict__ scores, int64_t nb,
    const int32_t* __restrict__ cu_sb, int64_t batch,
    const int32_t* __restrict__ cu_blk, int64_t n_tokens, int hkv, int topk,
    const int32_t* __restrict__ forced, int n_forced, int force_self,
    int32_t* __restrict__ topk_idx, int32_t* __restrict__ compact) {
  __shared__ int s_sel[4][SEL_MAXK];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t rowid = (int64_t)blockIdx.x * 4 + wv;
  if (rowid >= (int64_t)hkv * nb) return;  // whole wave
  const int h = (int)(rowid / nb);
  const int64_t b = rowid - (int64_t)h * nb;
  int* sel = s_sel[wv];
  const int64_t e = upper_index(cu_sb, 0, batch + 1, b);
  int32_t* crow = compact + ((int64_t)h * nb + b) * topk;
  if (e < 0 || e >= batch || b >= cu_sb[e + 1]) {
    clear_block_rows(cu_blk, b, n_tokens, topk, crow, topk_idx + (int64_t)h * n_tokens * topk,
                     lane, 64);
    return;
  }
  const int64_t cs = cu_sb[e];
  const int nbb = (int)(cu_sb[e + 1] - cs);
  const double* row = scores + ((int64_t)h * nb + b) * nb + cs;

  double v[M];
  uint32_t taken = 0u;  // bit m: candidate lane + 64 m is unavailable
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int i = lane + 64 * m;
    if (i < nbb) {
      const double x = row[i];
      v[m] = (x != x) ? -__builtin_inf() : x;
    } else {
      v[m] = -__builtin_inf();
      taken |= 1u << m;
    }
  }
  const int kmax = topk < nbb ? topk : nbb;
  int n = 0;
  auto take = [&](int id) {  // wave-uniform id
    if (n >= kmax || id < 0 || id >= nbb) return;
    const bool mine = (id & 63) == lane;
    const bool was = mine && ((taken >> (id >> 6)) & 1u);
    if (__builtin_amdgcn_ballot_w64(was) != 0) return;
    if (mine) taken |= 1u << (id >> 6);
    if (lane == 0) sel[n] = id;
    ++n;
  };
  if (force_self) take((int)(b - cs));
  for (int f = 0; f < n_forced; ++f) take(forced[f]);
  __shared__ double s_cs[4][64];
  __shared__ int s_ci[4][64];
  n += wave_best_r<M>(v, taken, 0, kmax - n, nullptr, sel + n, s_cs[wv], s_ci[wv]);
  asm volatile("" ::: "memory");
  // Ascending ids (distinct), -1 padding: id -> its rank among the chosen.
  __shared__ int s_out[4][SEL_MAXK];
  int* ord = s_out[wv];
  for (int j = lane; j < topk; j += 64) ord[j] = -1;
  for (int j = lane; j < kmax; j += 64) {
    const int id = sel[j];
    int r = 0;
    for (int t = 0; t < kmax; ++t) r += sel[t] < id;
    ord[r] = id;
  }
  for (int j = lane; j < topk; j += 64) crow[j] = ord[j];
  int64_t t0 = cu_blk[b], t1 = cu_blk[b + 1];
  t0 = t0 < 0 ? 0 : (t0 > n_tokens ? n_tokens : t0);
  t1 = t1 < t0 ? t0 : (t1 > n_tokens ? n_tokens : t1);
  int32_t* dst = topk_idx + ((int64_t)h * n_tokens + t0) * topk;
  const int64_t total = (t1 - t0) * topk;
  fill_token_rows(dst, total, ord, topk, lane, 64);
}

// One workgroup per (kv head, query block) row for rows of up to 4 * 64 * M
// candidates: the forced blocks are taken first; each wave keeps a quarter
// of the row in registers (M per lane) and lists its best R = k - forced
// candidates (score descending, id ascending; wave_best_r); the four lists
// are then merged by rank.  Every member of the row's best R is among its
// quarter's best R, so the result equals a selection over the whole row.
template <int M>
__global__ __launch_bounds__(256) void topk_split_kernel(
    const double* __restrict__ scores, int64_t nb,
    const int32_t* __restrict__ cu_sb, int64_t batch,
    const int32_t* __restrict__ cu_blk, int64_t n_tokens, int topk,
    const int32_t* __restrict__ forced, int n_forced, int force_self,
    int32_t* __restrict__ topk_idx, int32_t* __restrict__ compact) {
  __shared__ int s_forced[SEL_MAXK];
  __shared__ double s_ls[4][64];  // each wave's picks, best first: score, id
  __shared__ int s_li[4][64];
  __shared__ double s_cs[4][64];  // each wave's threshold survivors
  __shared__ int s_ci[4][64];
  __shared__ int s_nw[4];
  __shared__ int s_sel[SEL_MAXK];
  __shared__ int s_out[SEL_MAXK];
  __shared__ int s_nf;
  const int h = blockIdx.y;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t e = upper_index(cu_sb, 0, batch + 1, b);
  int32_t* crow = compact + ((int64_t)h * nb + b) * topk;
  if (e < 0 || e >= batch || b >= cu_sb[e + 1]) {
    clear_block_rows(cu_blk, b, n_tokens, topk, crow, topk_idx + (int64_t)h * n_tokens * topk,
                     tid, 256);
    return;
  }
  const int64_t cs = cu_sb[e];
  const int nbb = (int)(cu_sb[e + 1] - cs);
  const double* row = scores + ((int64_t)h * nb + b) * nb + cs;
  const int kmax = topk < nbb ? topk : nbb;
  // Forced blocks in order, distinct, valid, at most kmax.
  if (tid == 0) {
    int n = 0;
    auto add = [&](int id) {
      if (n >= kmax || id < 0 || id >= nbb) return;
      for (int t = 0; t < n; ++t)
        if (s_forced[t] == id) return;
      s_forced[n++] = id;
    };
    if (force_self) add((int)(b - cs));
    for (int f = 0; f < n_forced; ++f) add(forced[f]);
    s_nf = n;
  }
  __syncthreads();
  const int nf = s_nf, r_need = kmax - nf;
  // This wave's quarter [q0, q0 + 64 M) of the row.
  const int q0 = wv * 64 * M;
  double v[M];
  uint32_t taken = 0u;  // bit m: candidate q0 + lane + 64 m is unavailable
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int i = q0 + lane + 64 * m;
    if (i < nbb) {
      const double x = row[i];
      v[m] = (x != x) ? -__builtin_inf() : x;
    } else {
      v[m] = -__builtin_inf();
      taken |= 1u << m;
    }
  }
  for (int t = 0; t < nf; ++t) {
    const int i = s_forced[t] - q0;
    if (i >= 0 && i < 64 * M && (i & 63) == lane) taken |= 1u << (i >> 6);
  }
  const int nw = wave_best_r<M>(v, taken, q0, r_need, s_ls[wv], s_li[wv], s_cs[wv], s_ci[wv]);
  if (lane == 0) s_nw[wv] = nw;
  if (tid < nf) s_sel[tid] = s_forced[tid];
  __syncthreads();
  // Merge: the rank of each list entry in the union of the four lists
  // (each sorted best first) is its index plus, for every other list, the
  // number of that list's entries better than it (a binary search); the
  // entries of rank < r_need are the row's best r_need, since each member
  // of those is among its own quarter's best r_need.
  if (lane < nw) {
    const double es = s_ls[wv][lane];
    const int ei = s_li[wv][lane];
    int rank = lane;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t == wv) continue;
      int lo = 0, hi = s_nw[t];
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sel_better(s_ls[t][mid], s_li[t][mid], es, ei))
          lo = mid + 1;
        else
          hi = mid;
      }
      rank += lo;
    }
    if (rank < r_need) s_sel[nf + rank] = ei;
  }
  __syncthreads();
  // Ascending order by rank (ids are distinct), -1 padding.
  for (int j = tid; j < topk; j += 256) s_out[j] = -1;
  __syncthreads();
  for (int j = tid; j < kmax; j += 256) {
    const int id = s_sel[j];
    int r = 0;
    for (int m = 0; m < kmax; ++m) r += s_sel[m] < id;
    s_out[r] = id;
  }
  __syncthreads();
  for (int j = tid; j < topk; j += 256) crow[j] = s_out[j];
  int64_t t0 = cu_blk[b], t1 = cu_blk[b + 1];
  t0 = t0 < 0 ? 0 : (t0 > n_tokens ? n_tokens : t0);
  t1 = t1 < t0 ? t0 : (t1 > n_tokens ? n_tokens : t1);
  int32_t* dst = topk_idx + ((int64_t)h * n_tokens + t0) * topk;
  const int64_t total = (t1 - t0) * topk;
  fill_token_rows(dst, total, s_out, topk, tid, 256);
}

// Rows of tokens outside every block ([0, cu_blk[0]) and [cu_blk[nb], n),
// clamped) are -1: the top-k kernels write only the tokens of blocks.
__global__ __launch_bounds__(256) void uncovered_rows_kernel(const int32_t* __restrict__ cu_blk,
                                                             int64_t nb, int64_t n_tokens,
                                                             int topk,
                                                             int32_t* __restrict__ topk_idx) {
  const int h = blockIdx.y;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tokens) return;
  int64_t lo = cu_blk[0], hi = cu_blk[nb];
  lo = lo < 0 ? 0 : (lo > n_tokens ? n_tokens : lo);
  hi = hi < lo ? lo : (hi > n_tokens ? n_tokens : hi);
  if (t >= lo && t < hi) return;
  int32_t* row = topk_idx + ((int64_t)h * n_tokens + t) * topk;
  for (int j = 0; j < topk; ++j) row[j] = -1;
}

struct SelectWs {
  float* pq;
  float* pk;
  float* partial;
  int32_t* first;
  double* scores;
};

void carve_select(Carver& ws, int64_t n, int64_t nb, int64_t hq, int64_t hkv,
                  int64_t d, SelectWs& s) {
  const int64_t nbc = nb > 0 ? nb : 1;
  s.pq = ws.take<float>((size_t)(nbc * hq * d));
  s.pk = ws.take<float>((size_t)(nbc * hkv * d));
  s.partial = ws.take<float>((size_t)(pool_partial_rows(n, nbc) *
                                      (hq > hkv ? hq : hkv) * d));
  s.first = ws.take<int32_t>((size_t)pool_first_count(n));
  s.scores = ws.take<double>((size_t)(hkv * nbc * nbc));
}

}  // namespace lsrm

using namespace lsrm;

extern "C" size_t lsrm_select_blocks_workspace_size(int64_t n_tokens,
                                                    int64_t n_blocks,
                                                    int64_t hq, int64_t hkv,
                                                    int64_t head_dim) {
  if (n_tokens < 0 || n_blocks < 0 || hq <= 0 || hkv <= 0 || head_dim <= 0)
    return 0;
  Carver ws{nullptr, 0, 0};
  SelectWs s;
  carve_select(ws, n_tokens, n_blocks, hq, hkv, head_dim, s);
  return ws.used + 256;
}

// Shared body of lsrm_select_blocks (k given: pooled here) and
// lsrm_select_blocks_pooled (pooled_k given: the fp32 block means of k).
static int select_blocks_impl(const void* q, const void* k, const float* pooled_k, int dtype,
                              int64_t n_tokens, int64_t hq, int64_t hkv, int64_t head_dim,
                              const int32_t* cu_seqblocks, int64_t batch,
                              const int32_t* cu_block_tokens, int64_t n_blocks, int64_t topk,
                              const int32_t* forced_blocks, int64_t n_forced, int force_self,
                              int32_t* topk_idx, int32_t* topk_compact, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (n_tokens < 0 || hq <= 0 || hkv <= 0 || head_dim <= 0 || batch <= 0 ||
      n_blocks < 0 || topk <= 0 || n_forced < 0 || !cu_seqblocks ||
      !cu_block_tokens || (n_forced > 0 && !forced_blocks) ||
      (n_tokens > 0 && (!q || !(k || pooled_k) || !topk_idx)) ||
      (n_blocks > 0 && !topk_compact))
    return LSRM_ERR_INVALID_ARG;
  if (hq % hkv != 0) return LSRM_ERR_INVALID_ARG;
  if (dtype < LSRM_F32 || dtype > LSRM_BF16) return LSRM_ERR_UNSUPPORTED;
  if (head_dim > SEL_MAXD || topk > SEL_MAXK || n_blocks > SEL_MAX_CAND)
    return LSRM_ERR_UNSUPPORTED;
  const size_t need = lsrm_select_blocks_workspace_size(n_tokens, n_blocks, hq,
                                                        hkv, head_dim);
  if (workspace_bytes < need || !workspace) return LSRM_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  if (n_blocks == 0) {  // every token lies outside the (empty) block list
    if (n_tokens > 0) {
      hipLaunchKernelGGL(uncovered_rows_kernel, dim3(ceil_div(n_tokens, 256), (unsigned)hkv),
                         dim3(256), 0, st, cu_block_tokens, n_blocks, n_tokens, (int)topk,
                         topk_idx);
      LSRM_CHECK_LAUNCH();
    }
    return LSRM_OK;
  }
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0,
            workspace_bytes - 256};
  SelectWs s;
  carve_select(ws, n_tokens, n_blocks, hq, hkv, head_dim, s);
  if (!ws.ok()) return LSRM_ERR_WORKSPACE;

  int rc = launch_block_mean_pool(q, dtype, n_tokens, hq * head_dim,
                                  cu_block_tokens, n_blocks, s.pq, LSRM_F32,
                                  s.partial, s.first, st);
  if (rc) return rc;
  const float* pk = pooled_k;
  if (!pk) {
    rc = launch_block_mean_pool(k, dtype, n_tokens, hkv * head_dim, cu_block_tokens, n_blocks,
                                s.pk, LSRM_F32, s.partial, s.first, st);
    if (rc) return rc;
    pk = s.pk;
  }
  const unsigned nt = (unsigned)ceil_div(n_blocks, SCORE_TILE);
  hipLaunchKernelGGL(score_kernel, dim3(nt, nt, (unsigned)hkv), dim3(256), 0,
                     st, s.pq, pk, n_blocks, (int)hq, (int)hkv,
                     (int)head_dim, s.scores);
  LSRM_CHECK_LAUNCH();
  const unsigned rows4 = (unsigned)ceil_div(n_blocks * hkv, 4);
#define LSRM_TOPK_WAVE(M)                                                     \
  hipLaunchKernelGGL(topk_wave_kernel<M>, dim3(rows4), dim3(256), 0, st,      \
                     s.scores, n_blocks, cu_seqblocks, batch, cu_block_tokens, \
                     n_tokens, (int)hkv, (int)topk, forced_blocks,            \
                     (int)n_forced, force_self, topk_idx, topk_compact)
  if (n_blocks <= 64 * 4)
    LSRM_TOPK_WAVE(4);
  else if (n_blocks <= 64 * 8)
    LSRM_TOPK_WAVE(8);
  else if (n_blocks <= 64 * 16)
    LSRM_TOPK_WAVE(16);
  else if (n_blocks <= 64 * 32)
    LSRM_TOPK_WAVE(32);
  else if (n_blocks <= 4 * 64 * 32 && topk <= 64) {
#define LSRM_TOPK_SPLIT(M)                                                                \
  hipLaunchKernelGGL(topk_split_kernel<M>, dim3((unsigned)n_blocks, (unsigned)hkv),      \
                     dim3(256), 0, st, s.scores, n_blocks, cu_seqblocks, batch,            \
                     cu_block_tokens, n_tokens, (int)topk, forced_blocks, (int)n_forced,   \
                     force_self, topk_idx, topk_compact)
    if (n_blocks <= 4 * 64 * 12)
      LSRM_TOPK_SPLIT(12);
    else if (n_blocks <= 4 * 64 * 16)
      LSRM_TOPK_SPLIT(16);
    else if (n_blocks <= 4 * 64 * 20)
      LSRM_TOPK_SPLIT(20);
    else if (n_blocks <= 4 * 64 * 24)
      LSRM_TOPK_SPLIT(24);
    else
      LSRM_TOPK_SPLIT(32);
#undef LSRM_TOPK_SPLIT
  } else
    hipLaunchKernelGGL(topk_kernel, dim3((unsigned)n_blocks, (unsigned)hkv),
                       dim3(256), 0, st, s.scores, n_blocks, cu_seqblocks,
                       batch, cu_block_tokens, n_tokens, (int)topk,
                       forced_blocks, (int)n_forced, force_self, topk_idx,
                       topk_compact);
#undef LSRM_TOPK_WAVE
  LSRM_CHECK_LAUNCH();
  hipLaunchKernelGGL(uncovered_rows_kernel, dim3(ceil_div(n_tokens, 256), (unsigned)hkv),
                     dim3(256), 0, st, cu_block_tokens, n_blocks, n_tokens, (int)topk, topk_idx);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

extern "C" int lsrm_select_blocks(const void* q, const void* k, int dtype, int64_t n_tokens,
                                  int64_t hq, int64_t hkv, int64_t head_dim,
                                  const int32_t* cu_seqblocks, int64_t batch,
                                  const int32_t* cu_block_tokens, int64_t n_blocks, int64_t topk,
                                  const int32_t* forced_blocks, int64_t n_forced, int force_self,
                                  int32_t* topk_idx, int32_t* topk_compact, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (n_tokens > 0 && !k) return LSRM_ERR_INVALID_ARG;
  return select_blocks_impl(q, k, nullptr, dtype, n_tokens, hq, hkv, head_dim, cu_seqblocks,
                            batch, cu_block_tokens, n_blocks, topk, forced_blocks, n_forced,
                            force_self, topk_idx, topk_compact, workspace, workspace_bytes,
                            stream);
}

extern "C" int lsrm_select_blocks_pooled(const void* q, const float* pooled_k, int dtype,
                                         int64_t n_tokens, int64_t hq, int64_t hkv,
                                         int64_t head_dim, const int32_t* cu_seqblocks,
                                         int64_t batch, const int32_t* cu_block_tokens,
                                         int64_t n_blocks, int64_t topk,
                                         const int32_t* forced_blocks, int64_t n_forced,
                                         int force_self, int32_t* topk_idx,
                                         int32_t* topk_compact, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  if (n_blocks > 0 && !pooled_k) return LSRM_ERR_INVALID_ARG;
  return select_blocks_impl(q, nullptr, pooled_k, dtype, n_tokens, hq, hkv, head_dim,
                            cu_seqblocks, batch, cu_block_tokens, n_blocks, topk, forced_blocks,
                            n_forced, force_self, topk_idx, topk_compact, workspace,
                            workspace_bytes, stream);
}
