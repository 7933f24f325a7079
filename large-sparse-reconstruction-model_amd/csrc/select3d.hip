// 3D-aware per-token block selection (the use_3d_aware_attn branch of
// build_volume_to_volume_attn, misc/sparse_utils.py:1203-1280) on gfx950.
//
//   volume_points_kernel : integer volume coordinates (batch, c1, c2, c3) ->
//     fp32 points (x, y, z) = (f(c3), f(c2), f(c1)) with
//     f(c) = 2 * (c / (R - 1) - 0.5) * radius, evaluated in that order in
//     fp32 (from_volcoords_to_points, lines 644-650).
//   nearest_blocks_kernel : for every token, the min(topk, blocks of its
//     batch element) blocks whose centroid (the block mean of its points,
//     computed by lsrm_block_mean_pool) is nearest, listed ascending, -1
//     padded, written once per kv head (the reference stacks the same rows
//     for its kv heads, line 1273).  Distances rank by the squared
//     distance in fp64 (fp32 differences, squares and their three-term sum
//     are exact there), ties by the lower block id; one lane per token
//     keeps a running top-K list in registers while the wave walks the
//     centroids of its batch element with wave-uniform (scalar) loads.
//     topk in (64, 128] takes two launches of the 64-entry list: the first
//     writes its best k1 = min(64, topk - 3) ids and the k1-th (distance,
//     id) into head 0's row, the second keeps only blocks ranking after
//     that bound and merges both ascending lists.
#include "common.h"

namespace lsrm {

__global__ __launch_bounds__(256) void volume_points_kernel(
    const int32_t* __restrict__ coords, int64_t n, float den, float radius,
    float* __restrict__ points) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t* c = coords + i * 4;
  auto f = [&](int32_t v) { return 2.0f * ((float)v / den - 0.5f) * radius; };
  points[i * 3 + 0] = f(c[3]);
  points[i * 3 + 1] = f(c[2]);
  points[i * 3 + 2] = f(c[1]);
}

constexpr int NB_ONE = 0, NB_FIRST = 1, NB_SECOND = 2;

template <int K, int MODE>
__global__ __launch_bounds__(256) void nearest_blocks_kernel(
    const float* __restrict__ points, const float* __restrict__ centroids,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_sb, int64_t batch,
    int64_t n, int topk, int hkv, int k1, int32_t* __restrict__ out) {
  static_assert(MODE == NB_ONE || K == 64, "the two-pass roles use the 64-entry list");
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t w0 = (int64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~63);
  if (w0 >= n) return;
  const bool live = i < n;
  const int64_t ic = live ? i : n - 1;
  const double px = points[ic * 3 + 0], py = points[ic * 3 + 1], pz = points[ic * 3 + 2];
  const int64_t wl = w0 + 63 < n ? w0 + 63 : n - 1;
  const int b_first = (int)upper_index(cu_q, 0, batch + 1, w0);
  const int b_last = (int)upper_index(cu_q, 0, batch + 1, wl);
  const int my_b = (int)upper_index(cu_q, 0, batch + 1, ic);

  double tv[K];
  int ti[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    tv[k] = __builtin_inf();
    ti[k] = 0x7fffffff;  // empty: any candidate ranks before it
  }
  // ids this launch selects, and (second pass) the bound to rank after
  const int kout = MODE == NB_ONE ? topk : (MODE == NB_FIRST ? k1 : topk - k1);
  double bnd_d = -1.0;
  int bnd_i = 0x7fffffff;
  if constexpr (MODE == NB_SECOND) {
    if (live) {
      const int32_t* src = out + i * topk;  // head 0's row
      const uint64_t lo = (uint32_t)src[k1], hi = (uint32_t)src[k1 + 1];
      bnd_d = __longlong_as_double((long long)((hi << 32) | lo));
      bnd_i = src[k1 + 2];
    }
  }
  int kk = 0;
  for (int b = b_first < 0 ? 0 : b_first; b <= b_last && b < batch; ++b) {
    const int bs = cu_sb[b], be = cu_sb[b + 1];
    if (my_b == b) kk = be - bs < kout ? (be - bs > 0 ? be - bs : 0) : kout;
    for (int c = bs; c < be; ++c) {  // wave-uniform: scalar centroid loads
      const double dx = px - (double)centroids[(int64_t)c * 3 + 0];
      const double dy = py - (double)centroids[(int64_t)c * 3 + 1];
      const double dz = pz - (double)centroids[(int64_t)c * 3 + 2];
      double d = dx * dx;
      d = d + dy * dy;
      d = d + dz * dz;
      if (d != d) d = __builtin_inf();  // NaN ranks with +inf
      const int id = c - bs;
      // ids arrive ascending: an equal distance already listed keeps its
      // place, an empty slot (id INT_MAX) always yields.
      const bool after = MODE != NB_SECOND || d > bnd_d || (d == bnd_d && id > bnd_i);
      if (my_b == b && after && (d < tv[K - 1] || (d == tv[K - 1] && id < ti[K - 1]))) {
#pragma unroll
        for (int k = K - 1; k >= 0; --k) {
          const int kp = k > 0 ? k - 1 : 0;
          const bool prev_after = k > 0 && (tv[kp] > d || (tv[kp] == d && ti[kp] > id));
          const bool here_after = tv[k] > d || (tv[k] == d && ti[k] > id);
          if (here_after) {
            tv[k] = prev_after ? tv[kp] : d;
            ti[k] = prev_after ? ti[kp] : id;
          }
        }
      }
    }
  }
  if (!live) return;
  // The kk nearest ids, ascending (bitonic sort; unused slots last).
  int ids[K];
#pragma unroll
  for (int k = 0; k < K; ++k) ids[k] = (k < kk && ti[k] != 0x7fffffff) ? ti[k] : 0x7fffffff;
#pragma unroll
  for (int size = 2; size <= K; size <<= 1) {
#pragma unroll
    for (int j = size / 2; j > 0; j >>= 1) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int o = k ^ j;
        if (o > k) {
          const bool up = (k & size) == 0;
          const int lo = ids[k] < ids[o] ? ids[k] : ids[o];
          const int hi = ids[k] < ids[o] ? ids[o] : ids[k];
          ids[k] = up ? lo : hi;
          ids[o] = up ? hi : lo;
        }
      }
    }
  }
  if constexpr (MODE == NB_ONE) {
    for (int h = 0; h < hkv; ++h) {
      int32_t* dst = out + ((int64_t)h * n + i) * topk;
#pragma unroll
      for (int k = 0; k < K; ++k)
        if (k < topk) dst[k] = (k < kk && ids[k] != 0x7fffffff) ? ids[k] : -1;
    }
  } else if constexpr (MODE == NB_FIRST) {
    int32_t* dst = out + i * topk;  // head 0's row holds the first pass
    double bd = __builtin_inf();
    int bi = -1;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (k < k1) dst[k] = (k < kk && ids[k] != 0x7fffffff) ? ids[k] : -1;
      if (k == k1 - 1 && kk == k1 && ti[k] != 0x7fffffff) {  // the k1-th nearest
        bd = tv[k];
        bi = ti[k];
      }
    }
    // without k1 chosen blocks nothing may follow: +inf and the largest id
    const uint64_t bits = (uint64_t)__double_as_longlong(bd);
    dst[k1] = (int32_t)(uint32_t)bits;
    dst[k1 + 1] = (int32_t)(uint32_t)(bits >> 32);
    dst[k1 + 2] = bi >= 0 ? bi : 0x7fffffff;
  } else {
    // merge with the first pass's k1 ascending ids (0x7fffffff = none)
    const int32_t* src = out + i * topk;
    int first[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int x = k < k1 ? src[k] : -1;
      first[k] = x >= 0 ? x : 0x7fffffff;
    }
    int n1 = 0, n2 = 0, slot1[K], slot2[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      n1 += first[k] != 0x7fffffff ? 1 : 0;
      n2 += ids[k] != 0x7fffffff ? 1 : 0;
      int r1 = k, r2 = k;  // own index + ids of the other list below
#pragma unroll
      for (int j = 0; j < K; ++j) {
        r1 += ids[j] < first[k] ? 1 : 0;
        r2 += first[j] < ids[k] ? 1 : 0;
      }
      slot1[k] = r1;
      slot2[k] = r2;
    }
    for (int h = 0; h < hkv; ++h) {
      int32_t* dst = out + ((int64_t)h * n + i) * topk;
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (first[k] != 0x7fffffff) dst[slot1[k]] = first[k];
        if (ids[k] != 0x7fffffff) dst[slot2[k]] = ids[k];
      }
      for (int k = n1 + n2; k < topk; ++k) dst[k] = -1;
    }
  }
}

}  // namespace lsrm

using namespace lsrm;

extern "C" int lsrm_volume_points(const int32_t* coords, int64_t n_tokens, int64_t volume_res,
                                  float radius, float* points, void* stream) {
  if (n_tokens < 0 || volume_res < 2 || (n_tokens > 0 && (!coords || !points)))
    return LSRM_ERR_INVALID_ARG;
  if (n_tokens == 0) return LSRM_OK;
  hipLaunchKernelGGL(volume_points_kernel, dim3((unsigned)((n_tokens + 255) / 256)), dim3(256),
                     0, (hipStream_t)stream, coords, n_tokens, (float)(volume_res - 1), radius,
                     points);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

extern "C" int lsrm_nearest_blocks(const float* points, const float* centroids,
                                   const int32_t* cu_seqlens, const int32_t* cu_seqblocks,
                                   int64_t batch, int64_t n_tokens, int64_t topk,
                                   int64_t hkv, int32_t* block_topk, void* stream) {
  if (n_tokens < 0 || batch <= 0 || topk <= 0 || hkv <= 0 || !cu_seqlens || !cu_seqblocks ||
      (n_tokens > 0 && (!points || !centroids || !block_topk)))
    return LSRM_ERR_INVALID_ARG;
  if (topk > 128) return LSRM_ERR_UNSUPPORTED;
  if (n_tokens == 0) return LSRM_OK;
  const dim3 grid((unsigned)((n_tokens + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (topk > 64) {
    const int k1 = topk - 3 < 64 ? (int)topk - 3 : 64;
    hipLaunchKernelGGL((nearest_blocks_kernel<64, NB_FIRST>), grid, dim3(256), 0, st, points,
                       centroids, cu_seqlens, cu_seqblocks, batch, n_tokens, (int)topk, (int)hkv,
                       k1, block_topk);
    LSRM_CHECK_LAUNCH();
    hipLaunchKernelGGL((nearest_blocks_kernel<64, NB_SECOND>), grid, dim3(256), 0, st, points,
                       centroids, cu_seqlens, cu_seqblocks, batch, n_tokens, (int)topk, (int)hkv,
                       k1, block_topk);
    LSRM_CHECK_LAUNCH();
    return LSRM_OK;
  }
#define LSRM_NB_K(KV)                                                                   \
  hipLaunchKernelGGL((nearest_blocks_kernel<KV, NB_ONE>), grid, dim3(256), 0, st, points, \
                     centroids, cu_seqlens, cu_seqblocks, batch, n_tokens, (int)topk,     \
                     (int)hkv, 0, block_topk);                                           \
  break;
  switch (topk <= 8 ? 8 : topk <= 16 ? 16 : topk <= 32 ? 32 : 64) {
    case 8: LSRM_NB_K(8)
    case 16: LSRM_NB_K(16)
    case 32: LSRM_NB_K(32)
    default: LSRM_NB_K(64)
  }
#undef LSRM_NB_K
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}
