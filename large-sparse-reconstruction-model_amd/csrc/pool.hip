// Block mean pooling over variable-length token blocks (key/value block
// compression of LSRM, sparse/module/spatial_sparse_attention.py:27-37, which
// calls torch.segment_reduce(reduce="mean") on a [N, H*D] tensor).
//
// Streaming kernels:
//   pool_chunk_first : the block owning each chunk's first row (one binary
//                  search per chunk).
//   pool_pieces  : one thread per (64-row chunk, 8-channel group) sums its rows
//                  (16-bit rows: 16 packed 16-byte loads in flight per thread)
//                  in fp32, emitting a partial sum each time a block boundary
//                  is crossed.  Partial (block b, chunk j) lives at row b + j
//                  of the partial buffer (unique because blocks are
//                  contiguous and ordered).
//   pool_pieces_slab : the 16-bit, 512-channel-multiple form of pool_pieces
//                  (one wave per chunk and 512-channel slab, 64 VGPRs).
//   pool_pieces_rows : the same with two or three 512-channel slabs per wave
//                  (whole rows at 1536 channels).
//   pool_combine : one thread per (block, 4-channel group) adds the block's
//                  partials in chunk order, divides by the length and rounds.
//   pool_combine2: the same for two tensors (keys and values) in one launch.
// Every add is sequential, so the result is a fixed function of the input
// (the contract the CPU oracle restates bit for bit).  Input rows are read
// exactly once, with nontemporal loads (measured +8% on the cfg3 K tensor).
#include <mutex>

#include "common.h"

namespace lsrm {

constexpr int POOL_CHUNK = 64;  // rows per piece boundary (part of the contract)
constexpr int POOL_VEC = 8;     // channels per thread on the vector path

template <int DT>
struct Vec8 {
  // Loads channels [c, c+8) of row r as fp32.
  __device__ static inline void load(const void* x, int64_t off, float* v) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
        reinterpret_cast<const uint16_t*>(x) + off));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = to_f32<DT>((uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = to_f32<DT>((uint16_t)(w[i] >> 16));
    }
  }
};
template <>
struct Vec8<LSRM_F32> {
  __device__ static inline void load(const void* x, int64_t off, float* v) {
    const f32x4* p = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(x) + off);
    const f32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
    v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  }
};

template <int DT>
__device__ inline float load1(const void* x, int64_t off) {
  if constexpr (DT == LSRM_F32)
    return reinterpret_cast<const float*>(x)[off];
  else
    return to_f32<DT>(reinterpret_cast<const uint16_t*>(x)[off]);
}

// VEC channels per thread (8 on the 16-byte path, 1 on the scalar path).
// first[j] = last block whose start is <= 64 j (the block owning chunk j's
// first row, or -1 / nb outside the blocks): one binary search per chunk
// instead of one per thread.
__global__ __launch_bounds__(256) void pool_chunk_first(
    const int32_t* __restrict__ cu, int64_t nb, int64_t n_chunks,
    int32_t* __restrict__ first) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n_chunks) return;
  int64_t b = upper_index(cu, 0, nb + 1, j * POOL_CHUNK);
  first[j] = (int32_t)(b > nb ? nb : b);
}

// WU: every wave's items share one chunk (channel groups a multiple of 64),
// so the chunk index is made wave-uniform and all row / block-boundary control
// flow runs on the scalar unit.
template <int DT, int VEC, bool WU>
__global__ __launch_bounds__(256) void pool_pieces(
    const void* __restrict__ x, int64_t n, int64_t ch,
    const int32_t* __restrict__ cu, int64_t nb,
    const int32_t* __restrict__ first, float* __restrict__ partial) {
  const int64_t n_vec = ch / VEC;
  const int64_t n_chunks = (n + POOL_CHUNK - 1) / POOL_CHUNK;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= n_chunks * n_vec) return;
  int64_t j = item / n_vec;
  const int64_t c0 = (item - j * n_vec) * VEC;
  if constexpr (WU) j = __builtin_amdgcn_readfirstlane((int)j);
  const int64_t r0 = j * POOL_CHUNK;
  const int64_t r1 = r0 + POOL_CHUNK < n ? r0 + POOL_CHUNK : n;

  // b = last block whose start is <= r0 (-1: before the first block,
  // nb: past the last).  bs/be bound the rows block b owns.
  int64_t b = first[j];
  int64_t be = b < 0 ? (int64_t)cu[0] : (b < nb ? (int64_t)cu[b + 1] : INT64_MAX);
  int64_t bs = (b >= 0 && b < nb) ? (int64_t)cu[b] : INT64_MAX;

  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;
  bool have = false;

  auto flush = [&]() {
    float* dst = partial + (b + j) * ch + c0;
#pragma unroll
    for (int i = 0; i < VEC; ++i) dst[i] = acc[i];
  };

  constexpr int U = 16;  // rows in flight per thread
  for (int64_t r = r0; r < r1; r += U) {
    // 16-bit rows stay packed until they are added (fewer registers, more
    // loads in flight); all U loads are issued (rows past the chunk re-read
    // its last row and are skipped below) before any is used.
    u32x4 raw[U];
    float v1[U];
    if constexpr (VEC == 8 && DT != LSRM_F32) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr = r + u < r1 ? r + u : r1 - 1;
        raw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            reinterpret_cast<const uint16_t*>(x) + rr * ch + c0));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) asm volatile("" ::"v"(raw[u]));
    } else if constexpr (VEC == 1) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        v1[u] = r + u < r1 ? load1<DT>(x, (r + u) * ch + c0) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = r + u;
      if (row < r1) {
        while (b < nb && row >= be) {
          if (have) flush();
          have = false;
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;
          ++b;
          bs = b < nb ? (int64_t)cu[b] : INT64_MAX;
          be = b < nb ? (int64_t)cu[b + 1] : INT64_MAX;
        }
        if (b >= 0 && b < nb && row >= bs) {
          float v[VEC];
          if constexpr (VEC == 8 && DT != LSRM_F32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[2 * i] = to_f32<DT>((uint16_t)(raw[u][i] & 0xffffu));
              v[2 * i + 1] = to_f32<DT>((uint16_t)(raw[u][i] >> 16));
            }
          } else if constexpr (VEC == 8) {
            Vec8<DT>::load(x, row * ch + c0, v);
          } else {
            v[0] = v1[u];
          }
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = acc[i] + v[i];
          have = true;
        }
      }
    }
  }
  if (have && b >= 0 && b < nb) flush();
}

// 16-bit rows, channel count a multiple of 512: one wave per (64-row chunk,
// 512-channel slab), 8 channels per lane.  Rows stream in double-buffered
// groups of POOL_G; the kernel is held to 64 VGPRs (8 waves per SIMD) so a
// launch of a few thousand waves is resident at once instead of running in
// one and a half rounds.  With IF, the block owning the chunk's first row is
// found in the kernel (nb + 1 <= 512 offsets: lane l compares entries
// 8l..8l+7 with the row and the wave counts the hits); those loads are issued
// before the first row group, so the wave waits for them alone.  Otherwise
// the block comes from the pool_chunk_first table.  The end of the next
// block is loaded one crossing ahead, and row groups that lie inside the
// current block are added without per-row checks.  The sums are the same
// sequential fp32 sums as in pool_pieces.
constexpr int POOL_G = 4;  // rows per load group

// NT = 2 pools a second tensor of the same shape and blocks (x2 -> partial2)
// in the same launch: its items follow the first tensor's.  LPC = 32 (256
// channels, with the lookup table; kernel pool_pieces_half): a wave covers
// two chunks, one per half, the chunk index and block state per lane.
template <int DT, bool IF, int NT, int LPC, bool IF2 = false>
__device__ __forceinline__ void pool_slab_body(const uint16_t* __restrict__ x, int64_t n,
                                               int64_t ch, const int32_t* __restrict__ cu,
                                               int64_t nb, const int32_t* __restrict__ first,
                                               float* __restrict__ partial,
                                               const uint16_t* __restrict__ x2,
                                               float* __restrict__ partial2) {
  // Item counts stay below 2^31 (checked by the launcher): 32-bit indexing.
  const uint32_t n_vec = (uint32_t)(ch / 8);
  const uint32_t n_chunks = (uint32_t)((n + POOL_CHUNK - 1) / POOL_CHUNK);
  uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= NT * n_chunks * n_vec) return;  // whole waves (n_vec % 64 == 0)
  if constexpr (NT == 2) {
    if (item >= n_chunks * n_vec) {  // wave-uniform: the second tensor
      item -= n_chunks * n_vec;
      x = x2;
      partial = partial2;
    }
  }
  static_assert(LPC == 64 || !IF, "the in-kernel lookup needs one chunk per wave");
  const int64_t j =
      LPC == 64 ? (int64_t)__builtin_amdgcn_readfirstlane(item / n_vec) : (int64_t)(item / n_vec);
  const int64_t c0 = (int64_t)(item - (uint32_t)j * n_vec) * 8;
  const int64_t r0 = j * POOL_CHUNK;
  const int64_t r1 = r0 + POOL_CHUNK < n ? r0 + POOL_CHUNK : n;
  const uint16_t* xp = x + c0;

  u32x4 buf[2][POOL_G];
  auto load_group = [&](u32x4* dst, int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < POOL_G; ++u) {
      const int64_t rr = r + u < r1 ? r + u : r1 - 1;
      dst[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xp + rr * ch));
    }
  };

  // b = last block whose start is <= r0 (-1: before the first block,
  // nb: past the last).  bs/be bound the rows block b owns.
  int64_t b;
  if constexpr (IF) {
    const int lane = threadIdx.x & 63;
    int32_t cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t idx = 8 * lane + i;
      cv[i] = cu[idx <= nb ? idx : nb];
    }
    load_group(buf[0], r0);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      cnt += __popcll(__ballot((int64_t)cv[i] <= r0 && 8 * lane + i <= nb));
    b = __builtin_amdgcn_readfirstlane(cnt) - 1;
  } else if constexpr (IF2) {
    // Two-level count of the offsets <= r0 for this half-wave's chunk
    // (nb + 1 <= 8192): its 32 lanes read every S-th offset (S = ceil((nb +
    // 1) / 32) <= 256), then the S offsets from the last sampled hit on, up
    // to 8 per lane in one round.  Offsets are nondecreasing, so the hits
    // are a prefix and the count is base + the second round's hits.
    static_assert(LPC == 32, "one chunk per half-wave");
    const int lane = threadIdx.x & 63, hl = lane & 31;
    const uint64_t half = lane < 32 ? 0xffffffffull : 0xffffffff00000000ull;
    const int64_t S = (nb + 32) / 32;
    const int64_t i1 = hl * S;
    const int32_t v1 = cu[i1 <= nb ? i1 : nb];
    load_group(buf[0], r0);
    const int c1 = __popcll(__ballot(i1 <= nb && (int64_t)v1 <= r0) & half);
    const int64_t base = c1 > 0 ? (int64_t)(c1 - 1) * S : 0;
    int32_t v2[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int64_t i2 = base + hl + 32 * m;
      v2[m] = cu[hl + 32 * m < S && i2 <= nb ? i2 : 0];
    }
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int64_t i2 = base + hl + 32 * m;
      cnt += __popcll(__ballot(c1 > 0 && hl + 32 * m < S && i2 <= nb && (int64_t)v2[m] <= r0) &
                      half);
    }
    b = c1 > 0 ? base + cnt - 1 : -1;
  } else {
    load_group(buf[0], r0);
    b = first[j];
  }
  int64_t be = b < 0 ? (int64_t)cu[0] : (b < nb ? (int64_t)cu[b + 1] : INT64_MAX);
  int64_t bs = (b >= 0 && b < nb) ? (int64_t)cu[b] : INT64_MAX;

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  auto add_row = [&](const u32x4& w) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = acc[2 * i] + to_f32<DT>((uint16_t)(w[i] & 0xffffu));
      acc[2 * i + 1] = acc[2 * i + 1] + to_f32<DT>((uint16_t)(w[i] >> 16));
    }
  };
  auto flush = [&]() __attribute__((always_inline)) {
    float4* dst = reinterpret_cast<float4*>(partial + (b + j) * ch + c0);
    dst[0] = float4{acc[0], acc[1], acc[2], acc[3]};
    dst[1] = float4{acc[4], acc[5], acc[6], acc[7]};
  };
  constexpr int NG = POOL_CHUNK / POOL_G;

  if (b >= 0 && b < nb && bs <= r0 && be >= r1) {
    // The chunk lies inside block b: no boundary checks.
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g + 1 < NG) load_group(buf[(g + 1) & 1], r0 + (g + 1) * POOL_G);
#pragma unroll
      for (int u = 0; u < POOL_G; ++u)
        if (r0 + g * POOL_G + u < r1) add_row(buf[g & 1][u]);
    }
    flush();
    return;
  }
  // bn = end of block b + 1 (its start is be).
  int64_t bn = b + 1 < nb ? (int64_t)cu[b + 2] : INT64_MAX;
  bool have = false;
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g + 1 < NG) load_group(buf[(g + 1) & 1], r0 + (g + 1) * POOL_G);
    const int64_t g0 = r0 + g * POOL_G;
    if (b >= 0 && b < nb && bs <= g0 && be >= g0 + POOL_G && g0 + POOL_G <= r1) {
#pragma unroll
      for (int u = 0; u < POOL_G; ++u) add_row(buf[g & 1][u]);
      have = true;
      continue;
    }
#pragma unroll
    for (int u = 0; u < POOL_G; ++u) {
      const int64_t row = g0 + u;
      if (row < r1) {
        while (b < nb && row >= be) {
          if (have && b >= 0) flush();
          have = false;
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
          ++b;
          bs = b < nb ? be : INT64_MAX;
          be = b < nb ? bn : INT64_MAX;
          bn = b + 1 < nb ? (int64_t)cu[b + 2] : INT64_MAX;
        }
        if (b >= 0 && b < nb && row >= bs) {
          add_row(buf[g & 1][u]);
          have = true;
        }
      }
    }
  }
  if (have && b >= 0 && b < nb) flush();
}

template <int DT, bool IF, int NT = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8))) void
pool_pieces_slab(const uint16_t* __restrict__ x, int64_t n, int64_t ch,
                 const int32_t* __restrict__ cu, int64_t nb,
                 const int32_t* __restrict__ first, float* __restrict__ partial,
                 const uint16_t* __restrict__ x2 = nullptr,
                 float* __restrict__ partial2 = nullptr) {
  pool_slab_body<DT, IF, NT, 64>(x, n, ch, cu, nb, first, partial, x2, partial2);
}

// 256 channels: two chunks per wave (block state per lane, up to 128 VGPRs).
// IF2: the block lookup in the kernel (nb + 1 <= POOL_IF2_MAX), else the
// pool_chunk_first table.
constexpr int64_t POOL_IF2_MAX = 8192;
template <int DT, bool IF2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void
pool_pieces_half(const uint16_t* __restrict__ x, int64_t n, int64_t ch,
                 const int32_t* __restrict__ cu, int64_t nb,
                 const int32_t* __restrict__ first, float* __restrict__ partial) {
  pool_slab_body<DT, false, 1, 32, IF2>(x, n, ch, cu, nb, first, partial, nullptr, nullptr);
}

// 16-bit rows, channel count a multiple of S x 512 (S = 2 or 3): one wave
// per (64-row chunk, S x 512 channels) -- for S x 512 = C a wave reads whole
// rows, contiguous in memory -- with S 16-byte loads per lane per row, rows in
// double-buffered groups of two, up to 128 VGPRs (4 waves per SIMD).  Same
// pieces, same sequential fp32 sums and same block lookup as
// pool_pieces_slab (bit-identical partials); on config 3's 1536 channels the
// whole-row waves read 4% faster than three 512-channel waves per chunk.
constexpr int POOL_RG = 2;  // rows per load group of the whole-row kernel

template <int DT, bool IF, int S, int NT = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void
pool_pieces_rows(const uint16_t* __restrict__ x, int64_t n, int64_t ch,
                 const int32_t* __restrict__ cu, int64_t nb,
                 const int32_t* __restrict__ first, float* __restrict__ partial,
                 const uint16_t* __restrict__ x2 = nullptr,
                 float* __restrict__ partial2 = nullptr) {
  // Item counts stay below 2^31 (checked by the launcher): 32-bit indexing.
  const uint32_t n_thr = (uint32_t)(ch / 8) / S;  // threads per chunk
  const uint32_t n_chunks = (uint32_t)((n + POOL_CHUNK - 1) / POOL_CHUNK);
  uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= NT * n_chunks * n_thr) return;  // whole waves (n_thr % 64 == 0)
  if constexpr (NT == 2) {
    if (item >= n_chunks * n_thr) {  // wave-uniform: the second tensor
      item -= n_chunks * n_thr;
      x = x2;
      partial = partial2;
    }
  }
  const int64_t j = __builtin_amdgcn_readfirstlane(item / n_thr);
  const uint32_t t = item - (uint32_t)j * n_thr;
  const uint32_t w = t / 64, ln = t % 64;
  // channel groups of this lane: slabs w*S .. w*S + S - 1, 8 channels each
  int64_t c0[S];
  const uint16_t* xs[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    c0[s] = (int64_t)(((w * S + s) * 64 + ln) * 8);
    xs[s] = x + c0[s];
  }
  const int64_t r0 = j * POOL_CHUNK;
  const int64_t r1 = r0 + POOL_CHUNK < n ? r0 + POOL_CHUNK : n;

  u32x4 buf_a[POOL_RG][S], buf_b[POOL_RG][S];
  auto load_group = [&](auto& dst, int64_t r) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < POOL_RG; ++u) {
      const int64_t rr = r + u < r1 ? r + u : r1 - 1;
#pragma unroll
      for (int s = 0; s < S; ++s)
        dst[u][s] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xs[s] + rr * ch));
    }
  };

  // b = last block whose start is <= r0 (-1: before the first block,
  // nb: past the last).  bs/be bound the rows block b owns.
  int64_t b;
  if constexpr (IF) {
    const int lane = threadIdx.x & 63;
    int32_t cv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t idx = 8 * lane + i;
      cv[i] = cu[idx <= nb ? idx : nb];
    }
    load_group(buf_a, r0);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      cnt += __popcll(__ballot((int64_t)cv[i] <= r0 && 8 * lane + i <= nb));
    b = __builtin_amdgcn_readfirstlane(cnt) - 1;
  } else {
    load_group(buf_a, r0);
    b = first[j];
  }
  int64_t be = b < 0 ? (int64_t)cu[0] : (b < nb ? (int64_t)cu[b + 1] : INT64_MAX);
  int64_t bs = (b >= 0 && b < nb) ? (int64_t)cu[b] : INT64_MAX;
  int64_t bn = b + 1 < nb ? (int64_t)cu[b + 2] : INT64_MAX;  // end of block b + 1

  float acc[S][8];
  auto clear = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[s][i] = 0.0f;
  };
  clear();
  auto add_row = [&](const auto& bb, int u) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wv = bb[u][s][i];
        acc[s][2 * i] = acc[s][2 * i] + to_f32<DT>((uint16_t)(wv & 0xffffu));
        acc[s][2 * i + 1] = acc[s][2 * i + 1] + to_f32<DT>((uint16_t)(wv >> 16));
      }
  };
  auto flush = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      float4* dst = reinterpret_cast<float4*>(partial + (b + j) * ch + c0[s]);
      dst[0] = float4{acc[s][0], acc[s][1], acc[s][2], acc[s][3]};
      dst[1] = float4{acc[s][4], acc[s][5], acc[s][6], acc[s][7]};
    }
  };
  const bool inside = b >= 0 && b < nb && bs <= r0 && be >= r1;  // no boundary in the chunk
  bool have = false;
  // The rows of one group [g0, g0 + POOL_RG) from buffer bb.
  auto group = [&](const auto& bb, int64_t g0) __attribute__((always_inline)) {
    if (inside) {
#pragma unroll
      for (int u = 0; u < POOL_RG; ++u)
        if (g0 + u < r1) add_row(bb, u);
      have = true;
      return;
    }
    if (b >= 0 && b < nb && bs <= g0 && be >= g0 + POOL_RG && g0 + POOL_RG <= r1) {
#pragma unroll
      for (int u = 0; u < POOL_RG; ++u) add_row(bb, u);
      have = true;
      return;
    }
#pragma unroll
    for (int u = 0; u < POOL_RG; ++u) {
      const int64_t row = g0 + u;
      if (row < r1) {
        while (b < nb && row >= be) {
          if (have && b >= 0) flush();
          have = false;
          clear();
          ++b;
          bs = b < nb ? be : INT64_MAX;
          be = b < nb ? bn : INT64_MAX;
          bn = b + 1 < nb ? (int64_t)cu[b + 2] : INT64_MAX;
        }
        if (b >= 0 && b < nb && row >= bs) {
          add_row(bb, u);
          have = true;
        }
      }
    }
  };
  constexpr int NG = POOL_CHUNK / POOL_RG;
  static_assert(NG % 2 == 0, "groups alternate between the two buffers");
  for (int g = 0; g < NG; g += 2) {
    load_group(buf_b, r0 + (g + 1) * POOL_RG);
    group(buf_a, r0 + g * POOL_RG);
    if (g + 2 < NG) load_group(buf_a, r0 + (g + 2) * POOL_RG);
    group(buf_b, r0 + (g + 1) * POOL_RG);
  }
  if (have && b >= 0 && b < nb) flush();
}

// Slabs of 512 channels per wave for the 16-bit piece kernels: whole rows
// of 1536 channels (or any multiple of it) as 3, multiples of 1024 as 2,
// else one (pool_pieces_slab).
inline int pool_slabs_per_wave(int64_t ch) {
  const int64_t n_vec = ch / POOL_VEC;
  return n_vec % 192 == 0 ? 3 : (n_vec % 128 == 0 ? 2 : 1);
}

// The 16-bit piece launch for NT tensors (x2 / partial2: the second).
template <int DT, int NT>
void launch_pieces16(const uint16_t* x, const uint16_t* x2, int64_t n, int64_t ch,
                     const int32_t* cu, int64_t nb, const int32_t* first, float* partial,
                     float* partial2, bool inline_first, hipStream_t st) {
  const int64_t n_chunks = (n + POOL_CHUNK - 1) / POOL_CHUNK;
  const int S = pool_slabs_per_wave(ch);
  const int64_t items = NT * n_chunks * (ch / POOL_VEC) / S;
  const dim3 grid((unsigned)((items + 255) / 256)), block(256);
#define LSRM_PIECES(K) hipLaunchKernelGGL(K, grid, block, 0, st, x, n, ch, cu, nb, first, \
                                          partial, x2, partial2)
  if (S == 3) {
    if (inline_first) LSRM_PIECES((pool_pieces_rows<DT, true, 3, NT>));
    else LSRM_PIECES((pool_pieces_rows<DT, false, 3, NT>));
  } else if (S == 2) {
    if (inline_first) LSRM_PIECES((pool_pieces_rows<DT, true, 2, NT>));
    else LSRM_PIECES((pool_pieces_rows<DT, false, 2, NT>));
  } else {
    if (inline_first) LSRM_PIECES((pool_pieces_slab<DT, true, NT>));
    else LSRM_PIECES((pool_pieces_slab<DT, false, NT>));
  }
#undef LSRM_PIECES
}

template <int ODT>
__device__ inline void store_out(void* out, int64_t off, float v) {
  if constexpr (ODT == LSRM_F32)
    reinterpret_cast<float*>(out)[off] = v;
  else
    reinterpret_cast<uint16_t*>(out)[off] = from_f32<ODT>(v);
}

template <int ODT, int VEC>
__global__ __launch_bounds__(256) void pool_combine(
    const float* __restrict__ partial, int64_t n, int64_t ch,
    const int32_t* __restrict__ cu, int64_t nb, void* __restrict__ out) {
  const int64_t n_vec = ch / VEC;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= nb * n_vec) return;
  const int64_t b = item / n_vec;
  const int64_t c0 = (item - b * n_vec) * VEC;
  int64_t s = cu[b], e = cu[b + 1];
  s = s < 0 ? 0 : (s > n ? n : s);
  e = e < 0 ? 0 : (e > n ? n : e);
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;
  if (e > s) {
    const int64_t j0 = s / POOL_CHUNK, j1 = (e - 1) / POOL_CHUNK;
    // Up to PB pieces are loaded before any is added (one memory round trip
    // per PB pieces); the adds stay in chunk order.
    constexpr int PB = VEC == 1 ? 16 : 8;
    for (int64_t jb = j0; jb <= j1; jb += PB) {
      float v[PB][VEC];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int64_t j = jb + u <= j1 ? jb + u : j1;
        const float* src = partial + (b + j) * ch + c0;
        if constexpr (VEC == 4) {
          const float4 lo = reinterpret_cast<const float4*>(src)[0];
          v[u][0] = lo.x; v[u][1] = lo.y; v[u][2] = lo.z; v[u][3] = lo.w;
        } else {
          v[u][0] = src[0];
        }
      }
#pragma unroll
      for (int u = 0; u < PB; ++u)
        if (jb + u <= j1) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = acc[i] + v[u][i];
        }
    }
  }
  // IEEE quotient; a block with no rows gives 0/0 = NaN.
  const float len = e > s ? (float)(e - s) : 0.0f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) store_out<ODT>(out, b * ch + c0 + i, acc[i] / len);
}

// Both tensors' combines in one launch: items [0, nb * n_vec) of tensor a,
// then those of tensor b (output types ODTA, ODTB).
template <int ODTA, int ODTB>
__global__ __launch_bounds__(256) void pool_combine2(
    const float* __restrict__ partial_a, const float* __restrict__ partial_b, int64_t n,
    int64_t ch, const int32_t* __restrict__ cu, int64_t nb, void* __restrict__ out_a,
    void* __restrict__ out_b) {
  constexpr int VEC = 4;
  const int64_t n_vec = ch / VEC;
  int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= 2 * nb * n_vec) return;
  const bool second = item >= nb * n_vec;
  if (second) item -= nb * n_vec;
  const float* partial = second ? partial_b : partial_a;
  const int64_t b = item / n_vec;
  const int64_t c0 = (item - b * n_vec) * VEC;
  int64_t s = cu[b], e = cu[b + 1];
  s = s < 0 ? 0 : (s > n ? n : s);
  e = e < 0 ? 0 : (e > n ? n : e);
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.0f;
  if (e > s) {
    const int64_t j0 = s / POOL_CHUNK, j1 = (e - 1) / POOL_CHUNK;
    constexpr int PB = 8;
    for (int64_t jb = j0; jb <= j1; jb += PB) {
      float v[PB][VEC];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int64_t j = jb + u <= j1 ? jb + u : j1;
        const float* src = partial + (b + j) * ch + c0;
        const float4 lo = reinterpret_cast<const float4*>(src)[0];
        v[u][0] = lo.x; v[u][1] = lo.y; v[u][2] = lo.z; v[u][3] = lo.w;
      }
#pragma unroll
      for (int u = 0; u < PB; ++u)
        if (jb + u <= j1) {
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = acc[i] + v[u][i];
        }
    }
  }
  const float len = e > s ? (float)(e - s) : 0.0f;
  if (second) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) store_out<ODTB>(out_b, b * ch + c0 + i, acc[i] / len);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) store_out<ODTA>(out_a, b * ch + c0 + i, acc[i] / len);
  }
}

// 16-bit rows of 256 channels: the slab kernel with two chunks per wave
// (false for fp32 rows, which take pool_pieces).
template <int DT>
bool launch_half_chunks(const void* x, int64_t n, int64_t ch, const int32_t* cu, int64_t nb,
                        const int32_t* first, float* partial, dim3 grid, hipStream_t st) {
  if constexpr (DT == LSRM_F32) {
    return false;
  } else {
    if (nb + 1 <= POOL_IF2_MAX)
      hipLaunchKernelGGL((pool_pieces_half<DT, true>), grid, dim3(256), 0, st,
                         reinterpret_cast<const uint16_t*>(x), n, ch, cu, nb, first, partial);
    else
      hipLaunchKernelGGL((pool_pieces_half<DT, false>), grid, dim3(256), 0, st,
                         reinterpret_cast<const uint16_t*>(x), n, ch, cu, nb, first, partial);
    return true;
  }
}

int64_t pool_partial_rows(int64_t n, int64_t nb) {
  return nb + (n + POOL_CHUNK - 1) / POOL_CHUNK;
}

// Entries of the chunk -> first-block table.
int64_t pool_first_count(int64_t n) { return (n + POOL_CHUNK - 1) / POOL_CHUNK; }

// Launches the pooling kernels; partial needs pool_partial_rows * ch floats
// and first pool_first_count ints.
int launch_block_mean_pool(const void* x, int x_dtype, int64_t n, int64_t ch,
                           const int32_t* cu, int64_t nb, void* out,
                           int out_dtype, float* partial, int32_t* first,
                           hipStream_t st) {
  if (nb == 0) return LSRM_OK;
  const bool vec = (ch % POOL_VEC) == 0 && ((uintptr_t)x % 16) == 0 &&
                   ((uintptr_t)partial % 16) == 0;
  const int64_t n_vec = vec ? ch / POOL_VEC : ch;
  const int64_t n_chunks = (n + POOL_CHUNK - 1) / POOL_CHUNK;
  const bool slab = vec && x_dtype != LSRM_F32 && n_vec % 64 == 0 &&
                   n_chunks * n_vec < (int64_t{1} << 31);
  const bool inline_first = slab && nb + 1 <= 512;
  if (n > 0 && slab) {
    if (!inline_first)
      hipLaunchKernelGGL(pool_chunk_first, dim3((unsigned)((n_chunks + 255) / 256)),
                         dim3(256), 0, st, cu, nb, n_chunks, first);
    const uint16_t* xs = reinterpret_cast<const uint16_t*>(x);
    if (x_dtype == LSRM_F16)
      launch_pieces16<LSRM_F16, 1>(xs, nullptr, n, ch, cu, nb, first, partial, nullptr,
                                   inline_first, st);
    else
      launch_pieces16<LSRM_BF16, 1>(xs, nullptr, n, ch, cu, nb, first, partial, nullptr,
                                    inline_first, st);
    LSRM_CHECK_LAUNCH();
  } else if (n > 0) {
    // the 256-channel 16-bit kernel finds the blocks itself up to POOL_IF2_MAX
    const bool half_inline = vec && n_vec == 32 && x_dtype != LSRM_F32 &&
                             n_chunks * n_vec < (int64_t{1} << 31) && nb + 1 <= POOL_IF2_MAX;
    if (!half_inline)
      hipLaunchKernelGGL(pool_chunk_first, dim3((unsigned)((n_chunks + 255) / 256)),
                         dim3(256), 0, st, cu, nb, n_chunks, first);
    const int64_t items = n_chunks * n_vec;
    dim3 grid((unsigned)((items + 255) / 256));
#define LSRM_POOL_P(DT)                                                      \
  do {                                                                       \
    if (vec && n_vec == 32 && n_chunks * n_vec < (int64_t{1} << 31) &&      \
        launch_half_chunks<DT>(x, n, ch, cu, nb, first, partial, grid, st))  \
      ;                                                                      \
    else if (vec && n_vec % 64 == 0)                                         \
      hipLaunchKernelGGL((pool_pieces<DT, 8, true>), grid, dim3(256), 0, st, \
                         x, n, ch, cu, nb, first, partial);                  \
    else if (vec)                                                            \
      hipLaunchKernelGGL((pool_pieces<DT, 8, false>), grid, dim3(256), 0,    \
                         st, x, n, ch, cu, nb, first, partial);              \
    else                                                                     \
      hipLaunchKernelGGL((pool_pieces<DT, 1, false>), grid, dim3(256), 0,    \
                         st, x, n, ch, cu, nb, first, partial);              \
  } while (0)
    switch (x_dtype) {
      case LSRM_F32: LSRM_POOL_P(LSRM_F32); break;
      case LSRM_F16: LSRM_POOL_P(LSRM_F16); break;
      case LSRM_BF16: LSRM_POOL_P(LSRM_BF16); break;
      default: return LSRM_ERR_UNSUPPORTED;
    }
#undef LSRM_POOL_P
    LSRM_CHECK_LAUNCH();
  }
  {
    // 4 channels per thread on the vector path (twice the threads of the
    // piece kernel's 8: more loads in flight for the few blocks).
    const int64_t items = vec ? nb * (ch / 4) : nb * ch;
    dim3 grid((unsigned)((items + 255) / 256));
#define LSRM_POOL_C(ODT)                                                     \
  do {                                                                       \
    if (vec)                                                                 \
      hipLaunchKernelGGL((pool_combine<ODT, 4>), grid, dim3(256), 0, st,     \
                         partial, n, ch, cu, nb, out);                       \
    else                                                                     \
      hipLaunchKernelGGL((pool_combine<ODT, 1>), grid, dim3(256), 0, st,     \
                         partial, n, ch, cu, nb, out);                       \
  } while (0)
    switch (out_dtype) {
      case LSRM_F32: LSRM_POOL_C(LSRM_F32); break;
      case LSRM_F16: LSRM_POOL_C(LSRM_F16); break;
      case LSRM_BF16: LSRM_POOL_C(LSRM_BF16); break;
      default: return LSRM_ERR_UNSUPPORTED;
    }
#undef LSRM_POOL_C
    LSRM_CHECK_LAUNCH();
  }
  return LSRM_OK;
}

// Two tensors of one shape and block partition: one piece launch and one
// combine launch for both when the slab path applies, otherwise the
// single-tensor launches one after the other (identical results).
int launch_block_mean_pool2(const void* xa, const void* xb, int x_dtype, int64_t n, int64_t ch,
                            const int32_t* cu, int64_t nb, void* out_a, int out_a_dtype,
                            void* out_b, int out_b_dtype, float* partial_a, float* partial_b,
                            int32_t* first, hipStream_t st) {
  if (nb == 0) return LSRM_OK;
  const bool slab = (ch % POOL_VEC) == 0 && x_dtype != LSRM_F32 && (ch / POOL_VEC) % 64 == 0 &&
                    ((uintptr_t)xa % 16) == 0 && ((uintptr_t)xb % 16) == 0 &&
                    ((uintptr_t)partial_a % 16) == 0 && ((uintptr_t)partial_b % 16) == 0 &&
                    2 * ((n + POOL_CHUNK - 1) / POOL_CHUNK) * (ch / POOL_VEC) < (int64_t{1} << 31);
  if (!slab || n == 0) {
    int rc = launch_block_mean_pool(xa, x_dtype, n, ch, cu, nb, out_a, out_a_dtype, partial_a,
                                    first, st);
    if (rc) return rc;
    return launch_block_mean_pool(xb, x_dtype, n, ch, cu, nb, out_b, out_b_dtype, partial_b,
                                  first, st);
  }
  const int64_t n_vec = ch / POOL_VEC;
  const int64_t n_chunks = (n + POOL_CHUNK - 1) / POOL_CHUNK;
  const bool inline_first = nb + 1 <= 512;
  if (!inline_first)
    hipLaunchKernelGGL(pool_chunk_first, dim3((unsigned)((n_chunks + 255) / 256)), dim3(256), 0,
                       st, cu, nb, n_chunks, first);
  {
    const uint16_t* a = reinterpret_cast<const uint16_t*>(xa);
    const uint16_t* b = reinterpret_cast<const uint16_t*>(xb);
    if (x_dtype == LSRM_F16)
      launch_pieces16<LSRM_F16, 2>(a, b, n, ch, cu, nb, first, partial_a, partial_b,
                                   inline_first, st);
    else
      launch_pieces16<LSRM_BF16, 2>(a, b, n, ch, cu, nb, first, partial_a, partial_b,
                                    inline_first, st);
    LSRM_CHECK_LAUNCH();
  }
  {
    const int64_t items = 2 * nb * (ch / 4);
    dim3 grid((unsigned)((items + 255) / 256));
#define LSRM_POOL2_C(A, B)                                                                  \
  hipLaunchKernelGGL((pool_combine2<A, B>), grid, dim3(256), 0, st, partial_a, partial_b, n, \
                     ch, cu, nb, out_a, out_b)
#define LSRM_POOL2_CB(A)                                          \
  switch (out_b_dtype) {                                          \
    case LSRM_F32: LSRM_POOL2_C(A, LSRM_F32); break;              \
    case LSRM_F16: LSRM_POOL2_C(A, LSRM_F16); break;              \
    default: LSRM_POOL2_C(A, LSRM_BF16); break;                   \
  }
    switch (out_a_dtype) {
      case LSRM_F32: LSRM_POOL2_CB(LSRM_F32) break;
      case LSRM_F16: LSRM_POOL2_CB(LSRM_F16) break;
      default: LSRM_POOL2_CB(LSRM_BF16) break;
    }
#undef LSRM_POOL2_CB
#undef LSRM_POOL2_C
    LSRM_CHECK_LAUNCH();
  }
  return LSRM_OK;
}

}  // namespace lsrm

// Scratch of lsrm_block_mean_pool_noalloc: the piece partials and the
// chunk -> first-block table, laid out as in a caller's workspace.  Every
// GPU holds its own copy; host code reaches it only through the per-device
// address from hipGetSymbolAddress (the array's name on the host is not a
// device address).  Nothing in it needs to start at zero: every partial and
// table entry a launch reads was written earlier in the same launch.
static __device__ __align__(256) char scratch[LSRM_POOL_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {nullptr};

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
int scratch_address(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LSRM_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p)
      return LSRM_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return LSRM_OK;
}

}  // namespace

extern "C" size_t lsrm_block_mean_pool_workspace_size(int64_t n_tokens,
                                                      int64_t channels,
                                                      int64_t n_blocks) {
  if (n_tokens < 0 || channels < 0 || n_blocks < 0) return 0;
  return (size_t)lsrm::pool_partial_rows(n_tokens, n_blocks) *
             (size_t)channels * sizeof(float) +
         256 + (size_t)lsrm::pool_first_count(n_tokens) * 4 + 256;
}

extern "C" int lsrm_block_mean_pool(const void* x, int x_dtype,
                                    int64_t n_tokens, int64_t channels,
                                    const int32_t* cu_block_tokens,
                                    int64_t n_blocks, void* out, int out_dtype,
                                    void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (n_tokens < 0 || channels <= 0 || n_blocks < 0) return LSRM_ERR_INVALID_ARG;
  if (n_blocks > 0 && (!cu_block_tokens || !out)) return LSRM_ERR_INVALID_ARG;
  if (n_tokens > 0 && !x) return LSRM_ERR_INVALID_ARG;
  if (x_dtype < LSRM_F32 || x_dtype > LSRM_BF16) return LSRM_ERR_UNSUPPORTED;
  if (out_dtype < LSRM_F32 || out_dtype > LSRM_BF16) return LSRM_ERR_UNSUPPORTED;
  const size_t need =
      lsrm_block_mean_pool_workspace_size(n_tokens, channels, n_blocks);
  if (workspace_bytes < need || (need > 256 && !workspace)) return LSRM_ERR_WORKSPACE;
  float* partial = reinterpret_cast<float*>(lsrm::align_up((size_t)workspace, 256));
  int32_t* first = reinterpret_cast<int32_t*>(lsrm::align_up(
      (size_t)(partial + lsrm::pool_partial_rows(n_tokens, n_blocks) * channels), 256));
  return lsrm::launch_block_mean_pool(x, x_dtype, n_tokens, channels,
                                      cu_block_tokens, n_blocks, out, out_dtype,
                                      partial, first, (hipStream_t)stream);
}

extern "C" int lsrm_block_mean_pool_noalloc(const void* x, int x_dtype, int64_t n_tokens,
                                            int64_t channels,
                                            const int32_t* cu_block_tokens,
                                            int64_t n_blocks, void* out, int out_dtype,
                                            void* stream) {
  if (n_tokens < 0 || channels <= 0 || n_blocks < 0) return LSRM_ERR_INVALID_ARG;
  if (lsrm_block_mean_pool_workspace_size(n_tokens, channels, n_blocks) >
      LSRM_POOL_SCRATCH_BYTES)
    return LSRM_ERR_SCRATCH;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return lsrm_block_mean_pool(x, x_dtype, n_tokens, channels, cu_block_tokens, n_blocks, out,
                              out_dtype, ws, LSRM_POOL_SCRATCH_BYTES, stream);
}

extern "C" size_t lsrm_block_mean_pool2_workspace_size(int64_t n_tokens, int64_t channels,
                                                       int64_t n_blocks) {
  if (n_tokens < 0 || channels < 0 || n_blocks < 0) return 0;
  return 2 * ((size_t)lsrm::pool_partial_rows(n_tokens, n_blocks) * (size_t)channels *
              sizeof(float) + 256) +
         (size_t)lsrm::pool_first_count(n_tokens) * 4 + 256;
}

extern "C" int lsrm_block_mean_pool2(const void* x_a, const void* x_b, int x_dtype,
                                     int64_t n_tokens, int64_t channels,
                                     const int32_t* cu_block_tokens, int64_t n_blocks,
                                     void* out_a, int out_a_dtype, void* out_b, int out_b_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (n_tokens < 0 || channels <= 0 || n_blocks < 0) return LSRM_ERR_INVALID_ARG;
  if (n_blocks > 0 && (!cu_block_tokens || !out_a || !out_b)) return LSRM_ERR_INVALID_ARG;
  if (n_tokens > 0 && (!x_a || !x_b)) return LSRM_ERR_INVALID_ARG;
  if (x_dtype < LSRM_F32 || x_dtype > LSRM_BF16) return LSRM_ERR_UNSUPPORTED;
  if (out_a_dtype < LSRM_F32 || out_a_dtype > LSRM_BF16 || out_b_dtype < LSRM_F32 ||
      out_b_dtype > LSRM_BF16)
    return LSRM_ERR_UNSUPPORTED;
  const size_t need = lsrm_block_mean_pool2_workspace_size(n_tokens, channels, n_blocks);
  if (workspace_bytes < need || !workspace) return LSRM_ERR_WORKSPACE;
  const size_t part = (size_t)lsrm::pool_partial_rows(n_tokens, n_blocks) * (size_t)channels;
  float* partial_a = reinterpret_cast<float*>(lsrm::align_up((size_t)workspace, 256));
  float* partial_b = reinterpret_cast<float*>(lsrm::align_up((size_t)(partial_a + part), 256));
  int32_t* first =
      reinterpret_cast<int32_t*>(lsrm::align_up((size_t)(partial_b + part), 256));
  return lsrm::launch_block_mean_pool2(x_a, x_b, x_dtype, n_tokens, channels, cu_block_tokens,
                                       n_blocks, out_a, out_a_dtype, out_b, out_b_dtype,
                                       partial_a, partial_b, first, (hipStream_t)stream);
}
