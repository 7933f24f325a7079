// Learned block selection (get_block_score,
// sparse/ops/block_score.py:16-98) on gfx950.
//
// For query token i of batch element b, kv head h and compressed key c of b:
//   score(i, c) = sum over the G query heads g of h of
//                 exp2(q[i, hG+g] . ck[c, h] * qk_scale - lse[hG+g, i] * 1.44269504)
// (qk_scale = sm_scale * 1.44269504, the reference's constants, lines 53-56);
// the min(topk, n_compressed) best compressed keys (score descending, id
// ascending among equal scores; NaN scores are never chosen) are written
// ascending, the row padded with -1 (lines 61-63, 94-96).
//
// One wave per (kv head, 32-token tile).  S^T = Ck Q^T on 32x32x16 MFMA:
// the compressed keys (A operand, 16 contiguous bytes per lane) come
// straight from global memory, two 32-key blocks ahead of their use; a lane
// owns one query row and 16 of every 32 keys.  Each lane keeps a top-K list
// (K >= topk, a power of two) of its candidates in registers, sorted by
// (score desc, id asc) as 64-bit rank keys; with many keys per list entry a
// first pass bounds the row's K-th score from below and the second keeps
// only keys above the bound (in an LDS buffer, merged 16 at a time).  At the
// end the two lanes of a row merge their lists with a bitonic network and
// the chosen ids are sorted ascending.  Tiles that straddle a batch boundary
// are processed once per batch element they touch; rows of tokens outside
// every element are written as -1 rows.
//
// topk in (64, 128]: two launches of the 64-entry selection.  The first
// writes the row's best k1 = min(64, topk - 2) ids (ascending) and, in slots
// k1 and k1 + 1, its k1-th best (score bits, id) as a bound; the second
// keeps only keys that rank after the bound, selects the best topk - k1 of
// them and merges both ascending lists into the row (every id of one list
// differs from every id of the other, so a rank count places each).
#include "common.h"

namespace lsrm {

constexpr float LOG2E_REF = 1.44269504f;  // sparse/ops/block_score.py:53-56

struct BlockScoreArgs {
  const uint16_t* q;
  const uint16_t* ck;
  const float* lse;
  const int32_t* cu_q;
  const int32_t* cu_c;
  int32_t* out;
  int64_t nq, batch;
  int hq, hkv, g, topk;
  int kout;  // ids this launch selects per row (topk, or k1 / topk - k1)
  int k1;    // two-pass selection: ids of the first pass
  float qk_scale;
};

// Launch roles: the whole selection, or the two passes for topk > 64.
constexpr int BS_ONE = 0, BS_FIRST = 1, BS_SECOND = 2;

// (v, i) ranks before (w, j): larger score, equal scores by lower id.
__device__ inline bool ranks_before(float v, int i, float w, int j) {
  return v > w || (v == w && i < j);
}

// Rank key of a score >= 0 (its bits order as unsigned integers) and an id
// in [0, 2^31): a larger key ranks before, equal scores by lower id; every
// key is nonzero, so 0 marks an empty entry.
__device__ inline uint64_t rank_key(float v, int id) {
  return ((uint64_t)__float_as_uint(v) << 32) | (0x80000000u | (uint32_t)(0x7fffffff - id));
}

// Compare-exchange of two rank keys: x gets the larger when desc, else y.
__device__ inline void key_swap(uint64_t& x, uint64_t& y, bool desc) {
  const uint64_t hi = x > y ? x : y, lo = x > y ? y : x;
  x = desc ? hi : lo;
  y = desc ? lo : hi;
}

// Capacity (entries per lane) of the LDS buffer of the two-pass selection.
constexpr int BS_CAP = 32;

template <int DT, int D, int K, int MODE>
__global__ __launch_bounds__(256) void block_score_kernel(BlockScoreArgs a) {
  static_assert(MODE == BS_ONE || K == 64, "the two-pass roles use the 64-entry lists");
  constexpr int NS = D / 16;
  const int lane = threadIdx.x & 63, hb = lane >> 5, l32 = lane & 31;
  const int64_t tiles = (a.nq + 31) / 32;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wave >= tiles * a.hkv) return;
  const int h = __builtin_amdgcn_readfirstlane((int)(wave / tiles));
  const int64_t t0 = (wave - (int64_t)h * tiles) * 32;
  const int64_t t_last = t0 + 31 < a.nq ? t0 + 31 : a.nq - 1;
  const int b0 = (int)upper_index(a.cu_q, 0, a.batch + 1, t0);
  const int b1 = (int)upper_index(a.cu_q, 0, a.batch + 1, t_last);
  const int64_t row = t0 + l32;
  const int64_t ck_stride = (int64_t)a.hkv * D;

  // Every row of the output is written here: tokens outside every batch
  // element get -1 rows, the loop below the rest.
  if (hb == 0 && row < a.nq && (row < a.cu_q[0] || row >= a.cu_q[a.batch])) {
    int32_t* dst = a.out + ((int64_t)h * a.nq + row) * a.topk;
    for (int i = 0; i < a.topk; ++i) dst[i] = -1;
  }
  for (int b = b0 < 0 ? 0 : b0; b <= b1 && b < a.batch; ++b) {
    const int64_t qs = a.cu_q[b], qe = a.cu_q[b + 1];
    if (qe <= t0 || qs > t_last) continue;
    const bool row_ok = row >= qs && row < qe && row < a.nq;
    const int64_t ks = a.cu_c[b];
    const int64_t nc = (int64_t)a.cu_c[b + 1] - ks;
    const int kk = nc <= 0 ? 0 : (nc < a.kout ? (int)nc : a.kout);
    // second pass: only keys ranking after the first pass's 64th best
    float bnd_v = -2.0f;
    int bnd_i = -1;
    if constexpr (MODE == BS_SECOND) {
      if (row_ok) {
        const int32_t* src = a.out + ((int64_t)h * a.nq + row) * a.topk;
        bnd_v = __int_as_float(src[a.k1]);
        bnd_i = src[a.k1 + 1];
      }
    }

    float tv[K];
    int ti[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
      tv[i] = -1.0f;  // below every score (scores are >= 0)
      ti[i] = -1;
    }
    uint64_t tk[K];  // list as rank keys (K <= 32), 0 = empty
#pragma unroll
    for (int i = 0; i < K; ++i) tk[i] = 0ull;
    uint64_t mk_out[K];  // the row's merged list as rank keys (K <= 32)
    int mi[K];           // the row's best ids, best first (-1 = none)
    // Inserts (v, id) into the descending list; ids arrive ascending, so an
    // equal score already listed keeps its place.
    auto insert = [&](float v, int id) __attribute__((always_inline)) {
      if (v > tv[K - 1]) {
#pragma unroll
        for (int i = K - 1; i >= 0; --i) {
          const bool prev_less = i > 0 ? (tv[i > 0 ? i - 1 : 0] < v) : false;
          if (tv[i] < v) {
            tv[i] = prev_less ? tv[i > 0 ? i - 1 : 0] : v;
            ti[i] = prev_less ? ti[i > 0 ? i - 1 : 0] : id;
          }
        }
      }
    };

    const uint16_t* ckh = a.ck + ks * ck_stride + (int64_t)h * D + hb * 8;
    auto load_k = [&](int64_t c0, u32x4* ka) __attribute__((always_inline)) {
      const int64_t key = c0 + l32;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        ka[s] = key < nc ? *reinterpret_cast<const u32x4*>(ckh + key * ck_stride + s * 16)
                         : u32x4{0u, 0u, 0u, 0u};
    };
    // The row's query fragment and log2-scaled lse of query head g of this
    // kv head: loaded once when the group has one head, else one head ahead
    // of its use, so no block waits on a query load.
    auto load_q = [&](int g, u32x4* qb, float& l2) __attribute__((always_inline)) {
      const int hh = h * a.g + g;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        qb[s] = row_ok ? *reinterpret_cast<const u32x4*>(
                             a.q + (row * a.hq + hh) * D + s * 16 + hb * 8)
                       : u32x4{0u, 0u, 0u, 0u};
      l2 = row_ok ? a.lse[(int64_t)hh * a.nq + row] * LOG2E_REF : 0.0f;
    };
    u32x4 qcur[NS];
    float l2cur;
    load_q(0, qcur, l2cur);
    // p[v] = score of key c0 + acc_row(v, hb) for this lane's row: the sum
    // over the group's query heads of exp2(s * scale - lse * log2e).
    auto block_scores = [&](const u32x4* ka, float* p) __attribute__((always_inline)) {
#pragma unroll
      for (int v = 0; v < 16; ++v) p[v] = 0.0f;
      for (int g = 0; g < a.g; ++g) {
        u32x4 qn[NS];
        float l2n = 0.0f;
        if (a.g > 1) load_q(g + 1 < a.g ? g + 1 : 0, qn, l2n);
        f32x16 sacc;
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[v] = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) sacc = mfma32<DT>(ka[s], qcur[s], sacc);
#pragma unroll
        for (int v = 0; v < 16; ++v)
          p[v] += __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], a.qk_scale, -l2cur));
        if (a.g > 1) {
#pragma unroll
          for (int s = 0; s < NS; ++s) qcur[s] = qn[s];
          l2cur = l2n;
        }
      }
    };
    // Runs body(c0, p) over the element's 32-key blocks in order, two blocks
    // a step, with the next two blocks' compressed keys loading while the
    // current two are scored.
    auto for_blocks = [&](auto&& body) __attribute__((always_inline)) {
      u32x4 kc[2][NS], kn[2][NS];
      if (nc > 0) {
        load_k(0, kc[0]);
        load_k(32, kc[1]);
      }
      for (int64_t c0 = 0; c0 < nc; c0 += 64) {
        if (c0 + 64 < nc) {
          load_k(c0 + 64, kn[0]);
          load_k(c0 + 96, kn[1]);
        }
        float p[16];
        block_scores(kc[0], p);
        body(c0, p);
        if (c0 + 32 < nc) {
          block_scores(kc[1], p);
          body(c0 + 32, p);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          kc[0][s] = kn[0][s];
          kc[1][s] = kn[1][s];
        }
      }
    };

    if constexpr (K <= 32) {
      // Merges 16 candidate rank keys (0 = none) into the list: a bitonic
      // sort of the candidates, then the larger of list[i] and
      // candidate[K-1-i], a bitonic sequence holding the best K of both, is
      // sorted by a bitonic merge.
      auto merge16 = [&](uint64_t* ck) __attribute__((always_inline)) {
#pragma unroll
        for (int size = 2; size <= 16; size <<= 1)
#pragma unroll
          for (int j = size / 2; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int o = i ^ j;
              if (o > i) key_swap(ck[i], ck[o], (i & size) == 0);
            }
#pragma unroll
        for (int i = 0; i < K; ++i) {
          const uint64_t bk = K - 1 - i < 16 ? ck[K - 1 - i < 16 ? K - 1 - i : 0] : 0ull;
          tk[i] = tk[i] > bk ? tk[i] : bk;
        }
#pragma unroll
        for (int j = K / 2; j > 0; j >>= 1)
#pragma unroll
          for (int i = 0; i < K; ++i)
            if ((i & j) == 0) key_swap(tk[i], tk[i | j], true);
      };
      // Two passes when the element has many keys per list entry: the first
      // bounds the row's K-th best score from below by the K-th best of the
      // per-lane block maxima (each is a distinct key of the row), the second
      // keeps only keys at or above that bound, appending them to this lane's
      // LDS buffer, merged 16 at a time.  One pass otherwise: every block's
      // candidates merged as they come.
      __shared__ float2 s_buf[4][BS_CAP + 1][64];  // [wave][slot][lane]; slot BS_CAP: discard
      float2(*buf)[64] = s_buf[threadIdx.x >> 6];
      if (a.g <= 4 && nc >= 8 * K) {
        float mk[K];  // descending K best block maxima of this lane
#pragma unroll
        for (int i = 0; i < K; ++i) mk[i] = -1.0f;
        for_blocks([&](int64_t c0, const float* p) __attribute__((always_inline)) {
          // (fmax ignores a NaN score)
          const int lim = row_ok ? (int)(nc - c0) : 0;
          float bm = -1.0f;
#pragma unroll
          for (int v = 0; v < 16; ++v)
            bm = __builtin_fmaxf(bm, acc_row(v, hb) < lim ? p[v] : -1.0f);
          // insertion into the descending list: entry i becomes bm clamped
          // to [mk[i], mk[i-1]]
          if (__builtin_amdgcn_ballot_w64(bm > mk[K - 1]) != 0) {
#pragma unroll
            for (int i = K - 1; i > 0; --i) mk[i] = __builtin_amdgcn_fmed3f(mk[i], bm, mk[i - 1]);
            mk[0] = __builtin_fmaxf(mk[0], bm);
          }
        });
        float t = __builtin_inff();
#pragma unroll
        for (int i = 0; i < K; ++i) {
          const float pm = __shfl_xor(mk[K - 1 - i], 32);
          t = __builtin_fminf(t, __builtin_fmaxf(mk[i], pm));
        }
        // a little below the bound, so a rounding difference between the
        // passes can never drop a key
        const float tb = t > 0.0f && t < __builtin_inff() ? t * (1.0f - 0x1p-16f) : t;

        int cnt = 0;
        auto flush = [&]() __attribute__((always_inline)) {
          for (int base = 0; __builtin_amdgcn_ballot_w64(base < cnt) != 0; base += 16) {
            uint64_t ck[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int slot = base + i < BS_CAP ? base + i : BS_CAP;
              const float2 e = buf[slot][lane];
              ck[i] = base + i < cnt ? rank_key(e.x, __float_as_int(e.y)) : 0ull;
            }
            merge16(ck);
          }
          cnt = 0;
        };
        for_blocks([&](int64_t c0, const float* p) __attribute__((always_inline)) {
          if (__builtin_amdgcn_ballot_w64(cnt > BS_CAP - 16) != 0) flush();
          const int lim = row_ok ? (int)(nc - c0) : 0;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            // (a NaN score fails the comparison, so is never chosen)
            const bool ok = (acc_row(v, hb) < lim) & (p[v] >= tb);
            buf[ok ? cnt : BS_CAP][lane] = float2{p[v], __int_as_float((int)c0 + acc_row(v, hb))};
            cnt += ok ? 1 : 0;
          }
        });
        flush();
      } else {
        for_blocks([&](int64_t c0, const float* p) __attribute__((always_inline)) {
          // candidates that would enter the list; the merge is skipped when
          // no lane has one
          uint64_t ck[16];
          uint64_t best = 0ull;
          const int lim = (int)(nc - c0);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            // NaN scores are never chosen
            const bool ok = (acc_row(v, hb) < lim) & (p[v] == p[v]);
            ck[v] = ok ? rank_key(p[v], (int)c0 + acc_row(v, hb)) : 0ull;
            best = best > ck[v] ? best : ck[v];
          }
          const bool enter = best > tk[K - 1];
          if (__builtin_amdgcn_ballot_w64(enter) != 0) merge16(ck);
        });
      }
      // Merge with the partner lane's list (same row, the other 16 keys of
      // every block): the larger of own[i] and partner[K-1-i] is a bitonic
      // sequence holding the row's best K, sorted by a bitonic merge.
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const uint64_t x = tk[K - 1 - i];
        const uint32_t plo = (uint32_t)__shfl_xor((int)(uint32_t)x, 32);
        const uint32_t phi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), 32);
        const uint64_t pk = ((uint64_t)phi << 32) | plo;
        mk_out[i] = tk[i] > pk ? tk[i] : pk;
      }
#pragma unroll
      for (int j = K / 2; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < K; ++i)
          if ((i & j) == 0) key_swap(mk_out[i], mk_out[i | j], true);
#pragma unroll
      for (int i = 0; i < K; ++i)
        mi[i] = mk_out[i] != 0ull ? 0x7fffffff - (int)((uint32_t)mk_out[i] & 0x7fffffffu) : -1;
    } else {
      for_blocks([&](int64_t c0, const float* p) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t key = c0 + acc_row(v, hb);
          if constexpr (MODE == BS_SECOND) {
            if (key < nc && ranks_before(bnd_v, bnd_i, p[v], (int)key)) insert(p[v], (int)key);
          } else {
            if (key < nc) insert(p[v], (int)key);
          }
        }
      });
    }

    float mv[K];  // the row's merged scores, best first (K > 32)
    if constexpr (K > 32) {
      // Merge with the partner lane's list (same row, the other 16 keys of
      // every block): the better of (own[i], partner[K-1-i]) is a bitonic
      // sequence holding the row's best K, sorted by a bitonic merge.
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const float pv = __shfl_xor(tv[K - 1 - i], 32);
        const int pi = __shfl_xor(ti[K - 1 - i], 32);
        const bool own = ti[i] >= 0 && (pi < 0 || ranks_before(tv[i], ti[i], pv, pi));
        mv[i] = own ? tv[i] : pv;
        mi[i] = own ? ti[i] : pi;
      }
#pragma unroll
      for (int j = K / 2; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
          if ((i & j) == 0) {
            const int o = i | j;
            const bool keep = mi[i] >= 0 && (mi[o] < 0 || ranks_before(mv[i], mi[i], mv[o], mi[o]));
            const float v0 = keep ? mv[i] : mv[o], v1 = keep ? mv[o] : mv[i];
            const int i0 = keep ? mi[i] : mi[o], i1 = keep ? mi[o] : mi[i];
            mv[i] = v0; mv[o] = v1; mi[i] = i0; mi[o] = i1;
          }
        }
      }
    }
    // The best kk ids, sorted ascending (bitonic sort; unused slots last).
    int ids[K];
#pragma unroll
    for (int i = 0; i < K; ++i) ids[i] = (i < kk && mi[i] >= 0) ? mi[i] : 0x7fffffff;
#pragma unroll
    for (int size = 2; size <= K; size <<= 1) {
#pragma unroll
      for (int j = size / 2; j > 0; j >>= 1) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
          const int o = i ^ j;
          if (o > i) {
            const bool up = (i & size) == 0;
            const int lo = ids[i] < ids[o] ? ids[i] : ids[o];
            const int hi = ids[i] < ids[o] ? ids[o] : ids[i];
            ids[i] = up ? lo : hi;
            ids[o] = up ? hi : lo;
          }
        }
      }
    }
    if (row_ok && hb == 0) {
      int32_t* dst = a.out + ((int64_t)h * a.nq + row) * a.topk;
      if constexpr (MODE == BS_ONE) {
#pragma unroll
        for (int i = 0; i < K; ++i)
          if (i < a.topk) dst[i] = (i < kk && ids[i] != 0x7fffffff) ? ids[i] : -1;
      } else if constexpr (MODE == BS_FIRST) {
#pragma unroll
        for (int i = 0; i < K; ++i)
          if (i < a.k1) dst[i] = (i < kk && ids[i] != 0x7fffffff) ? ids[i] : -1;
        // bound: the k1-th best when the row has k1 chosen keys, else a value
        // nothing ranks after
        float bv = -2.0f;
        int bi = -1;
#pragma unroll
        for (int i = 0; i < K; ++i)
          if (i == a.k1 - 1 && kk == a.k1 && mi[i] >= 0) {
            bv = mv[i];
            bi = mi[i];
          }
        dst[a.k1] = __float_as_int(bv);
        dst[a.k1 + 1] = bi;
      } else {
        // merge with the first pass's k1 ascending ids (0x7fffffff = none)
        int first[K];
#pragma unroll
        for (int i = 0; i < K; ++i) {
          const int x = i < a.k1 ? dst[i] : -1;
          first[i] = x >= 0 ? x : 0x7fffffff;
        }
        int n1 = 0, n2 = 0;
#pragma unroll
        for (int i = 0; i < K; ++i) {
          n1 += first[i] != 0x7fffffff ? 1 : 0;
          n2 += (i < kk && ids[i] != 0x7fffffff) ? 1 : 0;
        }
#pragma unroll
        for (int i = 0; i < K; ++i) {
          int r1 = i, r2 = i;  // output slots: own index + ids of the other list below
#pragma unroll
          for (int j = 0; j < K; ++j) {
            const int y = (j < kk) ? ids[j] : 0x7fffffff;
            r1 += y < first[i] ? 1 : 0;
            r2 += first[j] < ids[i] ? 1 : 0;
          }
          if (first[i] != 0x7fffffff) dst[r1] = first[i];
          if (i < kk && ids[i] != 0x7fffffff) dst[r2] = ids[i];
        }
        for (int i = n1 + n2; i < a.topk; ++i) dst[i] = -1;
      }
    }
  }
}

template <int DT, int D>
int launch_block_score_d(const BlockScoreArgs& a0, hipStream_t st) {
  const int64_t waves = (a0.nq + 31) / 32 * a0.hkv;
  const dim3 grid((unsigned)((waves + 3) / 4));
  if (a0.topk > 64) {
    BlockScoreArgs a = a0;
    a.k1 = a0.topk - 2 < 64 ? a0.topk - 2 : 64;
    a.kout = a.k1;
    hipLaunchKernelGGL((block_score_kernel<DT, D, 64, BS_FIRST>), grid, dim3(256), 0, st, a);
    LSRM_CHECK_LAUNCH();
    a.kout = a0.topk - a.k1;
    hipLaunchKernelGGL((block_score_kernel<DT, D, 64, BS_SECOND>), grid, dim3(256), 0, st, a);
    LSRM_CHECK_LAUNCH();
    return LSRM_OK;
  }
  BlockScoreArgs a = a0;
  a.kout = a0.topk;
#define LSRM_BS_K(KV)                                                                    \
  hipLaunchKernelGGL((block_score_kernel<DT, D, KV, BS_ONE>), grid, dim3(256), 0, st, a); \
  break;
  switch (a.topk <= 8 ? 8 : a.topk <= 16 ? 16 : a.topk <= 32 ? 32 : 64) {
    case 8: LSRM_BS_K(8)
    case 16: LSRM_BS_K(16)
    case 32: LSRM_BS_K(32)
    default: LSRM_BS_K(64)
  }
#undef LSRM_BS_K
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

}  // namespace lsrm

using namespace lsrm;

extern "C" int lsrm_block_score(const void* q, const void* compressed_k, int dtype,
                                const float* lse, int64_t n_q, int64_t hq, int64_t hkv,
                                int64_t head_dim, const int32_t* cu_seqlens_q,
                                const int32_t* compressed_cu_seqlens, int64_t batch,
                                int64_t topk, float sm_scale, int32_t* block_topk,
                                void* stream) {
  if (n_q < 0 || hq <= 0 || hkv <= 0 || batch <= 0 || topk <= 0 || hq % hkv != 0 ||
      !cu_seqlens_q || !compressed_cu_seqlens ||
      (n_q > 0 && (!q || !compressed_k || !lse || !block_topk)))
    return LSRM_ERR_INVALID_ARG;
  if (dtype != LSRM_F16 && dtype != LSRM_BF16) return LSRM_ERR_UNSUPPORTED;
  if (topk > 128 || (head_dim != 32 && head_dim != 64 && head_dim != 128))
    return LSRM_ERR_UNSUPPORTED;
  if (n_q == 0) return LSRM_OK;
  BlockScoreArgs a;
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.ck = reinterpret_cast<const uint16_t*>(compressed_k);
  a.lse = lse;
  a.cu_q = cu_seqlens_q;
  a.cu_c = compressed_cu_seqlens;
  a.out = block_topk;
  a.nq = n_q;
  a.batch = batch;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.g = (int)(hq / hkv);
  a.topk = (int)topk;
  a.qk_scale = sm_scale * LOG2E_REF;
  hipStream_t st = (hipStream_t)stream;
#define LSRM_BS_D(DT)                                               \
  switch (head_dim) {                                               \
    case 32: return launch_block_score_d<DT, 32>(a, st);            \
    case 64: return launch_block_score_d<DT, 64>(a, st);            \
    default: return launch_block_score_d<DT, 128>(a, st);           \
  }
  if (dtype == LSRM_BF16) {
    LSRM_BS_D(LSRM_BF16)
  } else {
    LSRM_BS_D(LSRM_F16)
  }
#undef LSRM_BS_D
}
