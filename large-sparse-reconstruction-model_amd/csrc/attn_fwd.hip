// Selected-block attention forward on bf16/fp16 MFMA (gfx950).
//
// Semantics follow forward_kernel_varblock
// (sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:55-247): for
// every query row, an online softmax in base 2 (scale folded into the
// exponent) over the tokens of its selected blocks, P rounded to the input
// type before P.V, O = acc / l and LSE = m + log2(l) in log2 units.
//
// Design: a persistent grid pulls query tiles (128 rows of one kv head that
// share one selection) from an atomic queue.  Each wave owns 32 rows.  The
// tile's key stream is gathered through LDS 64 keys at a time (K row-major,
// V transposed), double buffered with a register prefetch of the next tile.
// Scores are computed transposed, S^T = K Q^T, so that a lane owns one query
// row through the whole softmax and the accumulator O^T = V^T P^T; the
// softmax statistics stay in-lane except one cross-half exchange.
#include "attn.h"

namespace lsrm {

// Largest growth (log2 units) of a row maximum over the running reference
// before O and l are rescaled.
constexpr float RESCALE_LOG2 = 8.0f;

template <int DT, int D>
__global__ __launch_bounds__(256) void sel_attn_fwd_kernel(AttnArgs a) {
  constexpr int KS = D + 8;   // sK row stride (elements)
  constexpr int VS = KT + 4;  // sV row stride (elements, 8-byte rows)
  constexpr int NS = D / 16;  // MFMA k-steps over the head dim
  constexpr int ND = D / 32;  // 32-wide output blocks over the head dim
  constexpr int NW = D / 16;  // 32-bit words a loader moves per key
  __shared__ __align__(16) uint16_t sK[2][KT * KS];
  __shared__ __align__(16) uint16_t sV[2][D * VS];
  __shared__ SelLds sel;
  __shared__ int s_slot;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int hb = lane >> 5, l32 = lane & 31;
  const int kp = tid >> 3, dg = tid & 7;  // loader: keys 2kp, 2kp+1; d group
  const int total = a.plan.head_off[a.hkv];

  for (;;) {
    const int w = fetch_work(a.plan.counter, &s_slot);
    if (w >= total) break;
    const int h = head_of(a.plan.head_off, a.hkv, w);
    const int2 tile = a.plan.tiles[(int64_t)h * a.nq + (w - a.plan.head_off[h])];
    const int q0 = tile.x, rows = tile.y * a.g;
    load_selection(a, h, q0, sel);
    const int nkeys = sel.cum[sel.n];
    const int ntiles = (nkeys + KT - 1) / KT;

    // This wave's row and its Q operand (B of S^T = K Q^T).
    const int r = wv * 32 + l32;
    const bool row_ok = r < rows;
    const bool wave_on = wv * 32 < rows;
    const int64_t qi = q0 + (row_ok ? r / a.g : 0);
    const int hh = h * a.g + (row_ok ? r % a.g : 0);
    u32x4 qb[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (row_ok)
        qb[s] = *reinterpret_cast<const u32x4*>(
            a.q + (qi * a.hq + hh) * D + s * 16 + hb * 8);
      else
        qb[s] = u32x4{0u, 0u, 0u, 0u};
    }

    f32x16 oacc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
    float m_run = -__builtin_inf(), l_run = 0.0f;

    int cur0 = 0, cur1 = 0;
    uint32_t kr[2][NW], vr[2][NW];
    auto gather = [&](int kt) {
      const int p0 = kt * KT + 2 * kp, p1 = p0 + 1;
      if (p0 < nkeys) {
        const int t = stream_token(sel, p0, cur0);
        const int64_t off = ((int64_t)t * a.hkv + h) * D + dg * (D / 8);
        gload<NW>(kr[0], a.k + off);
        gload<NW>(vr[0], a.v + off);
      } else {
#pragma unroll
        for (int i = 0; i < NW; ++i) kr[0][i] = vr[0][i] = 0u;
      }
      if (p1 < nkeys) {
        const int t = stream_token(sel, p1, cur1);
        const int64_t off = ((int64_t)t * a.hkv + h) * D + dg * (D / 8);
        gload<NW>(kr[1], a.k + off);
        gload<NW>(vr[1], a.v + off);
      } else {
#pragma unroll
        for (int i = 0; i < NW; ++i) kr[1][i] = vr[1][i] = 0u;
      }
    };
    auto stage = [&](int buf) {
      sstore<NW>(&sK[buf][(2 * kp) * KS + dg * (D / 8)], kr[0]);
      sstore<NW>(&sK[buf][(2 * kp + 1) * KS + dg * (D / 8)], kr[1]);
#pragma unroll
      for (int j = 0; j < NW; ++j) {
        const int d = dg * (D / 8) + 2 * j;
        *reinterpret_cast<uint32_t*>(&sV[buf][d * VS + 2 * kp]) =
            pair_lo(vr[0][j], vr[1][j]);
        *reinterpret_cast<uint32_t*>(&sV[buf][(d + 1) * VS + 2 * kp]) =
            pair_hi(vr[0][j], vr[1][j]);
      }
    };

    if (ntiles > 0) {
      gather(0);
      stage(0);
    }
    __syncthreads();

    for (int kt = 0; kt < ntiles; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < ntiles) gather(kt + 1);
      if (wave_on) {
        const uint16_t* k_s = sK[buf];
        const uint16_t* v_s = sV[buf];
        f32x16 sacc[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
          for (int v = 0; v < 16; ++v) sacc[blk][v] = 0.0f;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const u32x4 ka = *reinterpret_cast<const u32x4*>(
                k_s + (blk * 32 + l32) * KS + s * 16 + hb * 8);
            sacc[blk] = mfma32<DT>(ka, qb[s], sacc[blk]);
          }
        }
        const int kbase = kt * KT;
        if (kbase + KT > nkeys) {
#pragma unroll
          for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              if (kbase + blk * 32 + acc_row(v, hb) >= nkeys)
                sacc[blk][v] = -__builtin_inf();
        }
        float mx = sacc[0][0];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[blk][v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // Lazy rescaling: the running reference m_run only moves when a row
        // maximum exceeds it by more than RESCALE_LOG2 (so p <= 2^8); the
        // final O = acc / l is the same for any reference.
        const float m_tile = mx * a.scale_log2;
        if (__builtin_amdgcn_ballot_w64(m_tile > m_run + RESCALE_LOG2) != 0) {
          const float m_new = fmaxf(m_run, m_tile);
          const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
          m_run = m_new;
          l_run *= alpha;
#pragma unroll
          for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[db][v] *= alpha;
        }
        u32x4 pb[2][2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          float p[16];
#pragma unroll
          for (int v = 0; v < 16; ++v)
            p[v] = __builtin_amdgcn_exp2f(
                __builtin_fmaf(sacc[blk][v], a.scale_log2, -m_run));
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            pb[blk][c] = u32x4{pack2<DT>(p[c * 8 + 0], p[c * 8 + 1]),
                               pack2<DT>(p[c * 8 + 2], p[c * 8 + 3]),
                               pack2<DT>(p[c * 8 + 4], p[c * 8 + 5]),
                               pack2<DT>(p[c * 8 + 6], p[c * 8 + 7])};
#pragma unroll
            for (int w = 0; w < 4; ++w) l_run = sum2<DT>(pb[blk][c][w], l_run);
          }
        }
#pragma unroll
        for (int db = 0; db < ND; ++db) {
#pragma unroll
          for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const uint16_t* vp =
                  v_s + (db * 32 + l32) * VS + blk * 32 + c * 16 + hb * 4;
              const u32x2 lo = *reinterpret_cast<const u32x2*>(vp);
              const u32x2 hi = *reinterpret_cast<const u32x2*>(vp + 8);
              oacc[db] = mfma32<DT>(u32x4{lo[0], lo[1], hi[0], hi[1]},
                                    pb[blk][c], oacc[db]);
            }
        }
      }
      if (kt + 1 < ntiles) stage(buf ^ 1);
      __syncthreads();
    }

    // Epilogue: normalise, store O rows and LSE.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (row_ok) {
      const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      uint16_t* orow = a.out + (qi * a.hq + hh) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int v = gi * 4;
          *reinterpret_cast<u32x2*>(orow + db * 32 + gi * 8 + hb * 4) =
              u32x2{pack2<DT>(oacc[db][v] * inv, oacc[db][v + 1] * inv),
                    pack2<DT>(oacc[db][v + 2] * inv, oacc[db][v + 3] * inv)};
        }
      if (hb == 0)
        a.lse[(int64_t)hh * a.nq + qi] =
            l_tot > 0.0f ? m_run + log2f(l_tot) : -__builtin_inf();
    }
  }
  leave_queue(a.plan.counter, a.plan.counter + 2);
}

template <int DT, int D>
int launch_fwd_t(const AttnArgs& a, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&sel_attn_fwd_kernel<DT, D>);
  const int grid = persistent_grid(fn, 256, 0);
  if (grid <= 0) return LSRM_ERR_LAUNCH;
  hipLaunchKernelGGL((sel_attn_fwd_kernel<DT, D>), dim3(grid), dim3(256), 0, st,
                     a);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

int launch_fwd(int dtype, int d, const AttnArgs& a, hipStream_t st) {
#define LSRM_FWD_D(DT)                                        \
  switch (d) {                                                \
    case 32: return launch_fwd_t<DT, 32>(a, st);              \
    case 64: return launch_fwd_t<DT, 64>(a, st);              \
    case 128: return launch_fwd_t<DT, 128>(a, st);            \
    default: return LSRM_ERR_UNSUPPORTED;                     \
  }
  if (dtype == LSRM_BF16) {
    LSRM_FWD_D(LSRM_BF16)
  } else if (dtype == LSRM_F16) {
    LSRM_FWD_D(LSRM_F16)
  }
#undef LSRM_FWD_D
  return LSRM_ERR_UNSUPPORTED;
}

}  // namespace lsrm
