// Selected-block attention backward on bf16/fp16 MFMA (gfx950).
//
// dQ follows backward_kernel_dq
// (sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:262-478):
// Delta = rowsum(O * dO) in fp32 (fused), P = exp2(q.k * scale*log2e - lse),
// dP = dO V^T, dS = scale * P * (dP - Delta) rounded to the input type,
// dQ = dS K.  It runs on the forward's query tiles and key stream.
//
// dK/dV follow backward_kernel_dkdv_fastest (same file, 687-923): each
// workgroup owns one 64-key chunk of one block of one kv head and walks the
// query tiles that selected the block (tile-granular reverse map, ascending
// tile order), so every dK/dV element has a single writer and a fixed
// accumulation order.  Waves split the chunk 2 (keys) x 2 (rows); the two
// row halves are added in a fixed order at the end.
#include "attn.h"

namespace lsrm {

// ------------------------------------------------------------------- dQ --

template <int DT, int D>
__global__ __launch_bounds__(256) void sel_attn_dq_kernel(AttnArgs a) {
  constexpr int KS = D + 8;
  constexpr int VS = KT + 4;
  constexpr int NS = D / 16;
  constexpr int ND = D / 32;
  constexpr int NW = D / 16;
  __shared__ __align__(16) uint16_t sK[2][KT * KS];
  __shared__ __align__(16) uint16_t sKt[2][D * VS];
  __shared__ __align__(16) uint16_t sV[2][KT * KS];
  __shared__ SelLds sel;
  __shared__ int s_slot;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int hb = lane >> 5, l32 = lane & 31;
  const int kp = tid >> 3, dg = tid & 7;
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

    const int r = wv * 32 + l32;
    const bool row_ok = r < rows;
    const bool wave_on = wv * 32 < rows;
    const int64_t qi = q0 + (row_ok ? r / a.g : 0);
    const int hh = h * a.g + (row_ok ? r % a.g : 0);
    u32x4 qb[NS], dob[NS];
    float dpart = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (row_ok) {
        const int64_t off = (qi * a.hq + hh) * D + s * 16 + hb * 8;
        qb[s] = *reinterpret_cast<const u32x4*>(a.q + off);
        dob[s] = *reinterpret_cast<const u32x4*>(a.dout + off);
        const u32x4 ob = *reinterpret_cast<const u32x4*>(a.o + off);
        const uint32_t ow[4] = {ob[0], ob[1], ob[2], ob[3]};
        const uint32_t dw[4] = {dob[s][0], dob[s][1], dob[s][2], dob[s][3]};
#pragma unroll
        for (int i = 0; i < 8; ++i)
          dpart += to_f32<DT>((uint16_t)half_of(ow, i)) *
                   to_f32<DT>((uint16_t)half_of(dw, i));
      } else {
        qb[s] = u32x4{0u, 0u, 0u, 0u};
        dob[s] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    const float delta = dpart + __shfl_xor(dpart, 32);
    const float lse_row =
        row_ok ? a.lse_in[(int64_t)hh * a.nq + qi] : __builtin_inf();
    if (row_ok && hb == 0) a.lse[(int64_t)hh * a.nq + qi] = delta;

    f32x16 dqacc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) dqacc[i][v] = 0.0f;

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
      sstore<NW>(&sV[buf][(2 * kp) * KS + dg * (D / 8)], vr[0]);
      sstore<NW>(&sV[buf][(2 * kp + 1) * KS + dg * (D / 8)], vr[1]);
#pragma unroll
      for (int i = 0; i < D / 8; ++i) {
        const int d = dg * (D / 8) + i;
        *reinterpret_cast<uint32_t*>(&sKt[buf][d * VS + 2 * kp]) =
            half_of(kr[0], i) | (half_of(kr[1], i) << 16);
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
        const uint16_t* kt_s = sKt[buf];
        const uint16_t* v_s = sV[buf];
        const int kbase = kt * KT;
        u32x4 dsb[2][2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          f32x16 sacc, dpacc;
#pragma unroll
          for (int v = 0; v < 16; ++v) sacc[v] = dpacc[v] = 0.0f;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const int off = (blk * 32 + l32) * KS + s * 16 + hb * 8;
            sacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(k_s + off), qb[s],
                              sacc);
            dpacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(v_s + off),
                               dob[s], dpacc);
          }
          float ds[16];
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            float p = __builtin_amdgcn_exp2f(
                __builtin_fmaf(sacc[v], a.scale_log2, -lse_row));
            if (kbase + blk * 32 + acc_row(v, hb) >= nkeys) p = 0.0f;
            ds[v] = a.scale * p * (dpacc[v] - delta);
          }
#pragma unroll
          for (int c = 0; c < 2; ++c)
            dsb[blk][c] = u32x4{pack2<DT>(ds[c * 8 + 0], ds[c * 8 + 1]),
                                pack2<DT>(ds[c * 8 + 2], ds[c * 8 + 3]),
                                pack2<DT>(ds[c * 8 + 4], ds[c * 8 + 5]),
                                pack2<DT>(ds[c * 8 + 6], ds[c * 8 + 7])};
        }
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const uint16_t* kp_ =
                  kt_s + (db * 32 + l32) * VS + blk * 32 + c * 16 + hb * 4;
              const u32x2 lo = *reinterpret_cast<const u32x2*>(kp_);
              const u32x2 hi = *reinterpret_cast<const u32x2*>(kp_ + 8);
              dqacc[db] = mfma32<DT>(u32x4{lo[0], lo[1], hi[0], hi[1]},
                                     dsb[blk][c], dqacc[db]);
            }
      }
      if (kt + 1 < ntiles) stage(buf ^ 1);
      __syncthreads();
    }

    if (row_ok) {
      uint16_t* drow = a.out + (qi * a.hq + hh) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int v = gi * 4;
          *reinterpret_cast<u32x2*>(drow + db * 32 + gi * 8 + hb * 4) =
              u32x2{pack2<DT>(dqacc[db][v], dqacc[db][v + 1]),
                    pack2<DT>(dqacc[db][v + 2], dqacc[db][v + 3])};
        }
    }
  }
  leave_queue(a.plan.counter, a.plan.counter + 2);
}

// ----------------------------------------------------------------- dK/dV --

template <int DT, int D>
__global__ __launch_bounds__(256) void sel_attn_dkdv_kernel(AttnArgs a) {
  constexpr int KS = D + 8;      // row-major staging stride
  constexpr int QS = ROWS + 4;   // transposed staging stride
  constexpr int NS = D / 16;
  constexpr int ND = D / 32;
  constexpr int LW = D / 8;      // 32-bit words a loader moves per row
  constexpr int STAGE_BYTES = 2 * ROWS * KS * 2 + 2 * D * QS * 2;
  constexpr int RED_BYTES = 2 * 2 * ND * 16 * 64 * 4;
  constexpr int LDS_BYTES = STAGE_BYTES > RED_BYTES ? STAGE_BYTES : RED_BYTES;
  __shared__ __align__(16) char smem[LDS_BYTES];
  __shared__ float s_lse[ROWS];
  __shared__ float s_dl[ROWS];
  __shared__ int s_slot;
  uint16_t* sQ = reinterpret_cast<uint16_t*>(smem);
  uint16_t* sO = sQ + ROWS * KS;
  uint16_t* sQt = sO + ROWS * KS;
  uint16_t* sOt = sQt + D * QS;
  float* red = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int hb = lane >> 5, l32 = lane & 31;
  const int kh = wv & 1, rh = wv >> 1;   // key half, row half of this wave
  const int rp = tid >> 2, dq = tid & 3; // loader: rows 2rp, 2rp+1; d quarter
  const int n_items = a.items.n_items[0];
  const int total = n_items * a.hkv;

  for (;;) {
    const int w = fetch_work(a.plan.counter + 1, &s_slot);
    if (w >= total) break;
    const int h = w / n_items;
    const int4 item = a.items.items[w - h * n_items];
    const int c = item.x, t0 = item.y, nk_item = item.z;
    const int64_t e0 = a.rev.cu_rev[(int64_t)h * (a.nb + 1) + c];
    int64_t e1 = a.rev.cu_rev[(int64_t)h * (a.nb + 1) + c + 1];
    if (e1 > a.rev.cap) e1 = a.rev.cap;
    const int n_ent = e1 > e0 ? (int)(e1 - e0) : 0;
    const int32_t* ents = a.rev.rev + (int64_t)h * a.rev.cap + e0;

    // This wave's 32 keys as B operands (K^T, V^T columns).
    const int key = kh * 32 + l32;
    const bool key_ok = key < nk_item;
    u32x4 kb[NS], vb[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (key_ok) {
        const int64_t off = ((int64_t)(t0 + key) * a.hkv + h) * D + s * 16 + hb * 8;
        kb[s] = *reinterpret_cast<const u32x4*>(a.k + off);
        vb[s] = *reinterpret_cast<const u32x4*>(a.v + off);
      } else {
        kb[s] = vb[s] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    f32x16 dkacc[ND], dvacc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) dkacc[i][v] = dvacc[i][v] = 0.0f;

    uint32_t qr[2][LW], orr[2][LW];
    float lse_r = 0.0f, dl_r = 0.0f;
    int rows_next = 0;
    auto gather = [&](int e) {
      const int2 tile = a.plan.tiles[(int64_t)h * a.nq + ents[e]];
      const int rows = tile.y * a.g;
      rows_next = rows;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = 2 * rp + j;
        if (row < rows) {
          const int64_t qi = tile.x + row / a.g;
          const int hh = h * a.g + row % a.g;
          const int64_t off = (qi * a.hq + hh) * D + dq * (D / 4);
          gload<LW>(qr[j], a.q + off);
          gload<LW>(orr[j], a.dout + off);
        } else {
#pragma unroll
          for (int i = 0; i < LW; ++i) qr[j][i] = orr[j][i] = 0u;
        }
      }
      if (tid < ROWS) {
        if (tid < rows) {
          const int64_t qi = tile.x + tid / a.g;
          const int hh = h * a.g + tid % a.g;
          lse_r = a.lse_in[(int64_t)hh * a.nq + qi];
          dl_r = a.lse[(int64_t)hh * a.nq + qi];
        } else {
          lse_r = __builtin_inf();
          dl_r = 0.0f;
        }
      }
    };
    auto stage = [&]() {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        sstore<LW>(&sQ[(2 * rp + j) * KS + dq * (D / 4)], qr[j]);
        sstore<LW>(&sO[(2 * rp + j) * KS + dq * (D / 4)], orr[j]);
      }
#pragma unroll
      for (int i = 0; i < D / 4; ++i) {
        const int d = dq * (D / 4) + i;
        *reinterpret_cast<uint32_t*>(&sQt[d * QS + 2 * rp]) =
            half_of(qr[0], i) | (half_of(qr[1], i) << 16);
        *reinterpret_cast<uint32_t*>(&sOt[d * QS + 2 * rp]) =
            half_of(orr[0], i) | (half_of(orr[1], i) << 16);
      }
      if (tid < ROWS) {
        s_lse[tid] = lse_r;
        s_dl[tid] = dl_r;
      }
    };

    if (n_ent > 0) gather(0);
    for (int e = 0; e < n_ent; ++e) {
      __syncthreads();
      stage();
      const int rows = rows_next;
      __syncthreads();
      if (e + 1 < n_ent) gather(e + 1);
      {
        if (rh * 64 < rows && kh * 32 < nk_item) {
          u32x4 pb[2][2], dsb[2][2];
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            f32x16 sacc, dpacc;
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[v] = dpacc[v] = 0.0f;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
              const int off = (rh * 64 + rb * 32 + l32) * KS + s * 16 + hb * 8;
              sacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(sQ + off), kb[s],
                                sacc);
              dpacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(sO + off),
                                 vb[s], dpacc);
            }
            float p[16], ds[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int row = rh * 64 + rb * 32 + acc_row(v, hb);
              p[v] = __builtin_amdgcn_exp2f(
                  __builtin_fmaf(sacc[v], a.scale_log2, -s_lse[row]));
              ds[v] = a.scale * p[v] * (dpacc[v] - s_dl[row]);
            }
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
              pb[rb][cc] = u32x4{pack2<DT>(p[cc * 8 + 0], p[cc * 8 + 1]),
                                 pack2<DT>(p[cc * 8 + 2], p[cc * 8 + 3]),
                                 pack2<DT>(p[cc * 8 + 4], p[cc * 8 + 5]),
                                 pack2<DT>(p[cc * 8 + 6], p[cc * 8 + 7])};
              dsb[rb][cc] = u32x4{pack2<DT>(ds[cc * 8 + 0], ds[cc * 8 + 1]),
                                  pack2<DT>(ds[cc * 8 + 2], ds[cc * 8 + 3]),
                                  pack2<DT>(ds[cc * 8 + 4], ds[cc * 8 + 5]),
                                  pack2<DT>(ds[cc * 8 + 6], ds[cc * 8 + 7])};
            }
          }
#pragma unroll
          for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
              for (int cc = 0; cc < 2; ++cc) {
                const int off =
                    (db * 32 + l32) * QS + rh * 64 + rb * 32 + cc * 16 + hb * 4;
                const u32x2 olo = *reinterpret_cast<const u32x2*>(sOt + off);
                const u32x2 ohi = *reinterpret_cast<const u32x2*>(sOt + off + 8);
                dvacc[db] = mfma32<DT>(u32x4{olo[0], olo[1], ohi[0], ohi[1]},
                                       pb[rb][cc], dvacc[db]);
                const u32x2 qlo = *reinterpret_cast<const u32x2*>(sQt + off);
                const u32x2 qhi = *reinterpret_cast<const u32x2*>(sQt + off + 8);
                dkacc[db] = mfma32<DT>(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]},
                                       dsb[rb][cc], dkacc[db]);
              }
        }
      }
    }
    // Row-half reduction in a fixed order: rows 0-63 + rows 64-127.
    __syncthreads();
    if (rh == 1) {
      float* dst = red + kh * (2 * ND * 16 * 64);
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          dst[((0 * ND + db) * 16 + v) * 64 + lane] = dkacc[db][v];
          dst[((1 * ND + db) * 16 + v) * 64 + lane] = dvacc[db][v];
        }
    }
    __syncthreads();
    if (rh == 0 && key_ok) {
      const float* src = red + kh * (2 * ND * 16 * 64);
      const int64_t base = ((int64_t)(t0 + key) * a.hkv + h) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          float kv[4], vv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int v = gi * 4 + u;
            kv[u] = dkacc[db][v] + src[((0 * ND + db) * 16 + v) * 64 + lane];
            vv[u] = dvacc[db][v] + src[((1 * ND + db) * 16 + v) * 64 + lane];
          }
          const int d = db * 32 + gi * 8 + hb * 4;
          *reinterpret_cast<u32x2*>(a.dk + base + d) =
              u32x2{pack2<DT>(kv[0], kv[1]), pack2<DT>(kv[2], kv[3])};
          *reinterpret_cast<u32x2*>(a.dv + base + d) =
              u32x2{pack2<DT>(vv[0], vv[1]), pack2<DT>(vv[2], vv[3])};
        }
    }
    __syncthreads();
  }
  leave_queue(a.plan.counter + 1, a.plan.counter + 3);
}

template <int DT, int D>
int launch_bwd_t(const AttnArgs& a, hipStream_t st) {
  {
    const void* fn = reinterpret_cast<const void*>(&sel_attn_dq_kernel<DT, D>);
    const int grid = persistent_grid(fn, 256, 0);
    if (grid <= 0) return LSRM_ERR_LAUNCH;
    hipLaunchKernelGGL((sel_attn_dq_kernel<DT, D>), dim3(grid), dim3(256), 0,
                       st, a);
    LSRM_CHECK_LAUNCH();
  }
  {
    const void* fn = reinterpret_cast<const void*>(&sel_attn_dkdv_kernel<DT, D>);
    const int grid = persistent_grid(fn, 256, 0);
    if (grid <= 0) return LSRM_ERR_LAUNCH;
    hipLaunchKernelGGL((sel_attn_dkdv_kernel<DT, D>), dim3(grid), dim3(256), 0,
                       st, a);
    LSRM_CHECK_LAUNCH();
  }
  return LSRM_OK;
}

int launch_bwd(int dtype, int d, const AttnArgs& a, hipStream_t st) {
#define LSRM_BWD_D(DT)                               \
  switch (d) {                                       \
    case 32: return launch_bwd_t<DT, 32>(a, st);     \
    case 64: return launch_bwd_t<DT, 64>(a, st);     \
    case 128: return launch_bwd_t<DT, 128>(a, st);   \
    default: return LSRM_ERR_UNSUPPORTED;            \
  }
  if (dtype == LSRM_BF16) {
    LSRM_BWD_D(LSRM_BF16)
  } else if (dtype == LSRM_F16) {
    LSRM_BWD_D(LSRM_F16)
  }
#undef LSRM_BWD_D
  return LSRM_ERR_UNSUPPORTED;
}

}  // namespace lsrm
