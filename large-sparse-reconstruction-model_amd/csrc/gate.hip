// Gated merge of the sparse-attention branch outputs
// (sparse/module/spatial_sparse_attention.py:256-269):
//
//   out = g[:, 0:H] * o_cmp + g[:, H:2H] * o_slc  (+ g[:, 2H:3H] * o_win)
//
// evaluated as PyTorch evaluates that expression on tensors of one dtype:
// every product and every sum is a separate elementwise op computed in fp32
// and rounded to the dtype (round to nearest even), left to right:
//   t = rnd(rnd(g0 * c) + rnd(g1 * s));  out = rnd(t + rnd(g2 * w)).
// The backward is autograd of the same expression: d_o_x = rnd(dout * g_x),
// d_g_x = rnd(dout * o_x) (sums pass gradients through unchanged).
//
// HBM-bound streaming: one thread per 8 consecutive elements of a row
// (16-byte non-temporal loads and stores of the 16-bit types), no reuse.
#include "common.h"

namespace lsrm {

// Element access and rounding to the storage type.
template <int DT>
struct Ew {
  __device__ static inline float ld(const void* p, int64_t i) {
    return to_f32<DT>(reinterpret_cast<const uint16_t*>(p)[i]);
  }
  __device__ static inline void st(void* p, int64_t i, float v) {
    reinterpret_cast<uint16_t*>(p)[i] = from_f32<DT>(v);
  }
  __device__ static inline float rnd(float v) { return to_f32<DT>(from_f32<DT>(v)); }
  // 8 consecutive elements starting at i (16-byte aligned); streamed once,
  // so loaded and stored non-temporally.
  __device__ static inline void ld8(const void* p, int64_t i, float* v) {
    const u32x4 w = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p) + i));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = to_f32<DT>((uint16_t)(w[k] & 0xffffu));
      v[2 * k + 1] = to_f32<DT>((uint16_t)(w[k] >> 16));
    }
  }
  __device__ static inline void st8(void* p, int64_t i, const float* v) {
    __builtin_nontemporal_store(
        u32x4{pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]),
              pack2<DT>(v[6], v[7])},
        reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(p) + i));
  }
};
template <>
struct Ew<LSRM_F32> {
  __device__ static inline float ld(const void* p, int64_t i) {
    return reinterpret_cast<const float*>(p)[i];
  }
  __device__ static inline void st(void* p, int64_t i, float v) {
    reinterpret_cast<float*>(p)[i] = v;
  }
  __device__ static inline float rnd(float v) { return v; }
  __device__ static inline void ld8(const void* p, int64_t i, float* v) {
    const float* q = reinterpret_cast<const float*>(p) + i;
    const f32x4 a = *reinterpret_cast<const f32x4*>(q);
    const f32x4 b = *reinterpret_cast<const f32x4*>(q + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[4 + k] = b[k];
    }
  }
  __device__ static inline void st8(void* p, int64_t i, const float* v) {
    float* q = reinterpret_cast<float*>(p) + i;
    *reinterpret_cast<f32x4*>(q) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(q + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};

// VEC: 8 elements per thread (hidden % 8 == 0, 16-byte aligned rows), else 1.
template <int DT, bool WIN, int VEC>
__global__ __launch_bounds__(256) void gate_merge_kernel(
    const void* __restrict__ gate, const void* __restrict__ oc, const void* __restrict__ os,
    const void* __restrict__ ow, int64_t n, int64_t hid, void* __restrict__ out) {
#pragma clang fp contract(off)
  using E = Ew<DT>;
  // The host guarantees n * hid < 2^32 (32-bit index arithmetic).
  const uint32_t groups = (uint32_t)(hid / VEC), total = (uint32_t)n * groups;
  const uint32_t gs = (WIN ? 3u : 2u) * (uint32_t)hid;  // gate row stride
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += gridDim.x * blockDim.x) {
    const uint32_t r = t / groups, c = (t - r * groups) * VEC;
    const int64_t gi = (int64_t)r * gs + c, oi = (int64_t)r * hid + c;
    float g0[VEC], g1[VEC], g2[VEC], xc[VEC], xs[VEC], xw[VEC], y[VEC];
    if constexpr (VEC == 8) {
      E::ld8(gate, gi, g0);
      E::ld8(gate, gi + hid, g1);
      E::ld8(oc, oi, xc);
      E::ld8(os, oi, xs);
      if constexpr (WIN) {
        E::ld8(gate, gi + 2 * hid, g2);
        E::ld8(ow, oi, xw);
      }
    } else {
      g0[0] = E::ld(gate, gi);
      g1[0] = E::ld(gate, gi + hid);
      xc[0] = E::ld(oc, oi);
      xs[0] = E::ld(os, oi);
      if constexpr (WIN) {
        g2[0] = E::ld(gate, gi + 2 * hid);
        xw[0] = E::ld(ow, oi);
      }
    }
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      float v = E::rnd(E::rnd(g0[k] * xc[k]) + E::rnd(g1[k] * xs[k]));
      if constexpr (WIN) v = E::rnd(v + E::rnd(g2[k] * xw[k]));
      y[k] = v;
    }
    if constexpr (VEC == 8)
      E::st8(out, oi, y);
    else
      E::st(out, oi, y[0]);
  }
}

template <int DT, bool WIN, int VEC>
__global__ __launch_bounds__(256) void gate_merge_bwd_kernel(
    const void* __restrict__ dout, const void* __restrict__ gate,
    const void* __restrict__ oc, const void* __restrict__ os, const void* __restrict__ ow,
    int64_t n, int64_t hid, void* __restrict__ dgate, void* __restrict__ dc,
    void* __restrict__ ds, void* __restrict__ dw) {
#pragma clang fp contract(off)
  using E = Ew<DT>;
  const uint32_t groups = (uint32_t)(hid / VEC), total = (uint32_t)n * groups;
  const uint32_t gs = (WIN ? 3u : 2u) * (uint32_t)hid;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += gridDim.x * blockDim.x) {
    const uint32_t r = t / groups, c = (t - r * groups) * VEC;
    const int64_t gi = (int64_t)r * gs + c, oi = (int64_t)r * hid + c;
    constexpr int NB = WIN ? 3 : 2;  // branches
    for (int b = 0; b < NB; ++b) {
      const void* ob = b == 0 ? oc : (b == 1 ? os : ow);
      void* dob = b == 0 ? dc : (b == 1 ? ds : dw);
      float d[VEC], g[VEC], x[VEC], dg[VEC], dx[VEC];
      if constexpr (VEC == 8) {
        E::ld8(dout, oi, d);
        E::ld8(gate, gi + b * hid, g);
        E::ld8(ob, oi, x);
      } else {
        d[0] = E::ld(dout, oi);
        g[0] = E::ld(gate, gi + b * hid);
        x[0] = E::ld(ob, oi);
      }
#pragma unroll
      for (int k = 0; k < VEC; ++k) {
        dg[k] = E::rnd(d[k] * x[k]);
        dx[k] = E::rnd(d[k] * g[k]);
      }
      if constexpr (VEC == 8) {
        E::st8(dgate, gi + b * hid, dg);
        E::st8(dob, oi, dx);
      } else {
        E::st(dgate, gi + b * hid, dg[0]);
        E::st(dob, oi, dx[0]);
      }
    }
  }
}

// One thread per work item up to a large cap (the grid-stride loop only
// serves sizes beyond it): at 16 workgroups per CU the in-order loop kept too
// few loads in flight (cfg3 merge: 600 us against 476 us with one item per
// thread and non-temporal access).
int gate_grid(int64_t total) {
  const int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)(device_cu_count() > 0 ? device_cu_count() : 256) * 4096;
  return (int)(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

bool vec_ok(int64_t hid, const void* const* ptrs, int n) {
  if (hid % 8 != 0) return false;
  for (int i = 0; i < n; ++i)
    if (ptrs[i] && ((uintptr_t)ptrs[i] & 15u) != 0) return false;
  return true;
}

}  // namespace lsrm

using namespace lsrm;

extern "C" int lsrm_gate_merge(const void* gate, const void* o_cmp, const void* o_slc,
                               const void* o_win, int dtype, int64_t n_tokens, int64_t hidden,
                               void* out, void* stream) {
  if (n_tokens < 0 || hidden <= 0 || (n_tokens > 0 && (!gate || !o_cmp || !o_slc || !out)))
    return LSRM_ERR_INVALID_ARG;
  if (dtype != LSRM_BF16 && dtype != LSRM_F16 && dtype != LSRM_F32) return LSRM_ERR_UNSUPPORTED;
  if ((uint64_t)n_tokens * (uint64_t)hidden * 3u >= (1ull << 32)) return LSRM_ERR_UNSUPPORTED;
  if (n_tokens == 0) return LSRM_OK;
  hipStream_t st = (hipStream_t)stream;
  const void* ptrs[5] = {gate, o_cmp, o_slc, o_win, out};
  const bool vec = vec_ok(hidden, ptrs, 5);
  const int64_t total = n_tokens * (vec ? hidden / 8 : hidden);
  const dim3 grid(gate_grid(total));
#define LSRM_GM(DTV, WINV, VECV)                                                           \
  hipLaunchKernelGGL((gate_merge_kernel<DTV, WINV, VECV>), grid, dim3(256), 0, st, gate, \
                     o_cmp, o_slc, o_win, n_tokens, hidden, out)
#define LSRM_GM_DT(DTV)                  \
  if (o_win) {                           \
    if (vec) LSRM_GM(DTV, true, 8);      \
    else LSRM_GM(DTV, true, 1);          \
  } else {                               \
    if (vec) LSRM_GM(DTV, false, 8);     \
    else LSRM_GM(DTV, false, 1);         \
  }
  if (dtype == LSRM_BF16) {
    LSRM_GM_DT(LSRM_BF16)
  } else if (dtype == LSRM_F16) {
    LSRM_GM_DT(LSRM_F16)
  } else {
    LSRM_GM_DT(LSRM_F32)
  }
#undef LSRM_GM_DT
#undef LSRM_GM
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

extern "C" int lsrm_gate_merge_bwd(const void* dout, const void* gate, const void* o_cmp,
                                   const void* o_slc, const void* o_win, int dtype,
                                   int64_t n_tokens, int64_t hidden, void* d_gate, void* d_cmp,
                                   void* d_slc, void* d_win, void* stream) {
  if (n_tokens < 0 || hidden <= 0 || (!o_win) != (!d_win) ||
      (n_tokens > 0 && (!dout || !gate || !o_cmp || !o_slc || !d_gate || !d_cmp || !d_slc)))
    return LSRM_ERR_INVALID_ARG;
  if (dtype != LSRM_BF16 && dtype != LSRM_F16 && dtype != LSRM_F32) return LSRM_ERR_UNSUPPORTED;
  if ((uint64_t)n_tokens * (uint64_t)hidden * 3u >= (1ull << 32)) return LSRM_ERR_UNSUPPORTED;
  if (n_tokens == 0) return LSRM_OK;
  hipStream_t st = (hipStream_t)stream;
  const void* ptrs[9] = {dout, gate, o_cmp, o_slc, o_win, d_gate, d_cmp, d_slc, d_win};
  const bool vec = vec_ok(hidden, ptrs, 9);
  const int64_t total = n_tokens * (vec ? hidden / 8 : hidden);
  const dim3 grid(gate_grid(total));
#define LSRM_GMB(DTV, WINV, VECV)                                                          \
  hipLaunchKernelGGL((gate_merge_bwd_kernel<DTV, WINV, VECV>), grid, dim3(256), 0, st,   \
                     dout, gate, o_cmp, o_slc, o_win, n_tokens, hidden, d_gate, d_cmp,      \
                     d_slc, d_win)
#define LSRM_GMB_DT(DTV)                 \
  if (o_win) {                           \
    if (vec) LSRM_GMB(DTV, true, 8);     \
    else LSRM_GMB(DTV, true, 1);         \
  } else {                               \
    if (vec) LSRM_GMB(DTV, false, 8);    \
    else LSRM_GMB(DTV, false, 1);        \
  }
  if (dtype == LSRM_BF16) {
    LSRM_GMB_DT(LSRM_BF16)
  } else if (dtype == LSRM_F16) {
    LSRM_GMB_DT(LSRM_F16)
  } else {
    LSRM_GMB_DT(LSRM_F32)
  }
#undef LSRM_GMB_DT
#undef LSRM_GMB
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}
