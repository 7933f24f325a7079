// Shared device helpers for the gfx950 sparse-attention kernels: element
// conversions, 16-byte vector types, MFMA wrappers and launch utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsrm_hip.h"

namespace lsrm {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// ---------------------------------------------------------------- scalars --

__device__ __host__ inline float bf16_bits_to_f32(uint16_t h) {
  union {
    uint32_t u;
    float f;
  } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}

__device__ inline float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ inline float to_f32(uint16_t h);
template <>
__device__ inline float to_f32<LSRM_BF16>(uint16_t h) {
  return bf16_bits_to_f32(h);
}
template <>
__device__ inline float to_f32<LSRM_F16>(uint16_t h) {
  return f16_bits_to_f32(h);
}

// fp32 -> 16-bit, round to nearest even (gfx950 v_cvt_pk_{bf16,f16}_f32).
template <int DT>
__device__ inline uint16_t from_f32(float f);
template <>
__device__ inline uint16_t from_f32<LSRM_BF16>(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
template <>
__device__ inline uint16_t from_f32<LSRM_F16>(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// Two floats -> two packed 16-bit values (lo = a, hi = b), round to nearest
// even: one v_cvt_pk_*_f32.
template <int DT>
__device__ inline uint32_t pack2(float a, float b);
template <>
__device__ inline uint32_t pack2<LSRM_BF16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)a, (__bf16)b});
}
template <>
__device__ inline uint32_t pack2<LSRM_F16>(float a, float b) {
  return __builtin_bit_cast(uint32_t, f16x2{(_Float16)a, (_Float16)b});
}

// acc + lo(w) + hi(w) for a packed pair w, exact products (v_dot2c_f32_*).
template <int DT>
__device__ inline float sum2(uint32_t w, float acc);
template <>
__device__ inline float sum2<LSRM_BF16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w),
                                         bf16x2{(__bf16)1.0f, (__bf16)1.0f},
                                         acc, false);
}
template <>
__device__ inline float sum2<LSRM_F16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w),
                                f16x2{(_Float16)1.0f, (_Float16)1.0f}, acc,
                                false);
}

// {lo16(lo), lo16(hi)} and {hi16(lo), hi16(hi)} of two packed words
// (one v_perm_b32 each).
__device__ inline uint32_t pair_lo(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
__device__ inline uint32_t pair_hi(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// ------------------------------------------------------------------ MFMA --
// v_mfma_f32_32x32x16_{bf16,f16}: D[32x32] += A[32x16] * B[16x32].
// Lane l supplies A row (l % 32) and B column (l % 32), eight consecutive
// contraction elements each; both operands use the same contraction slots.
// Accumulator register v of lane l holds D[(v/4)*8 + (l/32)*4 + v%4][l%32].
template <int DT>
__device__ inline f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ inline f32x16 mfma32<LSRM_BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
      __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
      0);
}
template <>
__device__ inline f32x16 mfma32<LSRM_F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(
      __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Row (within a 32-row MFMA block) held by accumulator register v of a lane
// in half hb (= lane / 32).
__device__ __host__ constexpr int acc_row(int v, int hb) {
  return (v / 4) * 8 + hb * 4 + (v % 4);
}

// ------------------------------------------------------------ utilities --

__device__ inline int wave_id() { return threadIdx.x >> 6; }
__device__ inline int lane_id() { return threadIdx.x & 63; }

// Largest index j in [lo, hi) with a[j] <= x (a ascending), or lo - 1.
__device__ inline int64_t upper_index(const int32_t* a, int64_t lo,
                                      int64_t hi, int64_t x) {
  int64_t l = lo, h = hi;  // invariant: answer in [l-1, h-1]
  while (l < h) {
    int64_t m = (l + h) >> 1;
    if ((int64_t)a[m] <= x)
      l = m + 1;
    else
      h = m;
  }
  return l - 1;
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Bump allocator over a caller-provided workspace.
struct Carver {
  char* base;
  size_t used;
  size_t cap;
  bool dry = false;  // carve real pointers but launch nothing
  template <typename T>
  T* take(size_t count) {
    used = align_up(used, 256);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
  bool ok() const { return used <= cap; }
};

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace lsrm

#define LSRM_CHECK_LAUNCH()                                  \
  do {                                                       \
    if (hipGetLastError() != hipSuccess) return LSRM_ERR_LAUNCH; \
  } while (0)
