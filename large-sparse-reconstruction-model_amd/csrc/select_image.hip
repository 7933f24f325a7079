// 3D-aware per-token selection on the image side (the use_3d_aware_attn
// branches of build_image_to_image_attn and build_volume_to_image_attn,
// misc/sparse_utils.py:690-898 and 991-1200, with from_imcoords_to_points,
// 653-688, and compute_block_topk_dist_chunked, 16-57) on gfx950.
//
//   image_points_kernel : per image token, the dense surface point of its
//     patch with the largest mask value (the first among equal maxima).
//   image_candidates_kernel : one lane per query token.  For every image of
//     the token's batch element: project the token's point into the image
//     (fp32, each product and sum rounded on its own, in a fixed order),
//     keep the `win` kept blocks whose centres are nearest in block
//     coordinates (fp32 squared distance, lower block number first on
//     ties), then each candidate's exact squared 3D distance to the
//     nearest valid dense point under it (fp64: fp32 differences, squares
//     and their sum are exact there; an invalid point counts max_dist).
//     Writes the candidates of all images in (image, window rank) order.
//   image_select_kernel : one wave per token row.  The min(topk, C)
//     candidates with the smallest (distance, position) are written in
//     position order, block ids already offset per image, -1 padded, once
//     per kv head.
#include "common.h"
#include "plan.h"

namespace lsrm {

constexpr int IMG_CAM = 18;   // floats per camera record
constexpr int IMG_META = 4;   // ints per image record: kept, kept offset, column offset, id offset
constexpr int IMG_MAXWIN = 16;
constexpr int IMG_MAXCOLS = 1024;

__global__ __launch_bounds__(256) void image_points_kernel(
    const int32_t* __restrict__ coords, int64_t n, const float* __restrict__ sp,
    const float* __restrict__ mk, int64_t batch, int64_t n_img, int s, int patch_res,
    float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t* c = coords + i * 4;
  const int ps = s / patch_res;
  const int64_t b = c[0], m = c[1], r = c[2], col = c[3];
  float* o = out + i * 3;
  if (b < 0 || b >= batch || m < 0 || m >= n_img || r < 0 || r >= patch_res || col < 0 ||
      col >= patch_res || ps <= 0) {
    o[0] = o[1] = o[2] = __builtin_nanf("");
    return;
  }
  const int64_t base = ((b * n_img + m) * s + r * ps) * s + col * ps;
  float best = 0.0f;
  int bk = 0;
  for (int k = 0; k < ps * ps; ++k) {
    const float v = mk[base + (int64_t)(k / ps) * s + (k % ps)];
    // first maximum; a NaN counts as larger than every number (numpy argmax)
    const bool take = k == 0 || (best == best && (v > best || v != v));
    if (take) {
      best = v;
      bk = k;
    }
  }
  const float* p = sp + (base + (int64_t)(bk / ps) * s + (bk % ps)) * 3;
  o[0] = p[0];
  o[1] = p[1];
  o[2] = p[2];
}

// fp32 operations rounded one by one (no contraction into fused forms).
__device__ inline float fmul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ inline float fadd_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ inline float fsub_rn(float a, float b) { return __fsub_rn(a, b); }

__global__ __launch_bounds__(256) void image_candidates_kernel(
    const float* __restrict__ qpts, int64_t nq, const int32_t* __restrict__ cu_q,
    int64_t batch, int64_t n_img, const float* __restrict__ cam,
    const int32_t* __restrict__ meta, const int32_t* __restrict__ kept, int bw, int s,
    int ibs, const float* __restrict__ sp, const float* __restrict__ dmask, int win,
    float max_dist, int cols, double* __restrict__ cand_d, int32_t* __restrict__ cand_id) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nq) return;
  double* rd = cand_d + i * cols;
  int32_t* ri = cand_id + i * cols;
  for (int j = 0; j < cols; ++j) {
    rd[j] = __builtin_inf();
    ri[j] = -1;
  }
  if (batch <= 0 || i < cu_q[0] || i >= cu_q[batch]) return;
  const int b = batch_of(cu_q, batch, i);
  const float x = qpts[i * 3 + 0], y = qpts[i * 3 + 1], z = qpts[i * 3 + 2];
  const double px = x, py = y, pz = z;
  const double md2 = (double)max_dist * (double)max_dist;
  for (int m = 0; m < n_img; ++m) {
    const int64_t im = (int64_t)b * n_img + m;
    const int32_t* mt = meta + im * IMG_META;
    const int nsel = mt[0], soff = mt[1], coff = mt[2], idoff = mt[3];
    if (nsel <= 0) continue;
    const float* cr = cam + im * IMG_CAM;
    float pc[3];
#pragma unroll
    for (int r = 0; r < 3; ++r)
      pc[r] = fadd_rn(fadd_rn(fadd_rn(fmul_rn(x, cr[4 * r]), fmul_rn(y, cr[4 * r + 1])),
                              fmul_rn(z, cr[4 * r + 2])),
                      cr[4 * r + 3]);
    const float nz = -pc[2];
    const float den = (nz > 1e-6f || nz != nz) ? nz : 1e-6f;  // max(-p2, 1e-6), NaN kept
    float u = __fdiv_rn(pc[0], den);
    float v = __fdiv_rn(-pc[1], den);
    const float t = cr[12];
    u = fmul_rn(0.5f, fadd_rn(__fdiv_rn(u, t), 1.0f));
    v = fmul_rn(0.5f, fadd_rn(__fdiv_rn(v, t), 1.0f));
    const float sm1 = (float)(s - 1);
    float pxl, pyl;
    if (cr[13] != 0.0f) {
      pxl = fmul_rn(__fdiv_rn(fsub_rn(fmul_rn(u, cr[14]), cr[15]), cr[17]), sm1);
      pyl = fmul_rn(__fdiv_rn(fsub_rn(fmul_rn(v, cr[14]), cr[16]), cr[17]), sm1);
    } else {
      pxl = fmul_rn(u, sm1);
      pyl = fmul_rn(v, sm1);
    }
    const float bxf = __fdiv_rn(pxl, (float)ibs), byf = __fdiv_rn(pyl, (float)ibs);
    // window: the `win` nearest kept blocks, (fp32 d2, block number) ascending
    float wd[IMG_MAXWIN];
    int wj[IMG_MAXWIN];
#pragma unroll
    for (int k = 0; k < IMG_MAXWIN; ++k) {
      wd[k] = __builtin_inf();
      wj[k] = 0x7fffffff;
    }
    for (int j = 0; j < nsel; ++j) {
      const int blk = kept[soff + j];
      const float cx = (float)(blk % bw) + 0.5f, cy = (float)(blk / bw) + 0.5f;
      const float dx = fsub_rn(bxf, cx), dy = fsub_rn(byf, cy);
      float d = fadd_rn(fmul_rn(dx, dx), fmul_rn(dy, dy));
      if (d != d) d = __builtin_inf();
      if (d < wd[win - 1] || (d == wd[win - 1] && j < wj[win - 1])) {
        // insertion; candidates arrive in increasing j, so an equal distance
        // already listed stays in front
#pragma unroll
        for (int k = IMG_MAXWIN - 1; k >= 0; --k) {
          if (k >= win) continue;
          const int kp = k > 0 ? k - 1 : 0;
          const bool prev_after = k > 0 && (wd[kp] > d || (wd[kp] == d && wj[kp] > j));
          const bool here_after = wd[k] > d || (wd[k] == d && wj[k] > j);
          if (here_after) {
            wd[k] = prev_after ? wd[kp] : d;
            wj[k] = prev_after ? wj[kp] : j;
          }
        }
      }
    }
    const int nw = nsel < win ? nsel : win;
    const int64_t img_base = im * (int64_t)s * s;
#pragma unroll
    for (int k = 0; k < IMG_MAXWIN; ++k) {
      if (k >= nw) continue;
      const int blk = kept[soff + wj[k]];
      const int by = blk / bw, bx = blk % bw;
      double best = __builtin_inf();
      for (int a = 0; a < ibs; ++a) {
        const int64_t row = img_base + (int64_t)(by * ibs + a) * s + bx * ibs;
        for (int e = 0; e < ibs; ++e) {
          double d2;
          if (dmask[row + e] > 0.2f) {
            const float* q = sp + (row + e) * 3;
            const double ex = (double)q[0] - px, ey = (double)q[1] - py, ez = (double)q[2] - pz;
            d2 = ex * ex;
            d2 = d2 + ey * ey;
            d2 = d2 + ez * ez;
            if (d2 != d2) d2 = __builtin_inf();
          } else {
            d2 = md2;
          }
          best = d2 < best ? d2 : best;
        }
      }
      rd[coff + k] = best;
      ri[coff + k] = idoff + wj[k];
    }
  }
}

// One wave per token row: candidate p of the row is kept when fewer than
// k_out candidates precede it in (distance, position) order; kept
// candidates are written in position order.  Every lane reads the row's
// candidates in the same order (one cached line serves the wave).
__global__ __launch_bounds__(256) void image_select_kernel(
    const double* __restrict__ cand_d, const int32_t* __restrict__ cand_id, int64_t nq,
    const int32_t* __restrict__ cu_q, int64_t batch, const int32_t* __restrict__ cols_b,
    int cols, int topk, int hkv, int32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  if (t >= nq) return;  // whole wave
  int c_b = 0;
  if (batch > 0 && t >= cu_q[0] && t < cu_q[batch]) c_b = cols_b[batch_of(cu_q, batch, t)];
  c_b = c_b < cols ? (c_b > 0 ? c_b : 0) : cols;
  const int k_out = c_b < topk ? c_b : topk;
  const double* rd = cand_d + t * cols;
  const int32_t* ri = cand_id + t * cols;
  int base = 0;
  for (int p0 = 0; p0 < c_b; p0 += 64) {
    const int p = p0 + lane;
    bool keep = false;
    if (p < c_b) {
      const double dp = rd[p];
      int rank = 0;
      for (int q = 0; q < c_b; ++q) {
        const double dq = rd[q];
        rank += (dq < dp || (dq == dp && q < p)) ? 1 : 0;
      }
      keep = rank < k_out;
    }
    const unsigned long long m = __ballot(keep);
    if (keep) {
      const int slot = base + __popcll(m & ((1ull << lane) - 1ull));
      const int id = ri[p];
      for (int h = 0; h < hkv; ++h) out[((int64_t)h * nq + t) * topk + slot] = id;
    }
    base += __popcll(m);
  }
  for (int slot = k_out + lane; slot < topk; slot += 64)
    for (int h = 0; h < hkv; ++h) out[((int64_t)h * nq + t) * topk + slot] = -1;
}

}  // namespace lsrm

using namespace lsrm;

extern "C" int lsrm_image_points(const int32_t* imcoords, int64_t n_tokens,
                                 const float* surface_points, const float* masks, int64_t batch,
                                 int64_t n_images, int64_t dense_res, int64_t patch_res,
                                 float* points, void* stream) {
  if (n_tokens < 0 || batch <= 0 || n_images <= 0 || dense_res <= 0 || patch_res <= 0 ||
      dense_res < patch_res || (n_tokens > 0 && (!imcoords || !surface_points || !masks || !points)))
    return LSRM_ERR_INVALID_ARG;
  if (n_tokens == 0) return LSRM_OK;
  hipLaunchKernelGGL(image_points_kernel, dim3((unsigned)((n_tokens + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, imcoords, n_tokens, surface_points, masks, batch,
                     n_images, (int)dense_res, (int)patch_res, points);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}

extern "C" size_t lsrm_image_block_rank_workspace_size(int64_t n_q, int64_t cols) {
  if (n_q < 0 || cols < 0) return 0;
  return align_up((size_t)(n_q * cols) * sizeof(double), 256) +
         (size_t)(n_q * cols) * sizeof(int32_t) + 512;
}

extern "C" int lsrm_image_block_rank(
    const float* qpoints, int64_t n_q, const int32_t* cu_seqlens_q, int64_t batch,
    int64_t n_images, const float* cameras, const int32_t* image_meta,
    const int32_t* kept_blocks, const int32_t* cols_per_batch, int64_t cols, int64_t blocks_w,
    int64_t dense_res, int64_t ibs, const float* surface_points, const float* dense_masks,
    int64_t win, int64_t topk, float max_dist, int64_t hkv, int32_t* block_topk,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (n_q < 0 || batch <= 0 || n_images <= 0 || cols < 0 || blocks_w <= 0 || dense_res <= 0 ||
      ibs <= 0 || win <= 0 || topk <= 0 || hkv <= 0 || !cu_seqlens_q || !cameras ||
      !image_meta || !cols_per_batch ||
      (n_q > 0 && (!qpoints || !surface_points || !dense_masks || !block_topk)))
    return LSRM_ERR_INVALID_ARG;
  if (win > IMG_MAXWIN || cols > IMG_MAXCOLS) return LSRM_ERR_UNSUPPORTED;
  if (n_q == 0) return LSRM_OK;
  const size_t need = lsrm_image_block_rank_workspace_size(n_q, cols);
  if (!workspace || workspace_bytes < need) return LSRM_ERR_WORKSPACE;
  const int c = cols > 0 ? (int)cols : 1;
  char* ws = reinterpret_cast<char*>(align_up((size_t)workspace, 256));
  double* cand_d = reinterpret_cast<double*>(ws);
  int32_t* cand_id = reinterpret_cast<int32_t*>(
      ws + align_up((size_t)(n_q * cols) * sizeof(double), 256));
  hipStream_t st = (hipStream_t)stream;
  if (cols > 0) {
    hipLaunchKernelGGL(image_candidates_kernel, dim3((unsigned)((n_q + 255) / 256)), dim3(256),
                       0, st, qpoints, n_q, cu_seqlens_q, batch, n_images, cameras, image_meta,
                       kept_blocks, (int)blocks_w, (int)dense_res, (int)ibs, surface_points,
                       dense_masks, (int)win, max_dist, c, cand_d, cand_id);
    LSRM_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(image_select_kernel, dim3((unsigned)((n_q + 3) / 4)), dim3(256), 0, st,
                     cand_d, cand_id, n_q, cu_seqlens_q, batch, cols_per_batch,
                     (int)cols, (int)topk, (int)hkv, block_topk);
  LSRM_CHECK_LAUNCH();
  return LSRM_OK;
}
