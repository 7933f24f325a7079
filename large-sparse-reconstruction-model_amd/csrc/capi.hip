// C entry points of the selected-attention forward/backward, status strings
// and device queries shared by the launchers.
#include <mutex>

#include "attn.h"

namespace lsrm {

int launch_fwd(int dtype, int d, const AttnArgs& a, hipStream_t st);
int launch_bwd(int dtype, int d, const AttnArgs& a, hipStream_t st);

int device_cu_count() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
        hipSuccess)
      return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

int side_stream(SideStream& out) {
  static std::mutex mu;
  static std::mutex seq[64];
  static hipStream_t streams[64];
  static hipEvent_t forks[64], joins[64];
  static bool made[64] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return LSRM_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(mu);
  if (!made[dev]) {
    hipStream_t s = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return LSRM_ERR_LAUNCH;
    if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
      if (f) (void)hipEventDestroy(f);
      (void)hipStreamDestroy(s);
      return LSRM_ERR_LAUNCH;
    }
    streams[dev] = s;
    forks[dev] = f;
    joins[dev] = j;
    made[dev] = true;
  }
  out = SideStream{streams[dev], forks[dev], joins[dev], &seq[dev]};
  return LSRM_OK;
}

bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) return true;
  return cs != hipStreamCaptureStatusNone;
}

int persistent_grid(const void* kernel, int block, size_t dyn_lds) {
  static std::mutex mu;
  struct Entry {
    const void* fn;
    int dev;
    int per_cu;
  };
  static Entry cache[128];
  static int n_cache = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  const int cus = device_cu_count();
  if (cus <= 0) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n_cache; ++i)
    if (cache[i].fn == kernel && cache[i].dev == dev)
      return cus * cache[i].per_cu;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block,
                                                   dyn_lds) != hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  if (n_cache < 128) cache[n_cache++] = Entry{kernel, dev, per_cu};
  return cus * per_cu;
}

struct AttnWs {
  TilePlan plan;
  RevMap rev;
  RevMap qrev;
  KeyItems items;
  KcPlan kc;
};

// Carves (or sizes, when ws.base is null) the attention workspace and builds
// the plan on the stream.  flags: LSRM_PLAN_BACKWARD adds the backward part,
// LSRM_PLAN_KEY_CENTRIC the key-centric forward part (carved last, so that
// the entry points without flags find the other parts where they expect
// them); head_dim sizes the key-centric partial results.
int attn_plan(Carver& ws, const int32_t* topk, int64_t nq, int64_t nk,
              int64_t hkv, int64_t topk_n, const int32_t* cu_sb,
              const int32_t* cu_blk, int64_t nb, const int32_t* cu_q,
              int64_t batch, int g, int flags, int64_t head_dim, AttnWs& w,
              hipStream_t st) {
  const bool backward = (flags & LSRM_PLAN_BACKWARD) != 0;
  const int tq = ROWS / g;
  int rc = build_tile_plan(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, tq, ws,
                           w.plan, st, true);
  if (rc) return rc;
  if (backward) {
    // dK/dV rows: the run tiles that selected a block, then the queries of
    // grouped tiles that selected it.
    w.rev = RevMap{};
    w.rev.cap = nq * topk_n;
    rc = build_reverse_map(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, nb, true,
                           &w.plan, ws, w.rev, st);
    if (rc) return rc;
    uint8_t* grouped = reinterpret_cast<uint8_t*>(
        ws.take<int32_t>((size_t)((hkv * nq + 3) / 4 > 0 ? (hkv * nq + 3) / 4 : 1)));
    if (ws.base && !ws.dry) {
      if (!ws.ok()) return LSRM_ERR_WORKSPACE;
      rc = mark_grouped_queries(w.plan, hkv, nq, grouped, st);
      if (rc) return rc;
    }
    w.qrev = RevMap{};
    w.qrev.cap = nq * topk_n;
    if (flags & LSRM_PLAN_KEY_CENTRIC) {
      // The key-centric part lists the same queries per block (slot-encoded,
      // in the same order): the map is carved here and derived from that one
      // once it is built.
      Carver carve_only{ws.base, ws.used, ws.cap, true};
      rc = build_reverse_map(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, nb, false,
                             nullptr, carve_only, w.qrev, st, grouped);
      ws.used = carve_only.used;
    } else {
      rc = build_reverse_map(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, nb, false,
                             nullptr, ws, w.qrev, st, grouped);
    }
    if (rc) return rc;
    rc = build_key_items(cu_blk, nb, nk, ws, w.items, st);
    if (rc) return rc;
    if (ws.base && !ws.dry) {
      rc = mark_backward_plan(w.plan.counter, st);
      if (rc) return rc;
    }
  }
  w.kc = KcPlan{};
  if (flags & LSRM_PLAN_KEY_CENTRIC) {
    KcPlan& kc = w.kc;
    const size_t qwords = (size_t)((hkv * nq + 3) / 4 > 0 ? (hkv * nq + 3) / 4 : 1);
    kc.qmark = reinterpret_cast<uint8_t*>(ws.take<int32_t>(qwords));
    if (ws.base && !ws.dry) {
      if (!ws.ok()) return LSRM_ERR_WORKSPACE;
      // every grouped tile goes to the gathered pass: its queries are marked
      rc = mark_grouped_queries(w.plan, hkv, nq, kc.qmark, st);
      if (rc) return rc;
    }
    kc.grev = RevMap{};
    kc.grev.cap = nq * topk_n;
    rc = build_reverse_map(topk, hkv, nq, topk_n, cu_q, batch, cu_sb, nb, false, nullptr,
                           ws, kc.grev, st, kc.qmark, true);
    if (rc) return rc;
    kc_passes(nq, hkv, topk_n, g, head_dim, &kc.n_pass, &kc.pass_heads, &kc.q_span_max);
    rc = build_kc_items(kc.grev, cu_blk, nk, hkv, nb, tq, head_dim, topk_n, ws, kc,
                        w.plan.counter, kc_plan_marker(flags, (int)head_dim), st);
    if (rc) return rc;
    if (backward && ws.base && !ws.dry) {
      rc = derive_query_map(kc.grev, w.qrev, hkv, nb, topk_n, st);
      if (rc) return rc;
    }
    const size_t parts =
        (size_t)((kc.pass_heads > 0 ? kc.pass_heads : hkv) * kc.q_span_max * topk_n * g);
    kc.part_o = ws.take<uint16_t>(parts * (size_t)(head_dim > 0 ? head_dim : 1));
    kc.part_lse = ws.take<float>(parts);
    if (ws.base && !ws.ok()) return LSRM_ERR_WORKSPACE;
  }
  return LSRM_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_attn_args(int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                    int64_t hkv, int64_t head_dim, int64_t topk,
                    int64_t n_blocks, int64_t batch) {
  if (n_q < 0 || n_k < 0 || hq <= 0 || hkv <= 0 || topk <= 0 || n_blocks < 0 ||
      batch <= 0)
    return LSRM_ERR_INVALID_ARG;
  if (hq % hkv != 0) return LSRM_ERR_INVALID_ARG;
  if (dtype != LSRM_BF16 && dtype != LSRM_F16) return LSRM_ERR_UNSUPPORTED;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return LSRM_ERR_UNSUPPORTED;
  if (hq / hkv > 64 || topk > MAXSEL) return LSRM_ERR_UNSUPPORTED;
  if (n_q > INT32_MAX / (topk > 0 ? topk : 1) || n_k > INT32_MAX)
    return LSRM_ERR_UNSUPPORTED;
  // The attention kernels address K and V rows with 32-bit byte offsets.
  if ((uint64_t)n_k * (uint64_t)hkv * (uint64_t)head_dim * 2u >= (1ull << 32))
    return LSRM_ERR_UNSUPPORTED;
  return LSRM_OK;
}

}  // namespace lsrm

using namespace lsrm;

extern "C" const char* lsrm_status_string(int status) {
  switch (status) {
    case LSRM_OK: return "ok";
    case LSRM_ERR_INVALID_ARG: return "invalid argument";
    case LSRM_ERR_UNSUPPORTED: return "unsupported dtype, head_dim, group size or size";
    case LSRM_ERR_WORKSPACE: return "workspace too small";
    case LSRM_ERR_LAUNCH: return "HIP launch or device query failed";
    case LSRM_ERR_SCRATCH:
      return "input larger than the fixed scratch of the allocation-free entry point";
    default: return "unknown status";
  }
}

extern "C" int lsrm_version(void) { return 100; }

extern "C" size_t lsrm_sel_attn_workspace_size2(int64_t n_q, int64_t n_k, int64_t hq,
                                                int64_t hkv, int64_t head_dim, int64_t topk,
                                                int64_t n_blocks, int flags) {
  if (n_q < 0 || n_k < 0 || hq <= 0 || hkv <= 0 || topk <= 0 || n_blocks < 0 ||
      hq % hkv != 0 || (flags & ~(LSRM_PLAN_BACKWARD | LSRM_PLAN_KEY_CENTRIC)) != 0 ||
      ((flags & LSRM_PLAN_KEY_CENTRIC) && head_dim <= 0))
    return 0;
  Carver ws{nullptr, 0, 0};
  AttnWs w{};
  attn_plan(ws, nullptr, n_q, n_k, hkv, topk, nullptr, nullptr, n_blocks,
            nullptr, 1, (int)(hq / hkv), flags, head_dim, w, nullptr);
  return ws.used + 256;
}

extern "C" size_t lsrm_sel_attn_workspace_size(int64_t n_q, int64_t n_k,
                                               int64_t hq, int64_t hkv,
                                               int64_t topk, int64_t n_blocks,
                                               int backward) {
  return lsrm_sel_attn_workspace_size2(n_q, n_k, hq, hkv, 0, topk, n_blocks,
                                       backward ? LSRM_PLAN_BACKWARD : 0);
}

namespace {

// Validates the arguments shared by every attention entry point and fills
// AttnArgs; `plan` builds the device plan, otherwise the workspace must
// already hold the plan lsrm_sel_attn_plan built for the same inputs.
int attn_setup(const void* q, const void* k, const void* v, int dtype,
               int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv,
               int64_t head_dim, const int32_t* topk_idx, int64_t topk,
               const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
               int64_t n_blocks, const int32_t* cu_seqlens_q, int64_t batch,
               float softmax_scale, int flags, bool plan,
               void* workspace, size_t workspace_bytes, hipStream_t st,
               AttnArgs& a) {
  const bool backward = (flags & LSRM_PLAN_BACKWARD) != 0;
  int rc = check_attn_args(dtype, n_q, n_k, hq, hkv, head_dim, topk, n_blocks,
                           batch);
  if (rc) return rc;
  // The backward dK/dV kernel addresses Q and dO rows with 32-bit byte
  // offsets as well.
  if (backward &&
      (uint64_t)n_q * (uint64_t)hq * (uint64_t)head_dim * 2u >= (1ull << 32))
    return LSRM_ERR_UNSUPPORTED;
  if (!q || !k || !v || !topk_idx || !cu_seqblocks || !cu_block_tokens ||
      !cu_seqlens_q || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !(softmax_scale > 0.0f))
    return LSRM_ERR_INVALID_ARG;
  const size_t need = lsrm_sel_attn_workspace_size2(n_q, n_k, hq, hkv, head_dim, topk,
                                                    n_blocks, flags);
  if (need == 0 || workspace_bytes < need || !workspace) return LSRM_ERR_WORKSPACE;
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0,
            workspace_bytes - 256};
  const int g = (int)(hq / hkv);
  AttnWs w{};
  if (plan) {
    rc = attn_plan(ws, topk_idx, n_q, n_k, hkv, topk, cu_seqblocks,
                   cu_block_tokens, n_blocks, cu_seqlens_q, batch, g, flags,
                   head_dim, w, st);
    if (rc) return rc;
  } else {
    // Same carving, no launches: recover the plan built earlier.
    Carver dry{ws.base, 0, ws.cap, true};
    rc = attn_plan(dry, topk_idx, n_q, n_k, hkv, topk, cu_seqblocks,
                   cu_block_tokens, n_blocks, cu_seqlens_q, batch, g, flags,
                   head_dim, w, st);
    if (rc) return rc;
    if (!dry.ok()) return LSRM_ERR_WORKSPACE;
  }
  a = AttnArgs{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.topk = topk_idx;
  a.cu_sb = cu_seqblocks;
  a.cu_blk = cu_block_tokens;
  a.cu_q = cu_seqlens_q;
  a.nb = n_blocks;
  a.batch = batch;
  a.nq = n_q;
  a.nk = n_k;
  a.topk_n = (int)topk;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.g = g;
  a.scale = softmax_scale;
  a.scale_log2 = softmax_scale * 1.44269504f;  // as the reference (kvcentric:125)
  a.plan = w.plan;
  a.rev = w.rev;
  a.qrev = w.qrev;
  a.items = w.items;
  a.kc = w.kc;
  a.kc_marker = kc_plan_marker(flags, (int)head_dim);
  return LSRM_OK;
}

}  // namespace

extern "C" int lsrm_sel_attn_plan2(
    const int32_t* topk_idx, int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv,
    int64_t head_dim, int64_t topk, const int32_t* cu_seqblocks,
    const int32_t* cu_block_tokens, int64_t n_blocks, const int32_t* cu_seqlens_q,
    int64_t batch, int flags, void* workspace, size_t workspace_bytes, void* stream) {
  const bool kc = (flags & LSRM_PLAN_KEY_CENTRIC) != 0;
  int rc = check_attn_args(LSRM_BF16, n_q, n_k, hq, hkv, kc ? head_dim : 64, topk,
                           n_blocks, batch);
  if (rc) return rc;
  if (n_q == 0) return LSRM_OK;
  if (!topk_idx || !cu_seqblocks || !cu_block_tokens || !cu_seqlens_q)
    return LSRM_ERR_INVALID_ARG;
  const size_t need = lsrm_sel_attn_workspace_size2(n_q, n_k, hq, hkv, head_dim, topk,
                                                    n_blocks, flags);
  if (need == 0) return LSRM_ERR_INVALID_ARG;
  if (workspace_bytes < need || !workspace) return LSRM_ERR_WORKSPACE;
  Carver ws{reinterpret_cast<char*>(align_up((size_t)workspace, 256)), 0,
            workspace_bytes - 256};
  AttnWs w{};
  return attn_plan(ws, topk_idx, n_q, n_k, hkv, topk, cu_seqblocks,
                   cu_block_tokens, n_blocks, cu_seqlens_q, batch,
                   (int)(hq / hkv), flags, head_dim, w, (hipStream_t)stream);
}

extern "C" int lsrm_sel_attn_plan(
    const int32_t* topk_idx, int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv,
    int64_t topk, const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
    int64_t n_blocks, const int32_t* cu_seqlens_q, int64_t batch, int backward,
    void* workspace, size_t workspace_bytes, void* stream) {
  return lsrm_sel_attn_plan2(topk_idx, n_q, n_k, hq, hkv, 0, topk, cu_seqblocks,
                             cu_block_tokens, n_blocks, cu_seqlens_q, batch,
                             backward ? LSRM_PLAN_BACKWARD : 0, workspace, workspace_bytes,
                             stream);
}

static int fwd_impl(const void* q, const void* k, const void* v, int dtype,
                    int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv,
                    int64_t head_dim, const int32_t* topk_idx, int64_t topk,
                    const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
                    int64_t n_blocks, const int32_t* cu_seqlens_q,
                    int64_t batch, float softmax_scale, void* out, float* lse,
                    void* workspace, size_t workspace_bytes, void* stream,
                    bool plan, int flags) {
  const int arc = check_attn_args(dtype, n_q, n_k, hq, hkv, head_dim, topk,
                                  n_blocks, batch);
  if (arc || n_q == 0) return arc;
  if (!out || !lse || !aligned16(out)) return LSRM_ERR_INVALID_ARG;
  hipStream_t st = (hipStream_t)stream;
  AttnArgs a;
  int rc = attn_setup(q, k, v, dtype, n_q, n_k, hq, hkv, head_dim, topk_idx,
                      topk, cu_seqblocks, cu_block_tokens, n_blocks,
                      cu_seqlens_q, batch, softmax_scale, flags, plan,
                      workspace, workspace_bytes, st, a);
  if (rc) return rc;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  return launch_fwd(dtype, (int)head_dim, a, st);
}

extern "C" int lsrm_sel_attn_fwd(
    const void* q, const void* k, const void* v, int dtype, int64_t n_q,
    int64_t n_k, int64_t hq, int64_t hkv, int64_t head_dim,
    const int32_t* topk_idx, int64_t topk, const int32_t* cu_seqblocks,
    const int32_t* cu_block_tokens, int64_t n_blocks,
    const int32_t* cu_seqlens_q, int64_t batch, float softmax_scale, void* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_impl(q, k, v, dtype, n_q, n_k, hq, hkv, head_dim, topk_idx, topk,
                  cu_seqblocks, cu_block_tokens, n_blocks, cu_seqlens_q, batch,
                  softmax_scale, out, lse, workspace, workspace_bytes, stream,
                  true, 0);
}

extern "C" int lsrm_sel_attn_fwd_run(
    const void* q, const void* k, const void* v, int dtype, int64_t n_q,
    int64_t n_k, int64_t hq, int64_t hkv, int64_t head_dim,
    const int32_t* topk_idx, int64_t topk, const int32_t* cu_seqblocks,
    const int32_t* cu_block_tokens, int64_t n_blocks,
    const int32_t* cu_seqlens_q, int64_t batch, float softmax_scale, void* out,
    float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  return fwd_impl(q, k, v, dtype, n_q, n_k, hq, hkv, head_dim, topk_idx, topk,
                  cu_seqblocks, cu_block_tokens, n_blocks, cu_seqlens_q, batch,
                  softmax_scale, out, lse, workspace, workspace_bytes, stream,
                  false, 0);
}

extern "C" int lsrm_sel_attn_fwd_run2(
    const void* q, const void* k, const void* v, int dtype, int64_t n_q,
    int64_t n_k, int64_t hq, int64_t hkv, int64_t head_dim,
    const int32_t* topk_idx, int64_t topk, const int32_t* cu_seqblocks,
    const int32_t* cu_block_tokens, int64_t n_blocks,
    const int32_t* cu_seqlens_q, int64_t batch, float softmax_scale, void* out,
    float* lse, void* workspace, size_t workspace_bytes, int flags, void* stream) {
  if ((flags & ~(LSRM_PLAN_BACKWARD | LSRM_PLAN_KEY_CENTRIC)) != 0)
    return LSRM_ERR_INVALID_ARG;
  return fwd_impl(q, k, v, dtype, n_q, n_k, hq, hkv, head_dim, topk_idx, topk,
                  cu_seqblocks, cu_block_tokens, n_blocks, cu_seqlens_q, batch,
                  softmax_scale, out, lse, workspace, workspace_bytes, stream,
                  false, flags);
}

static int bwd_impl(const void* dout, const void* q, const void* k,
                    const void* v, const void* out, const float* lse,
                    int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                    int64_t hkv, int64_t head_dim, const int32_t* topk_idx,
                    int64_t topk, const int32_t* cu_seqblocks,
                    const int32_t* cu_block_tokens, int64_t n_blocks,
                    const int32_t* cu_seqlens_q, int64_t batch,
                    float softmax_scale, void* dq, void* dk, void* dv,
                    float* delta, void* workspace, size_t workspace_bytes,
                    void* stream, bool plan, int flags = LSRM_PLAN_BACKWARD) {
  const int arc = check_attn_args(dtype, n_q, n_k, hq, hkv, head_dim, topk,
                                  n_blocks, batch);
  if (arc || n_q == 0) return arc;
  if (!dout || !out || !lse || !dq || !dk || !dv || !delta ||
      !aligned16(dout) || !aligned16(out) || !aligned16(dq) || !aligned16(dk) ||
      !aligned16(dv))
    return LSRM_ERR_INVALID_ARG;
  hipStream_t st = (hipStream_t)stream;
  AttnArgs a;
  int rc = attn_setup(q, k, v, dtype, n_q, n_k, hq, hkv, head_dim, topk_idx,
                      topk, cu_seqblocks, cu_block_tokens, n_blocks,
                      cu_seqlens_q, batch, softmax_scale, flags | LSRM_PLAN_BACKWARD, plan,
                      workspace, workspace_bytes, st, a);
  if (rc) return rc;
  a.o = static_cast<const uint16_t*>(out);
  a.dout = static_cast<const uint16_t*>(dout);
  a.lse_in = lse;
  a.out = static_cast<uint16_t*>(dq);
  a.lse = delta;
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  return launch_bwd(dtype, (int)head_dim, a, st);
}

extern "C" int lsrm_sel_attn_bwd(
    const void* dout, const void* q, const void* k, const void* v,
    const void* out, const float* lse, int dtype, int64_t n_q, int64_t n_k,
    int64_t hq, int64_t hkv, int64_t head_dim, const int32_t* topk_idx,
    int64_t topk, const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
    int64_t n_blocks, const int32_t* cu_seqlens_q, int64_t batch,
    float softmax_scale, void* dq, void* dk, void* dv, float* delta,
    void* workspace, size_t workspace_bytes, void* stream) {
  return bwd_impl(dout, q, k, v, out, lse, dtype, n_q, n_k, hq, hkv, head_dim,
                  topk_idx, topk, cu_seqblocks, cu_block_tokens, n_blocks,
                  cu_seqlens_q, batch, softmax_scale, dq, dk, dv, delta,
                  workspace, workspace_bytes, stream, true);
}

extern "C" int lsrm_sel_attn_bwd_run(
    const void* dout, const void* q, const void* k, const void* v,
    const void* out, const float* lse, int dtype, int64_t n_q, int64_t n_k,
    int64_t hq, int64_t hkv, int64_t head_dim, const int32_t* topk_idx,
    int64_t topk, const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
    int64_t n_blocks, const int32_t* cu_seqlens_q, int64_t batch,
    float softmax_scale, void* dq, void* dk, void* dv, float* delta,
    void* workspace, size_t workspace_bytes, void* stream) {
  return bwd_impl(dout, q, k, v, out, lse, dtype, n_q, n_k, hq, hkv, head_dim,
                  topk_idx, topk, cu_seqblocks, cu_block_tokens, n_blocks,
                  cu_seqlens_q, batch, softmax_scale, dq, dk, dv, delta,
                  workspace, workspace_bytes, stream, false);
}

extern "C" int lsrm_sel_attn_bwd_run2(
    const void* dout, const void* q, const void* k, const void* v,
    const void* out, const float* lse, int dtype, int64_t n_q, int64_t n_k,
    int64_t hq, int64_t hkv, int64_t head_dim, const int32_t* topk_idx,
    int64_t topk, const int32_t* cu_seqblocks, const int32_t* cu_block_tokens,
    int64_t n_blocks, const int32_t* cu_seqlens_q, int64_t batch,
    float softmax_scale, void* dq, void* dk, void* dv, float* delta,
    void* workspace, size_t workspace_bytes, int flags, void* stream) {
  if ((flags & ~(LSRM_PLAN_BACKWARD | LSRM_PLAN_KEY_CENTRIC)) != 0 ||
      !(flags & LSRM_PLAN_BACKWARD))
    return LSRM_ERR_INVALID_ARG;
  return bwd_impl(dout, q, k, v, out, lse, dtype, n_q, n_k, hq, hkv, head_dim,
                  topk_idx, topk, cu_seqblocks, cu_block_tokens, n_blocks,
                  cu_seqlens_q, batch, softmax_scale, dq, dk, dv, delta,
                  workspace, workspace_bytes, stream, false, flags);
}
