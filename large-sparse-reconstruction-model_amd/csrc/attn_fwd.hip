// Selected-block attention forward on bf16/fp16 MFMA (gfx950).
//
// Semantics follow forward_kernel_varblock
// (sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:55-247): for
// every query row, an online softmax in base 2 (scale folded into the
// exponent) over the tokens of its selected blocks, P rounded to the input
// type before P.V, O = acc / l and LSE = m + log2(l) in log2 units.
//
// Design: a persistent grid pulls query tiles (up to 128 rows of one kv head
// that share one selection) from an atomic queue.  Each wave owns 32 rows.
// The tile's key stream (the concatenated token ranges of its selected
// blocks) is staged through LDS 64 keys at a time:
//   * K and V tiles are copied global -> LDS by the load unit
//     (global_load_lds_dwordx4, no register staging), both row-major with a
//     16-byte-chunk XOR swizzle that keeps the MFMA operand reads free of
//     bank conflicts;
//   * scores are computed transposed, S^T = K Q^T (32x32x16 MFMA, K from LDS,
//     Q in registers), so that a lane owns one query row through the whole
//     softmax (base 2, scale folded into one FMA per score); O^T = V^T P^T
//     takes its V^T operand straight from the row-major V tile with
//     ds_read_b64_tr_b16 and P^T from the score registers, so V is never
//     transposed in memory;
//   * the loop is a three-stage software pipeline: step t issues the score
//     MFMAs of tile t+1 and the P.V MFMAs of tile t-1 (alternating) next to
//     the softmax arithmetic of tile t, in a fixed order of slots (one MFMA,
//     then two scores' worth of softmax) so that matrix and vector work
//     co-issue inside one wave; K and V live in four-slot LDS rings whose
//     copies are issued two or three steps before they are read, one
//     barrier per tile; only the steps that can hold the stream's last
//     (partial) key tile carry the tail mask;
//   * the softmax reference is the row maximum of the first key tile and is
//     not updated afterwards (no per-tile maximum, no rescaling); a tile
//     whose row sums leave the safe range is recomputed with the exact
//     online maximum.
#include <type_traits>

#include "attn.h"

namespace lsrm {

// Softmax reference: p = exp2(scale*log2(e)*s - m_run) with a per-row
// reference m_run (log2 units) that is the row maximum after the first tile
// and afterwards only moves when a row maximum exceeds it by more than
// RESCALE_LOG2 (so p <= 2^8); the final O = acc / l is the same for any
// reference.
constexpr float RESCALE_LOG2 = 8.0f;

// Maximum of a lane's 32 scores (a v_maximum3 tree), combined with the lane
// holding the other 16 keys of the same row (v_permlane32_swap).
__device__ inline float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ inline float row_max(const f32x16* sc) {
  float t[11];
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const int a = 3 * i, b = 3 * i + 1, c = 3 * i + 2;
    t[i] = max3f(sc[a >> 4][a & 15], sc[b >> 4][b & 15], sc[c >> 4][c & 15]);
  }
  t[10] = __builtin_elementwise_maximum(sc[1][14], sc[1][15]);
  const float m = max3f(max3f(t[0], t[1], t[2]), max3f(t[3], t[4], t[5]),
                        max3f(t[6], t[7], max3f(t[8], t[9], t[10])));
  const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, m),
                                                   __builtin_bit_cast(unsigned, m),
                                                   false, false);
  return __builtin_elementwise_maximum(__builtin_bit_cast(float, (unsigned)sw[0]),
                                       __builtin_bit_cast(float, (unsigned)sw[1]));
}

// MODE 0 (FWD_RUN): the run tiles of the plan (every row of a tile shares
// one key stream).  MODE 1 (FWD_UNION): the grouped tiles (see build_union),
// run with per-row key masks; a key-centric plan does not launch it (its
// grouped tiles' rows run as gathered tiles).  MODE 2 (FWD_GATHER): gathered
// tiles of a key-centric plan
// -- the queries that listed one block, attending that block alone, each row
// written as a partial result (O over the block normalised by its own sum,
// in the input type, and its log2 LSE) for kc_merge_kernel.  Separate
// instantiations, so the run-tile kernel carries none of the other modes'
// code or state.
constexpr int FWD_RUN = 0, FWD_UNION = 1, FWD_GATHER = 2;

template <int DT, int D, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sel_attn_fwd_kernel(AttnArgs a) {
  constexpr bool UNION = MODE == FWD_UNION;
  constexpr bool GATHER = MODE == FWD_GATHER;
  using G = KvTile<D>;
  constexpr int NS = D / 16;  // MFMA k-steps over the head dim
  constexpr int ND = D / 32;  // 32-wide output blocks over the head dim
  __shared__ __align__(1024) char sK[4][G::BYTES];
  __shared__ __align__(1024) char sV[4][G::BYTES];
  __shared__ SelLds sel;
  __shared__ typename std::conditional<UNION, UnionLds, int>::type ul;
  // Run tiles whose key stream has at most KMAP_KEYS positions: the token
  // of every position (build_token_map), read by the copy groups that cross
  // block boundaries.
  __shared__ int s_tokmap[MODE == FWD_RUN ? KMAP_KEYS : 1];
  __shared__ int s_slot;

  const int tid = threadIdx.x, lane = tid & 63, wv = uniform(tid >> 6);
  const int hb = lane >> 5, l32 = lane & 31;
  const int32_t* head_off =
      GATHER ? a.kc.fitem_off : (UNION ? a.plan.ghead_off : a.plan.head_off);
  const int2* tiles = UNION ? a.plan.gtiles : a.plan.tiles;
  int32_t* queue = a.plan.counter + (GATHER ? KC_QUEUE_SLOT : (UNION ? 4 : 0));
  if constexpr (GATHER) {
    if (!kc_plan_ok(a)) return;  // no key-centric part for this run: read nothing
  }
  const int total = head_off[a.hkv];
  // An empty queue: leave it untouched (no fetch, so nothing to reset).
  if (total == 0) return;

  // Loader geometry: load j of this wave covers keys (wv*LPW + j)*KPL + ...
  int ld_key[G::LPW], ld_byte[G::LPW];
#pragma unroll
  for (int j = 0; j < G::LPW; ++j) {
    ld_key[j] = (wv * G::LPW + j) * G::KPL + lane / G::CH;
    ld_byte[j] = (((lane % G::CH) ^ G::swz(ld_key[j])) << 4);
  }
  // Bytes between consecutive tokens; K and V are below 4 GiB (checked by
  // the host), so token offsets fit 32 bits.
  const uint32_t row_bytes = (uint32_t)a.hkv * D * 2;
  const int ld_row = lane / G::CH;  // row of this lane within a load group
  uint32_t ld_lane_off[G::LPW];
#pragma unroll
  for (int j = 0; j < G::LPW; ++j) ld_lane_off[j] = (uint32_t)ld_row * row_bytes + ld_byte[j];

  for (;;) {
    const int w = uniform(fetch_work(queue, &s_slot));
    if (w >= total) break;
    const int h = head_of(head_off, a.hkv, w);
    int q0, qn, gblk = 0, ge0 = 0;
    if constexpr (GATHER) {
      const int4 it = a.kc.fitems[(int64_t)h * a.kc.fitem_cap + (w - head_off[h])];
      gblk = it.x;
      ge0 = it.y;
      q0 = 0;
      qn = it.z;
    } else {
      const int2 tile = tiles[(int64_t)h * a.nq + (w - head_off[h])];
      q0 = tile.x;
      qn = tile.y;
    }
    const int rows = qn * a.g;
    // Passes over the tile: umode 0 -- one key stream shared by every row
    // (a run tile); umode 1 -- a grouped tile run once over the union of
    // its rows' blocks, each row masked to the blocks it selected; umode 2
    // -- a grouped tile run once per run of identical rows, the other rows
    // masked off.  All modes take the fast pass first (modes 1 and 2 with
    // their key masks), falling back to the exact online-maximum pass.
    int umode = 0, n_pass = 1;
    if constexpr (UNION) {
      build_union(a, h, q0, qn, sel, ul);
      umode = ul.ok ? 1 : 2;
      n_pass = ul.ok ? 1 : ul.n_runs;
    } else if constexpr (GATHER) {
      load_block(a, gblk, sel);
    } else {
      load_selection(a, h, q0, sel);
    }
    for (int pass = 0; pass < n_pass; ++pass) {
    int q_lo = 0, q_hi = qn;  // the pass writes the rows of queries [q_lo, q_hi)
    if constexpr (UNION) {
      if (umode == 2) {
        q_lo = ul.run_start[pass];
        q_hi = ul.run_start[pass + 1];
        load_selection(a, h, q0 + q_lo, sel);
      }
    }
    const int nkeys = uniform(sel.cum[sel.n]);
    const int ntiles = (nkeys + KT - 1) / KT;
    const int t_safe = uniform(sel.n > 0 ? sel.tok[0] : 0);  // in-bounds filler token
    const bool use_map = MODE == FWD_RUN && nkeys <= KMAP_KEYS;
    if constexpr (MODE == FWD_RUN) {
      if (use_map) build_token_map(sel, s_tokmap, wv, lane);
    }

    // This wave's row and its Q operand (B of S^T = K Q^T).
    const int r = wv * 32 + l32;
    const bool row_ok = r < rows;
    const int qr = row_ok ? r / a.g : 0;  // the row's query within the tile
    const bool row_in_pass = row_ok && qr >= q_lo && qr < q_hi;
    const bool wave_on = uniform(wv * 32 < q_hi * a.g && wv * 32 + 32 > q_lo * a.g) != 0;
    // Gathered tiles: row r is listing ge0 + r / g of the block's segment,
    // which stores query * topk + slot.
    int64_t qi, gslot = 0;
    if constexpr (GATHER) {
      const int64_t lv = a.kc.grev.rev[(int64_t)h * a.kc.grev.cap + ge0 + (row_ok ? r / a.g : 0)];
      qi = lv / a.topk_n;
      gslot = lv - qi * a.topk_n;
    } else {
      qi = q0 + (row_ok ? r / a.g : 0);
    }
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

    const char* kbase = reinterpret_cast<const char*>(a.k + (int64_t)h * D);
    const char* vbase = reinterpret_cast<const char*>(a.v + (int64_t)h * D);
    // The lane-dependent parts of the LDS operand addresses (the 32-key
    // block, 16-key half and ring slot are compile-time offsets): the K row
    // block read of head-dim step s, and the two transposed V reads (rows
    // k0, k0 + 8) of output block db.  Pinned in registers so the reads
    // take them as base plus an immediate offset.
    uint32_t kl_off[NS], vl_off[ND][2];
    {
      const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
      for (int s2 = 0; s2 < NS; ++s2) {
        kl_off[s2] = (uint32_t)G::off(l32, 2 * s2 + hb);
        asm volatile("" : "+v"(kl_off[s2]));
      }
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
        const int k0 = hb * 4 + (gi >> 2);
        const int cb = dcol >> 3, half = (dcol & 4) * 2;
        vl_off[db][0] = (uint32_t)(G::off(k0, cb) + half);
        vl_off[db][1] = (uint32_t)(G::off(k0 + 8, cb) + half);
        asm volatile("" : "+v"(vl_off[db][0]), "+v"(vl_off[db][1]));
      }
    }

    // Scalar cursors of the K copies (three tiles ahead, one per load
    // group); the V copies (two tiles ahead) reuse the K offsets of the
    // previous tile.
    GroupCursor cur[G::LPW];
#pragma unroll
    for (int j = 0; j < G::LPW; ++j) group_init(sel, cur[j], use_map);
    int ld_tile = 0;  // next tile whose K copies are issued
    uint32_t koff[G::LPW], voff[G::LPW];
    // Byte offsets of the rows of tile ld_tile for this lane's loads.
    auto advance = [&](uint32_t* off) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) {
        const int P = ld_tile * KT + (wv * G::LPW + j) * G::KPL;
        off[j] = group_offset<G::KPL>(sel, cur[j], P, nkeys, t_safe, row_bytes, ld_row,
                                      ld_lane_off[j], ld_byte[j], use_map ? s_tokmap : nullptr);
      }
      ++ld_tile;
    };
    auto voff_keep = [&](const uint32_t* off) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) voff[j] = off[j];
    };
    auto load_tile = [&](const char* base, const uint32_t* off, char* dst) __attribute__((always_inline)) {
      const uint32_t d0 = lds_addr(dst) + wv * G::LPW * 1024;
#pragma unroll
      for (int j = 0; j < G::LPW; ++j)
        copy16_to_lds(base, off[j], d0 + j * 1024);
    };

    f32x16 oacc[ND];
    // Online softmax state of this lane's row: the reference m_run (log2
    // units) and the partial row sum.
    float m_run = 0.0f, l_run = 0.0f;
    uint64_t km = ~0ull;  // grouped tiles: keys of the current tile the row attends

    auto scores = [&](const char* ks, f32x16* sacc) __attribute__((always_inline)) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[blk][v] = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const u32x4 ka = *reinterpret_cast<const u32x4*>(
              ks + G::off(blk * 32 + l32, 2 * s + hb));
          sacc[blk] = mfma32<DT>(ka, qb[s], sacc[blk]);
        }
      }
    };
    // Keys past the stream (last tile only) score -inf.
    auto mask_tail = [&](int kt, f32x16* sc) __attribute__((always_inline)) {
      const int kb0 = kt * KT;
      if (kb0 + KT > nkeys) {
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (kb0 + blk * 32 + acc_row(v, hb) >= nkeys) sc[blk][v] = -__builtin_inf();
      }
    };
    // Grouped passes: keys a row does not attend score -inf.  umode 1: the
    // 64-bit mask of tile kt's positions covered by union segments the row's
    // query selected (segments are walked with a cursor, `useg`); umode 2:
    // all or nothing by run membership.
    int useg = 0;
    auto key_mask = [&](int kt) __attribute__((always_inline)) {
      uint64_t m = ~0ull;
      if constexpr (UNION) {
      if (umode == 1) {
        m = 0ull;
        const int p0 = kt * KT;
        int sg = useg;
        while (sel.cum[sg + 1] <= p0) ++sg;  // stops at the sentinel
        useg = sg;
        for (; sg < sel.n && sel.cum[sg] < p0 + KT; ++sg) {
          const int lo = sel.cum[sg] > p0 ? sel.cum[sg] - p0 : 0;
          const int hi = sel.cum[sg + 1] - p0 < KT ? sel.cum[sg + 1] - p0 : KT;
          const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
          const uint64_t range = upto & ~((1ull << lo) - 1ull);
          if ((ul.seg_q[sg][qr >> 5] >> (qr & 31)) & 1u) m |= range;
        }
      } else {
        m = row_in_pass ? ~0ull : 0ull;
        if (kt * KT + KT > nkeys) {
          const int hi = nkeys - kt * KT;
          m &= hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
        }
      }
      }
      return m;
    };
    auto apply_mask = [&](uint64_t m, f32x16* sc) __attribute__((always_inline)) {
      const uint64_t mh = m >> (hb * 4);  // position of slot v: (v/4)*8 + hb*4 + v%4
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (!((mh >> (blk * 32 + (v / 4) * 8 + (v % 4))) & 1ull)) sc[blk][v] = -__builtin_inf();
    };
    auto mask_keys = [&](int kt, f32x16* sc) __attribute__((always_inline)) {
      if constexpr (UNION) apply_mask(key_mask(kt), sc);
    };

    // Softmax of one score tile against m_run: P packed to the 16-bit type
    // (the MFMA B operand of O^T += V^T P^T) and added to the row sum.
    auto softmax = [&](const f32x16* sc, u32x4 (*pb)[2]) __attribute__((always_inline)) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        float p[16];
#pragma unroll
        for (int v = 0; v < 16; ++v)
          p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v], a.scale_log2, -m_run));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          pb[blk][c] = u32x4{pack2<DT>(p[c * 8 + 0], p[c * 8 + 1]),
                             pack2<DT>(p[c * 8 + 2], p[c * 8 + 3]),
                             pack2<DT>(p[c * 8 + 4], p[c * 8 + 5]),
                             pack2<DT>(p[c * 8 + 6], p[c * 8 + 7])};
#pragma unroll
          for (int e = 0; e < 4; ++e) l_run = sum2<DT>(pb[blk][c][e], l_run);
        }
      }
    };
    // O^T += V^T P^T.  Slot e of lane (hb, row d) holds key
    // blk*32 + c*16 + (e/4)*8 + hb*4 + e%4 (the score layout); the two
    // transposed reads return those keys' column d.
    auto pv = [&](const char* vs, const u32x4 (*pb)[2]) __attribute__((always_inline)) {
      const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
      for (int db = 0; db < ND; ++db) {
        const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;  // 4 d values
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const int k0 = blk * 32 + c * 16 + hb * 4 + (gi >> 2);
            const int cb = dcol >> 3, half = (dcol & 4) * 2;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(vs + G::off(k0, cb) + half));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(vs + G::off(k0 + 8, cb) + half));
            const u32x2 lw = __builtin_bit_cast(u32x2, lo);
            const u32x2 hw = __builtin_bit_cast(u32x2, hi);
            oacc[db] = mfma32<DT>(u32x4{lw[0], lw[1], hw[0], hw[1]}, pb[blk][c], oacc[db]);
          }
      }
    };

    // K operands of one score tile (S^T = K Q^T), read ahead of the MFMAs.
    auto read_k = [&](const char* ks, u32x4 (*ka)[NS]) __attribute__((always_inline)) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int s = 0; s < NS; ++s)
          ka[blk][s] = *reinterpret_cast<const u32x4*>(ks + G::off(blk * 32 + l32, 2 * s + hb));
    };
    // One softmax pair (scores 2j, 2j+1 of a lane's 32) against m_run: two
    // exponentials packed to the 16-bit type and added to the row sum.
    auto softmax_pair = [&](const f32x16* sc, u32x4 (*pb)[2], int j, float negm) __attribute__((always_inline)) {
      const int blk = j >> 3, c = (j >> 2) & 1, e = j & 3, v0 = c * 8 + 2 * e;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0], a.scale_log2, negm));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0 + 1], a.scale_log2, negm));
      pb[blk][c][e] = pack2<DT>(p0, p1);
      l_run = sum2<DT>(pb[blk][c][e], l_run);
    };
    // The fast step's matrix and vector work in a fixed issue order: slot i
    // issues one MFMA -- score MFMAs of tile kt+1 and P.V MFMAs of tile kt-1
    // alternate, so consecutive MFMAs on one accumulator are three slots
    // apart -- followed by its share of the softmax of tile kt, so that the
    // vector ALU works while the matrix core runs.  Each MFMA's operand (a K
    // row block, or the two transposed V reads) is read from LDS two slots
    // ahead: only three operands are live at a time, which keeps the step
    // within the register budget.  Scheduling barriers keep the compiler
    // from regrouping the slots.
    auto fast_body = [&](auto first, const char* ks, const char* vs, const f32x16* sc,
                         f32x16* sn, const u32x4 (*pp)[2], u32x4 (*pc)[2],
                         float negm) __attribute__((always_inline)) {
      constexpr bool FIRST = decltype(first)::value != 0;
      constexpr int NSM = 2 * NS;              // score MFMAs
      constexpr int NPV = FIRST ? 0 : 4 * ND;  // P.V MFMAs
      constexpr int NSLOT = NSM + NPV;
      constexpr int NPAIR = 16;
      constexpr int LA = 2;  // operand reads run LA slots ahead of their MFMA
      // Slot i's MFMA: score and P.V MFMAs alternate (a score MFMA when the
      // step has no P.V work).  kind 0: score MFMA idx (32-key block idx & 1,
      // head-dim step idx >> 1); kind 1: P.V MFMA idx.
      auto kind_of = [](int i) constexpr { return (NPV == 0 || (i & 1) == 0) ? 0 : 1; };
      auto idx_of = [](int i) constexpr { return NPV == 0 ? i : (i >> 1); };
      const int gi = lane & 15, dh = (lane >> 4) & 1;
      auto read_op = [&](int i, u32x4& dst) __attribute__((always_inline)) {
        const int x = idx_of(i);
        if (kind_of(i) == 0) {
          const int blk = x & 1, s = x >> 1;
          // row blk * 32 + l32: the swizzle sees only l32's low bits
          dst = *reinterpret_cast<const u32x4*>(ks + blk * 32 * (D * 2) + kl_off[s]);
        } else {
          const int db = x % ND, bc = x / ND, blk = bc >> 1, c = bc & 1;
          // rows blk * 32 + c * 16 + k0 (+ 8): the swizzle sees only k0's bits
          const int rb = (blk * 32 + c * 16) * (D * 2);
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vs + rb + vl_off[db][0]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vs + rb + vl_off[db][1]));
          const u32x2 lw = __builtin_bit_cast(u32x2, lo);
          const u32x2 hw = __builtin_bit_cast(u32x2, hi);
          dst = u32x4{lw[0], lw[1], hw[0], hw[1]};
        }
      };
      u32x4 op[LA + 1];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < LA && i < NSLOT; ++i) read_op(i, op[i % (LA + 1)]);
#pragma unroll
      for (int i = 0; i < NSLOT; ++i) {
        if (i + LA < NSLOT) read_op(i + LA, op[(i + LA) % (LA + 1)]);
        const int x = idx_of(i);
        if (kind_of(i) == 0) {
          const int blk = x & 1, s = x >> 1;
          if (s == 0) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sn[blk][v] = 0.0f;
          }
          sn[blk] = mfma32<DT>(op[i % (LA + 1)], qb[s], sn[blk]);
        } else {
          const int db = x % ND, bc = x / ND, blk = bc >> 1, c = bc & 1;
          oacc[db] = mfma32<DT>(op[i % (LA + 1)], pp[blk][c], oacc[db]);
        }
#pragma unroll
        for (int j = (i * NPAIR) / NSLOT; j < ((i + 1) * NPAIR) / NSLOT; ++j)
          softmax_pair(sc, pc, j, negm);
        __builtin_amdgcn_sched_barrier(0);
      }
    };

    // Pipeline over key tiles (K and V in four-slot LDS rings).  Step kt
    // copies K(kt+3) and V(kt+2), computes S(kt+1) = K(kt+1) Q^T, adds
    // P(kt-1) V(kt-1) into O and turns S(kt) into P(kt): the step's 16 MFMAs
    // are independent of its softmax arithmetic, so the two interleave.
    // Every step issues the same number of copies (positions past the stream
    // load a resident token), so one counted wait at its end retires exactly
    // the copies the next step reads.
    f32x16 sA[2], sB[2];
    u32x4 pA[2][2], pB[2][2];
    // Prologue: K(0), V(0), K(1) resident, S(0) computed, K(2) and V(1) in
    // flight; oacc / l_run cleared, m_run = the row maximum of tile 0.
    auto prologue = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
      l_run = 0.0f;
      m_run = 0.0f;
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) group_init(sel, cur[j], use_map);
      ld_tile = 0;
      if (ntiles > 0) {
        advance(koff);
        load_tile(kbase, koff, sK[0]);
        load_tile(vbase, koff, sV[0]);
        advance(koff);
        load_tile(kbase, koff, sK[1]);
        voff_keep(koff);
      }
      wait_copies();
      __syncthreads();
      if (wave_on && ntiles > 0) {
        scores(sK[0], sA);
        if (umode == 0) {
          mask_tail(0, sA);
          m_run = row_max(sA) * a.scale_log2;
        } else {
          // A row may attend nothing in tile 0: keep the reference finite so
          // that masked scores give exp2(-inf) = 0, never inf - inf.
          useg = 0;
          mask_keys(0, sA);
          m_run = __builtin_elementwise_maximum(row_max(sA) * a.scale_log2, -1.0e30f);
        }
      }
      if (ntiles > 0) {
        advance(koff);
        load_tile(kbase, koff, sK[2]);
        load_tile(vbase, voff, sV[1]);
        voff_keep(koff);
      }
    };
    // `ph` is kt % 4 as a compile-time constant (ring slots then become
    // immediate LDS offsets), or -1 to compute it at run time.  `first`
    // marks step 0 (no P(-1)).  With `safe` false the reference m_run stays
    // at tile 0's row maximum (p may exceed 1; the caller checks the row sums
    // afterwards); with `safe` true it follows the online maximum with lazy
    // rescaling.
    auto step = [&](auto ph, auto safe, auto first, auto tail, int kt, f32x16* sc, f32x16* sn,
                    const u32x4 (*pp)[2], u32x4 (*pc)[2]) __attribute__((always_inline)) {
      constexpr int PH = decltype(ph)::value;
      constexpr bool SAFE = decltype(safe)::value != 0;
      constexpr bool FIRST = decltype(first)::value != 0;
      // TAIL: this step may hold the stream's last (partial) key tile
      constexpr bool TAIL = decltype(tail)::value != 0;
      const int k_rd = PH >= 0 ? (PH + 1) & 3 : (kt + 1) & 3;  // K(kt+1)
      const int k_wr = PH >= 0 ? (PH + 3) & 3 : (kt + 3) & 3;  // K(kt+3), = V(kt-1)
      const int v_wr = PH >= 0 ? (PH + 2) & 3 : (kt + 2) & 3;  // V(kt+2)
      advance(koff);
      load_tile(kbase, koff, sK[k_wr]);
      load_tile(vbase, voff, sV[v_wr]);
      voff_keep(koff);

      if (wave_on) {
        if constexpr (SAFE) {
          if (umode == 0) {
            if constexpr (TAIL) mask_tail(kt, sc);
          } else {
            mask_keys(kt, sc);
          }
        } else {
          if (umode == 0) {
            if constexpr (TAIL) mask_tail(kt, sc);
          } else {
            // Grouped tiles.  A 64-key tile mostly lies inside one block, so
            // a row attends all of it or none of it: a row with no key here
            // gets the reference +inf (p = 0, no per-score work); scores are
            // masked one by one only when some row attends part of the tile.
            km = key_mask(kt);
            if (__builtin_amdgcn_ballot_w64(km != 0ull && km != ~0ull) != 0) apply_mask(km, sc);
            // A row that attended nothing so far has l = 0 and O = 0 under
            // the placeholder reference -1e30; it takes its first attended
            // tile's row maximum as its reference (no rescale needed).
            if (__builtin_amdgcn_ballot_w64(m_run <= -1.0e30f && km != 0ull) != 0) {
              const float m_tile =
                  __builtin_elementwise_maximum(row_max(sc) * a.scale_log2, -1.0e30f);
              if (m_run <= -1.0e30f && km != 0ull) m_run = m_tile;
            }
          }
        }
        if constexpr (SAFE) {
          if constexpr (!FIRST) pv(sV[k_wr], pp);  // before any rescale of O
          const float m_tile = row_max(sc) * a.scale_log2;
          if (__builtin_amdgcn_ballot_w64(m_tile > m_run + RESCALE_LOG2) != 0) {
            const float m_new = __builtin_elementwise_maximum(m_run, m_tile);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < ND; ++db)
#pragma unroll
              for (int v = 0; v < 16; ++v) oacc[db][v] *= alpha;
          }
        }
        // S(kt+1); on the last tile this scores stale keys and is discarded,
        // which keeps the score registers free of a select per element.
        if constexpr (SAFE) {
          scores(sK[k_rd], sn);
          softmax(sc, pc);
        } else {
          fast_body(first, sK[k_rd], sV[k_wr], sc, sn, pp, pc,
                    (UNION && km == 0ull) ? -__builtin_inf() : -m_run);
        }
      }
      // Copies complete in issue order (per step: K, then V).  The next step
      // reads K(kt+2), issued one step ago, and V(kt), issued three steps
      // ago; V(kt+1) and this step's copies may stay in flight.
      wait_prev_copies<3 * G::LPW>();
      __syncthreads();
    };
    // All steps of one pass, then O += P(last) V(last).
    auto run = [&](auto safe) __attribute__((always_inline)) {
      if (ntiles == 0) return;
      step(Phase<0>{}, safe, Phase<1>{}, Phase<1>{}, 0, sA, sB, pB, pA);
      int kt = 1;
      // The loop never reaches the last key tile (kt + 3 <= ntiles - 2), so
      // its steps carry no tail mask.
      for (; kt + 4 < ntiles; kt += 4) {
        step(Phase<1>{}, safe, Phase<0>{}, Phase<0>{}, kt, sB, sA, pA, pB);
        step(Phase<2>{}, safe, Phase<0>{}, Phase<0>{}, kt + 1, sA, sB, pB, pA);
        step(Phase<3>{}, safe, Phase<0>{}, Phase<0>{}, kt + 2, sB, sA, pA, pB);
        step(Phase<0>{}, safe, Phase<0>{}, Phase<0>{}, kt + 3, sA, sB, pB, pA);
      }
      // kt % 4 == 1 here; at most four tiles remain
      if (kt < ntiles) step(Phase<1>{}, safe, Phase<0>{}, Phase<1>{}, kt, sB, sA, pA, pB);
      if (kt + 1 < ntiles) step(Phase<2>{}, safe, Phase<0>{}, Phase<1>{}, kt + 1, sA, sB, pB, pA);
      if (kt + 2 < ntiles) step(Phase<3>{}, safe, Phase<0>{}, Phase<1>{}, kt + 2, sB, sA, pA, pB);
      if (kt + 3 < ntiles) step(Phase<0>{}, safe, Phase<0>{}, Phase<1>{}, kt + 3, sA, sB, pB, pA);
      if (wave_on) {
        const char* vs = sV[(ntiles - 1) & 3];
        if ((ntiles - 1) & 1)
          pv(vs, pB);
        else
          pv(vs, pA);
      }
    };

    // Fast pass: reference fixed at tile 0's row maximum.  p = 2^(x - m_run)
    // only exceeds 1 by the amount later tiles beat tile 0, which leaves the
    // result unchanged up to rounding unless P overflows its 16-bit type or
    // the sums grow out of range; a row sum that is not below 2^32 (inf and
    // NaN included) sends the whole tile through the exact online pass.
    // Grouped tiles run the same fast pass with their key masks; a row's
    // reference is its first attended tile's row maximum.
    prologue();
    run(Phase<0>{});
    const float l_fast = l_run + __shfl_xor(l_run, 32);
    if (uniform(__syncthreads_or(!(l_fast < 4294967296.0f)))) {
      wait_copies();  // the fast pass's trailing copies land before reuse
      __syncthreads();
      prologue();
      run(Phase<1>{});
    }

    // Epilogue: normalise, store O rows and LSE (gathered tiles: the
    // partial result of the row's listing).
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    if (row_in_pass) {
      const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      const int64_t pidx = GATHER ? a.kc.pidx(h, qi, gslot, a.topk_n, a.g, r % a.g) : 0;
      uint16_t* orow = GATHER ? a.kc.part_o + pidx * D : a.out + (qi * a.hq + hh) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int v = gi * 4;
          *reinterpret_cast<u32x2*>(orow + db * 32 + gi * 8 + hb * 4) =
              u32x2{pack2<DT>(oacc[db][v] * inv, oacc[db][v + 1] * inv),
                    pack2<DT>(oacc[db][v + 2] * inv, oacc[db][v + 3] * inv)};
        }
      if (hb == 0) {
        const float lse_row = l_tot > 0.0f ? m_run + log2f(l_tot) : -__builtin_inf();
        if constexpr (GATHER)
          a.kc.part_lse[pidx] = lse_row;
        else
          a.lse[(int64_t)hh * a.nq + qi] = lse_row;
      }
    }
    if (n_pass > 1) {
      wait_copies();  // this pass's trailing copies land before the next pass
      __syncthreads();
    }
    }  // passes
  }
  wait_copies();  // no copy into LDS outlives the workgroup
  leave_queue(queue, queue + 2);
}

// Key-centric forward of blocks held whole in LDS: the block's K and V (at
// most NT 64-key tiles) are copied into LDS once per item and stay resident
// while the item's query chunks (up to KC_RES_CHUNKS x 128 rows of gathered
// listings) run over them: S^T = K Q^T and O^T += V^T P^T as in the
// streaming kernel.  BIG = 0: four waves, blocks of 1..KC_RES_KEYS keys;
// BIG = 1 (head dim <= 64): eight waves in two groups of four, each group
// running its own chunks, blocks of KC_RES_KEYS+1..KC_RES2_KEYS keys.  The
// tiles are taken four at a time: a group of four first computes all of its
// scores and their exact row maximum (the softmax reference, raised from
// the previous group's with O and the row sum rescaled), then the
// exponentials, row sums and P.V tile by tile; the row's partial result
// (O / l in the input type and its log2 LSE) is written at [head, query,
// slot] for kc_merge_kernel.
template <int DT, int D, int BIG>
__global__ __launch_bounds__(BIG ? 512 : 256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
kc_resident_fwd_kernel(AttnArgs a) {
  using G = KvTile<D>;
  constexpr int NS = D / 16;
  constexpr int ND = D / 32;
  constexpr int NT = (BIG ? KC_RES2_KEYS : KC_RES_KEYS) / KT;
  constexpr int NWG = BIG ? 2 : 1;  // groups of four waves
  __shared__ __align__(1024) char sK[NT][G::BYTES];
  __shared__ __align__(1024) char sV[NT][G::BYTES];
  __shared__ int s_slot;
  const int tid = threadIdx.x, lane = tid & 63, wv = uniform(tid >> 6);
  const int wg = wv >> 2, wl = wv & 3;  // wave group, wave inside the group
  const int hb = lane >> 5, l32 = lane & 31;
  if (!kc_plan_ok(a)) return;  // no key-centric part for this run: read nothing
  const int32_t* head_off = BIG ? a.kc.r2item_off : a.kc.ritem_off;
  const int4* items = BIG ? a.kc.r2items : a.kc.ritems;
  const int64_t item_cap = BIG ? a.kc.r2item_cap : a.kc.ritem_cap;
  int32_t* queue = a.plan.counter + (BIG ? KC_R2QUEUE_SLOT : KC_RQUEUE_SLOT);
  const int total = head_off[a.hkv];
  // An empty queue: leave it untouched (no fetch, so nothing to reset).
  if (total == 0) return;
  const uint32_t row_bytes = (uint32_t)a.hkv * D * 2;
  const int tq = ROWS / a.g;
  const int64_t cap = a.kc.grev.cap;
  // Lane-dependent parts of the LDS operand addresses (see the streaming
  // kernel), pinned in registers: K row block reads per head-dim step,
  // transposed V reads (rows k0, k0 + 8) per output block.
  uint32_t kl_off[NS], vl_off[ND][2];
  {
    const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
    for (int s2 = 0; s2 < NS; ++s2) {
      kl_off[s2] = (uint32_t)G::off(l32, 2 * s2 + hb);
      asm volatile("" : "+v"(kl_off[s2]));
    }
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
      const int k0 = hb * 4 + (gi >> 2);
      const int cb = dcol >> 3, half = (dcol & 4) * 2;
      vl_off[db][0] = (uint32_t)(G::off(k0, cb) + half);
      vl_off[db][1] = (uint32_t)(G::off(k0 + 8, cb) + half);
      asm volatile("" : "+v"(vl_off[db][0]), "+v"(vl_off[db][1]));
    }
  }

  for (;;) {
    const int w = uniform(fetch_work(queue, &s_slot));
    if (w >= total) break;
    const int h = head_of(head_off, a.hkv, w);
    const int4 it = items[(int64_t)h * item_cap + (w - head_off[h])];
    const int c = it.x, e0 = it.y, n = it.z;
    int64_t s0 = a.cu_blk[c], s1 = a.cu_blk[c + 1];
    s0 = s0 < 0 ? 0 : (s0 > a.nk ? a.nk : s0);
    s1 = s1 < s0 ? s0 : (s1 > a.nk ? a.nk : s1);
    const int len = uniform((int)(s1 - s0));  // 1..NT * KT (plan)
    const int ntiles = (len + KT - 1) / KT;
    const char* kbase = reinterpret_cast<const char*>(a.k + (int64_t)h * D);
    const char* vbase = reinterpret_cast<const char*>(a.v + (int64_t)h * D);
    // The block into LDS: wave group t % NWG copies tile t; load j of its
    // wave wl covers rows (wl * LPW + j) * KPL + lane / CH; keys past the
    // block load its first token (in bounds; masked below).
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < ntiles && t % NWG == wg) {
#pragma unroll
        for (int j = 0; j < G::LPW; ++j) {
          const int row = (wl * G::LPW + j) * G::KPL + lane / G::CH;
          const int key = t * KT + row;
          const uint32_t tok = (uint32_t)(key < len ? s0 + key : s0);
          const uint32_t voff = tok * row_bytes + (((lane % G::CH) ^ G::swz(row)) << 4);
          const uint32_t dst = (uint32_t)(wl * G::LPW + j) * 1024;
          copy16_to_lds(kbase, voff, lds_addr(sK[t]) + dst);
          copy16_to_lds(vbase, voff, lds_addr(sV[t]) + dst);
        }
      }
    }
    wait_copies();
    __syncthreads();

    // The gathered rows of chunk cb: listing -> (query, slot) -> Q row.  A
    // wave group runs chunks wg * tq, wg * tq + step, ...  The listings are
    // loaded two chunks ahead and the Q rows one chunk ahead, so a chunk's
    // dependent gathers are in flight during the chunk before.
    const int r = wl * 32 + l32;
    const int step = NWG * tq;
    auto chunk_ok = [&](int cbx) { return r < (n - cbx < tq ? n - cbx : tq) * a.g; };
    auto load_listing = [&](int cbx) -> int32_t {
      return cbx < n ? a.kc.grev.rev[(int64_t)h * cap + e0 + cbx + (chunk_ok(cbx) ? r / a.g : 0)]
                     : 0;
    };
    auto load_q = [&](int cbx, int32_t lv, u32x4* dst) {
      const int64_t qx = lv / a.topk_n;
      const int hx = h * a.g + (chunk_ok(cbx) ? r % a.g : 0);
#pragma unroll
      for (int s = 0; s < NS; ++s)
        dst[s] = (cbx < n && chunk_ok(cbx))
                     ? *reinterpret_cast<const u32x4*>(a.q + (qx * a.hq + hx) * D + s * 16 + hb * 8)
                     : u32x4{0u, 0u, 0u, 0u};
    };
    const int cb0 = wg * tq;
    int32_t lv_cur = load_listing(cb0);
    u32x4 q_next[NS];
    load_q(cb0, lv_cur, q_next);
    int32_t lv_next = load_listing(cb0 + step);
    for (int cb = cb0; cb < n; cb += step) {
      const int rows = (n - cb < tq ? n - cb : tq) * a.g;
      const bool row_ok = r < rows;
      u32x4 qb[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) qb[s] = q_next[s];
      const int64_t qi = lv_cur / a.topk_n;
      const int64_t slot = lv_cur - qi * a.topk_n;
      // next chunk: its Q rows from the listing loaded one chunk ago; the
      // listing after it
      load_q(cb + step, lv_next, q_next);
      lv_cur = lv_next;
      lv_next = load_listing(cb + 2 * step);
      if (wl * 32 >= rows) continue;  // wave-uniform: no row of this chunk
      f32x16 oacc[ND];
      float m_run = 0.0f, l_run = 0.0f;
      // Fast pass over the resident tiles, as the streaming kernel's: the
      // reference is tile 0's row maximum (tile 0 holds a key, so it is
      // finite) and stays fixed; step t issues the score MFMAs of tile t+1 and
      // the P.V MFMAs of tile t-1, alternating, beside the softmax of tile t,
      // with each MFMA's LDS operand read two slots ahead.
      {
#pragma unroll
        for (int i = 0; i < ND; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
        f32x16 sA[2], sB[2];
        u32x4 pA[2][2], pB[2][2];
        auto mask_last = [&](int kt, f32x16* sc) __attribute__((always_inline)) {
          if (kt * KT + KT > len) {  // uniform: the block's last, partial tile
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                if (kt * KT + blk * 32 + acc_row(v, hb) >= len) sc[blk][v] = -__builtin_inf();
          }
        };
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
          for (int v = 0; v < 16; ++v) sA[blk][v] = 0.0f;
#pragma unroll
          for (int s2 = 0; s2 < NS; ++s2)
            sA[blk] = mfma32<DT>(*reinterpret_cast<const u32x4*>(sK[0] + blk * 32 * (D * 2) +
                                                                 kl_off[s2]),
                                 qb[s2], sA[blk]);
        }
        // keys past the block load its first key, so tile 0's unmasked maximum is the block's
        m_run = row_max(sA) * a.scale_log2;
        // One softmax pair (scores 2j, 2j+1 of the lane's 32) against the
        // reference, packed to the 16-bit type and added to the row sum.
        auto softmax_pair = [&](const f32x16* sc, u32x4 (*pb)[2], int j, float negm)
                                __attribute__((always_inline)) {
          const int blk = j >> 3, c = (j >> 2) & 1, e = j & 3, v0 = c * 8 + 2 * e;
          const float p0 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0], a.scale_log2, negm));
          const float p1 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0 + 1], a.scale_log2, negm));
          pb[blk][c][e] = pack2<DT>(p0, p1);
          l_run = sum2<DT>(pb[blk][c][e], l_run);
        };
        // Step body: HS = the step has score MFMAs (a next tile exists), FP =
        // the step has P.V MFMAs (a previous tile exists).
        auto body = [&](auto hs, auto fp, const char* ks, const char* vs, const f32x16* sc,
                        f32x16* sn, const u32x4 (*pp)[2], u32x4 (*pc)[2], float negm)
                        __attribute__((always_inline)) {
          constexpr bool HS = decltype(hs)::value != 0;
          constexpr bool FP = decltype(fp)::value != 0;
          constexpr int NSM = HS ? 2 * NS : 0;
          constexpr int NPV = FP ? 4 * ND : 0;
          constexpr int NSLOT = NSM + NPV;
          constexpr int NPAIR = 16;
          constexpr int LA = 2;
          auto kind_of = [](int i) constexpr {
            return NPV == 0 ? 0 : (NSM == 0 ? 1 : ((i & 1) == 0 ? 0 : 1));
          };
          auto idx_of = [](int i) constexpr { return (NPV == 0 || NSM == 0) ? i : (i >> 1); };
          auto read_op = [&](int i, u32x4& dst) __attribute__((always_inline)) {
            const int x = idx_of(i);
            if (kind_of(i) == 0) {
              const int blk = x & 1, s2 = x >> 1;
              dst = *reinterpret_cast<const u32x4*>(ks + blk * 32 * (D * 2) + kl_off[s2]);
            } else {
              const int db = x % ND, bc = x / ND, blk = bc >> 1, c = bc & 1;
              const int rb = (blk * 32 + c * 16) * (D * 2);
              const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(vs + rb + vl_off[db][0]));
              const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(vs + rb + vl_off[db][1]));
              const u32x2 lw = __builtin_bit_cast(u32x2, lo);
              const u32x2 hw = __builtin_bit_cast(u32x2, hi);
              dst = u32x4{lw[0], lw[1], hw[0], hw[1]};
            }
          };
          if constexpr (NSLOT == 0) {
#pragma unroll
            for (int j = 0; j < NPAIR; ++j) softmax_pair(sc, pc, j, negm);
          } else {
            u32x4 op[LA + 1];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < LA && i < NSLOT; ++i) read_op(i, op[i % (LA + 1)]);
#pragma unroll
            for (int i = 0; i < NSLOT; ++i) {
              if (i + LA < NSLOT) read_op(i + LA, op[(i + LA) % (LA + 1)]);
              const int x = idx_of(i);
              if (kind_of(i) == 0) {
                const int blk = x & 1, s2 = x >> 1;
                if (s2 == 0) {
#pragma unroll
                  for (int v = 0; v < 16; ++v) sn[blk][v] = 0.0f;
                }
                sn[blk] = mfma32<DT>(op[i % (LA + 1)], qb[s2], sn[blk]);
              } else {
                const int db = x % ND, bc = x / ND, blk = bc >> 1, c = bc & 1;
                oacc[db] = mfma32<DT>(op[i % (LA + 1)], pp[blk][c], oacc[db]);
              }
#pragma unroll
              for (int j = (i * NPAIR) / NSLOT; j < ((i + 1) * NPAIR) / NSLOT; ++j)
                softmax_pair(sc, pc, j, negm);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
        };
        using T1 = std::integral_constant<int, 1>;
        using T0 = std::integral_constant<int, 0>;
        const float negm = -m_run;
        // Steps 0 .. ntiles-1 (ntiles <= NT, unrolled; the score and packed-P
        // buffers alternate by step parity).
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
          if (kt < ntiles) {
            f32x16* sc = (kt & 1) ? sB : sA;
            f32x16* sn = (kt & 1) ? sA : sB;
            u32x4 (*pc)[2] = (kt & 1) ? pB : pA;
            const u32x4 (*pp)[2] = (kt & 1) ? pA : pB;
            mask_last(kt, sc);
            const char* vs = sV[kt > 0 ? kt - 1 : 0];
            if (kt + 1 < ntiles) {
              const char* ks = sK[kt + 1 < NT ? kt + 1 : 0];
              if (kt == 0) body(T1{}, T0{}, ks, vs, sc, sn, pp, pc, negm);
              else body(T1{}, T1{}, ks, vs, sc, sn, pp, pc, negm);
            } else {
              if (kt == 0) body(T0{}, T0{}, sK[0], vs, sc, sn, pp, pc, negm);
              else body(T0{}, T1{}, sK[0], vs, sc, sn, pp, pc, negm);
            }
          }
        }
        // P.V of the last tile
        {
          const int kl = ntiles - 1;
          const u32x4 (*pl)[2] = (kl & 1) ? pB : pA;
#pragma unroll
          for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int cc = 0; cc < 2; ++cc) {
                const int rb = (blk * 32 + cc * 16) * (D * 2);
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(sV[kl] + rb + vl_off[db][0]));
                const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(sV[kl] + rb + vl_off[db][1]));
                const u32x2 lw = __builtin_bit_cast(u32x2, lo);
                const u32x2 hw = __builtin_bit_cast(u32x2, hi);
                oacc[db] = mfma32<DT>(u32x4{lw[0], lw[1], hw[0], hw[1]}, pl[blk][cc], oacc[db]);
              }
        }
      }
      // A row sum out of [0, 2^32) (inf and NaN included): the wave reruns its
      // rows tile by tile with the exact online maximum (O and the row sum
      // rescaled whenever a tile raises a row's maximum).
      if (uniform(__builtin_amdgcn_ballot_w64(!(l_run + __shfl_xor(l_run, 32) < 4294967296.0f)) !=
                  0 ? 1 : 0)) {
#pragma unroll
        for (int i = 0; i < ND; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
        m_run = -__builtin_inf();
        l_run = 0.0f;
#pragma unroll 1
        for (int kt = 0; kt < ntiles; ++kt) {
          const char* ks = sK[0] + kt * G::BYTES;
          const char* vs = sV[0] + kt * G::BYTES;
          f32x16 sc[2];
#pragma unroll
          for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sc[blk][v] = 0.0f;
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2)
              sc[blk] = mfma32<DT>(
                  *reinterpret_cast<const u32x4*>(ks + blk * 32 * (D * 2) + kl_off[s2]), qb[s2],
                  sc[blk]);
          }
          if (kt * KT + KT > len) {
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                if (kt * KT + blk * 32 + acc_row(v, hb) >= len) sc[blk][v] = -__builtin_inf();
          }
          // the tile holds a key of the block: its row maximum is finite
          const float m_new = __builtin_elementwise_maximum(m_run, row_max(sc) * a.scale_log2);
          const float al = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 on the first tile
          l_run *= al;
#pragma unroll
          for (int i = 0; i < ND; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[i][v] *= al;
          m_run = m_new;
          u32x4 pb[2][2];
#pragma unroll
          for (int blk = 0; blk < 2; ++blk) {
            float p[16];
#pragma unroll
            for (int v = 0; v < 16; ++v)
              p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v], a.scale_log2, -m_run));
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
              pb[blk][cc] = u32x4{pack2<DT>(p[cc * 8 + 0], p[cc * 8 + 1]),
                                  pack2<DT>(p[cc * 8 + 2], p[cc * 8 + 3]),
                                  pack2<DT>(p[cc * 8 + 4], p[cc * 8 + 5]),
                                  pack2<DT>(p[cc * 8 + 6], p[cc * 8 + 7])};
#pragma unroll
              for (int e = 0; e < 4; ++e) l_run = sum2<DT>(pb[blk][cc][e], l_run);
            }
          }
#pragma unroll
          for (int db = 0; db < ND; ++db)
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int cc = 0; cc < 2; ++cc) {
                const int rb = (blk * 32 + cc * 16) * (D * 2);
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(vs + rb + vl_off[db][0]));
                const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(vs + rb + vl_off[db][1]));
                const u32x2 lw = __builtin_bit_cast(u32x2, lo);
                const u32x2 hw = __builtin_bit_cast(u32x2, hi);
                oacc[db] = mfma32<DT>(u32x4{lw[0], lw[1], hw[0], hw[1]}, pb[blk][cc], oacc[db]);
              }
        }
      }
      const float l_tot = l_run + __shfl_xor(l_run, 32);
      if (row_ok) {
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        const int64_t pidx = a.kc.pidx(h, qi, slot, a.topk_n, a.g, r % a.g);
        uint16_t* orow = a.kc.part_o + pidx * D;
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
          a.kc.part_lse[pidx] = l_tot > 0.0f ? m_run + log2f(l_tot) : -__builtin_inf();
      }
    }
    __syncthreads();  // the item's reads of sK / sV end before the next copies
  }
  wait_copies();
  leave_queue(queue, queue + 2);
}

// Key-centric merge: one thread per (kv head, query, query head, 8 output
// channels) of the marked queries.  The partials of the row's valid slots
// (the gathered tiles wrote one per slot naming a block) are combined in
// slot order: M = max LSE_j, W = sum 2^(LSE_j - M), O = sum 2^(LSE_j - M)
// O_j / W, LSE = M + log2 W.  Slots are taken 16 at a time with their ids,
// LSEs and partials loaded together (a slot without a block is loaded and
// ignored: the buffers cover every slot); M is the maximum over the chunks
// seen so far and earlier terms are rescaled when a chunk raises it, which
// for rows of at most 16 slots is the single maximum above.  A row without
// a partial that attended a key gives O = 0 and LSE = -inf.
template <int DT, int D>
__global__ __launch_bounds__(256) void kc_merge_kernel(AttnArgs a) {
  constexpr int CPT = 8;  // output channels per thread: one 16-byte load per slot
  constexpr int U = 16;   // slots loaded together
  if (!kc_plan_ok(a)) return;  // no key-centric part for this run: read nothing
  const int64_t per_q = (int64_t)a.g * (D / CPT);
  // the queries of this launch's pass
  const int64_t n_items = (int64_t)a.kc.h_count * a.kc.q_span * per_q;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < n_items;
       it += (int64_t)gridDim.x * blockDim.x) {
    const int64_t hq_rel = it / per_q;  // (h - h_base) * q_span + (q - q_base)
    const int hr = (int)(hq_rel / a.kc.q_span);
    const int h = a.kc.h_base + hr;
    const int64_t q = a.kc.q_base + (hq_rel - (int64_t)hr * a.kc.q_span);
    const int64_t hq_idx = (int64_t)h * a.nq + q;
    if (!a.kc.qmark[hq_idx]) continue;
    const int sub = (int)(it - hq_rel * per_q);
    const int gi = sub / (D / CPT), d0 = (sub % (D / CPT)) * CPT;
    int b, bs, nbb;
    bool st;
    query_batch(a.cu_q, a.batch, a.cu_sb, q, &b, &bs, &nbb, &st);
    const int32_t* row = a.topk + hq_idx * a.topk_n;
    const int64_t pbase = hq_rel * a.topk_n;  // partial (q, slot 0) of the pass
    float mx = -__builtin_inf();
    float acc[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) acc[c] = 0.0f;
    float wsum = 0.0f;
    for (int j0 = 0; j0 < a.topk_n; j0 += U) {
      int v[U];
      float l[U];
      u32x4 ov[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u;
        const bool in = j < a.topk_n;
        v[u] = in ? row[j] : -1;
        const int64_t pidx = (pbase + (in ? j : 0)) * a.g + gi;
        l[u] = a.kc.part_lse[pidx];
        ov[u] = *reinterpret_cast<const u32x4*>(a.kc.part_o + pidx * D + d0);
      }
      bool ok[U];
      float cm = -__builtin_inf();
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ok[u] = v[u] >= 0 && v[u] < nbb && (int64_t)bs + v[u] < a.nb;
        if (ok[u]) cm = __builtin_elementwise_maximum(cm, l[u]);
      }
      const float m_new = __builtin_elementwise_maximum(mx, cm);
      if (!(m_new > -__builtin_inf())) continue;  // no finite LSE yet
      if (m_new != mx) {  // the first finite chunk (scale 0 on zeros) or a larger maximum
        const float sc = __builtin_amdgcn_exp2f(mx - m_new);
        wsum *= sc;
#pragma unroll
        for (int c = 0; c < CPT; ++c) acc[c] *= sc;
        mx = m_new;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!ok[u]) continue;
        const float wj = __builtin_amdgcn_exp2f(l[u] - mx);
        wsum += wj;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += wj * to_f32<DT>((uint16_t)(ov[u][e] & 0xffffu));
          acc[2 * e + 1] += wj * to_f32<DT>((uint16_t)(ov[u][e] >> 16));
        }
      }
    }
    const float inv = wsum > 0.0f ? 1.0f / wsum : 0.0f;
    const int hh = h * a.g + gi;
    *reinterpret_cast<u32x4*>(a.out + (q * a.hq + hh) * D + d0) =
        u32x4{pack2<DT>(acc[0] * inv, acc[1] * inv), pack2<DT>(acc[2] * inv, acc[3] * inv),
              pack2<DT>(acc[4] * inv, acc[5] * inv), pack2<DT>(acc[6] * inv, acc[7] * inv)};
    if (d0 == 0)
      a.lse[(int64_t)hh * a.nq + q] = wsum > 0.0f ? mx + log2f(wsum) : -__builtin_inf();
  }
}

template <int DT, int D>
int launch_fwd_t(const AttnArgs& a, hipStream_t st) {
  const void* fn = reinterpret_cast<const void*>(&sel_attn_fwd_kernel<DT, D, FWD_RUN>);
  const int grid = persistent_grid(fn, 256, 0);
  if (grid <= 0) return LSRM_ERR_LAUNCH;
  hipLaunchKernelGGL((sel_attn_fwd_kernel<DT, D, FWD_RUN>), dim3(grid), dim3(256), 0, st,
                     a);
  LSRM_CHECK_LAUNCH();
  if (a.plan.gtiles && !a.kc.fitems) {  // the grouped tiles (key-centric plans: gathered)
    const void* fu = reinterpret_cast<const void*>(&sel_attn_fwd_kernel<DT, D, FWD_UNION>);
    const int gu = persistent_grid(fu, 256, 0);
    if (gu <= 0) return LSRM_ERR_LAUNCH;
    hipLaunchKernelGGL((sel_attn_fwd_kernel<DT, D, FWD_UNION>), dim3(gu), dim3(256), 0, st,
                       a);
    LSRM_CHECK_LAUNCH();
  }
  if (a.kc.fitems) {  // key-centric plans: gathered tiles, then the merge
    const void* fg = reinterpret_cast<const void*>(&sel_attn_fwd_kernel<DT, D, FWD_GATHER>);
    const int gg = persistent_grid(fg, 256, 0);
    const void* fr = reinterpret_cast<const void*>(&kc_resident_fwd_kernel<DT, D, 0>);
    const int gr = persistent_grid(fr, 256, 0);
    int gr2 = 1;
    if constexpr (kc_res_max(D) > KC_RES_KEYS)
      gr2 = persistent_grid(reinterpret_cast<const void*>(&kc_resident_fwd_kernel<DT, D, 1>),
                            512, 0);
    const int gm = device_cu_count() * 16;
    if (gg <= 0 || gr <= 0 || gr2 <= 0 || gm <= 0) return LSRM_ERR_LAUNCH;
    // One range of queries at a time: its gathered tiles, then their merge,
    // before the next range reuses the partial buffer.  The range's three
    // gathered-tile kernels write disjoint partials: the streaming and
    // eight-wave ones run on a second stream beside the four-wave one, so
    // that each kernel's last workgroups overlap the other's work.
    SideStream ss{};
    const bool two = !stream_capturing(st) && side_stream(ss) == LSRM_OK;
    std::unique_lock<std::mutex> seq;
    if (two) seq = std::unique_lock<std::mutex>(*ss.m);
    hipStream_t s2 = two ? ss.s : st;
    for (int p = 0; p < a.kc.n_pass; ++p) {
      AttnArgs ap = a;
      ap.kc = a.kc.pass(p, a.hkv, a.nq);
      if (two && (hipEventRecord(ss.fork, st) != hipSuccess ||
                  hipStreamWaitEvent(ss.s, ss.fork, 0) != hipSuccess))
        return LSRM_ERR_LAUNCH;
      if constexpr (kc_res_max(D) > KC_RES_KEYS) {
        hipLaunchKernelGGL((kc_resident_fwd_kernel<DT, D, 1>), dim3(gr2), dim3(512), 0, s2, ap);
        LSRM_CHECK_LAUNCH();
      }
      hipLaunchKernelGGL((sel_attn_fwd_kernel<DT, D, FWD_GATHER>), dim3(gg), dim3(256), 0, s2,
                         ap);
      LSRM_CHECK_LAUNCH();
      hipLaunchKernelGGL((kc_resident_fwd_kernel<DT, D, 0>), dim3(gr), dim3(256), 0, st, ap);
      LSRM_CHECK_LAUNCH();
      if (two && (hipEventRecord(ss.join, ss.s) != hipSuccess ||
                  hipStreamWaitEvent(st, ss.join, 0) != hipSuccess))
        return LSRM_ERR_LAUNCH;
      hipLaunchKernelGGL((kc_merge_kernel<DT, D>), dim3(gm), dim3(256), 0, st, ap);
      LSRM_CHECK_LAUNCH();
    }
  }
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
