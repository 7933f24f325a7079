// Selected-block attention backward on bf16/fp16 MFMA (gfx950).
//
// dQ follows backward_kernel_dq
// (sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:262-478):
// Delta = rowsum(O * dO) in fp32 (fused), P = exp2(q.k * scale*log2e - lse),
// dP = dO V^T, dS = scale * P * (dP - Delta) rounded to the input type,
// dQ = dS K.  It runs on the forward's query tiles and key stream, with the
// forward's streaming scheme: K and V tiles copied straight into three-slot
// LDS rings (swizzled, row-major), S^T = K Q^T and dP^T = V dO^T from
// row-major reads, dQ^T = K^T dS^T with K^T taken by ds_read_b64_tr_b16.
//
// Per-token selection rows (consecutive queries with different rows) come
// as the plan's grouped tiles: dQ runs them over the union of their blocks
// with per-row key masks, or run by run.
//
// dK/dV follow backward_kernel_dkdv_fastest (same file, 687-923): each
// workgroup owns one key chunk of one block of one kv head and walks the
// run tiles that selected the block (tile-granular reverse map, ascending
// tile order), then the queries of grouped tiles that selected it
// (query-granular reverse map, ascending, 128 / g queries gathered per
// step), so every dK/dV element has a single writer and a fixed
// accumulation order.  The Q and dO rows are copied into two-slot LDS
// rings; S = Q K^T and dP = dO V^T take the rows directly, dV^T = dO^T P and
// dK^T = Q^T dS take Q^T / dO^T by transposed reads.  Chunks hold up to 128
// keys: each wave owns 32 of them and runs every step's 128 rows as two
// 64-row halves, so one copy of a step's Q / dO rows feeds 128 keys.
#include <algorithm>
#include <type_traits>

#include "attn.h"

namespace lsrm {

// ------------------------------------------------------------------- dQ --

// MODE 0 (DQ_RUN): the run tiles of the plan.  MODE 1 (DQ_UNION): the
// grouped tiles, run once over the union of their rows' blocks with per-row
// key masks, or once per run of identical rows with the other rows' P forced
// to zero (the passes of the forward's grouped tiles; no softmax state is
// carried, so either way each row's dQ is a plain sum over the keys it
// attends); a key-centric plan does not launch it (its grouped tiles' rows
// run as gathered tiles).
// MODE 2 (DQ_GATHER): the gathered tiles of a key-centric plan over blocks
// the resident kernels do not take (no keys, or more than kc_res_max), each
// row writing the block's share of its dQ (one slot of its row, in the
// input type) for kc_dq_merge_kernel.
constexpr int DQ_RUN = 0, DQ_UNION = 1, DQ_GATHER = 2;

template <int DT, int D, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sel_attn_dq_kernel(AttnArgs a) {
  constexpr bool UNION = MODE == DQ_UNION;
  constexpr bool GATHER = MODE == DQ_GATHER;
  using G = KvTile<D>;
  constexpr int NS = D / 16;  // MFMA k-steps over the head dim
  constexpr int ND = D / 32;  // 32-wide output blocks over the head dim
  __shared__ __align__(1024) char sK[3][G::BYTES];
  __shared__ __align__(1024) char sV[3][G::BYTES];
  __shared__ SelLds sel;
  __shared__ typename std::conditional<UNION, UnionLds, int>::type ul;
  // Run tiles whose key stream has at most KMAP_KEYS positions: the token
  // of every position (build_token_map), read at each segment crossing.
  __shared__ int s_tokmap[MODE == DQ_RUN ? KMAP_KEYS : 1];
  __shared__ int s_slot;

  const int tid = threadIdx.x, lane = tid & 63, wv = uniform(tid >> 6);
  const int hb = lane >> 5, l32 = lane & 31;
  const int32_t* head_off =
      GATHER ? a.kc.fitem_off : (UNION ? a.plan.ghead_off : a.plan.head_off);
  const int2* tiles = UNION ? a.plan.gtiles : a.plan.tiles;
  int32_t* queue = a.plan.counter + (GATHER ? KC_QUEUE_SLOT : (UNION ? 4 : 0));
  // A plan built without its backward part: nothing here is valid to read.
  if (a.plan.counter[PLAN_BWD_SLOT] != PLAN_BWD_MAGIC) return;
  if constexpr (GATHER) {
    if (!kc_plan_ok(a)) return;  // nor without the key-centric part of this run
  }
  const int total = head_off[a.hkv];
  // An empty queue: leave it untouched (no fetch, so nothing to reset).
  if (total == 0) return;

  int ld_key[G::LPW], ld_byte[G::LPW];
#pragma unroll
  for (int j = 0; j < G::LPW; ++j) {
    ld_key[j] = (wv * G::LPW + j) * G::KPL + lane / G::CH;
    ld_byte[j] = (((lane % G::CH) ^ G::swz(ld_key[j])) << 4);
  }
  const uint32_t row_bytes = (uint32_t)a.hkv * D * 2;
  // Per-lane LDS offsets of the operand reads, fixed for the kernel (the
  // swizzle repeats every 16 rows, so a 16- or 32-key block adds a constant
  // that folds into the read's immediate): row-major K / V rows of head-dim
  // step s, and the transposed K reads (rows k0, k0 + 8) of output block db.
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
      const int cb = dcol >> 3, half = (dcol & 4) * 2;
      const int k0 = hb * 4 + (gi >> 2);
      vl_off[db][0] = (uint32_t)(G::off(k0, cb) + half);
      vl_off[db][1] = (uint32_t)(G::off(k0 + 8, cb) + half);
      asm volatile("" : "+v"(vl_off[db][0]), "+v"(vl_off[db][1]));
    }
  }

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
    // umode 0: a run tile (or a gathered tile); 1: a grouped tile over the
    // union of its blocks, rows masked to their own; 2: a grouped tile run
    // by run.
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
    const int nkeys = sel.cum[sel.n];
    const int ntiles = (nkeys + KT - 1) / KT;
    const int t_safe = sel.n > 0 ? sel.tok[0] : 0;
    const bool use_map = MODE == DQ_RUN && uniform(nkeys) <= KMAP_KEYS;
    if constexpr (MODE == DQ_RUN) {
      if (use_map) build_token_map(sel, s_tokmap, wv, lane);
    }

    const int r = wv * 32 + l32;
    const bool row_ok = r < rows;
    const int qr = row_ok ? r / a.g : 0;  // the row's query within the tile
    const bool row_in_pass = row_ok && qr >= q_lo && qr < q_hi;
    const bool wave_on = uniform(wv * 32 < q_hi * a.g && wv * 32 + 32 > q_lo * a.g) != 0;
    // Gathered tiles: row r is listing ge0 + r / g (query * topk + slot).
    int64_t qi, gslot = 0;
    if constexpr (GATHER) {
      const int64_t lv = a.kc.grev.rev[(int64_t)h * a.kc.grev.cap + ge0 + qr];
      qi = lv / a.topk_n;
      gslot = lv - qi * a.topk_n;
    } else {
      qi = q0 + qr;
    }
    const int hh = h * a.g + (row_ok ? r % a.g : 0);
    u32x4 qb[NS], dob[NS];
    float dpart = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (row_ok) {
        const int64_t off = (qi * a.hq + hh) * D + s * 16 + hb * 8;
        qb[s] = *reinterpret_cast<const u32x4*>(a.q + off);
        dob[s] = *reinterpret_cast<const u32x4*>(a.dout + off);
        if constexpr (!GATHER) {
          const u32x4 ob = *reinterpret_cast<const u32x4*>(a.o + off);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dpart += to_f32<DT>((uint16_t)(ob[i] & 0xffffu)) *
                     to_f32<DT>((uint16_t)(dob[s][i] & 0xffffu));
            dpart += to_f32<DT>((uint16_t)(ob[i] >> 16)) *
                     to_f32<DT>((uint16_t)(dob[s][i] >> 16));
          }
        }
      } else {
        qb[s] = u32x4{0u, 0u, 0u, 0u};
        dob[s] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    // Delta: fused here for run and grouped tiles; gathered rows read the
    // value kc_delta_kernel wrote for their query.
    float delta;
    if constexpr (GATHER)
      delta = row_ok ? a.lse[(int64_t)hh * a.nq + qi] : 0.0f;
    else
      delta = dpart + __shfl_xor(dpart, 32);
    // Exponent bias -lse.  Rows outside the tile or the pass get -inf (P =
    // 0), and so does a row that attends nothing (lse = -inf; in a grouped
    // tile its masked scores would otherwise give -inf + inf).
    float bias = -__builtin_inf();
    if (row_in_pass) {
      const float l = a.lse_in[(int64_t)hh * a.nq + qi];
      if (l > -__builtin_inf()) bias = -l;
    }
    if (!GATHER && row_in_pass && hb == 0) a.lse[(int64_t)hh * a.nq + qi] = delta;

    const char* kbase = reinterpret_cast<const char*>(a.k + (int64_t)h * D);
    const char* vbase = reinterpret_cast<const char*>(a.v + (int64_t)h * D);
    StreamCursor cur[G::LPW];
    uint32_t koff[G::LPW];
#pragma unroll
    for (int j = 0; j < G::LPW; ++j) {
      cur[j].p = ld_key[j] - KT;
      cur[j].seg = 0;
      cur[j].tok = 0;
      cur[j].segend = -1;  // mapped streams keep it: every step reads the map
      cur[j].ntb = 0;
      cur[j].nend = -1;
    }
    auto advance = [&]() {
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) {
        StreamCursor& c = cur[j];
        c.p += KT;
        int t = t_safe;
        if (c.p < nkeys) {
          c.tok += KT;
          if (c.p >= c.segend) {
            if (use_map) {
              c.tok = s_tokmap[c.p];
            } else {
              if (c.p < c.nend) {
                ++c.seg;
                c.tok = c.p + c.ntb;
                c.segend = c.nend;
              } else {
                cursor_seek(sel, c);
              }
              cursor_prefetch(sel, c);
            }
          }
          t = c.tok;
        }
        koff[j] = (uint32_t)t * row_bytes + ld_byte[j];
      }
    };
    auto load_tiles = [&](int slot) {
      const uint32_t dk = lds_addr(sK[slot]) + wv * G::LPW * 1024;
      const uint32_t dv = lds_addr(sV[slot]) + wv * G::LPW * 1024;
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) copy16_to_lds(kbase, koff[j], dk + j * 1024);
#pragma unroll
      for (int j = 0; j < G::LPW; ++j) copy16_to_lds(vbase, koff[j], dv + j * 1024);
    };

    f32x16 dqacc[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) dqacc[i][v] = 0.0f;
    int useg = 0;  // union segment cursor of the key masks

    // Prologue: tile 0 resident, tile 1 in flight (a step's copies are
    // consumed two steps later, retired by a counted wait).
    if (ntiles > 0) {
      advance();
      load_tiles(0);
    }
    wait_copies();
    __syncthreads();
    if (ntiles > 0) {
      advance();
      load_tiles(1);
    }

    for (int kt = 0; kt < ntiles; ++kt) {
      const int s0 = kt % 3, s2 = (kt + 2) % 3;
      advance();
      load_tiles(s2);
      if constexpr (D <= 64) {
      if (wave_on) {
        const char* ks = sK[s0];
        const char* vs = sV[s0];
        const int kb0 = kt * KT;
        // Keys of this tile the row attends (bit p = stream position kb0 + p):
        // union segments its query selected (umode 1), else the stream tail.
        uint64_t m = ~0ull;
        if (umode == 1) {
          if constexpr (UNION) {
            m = 0ull;
            int sg = useg;
            while (sel.cum[sg + 1] <= kb0) ++sg;  // stops at the sentinel
            useg = sg;
            for (; sg < sel.n && sel.cum[sg] < kb0 + KT; ++sg) {
              const int lo = sel.cum[sg] > kb0 ? sel.cum[sg] - kb0 : 0;
              const int hi = sel.cum[sg + 1] - kb0 < KT ? sel.cum[sg + 1] - kb0 : KT;
              const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
              const uint64_t range = upto & ~((1ull << lo) - 1ull);
              if ((ul.seg_q[sg][qr >> 5] >> (qr & 31)) & 1u) m |= range;
            }
          }
        } else if (kb0 + KT > nkeys) {
          const int hi = nkeys - kb0;
          m = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
        }
        // A row attends all of a 64-key tile or none of it except at block
        // edges and the stream tail: a row with no key here gets the bias
        // -inf (P = 0); scores are masked one by one only when some row of
        // the wave attends part of the tile.
        const bool masked =
            uniform(__builtin_amdgcn_ballot_w64(m != 0ull && m != ~0ull) != 0 ? 1 : 0) != 0;
        const float bias_t = m == 0ull ? -__builtin_inf() : bias;
        const uint64_t mh = m >> (hb * 4);  // slot v: key (v/4)*8 + hb*4 + v%4
        // The step's MFMAs in a fixed issue order, in four phases:
        //   A  S^T, dP^T of key block 0     (2 * NS)
        //   B  S^T, dP^T of key block 1     (2 * NS)   + dS of key block 0
        //   C  dQ^T += K^T dS^T, block 0    (2 * ND)   + dS of key block 1
        //   D  dQ^T += K^T dS^T, block 1    (2 * ND)
        // Each slot issues the LDS reads of the MFMA LA slots ahead, its
        // MFMA, then its share of the vector work; scheduling barriers keep
        // the order.  dS is kept unscaled (dQ is scaled once at the end).
        constexpr int NA = 2 * NS, NC = 2 * ND, NSLOT = 2 * NA + 2 * NC, LA = 2;
        f32x16 sc[2], dp[2];
        u32x4 dsb[2][2];
        u32x4 opnd[LA + 1];
        // Operand of MFMA i: K / V rows (S^T, dP^T), or K^T by transposed
        // reads (slot e of lane (hb, row d) = key blk*32 + c*16 + (e/4)*8 +
        // hb*4 + e%4, the score layout).
        auto read_op = [&](int i) __attribute__((always_inline)) {
          if (i < 2 * NA) {
            const int blk = i / NA, j = i % NA, sk = j >> 1;
            const char* src = (j & 1) ? vs : ks;
            opnd[i % (LA + 1)] =
                *reinterpret_cast<const u32x4*>(src + blk * 32 * (D * 2) + kl_off[sk]);
          } else {
            const int j = (i - 2 * NA) % NC, blk = (i - 2 * NA) / NC;
            const int db = j >> 1, c = j & 1;
            const int rb = (blk * 32 + c * 16) * (D * 2);
            const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(ks + rb + vl_off[db][0])));
            const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)(ks + rb + vl_off[db][1])));
            opnd[i % (LA + 1)] = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
        };
        auto apply_mask = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if (!((mh >> (blk * 32 + (v / 4) * 8 + (v % 4))) & 1ull))
              sc[blk][v] = -__builtin_inf();
        };
        // dS of score registers 2k, 2k+1 of key block blk, packed.
        auto ds_pair = [&](int blk, int k) __attribute__((always_inline)) {
          const int v0 = 2 * k;
          const float p0 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0], a.scale_log2, bias_t));
          const float p1 =
              __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0 + 1], a.scale_log2, bias_t));
          dsb[blk][k >> 2][k & 3] =
              pack2<DT>(p0 * (dp[blk][v0] - delta), p1 * (dp[blk][v0 + 1] - delta));
        };
#pragma unroll
        for (int i = 0; i < LA; ++i) read_op(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
          if (i + LA < NSLOT) read_op(i + LA);
          const u32x4 op = opnd[i % (LA + 1)];
          if (i < 2 * NA) {
            const int blk = i / NA, j = i % NA, sk = j >> 1;
            if (j & 1) {
              if (sk == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) dp[blk][v] = 0.0f;
              }
              dp[blk] = mfma32<DT>(op, dob[sk], dp[blk]);
            } else {
              if (sk == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) sc[blk][v] = 0.0f;
              }
              sc[blk] = mfma32<DT>(op, qb[sk], sc[blk]);
            }
          } else {
            const int j = (i - 2 * NA) % NC, blk = (i - 2 * NA) / NC;
            const int db = j >> 1, c = j & 1;
            dqacc[db] = mfma32<DT>(op, dsb[blk][c], dqacc[db]);
          }
          // vector work: key block 0 during phase B, key block 1 during C
          if (i == NA && masked) apply_mask(0);
          if (i == 2 * NA && masked) apply_mask(1);
          if (i >= NA && i < 2 * NA) {
            const int t = i - NA;
#pragma unroll
            for (int k = (t * 8) / NA; k < ((t + 1) * 8) / NA; ++k) ds_pair(0, k);
          } else if (i >= 2 * NA && i < 2 * NA + NC) {
            const int t = i - 2 * NA;
#pragma unroll
            for (int k = (t * 8) / NC; k < ((t + 1) * 8) / NC; ++k) ds_pair(1, k);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      } else {
      if (D > 64 && wave_on) {
        const char* ks = sK[s0];
        const char* vs = sV[s0];
        f32x16 sacc[2], dpacc[2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
          for (int v = 0; v < 16; ++v) sacc[blk][v] = dpacc[blk][v] = 0.0f;
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            const int o = G::off(blk * 32 + l32, 2 * s + hb);
            sacc[blk] = mfma32<DT>(*reinterpret_cast<const u32x4*>(ks + o), qb[s],
                                   sacc[blk]);
            dpacc[blk] = mfma32<DT>(*reinterpret_cast<const u32x4*>(vs + o),
                                    dob[s], dpacc[blk]);
          }
        }
        const int kb0 = kt * KT;
        if (umode == 1) {
          if constexpr (UNION) {
            // Keys of union segments the row's query did not select (and
            // positions past the stream) score -inf.
            uint64_t m = 0ull;
            int sg = useg;
            while (sel.cum[sg + 1] <= kb0) ++sg;  // stops at the sentinel
            useg = sg;
            for (; sg < sel.n && sel.cum[sg] < kb0 + KT; ++sg) {
              const int lo = sel.cum[sg] > kb0 ? sel.cum[sg] - kb0 : 0;
              const int hi = sel.cum[sg + 1] - kb0 < KT ? sel.cum[sg + 1] - kb0 : KT;
              const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
              const uint64_t range = upto & ~((1ull << lo) - 1ull);
              if ((ul.seg_q[sg][qr >> 5] >> (qr & 31)) & 1u) m |= range;
            }
            const uint64_t mh = m >> (hb * 4);  // slot v: key (v/4)*8 + hb*4 + v%4
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                if (!((mh >> (blk * 32 + (v / 4) * 8 + (v % 4))) & 1ull))
                  sacc[blk][v] = -__builtin_inf();
          }
        } else if (kb0 + KT > nkeys) {
#pragma unroll
          for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int v = 0; v < 16; ++v)
              if (kb0 + blk * 32 + acc_row(v, hb) >= nkeys)
                sacc[blk][v] = -__builtin_inf();
        }
        u32x4 dsb[2][2];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
          float ds[16];
#pragma unroll
          for (int v = 0; v < 16; ++v)
            ds[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[blk][v], a.scale_log2, bias)) *
                    (dpacc[blk][v] - delta);
#pragma unroll
          for (int c = 0; c < 2; ++c)
            dsb[blk][c] = u32x4{pack2<DT>(ds[c * 8 + 0], ds[c * 8 + 1]),
                                pack2<DT>(ds[c * 8 + 2], ds[c * 8 + 3]),
                                pack2<DT>(ds[c * 8 + 4], ds[c * 8 + 5]),
                                pack2<DT>(ds[c * 8 + 6], ds[c * 8 + 7])};
        }
        // dQ^T += K^T dS^T: K^T from the row-major K tile by transposed reads
        // (slot e of lane (hb, row d) = key blk*32 + c*16 + (e/4)*8 + hb*4 +
        // e%4, the score layout).
        const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
        for (int db = 0; db < ND; ++db) {
          const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
          const int cb = dcol >> 3, half = (dcol & 4) * 2;
#pragma unroll
          for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const int k0 = blk * 32 + c * 16 + hb * 4 + (gi >> 2);
              const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(ks + G::off(k0, cb) + half));
              const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(ks + G::off(k0 + 8, cb) + half));
              const u32x2 lw = __builtin_bit_cast(u32x2, lo);
              const u32x2 hw = __builtin_bit_cast(u32x2, hi);
              dqacc[db] = mfma32<DT>(u32x4{lw[0], lw[1], hw[0], hw[1]},
                                     dsb[blk][c], dqacc[db]);
            }
        }
      }
      }
      wait_prev_copies<2 * G::LPW>();
      __syncthreads();
    }

    if (row_in_pass) {
      // gathered rows: the slot's share of dQ, summed by kc_dq_merge_kernel
      uint16_t* drow =
          GATHER ? a.kc.part_o + a.kc.pidx(h, qi, gslot, a.topk_n, a.g, r % a.g) * D
                 : a.out + (qi * a.hq + hh) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          const int v = gi * 4;
          // dS was kept unscaled: dQ = scale * (dS' K)
          *reinterpret_cast<u32x2*>(drow + db * 32 + gi * 8 + hb * 4) =
              u32x2{pack2<DT>(a.scale * dqacc[db][v], a.scale * dqacc[db][v + 1]),
                    pack2<DT>(a.scale * dqacc[db][v + 2], a.scale * dqacc[db][v + 3])};
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

// ----------------------------------------------------------------- dK/dV --

template <int DT, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
sel_attn_dkdv_kernel(AttnArgs a) {
  using G = KvTile<D, ROWS>;  // 128-row Q / dO tiles
  constexpr int NS = D / 16;
  constexpr int ND = D / 32;
  __shared__ __align__(1024) char sQ[2][G::BYTES];
  __shared__ __align__(1024) char sO[2][G::BYTES];
  __shared__ __align__(16) float s_lse[2][ROWS];  // lse per row (+inf: none)
  __shared__ __align__(16) float s_dl[2][ROWS];   // delta per row
  __shared__ int s_qi[2][ROWS];                   // gathered rows' queries
  __shared__ int s_slot;

  const int tid = threadIdx.x, lane = tid & 63, wv = uniform(tid >> 6);
  const int hb = lane >> 5, l32 = lane & 31;
  static_assert(KEY_CHUNK == 4 * 32, "four waves of 32 keys cover a chunk");
  // Lane-dependent parts of the Q / dO tile reads (the tile row's high bits
  // do not enter the swizzle): row-major reads of head-dim step sk, and the
  // two transposed reads (rows k0, k0 + 8) of output block db.
  uint32_t kl_off[NS], vl_off[ND][2];
  {
    const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
    for (int sk = 0; sk < NS; ++sk) kl_off[sk] = (uint32_t)G::off(l32, 2 * sk + hb);
#pragma unroll
    for (int db = 0; db < ND; ++db) {
      const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
      const int k0 = hb * 4 + (gi >> 2);
      const int cb = dcol >> 3, half = (dcol & 4) * 2;
      vl_off[db][0] = (uint32_t)(G::off(k0, cb) + half);
      vl_off[db][1] = (uint32_t)(G::off(k0 + 8, cb) + half);
    }
  }
  // A plan built without its backward part: no reverse maps or key chunks.
  if (a.plan.counter[PLAN_BWD_SLOT] != PLAN_BWD_MAGIC) return;
  const int n_items = a.items.n_items[0];
  const int total = n_items * a.hkv;

  int ld_row[G::LPW], ld_byte[G::LPW];
  // Row r of a step <-> (query r / g of the step, query head r % g): the
  // quotients of this lane's copy rows and of stats row tid, computed once.
  int ld_q[G::LPW], ld_hh[G::LPW];
#pragma unroll
  for (int j = 0; j < G::LPW; ++j) {
    ld_row[j] = (wv * G::LPW + j) * G::KPL + lane / G::CH;
    ld_byte[j] = (((lane % G::CH) ^ G::swz(ld_row[j])) << 4);
    ld_q[j] = ld_row[j] / a.g;
    ld_hh[j] = ld_row[j] - ld_q[j] * a.g;
  }
  const int st_q = tid / a.g, st_hh = tid - st_q * a.g;

  // The item loop is instantiated twice: with the grouped-query phase, and
  // without it for plans that have no grouped tiles (its loop then carries
  // none of that phase's branches or state).
  // Items (64-key chunks, block-major within a head) are handed out in
  // segments of 64 per XCD, so the chunks of one block, which read the same
  // Q / dO tiles in the same order, run side by side on one XCD and share
  // its L2.
  const int home = xcd_id();
  int tries = 0;
  auto items_loop = [&](auto qmap) __attribute__((always_inline)) {
  constexpr bool QM = decltype(qmap)::value != 0;
  for (;;) {
    const int w = uniform(fetch_work_xcd(a.plan.counter + 8, 64, total, home, tries, &s_slot));
    if (w >= total) break;
    const int h = w / n_items;
    const int4 item = a.items.items[w - h * n_items];
    const int c = item.x, t0 = item.y, nk_item = item.z;
    const int64_t e0 = a.rev.cu_rev[(int64_t)h * (a.nb + 1) + c];
    int64_t e1 = a.rev.cu_rev[(int64_t)h * (a.nb + 1) + c + 1];
    if (e1 > a.rev.cap) e1 = a.rev.cap;
    const int n_ent = e1 > e0 ? (int)(e1 - e0) : 0;
    const int32_t* ents = a.rev.rev + (int64_t)h * a.rev.cap + e0;
    // Then the queries of grouped tiles that selected the block, QC per step.
    int n_qent = 0;
    const int32_t* qents = nullptr;
    if constexpr (QM) {
      const int64_t f0 = a.qrev.cu_rev[(int64_t)h * (a.nb + 1) + c];
      int64_t f1 = a.qrev.cu_rev[(int64_t)h * (a.nb + 1) + c + 1];
      if (f1 > a.qrev.cap) f1 = a.qrev.cap;
      n_qent = f1 > f0 ? (int)(f1 - f0) : 0;
      qents = a.qrev.rev + (int64_t)h * a.qrev.cap + f0;
    }
    const int QC = ROWS / a.g;
    const int n_steps = QM ? n_ent + (n_qent + QC - 1) / QC : n_ent;

    // This wave's 32 keys of the chunk (kh) and the row halves of every step
    // it computes.  Chunks of at most 64 keys at head dim <= 64 split the
    // rows too: wave w takes keys (w & 1) * 32 .. +32 and row half w >> 1,
    // so that four waves work instead of one or two; the halves' dK / dV are
    // added in LDS at the end (half 0 + half 1).
    const bool rsplit = D <= 64 && nk_item <= 64;
    const int kh = rsplit ? (wv & 1) : wv;
    const int rh_lo = rsplit ? (wv >> 1) : 0, rh_hi = rsplit ? rh_lo + 1 : 2;
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

    // Copies of entry e's Q and dO rows into ring slot `slot`, and its lse /
    // delta into registers (stored to LDS by store_stats).
    float lse_r = __builtin_inf(), dl_r = 0.0f;
    // Step e >= n_ent gathers the rows of queries qents[(e - n_ent) * QC +
    // r / g]: thread r reads row r's query two steps ahead into nq_r and
    // publishes it in s_qi[e & 1] (-1 past the list) for the copies.
    int nq_r = -1;
    auto fetch_queries = [&](int e) __attribute__((always_inline)) {
      if (!QM || e < n_ent || e >= n_steps || tid >= ROWS) return;
      const int i = (e - n_ent) * QC + st_q;
      nq_r = i < n_qent ? qents[i] : -1;
    };
    auto publish_queries = [&](int e) __attribute__((always_inline)) {
      if (!QM || e < n_ent || e >= n_steps || tid >= ROWS) return;
      s_qi[e & 1][tid] = nq_r;
    };
    // The run tiles of entries tc_base .. tc_base + 63, lane i holding entry
    // tc_base + i: one load round trip per 64 entries instead of two
    // dependent ones per step.  Entries are visited in increasing order.
    int tc_base = -64, tc_x = 0, tc_y = 0;
    auto tile_of = [&](int e) __attribute__((always_inline)) {
      if (e - tc_base >= 64) {
        tc_base = e;
        int2 t = make_int2(0, 0);
        if (e + lane < n_ent) t = a.plan.tiles[(int64_t)h * a.nq + ents[e + lane]];
        tc_x = t.x;
        tc_y = t.y;
      }
      const int sl = e - tc_base;
      return make_int2(__builtin_amdgcn_readlane(tc_x, sl), __builtin_amdgcn_readlane(tc_y, sl));
    };
    // prepare(e, slot): the rows of step e (byte offsets of this lane's Q /
    // dO pieces, which both tensors share) and its lse / delta loads;
    // copy_part(c) then issues copy c of the 2 * LPW (Q, dO alternating).
    uint32_t cp_off[G::LPW], cp_dq = 0, cp_do = 0;
    auto prepare = [&](int e, int slot) __attribute__((always_inline)) {
      cp_dq = lds_addr(sQ[slot]) + wv * G::LPW * 1024;
      cp_do = lds_addr(sO[slot]) + wv * G::LPW * 1024;
      int rows;
      int64_t sqi = -1;  // query of stats row tid (-1: none)
      if (!QM || e < n_ent) {
        const int2 tl = tile_of(e);
        rows = tl.y * a.g;
#pragma unroll
        for (int j = 0; j < G::LPW; ++j) {
          const bool in = ld_row[j] < rows;  // else an in-bounds filler (row 0)
          cp_off[j] = (uint32_t)(((int64_t)(tl.x + (in ? ld_q[j] : 0)) * a.hq + h * a.g +
                                  (in ? ld_hh[j] : 0)) *
                                 D * 2) +
                      ld_byte[j];
        }
        if (tid < rows) sqi = tl.x + st_q;
      } else {
        const int left = n_qent - (e - n_ent) * QC;
        rows = (left < QC ? left : QC) * a.g;
        const int* qi_row = s_qi[e & 1];
#pragma unroll
        for (int j = 0; j < G::LPW; ++j) {
          const int qv = qi_row[ld_row[j]];
          const int64_t qj = qv >= 0 ? qv : 0;  // query 0: in-bounds filler
          cp_off[j] = (uint32_t)((qj * a.hq + h * a.g + ld_hh[j]) * D * 2) + ld_byte[j];
        }
        if (tid < rows && qi_row[tid] >= 0) sqi = qi_row[tid];
      }
      if (tid < ROWS) {
        if (sqi >= 0) {
          const int hh = h * a.g + st_hh;
          lse_r = a.lse_in[(int64_t)hh * a.nq + sqi];  // consumed by store_stats
          dl_r = a.lse[(int64_t)hh * a.nq + sqi];
        } else {
          lse_r = __builtin_inf();
          dl_r = 0.0f;
        }
      }
      return rows;
    };
    auto copy_part = [&](int c) __attribute__((always_inline)) {
      const int j = c >> 1;
      if (c & 1)
        copy16_to_lds(a.dout, cp_off[j], cp_do + j * 1024);
      else
        copy16_to_lds(a.q, cp_off[j], cp_dq + j * 1024);
    };
    auto issue = [&](int e, int slot) __attribute__((always_inline)) {
      const int rows = prepare(e, slot);
#pragma unroll
      for (int c = 0; c < 2 * G::LPW; ++c) copy_part(c);
      return rows;
    };
    auto store_stats = [&](int slot) __attribute__((always_inline)) {
      if (tid < ROWS) {
        // a row without keys (lse = -inf) gets P = 0
        s_lse[slot][tid] = lse_r > -__builtin_inf() ? lse_r : __builtin_inf();
        s_dl[slot][tid] = dl_r;
      }
    };

    int rows_cur = 0;
    if (n_steps > 0) {
      if constexpr (QM) {
        fetch_queries(0);
        publish_queries(0);
        fetch_queries(1);
        publish_queries(1);
        __syncthreads();
      }
      rows_cur = issue(0, 0);
      store_stats(0);
    }
    wait_copies();
    __syncthreads();
    for (int e = 0; e < n_steps; ++e) {
      const int slot = e & 1;
      int rows_next = 0;
      const bool has_next = e + 1 < n_steps;
      if (has_next) {
        rows_next = prepare(e + 1, slot ^ 1);
        fetch_queries(e + 2);
      }
      const bool computes = kh * 32 < nk_item;
      if (has_next) {
#pragma unroll
        for (int c = 0; c < 2 * G::LPW; ++c) copy_part(c);
      }
      if constexpr (D > 64) {
        // Head dim 128: one block of copies, then the matrix work row block
        // by row block (the slot schedule below does not fit its registers).
        if (computes) {
#pragma unroll 1
          for (int rh = 0; rh < 2 && rh * 64 < rows_cur; ++rh) {  // row halves
          const char* qs = sQ[slot];
          const char* os = sO[slot];
          u32x4 pb[2][2], dsb[2][2];
  #pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            const int rbase = rh * 64 + rb * 32;
            f32x16 sacc, dpacc;
  #pragma unroll
            for (int v = 0; v < 16; ++v) sacc[v] = dpacc[v] = 0.0f;
  #pragma unroll
            for (int s = 0; s < NS; ++s) {
              const int o = G::off(rbase + l32, 2 * s + hb);
              sacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(qs + o), kb[s], sacc);
              dpacc = mfma32<DT>(*reinterpret_cast<const u32x4*>(os + o), vb[s], dpacc);
            }
            float p[16], ds[16];
  #pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              // registers 4*g4 .. 4*g4+3 hold rows rbase + g4*8 + hb*4 + 0..3
              const f32x4 lv = *reinterpret_cast<const f32x4*>(
                  &s_lse[slot][rbase + g4 * 8 + hb * 4]);
              const f32x4 dv = *reinterpret_cast<const f32x4*>(
                  &s_dl[slot][rbase + g4 * 8 + hb * 4]);
  #pragma unroll
              for (int u = 0; u < 4; ++u) {
                const int v = g4 * 4 + u;
                p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[v], a.scale_log2, -lv[u]));
                ds[v] = p[v] * (dpacc[v] - dv[u]);
              }
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
          // dV^T += dO^T P and dK^T += Q^T dS: the transposed operands come
          // from the row-major tiles (slot e of lane (hb, row d) = query row
          // rh*64 + rb*32 + cc*16 + (e/4)*8 + hb*4 + e%4, the P / dS layout).
          const int gi = lane & 15, dh = (lane >> 4) & 1;
  #pragma unroll
          for (int db = 0; db < ND; ++db) {
            const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
            const int cb = dcol >> 3, half = (dcol & 4) * 2;
  #pragma unroll
            for (int rb = 0; rb < 2; ++rb)
  #pragma unroll
              for (int cc = 0; cc < 2; ++cc) {
                const int r0 = rh * 64 + rb * 32 + cc * 16 + hb * 4 + (gi >> 2);
                const int o0 = G::off(r0, cb) + half, o1 = G::off(r0 + 8, cb) + half;
                const u32x2 olo = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(os + o0)));
                const u32x2 ohi = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(os + o1)));
                dvacc[db] = mfma32<DT>(u32x4{olo[0], olo[1], ohi[0], ohi[1]},
                                       pb[rb][cc], dvacc[db]);
                const u32x2 qlo = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(qs + o0)));
                const u32x2 qhi = __builtin_bit_cast(
                    u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(qs + o1)));
                dkacc[db] = mfma32<DT>(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]},
                                       dsb[rb][cc], dkacc[db]);
              }
          }
          }  // row halves
        }
      } else if (computes) {
#pragma unroll 1
        for (int rh = rh_lo; rh < rh_hi && rh * 64 < rows_cur; ++rh) {  // row halves
        const char* qs = sQ[slot];
        const char* os = sO[slot];
        // The step's 8 * NS MFMAs in a fixed issue order, in four phases:
        //   A  S, dP of row block 0          (2 * NS)
        //   B  S, dP of row block 1          (2 * NS)   + P, dS of row block 0
        //   C  dV, dK of row block 0         (4 * ND)   + P, dS of row block 1
        //   D  dV, dK of row block 1         (4 * ND)
        // so that the vector work of one row block runs while the matrix
        // core works on the other.  Each slot issues the LDS reads of the
        // MFMA LA slots ahead, then its MFMA, then its share of the vector
        // work; scheduling barriers keep the compiler from regrouping the
        // slots.
        // dS is kept unscaled (dK is scaled once at the end).
        constexpr int NA = 2 * NS, NC = 4 * ND, NSLOT = 2 * NA + 2 * NC, LA = 2;
        f32x16 sc[2], dp[2];
        // Per-lane LDS addresses of this row half's reads (ring slot and row
        // half added once; row block, 16-row half and transposed-row offsets
        // are immediates): row-major Q / dO rows of head-dim step sk, and
        // transposed Q / dO reads (rows r0, r0 + 8) of output block db.
        const uint32_t qh = lds_addr(qs) + (uint32_t)(rh * 64 * (D * 2));
        const uint32_t oh = lds_addr(os) + (uint32_t)(rh * 64 * (D * 2));
        uint32_t rq[NS], ro[NS], tq[ND][2], to[ND][2];
#pragma unroll
        for (int sk = 0; sk < NS; ++sk) {
          rq[sk] = qh + kl_off[sk];
          ro[sk] = oh + kl_off[sk];
          asm volatile("" : "+v"(rq[sk]), "+v"(ro[sk]));
        }
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            tq[db][x] = qh + vl_off[db][x];
            to[db][x] = oh + vl_off[db][x];
            asm volatile("" : "+v"(tq[db][x]), "+v"(to[db][x]));
          }
        u32x4 pb[2][2], dsb[2][2];
        f32x4 lv[2][4], dl[2][4];
        u32x4 opnd[LA + 1];
        // Operand of MFMA i (row-major Q / dO rows for S, dP; transposed
        // dO / Q columns for dV, dK: slot e of lane (hb, row d) = query row
        // rh*64 + rb*32 + cc*16 + (e/4)*8 + hb*4 + e%4, the P / dS layout).
        auto read_op = [&](int i) __attribute__((always_inline)) {
          if (i < 2 * NA) {
            const int rb = i / NA, j = i % NA, sk = j >> 1;
            const uint32_t ad = ((j & 1) ? ro[sk] : rq[sk]) + rb * 32 * (D * 2);
            opnd[i % (LA + 1)] = *lds_ptr<u32x4>(ad);
          } else {
            const int j = (i - 2 * NA) % NC, rb = (i - 2 * NA) / NC;
            const int db = j >> 2, cc = (j >> 1) & 1;
            const uint32_t (*t)[2] = (j & 1) ? tq : to;
            const uint32_t rbc = (uint32_t)((rb * 32 + cc * 16) * (D * 2));
            const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                lds_ptr<s16x4>(t[db][0] + rbc)));
            const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                lds_ptr<s16x4>(t[db][1] + rbc)));
            opnd[i % (LA + 1)] = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
        };
        // lse / delta of score registers 4*g4 .. 4*g4+3 of row block rb
        // (rows rh*64 + rb*32 + g4*8 + hb*4 + 0..3)
        auto read_stats = [&](int rb, int g4) __attribute__((always_inline)) {
          const int r = rh * 64 + rb * 32 + g4 * 8 + hb * 4;
          lv[rb][g4] = *reinterpret_cast<const f32x4*>(&s_lse[slot][r]);
          dl[rb][g4] = *reinterpret_cast<const f32x4*>(&s_dl[slot][r]);
        };
        // Slot of softmax pair k of row block rb (pairs spread evenly over
        // phase B for block 0, phase C for block 1); the stats of a group of
        // two pairs are read three slots before its first pair.
        auto pair_slot = [](int rb, int k) constexpr {
          return rb == 0 ? NA + ((k + 1) * NA + 7) / 8 - 1
                         : 2 * NA + ((k + 1) * NC + 7) / 8 - 1;
        };
        // P and dS of elements 2k, 2k+1 of row block rb, packed.
        auto softmax_pair = [&](int rb, int k) __attribute__((always_inline)) {
          const int v0 = 2 * k, g4 = v0 >> 2, u = v0 & 3;
          const float p0 = __builtin_amdgcn_exp2f(
              __builtin_fmaf(sc[rb][v0], a.scale_log2, -lv[rb][g4][u]));
          const float p1 = __builtin_amdgcn_exp2f(
              __builtin_fmaf(sc[rb][v0 + 1], a.scale_log2, -lv[rb][g4][u + 1]));
          const float d0 = p0 * (dp[rb][v0] - dl[rb][g4][u]);
          const float d1 = p1 * (dp[rb][v0 + 1] - dl[rb][g4][u + 1]);
          pb[rb][k >> 2][k & 3] = pack2<DT>(p0, p1);
          dsb[rb][k >> 2][k & 3] = pack2<DT>(d0, d1);
        };
#pragma unroll
        for (int i = 0; i < LA; ++i) read_op(i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NSLOT; ++i) {
          if (i + LA < NSLOT) read_op(i + LA);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int at = pair_slot(rb, 2 * g4) - 3;
              if (i == (at > 0 ? at : 0)) read_stats(rb, g4);
            }
          const u32x4 op = opnd[i % (LA + 1)];
          if (i < 2 * NA) {
            const int rb = i / NA, j = i % NA, sk = j >> 1;
            if (j & 1) {
              if (sk == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) dp[rb][v] = 0.0f;
              }
              dp[rb] = mfma32<DT>(op, vb[sk], dp[rb]);
            } else {
              if (sk == 0) {
#pragma unroll
                for (int v = 0; v < 16; ++v) sc[rb][v] = 0.0f;
              }
              sc[rb] = mfma32<DT>(op, kb[sk], sc[rb]);
            }
          } else {
            const int j = (i - 2 * NA) % NC, rb = (i - 2 * NA) / NC;
            const int db = j >> 2, cc = (j >> 1) & 1;
            if (j & 1)
              dkacc[db] = mfma32<DT>(op, dsb[rb][cc], dkacc[db]);
            else
              dvacc[db] = mfma32<DT>(op, pb[rb][cc], dvacc[db]);
          }
          // vector work: row block 0 during phase B, row block 1 during C
          if (i >= NA && i < 2 * NA) {
            const int t = i - NA;
#pragma unroll
            for (int k = (t * 8) / NA; k < ((t + 1) * 8) / NA; ++k) softmax_pair(0, k);
          } else if (i >= 2 * NA && i < 2 * NA + NC) {
            const int t = i - 2 * NA;
#pragma unroll
            for (int k = (t * 8) / NC; k < ((t + 1) * 8) / NC; ++k) softmax_pair(1, k);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        }  // row halves
      }
      if (e + 1 < n_steps) store_stats(slot ^ 1);
      wait_copies();
      publish_queries(e + 2);  // s_qi[e & 1] was last read by issue(e)
      __syncthreads();
      rows_cur = rows_next;
    }
    if (rsplit) {
      // Row half 1 hands its sums to half 0 through LDS.  The Q ring is
      // free: every copy has landed and every wave has passed the last
      // step's barrier; the next item's copies follow the barrier below.
      float* red = reinterpret_cast<float*>(sQ[0]) + kh * (2 * ND * 16 * 64);
      static_assert(2 * 2 * ND * 16 * 64 * 4 <= 2 * G::BYTES, "reduction fits the Q ring");
      if (rh_lo == 1) {
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            red[((0 * ND + db) * 16 + v) * 64 + lane] = dkacc[db][v];
            red[((1 * ND + db) * 16 + v) * 64 + lane] = dvacc[db][v];
          }
      }
      __syncthreads();
      if (rh_lo == 0) {
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            dkacc[db][v] += red[((0 * ND + db) * 16 + v) * 64 + lane];
            dvacc[db][v] += red[((1 * ND + db) * 16 + v) * 64 + lane];
          }
      }
    }
    // Each wave owns its keys: dK (scaled by the softmax scale, dS was kept
    // unscaled) and dV straight from the accumulators.
    if (key_ok && rh_lo == 0) {
      const int64_t base = ((int64_t)(t0 + key) * a.hkv + h) * D;
#pragma unroll
      for (int db = 0; db < ND; ++db)
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
          float kv[4], vv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            kv[u] = a.scale * dkacc[db][gi * 4 + u];
            vv[u] = dvacc[db][gi * 4 + u];
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
  };
  if (uniform(a.plan.ghead_off[a.hkv]) > 0)
    items_loop(Phase<1>{});
  else
    items_loop(Phase<0>{});
  leave_queue_xcd(a.plan.counter + 8, a.plan.counter + 3);
}

// Key-centric dQ of blocks held whole in LDS (the forward's resident items:
// BIG = 0, four waves, blocks of 1..KC_RES_KEYS keys; BIG = 1, eight waves
// in two groups running their own chunks, blocks of KC_RES_KEYS+1 ..
// KC_RES2_KEYS keys at head dim <= 64).  The block's K and V are copied
// into LDS once per item; each chunk of up to 128 gathered rows loads its Q
// and dO rows (one chunk ahead, listings two ahead) and its rows' Delta
// (written by kc_delta_kernel), and for every key tile computes S^T = K Q^T and dP^T = V
// dO^T, dS = P (dP - Delta) with P = 2^(S scale log2 e - LSE), and dQ^T +=
// K^T dS^T: the arithmetic of the streaming gathered tiles, key tile by key
// tile in the same order.  Each row writes its share of dQ at [head, query,
// slot] for kc_dq_merge_kernel.
template <int DT, int D, int BIG>
__global__ __launch_bounds__(BIG ? 512 : 256) __attribute__((amdgpu_waves_per_eu(2, 2))) void
kc_resident_dq_kernel(AttnArgs a) {
  using G = KvTile<D>;
  constexpr int NS = D / 16;
  constexpr int ND = D / 32;
  constexpr int NT = (BIG ? KC_RES2_KEYS : KC_RES_KEYS) / KT;
  constexpr int NWG = BIG ? 2 : 1;  // groups of four waves
  constexpr bool PF = D <= 64;      // Q / dO / O rows loaded one chunk ahead
  __shared__ __align__(1024) char sK[NT][G::BYTES];
  __shared__ __align__(1024) char sV[NT][G::BYTES];
  __shared__ int s_slot;
  const int tid = threadIdx.x, lane = tid & 63, wv = uniform(tid >> 6);
  const int wg = wv >> 2, wl = wv & 3;  // wave group, wave inside the group
  const int hb = lane >> 5, l32 = lane & 31;
  // A plan built without its backward part: nothing here is valid to read.
  if (a.plan.counter[PLAN_BWD_SLOT] != PLAN_BWD_MAGIC) return;
  if (!kc_plan_ok(a)) return;  // nor without the key-centric part of this run
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
  // Lane-dependent parts of the LDS operand addresses, pinned in registers:
  // K / V row block reads per head-dim step, transposed K reads (rows k0,
  // k0 + 8) per output block.
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

    const int r = wl * 32 + l32;
    const int step = NWG * tq;
    auto chunk_ok = [&](int cbx) { return r < (n - cbx < tq ? n - cbx : tq) * a.g; };
    auto load_listing = [&](int cbx) -> int32_t {
      return cbx < n ? a.kc.grev.rev[(int64_t)h * cap + e0 + cbx + (chunk_ok(cbx) ? r / a.g : 0)]
                     : 0;
    };
    // Q, dO and O of the row of listing lv (zeros for rows outside the chunk)
    auto load_rows = [&](int cbx, int32_t lv, u32x4* qd, u32x4* dd) {
      const int64_t qx = lv / a.topk_n;
      const bool ok = cbx < n && chunk_ok(cbx);
      const int hx = h * a.g + (ok ? r % a.g : 0);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int64_t off = (qx * a.hq + hx) * D + s * 16 + hb * 8;
        qd[s] = ok ? *reinterpret_cast<const u32x4*>(a.q + off) : u32x4{0u, 0u, 0u, 0u};
        dd[s] = ok ? *reinterpret_cast<const u32x4*>(a.dout + off) : u32x4{0u, 0u, 0u, 0u};
      }
    };
    const int cb0 = wg * tq;
    int32_t lv_cur = load_listing(cb0);
    u32x4 qn_[PF ? NS : 1], dn_[PF ? NS : 1];
    if constexpr (PF) load_rows(cb0, lv_cur, qn_, dn_);
    int32_t lv_next = load_listing(cb0 + step);
    for (int cb = cb0; cb < n; cb += step) {
      const int rows = (n - cb < tq ? n - cb : tq) * a.g;
      const bool row_ok = r < rows;
      u32x4 qb[NS], dob[NS];
      if constexpr (PF) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          qb[s] = qn_[s];
          dob[s] = dn_[s];
        }
      } else {
        load_rows(cb, lv_cur, qb, dob);
      }
      const int64_t qi = lv_cur / a.topk_n;
      const int64_t slot = lv_cur - qi * a.topk_n;
      const int hh = h * a.g + (row_ok ? r % a.g : 0);
      // next chunk: its rows from the listing loaded one chunk ago; the
      // listing after it
      if constexpr (PF) load_rows(cb + step, lv_next, qn_, dn_);
      lv_cur = lv_next;
      lv_next = load_listing(cb + 2 * step);
      if (wl * 32 >= rows) continue;  // wave-uniform: no row of this chunk
      // Delta of the row's query (kc_delta_kernel); exponent bias -lse, -inf
      // (P = 0) for rows outside the chunk and rows that attend nothing.
      float delta = 0.0f;
      float bias = -__builtin_inf();
      if (row_ok) {
        delta = a.lse[(int64_t)hh * a.nq + qi];
        const float l = a.lse_in[(int64_t)hh * a.nq + qi];
        if (l > -__builtin_inf()) bias = -l;
      }
      f32x16 dqacc[ND];
#pragma unroll
      for (int i = 0; i < ND; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) dqacc[i][v] = 0.0f;
#pragma unroll
      for (int kt = 0; kt < NT; ++kt) {
        if (kt < ntiles && D <= 64) {
          // The streaming dQ kernel's fixed slot order over the resident
          // tile: S^T, dP^T of key block 0 (phase A), of key block 1 with
          // dS of block 0 (B), dQ^T += K^T dS^T of block 0 with dS of block
          // 1 (C), of block 1 (D); each MFMA's operand read two slots ahead.
          const char* ks = sK[kt];
          const char* vs = sV[kt];
          constexpr int NA = 2 * NS, NC = 2 * ND, NSLOT = 2 * NA + 2 * NC, LA = 2;
          // keys of the tile inside the block (bit p = key kt * KT + p)
          const int hi = len - kt * KT;
          const uint64_t m = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
          const bool masked = m != ~0ull;  // uniform: the block's last, partial tile
          const uint64_t mh = m >> (hb * 4);  // slot v: key (v/4)*8 + hb*4 + v%4
          f32x16 sc[2], dp[2];
          u32x4 dsb[2][2];
          u32x4 opnd[LA + 1];
          auto read_op = [&](int i) __attribute__((always_inline)) {
            if (i < 2 * NA) {
              const int blk = i / NA, j = i % NA, sk = j >> 1;
              const char* src = (j & 1) ? vs : ks;
              opnd[i % (LA + 1)] =
                  *reinterpret_cast<const u32x4*>(src + blk * 32 * (D * 2) + kl_off[sk]);
            } else {
              const int j = (i - 2 * NA) % NC, blk = (i - 2 * NA) / NC;
              const int db = j >> 1, c = j & 1;
              const int rb = (blk * 32 + c * 16) * (D * 2);
              const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(ks + rb + vl_off[db][0])));
              const u32x2 hi2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                  (lds_s16x4*)(ks + rb + vl_off[db][1])));
              opnd[i % (LA + 1)] = u32x4{lo[0], lo[1], hi2[0], hi2[1]};
            }
          };
          auto apply_mask = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
            for (int v = 0; v < 16; ++v)
              if (!((mh >> (blk * 32 + (v / 4) * 8 + (v % 4))) & 1ull))
                sc[blk][v] = -__builtin_inf();
          };
          // dS of score registers 2k, 2k+1 of key block blk, packed (kept
          // unscaled: dQ is scaled once at the end).
          auto ds_pair = [&](int blk, int k) __attribute__((always_inline)) {
            const int v0 = 2 * k;
            const float p0 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0], a.scale_log2, bias));
            const float p1 =
                __builtin_amdgcn_exp2f(__builtin_fmaf(sc[blk][v0 + 1], a.scale_log2, bias));
            dsb[blk][k >> 2][k & 3] =
                pack2<DT>(p0 * (dp[blk][v0] - delta), p1 * (dp[blk][v0 + 1] - delta));
          };
#pragma unroll
          for (int i = 0; i < LA; ++i) read_op(i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < NSLOT; ++i) {
            if (i + LA < NSLOT) read_op(i + LA);
            const u32x4 op = opnd[i % (LA + 1)];
            if (i < 2 * NA) {
              const int blk = i / NA, j = i % NA, sk = j >> 1;
              if (j & 1) {
                if (sk == 0) {
#pragma unroll
                  for (int v = 0; v < 16; ++v) dp[blk][v] = 0.0f;
                }
                dp[blk] = mfma32<DT>(op, dob[sk], dp[blk]);
              } else {
                if (sk == 0) {
#pragma unroll
                  for (int v = 0; v < 16; ++v) sc[blk][v] = 0.0f;
                }
                sc[blk] = mfma32<DT>(op, qb[sk], sc[blk]);
              }
            } else {
              const int j = (i - 2 * NA) % NC, blk = (i - 2 * NA) / NC;
              const int db = j >> 1, c = j & 1;
              dqacc[db] = mfma32<DT>(op, dsb[blk][c], dqacc[db]);
            }
            if (i == NA && masked) apply_mask(0);
            if (i == 2 * NA && masked) apply_mask(1);
            if (i >= NA && i < 2 * NA) {
              const int t = i - NA;
#pragma unroll
              for (int k = (t * 8) / NA; k < ((t + 1) * 8) / NA; ++k) ds_pair(0, k);
            } else if (i >= 2 * NA && i < 2 * NA + NC) {
              const int t = i - 2 * NA;
#pragma unroll
              for (int k = (t * 8) / NC; k < ((t + 1) * 8) / NC; ++k) ds_pair(1, k);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        } else if (kt < ntiles) {
          const char* ks = sK[kt];
          const char* vs = sV[kt];
          f32x16 sacc[2], dpacc[2];
          const int nblk = kt * KT + 32 < len ? 2 : 1;  // halves holding keys (dS = 0 past)
#pragma unroll
          for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[blk][v] = dpacc[blk][v] = 0.0f;
            if (blk < nblk) {
#pragma unroll
              for (int s = 0; s < NS; ++s) {
                const int o = G::off(blk * 32 + l32, 2 * s + hb);
                sacc[blk] = mfma32<DT>(*reinterpret_cast<const u32x4*>(ks + o), qb[s], sacc[blk]);
                dpacc[blk] = mfma32<DT>(*reinterpret_cast<const u32x4*>(vs + o), dob[s], dpacc[blk]);
              }
            }
          }
          if (kt * KT + KT > len) {
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                if (kt * KT + blk * 32 + acc_row(v, hb) >= len) sacc[blk][v] = -__builtin_inf();
          }
          u32x4 dsb[2][2];
#pragma unroll
          for (int blk = 0; blk < 2; ++blk) {
            float ds[16];
#pragma unroll
            for (int v = 0; v < 16; ++v)
              ds[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[blk][v], a.scale_log2, bias)) *
                      (dpacc[blk][v] - delta);
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
              dsb[blk][cc] = u32x4{pack2<DT>(ds[cc * 8 + 0], ds[cc * 8 + 1]),
                                   pack2<DT>(ds[cc * 8 + 2], ds[cc * 8 + 3]),
                                   pack2<DT>(ds[cc * 8 + 4], ds[cc * 8 + 5]),
                                   pack2<DT>(ds[cc * 8 + 6], ds[cc * 8 + 7])};
          }
          // dQ^T += K^T dS^T: K^T by transposed reads (slot e of lane (hb,
          // row d) = key blk*32 + cc*16 + (e/4)*8 + hb*4 + e%4, the score
          // layout).
          const int gi = lane & 15, dh = (lane >> 4) & 1;
#pragma unroll
          for (int db = 0; db < ND; ++db) {
            const int dcol = db * 32 + dh * 16 + (gi & 3) * 4;
            const int cbk = dcol >> 3, half = (dcol & 4) * 2;
#pragma unroll
            for (int blk = 0; blk < 2; ++blk)
              if (blk < nblk)
#pragma unroll
              for (int cc = 0; cc < 2; ++cc) {
                const int k0 = blk * 32 + cc * 16 + hb * 4 + (gi >> 2);
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(ks + G::off(k0, cbk) + half));
                const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)(ks + G::off(k0 + 8, cbk) + half));
                const u32x2 lw = __builtin_bit_cast(u32x2, lo);
                const u32x2 hw = __builtin_bit_cast(u32x2, hi);
                dqacc[db] = mfma32<DT>(u32x4{lw[0], lw[1], hw[0], hw[1]}, dsb[blk][cc], dqacc[db]);
              }
          }
        }
      }
      if (row_ok) {
        uint16_t* drow = a.kc.part_o + a.kc.pidx(h, qi, slot, a.topk_n, a.g, r % a.g) * D;
#pragma unroll
        for (int db = 0; db < ND; ++db)
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            const int v = gi * 4;
            // dS was kept unscaled: dQ = scale * (dS' K)
            *reinterpret_cast<u32x2*>(drow + db * 32 + gi * 8 + hb * 4) =
                u32x2{pack2<DT>(a.scale * dqacc[db][v], a.scale * dqacc[db][v + 1]),
                      pack2<DT>(a.scale * dqacc[db][v + 2], a.scale * dqacc[db][v + 3])};
          }
      }
    }
    __syncthreads();  // the item's reads of sK / sV end before the next copies
  }
  wait_copies();
  leave_queue(queue, queue + 2);
}

// Delta = rowsum(O dO) of the rows of the marked queries (key-centric
// plans), once per row, for the resident dQ kernels (which then gather only
// the Q and dO rows of a listing): one thread per (kv head, query, query
// head), 16-byte loads, fp32 sum in channel order.
template <int DT, int D>
__global__ __launch_bounds__(256) void kc_delta_kernel(AttnArgs a) {
  if (a.plan.counter[PLAN_BWD_SLOT] != PLAN_BWD_MAGIC || !kc_plan_ok(a)) return;
  const int64_t n_items = (int64_t)a.hkv * a.nq * a.g;
  for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < n_items;
       it += (int64_t)gridDim.x * blockDim.x) {
    const int64_t hq_idx = it / a.g;  // h * nq + q
    if (!a.kc.qmark[hq_idx]) continue;
    const int gi = (int)(it - hq_idx * a.g);
    const int h = (int)(hq_idx / a.nq);
    const int64_t q = hq_idx - (int64_t)h * a.nq;
    const int hh = h * a.g + gi;
    const uint16_t* orow = a.o + (q * a.hq + hh) * D;
    const uint16_t* drow = a.dout + (q * a.hq + hh) * D;
    float dl = 0.0f;
#pragma unroll
    for (int c = 0; c < D; c += 8) {
      const u32x4 ov = *reinterpret_cast<const u32x4*>(orow + c);
      const u32x4 dv = *reinterpret_cast<const u32x4*>(drow + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dl += to_f32<DT>((uint16_t)(ov[e] & 0xffffu)) * to_f32<DT>((uint16_t)(dv[e] & 0xffffu));
        dl += to_f32<DT>((uint16_t)(ov[e] >> 16)) * to_f32<DT>((uint16_t)(dv[e] >> 16));
      }
    }
    a.lse[(int64_t)hh * a.nq + q] = dl;
  }
}

// Key-centric dQ merge: one thread per (kv head, query, query head, 8
// channels) of the marked queries; the slot shares of dQ written by the
// gathered tiles are added in slot order in fp32 and rounded once.  Slots
// are taken 16 at a time with their ids and shares loaded together (a slot
// without a block is loaded and ignored: the buffer covers every slot).
// These rows' Delta was written by kc_delta_kernel.
template <int DT, int D>
__global__ __launch_bounds__(256) void kc_dq_merge_kernel(AttnArgs a) {
  constexpr int CPT = 8;  // output channels per thread: one 16-byte load per slot
  constexpr int U = 16;   // slots whose shares are loaded together
  if (a.plan.counter[PLAN_BWD_SLOT] != PLAN_BWD_MAGIC || !kc_plan_ok(a)) return;
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
    float acc[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) acc[c] = 0.0f;
    for (int j0 = 0; j0 < a.topk_n; j0 += U) {
      int v[U];
      u32x4 pv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u;
        const bool in = j < a.topk_n;
        v[u] = in ? row[j] : -1;
        const int64_t pidx = (hq_rel * a.topk_n + (in ? j : 0)) * a.g + gi;
        pv[u] = *reinterpret_cast<const u32x4*>(a.kc.part_o + pidx * D + d0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (!(v[u] >= 0 && v[u] < nbb && (int64_t)bs + v[u] < a.nb)) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[2 * e] += to_f32<DT>((uint16_t)(pv[u][e] & 0xffffu));
          acc[2 * e + 1] += to_f32<DT>((uint16_t)(pv[u][e] >> 16));
        }
      }
    }
    const int hh = h * a.g + gi;
    *reinterpret_cast<u32x4*>(a.out + (q * a.hq + hh) * D + d0) =
        u32x4{pack2<DT>(acc[0], acc[1]), pack2<DT>(acc[2], acc[3]), pack2<DT>(acc[4], acc[5]),
              pack2<DT>(acc[6], acc[7])};
  }
}

template <int DT, int D>
int launch_bwd_t(const AttnArgs& a, hipStream_t st) {
  {
    const void* fn = reinterpret_cast<const void*>(&sel_attn_dq_kernel<DT, D, DQ_RUN>);
    const int grid = persistent_grid(fn, 256, 0);
    if (grid <= 0) return LSRM_ERR_LAUNCH;
    hipLaunchKernelGGL((sel_attn_dq_kernel<DT, D, DQ_RUN>), dim3(grid), dim3(256), 0,
                       st, a);
    LSRM_CHECK_LAUNCH();
  }
  if (a.plan.gtiles && !a.kc.fitems) {  // the grouped tiles (key-centric plans: gathered)
    const void* fn = reinterpret_cast<const void*>(&sel_attn_dq_kernel<DT, D, DQ_UNION>);
    const int grid = persistent_grid(fn, 256, 0);
    if (grid <= 0) return LSRM_ERR_LAUNCH;
    hipLaunchKernelGGL((sel_attn_dq_kernel<DT, D, DQ_UNION>), dim3(grid), dim3(256), 0,
                       st, a);
    LSRM_CHECK_LAUNCH();
  }
  if (a.kc.fitems) {  // key-centric plans: Delta, gathered dQ tiles, then the merge
    {
      const int64_t items = (int64_t)a.hkv * a.nq * a.g;
      const int64_t gd = std::min<int64_t>((items + 255) / 256 > 0 ? (items + 255) / 256 : 1,
                                           (int64_t)device_cu_count() * 64);
      hipLaunchKernelGGL((kc_delta_kernel<DT, D>), dim3((unsigned)gd), dim3(256), 0, st, a);
      LSRM_CHECK_LAUNCH();
    }
    const void* fn = reinterpret_cast<const void*>(&sel_attn_dq_kernel<DT, D, DQ_GATHER>);
    const int grid = persistent_grid(fn, 256, 0);
    const void* fr = reinterpret_cast<const void*>(&kc_resident_dq_kernel<DT, D, 0>);
    const int gr = persistent_grid(fr, 256, 0);
    int gr2 = 1;
    if constexpr (kc_res_max(D) > KC_RES_KEYS)
      gr2 = persistent_grid(reinterpret_cast<const void*>(&kc_resident_dq_kernel<DT, D, 1>),
                            512, 0);
    const int gm = device_cu_count() * 16;
    if (grid <= 0 || gr <= 0 || gr2 <= 0 || gm <= 0) return LSRM_ERR_LAUNCH;
    // One range of queries at a time: its gathered dQ shares, then their
    // merge, before the next range reuses the partial buffer; the streaming
    // and eight-wave kernels run on a second stream beside the four-wave one
    // (disjoint partials), as in the forward.
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
        hipLaunchKernelGGL((kc_resident_dq_kernel<DT, D, 1>), dim3(gr2), dim3(512), 0, s2, ap);
        LSRM_CHECK_LAUNCH();
      }
      hipLaunchKernelGGL((sel_attn_dq_kernel<DT, D, DQ_GATHER>), dim3(grid), dim3(256), 0,
                         s2, ap);
      LSRM_CHECK_LAUNCH();
      hipLaunchKernelGGL((kc_resident_dq_kernel<DT, D, 0>), dim3(gr), dim3(256), 0, st, ap);
      LSRM_CHECK_LAUNCH();
      if (two && (hipEventRecord(ss.join, ss.s) != hipSuccess ||
                  hipStreamWaitEvent(st, ss.join, 0) != hipSuccess))
        return LSRM_ERR_LAUNCH;
      hipLaunchKernelGGL((kc_dq_merge_kernel<DT, D>), dim3(gm), dim3(256), 0, st, ap);
      LSRM_CHECK_LAUNCH();
    }
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
