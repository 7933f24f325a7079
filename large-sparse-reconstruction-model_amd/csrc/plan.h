// Device-side planning shared by the selected-attention kernels: query tiles
// (runs of identical top-k rows cut into pieces of at most TQ queries) and
// reverse (CSR) maps from blocks to the rows that selected them.
#pragma once

#include "common.h"

namespace lsrm {

// Queries of one kv head that share a selection row: [q0, q0 + qn) as
// int2 {q0, qn}.  A forward plan also lists grouped tiles: consecutive short
// runs of one batch element whose rows differ, run over the union of their
// blocks (a second work queue).
struct TilePlan {
  int2* tiles;           // [hkv, n_q]; tile t of head h at tiles[h * n_q + t]
  int32_t* tile_count;   // [hkv]
  int32_t* head_off;     // [hkv + 1] exclusive prefix of tile_count
  int32_t* counter;      // work counters, zeroed by the plan: [0], [2] run
                         // tiles (fwd / dq), [8..15], [3] key chunks (dK/dV,
                         // one queue per XCD), [4], [6] grouped tiles;
                         // [PLAN_BWD_SLOT] = PLAN_BWD_MAGIC once the backward
                         // part (reverse maps, key chunks) is built
  int2* gtiles;          // [hkv, n_q] grouped tiles (forward plans)
  int32_t* gtile_count;  // [hkv]
  int32_t* ghead_off;    // [hkv + 1]
};

// Marks a plan whose backward part was built: the backward kernels exit
// without touching memory when the slot does not hold the magic word (a
// forward-only plan in a workspace large enough for the backward).
constexpr int PLAN_BWD_SLOT = 32;
constexpr int32_t PLAN_BWD_MAGIC = 0x4c42574b;
int mark_backward_plan(int32_t* counter, hipStream_t st);

// CSR map block -> rows (tiles or queries) that selected it, per kv head.
struct RevMap {
  int32_t* cu_rev;  // [hkv, n_blocks + 1]
  int32_t* rev;     // [hkv, cap]
  int32_t* totals;  // [hkv]
  int64_t cap;
};

// Workspace carving: pass a Carver with base == nullptr to size.
// group_short: move consecutive short run tiles into grouped tiles.
int build_tile_plan(const int32_t* topk, int64_t hkv, int64_t nq,
                    int64_t topk_n, const int32_t* cu_q, int64_t batch,
                    const int32_t* cu_sb, int tq, Carver& ws, TilePlan& plan,
                    hipStream_t st, bool group_short = false);

// rows_are_tiles: rows are the tiles of `plan` (row r of head h reads the
// selection of query tiles[h*nq + r].x); otherwise rows are queries, and
// with `only` (a [hkv, nq] byte mask) only the queries it marks.
// encode_slot (rows are queries): a listing stores q * topk_n + j, j the
// slot of the row that lists the block (ascending order is unchanged).
int build_reverse_map(const int32_t* topk, int64_t hkv, int64_t nq,
                      int64_t topk_n, const int32_t* cu_q, int64_t batch,
                      const int32_t* cu_sb, int64_t nb, bool rows_are_tiles,
                      const TilePlan* plan, Carver& ws, RevMap& map,
                      hipStream_t st, const uint8_t* only = nullptr,
                      bool encode_slot = false);

// flags[h, q] = 1 for the queries of the grouped tiles of `plan`, else 0.
int mark_grouped_queries(const TilePlan& plan, int64_t hkv, int64_t nq,
                         uint8_t* flags, hipStream_t st);

// Key-centric part of a plan (plan flag LSRM_PLAN_KEY_CENTRIC): the grouped
// tiles are taken out of the grouped-tile kernels (which a key-centric plan
// does not launch); their queries are listed per block (`grev`, ascending, one
// listing q * topk + j per slot j that names the block), and each block's
// list is cut into items {c, e0, n, 0} = block c, listings e0 .. e0 + n of
// grev's segment of head h.  The forward writes one partial result per
// (query, slot, query head) -- O normalised by its own row sum in the input
// type and its log2 LSE -- and the dQ pass the slot's share of dQ; merge
// passes combine each query's partials in slot order.
//
// The partial buffer holds the rows of one pass, sized so that a pass's
// partials stay within KC_PART_BUDGET bytes: when one kv head's partials
// fit, pass p takes kv heads [p * pass_heads, (p + 1) * pass_heads) with all
// their queries (every block's listings stay in one pass); otherwise pass p
// takes queries [p * q_span_max, (p + 1) * q_span_max) of every head (items
// are then cut at the range's bounds).  Each pass's gathered tiles run and
// merge before the next pass reuses the buffer.  The item lists are stored
// per (pass, kv head): entry (p, h) of a list is "head" p * hkv + h.
struct KcPlan {
  uint8_t* qmark;        // [hkv, n_q] queries of grouped tiles
  RevMap grev;           // block -> marked queries, cap = n_q * topk per head
  uint16_t* part_o;      // [hkv, q_span_max, topk, g, D] input type
  float* part_lse;       // [hkv, q_span_max, topk, g]
  int n_pass;
  int64_t q_span_max;
  int pass_heads;  // kv heads per pass (head passes), 0 for query passes
  // the pass a launch works on (set by the launcher): queries
  // [q_base, q_base + q_span) of kv heads [h_base, h_base + h_count); the
  // item lists below then point at that pass's entries
  int64_t q_base, q_span;
  int h_base, h_count;
  // Items of blocks with 1..KC_RES_KEYS keys, run with the block resident
  // in LDS (forward and dQ): up to KC_RES_CHUNKS * tq listings each.
  int4* ritems;          // [n_pass * hkv, ritem_cap]
  int64_t ritem_cap;
  int32_t* ritem_count;  // [n_pass * hkv]
  int32_t* ritem_off;    // [n_pass, hkv + 1]
  // The same for blocks of KC_RES_KEYS + 1 .. KC_RES2_KEYS keys (head dim
  // <= 64; empty otherwise), run by the eight-wave resident kernels.
  int4* r2items;
  int64_t r2item_cap;
  int32_t* r2item_count;  // [n_pass * hkv]
  int32_t* r2item_off;    // [n_pass, hkv + 1]
  // The streaming gathered tiles' items: blocks the resident kernels do not
  // take (no keys, or more than kc_res_max of the plan's head dim), at most
  // tq listings each.  fitems is null in plans without this part.
  int4* fitems;
  int64_t fitem_cap;
  int32_t* fitem_count;  // [n_pass * hkv]
  int32_t* fitem_off;    // [n_pass, hkv + 1]

  // The plan's pass p: the item lists of that pass and its query range.
  __host__ __device__ KcPlan pass(int p, int64_t hkv, int64_t n_q) const {
    KcPlan k = *this;
    if (pass_heads > 0) {
      k.h_base = p * pass_heads;
      k.h_count = (int)(hkv - k.h_base < pass_heads ? hkv - k.h_base : pass_heads);
      k.q_base = 0;
      k.q_span = n_q;
    } else {
      k.h_base = 0;
      k.h_count = (int)hkv;
      k.q_base = p * q_span_max;
      k.q_span = n_q - k.q_base < q_span_max ? n_q - k.q_base : q_span_max;
    }
    k.ritems = ritems + p * hkv * ritem_cap;
    k.ritem_off = ritem_off + p * (hkv + 1);
    k.r2items = r2items + p * hkv * r2item_cap;
    k.r2item_off = r2item_off + p * (hkv + 1);
    k.fitems = fitems + p * hkv * fitem_cap;
    k.fitem_off = fitem_off + p * (hkv + 1);
    return k;
  }
  // Index of the partial of (kv head h, query q of this pass, slot, query
  // head gi of the group) in part_lse (times D in part_o).
  __device__ int64_t pidx(int h, int64_t q, int64_t slot, int topk, int g, int gi) const {
    return (((int64_t)(h - h_base) * q_span + (q - q_base)) * topk + slot) * g + gi;
  }
};
// Bytes of key-centric partial results one pass may hold.
constexpr int64_t KC_PART_BUDGET = int64_t{1} << 30;
// Work counters of the gathered-tile kernels inside TilePlan::counter.
constexpr int KC_QUEUE_SLOT = 16, KC_EXIT_SLOT = 18;
constexpr int KC_RQUEUE_SLOT = 20, KC_REXIT_SLOT = 22;
constexpr int KC_R2QUEUE_SLOT = 24, KC_R2EXIT_SLOT = 26;
constexpr int KC_RES_KEYS = 256;   // 4 key tiles of K and V resident in LDS
constexpr int KC_RES2_KEYS = 512;  // 8 key tiles (head dim <= 64: 128 KB of LDS)
constexpr int KC_RES_CHUNKS = 16;  // query chunks of tq listings per resident item
// Largest block the resident forward takes at head dim d; larger blocks run
// as streaming gathered tiles.
__host__ __device__ constexpr int kc_res_max(int d) { return d <= 64 ? KC_RES2_KEYS : KC_RES_KEYS; }
// Marks a plan whose key-centric part was built, with the plan flags and the
// head dim's resident-block limit it was built for: the key-centric kernels
// exit without touching memory unless the slot holds the marker of the flags
// and head dim they run with (a plan built without the part, with other
// flags -- a different workspace carving -- or for a head dim whose blocks
// of 257..512 keys take another kernel).
constexpr int PLAN_KC_SLOT = 33;
__host__ __device__ constexpr int32_t kc_plan_marker(int flags, int head_dim) {
  return (int32_t)(0x4b430000 | ((flags & 3) << 12) | kc_res_max(head_dim));
}

// plain = enc with every listing q * topk + slot replaced by q (the same
// blocks, counts and order: the map of the same queries without slots).
int derive_query_map(const RevMap& enc, const RevMap& plain, int64_t hkv, int64_t nb,
                     int64_t topk_n, hipStream_t st);
// Passes of a key-centric plan so that one pass's partials fit
// KC_PART_BUDGET: kv heads per pass (0: query ranges), queries per pass.
void kc_passes(int64_t n_q, int64_t hkv, int64_t topk, int g, int64_t head_dim, int* n_pass,
               int* pass_heads, int64_t* q_span);
int build_kc_items(const RevMap& grev, const int32_t* cu_blk, int64_t nk, int64_t hkv,
                   int64_t nb, int tq, int64_t head_dim, int64_t topk_n, Carver& ws,
                   KcPlan& kc, int32_t* counter, int32_t marker, hipStream_t st);

// Key chunks of at most KEY_CHUNK tokens inside each block (head
// independent): item i = (block, first token, length) packed in an int4
// {c, t0, len, 0}.
constexpr int KEY_CHUNK = 128;
struct KeyItems {
  int4* items;        // [n_blocks + n_k / KEY_CHUNK + 2]
  int32_t* n_items;   // device scalar
};
int build_key_items(const int32_t* cu_blk, int64_t nb, int64_t nk, Carver& ws,
                    KeyItems& ki, hipStream_t st);

int launch_zero_i32(int32_t* p, int64_t n, hipStream_t st);

// Batch element owning query i (cu_q ascending), clamped to [0, batch).
__device__ inline int batch_of(const int32_t* cu_q, int64_t batch, int64_t i) {
  int64_t b = upper_index(cu_q, 0, batch + 1, i);
  if (b < 0) b = 0;
  if (b >= batch) b = batch - 1;
  return (int)b;
}

// Query i's batch element and its block range; nbb = 0 when i lies outside
// every sequence.
__device__ inline void query_batch(const int32_t* cu_q, int64_t batch,
                                   const int32_t* cu_sb, int64_t i, int* b_out,
                                   int* bs_out, int* nbb_out,
                                   bool* seq_start) {
  if (batch <= 0 || i < cu_q[0] || i >= cu_q[batch]) {
    *b_out = -1;
    *bs_out = 0;
    *nbb_out = 0;
    *seq_start = true;
    return;
  }
  const int b = batch_of(cu_q, batch, i);
  *b_out = b;
  *bs_out = cu_sb[b];
  const int nbb = cu_sb[b + 1] - cu_sb[b];
  *nbb_out = nbb > 0 ? nbb : 0;
  *seq_start = (i == cu_q[b]);
}

}  // namespace lsrm
