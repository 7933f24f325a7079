// Pieces shared by the selected-attention forward and backward kernels.
//
// A query tile is a run of queries of one kv head whose top-k rows are
// identical (tiles come from the device-side plan).  Its rows are
// (query, query head) pairs: row r <-> query q0 + r / g, head h * g + r % g,
// 128 rows per tile, 32 rows per wave.  The tile attends to the key stream
// formed by concatenating the token ranges of its valid selected blocks in
// list order; the stream is processed in 64-key LDS tiles, so only the very
// last key tile of a query tile is partial.
#pragma once

#include <mutex>

#include "common.h"
#include "plan.h"

namespace lsrm {

constexpr int KT = 64;       // keys per LDS tile
constexpr int ROWS = 128;    // rows per query tile (4 waves x 32)
constexpr int MAXSEL = 256;  // top-k entries per row supported

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;    // forward output (backward only)
  const uint16_t* dout; // backward only
  const float* lse_in;  // backward only
  uint16_t* out;        // forward: O; backward dq kernel: dQ
  float* lse;           // forward: LSE; backward: delta
  uint16_t* dk;
  uint16_t* dv;
  const int32_t* topk;
  const int32_t* cu_sb;
  const int32_t* cu_blk;
  const int32_t* cu_q;
  int64_t nb, batch, nq, nk;
  int topk_n, hq, hkv, g;
  float scale;       // softmax scale
  float scale_log2;  // softmax scale * log2(e)
  TilePlan plan;
  RevMap rev;        // backward: block -> run tiles that selected it
  RevMap qrev;       // backward: block -> queries of grouped tiles that
                     // selected it (one entry per listing, ascending)
  KeyItems items;    // backward: key chunks of every block
  KcPlan kc;         // key-centric plans only (kc.fitems null otherwise)
  int32_t kc_marker; // kc_plan_marker of the flags and head dim of this run
};

// A key-centric kernel runs only on a plan whose key-centric part was built
// for this run's flags and head dim (see PLAN_KC_SLOT).
__device__ inline bool kc_plan_ok(const AttnArgs& a) {
  return a.plan.counter[PLAN_KC_SLOT] == a.kc_marker;
}

// Compile-time value tag (e.g. a ring-slot phase).
template <int V>
struct Phase {
  static constexpr int value = V;
};

// Valid selected blocks of one selection row, compacted, with the prefix of
// their lengths (the key stream).
struct SelLds {
  int tok[MAXSEL];
  int cum[MAXSEL + 2];  // cum[n] = total keys, cum[n + 1] = INT_MAX sentinel
  int tb[MAXSEL + 1];   // tok[i] - cum[i]: token of stream position p in
                        // segment i is p + tb[i]; tb[n] = 0
  int len_tmp[MAXSEL];
  int tok_tmp[MAXSEL];
  int n;
};

// All 256 threads: reads row `q` of kv head h and fills s.  Entries that are
// invalid or name an empty block are dropped; list order is kept.
__device__ inline void load_selection(const AttnArgs& a, int h, int64_t q,
                                      SelLds& s) {
  const int tid = threadIdx.x, lane = tid & 63;
  int b, bs, nbb;
  bool st;
  query_batch(a.cu_q, a.batch, a.cu_sb, q, &b, &bs, &nbb, &st);
  const int32_t* row = a.topk + ((int64_t)h * a.nq + q) * a.topk_n;
  for (int j = tid; j < a.topk_n; j += blockDim.x) {
    const int v = row[j];
    int len = 0, t0 = 0;
    if (v >= 0 && v < nbb && (int64_t)bs + v < a.nb) {
      int64_t s0 = a.cu_blk[bs + v], s1 = a.cu_blk[bs + v + 1];
      s0 = s0 < 0 ? 0 : (s0 > a.nk ? a.nk : s0);
      s1 = s1 < s0 ? s0 : (s1 > a.nk ? a.nk : s1);
      t0 = (int)s0;
      len = (int)(s1 - s0);
    }
    s.len_tmp[j] = len;
    s.tok_tmp[j] = t0;
  }
  __syncthreads();
  if (tid < 64) {
    int cn = 0, cc = 0;
    for (int base = 0; base < a.topk_n; base += 64) {
      const int j = base + lane;
      int len = 0, t0 = 0;
      if (j < a.topk_n) {
        len = s.len_tmp[j];
        t0 = s.tok_tmp[j];
      }
      const bool keep = len > 0;
      const unsigned long long m = __ballot(keep);
      const int pos = cn + __popcll(m & ((1ull << lane) - 1ull));
      int x = len;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      if (keep) {
        s.tok[pos] = t0;
        s.cum[pos + 1] = cc + x;
        s.tb[pos] = t0 - (cc + x - len);
      }
      cn += __popcll(m);
      cc += __shfl(x, 63);
    }
    if (lane == 0) {
      s.cum[0] = 0;
      s.cum[cn + 1] = 0x7fffffff;
      s.tb[cn] = 0;
      s.n = cn;
    }
  }
  __syncthreads();
}

// All 256 threads: the key stream of one block (global id c, token range
// clamped as load_selection does), for the gathered tiles of key-centric
// plans.
__device__ inline void load_block(const AttnArgs& a, int c, SelLds& s) {
  if (threadIdx.x == 0) {
    int64_t s0 = a.cu_blk[c], s1 = a.cu_blk[c + 1];
    s0 = s0 < 0 ? 0 : (s0 > a.nk ? a.nk : s0);
    s1 = s1 < s0 ? s0 : (s1 > a.nk ? a.nk : s1);
    s.cum[0] = 0;
    if (s1 > s0) {
      s.tok[0] = (int)s0;
      s.tb[0] = (int)s0;
      s.cum[1] = (int)(s1 - s0);
      s.cum[2] = 0x7fffffff;
      s.tb[1] = 0;
      s.n = 1;
    } else {
      s.cum[1] = 0x7fffffff;
      s.tb[0] = 0;
      s.n = 0;
    }
  }
  __syncthreads();
}

// ------------------------------------------------ grouped (union) tiles --
// A TILE_GROUPED tile holds consecutive queries whose selection rows differ.
// build_union() collects the union of their selected blocks (ascending block
// id, each block once) as the tile's key stream in SelLds, and for every
// union segment the set of the tile's queries that selected it.  The tile is
// then either run once over the union, each query masked to its own blocks
// (UnionLds::ok), or once per run of identical rows.
constexpr int UMAXW = 256;  // bitmap words: batch elements of <= 8192 blocks

struct UnionLds {
  uint32_t bits[UMAXW];         // selected batch-local block ids
  int word_off[UMAXW];          // exclusive prefix of popcount(bits)
  uint32_t seg_q[MAXSEL][4];    // segment s: bit q = tile query q selected it
  int run_start[ROWS + 1];      // tile-local query offsets where runs begin
  int n_runs, n_union, dup, run_keys, feasible, ok;
};

// Length and first token of batch-local block v of batch element (bs, nbb),
// clamped as load_selection does; len 0 for an invalid or empty block.
__device__ inline void block_span(const AttnArgs& a, int bs, int nbb, int v, int& t0,
                                  int& len) {
  t0 = 0;
  len = 0;
  if (v >= 0 && v < nbb && (int64_t)bs + v < a.nb) {
    int64_t s0 = a.cu_blk[bs + v], s1 = a.cu_blk[bs + v + 1];
    s0 = s0 < 0 ? 0 : (s0 > a.nk ? a.nk : s0);
    s1 = s1 < s0 ? s0 : (s1 > a.nk ? a.nk : s1);
    t0 = (int)s0;
    len = (int)(s1 - s0);
  }
}

// All 256 threads.  Queries q0 .. q0+qn-1 of kv head h (one batch element,
// qn <= ROWS).  Fills s (the union stream) and u; u.ok says whether one
// masked pass over the union is valid and no more keys than the runs' own
// streams together (valid: the union has at most MAXSEL blocks, the batch
// element at most UMAXW * 32 blocks, and no row lists a block twice --
// repeated ids count twice and need the run-by-run passes).
__device__ inline void build_union(const AttnArgs& a, int h, int64_t q0, int qn,
                                   SelLds& s, UnionLds& u) {
  const int tid = threadIdx.x, lane = tid & 63;
  int b, bs, nbb;
  bool st;
  query_batch(a.cu_q, a.batch, a.cu_sb, q0, &b, &bs, &nbb, &st);
  const int nw = (nbb + 31) / 32;
  const bool feasible = nw <= UMAXW;
  for (int i = tid; i < UMAXW; i += blockDim.x) u.bits[i] = 0u;
  if (tid == 0) {
    u.dup = 0;
    u.run_keys = 0;
    u.feasible = feasible ? 1 : 0;
  }
  __syncthreads();
  const int32_t* rows = a.topk + ((int64_t)h * a.nq + q0) * a.topk_n;
  // Selected blocks (bitmap) and the run structure with each run's keys.
  for (int e = tid; e < qn * a.topk_n; e += blockDim.x) {
    int t0, len;
    const int v = rows[e];
    block_span(a, bs, nbb, v, t0, len);
    if (len > 0 && feasible) atomicOr(&u.bits[v >> 5], 1u << (v & 31));
  }
  for (int q = tid; q < qn; q += blockDim.x) {
    const int32_t* r1 = rows + (int64_t)q * a.topk_n;
    bool start = q == 0;
    if (!start) {
      const int32_t* r0 = r1 - a.topk_n;
      for (int j = 0; j < a.topk_n; ++j) {
        const int x = (r1[j] >= 0 && r1[j] < nbb) ? r1[j] : -1;
        const int y = (r0[j] >= 0 && r0[j] < nbb) ? r0[j] : -1;
        if (x != y) {
          start = true;
          break;
        }
      }
    }
    u.word_off[q] = start ? 1 : 0;  // run-start flags, compacted below
    if (start) {
      int keys = 0;
      for (int j = 0; j < a.topk_n; ++j) {
        int t0, len;
        block_span(a, bs, nbb, r1[j], t0, len);
        keys += len;
      }
      atomicAdd(&u.run_keys, keys);
    }
  }
  __syncthreads();
  // Run starts in query order (one wave; qn <= ROWS).
  if (tid < 64) {
    int cnt = 0;
    for (int base = 0; base < qn; base += 64) {
      const int q = base + lane;
      const bool f = q < qn && u.word_off[q] != 0;
      const unsigned long long m = __ballot(f);
      if (f) u.run_start[cnt + __popcll(m & ((1ull << lane) - 1ull))] = q;
      cnt += __popcll(m);
    }
    if (lane == 0) {
      u.run_start[cnt] = qn;
      u.n_runs = cnt;
    }
  }
  __syncthreads();
  // Ranks of the selected blocks: exclusive prefix of the word popcounts.
  if (tid < 64) {
    int carry = 0;
    for (int base = 0; base < UMAXW; base += 64) {
      const int i = base + lane;
      const int c = i < nw ? __popc(u.bits[i]) : 0;
      int x = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      u.word_off[i] = carry + x - c;
      carry += __shfl(x, 63);
    }
    if (lane == 0) u.n_union = carry;
  }
  __syncthreads();
  const int nu = u.n_union;
  const bool fits = feasible && nu <= MAXSEL;
  if (fits) {
    for (int i = tid; i < nu * 4; i += blockDim.x) u.seg_q[i >> 2][i & 3] = 0u;
    for (int i = tid; i < nw; i += blockDim.x) {
      uint32_t m = u.bits[i];
      int rank = u.word_off[i];
      while (m) {
        const int bit = __ffs(m) - 1;
        m &= m - 1u;
        int t0, len;
        block_span(a, bs, nbb, i * 32 + bit, t0, len);
        s.tok_tmp[rank] = t0;
        s.len_tmp[rank] = len;
        ++rank;
      }
    }
  }
  __syncthreads();
  if (fits) {
    // Membership; a block listed twice by one query needs the run passes.
    for (int e = tid; e < qn * a.topk_n; e += blockDim.x) {
      const int q = e / a.topk_n;
      int t0, len;
      const int v = rows[e];
      block_span(a, bs, nbb, v, t0, len);
      if (len > 0) {
        const uint32_t w = u.bits[v >> 5];
        const int rank = u.word_off[v >> 5] + __popc(w & ((1u << (v & 31)) - 1u));
        const uint32_t bit = 1u << (q & 31);
        if (atomicOr(&u.seg_q[rank][q >> 5], bit) & bit) u.dup = 1;
      }
    }
  }
  // The union stream: tok / cum / tb as load_selection builds them.
  if (tid < 64 && fits) {
    int cc = 0;
    for (int base = 0; base < nu; base += 64) {
      const int j = base + lane;
      const int len = j < nu ? s.len_tmp[j] : 0;
      const int t0 = j < nu ? s.tok_tmp[j] : 0;
      int x = len;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
      }
      if (j < nu) {
        s.tok[j] = t0;
        s.cum[j + 1] = cc + x;
        s.tb[j] = t0 - (cc + x - len);
      }
      cc += __shfl(x, 63);
    }
    if (lane == 0) {
      s.cum[0] = 0;
      s.cum[nu + 1] = 0x7fffffff;
      s.tb[nu] = 0;
      s.n = nu;
    }
  }
  __syncthreads();
  if (tid == 0)
    u.ok = (fits && !u.dup && s.cum[nu] <= u.run_keys) ? 1 : 0;
  __syncthreads();
}

// Token of stream position p (< total keys); `cur` is a monotone cursor.
__device__ inline int stream_token(const SelLds& s, int p, int& cur) {
  while (cur + 1 < s.n && s.cum[cur + 1] <= p) ++cur;
  return s.tok[cur] + (p - s.cum[cur]);
}

// Copies n_words 32-bit words (n_words in {2, 4, 8}) from global memory.
template <int NW>
__device__ inline void gload(uint32_t* dst, const uint16_t* src) {
  if constexpr (NW == 2) {
    const u32x2 w = *reinterpret_cast<const u32x2*>(src);
    dst[0] = w[0];
    dst[1] = w[1];
  } else {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
      const u32x4 w = reinterpret_cast<const u32x4*>(src)[i];
      dst[4 * i] = w[0];
      dst[4 * i + 1] = w[1];
      dst[4 * i + 2] = w[2];
      dst[4 * i + 3] = w[3];
    }
  }
}

template <int NW>
__device__ inline void sstore(uint16_t* dst, const uint32_t* src) {
  if constexpr (NW == 2) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{src[0], src[1]};
  } else {
#pragma unroll
    for (int i = 0; i < NW / 4; ++i)
      reinterpret_cast<u32x4*>(dst)[i] =
          u32x4{src[4 * i], src[4 * i + 1], src[4 * i + 2], src[4 * i + 3]};
  }
}

// 16-bit element i of a packed word array.
__device__ inline uint32_t half_of(const uint32_t* w, int i) {
  return (w[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
}

// Fetches the next work item with one atomic; returns the item index (or a
// value >= total when the queue is drained), broadcast through LDS.
__device__ inline int fetch_work(int32_t* counter, int* s_slot) {
  if (threadIdx.x == 0) *s_slot = atomicAdd(counter, 1);
  __syncthreads();
  return *s_slot;
}

// Called by every workgroup once it has drained the queue `work`: the last
// one to leave resets the queue and the exit count `exits`, so the plan can
// be replayed by later launches without a host-side memset.
__device__ inline void leave_queue(int32_t* work, int32_t* exits) {
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(exits, 1) == (int)(gridDim.x * gridDim.y * gridDim.z) - 1) {
      atomicExch(work, 0);
      atomicExch(exits, 0);
    }
  }
}

// XCD (accelerator complex die) executing this wave: 0..7 on MI355X.  Each
// XCD has its own L2, so work that shares inputs should run on one XCD.
__device__ inline int xcd_id() {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
  return (int)(x & 7u);
}

constexpr int NXCD = 8;

// XCD-affine work queue over items 0 .. total-1: the items come in segments
// of `seg` consecutive indices, segment j belonging to XCD j % 8, and
// counter cnt[x] hands out XCD x's items in increasing order.  A workgroup
// drains the queue of its own XCD first, then those of the others
// (`tries` counts the queues it found empty; thread 0 keeps it).  Returns
// the item (or total once every queue is drained), broadcast through LDS.
__device__ inline int fetch_work_xcd(int32_t* cnt, int seg, int total, int home,
                                     int& tries, int* s_slot) {
  if (threadIdx.x == 0) {
    int w = total;
    while (tries < NXCD) {
      const int x = (home + tries) % NXCD;
      const int k = atomicAdd(&cnt[x], 1);
      const int ww = (k / seg) * (NXCD * seg) + x * seg + (k % seg);
      if (ww < total) {
        w = ww;
        break;
      }
      ++tries;  // this queue's items only increase with k: it is drained
    }
    *s_slot = w;
  }
  __syncthreads();
  return *s_slot;
}

// leave_queue for the NXCD counters of fetch_work_xcd.
__device__ inline void leave_queue_xcd(int32_t* cnt, int32_t* exits) {
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(exits, 1) == (int)(gridDim.x * gridDim.y * gridDim.z) - 1) {
      for (int x = 0; x < NXCD; ++x) atomicExch(&cnt[x], 0);
      atomicExch(exits, 0);
    }
  }
}

// Kv head owning global tile index w (head_off ascending, hkv small).
__device__ inline int head_of(const int32_t* head_off, int hkv, int w) {
  int h = 0;
  while (h + 1 < hkv && head_off[h + 1] <= w) ++h;
  return h;
}

// Persistent-grid size for a kernel: CUs x resident workgroups per CU.
int persistent_grid(const void* kernel, int block, size_t dyn_lds);

// A second stream of the current device (created on first use, default
// priority, non-blocking) with a fork and a join event, for launch sequences
// that put independent kernels on two streams: record `fork` on the caller's
// stream and make `s` wait for it, launch, then record `join` on `s` and make
// the caller's stream wait for it.  The events are shared per device, so such
// a sequence holds `*m` from its first fork to its last join.
struct SideStream {
  hipStream_t s;
  hipEvent_t fork, join;
  std::mutex* m;
};
int side_stream(SideStream& out);
// True when `st` is capturing a graph (or the query fails): launch sequences
// then stay on `st`.
bool stream_capturing(hipStream_t st);

// ------------------------------------------------ LDS tile streaming --
// Shared by the forward and backward kernels: 16-byte global -> LDS copies,
// swizzled row-major tiles of 64-element-wide rows, and the per-lane cursor
// over a key stream.

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short s16x4;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// LDS byte address of a __shared__ object.
__device__ inline uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)((__attribute__((address_space(3))) const char*)p);
}

// LDS pointer of byte address a (the inverse of lds_addr); used for reads
// (the transposed-read builtin takes a non-const pointer).
template <typename T>
__device__ inline __attribute__((address_space(3))) T* lds_ptr(uint32_t a) {
  return reinterpret_cast<__attribute__((address_space(3))) T*>((size_t)a);
}

// One 16-byte-per-lane global -> LDS copy: lane l's bytes base + voff land at
// LDS address lds + 16 * l.  Issued as inline assembly so that the compiler
// does not order every later LDS read behind it (it cannot tell which LDS
// buffer the copy targets); completion is awaited explicitly with
// wait_copies() before the barrier that publishes the buffer.
// `base` and `lds` must be wave-uniform values held in SGPRs.
__device__ inline void copy16_to_lds(const void* base, uint32_t voff,
                                     uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 4\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(base), "s"(lds)
      : "memory");
}

__device__ inline int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// s_waitcnt vmcnt(0) as a compiler-visible instruction: the compiler then
// knows every earlier vector-memory load (Q rows included) has completed and
// does not insert its own vmcnt(0) waits inside the key loop, which would
// also stall on the tile copies issued ahead.
__device__ inline void wait_copies() {
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0), expcnt/lgkmcnt untouched
}

// s_waitcnt vmcnt(N): all but this wave's N most recent vector-memory loads
// have completed (loads complete in issue order).
template <int N>
__device__ inline void wait_prev_copies() {
  static_assert(N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0f70 | N);
}

// Row geometry of one LDS tile (NR rows x D, 16-bit): 16-byte chunks per
// row, rows per 1 KB direct-load instruction, and the chunk swizzle of a row.
template <int D, int NR = KT>
struct KvTile {
  static constexpr int CH = D / 8;          // 16-byte chunks per row
  static constexpr int KPL = 64 / CH;       // rows per 1 KB load
  static constexpr int LPW = (NR / KPL) / 4;  // loads per wave per tile (4 waves)
  static constexpr int BYTES = NR * D * 2;
  // Physical chunk = logical chunk ^ swz(row), a linear map of the row's low
  // four bits.  LDS has 64 four-byte banks; a ds_read_b128 is served 16
  // lanes at a time and a ds_read_b64_tr_b16 32 lanes at a time.  The maps
  // give distinct banks to every lane of a service group both for the
  // row-strided reads (16 consecutive rows, one chunk each) and for the
  // transposed reads (rows r0..r0+3 and r0+4..r0+7, two to four chunks
  // each): rows whose 16-byte chunks would share banks differ in the
  // swizzle bit that moves a chunk to the other half of the bank range.
  __device__ static constexpr int swz(int r) {
    if constexpr (D == 32)
      return (r >> 2) & 3;
    else if constexpr (D == 64)
      return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else
      return ((r & 3) << 2) | ((r >> 2) & 3);
  }
  // Byte offset of (row, logical chunk) inside a tile.
  __device__ static constexpr int off(int r, int c) {
    return r * (D * 2) + ((c ^ swz(r)) << 4);
  }
};

// Per-lane cursor over the key stream: the token of stream position p, the
// end of its segment, and (prefetched) the next segment's token base
// (token of position q in it = q + ntb) and end.  Advanced by one tile (64
// positions) at a time; crossing one boundary uses the prefetched values, so
// the common step has no dependent LDS read.
struct StreamCursor {
  int p, seg, tok, segend, ntb, nend;
};

// Longest key stream of a run tile that gets a position -> token map in LDS
// (8 KB: two workgroups per CU still fit at head dim 64).  With blocks of a
// few dozen keys nearly every copy group crosses a block boundary, and the
// map replaces the walk over the segment list by one LDS read per lane.
constexpr int KMAP_KEYS = 2048;

// All 256 threads: map[p] = token of stream position p for the selection in
// s (at most KMAP_KEYS positions); wave wv (wave-uniform) writes segments
// wv, wv + 4, ...
__device__ inline void build_token_map(const SelLds& s, int* map, int wv, int lane) {
  for (int sg = wv; sg < s.n; sg += 4) {
    const int p0 = s.cum[sg], p1 = s.cum[sg + 1], tb = s.tb[sg];
    for (int p = p0 + lane; p < p1; p += 64) map[p] = p + tb;
  }
  __syncthreads();
}

// Plain LDS reads (seg < n, so both indices are in range thanks to the
// sentinels); their results are first needed at the next crossing.
__device__ inline void cursor_prefetch(const SelLds& s, StreamCursor& c) {
  c.ntb = s.tb[c.seg + 1];
  c.nend = s.cum[c.seg + 2];
}

// Walks forward to the segment containing c.p (several boundaries crossed;
// c.p < total keys, so the walk stops at the last segment at the latest).
__device__ inline void cursor_seek(const SelLds& s, StreamCursor& c) {
  while (s.cum[c.seg + 1] <= c.p) ++c.seg;
  c.tok = c.p + s.tb[c.seg];
  c.segend = s.cum[c.seg + 1];
}

// Wave-uniform cursor of one load group: the KPL consecutive stream
// positions P .. P+KPL-1 that one 1 KB copy instruction of a wave covers (P
// is wave-uniform).  The segment holding the group's last row -- index,
// token base tb[seg] and end cum[seg+1] -- is kept in scalar registers, so a
// group that lies inside that segment costs one vector add; a group that
// crosses a boundary, or runs past the stream, takes the per-lane path.
struct GroupCursor {
  int seg, tbase, send;
  int ntb, nend;  // token base and end of segment seg + 1 (read one crossing ahead)
};

// With a position -> token map every group takes the map (send = -1).
__device__ inline void group_init(const SelLds& s, GroupCursor& c, bool mapped = false) {
  c.seg = 0;
  c.tbase = uniform(s.tb[0]);
  c.send = mapped ? -1 : uniform(s.cum[1]);  // INT_MAX sentinel when the stream is empty
  c.ntb = uniform(s.tb[1]);
  c.nend = uniform(s.cum[2]);
}

// Byte offset of this lane's 16-byte piece for the group at stream position
// P.  lane_row = lane's row in the group, lane_off = lane_row * row_bytes +
// chunk_byte (precomputed).  Positions past the stream load token t_safe.
// Groups must be visited in increasing P.  `map` (LDS, or null): the token
// of every stream position, read instead of walking the segments.
template <int KPL>
__device__ inline uint32_t group_offset(const SelLds& s, GroupCursor& c, int P,
                                        int nkeys, int t_safe, uint32_t row_bytes,
                                        int lane_row, uint32_t lane_off,
                                        uint32_t chunk_byte, const int* map = nullptr) {
  if (P + KPL <= c.send) {  // wave-uniform: the whole group is in segment c.seg
    // Scalar row offset plus the lane's constant part: one vector add.
    const uint32_t base = (uint32_t)uniform((int)((uint32_t)(P + c.tbase) * row_bytes));
    return base + lane_off;
  }
  const int p = P + lane_row;
  if (map) return (uint32_t)(p < nkeys ? map[p] : t_safe) * row_bytes + chunk_byte;
  if (P + KPL <= c.nend && c.nend <= nkeys) {
    // wave-uniform: the group ends inside segment seg + 1 (which exists), so
    // it crosses at most the one boundary c.send: tokens from the two token
    // bases in scalar registers, then the cursor moves on one segment.
    const int tok = p + (p < c.send ? c.tbase : c.ntb);
    c.seg += 1;
    c.tbase = c.ntb;
    c.send = c.nend;
    c.ntb = uniform(s.tb[c.seg + 1]);
    c.nend = uniform(s.cum[c.seg + 2]);
    return (uint32_t)tok * row_bytes + chunk_byte;
  }
  int tok = t_safe;
  if (p < nkeys) {
    int sg = c.seg;
    while (s.cum[sg + 1] <= p) ++sg;  // stops at the last segment at latest
    tok = p + s.tb[sg];
  }
  if (P < nkeys) {
    // Advance the scalar state to the segment of the group's last row (the
    // same scan on every lane, so the result is uniform).
    const int last = (P + KPL - 1 < nkeys ? P + KPL - 1 : nkeys - 1);
    int sg = c.seg;
    while (s.cum[sg + 1] <= last) ++sg;
    c.seg = uniform(sg);
    c.tbase = uniform(s.tb[c.seg]);
    c.send = uniform(s.cum[c.seg + 1]);
    c.ntb = uniform(s.tb[c.seg + 1]);
    c.nend = uniform(s.cum[c.seg + 2]);
  }
  return (uint32_t)tok * row_bytes + chunk_byte;
}

}  // namespace lsrm
