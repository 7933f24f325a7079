/*
 * lsrm_hip.h -- C ABI of the MI355X (gfx950) variable-block native sparse
 * attention library (liblsrm_hip.so).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), launches its kernels on that stream and returns a
 * status code without synchronising the host.  No entry point allocates
 * device memory: callers pass a workspace whose size the matching
 * *_workspace_size() function reports.  All index tensors are int32 and all
 * tensors are dense row-major (contiguous) in the layouts stated below.
 *
 * Reference interfaces replaced (paths relative to the LSRM repository):
 *   lsrm_block_mean_pool      sparse/module/spatial_sparse_attention.py:27-37
 *                             (SpatialSparseAttentionIn.sparse3d_compression,
 *                              torch.segment_reduce(reduce="mean"))
 *   lsrm_select_blocks(_pooled) no reference function (the block-selection
 *                             rule of the benchmark); nearest analogue
 *                             sparse/ops/block_score.py:16-98
 *   lsrm_sel_attn_validate    the asserts of
 *                             sparse/ops/triton_native_sparse_attention_impl_kvcentric.py:1295-1301
 *                             plus the metadata contract the kernels assume
 *   lsrm_sel_attn_fwd         ..._impl_kvcentric.py:931-1010 (native_sparse_attn_forward)
 *   lsrm_sel_attn_bwd         ..._impl_kvcentric.py:1018-1263 (native_sparse_attn_backward)
 *   lsrm_sel_attn_*2          the same with plan flags (LSRM_PLAN_KEY_CENTRIC: the
 *                             key-centric forward and dQ for per-token rows)
 *   lsrm_reverse_query_map    ..._impl_kvcentric.py:575-684 (_build_reverse_query_mapping)
 *   lsrm_block_ids            builds the self-block selection that turns the
 *                             selected-attention kernels into
 *                             sparse/ops/block_window_attention.py:14-31
 *                             (sparse_window_attention)
 *   lsrm_block_score          sparse/ops/block_score.py:16-98 (get_block_score,
 *                             the learned per-token block selection)
 *   lsrm_volume_points        misc/sparse_utils.py:644-650 (from_volcoords_to_points)
 *   lsrm_nearest_blocks       misc/sparse_utils.py:1219-1273 (the 3D-aware
 *                             per-token selection of build_volume_to_volume_attn;
 *                             with image points as queries, 960-980 of
 *                             build_image_to_volume_attn)
 *   lsrm_image_points         misc/sparse_utils.py:653-688 (from_imcoords_to_points)
 *   lsrm_image_block_rank     misc/sparse_utils.py:690-898, 991-1200 (the 3D-aware
 *                             per-token selection of build_image_to_image_attn and
 *                             build_volume_to_image_attn) and 16-57
 *                             (compute_block_topk_dist_chunked)
 *   lsrm_block_separation     misc/sparse_utils.py:592-641 (compute_block_separation)
 *   lsrm_gate_merge(_bwd)     sparse/module/spatial_sparse_attention.py:256-269
 *                             (the gated sum of the attention branches)
 *   lsrm_block_sort           misc/sparse_utils.py:95-152 (sort_image_blocks,
 *                             sort_volume_blocks: the sort permutation)
 */
#ifndef LSRM_HIP_H
#define LSRM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes. */
enum lsrm_dtype {
  LSRM_F32 = 0,
  LSRM_F16 = 1,
  LSRM_BF16 = 2
};

/* Status codes returned by every entry point. */
enum lsrm_status {
  LSRM_OK = 0,
  LSRM_ERR_INVALID_ARG = 1, /* null pointer, negative size, bad combination */
  LSRM_ERR_UNSUPPORTED = 2, /* dtype / head_dim / group size not built      */
  LSRM_ERR_WORKSPACE = 3,   /* workspace smaller than *_workspace_size()    */
  LSRM_ERR_LAUNCH = 4,      /* a HIP launch or device query failed          */
  LSRM_ERR_SCRATCH = 5      /* input larger than the fixed scratch of an
                               allocation-free entry point                  */
};

/* Bits of the flag word written by lsrm_sel_attn_validate. */
enum lsrm_meta_error {
  LSRM_META_OFFSETS_NOT_MONOTONE = 1,  /* cu_block_include_tokens decreases  */
  LSRM_META_BLOCK_OUT_OF_RANGE = 2,    /* a block's tokens outside [0, n_k)  */
  LSRM_META_SEQBLOCKS_BAD = 4,         /* cu_seqblocks not monotone / > n_blocks */
  LSRM_META_SEQLENS_BAD = 8,           /* cu_seqlens_q/k not monotone / too big */
  LSRM_META_TOPK_NOT_PREFIX = 16,      /* a valid index after an invalid one  */
  LSRM_META_TOPK_EMPTY_ROW = 32,       /* a query row selects no block        */
  LSRM_META_BLOCK_OUTSIDE_SEQ = 64     /* a batch's blocks leave its k range  */
};

const char* lsrm_status_string(int status);
int lsrm_version(void);

/* ------------------------------------------------------------------------
 * Block mean pooling (key/value block compression).
 *   x               [n_tokens, channels] of x_dtype
 *   cu_block_tokens [n_blocks + 1] int32, block b = rows [cu[b], cu[b+1])
 *   out             [n_blocks, channels] of out_dtype
 * Arithmetic contract (bit-exact, shared with the CPU oracle): rows are cut
 * into pieces at every multiple of 64 of the global row index and at block
 * boundaries; each piece is summed in fp32 in row order starting from +0.0;
 * a block's piece sums are added in order starting from +0.0; the mean is the
 * IEEE fp32 quotient sum / length, rounded to out_dtype to nearest-even.  An
 * empty block yields NaN (0/0), as torch.segment_reduce(mean) does.
 * Replaces: sparse/module/spatial_sparse_attention.py:27-37.
 * ---------------------------------------------------------------------- */
size_t lsrm_block_mean_pool_workspace_size(int64_t n_tokens, int64_t channels,
                                           int64_t n_blocks);
int lsrm_block_mean_pool(const void* x, int x_dtype, int64_t n_tokens,
                         int64_t channels, const int32_t* cu_block_tokens,
                         int64_t n_blocks, void* out, int out_dtype,
                         void* workspace, size_t workspace_bytes, void* stream);

/* The two sparse3d_compression calls of the compression module (keys and
 * values: same token count, channels and block partition) in one piece
 * launch and one combine launch; out_a and out_b may have different dtypes.
 * Each output equals lsrm_block_mean_pool of its input bit for bit.
 * Replaces: sparse/module/spatial_sparse_attention.py:49-66 (the pair of
 * sparse3d_compression calls, each 27-37). */
size_t lsrm_block_mean_pool2_workspace_size(int64_t n_tokens, int64_t channels,
                                            int64_t n_blocks);
int lsrm_block_mean_pool2(const void* x_a, const void* x_b, int x_dtype,
                          int64_t n_tokens, int64_t channels,
                          const int32_t* cu_block_tokens, int64_t n_blocks,
                          void* out_a, int out_a_dtype, void* out_b,
                          int out_b_dtype, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Allocation-free variant of lsrm_block_mean_pool (no counterpart in the
 * reference): for callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight serving loops).  Same
 * arguments and results without the workspace; the kernels use a scratch
 * array of LSRM_POOL_SCRATCH_BYTES that the library holds in device memory
 * on every GPU it runs on until the process ends.  Inputs whose workspace
 * (lsrm_block_mean_pool_workspace_size) exceeds it return LSRM_ERR_SCRATCH
 * without launching anything.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (different streams, or host
 * threads without ordering) race and must be serialised by the caller. */
#define LSRM_POOL_SCRATCH_BYTES (64ull << 20)
int lsrm_block_mean_pool_noalloc(const void* x, int x_dtype, int64_t n_tokens,
                                 int64_t channels, const int32_t* cu_block_tokens,
                                 int64_t n_blocks, void* out, int out_dtype,
                                 void* stream);

/* ------------------------------------------------------------------------
 * Per-query-block top-k block selection (self attention: queries and keys
 * share tokens and the block partition).
 *   q [n_tokens, hq, head_dim], k [n_tokens, hkv, head_dim] of dtype
 *   cu_seqblocks [batch + 1], cu_block_tokens [n_blocks + 1]
 *   forced_blocks [n_forced] batch-local block ids always selected (may be
 *   NULL when n_forced == 0); force_self != 0 also forces the query's block.
 * Rule: pooled means (fp32, lsrm_block_mean_pool contract) of Q and K per
 * block; score(b, c) = sum over the hq/hkv query heads g of kv head h, then
 * over d, of (double)pq[b,g,d] * (double)pk[c,h,d], accumulated in fp64 in
 * that order; candidates are the blocks of the query block's batch element;
 * forced blocks first (self, then forced_blocks in order, duplicates and
 * out-of-range ids dropped, truncated to topk), remaining slots by (score
 * descending, block id ascending).  Output rows list the selected
 * batch-local ids ascending, padded with -1.
 *   topk_idx     [hkv, n_tokens, topk] int32 (every token of a block gets the
 *                block's row, tokens outside every block get -1 rows; the
 *                layout spatial_selection_attention reads)
 *   topk_compact [hkv, n_blocks, topk] int32 (one row per query block)
 * No reference function; nearest analogue sparse/ops/block_score.py:16-98.
 * ---------------------------------------------------------------------- */
size_t lsrm_select_blocks_workspace_size(int64_t n_tokens, int64_t n_blocks,
                                         int64_t hq, int64_t hkv,
                                         int64_t head_dim);
int lsrm_select_blocks(const void* q, const void* k, int dtype,
                       int64_t n_tokens, int64_t hq, int64_t hkv,
                       int64_t head_dim, const int32_t* cu_seqblocks,
                       int64_t batch, const int32_t* cu_block_tokens,
                       int64_t n_blocks, int64_t topk,
                       const int32_t* forced_blocks, int64_t n_forced,
                       int force_self, int32_t* topk_idx,
                       int32_t* topk_compact, void* workspace,
                       size_t workspace_bytes, void* stream);
/* Same selection with k already pooled: pooled_k is the fp32 block mean of
 * k, [n_blocks, hkv * head_dim] (lsrm_block_mean_pool with out_dtype
 * LSRM_F32), so a caller that also needs the compressed keys pools k once
 * (rounding that fp32 mean to the key dtype gives the same compressed keys).
 * No reference function; the same rule as lsrm_select_blocks. */
int lsrm_select_blocks_pooled(const void* q, const float* pooled_k, int dtype,
                              int64_t n_tokens, int64_t hq, int64_t hkv,
                              int64_t head_dim, const int32_t* cu_seqblocks,
                              int64_t batch, const int32_t* cu_block_tokens,
                              int64_t n_blocks, int64_t topk,
                              const int32_t* forced_blocks, int64_t n_forced,
                              int force_self, int32_t* topk_idx,
                              int32_t* topk_compact, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Metadata validation for the selected-attention entry points.  Writes the
 * OR of lsrm_meta_error bits into *flags (device int32, overwritten).
 * Replaces the host asserts of ..._impl_kvcentric.py:1295-1301 and checks
 * the contract the reference leaves unchecked.
 * ---------------------------------------------------------------------- */
int lsrm_sel_attn_validate(const int32_t* topk_idx, int64_t hkv, int64_t n_q,
                           int64_t topk, const int32_t* cu_seqblocks,
                           const int32_t* cu_block_tokens, int64_t n_blocks,
                           const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int64_t batch,
                           int64_t n_k, int32_t* flags, void* stream);

/* ------------------------------------------------------------------------
 * Selected-block attention, forward.
 *   q [n_q, hq, head_dim], k/v [n_k, hkv, head_dim] of dtype (F16 or BF16)
 *   topk_idx [hkv, n_q, topk] int32 batch-local block ids; an entry is valid
 *   when 0 <= id < blocks of the query's batch element; every valid entry is
 *   used, in list order (a repeated block counts twice).
 *   out [n_q, hq, head_dim] dtype; lse [hq, n_q] fp32 in log2 units
 *   (lse = log2 sum exp2(scale*log2(e)*q.k)).  A row with no valid entry
 *   gives out = 0 and lse = -inf.
 * head_dim in {32, 64, 128}; hq % hkv == 0 and hq / hkv <= 64; topk <= 256;
 * k and v each below 4 GiB (rows are addressed with 32-bit byte offsets).
 * Replaces: ..._impl_kvcentric.py:931-1010 (forward_kernel_varblock 55-247).
 * ---------------------------------------------------------------------- */
size_t lsrm_sel_attn_workspace_size(int64_t n_q, int64_t n_k, int64_t hq,
                                    int64_t hkv, int64_t topk,
                                    int64_t n_blocks, int backward);
int lsrm_sel_attn_fwd(const void* q, const void* k, const void* v, int dtype,
                      int64_t n_q, int64_t n_k, int64_t hq, int64_t hkv,
                      int64_t head_dim, const int32_t* topk_idx, int64_t topk,
                      const int32_t* cu_seqblocks,
                      const int32_t* cu_block_tokens, int64_t n_blocks,
                      const int32_t* cu_seqlens_q, int64_t batch,
                      float softmax_scale, void* out, float* lse,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Split form of the two calls above and below, for callers that reuse one
 * selection across launches (timing loops, activation-checkpoint recompute,
 * forward followed by backward on the same top-k).  lsrm_sel_attn_plan
 * builds the device plan (query tiles; with backward != 0 also the reverse
 * map and key chunks) in the workspace; the *_run variants take the same
 * arguments as lsrm_sel_attn_fwd / lsrm_sel_attn_bwd, expect that workspace
 * (same sizes, same topk_idx and metadata) and launch only the attention
 * kernels.  The plan's work queues reset themselves at the end of each
 * launch, so a plan can be replayed any number of times on one stream.
 * lsrm_sel_attn_fwd == lsrm_sel_attn_plan + lsrm_sel_attn_fwd_run.
 * Precondition of lsrm_sel_attn_bwd_run: the plan was built with
 * backward != 0.  A plan built with backward == 0 carries no reverse maps;
 * the backward kernels detect it (a marker word the backward build writes
 * into the plan) and exit without reading or writing anything, leaving
 * dq / dk / dv / delta as they were.
 * ---------------------------------------------------------------------- */
int lsrm_sel_attn_plan(const int32_t* topk_idx, int64_t n_q, int64_t n_k,
                       int64_t hq, int64_t hkv, int64_t topk,
                       const int32_t* cu_seqblocks,
                       const int32_t* cu_block_tokens, int64_t n_blocks,
                       const int32_t* cu_seqlens_q, int64_t batch,
                       int backward, void* workspace, size_t workspace_bytes,
                       void* stream);
int lsrm_sel_attn_fwd_run(const void* q, const void* k, const void* v,
                          int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                          int64_t hkv, int64_t head_dim,
                          const int32_t* topk_idx, int64_t topk,
                          const int32_t* cu_seqblocks,
                          const int32_t* cu_block_tokens, int64_t n_blocks,
                          const int32_t* cu_seqlens_q, int64_t batch,
                          float softmax_scale, void* out, float* lse,
                          void* workspace, size_t workspace_bytes,
                          void* stream);

/* ------------------------------------------------------------------------
 * Plans with flags.  LSRM_PLAN_BACKWARD is the backward != 0 of the calls
 * above.  LSRM_PLAN_KEY_CENTRIC adds the key-centric forward and dQ for
 * per-token rows (learned selections, 3D-aware maps): the query tiles of
 * consecutive queries whose rows differ (the grouped tiles) are taken out of
 * the grouped-tile pass; for every block, the queries of those tiles that
 * listed it are gathered into tiles of up to 128 rows (blocks of up to 256
 * keys, 512 at head_dim <= 64, held whole in LDS) that attend that block
 * alone, each writing a partial result
 * (O over the block normalised by its own sum, in the input type, and the
 * log2 LSE); a merge combines each query's partials in the order of its
 * top-k row (M = max LSE_j, W = sum 2^(LSE_j - M), O = sum 2^(LSE_j - M)
 * O_j / W, LSE = M + log2 W).  Results agree with the other paths to
 * rounding and are bitwise repeatable run to run (no float atomics).  The
 * workspace then also holds the partials: hq * n_q * topk * (head_dim * 2
 * + 4) bytes at most, which is why the part is opt-in.  The key-centric
 * part is carved after the others, so lsrm_sel_attn_fwd_run and
 * lsrm_sel_attn_bwd_run accept such a workspace (they then run the grouped
 * tiles in the grouped-tile passes); lsrm_sel_attn_fwd_run2 with the
 * plan's flags runs the key-centric pass.  head_dim sizes the partials and
 * sets which blocks the forward keeps whole in LDS (up to 512 keys at
 * head_dim <= 64, 256 above), so the runs pass the plan's head_dim like its
 * other inputs (ignored without LSRM_PLAN_KEY_CENTRIC).
 * Replaces: ..._impl_kvcentric.py:931-1010 for per-token rows (the
 * reference has no key-centric forward; the queries of a block are the
 * reverse map of 575-684, which its backward builds).
 * ---------------------------------------------------------------------- */
#define LSRM_PLAN_BACKWARD 1
#define LSRM_PLAN_KEY_CENTRIC 2
size_t lsrm_sel_attn_workspace_size2(int64_t n_q, int64_t n_k, int64_t hq,
                                     int64_t hkv, int64_t head_dim,
                                     int64_t topk, int64_t n_blocks, int flags);
int lsrm_sel_attn_plan2(const int32_t* topk_idx, int64_t n_q, int64_t n_k,
                        int64_t hq, int64_t hkv, int64_t head_dim,
                        int64_t topk, const int32_t* cu_seqblocks,
                        const int32_t* cu_block_tokens, int64_t n_blocks,
                        const int32_t* cu_seqlens_q, int64_t batch, int flags,
                        void* workspace, size_t workspace_bytes, void* stream);
int lsrm_sel_attn_fwd_run2(const void* q, const void* k, const void* v,
                           int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                           int64_t hkv, int64_t head_dim,
                           const int32_t* topk_idx, int64_t topk,
                           const int32_t* cu_seqblocks,
                           const int32_t* cu_block_tokens, int64_t n_blocks,
                           const int32_t* cu_seqlens_q, int64_t batch,
                           float softmax_scale, void* out, float* lse,
                           void* workspace, size_t workspace_bytes, int flags,
                           void* stream);
/* Backward on a plan built with LSRM_PLAN_BACKWARD (and optionally
 * LSRM_PLAN_KEY_CENTRIC): with the key-centric part, dQ of the gathered
 * queries is computed per (query, slot) by the gathered tiles (the block's
 * share, in the input type, in the partial buffer of the forward) and added
 * in slot order; dK/dV are unchanged (they are already key-centric).
 * Replaces: ..._impl_kvcentric.py:1018-1263 for per-token rows. */
int lsrm_sel_attn_bwd_run2(const void* dout, const void* q, const void* k,
                           const void* v, const void* out, const float* lse,
                           int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                           int64_t hkv, int64_t head_dim,
                           const int32_t* topk_idx, int64_t topk,
                           const int32_t* cu_seqblocks,
                           const int32_t* cu_block_tokens, int64_t n_blocks,
                           const int32_t* cu_seqlens_q, int64_t batch,
                           float softmax_scale, void* dq, void* dk, void* dv,
                           float* delta, void* workspace,
                           size_t workspace_bytes, int flags, void* stream);

/* ------------------------------------------------------------------------
 * Selected-block attention, backward.  Inputs as for the forward plus
 * dout [n_q, hq, head_dim] and the forward's out and lse.  Writes
 * dq [n_q, hq, head_dim], dk/dv [n_k, hkv, head_dim] (dtype) and
 * delta [hq, n_q] fp32 (rowsum(out * dout)).  dK/dV are accumulated per
 * 64-key tile by a single writer in a fixed order (deterministic, no float
 * atomics).  Keys no query selects get zero gradient.  Besides the
 * forward's limits, q and dout must each be below 4 GiB.
 * Replaces: ..._impl_kvcentric.py:1018-1263 (backward_kernel_dq 262-478,
 * _build_reverse_query_mapping 575-684, backward_kernel_dkdv_fastest 687-923).
 * ---------------------------------------------------------------------- */
int lsrm_sel_attn_bwd(const void* dout, const void* q, const void* k,
                      const void* v, const void* out, const float* lse,
                      int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                      int64_t hkv, int64_t head_dim, const int32_t* topk_idx,
                      int64_t topk, const int32_t* cu_seqblocks,
                      const int32_t* cu_block_tokens, int64_t n_blocks,
                      const int32_t* cu_seqlens_q, int64_t batch,
                      float softmax_scale, void* dq, void* dk, void* dv,
                      float* delta, void* workspace, size_t workspace_bytes,
                      void* stream);
int lsrm_sel_attn_bwd_run(const void* dout, const void* q, const void* k,
                          const void* v, const void* out, const float* lse,
                          int dtype, int64_t n_q, int64_t n_k, int64_t hq,
                          int64_t hkv, int64_t head_dim,
                          const int32_t* topk_idx, int64_t topk,
                          const int32_t* cu_seqblocks,
                          const int32_t* cu_block_tokens, int64_t n_blocks,
                          const int32_t* cu_seqlens_q, int64_t batch,
                          float softmax_scale, void* dq, void* dk, void* dv,
                          float* delta, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Reverse (CSR) query map of a top-k selection: for each kv head h and
 * global block c, the ascending list of query ids that selected c (a query
 * selecting c twice appears twice).
 *   cu_reverse_count      [hkv, n_blocks + 1] int32 exclusive prefix
 *   reverse_query_indices [hkv, capacity] int32; capacity >= the largest
 *                         per-head entry count (n_q * topk always suffices)
 *   totals                [hkv] int32 entry count per head
 * Replaces: ..._impl_kvcentric.py:575-684 (_build_reverse_query_mapping).
 * ---------------------------------------------------------------------- */
size_t lsrm_reverse_query_map_workspace_size(int64_t n_q, int64_t hkv,
                                             int64_t topk, int64_t n_blocks);
int lsrm_reverse_query_map(const int32_t* topk_idx, int64_t hkv, int64_t n_q,
                           int64_t topk, const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqblocks, int64_t batch,
                           int64_t n_blocks, int32_t* cu_reverse_count,
                           int32_t* reverse_query_indices, int64_t capacity,
                           int32_t* totals, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Batch-local block id of every token: ids[hkv, n_tokens, 1] with
 * ids[h, t, 0] = b - cu_seqblocks[batch of b] for cu[b] <= t < cu[b+1].
 * Feeding it to lsrm_sel_attn_fwd/bwd gives block-diagonal ("window")
 * attention, the semantics of sparse/ops/block_window_attention.py:14-31.
 * ---------------------------------------------------------------------- */
int lsrm_block_ids(const int32_t* cu_seqblocks, int64_t batch,
                   const int32_t* cu_block_tokens, int64_t n_blocks,
                   int64_t n_tokens, int64_t hkv, int32_t* ids, void* stream);

/* ------------------------------------------------------------------------
 * Learned per-token block selection (get_block_score).
 *   q [n_q, hq, head_dim], compressed_k [n_compressed, hkv, head_dim] of
 *   dtype (F16 or BF16); lse [hq, n_q] fp32 in natural-log units (the
 *   softmax LSE of the queries against the compressed keys, as flash-attn
 *   returns it); cu_seqlens_q / compressed_cu_seqlens [batch + 1].
 * For token i of batch element b and kv head h, the score of compressed key
 * c of b is the sum over the hq/hkv query heads g of h of
 *   exp2(q[i, g] . ck[c, h] * sm_scale * 1.44269504 - lse[g, i] * 1.44269504)
 * (fp32); the min(topk, keys of b) best keys (score descending, lower id
 * first among equal scores, NaN never chosen) are written to
 *   block_topk [hkv, n_q, topk] int32 as batch-local ids ascending, the row
 *   padded with -1 (all -1 for a batch element without compressed keys).
 * topk <= 128 (above 64 in two launches: the best min(64, topk - 2), then
 * the best of the keys ranking after them); head_dim in {32, 64, 128}.
 * No workspace.
 * Replaces sparse/ops/block_score.py:16-98.
 * ---------------------------------------------------------------------- */
int lsrm_block_score(const void* q, const void* compressed_k, int dtype,
                     const float* lse, int64_t n_q, int64_t hq, int64_t hkv,
                     int64_t head_dim, const int32_t* cu_seqlens_q,
                     const int32_t* compressed_cu_seqlens, int64_t batch,
                     int64_t topk, float sm_scale, int32_t* block_topk,
                     void* stream);

/* ------------------------------------------------------------------------
 * 3D-aware per-token block selection (volume to volume).
 * lsrm_volume_points: coords [n_tokens, 4] int32 (batch, c1, c2, c3) ->
 *   points [n_tokens, 3] fp32 (x, y, z) = (f(c3), f(c2), f(c1)),
 *   f(c) = 2 * (c / (volume_res - 1) - 0.5) * radius in fp32, radius =
 *   bbox_radius * 1.05 (misc/sparse_utils.py:644-650).
 * lsrm_nearest_blocks: points [n_tokens, 3] fp32, centroids [n_blocks, 3]
 *   fp32 (block means of the points: lsrm_block_mean_pool of the points),
 *   cu_seqlens / cu_seqblocks [batch + 1]; for every token the
 *   min(topk, blocks of its batch element) blocks with the nearest centroid
 *   (squared distance in fp64, ties to the lower id), batch-local ids
 *   ascending, -1 padded, written identically for each of the hkv heads:
 *   block_topk [hkv, n_tokens, topk] int32.  topk <= 128.  No workspace.
 * Replaces misc/sparse_utils.py:1219-1273 (use_3d_aware_attn branch).
 * ---------------------------------------------------------------------- */
int lsrm_volume_points(const int32_t* coords, int64_t n_tokens, int64_t volume_res,
                       float radius, float* points, void* stream);
int lsrm_nearest_blocks(const float* points, const float* centroids,
                        const int32_t* cu_seqlens, const int32_t* cu_seqblocks,
                        int64_t batch, int64_t n_tokens, int64_t topk, int64_t hkv,
                        int32_t* block_topk, void* stream);

/* ------------------------------------------------------------------------
 * 3D-aware per-token selection on the image side.
 * lsrm_image_points: imcoords [n_tokens, 4] int32 (batch, image, patch row,
 *   patch column), surface_points [batch, n_images, dense_res, dense_res, 3]
 *   fp32, masks [batch, n_images, dense_res, dense_res] fp32 -> points
 *   [n_tokens, 3] fp32: the point of the token's patch (dense_res /
 *   patch_res pixels a side) with the largest mask value, the first in
 *   (row, column) order among equal maxima; NaN for coordinates outside the
 *   arrays.  Replaces misc/sparse_utils.py:653-688 (from_imcoords_to_points).
 * lsrm_image_block_rank: for every query point (qpoints [n_q, 3] fp32,
 *   batch elements by cu_seqlens_q [batch + 1]) and every image m of its
 *   batch element b, with the per-image records
 *     cameras [batch, n_images, 18] fp32: rows 0..2 of the world-to-camera
 *       matrix (12), tan(fov / 2), crop flag, origin_size - 1, crop x0,
 *       crop y0, crop_size - 1;
 *     image_meta [batch, n_images, 4] int32: kept blocks of the image, their
 *       offset in kept_blocks, the image's first candidate column, the
 *       image's first block id (kept blocks of the earlier images);
 *     kept_blocks: row-major block numbers (blocks_w blocks a row) of the
 *       kept blocks, image after image;
 *   projects the point into the image, takes the win nearest kept block
 *   centres (fp32 squared distance in block units, ties to the lower kept
 *   number), measures each candidate's smallest 3D distance to its valid
 *   dense points (ibs x ibs points of surface_points under the block,
 *   valid where dense_masks > 0.2, an invalid point counting max_dist),
 *   and writes the min(topk, candidates of b) nearest candidates (ties to
 *   the earlier column; cols_per_batch[b] columns) in column order as block
 *   ids, -1 padded, identically for hkv heads: block_topk [hkv, n_q, topk]
 *   int32.  win <= 16, cols (the widest batch element) <= 1024.
 * Replaces the use_3d_aware_attn branches of misc/sparse_utils.py:690-898
 * (build_image_to_image_attn) and 991-1200 (build_volume_to_image_attn),
 * with compute_block_topk_dist_chunked (16-57).
 * ---------------------------------------------------------------------- */
int lsrm_image_points(const int32_t* imcoords, int64_t n_tokens,
                      const float* surface_points, const float* masks, int64_t batch,
                      int64_t n_images, int64_t dense_res, int64_t patch_res, float* points,
                      void* stream);
size_t lsrm_image_block_rank_workspace_size(int64_t n_q, int64_t cols);
int lsrm_image_block_rank(const float* qpoints, int64_t n_q, const int32_t* cu_seqlens_q,
                          int64_t batch, int64_t n_images, const float* cameras,
                          const int32_t* image_meta, const int32_t* kept_blocks,
                          const int32_t* cols_per_batch, int64_t cols, int64_t blocks_w,
                          int64_t dense_res, int64_t ibs, const float* surface_points,
                          const float* dense_masks, int64_t win, int64_t topk,
                          float max_dist, int64_t hkv, int32_t* block_topk,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Block separation (compute_block_separation).
 *   coords [n_tokens, 1 + dim] int32: batch id (tokens sorted by batch,
 *   ids 0..batch-1), then dim (1..3) non-negative grid coordinates;
 *   block_size / resolution: host arrays of dim ints.  A token lies in block
 *   (c[d] / block_size[d])_d, flattened row-major over
 *   resolution[d] / block_size[d] blocks per dimension; tokens outside the
 *   grid are not counted.  Outputs: cu_seqblocks [batch + 1] (non-empty
 *   blocks per batch element, prefix), cu_block_tokens [batch * bins + 1]
 *   (prefix of the non-empty blocks' token counts in (batch, block) order;
 *   the first *n_blocks + 1 entries are valid), n_blocks (device int32).
 * Replaces misc/sparse_utils.py:592-641.
 * ---------------------------------------------------------------------- */
size_t lsrm_block_separation_workspace_size(int64_t batch, int dim,
                                            const int32_t* block_size,
                                            const int32_t* resolution);
int lsrm_block_separation(const int32_t* coords, int64_t n_tokens, int dim,
                          const int32_t* block_size, const int32_t* resolution,
                          int64_t batch, int32_t* cu_seqblocks, int32_t* cu_block_tokens,
                          int32_t* n_blocks, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ------------------------------------------------------------------------
 * Block sort permutation (sort_volume_blocks / sort_image_blocks).
 *   coords [n_tokens, 4] int32, non-negative: layout 0 (volume) =
 *   (batch, c1, c2, c3) with dims = {volume_res}; layout 1 (image) =
 *   (batch, image, row, col) with dims = {n_images, patch_res} (host
 *   int64 arrays).  Sort key: the reference's offsets (batch, then block
 *   coordinates c / block_size, then in-block coordinates c % block_size);
 *   perm [n_tokens] int32 receives the token indices in ascending key
 *   order (stable: equal keys keep token order).
 * Replaces the torch.argsort of misc/sparse_utils.py:95-152.
 * ---------------------------------------------------------------------- */
size_t lsrm_block_sort_workspace_size(int64_t n_tokens);
int lsrm_block_sort(const int32_t* coords, int64_t n_tokens, int layout, int64_t block_size,
                    const int64_t* dims, int32_t* perm, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Gated merge of the attention branches
 * (sparse/module/spatial_sparse_attention.py:256-269):
 *   out = g[:, 0:H] * o_cmp + g[:, H:2H] * o_slc (+ g[:, 2H:3H] * o_win)
 *   gate [n_tokens, 2H or 3H], o_* / out [n_tokens, H], one dtype
 *   (LSRM_BF16, LSRM_F16 or LSRM_F32), row-major contiguous; o_win NULL for
 *   the two-branch form.  Each product and sum is rounded to the dtype in
 *   the expression's left-to-right order, as PyTorch evaluates it.
 *   n_tokens * 3 * hidden must stay below 2^32 (LSRM_ERR_UNSUPPORTED).
 * lsrm_gate_merge_bwd: autograd of the same expression, d_o_x = dout * g_x
 *   and d_g_x = dout * o_x rounded to the dtype; d_gate has gate's shape;
 *   d_win must be NULL exactly when o_win is.
 * ---------------------------------------------------------------------- */
int lsrm_gate_merge(const void* gate, const void* o_cmp, const void* o_slc,
                    const void* o_win, int dtype, int64_t n_tokens, int64_t hidden,
                    void* out, void* stream);
int lsrm_gate_merge_bwd(const void* dout, const void* gate, const void* o_cmp,
                        const void* o_slc, const void* o_win, int dtype, int64_t n_tokens,
                        int64_t hidden, void* d_gate, void* d_cmp, void* d_slc, void* d_win,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LSRM_HIP_H */
