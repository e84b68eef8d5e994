/*
 * mrl_scan.h -- C ABI of the MI355X (gfx950) PaxBlock64 bitplane scan.
 *
 * Drop-in backend for the reference crate's scan path
 * (tcondello/mrl-index-rust-vector, src/scan.rs + src/pipeline.rs).  Plain C
 * types only: a Rust `extern "C"` block, ctypes or any other FFI binds it.
 *
 * Conventions
 *  - Every function returns an mrl_status; MRL_OK == 0.  On error the calling
 *    thread's mrl_last_error() holds a message.  Nothing panics or throws
 *    across the boundary (the reference panics on bad plan input and on a NaN
 *    score in Shortlist::into_sorted, src/scan.rs:113-124,392; here those are
 *    MRL_ERR_INVALID_ARG and MRL_ERR_NAN).
 *  - A context owns one HIP stream on one device.  Calls on one context are
 *    serialised by a context mutex, so a host wrapper may be Send + Sync.
 *  - Blocks are raw 4096-byte little-endian PaxBlock64 records
 *    (src/block.rs:130-147).  They are uploaded to HBM once and re-laid out
 *    on the device (see mrl_index_upload); mrl_index_download restores the
 *    original bytes exactly.
 *  - Hit ids use VectorId::as_u64: block << 16 | slot (src/block.rs:213-215).
 *  - Results per query are sorted by score descending (ties: smaller id first)
 *    and hold min(K, #scored vectors) entries, the same set the reference's
 *    scan_blocks returns apart from the choice among exactly tied scores at
 *    the K boundary.
 */
#ifndef MRL_SCAN_H
#define MRL_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MRL_ABI_VERSION 2
#define MRL_BLOCK_BYTES 4096
#define MRL_VECTORS_PER_BLOCK 64
#define MRL_MAX_SHORTLIST 4096
#define MRL_MAX_DIMS 8192
#define MRL_NOALLOC_MAX_QUERIES 64
/* block_flags bit of the cluster-grouped layout (see mrl_encode_corpus_clustered) */
#define MRL_BLOCK_FLAG_ONE_CLUSTER 0x0001u

typedef enum mrl_status {
  MRL_OK = 0,
  MRL_ERR_INVALID_ARG = 1,
  MRL_ERR_HIP = 2,
  MRL_ERR_NAN = 3,
  MRL_ERR_OUT_OF_MEMORY = 4,
  MRL_ERR_NO_DEVICE = 5,
  MRL_ERR_CORRUPT = 6,
  MRL_ERR_IO = 7
} mrl_status;

/* src/config.rs:10-16 */
typedef enum mrl_prefix_codec { MRL_PREFIX_MINMAX4 = 0, MRL_PREFIX_EDEN_PROD = 1 } mrl_prefix_codec;
/* src/config.rs:21-28 */
typedef enum mrl_mid_codec { MRL_MID_RABITQ = 0, MRL_MID_EDEN_B1 = 1 } mrl_mid_codec;
/* src/config.rs:36-67 */
typedef enum mrl_strata_depth {
  MRL_STRATA_L0_ONLY = 0,
  MRL_STRATA_L1_RABITQ = 1,
  MRL_STRATA_FULL64B = 2
} mrl_strata_depth;

/* EdenFit (src/eden.rs:105-113).  `mean` has `dim` floats. */
typedef struct mrl_eden_fit {
  uint32_t dim;
  uint32_t bits;
  uint64_t seed;
  const float *mean;
  uint64_t n_observed;
} mrl_eden_fit;

/* ScanConfig (src/config.rs:81-114) plus one build-specific switch.
 * Like the reference's scan_blocks, values are not range-checked except K:
 * shortlist_cand 0 behaves as 1 (Shortlist::new, src/scan.rs:321-329) and
 * values above MRL_MAX_SHORTLIST are rejected. */
typedef struct mrl_scan_config {
  uint32_t shortlist_cand;          /* K_cand */
  float cs_tolerance;               /* alpha, admissible-bound multiplier */
  float stratum4_weight;            /* w_s4 */
  int32_t strata_depth;             /* mrl_strata_depth */
  int32_t temporal_filter_enable;
  int32_t numa_sharding;            /* accepted for API parity; the GPU result does not depend on it */
  int32_t exhaustive;               /* 1: score every active vector through every gated stage (no bound pruning) */
  int32_t reserved;
} mrl_scan_config;

/* Temporal filter bounds: the Option<u32> pair of scan_blocks (src/scan.rs:802-810). */
typedef struct mrl_time_range {
  int32_t has_lo;
  uint32_t lo;
  int32_t has_hi;
  uint32_t hi;
} mrl_time_range;

/* ScanStats (src/scan.rs:270-278), summed over all queries of a call.  The
 * GPU prunes against its own running threshold, so prune counts are
 * reported, not compared; the per-stage masks of mrl_scan_fixed_tau are the
 * tau-independent comparison.  Calls of 8 or more queries on the
 * MFMA-bounded path (RaBitQ mid-band, admissible weights) count
 * after_prefix = pairs whose f16 bound reached the floor, after_s1 =
 * after_s4_budget = pairs scored exactly, pushed = exactly scored pairs
 * kept as candidates.  The last two fields have no reference counterpart:
 * reruns_safe counts queries whose final floor (taken from a sample of the
 * index) left fewer than K candidates, reruns_dense queries whose candidate
 * lists overflowed; mrl_results_fetch re-runs those of the last scan (at
 * the safe floor / densely), so results never depend on the sample. */
typedef struct mrl_scan_stats {
  uint64_t blocks;
  uint64_t active_vecs;
  uint64_t after_prefix;
  uint64_t after_s1;
  uint64_t after_s4_budget;
  uint64_t pushed;
  uint64_t reruns_safe;
  uint64_t reruns_dense;
} mrl_scan_stats;

/* QueryPlan (src/scan.rs:20-71) with every reference field, followed by the
 * values the reference recomputes from the plan inside the stages:
 * prefix_weight (scan.rs:457-461) and the EdenB1 base/deltas (scan.rs:523-532). */
typedef struct mrl_query_plan {
  uint32_t dims;
  int32_t prefix_codec;
  int32_t mid_codec;
  uint32_t has_tail_fold;
  float prefix[64];
  float bit_weights[64][4];
  float rabitq_q[128];
  float rabitq_scale;
  float rabitq_weights2[128];
  float rabitq_base;
  float rabitq_lut[32][16];
  float tail_fold_q[64];
  float tail_fold_weights2[64];
  float tail_fold_base;
  float q_tail_norm;
  float q_mid_norm;
  float q_after_prefix;
  float q_after_s1;
  float s4_abs_budget;
  float prefix_l1;
  float prefix_sum;
  float eden_q_rot[64];
  float eden_mean_ip;
  float eden_inv_sqrt_d;
  float eden_codebook[16];
  float eden_mid_q_rot[128];
  float eden_mid_mean_ip;
  float eden_mid_inv_sqrt_d;
  float eden_mid_codebook[2];
  float prefix_weight[64];
  float eden_mid_base;
  float eden_mid_deltas[128];
  float pad[27];
} mrl_query_plan;

typedef struct mrl_ctx mrl_ctx;
typedef struct mrl_index mrl_index;
typedef struct mrl_plans mrl_plans;
typedef struct mrl_results mrl_results;

/* ---------------------------------------------------------------- */
/* library / context                                                */
/* ---------------------------------------------------------------- */
int mrl_abi_version(void);
/* Message for the last failing call on this thread ("" if none). */
const char *mrl_last_error(void);
size_t mrl_query_plan_size(void);

/* No reference counterpart (the reference scan runs on the global Rayon pool).
 * Destroy order: every index, plans, results and rerank store made on a
 * context keeps the context alive, so mrl_ctx_destroy and the objects'
 * destroy calls may come in any order; the context's stream and buffers are
 * freed with the last of them.  After mrl_ctx_destroy the handle may not be
 * passed to any call (its objects' own destroy calls remain valid).  Memory
 * from mrl_device_alloc is freed with mrl_device_free(ctx, ...) before
 * mrl_ctx_destroy.  Destroy calls wait for the context's stream first. */
int mrl_ctx_create(int device, mrl_ctx **out);
void mrl_ctx_destroy(mrl_ctx *ctx);
int mrl_ctx_synchronize(mrl_ctx *ctx);

/* ---------------------------------------------------------------- */
/* index: a device-resident slab of blocks                          */
/* ---------------------------------------------------------------- */
/* Replaces the `&[PaxBlock64]` slab handed to scan_blocks
 * (src/scan.rs:802-810, src/pipeline.rs:77-98, src/segment.rs:187-193).
 * Copies n_blocks * 4096 bytes to HBM once.  verify_crc=1 checks every block
 * like PaxBlock64::verify_crc (src/block.rs:192-197) and fails with
 * MRL_ERR_CORRUPT on a mismatch.
 * Sharing: an index is read-only once made, so every context on its device
 * may scan it, the way the reference's engine serves `&self` queries from
 * many threads over one slab (src/engine.rs:572-580).  Each context's scans
 * run on its own stream, so scans through two contexts overlap on the GPU.
 * mrl_index_destroy waits for every stream of the device first; a scan
 * enqueued after it is the caller's error. */
int mrl_index_upload(mrl_ctx *ctx, const void *blocks, uint64_t n_blocks, int verify_crc,
                     mrl_index **out);
/* Same, from a segments/NNNNNN.pax file (SegmentReader::open, src/segment.rs:89-162):
 * a size that is not a multiple of 4096 is MRL_ERR_CORRUPT
 * (SegmentError::CorruptSize); a missing file gives an empty index. */
int mrl_index_open_segment(mrl_ctx *ctx, const char *path, int verify_crc, mrl_index **out);
int mrl_index_block_count(const mrl_index *index, uint64_t *out);
/* Inverse of the device re-layout: writes the original n_blocks*4096 bytes. */
int mrl_index_download(mrl_ctx *ctx, const mrl_index *index, void *out_blocks);
void mrl_index_destroy(mrl_index *index);

/* ---------------------------------------------------------------- */
/* query plans (batched HIP kernel)                                 */
/* ---------------------------------------------------------------- */
/* QueryPlan::from_query_codec (src/scan.rs:105-266) for n_queries row-major
 * queries of `dims` floats (host memory).  Errors where the reference
 * asserts: dims < 192, EdenProd without a 64-d 4-bit fit, EdenB1 without a
 * 128-d 1-bit fit.  Pipeline selection (src/pipeline.rs:63-74) is the
 * caller's choice of codecs and fits. */
int mrl_plans_build(mrl_ctx *ctx, const float *queries, uint32_t n_queries, uint32_t dims,
                    int prefix_codec, int mid_codec, const mrl_eden_fit *eden,
                    const mrl_eden_fit *eden_mid, mrl_plans **out);
/* Same, with the queries already in device memory (no copy, no sync). */
int mrl_plans_build_device(mrl_ctx *ctx, const float *d_queries, uint32_t n_queries, uint32_t dims,
                           int prefix_codec, int mid_codec, const mrl_eden_fit *eden,
                           const mrl_eden_fit *eden_mid, mrl_plans **out);
/* Plans keep a device copy of their queries.  Re-run the plan kernel on it,
 * enqueued on the context stream (no copy, no allocation, no sync): the
 * query-side half of one scan step with its input resident in HBM. */
int mrl_plans_rebuild(mrl_ctx *ctx, mrl_plans *plans);
int mrl_plans_count(const mrl_plans *plans, uint32_t *out);
/* Copies plans [first, first+count) to host. */
int mrl_plans_export(mrl_ctx *ctx, const mrl_plans *plans, uint32_t first, uint32_t count,
                     mrl_query_plan *out);
void mrl_plans_destroy(mrl_plans *plans);

/* ---------------------------------------------------------------- */
/* scan                                                             */
/* ---------------------------------------------------------------- */
/* scan_blocks_stats (src/scan.rs:813-886) for every plan at once.
 * out_ids / out_scores: n_queries * K entries (K = max(shortlist_cand,1)),
 * row q at offset q*K; out_counts[q] = hits for query q.  stats may be NULL.
 * time may be NULL (no bounds). */
int mrl_scan(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
             const mrl_scan_config *cfg, const mrl_time_range *time, uint64_t *out_ids,
             float *out_scores, uint32_t *out_counts, mrl_scan_stats *stats);

/* Device-resident results for callers that keep outputs in HBM. */
int mrl_results_create(mrl_ctx *ctx, uint32_t n_queries, uint32_t k, mrl_results **out);
void mrl_results_destroy(mrl_results *res);
/* Enqueue a scan on the context stream; returns without waiting. */
int mrl_scan_async(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
                   const mrl_scan_config *cfg, const mrl_time_range *time, mrl_results *res);
/* Waits for the stream, then copies results (any pointer may be NULL). */
int mrl_results_fetch(mrl_ctx *ctx, mrl_results *res, uint64_t *out_ids, float *out_scores,
                      uint32_t *out_counts, mrl_scan_stats *stats);
/* Diagnostic (no reference counterpart): for each query of the last scan on
 * res, after mrl_results_fetch, the floor its list was selected at: every
 * vector whose stage checks (src/scan.rs:453-634) fail at that threshold, or
 * whose score is below it, was dropped; -inf when no floor was used.  Where
 * the reference's stage bounds are admissible (RaBitQ mid-band, alpha >= 1,
 * 0 <= w_s4 <= alpha / 2.4) the floor is <= the K-th best score and the list
 * is the reference's top K.  Otherwise (EdenB1, other alpha / w_s4) the
 * reference's own result depends on its running threshold's order; the list
 * is then the top K of the vectors the stage functions keep at this fixed
 * floor, scored by them.  out_floors: one float per query. */
int mrl_results_floors(mrl_ctx *ctx, mrl_results *res, float *out_floors);

/* Allocation-free variant of mrl_scan_async.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It allocates nothing: the scan's scratch (candidate lists,
 * histograms, floors, counters) lives in a fixed 13 MiB device array of the
 * library, one per GPU, held until the process ends.  The caller passes the
 * inputs and device-memory outputs: d_out_ids / d_out_scores [n_queries][K]
 * (K = max(shortlist_cand, 1)), d_out_counts and d_out_status [n_queries].
 * Enqueued on the context stream; returns without waiting.  Results are
 * those of mrl_scan_async + mrl_results_fetch: a query whose final floor
 * left it short of K is re-run at the safe floor on the device.  Status bits
 * per query: 1 a NaN score (mrl_results_fetch reports MRL_ERR_NAN); 2 a
 * candidate list overflowed, so that query's list is not exact: scan it with
 * mrl_scan, which re-runs it densely.  Besides massive exact ties, a
 * safe-floor re-run can overflow: the room per query is 16 segments of 4096
 * entries up to 16 queries, 2048 up to 32, 1024 up to 64, while about
 * K x (blocks / sampled blocks) vectors reach the safe floor (some 16K at
 * K = 256 on a 1M-vector index, more on larger ones).  8: fewer than K hits
 * at a floor no tighter than the safe one, possible only where the stage
 * bounds are not admissible (see mrl_results_floors); mrl_scan re-runs such
 * a query with no floor.  At most
 * MRL_NOALLOC_MAX_QUERIES queries per call (more: MRL_ERR_INVALID_ARG).
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls on one context are ordered on its stream, but calls from
 * two contexts on the same GPU that overlap in time race. */
int mrl_scan_noalloc(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
                     const mrl_scan_config *cfg, const mrl_time_range *time, uint64_t *d_out_ids,
                     float *d_out_scores, uint32_t *d_out_counts, uint32_t *d_out_status);

/* Diagnostic scan at a fixed threshold per query: the stage functions of
 * src/scan.rs:453-634 composed as scan_block_stats does (709-799) with
 * tau[q] in place of shortlist.threshold().  Outputs, per (query, block):
 *   masks[5]   active, after prefix, after S1+CS, after S4 budget, pushed
 *   prefix_ip[64]  stage-1 score of every active slot
 *   scores[64]     block state scores after the stages (valid where pushed)
 * Array layout is [query][block][...].  Skipped blocks report zero masks. */
int mrl_scan_fixed_tau(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
                       const mrl_scan_config *cfg, const mrl_time_range *time, const float *tau,
                       uint64_t *out_masks, float *out_prefix_ip, float *out_scores);

/* Diagnostic of the batched path's MFMA bounds (no counterpart in the
 * reference; it exposes the intermediate that batched mrl_scan calls prune
 * on): for every (query, slot) pair, upper and lower bounds of the full
 * score of src/scan.rs:453-634 with every stage run, from the f16 MFMA
 * tiles.  Outputs are [query][block * 64 + slot]; inactive slots (tombstoned,
 * time-filtered, past the corpus end) and queries with non-finite operands
 * read NaN; slots beyond the operand range read +inf / -inf.  Requires the
 * RaBitQ mid-band and a depth other than L0Only; at most 2^24 slots. */
int mrl_scan_mma_bounds(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
                        const mrl_scan_config *cfg, const mrl_time_range *time, float *out_upper,
                        float *out_lower);

/* Diagnostic of block skipping (no reference counterpart): for every
 * (query, block) the upper bound on the full score (src/scan.rs:453-634,
 * every stage run) of the block's active slots that the scan compares with
 * the query's floor to skip the block.  out_bounds is [query][block]; blocks
 * without bounds (no MRL_BLOCK_FLAG_ONE_CLUSTER, or an index with none) read
 * NaN.  Requires the RaBitQ mid-band and an S1 stage. */
int mrl_index_block_bounds(mrl_ctx *ctx, const mrl_index *index, const mrl_plans *plans,
                           const mrl_scan_config *cfg, float *out_bounds);

/* ---------------------------------------------------------------- */
/* post-scan rerank (src/pipeline.rs:157-180, src/lowprec.rs:18-121) */
/* ---------------------------------------------------------------- */
/* RerankPrecision (src/lowprec.rs:18-23) */
typedef enum mrl_rerank_precision {
  MRL_RERANK_FP32 = 0, /* dot (src/embed.rs:115-124): dot_768 at 768 dims, else sequential */
  MRL_RERANK_FP16 = 1, /* Fp16Vec768 + dot_f16_768 (lowprec.rs:43-61, embed.rs:158-180) */
  MRL_RERANK_INT8 = 2  /* Int8Vec768 + dot_i8_768 (lowprec.rs:63-95, embed.rs:184-206) */
} mrl_rerank_precision;

typedef struct mrl_rerank_store mrl_rerank_store;

/* Corpus rows resident in HBM at one rerank precision.  Replaces the
 * corpus_row closure of rerank_exact_rows (src/pipeline.rs:160) and
 * data.corpus_vector(i) in the precision loop (src/retrieval_bench.rs:742);
 * the per-call Fp16Vec768::from_f32 / Int8Vec768::from_f32 of rerank_dot
 * (src/lowprec.rs:112-119) is done once, on the GPU, with the same
 * arithmetic.  rows: n_rows x dims f32, in host memory, or in device memory
 * when rows_on_device (e.g. mrl_device_alloc).  FP16 and INT8 need
 * dims == 768 (the assert_eq! of lowprec.rs:50,73). */
int mrl_rerank_store_create(mrl_ctx *ctx, const float *rows, int rows_on_device, uint64_t n_rows,
                            uint32_t dims, int precision, mrl_rerank_store **out);
void mrl_rerank_store_destroy(mrl_rerank_store *store);
/* The stored rows in the reference's form, row-major: FP32 f32[n][dims],
 * FP16 f16 bits u16[n][768] (Fp16Vec768.data), INT8 i8[n][768] codes plus
 * out_scales[n] f16 bits (Int8Vec768.codes / .scale).  out_scales is used
 * only for INT8. */
int mrl_rerank_store_download(mrl_ctx *ctx, const mrl_rerank_store *store, void *out_rows,
                              uint16_t *out_scales);

/* QueryPipeline::rerank_exact_rows (src/pipeline.rs:157-169), and the
 * precision loop (src/retrieval_bench.rs:739-745) at the store's precision,
 * for n_queries queries in one call.  Query q (queries + q*dims) scores its
 * counts[q] candidate rows cand_rows[q*stride ..], which are then stably
 * sorted by score, descending, into out_rows / out_scores row q (stride
 * entries per row; counts[q] of them written).  Host buffers; returns when
 * done.  stride <= MRL_MAX_SHORTLIST.  MRL_ERR_NAN where the reference's
 * partial_cmp().unwrap() would panic, MRL_ERR_INVALID_ARG for a row >=
 * n_rows (the reference's slice index would panic). */
int mrl_rerank_rows(mrl_ctx *ctx, const mrl_rerank_store *store, const float *queries, uint32_t n_queries,
                    uint32_t dims, const uint64_t *cand_rows, const uint32_t *counts, uint32_t stride,
                    uint64_t *out_rows, float *out_scores);

/* scored_hits_to_row_ids + rerank (src/pipeline.rs:157-180, the bench's
 * scan-then-rerank, src/retrieval_bench.rs:736-745) on the device-resident
 * shortlists of the last mrl_scan_async on res, without a host round trip.
 * Candidates are each query's hits in hit order (row = block * 64 + slot);
 * the queries are those the scan's plans were built from (the plans must
 * still exist).  out_rows / out_scores: n_queries x K, out_counts n_queries
 * (host; any may be null).  Resolves a pending scan like mrl_results_fetch
 * first (MRL_ERR_NAN if the scan itself failed so). */
int mrl_results_rerank(mrl_ctx *ctx, mrl_results *res, const mrl_rerank_store *store, uint64_t *out_rows,
                       float *out_scores, uint32_t *out_counts);

/* RingBuffer::search_exact (src/ring.rs:109-119) for n_queries queries:
 * every pending (unflushed) row, n_pending x dims f32 in host memory, is
 * scored with dot (src/embed.rs:115-124) against each query, stably sorted by
 * score descending and cut at top_k.  Row q of out_local / out_scores holds
 * min(top_k, n_pending) entries (index into the pending rows, score); that
 * count goes to out_counts[q].  n_pending <= MRL_MAX_SHORTLIST.
 * MRL_ERR_NAN where partial_cmp().unwrap() would panic. */
int mrl_ring_search(mrl_ctx *ctx, const float *pending, uint32_t n_pending, uint32_t dims,
                    const float *queries, uint32_t n_queries, uint32_t top_k, uint64_t *out_local,
                    float *out_scores, uint32_t *out_counts);

/* The ring merge of IndexEngine::query_filtered (src/engine.rs:584-594) on
 * the device-resident shortlists of the last scan on res: each query's ring
 * hits (search_exact with top_k = K) are pushed into its shortlist with
 * Shortlist::push semantics (src/scan.rs:351-369) and the list re-sorted, in
 * place; a later mrl_results_fetch returns the merged lists and
 * mrl_results_rerank skips the ring hits as scored_hits_to_row_ids does.
 * Ring hits carry VectorId::new(u32::MAX, local index) ids.  Which of several
 * entries of exactly equal score is kept or comes first can differ from the
 * reference's heap order, as for the scan itself. */
int mrl_results_merge_ring(mrl_ctx *ctx, mrl_results *res, const float *pending, uint32_t n_pending,
                           uint32_t dims);

/* ---------------------------------------------------------------- */
/* kernel timing (no reference counterpart; the reference times     */
/* scans with Instant, src/pipeline.rs:85-95)                       */
/* ---------------------------------------------------------------- */
typedef enum mrl_kernel_kind {
  MRL_KERNEL_PLAN = 0,   /* batched query plan + LUT build */
  MRL_KERNEL_SCAN = 1,   /* one scan pass over a block range */
  MRL_KERNEL_SELECT = 2, /* final top-K selection */
  MRL_KERNEL_THRESH = 3, /* per-query threshold between passes */
  MRL_KERNEL_RERANK = 4, /* rerank scoring of shortlist rows */
  MRL_KERNEL_RERANK_SORT = 5, /* stable sort of the reranked shortlist */
  MRL_KERNEL_FINISH = 6,      /* candidates of the MFMA-bounded scan to score exactly */
  MRL_KERNEL_MMA_PREP = 7,    /* query operands of the MFMA-bounded scan */
  MRL_KERNEL_EXACT = 8,       /* exact scores of those candidates */
  MRL_KERNEL_BOUNDS = 9,      /* block bounds: cluster x query table (pass 0), block lists (passes 1, 2) */
  MRL_KERNEL_PLAN_SCAN = 10,  /* a one-query sampling pass that also built the query's plan */
  MRL_KERNEL_PLAN_PREP = 11   /* the batch's plans and the MFMA query operands, in one launch */
} mrl_kernel_kind;

typedef struct mrl_kernel_time {
  int32_t kind;      /* mrl_kernel_kind */
  int32_t pass;      /* pass index within its scan (0 for plans; -1: the safe-floor re-run an async scan enqueues) */
  uint32_t n_blocks; /* blocks this launch scanned */
  uint32_t n_queries;
  float ms;          /* kernel duration from events recorded by the dispatch itself */
  uint32_t flags;    /* MRL_KT_S4_BOUNDED: an MFMA final pass that bounded the S1 and S4 stages (5 K-steps a tile) */
} mrl_kernel_time;
#define MRL_KT_S4_BOUNDED 1u

/* While enabled, every plan / scan-pass / threshold / select / rerank launch on the
 * context records its kernel start and end (events written by the dispatch). */
int mrl_ctx_set_profiling(mrl_ctx *ctx, int enable);
/* Waits for the stream, returns up to max recorded launches (oldest first),
 * total count in *n_recorded, and clears the record. */
int mrl_ctx_profile_collect(mrl_ctx *ctx, mrl_kernel_time *out, uint32_t max, uint32_t *n_recorded);
/* Measurement helper (no reference counterpart): enqueues a read of `bytes`
 * (at most 4 GiB) of a device buffer the context owns (allocated on first
 * use), which evicts the L2 caches and the Infinity Cache before a
 * cold-cache measurement.  Not timed as a scan kernel. */
int mrl_ctx_evict_caches(mrl_ctx *ctx, uint64_t bytes);
/* Cost policy of the MFMA final pass (no reference counterpart: the
 * reference's scan has no tiles).  The pass may replace its eight S1 and
 * four S4 K-steps by bounds of the two stages' scores; each pair that passes
 * is then given its S1 and S4 sums from the query operands and the slot's
 * bits before it is written out, so the results are the same either way.
 * AUTO takes the bounds when the pass is expected to append few pairs (from
 * the sample's floor rank); ALWAYS takes them wherever they apply
 * (w_s4 <= 4); NEVER runs the full tiles.  mrl_scan_mma_bounds reports the
 * bounds of the bounded pass under ALWAYS and of the full tiles otherwise. */
typedef enum { MRL_S4_BOUND_AUTO = 0, MRL_S4_BOUND_ALWAYS = 1, MRL_S4_BOUND_NEVER = 2 } mrl_s4_bound_policy;
int mrl_ctx_set_s4_bound(mrl_ctx *ctx, int policy);

/* ---------------------------------------------------------------- */
/* ingest-side helpers (host C++, multi-threaded)                   */
/* ---------------------------------------------------------------- */
/* encode_block_with_fits (src/quantize.rs:36-96): n <= 64 vectors of `dims`
 * floats into one 4096-byte block.  eden selects the EDEN-prod prefix,
 * eden_mid the EdenB1 mid-band. */
int mrl_encode_block(const float *vectors, uint32_t n, uint32_t dims, const uint32_t *timestamps,
                     const uint32_t *sources, const mrl_eden_fit *eden,
                     const mrl_eden_fit *eden_mid, void *out_block);
/* encode_f32_corpus_par (src/encoder.rs:195-219): n rows -> ceil(n/64)
 * blocks, timestamp = row index, source = default_source. */
int mrl_encode_corpus(const float *matrix, uint64_t n, uint32_t dims, uint32_t default_source,
                      const mrl_eden_fit *eden, const mrl_eden_fit *eden_mid, int n_threads,
                      void *out_blocks);
/* Cluster-grouped layout (no reference counterpart; an encoder convention
 * for block skipping): mrl_encode_corpus with cluster[i] the coarse cluster
 * of row i, rows grouped by cluster.  A block whose rows all share one
 * cluster below 65536 records it in coarse_cluster_id (src/block.rs:38) and
 * sets MRL_BLOCK_FLAG_ONE_CLUSTER in block_flags (block.rs:39).  The
 * reference's scan reads neither field, so the records stay valid PaxBlock64
 * blocks; every other byte, the CRC aside, equals mrl_encode_corpus's.  An
 * index of such blocks gets per-block score bounds at upload
 * (mrl_index_upload), which let every scan skip blocks no query can reach. */
int mrl_encode_corpus_clustered(const float *matrix, uint64_t n, uint32_t dims, const uint32_t *cluster,
                                uint32_t default_source, const mrl_eden_fit *eden, const mrl_eden_fit *eden_mid,
                                int n_threads, void *out_blocks);
/* encode_f32_corpus_par (src/encoder.rs:195-219) on the GPU: n rows of `dims`
 * floats already in device memory -> ceil(n/64) records in device memory, in
 * the reference byte layout with the CRC set, byte-identical to
 * mrl_encode_corpus.  Returns when the records are written. */
int mrl_encode_corpus_device(mrl_ctx *ctx, const float *d_matrix, uint64_t n, uint32_t dims,
                             uint32_t default_source, const mrl_eden_fit *eden,
                             const mrl_eden_fit *eden_mid, void *d_out_blocks);
/* mrl_encode_corpus_device with the cluster-grouped layout: d_cluster holds
 * the n rows' clusters in device memory; byte-identical to
 * mrl_encode_corpus_clustered. */
int mrl_encode_corpus_device_clustered(mrl_ctx *ctx, const float *d_matrix, uint64_t n, uint32_t dims,
                                       const uint32_t *d_cluster, uint32_t default_source,
                                       const mrl_eden_fit *eden, const mrl_eden_fit *eden_mid, void *d_out_blocks);
/* Device memory on the context's GPU, for callers without a HIP allocator of
 * their own (no reference counterpart).  Copies are synchronous. */
int mrl_device_alloc(mrl_ctx *ctx, size_t bytes, void **out);
void mrl_device_free(mrl_ctx *ctx, void *d_ptr);
int mrl_copy_to_device(mrl_ctx *ctx, void *d_dst, const void *src, size_t bytes);
int mrl_copy_to_host(mrl_ctx *ctx, void *dst, const void *d_src, size_t bytes);
/* Free and total device memory of the context's GPU (hipMemGetInfo), after
 * its stream is done; no reference counterpart (callers and tests that check
 * that a path allocates nothing). */
int mrl_device_mem_info(mrl_ctx *ctx, uint64_t *free_bytes, uint64_t *total_bytes);
/* mrl_index_upload for records already in device memory (e.g. written by
 * mrl_encode_corpus_device); no host copy. */
int mrl_index_from_device(mrl_ctx *ctx, const void *d_blocks, uint64_t n_blocks, mrl_index **out);
/* EdenFit::fit_band (src/eden.rs:130-159): mean of row[start..start+dim]. */
int mrl_eden_fit_band(const float *rows, uint64_t n_rows, uint32_t row_stride, uint32_t start,
                      uint32_t dim, float *out_mean);

#ifdef __cplusplus
}
#endif
#endif /* MRL_SCAN_H */
