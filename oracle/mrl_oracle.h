/*
 * mrl_oracle.h -- CPU restatement of the reference PaxBlock64 scan path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X scan library: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product never links or calls it.
 *
 * Every function restates the reference Rust crate (tcondello/mrl-index-rust-vector)
 * in plain C with the same IEEE-754 single-precision operations in the same
 * order (build with -ffp-contract=off, no fast-math; x86-64 SSE arithmetic).
 * Citations are path:line into the reference tree.
 *
 * How each part is pinned (the reference holds no golden vectors and cannot
 * be built here: no Rust toolchain):
 *  - f16 decode/encode: all 65536 patterns against numpy's IEEE binary16.
 *  - CRC-32: the "123456789" known answer and zlib.crc32.
 *  - FWHT, mid-band and tail-fold rotations: the Sylvester Hadamard matrix and
 *    the operator's Gram structure (float64).
 *  - Plan fields, encoder fields and every per-vector stage score: float64
 *    closed forms recomputed from the inputs; hand-built blocks whose scores
 *    follow from single set bits; the pruned scan against the exhaustive
 *    top-K (admissibility); stage-mask monotonicity and stats consistency.
 *  - EDEN nearest_centroid: brute force incl. the lower-index tie rule.
 *  - ora_lloyd_max_normal (eden.rs:15-44): the f32 bits of every level equal
 *    the reference's literals, parsed from eden.rs by
 *    tests/golden/make_codebooks.py into tests/golden/eden_codebooks.json;
 *    each level is also within 2e-6 of the N(0,1) Lloyd-Max centroid.
 *  - ora_rademacher_diag / ora_tail_rademacher (eden.rs:75-88,
 *    rotate.rs:53-67): tests/golden/make_sign_hash.py parses both reference
 *    function bodies into their 64-bit operation sequence
 *    (tests/golden/sign_hash.json); the signs of every (seed, i) and
 *    (block, dim) pair the path uses equal the ones that sequence gives.
 * Not pinned bit for bit (no independent check fixes them; the parity
 * contract excludes them):
 *  - ora_scan_blocks with sharding on: which of several exactly tied scores
 *    survive at the K boundary (Rayon's merge order, scan.rs:846-865).
 *  - ora_dot for n != 768: the sign of an exactly zero sum (Sum for f32
 *    starts from -0.0 in the Rust releases that write Cargo.lock version 4,
 *    the reference's; older releases start from +0.0).
 */
#ifndef MRL_ORACLE_H
#define MRL_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/block.rs:9-21 */
#define ORA_VECTORS_PER_BLOCK 64
#define ORA_BLOCK_BYTES 4096
#define ORA_PREFIX_DIMS 64
#define ORA_RABITQ_DIMS 128
#define ORA_TAIL_START 192
#define ORA_TAIL_FOLD_DIMS 64
#define ORA_TAIL_FOLD_BLOCKS 9

/* Byte offsets inside one PaxBlock64 (src/block.rs:34-44,133-142;
 * tests/test_challenger_architecture.rs:286-311). */
#define ORA_OFF_MIN_TS 0
#define ORA_OFF_MAX_TS 4
#define ORA_OFF_SOURCE_MASK 8
#define ORA_OFF_CLUSTER_ID 12
#define ORA_OFF_BLOCK_FLAGS 14
#define ORA_OFF_TOMBSTONE 16
#define ORA_OFF_CRC 24
#define ORA_OFF_META 64
#define ORA_OFF_S0 512
#define ORA_OFF_S1 1024
#define ORA_OFF_S2 2048
#define ORA_OFF_S3 2560
#define ORA_OFF_S4 3072
#define ORA_OFF_S5 3584

/* src/config.rs:8-67 */
enum { ORA_PREFIX_MINMAX4 = 0, ORA_PREFIX_EDEN_PROD = 1 };
enum { ORA_MID_RABITQ = 0, ORA_MID_EDEN_B1 = 1 };
enum { ORA_STRATA_L0_ONLY = 0, ORA_STRATA_L1_RABITQ = 1, ORA_STRATA_FULL64B = 2 };

enum {
  ORA_OK = 0,
  ORA_ERR_ARG = 1,
  ORA_ERR_NAN = 3
};

/* src/eden.rs:386-395 (EdenFit). */
typedef struct ora_eden_fit {
  uint32_t dim;
  uint32_t bits;
  uint64_t seed;
  const float *mean;
  uint64_t n_observed;
} ora_eden_fit;

/* src/config.rs:81-114 (ScanConfig) plus the engine fields the scan reads. */
typedef struct ora_scan_config {
  uint32_t shortlist_cand;
  float cs_tolerance;
  float stratum4_weight;
  int32_t strata_depth;
  int32_t temporal_filter_enable;
  int32_t numa_sharding;
  int32_t n_threads;        /* stands in for rayon::current_num_threads() */
  int32_t reserved;
} ora_scan_config;

/* src/scan.rs:20-71 (QueryPlan).  Field order is shared with the product's
 * mrl_query_plan; the trailing "derived" fields are values the reference
 * recomputes inside the stages (scan.rs:457-461, 523-532). */
typedef struct ora_plan {
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
} ora_plan;

/* src/scan.rs:270-278 */
typedef struct ora_scan_stats {
  uint64_t blocks;
  uint64_t active_vecs;
  uint64_t after_prefix;
  uint64_t after_s1;
  uint64_t after_s4_budget;
  uint64_t pushed;
} ora_scan_stats;

size_t ora_plan_size(void);

/* ---- half / meta ---- */
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_f16(float f);
void ora_f16_to_f32_array(const uint16_t *in, float *out, size_t n);
void ora_f32_to_f16_array(const float *in, uint16_t *out, size_t n);
/* out = {scale, offset, tail_norm, rho, mid_norm, high_tail_norm} */
void ora_meta_decode(const uint8_t *block, int slot, float out[6]);
uint8_t ora_pack_rho_flags(float high_tail_norm, float rest_norm);
uint32_t ora_crc32(const uint8_t *data, size_t n);
int ora_verify_crc(const uint8_t *block);

/* ---- rotations (src/rotate.rs) ---- */
void ora_fwht_inplace(float *a, int n);
void ora_rotate_mid_band(const float *mid128, float *out128);
float ora_rabitq_bit_scale(void);
float ora_tail_rademacher(uint64_t block, uint64_t dim);
void ora_fold_tail(const float *vec, int len, float *out64);
void ora_rotate_tail_fold(const float *vec, int len, float *out64);
float ora_tail_fold_bit_scale(void);

/* ---- EDEN (src/eden.rs) ---- */
int ora_lloyd_max_normal(int bits, const float **out);
int ora_nearest_centroid(const float *codebook, int n, float z);
float ora_rademacher_diag(uint64_t seed, uint64_t i);
void ora_structured_hadamard_inplace(float *v, int d, uint64_t seed);
int ora_eden_fit_band(const float *rows, uint64_t n_rows, uint64_t row_stride,
                      uint32_t start, uint32_t dim, float *out_mean);
void ora_eden_observe(float *mean, uint32_t dim, uint64_t *n_observed, const float *x);
int ora_eden_encode_slice(const ora_eden_fit *fit, const float *x, uint8_t *levels,
                          float *centered_norm, float *scale_s);
void ora_eden_rotate_query(const ora_eden_fit *fit, const float *q, float *out);
float ora_eden_score_ip(const ora_eden_fit *fit, const float *q, const float *q_rot,
                        const uint8_t *levels, float alpha);

/* ---- encoder (src/quantize.rs, fixture generation only) ---- */
int ora_encode_block(const float *vecs, int n, int dims, const uint32_t *timestamps,
                     const uint32_t *sources, const ora_eden_fit *eden,
                     const ora_eden_fit *eden_mid, uint8_t *out_block);
void ora_extract_bits4(const uint8_t *block, int slot, uint8_t *out64);

/* ---- query plan (src/scan.rs:105-266) ---- */
int ora_plan_build(const float *query, int dims, int prefix_codec, int mid_codec,
                   const ora_eden_fit *eden, const ora_eden_fit *eden_mid, ora_plan *out);

/* ---- stages at a fixed tau (src/scan.rs:453-691, 709-799) ----
 * masks: [0] active, [1] after prefix, [2] after S1 + CS tail, [3] after S4
 * budget, [4] pushed.  prefix_ip[64]: stage-1 score per active slot.
 * score[64]: state.scores after the stages (meaningful for pushed slots).
 * Returns 0 when the block is skipped (temporal filter / all tombstoned). */
int ora_block_stages(const uint8_t *block, const ora_plan *plan, const ora_scan_config *cfg,
                     float tau, int has_lo, uint32_t lo, int has_hi, uint32_t hi,
                     uint64_t masks[5], float prefix_ip[64], float score[64]);

/* ---- full scan (src/scan.rs:802-886) ----
 * Writes up to K hits sorted as into_sorted() does; returns hit count or <0 on
 * error (-ORA_ERR_NAN when into_sorted would panic on a NaN score). */
int64_t ora_scan_blocks(const uint8_t *blocks, uint64_t n_blocks, const ora_plan *plan,
                        const ora_scan_config *cfg, int has_lo, uint32_t lo, int has_hi,
                        uint32_t hi, uint64_t *out_ids, float *out_scores,
                        ora_scan_stats *stats);

/* Exhaustive scores: every active, time-admitted vector scored through every
 * gated stage at tau = -inf.  out_scores[n_blocks*64]; NaN marks slots that are
 * tombstoned or filtered out. */
void ora_exhaustive_scores(const uint8_t *blocks, uint64_t n_blocks, const ora_plan *plan,
                           const ora_scan_config *cfg, int has_lo, uint32_t lo, int has_hi,
                           uint32_t hi, float *out_scores, uint8_t *out_valid);

/* ---- post-scan rerank (src/pipeline.rs:157-169, src/lowprec.rs:19-121,
 *      src/embed.rs:115-206) ---- */
enum { ORA_RERANK_FP32 = 0, ORA_RERANK_FP16 = 1, ORA_RERANK_INT8 = 2 };
/* dot (embed.rs:115-124): dot_768 for n == 768 (eight accumulators over
 * i mod 8, then acc0 + ... + acc7), otherwise the sequential sum of x*y
 * starting from -0.0 (Sum for f32). */
float ora_dot(const float *a, const float *b, uint32_t n);
/* dot_f16_768 (embed.rs:158-180) of q with Fp16Vec768::from_f32(v) */
float ora_dot_fp16_768(const float *q, const float *v);
/* Int8Vec768::from_f32 (lowprec.rs:72-94): codes[768] and the f16 scale bits */
void ora_int8_quantize_768(const float *v, int8_t *codes, uint16_t *scale_f16);
/* dot_i8_768 (embed.rs:184-206) with the f16 scale read back as f32 */
float ora_dot_int8_768(const float *q, const int8_t *codes, uint16_t scale_f16);
/* rerank_dot (lowprec.rs:103-121): fp16 and int8 need n == 768 */
float ora_rerank_dot(int precision, const float *q, const float *row, uint32_t n);
/* rerank_exact_rows / the precision loop (retrieval_bench.rs:736-745): score
 * every candidate row, stable sort by score descending.  rows: [n_rows][n].
 * Returns 0, or -ORA_ERR_NAN when partial_cmp().unwrap() would panic. */
int ora_rerank(int precision, const float *q, const float *rows, uint32_t n, const uint64_t *cand_rows,
               uint32_t n_cand, uint64_t *out_rows, float *out_scores);

/* RingBuffer::search_exact (src/ring.rs:109-119): dot of every pending row
 * with q, stable sort descending, first top_k.  Returns the count or
 * -ORA_ERR_NAN. */
int ora_ring_search_exact(const float *pending, uint32_t n_pending, uint32_t dims, const float *q,
                          uint32_t top_k, uint64_t *out_local, float *out_scores);
/* Shortlist (src/scan.rs:311-399) of `capacity` holding n hits in the given
 * internal order: push every push_* hit in order, then into_sorted.  Returns
 * the count or -ORA_ERR_NAN.  The engine's ring merge (src/engine.rs:584-594). */
int ora_shortlist_push_sorted(uint32_t capacity, const uint64_t *ids, const float *scores, uint32_t n,
                              const uint64_t *push_ids, const float *push_scores, uint32_t n_push,
                              uint64_t *out_ids, float *out_scores);

#ifdef __cplusplus
}
#endif
#endif
