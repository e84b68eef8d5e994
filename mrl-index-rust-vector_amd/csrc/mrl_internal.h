// mrl_internal.h -- definitions shared by the HIP kernels and the host runtime.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "../../include/mrl_scan.h"

namespace mrl {

constexpr int kBlockBytes = 4096;
constexpr int kVecs = 64;
constexpr int kPrefixDims = 64;
constexpr int kRabitqDims = 128;
constexpr int kTailStart = 192;
constexpr int kTailFoldDims = 64;
constexpr int kTailFoldBlocks = 9;

// Reference PaxBlock64 layout (src/block.rs:34-44,133-142).
constexpr int kOrigMinTs = 0;
constexpr int kOrigMaxTs = 4;
constexpr int kOrigTombstone = 16;
constexpr int kOrigCrc = 24;
constexpr int kOrigMeta = 64;  // 64 x 7 bytes: scale f16, offset f16, tail_norm f16, flags u8
constexpr int kOrigS0 = 512;   // bit 3 of each 4-bit prefix level
constexpr int kOrigS1 = 1024;  // RaBitQ / EdenB1 plane, 128 x u64
constexpr int kOrigS2 = 2048;  // bit 2
constexpr int kOrigS3 = 2560;  // bit 1
constexpr int kOrigS4 = 3072;  // folded tail, 64 x u64
constexpr int kOrigS5 = 3584;  // bit 0

// Device-resident layout of one block (same 4096 bytes, same information).
// The header is kept verbatim.  Per-vector fields become structure-of-arrays
// so lane v of a wave reads slot v with one coalesced load, and the four
// prefix bitplanes become per-vector 4-bit levels: u32 word (v, j) at
// kDevNibbles + 4*(8*v + j) holds the levels of dims 8j..8j+7 of slot v,
// dim 8j+i in bits 4i..4i+3 (a slot's 32 bytes are contiguous, so a lane
// takes its levels with two 16-byte loads).  S1 and S4 stay bit-transposed (bit v of word d
// is slot v), which is exactly a wave64 lane mask.
constexpr int kDevHeader = 0;
constexpr int kDevScale = 64;     // u16[64]
constexpr int kDevOffset = 192;   // u16[64]
constexpr int kDevTail = 320;     // u16[64]
constexpr int kDevFlags = 448;    // u8[64]
constexpr int kDevNibbles = 512;  // u32[64][8]
constexpr int kDevS1 = 2560;      // u64[128]
constexpr int kDevS4 = 3584;      // u64[64]
static_assert(kDevS4 + 64 * 8 == kBlockBytes, "device layout fills the block");

static_assert(sizeof(mrl_query_plan) == 1664 * 4, "mrl_query_plan layout");

// Scan constants of one query, written by the plan kernel next to its plan
// (floats): the prefix LUT (codebook[level] * weight[d] at 16 d + level), the
// S1 weights of the query's mid codec, the folded-tail weights, and the
// upper ends of the S1 / S4 sums (base + positive weights).
constexpr int kQdLut = 0;
constexpr int kQdW1 = 1024;
constexpr int kQdW4 = 1152;
constexpr int kQdU1 = 1216;
constexpr int kQdU4 = 1217;
// Histogram scale of the query: scores are binned as s * 2^-e with
// e = round(log2 |q|) clamped to [-60, 60] (0 for a zero or non-finite
// query), so the bins cover [-2, 2) x |q| at 512 / |q| bins per unit score
// whatever the query's norm.  kQdHistInv holds 2^-e, kQdHistScale 2^e.
constexpr int kQdHistInv = 1218;
constexpr int kQdHistScale = 1219;
constexpr int kQData = 1280;

// Scan-time parameters passed by value to the kernels.
struct ScanParams {
  float alpha;        // cs_tolerance
  float w_s4;         // stratum4_weight
  int32_t strata;     // mrl_strata_depth
  int32_t temporal;   // temporal_filter_enable
  int32_t has_lo;
  int32_t has_hi;
  uint32_t lo;
  uint32_t hi;
  int32_t exhaustive;
  int32_t pad;
};

// Host-computed IEEE constants for the plan kernel (each is the exact f32
// value the reference computes with the same operations).
struct PlanConsts {
  float inv_sqrt64;       // 1.0 / sqrt(64)  (fwht_inplace, n = 64)
  float inv_sqrt128;      // 1.0 / sqrt(128) (fwht_inplace, n = 128)
  float rabitq_scale;     // rabitq_bit_scale()
  float tail_fold_scale;  // tail_fold_bit_scale()
  float eden_codebook[16];
  float eden_mid_codebook[2];
};

// Per-query statistic counters (ScanStats) accumulated on the device.
// kStatRerunSafe / kStatRerunDense count the queries a final selection
// flagged for a re-run at the safe floor / a dense re-run.
enum {
  kStatBlocks = 0,
  kStatActive,
  kStatPrefix,
  kStatS1,
  kStatS4Budget,
  kStatPushed,
  kStatRerunSafe,
  kStatRerunDense,
  kStatCount
};
// Workgroup w adds its counts into copy w % kStatCopies of the counters (one
// address per counter would serialise the atomics of every workgroup); the
// reader sums the copies.
constexpr int kStatCopies = 64;

// Kernel argument blocks (passed by value as kernarg segments).
struct PlanArgs {
  const float* queries;
  uint32_t n_q;
  uint32_t dims;
  int32_t prefix_codec;
  int32_t mid_codec;
  const float* eden_mean;  // 64 floats or null
  uint64_t eden_seed;
  const float* mid_mean;   // 128 floats or null
  uint64_t mid_seed;
  PlanConsts c;
  mrl_query_plan* out;
  float* luts;  // [n_q][kQData] scan constants
};

// Candidate lists: per query, kSegs segments with their own counters.  A
// workgroup stages its appends in LDS and flushes them with one atomic on
// its segment.  Sampling passes append nothing: they count the exact scores
// of their survivors in a per-query histogram, bin = trunc(clamp((s * 2^-e +
// 2) * 512, 0, 2047)) with the query's histogram scale e (kQdHistInv); the
// lower edge of the bin holding the K-th best counted score is <= the final
// K-th score.
constexpr int kSegs = 16;
// A one-query final pass may instead give every workgroup a segment of its
// own (ScanArgs::excl): then nseg = the grid (at most kMaxSegs), and a
// workgroup writes its count with a plain store, no atomic.
constexpr int kMaxSegs = 512;
constexpr int kHistBins = 2048;
// Per-slot records beside the blocks (64 B = 4 uint4 per slot, slot-major):
// everything one slot's stages read, in one line.  kRecLev0 / kRecLev1: the
// slot's level words 0..3 / 4..7 (nibble i of word j = dim 8j + i); kRecS1:
// its S1 bits (dword k = dims 32k..32k+31); kRecS4Meta: {S4 dword 0, S4
// dword 1, scale | offset << 16, tail_norm | flags << 16} (f16 bits).
constexpr int kRecWords = 4;
constexpr uint32_t kBlockFlagOneCluster = 0x0001;  // block_flags bit: every row of the block is in coarse_cluster_id
constexpr int kRecLev0 = 0, kRecLev1 = 1, kRecS1 = 2, kRecS4Meta = 3;

// MFMA-bounded batched scan (k_mma_prep, k_scan_mma, k_mma_floors, k_finish).
// Each (vector, query) pair gets an upper and a lower bound of the full score
// from f16 32x32x16 MFMA tiles (queries x vectors, K = 16 per step); only the
// pairs whose upper bound reaches the K-th best lower bound are scored exactly.
constexpr int kMmaSteps = 17;   // K-steps of a tile: prefix 4, S1 8, S4 4, error columns 1
constexpr int kMmaQ = 64;       // queries per workgroup (two 32-query tiles per wave)
constexpr int kMmaWaves = 8;    // waves per MFMA scan workgroup (four waves per SIMD)
constexpr int kMmaMinQ = 8;     // batches of at least this many queries take the MFMA path
constexpr int kTileQ = 8;       // queries per tile of the batched exact kernel (k_scan_tile)
constexpr int kFuseMaxDims = 1024;  // queries up to this many dims may build their plan inside the sampling pass
// Per-query constants written by k_mma_prep (floats).
enum {
  kMcS = 0,   // power-of-two scale of the query operand
  kMcInvS,    // its inverse
  kMcMean,    // eden_mean_ip (EdenProd) or 0 (MinMax4)
  kMcEP,      // error bound coefficients (score units): per |scale|,
  kMcE1,      //   per mid_n,
  kMcE4,      //   per max(high_n, 1e-6),
  kMcEO,      //   per |offset|,
  kMcE0,      //   and constant
  kMcR,       // bound on |score| + error for vectors whose meta magnitudes are <= kMmaSafe
  kMcOk,      // 1: operands finite; 0: the query is re-run by the exact kernels
  kMcLMax,    // (u32 bits, cleared here) the final pass's largest written lower-bound key, for k_finish
  kMcCount = 16
};
constexpr float kMmaSafe = 4096.0f;  // larger |scale|, mid_n, high_n or |offset|: always a candidate
// The final pass may replace the four S4 K-steps by a bound of the S4 score
// (ScanArgs::mma_wide) for stratum weights up to this value.
constexpr float kMmaWideMaxWs4 = 4.0f;

struct MmaPrepArgs {
  const mrl_query_plan* plans;
  const float* luts;   // [n_q][kQData]
  uint32_t n_q;
  ScanParams sp;
  uint4* ops;          // [n_q][kMmaSteps][2]: 8 f16 query-operand values per (step, half of K)
  float* consts;       // [n_q][kMcCount]
  uint32_t* work;      // k_exact's work list; its count is cleared here
};

struct ScanArgs {
  const uint8_t* idx;          // device-layout blocks
  const uint4* recs;           // [n_blocks * 64 * kRecWords] each slot's record (kRecLev0 ..)
  uint64_t n_blocks;
  // Blocks of this pass: b = pos << shift for pos < n_pos, except those an
  // earlier pass covered (prev_shift >= 0 and b a multiple of 1 << prev_shift).
  uint32_t n_pos;
  uint32_t shift;
  int32_t prev_shift;
  int32_t fuse_plan;  // one-query sampling pass that also builds the query's plan (`plan`)
  PlanArgs plan;
  const mrl_query_plan* plans;
  const float* luts;           // [n_q][kQData] scan constants (prefix LUT, stage weights, sum bounds)
  uint32_t n_q;
  const float* flag_tabs;      // [0,256) rho = f/255, [256,512) sqrt(max(1-rho^2,0))
  ScanParams sp;
  const float* tau;            // per query: pruning threshold and candidate floor (null: -inf)
  uint32_t* hist;              // sampling pass: [n_q][kHistBins] score counts, no appends (null: final pass)
  const uint32_t* floor_hist;  // final pass: floor = bin floor of the floor_rank-th best count
  uint32_t floor_rank;         //   of this histogram (replaces tau when set)
  uint32_t safe_rank;          // K: the safe floor, also taken from floor_hist
  float* floor_out;            // [n_q] out: the final floor (written by one workgroup per query)
  float* safe_out;             // [n_q] out: the safe floor
  float* cand_score;           // [n_q][nseg][seg_cap]
  uint32_t* cand_row;
  uint32_t* seg_count;         // [n_q][nseg]
  uint32_t nseg;
  uint32_t seg_cap;
  // nseg = gridDim.x and segment = workgroup: the workgroup stores its append
  // count (which may exceed seg_cap: then the entries past it are dropped and
  // k_select flags the overflow); one-query kernel only
  uint32_t excl;
  unsigned long long* stats;   // [kStatCopies][kStatCount] counters, or null
  uint32_t* err;               // [n_q] bit 0: NaN score among pushed survivors
  uint64_t* d_masks;           // diagnostic outputs, [n_q][n_blocks][5]
  float* d_prefix;             // [n_q][n_blocks][64]
  float* d_score;              // [n_q][n_blocks][64]
  // MFMA path: query operands and constants from k_mma_prep; appends store
  // the upper bound in cand_score and the lower bound in cand_lower
  const uint4* mma_ops;
  const float* mma_consts;
  float* cand_lower;
  // MFMA final pass: the largest score_key of the lower bounds it writes, per
  // query, raised with atomicMax at lmax[q * kMcCount] (mma_consts' kMcLMax
  // slot; null: not kept)
  uint32_t* lmax;
  // Gated re-run (one-query kernel only): a workgroup of query q exits at
  // once unless bit 2 of gate[q] (a final floor left the query short of K) is set.
  const uint32_t* gate;
  // Block lists (final passes on an index with block bounds): the pass
  // scans blist[y * blist_stride + pos] for pos < bcount[y], y = the
  // launch's query tile (blockIdx.y), instead of pos << shift.
  const uint32_t* blist;
  const uint32_t* bcount;
  uint32_t blist_stride;
  // MFMA sampling pass without a previous floor: instead of counting the
  // lower bounds in a.hist, store every pair's (-inf for pairs that do not
  // count) at lbuf[q * lbuf_stride + 64 pos + slot]; k_mma_floors_lb then
  // builds each query's histogram from them.
  float* lbuf;
  uint32_t lbuf_stride;
  // MFMA sampling pass with a previous floor, when lcount is set: workgroup
  // w lists the lower bounds that count for query q at
  // lbuf[q * lbuf_stride + w * lcap + i], i < lcount[q * lbuf_stride + w]
  // (past lcap entries they go to a.hist); k_mma_floors_seg builds each
  // query's histogram from the lists and a.hist.
  uint32_t* lcount;
  uint32_t lcap;
  // Final MFMA pass (MODE 1) with mma_wide set (the kernel's WIDE
  // instantiation): the tiles run 13 K-steps and
  // the error step's K-half 1 carries a bound of the S4 stage score in place
  // of the four S4 steps; each pair that passes is staged with the flag
  // kMmaWideFlag and its S4 sum is taken from the query operands and the
  // slot's S4 bits before it is written out.  A wave whose appends exceed
  // wide_lim per 1024 pairs it scanned (plus kMmaWideSlack) runs the 17
  // K-steps for the rest of the pass.
  uint32_t mma_wide;
  uint32_t wide_lim;
  // Final pass beside another context's scan: the MFMA pass leaves 1/16 of
  // the resident workgroup slots free, the one-query pass a quarter of its
  // workgroups (the other context's launches then start beside it).
  uint32_t leave_room;
  // MFMA final pass without leave_room: the device's CU count (set by
  // launch_scan_mma; 0: none).
  // The hardware gives workgroup w the first slot of CU w and workgroup
  // w + pair_cols the second slot of the same CU, whose waves then lose the
  // CU's issue arbitration to the first's: the two split the items of column
  // w (w + pair_cols k), the first taking kMmaFirstShare / 256 of them.
  uint32_t pair_cols;
};
constexpr uint8_t kMmaWideFlag = 0x80;   // staged query index: the tile value holds the S4 bound
constexpr uint8_t kMmaDropped = 0xff;    // staged entry dropped (upper bound below the floor)
constexpr uint32_t kMmaWideSlack = 16;
// A final-pass wave writes out its staging region once fewer than this many
// of its entries are free (the next tile's appends, on clustered data
// rarely more; those past the end go straight to their segments).
constexpr uint32_t kMmaFlushRoom = 40;
// The first workgroup's share of a CU's column of items (ScanArgs::pair_cols), in 256ths.
constexpr uint32_t kMmaFirstShare = 141;
constexpr int kMaxListWg = 1024;  // workgroup lists per query a later sampling stage may keep

// Exact finishing of the MFMA path.  k_finish, one workgroup per query: a
// key at or below the K-th best lower bound among the query's candidates, and
// the list of candidates whose upper bound reaches it (written over the
// query's lower-bound area: count, then rows); the query's segment counts are
// cleared.  k_exact, over the whole GPU: the reference's f32 score of every
// listed candidate, appended to the query's segments (at or above the final
// floor) for k_select.
constexpr int kFinCap = 32768;    // exact-scoring list room per query (at most 256 work items)
constexpr int kExactItem = 256;   // list entries per k_exact work item (one per thread)
// The list room of a query whose candidate area holds nseg * seg_cap entries
// (its first entry holds the count).
__host__ __device__ inline uint32_t fin_room(uint32_t nseg, uint32_t seg_cap) {
  const uint64_t room = (uint64_t)nseg * seg_cap - 1u;
  return room < (uint64_t)kFinCap ? (uint32_t)room : (uint32_t)kFinCap;
}
static_assert(kFinCap / kExactItem <= 256, "a work item holds its chunk index in 8 bits");
struct FinishArgs {
  const uint8_t* idx;
  uint64_t n_blocks;
  const uint4* recs;
  const mrl_query_plan* plans;
  const float* luts;
  const float* mma_consts;
  ScanParams sp;
  uint32_t k;
  float* cand_score;        // in: upper bounds; out: exact scores
  float* cand_lower;
  uint32_t* cand_row;
  uint32_t* seg_count;
  uint32_t nseg;
  uint32_t seg_cap;
  const float* tau_final;   // [n_q] floor of the final pass (null: none)
  uint32_t* err;
  unsigned long long* stats;  // or null: listed pairs go to kStatS1 / kStatS4Budget, kept ones to kStatPushed
  uint32_t n_q;
  uint32_t* work;           // [0] item count, [2..] items (q << 8 | chunk): n_q * kFinCap / kExactItem + 2 words
};

struct SelectArgs {
  const float* luts;      // [n_q][kQData] scan constants (the histogram scale of each query)
  const float* cand_score;
  const uint32_t* cand_row;
  uint32_t* seg_count;    // consumed and zeroed
  uint32_t nseg;
  uint32_t seg_cap;
  uint32_t* err;          // consumed and zeroed
  uint32_t k;
  uint32_t* status;       // out per query: bit 0 NaN seen, bit 1 a segment overflowed,
                          // bit 2 fewer than k candidates above a floor tighter than the safe one,
                          // bit 3 fewer than k candidates above a finite floor no tighter than it
                          // (stage bounds that are not admissible rejected vectors above the floor)
  uint32_t* hist;         // sampling histogram [n_q][kHistBins] (null: none); zeroed for the next scan
  const float* tau_final; // [n_q] floor of the final pass (with hist)
  const float* tau_safe;  // [n_q] safe floor (with hist)
  const float* tau_used;  // [n_q] the floor the final pass used (null: -inf, no floor)
  float* floor_record;    // [n_q] or null: a selected query's tau_used is written here
  uint64_t* out_ids;      // [n_q][k]
  float* out_scores;
  uint32_t* out_counts;
  unsigned long long* stats;  // [kStatCopies][kStatCount] or null: flagged re-runs are counted here
  // Gated re-run: query q is selected only if bit 2 of gate[q] is set
  // (gate is the status array this launch rewrites); null: every query.
  const uint32_t* gate;
};

// GPU encoder (mrl_encode.hip): rows -> PaxBlock64 records in the reference layout.
struct EncodeArgs {
  const float* x;          // [n][dims] row-major, device
  uint64_t n;
  uint32_t dims;
  const uint32_t* cluster; // [n] coarse cluster of each row (device) or null: the cluster-grouped convention
  uint32_t source;         // source id of every row
  const float* eden_mean;  // 64 floats (device) or null: MinMax4 prefix
  uint64_t eden_seed;
  const float* mid_mean;   // 128 floats (device) or null: RaBitQ mid-band
  uint64_t mid_seed;
  const uint32_t* crc_tab; // [256] CRC-32 byte table
  const uint32_t* crc_zt;  // [64][32]: register bit i of chunk k carried past the following 64*(63-k) bytes
  uint32_t crc_const;      // CRC of 4096 zero bytes (initial register and final xor folded in)
  PlanConsts c;
  float sqrt64, sqrt128;
  uint8_t* out;            // [n_blocks][4096], device
  uint64_t n_blocks;
};
hipError_t launch_encode(const EncodeArgs& a, hipStream_t s);

// Post-scan rerank (mrl_rerank.hip).  At 768 dims the store rows are
// accumulator-major: element i = 8t + j at position 96j + t.
struct RerankArgs {
  const void* data;         // store rows: f32 / f16 bits / int8 codes
  const uint16_t* scales;   // int8: f16 scale bits per row
  uint64_t n_rows;
  uint32_t dims;
  int32_t precision;        // mrl_rerank_precision
  const float* queries;     // [n_q][dims]
  const uint64_t* cand;     // [n_q][stride]: row ids, or VectorId::as_u64 ids when cand_ids;
                            // null: candidate c is row c (every row of the store)
  const uint32_t* counts;   // [n_q], each <= stride; null: stride for every query
  uint32_t stride;          // <= MRL_MAX_SHORTLIST
  uint32_t n_q;
  int32_t cand_ids;
  float* score;             // scratch [n_q][stride]
  uint64_t* row;            // scratch [n_q][stride]
  uint64_t* out_rows;       // [n_q][stride], sorted
  float* out_scores;
  uint32_t* status;         // [n_q]: bit 0 NaN score, bit 1 row out of range
  uint32_t* out_counts;     // [n_q] or null: entries written per query (ring hits excluded)
  const uint32_t* scan_status;  // [n_q] or null: copied into status bits 8..10
};

// Ring merge (mrl_rerank.hip): push the sorted ring hits of each query into
// its sorted scan shortlist with Shortlist::push semantics, then sort.
struct RingMergeArgs {
  const uint64_t* ids;        // [n_q][k] scan shortlist, sorted
  const float* scores;
  const uint32_t* counts;     // [n_q]
  const uint64_t* ring_rows;  // [n_q][n_ring] ring hits (pending-row index), sorted
  const float* ring_scores;
  const uint32_t* ring_status;  // [n_q]: a query whose ring search failed is left as is
  uint32_t n_ring;            // ring hits per query
  uint32_t k;
  uint32_t n_q;
  uint64_t* out_ids;          // [n_q][k]
  float* out_scores;
  uint32_t* out_counts;       // [n_q]
};

// Block bounds of an index with cluster-grouped blocks (MRL_BLOCK_FLAG_ONE_CLUSTER).
// The full score of a slot (scan.rs:453-634, every stage run) is, in real
// arithmetic, mean_ip + <rho_v, c_q>: a code-space row per slot against a
// column per query.  The row's parts, by stage:
//   [kBndEden, +64)  EdenProd prefix: scale * codebook[level_d]   (column: prefix_weight)
//   [kBndMm, +64)    MinMax4 prefix: scale * level_d               (column: q_d)
//   kBndOff          MinMax4: offset                               (column: prefix_sum)
//   [kBndS1, +128)   S1: mid_n * (2 bit_d - 1)                     (column: rabitq_weights2 / 2)
//   [kBndS4, +64)    S4: hn * (2 bit_d - 1)                        (column: w_s4 tail_fold_weights2 / 2)
// At upload each cluster gets its center (the mean row of its slots) and
// each flagged block one radius per stage (the largest distance of its
// slots' stage part from the center's); by Cauchy-Schwarz every slot's score
// is at most mean_ip + <center, c_q> + sum_stages radius * |c_q stage part|,
// plus a relative margin of 2^-10 for f32 rounding (the reference's own
// stage sums round by less than 2^-14 of the summed magnitudes).
constexpr int kBndEden = 0, kBndMm = 64, kBndOff = 128, kBndS1 = 129, kBndS4 = 257, kBndDims = 321;
constexpr int kBndStride = 324;  // floats per center
constexpr float kBndMargin = 1.0f / 1024.0f;
// radius / norm slots: 0 EdenProd prefix, 1 MinMax4 prefix with the offset, 2 S1, 3 S4
struct BoundBuildArgs {
  const uint8_t* idx;
  const uint4* recs;
  uint64_t n_blocks;
  const uint32_t* cl_start;   // [n_cl + 1] offsets into cl_blocks
  const uint32_t* cl_blocks;  // the flagged blocks of each cluster, grouped
  uint32_t n_cl;
  const float* flag_tabs;     // rho and sqrt(1 - rho^2) per flags byte
  float cb[16];               // EdenProd codebook (eden.rs:27-44)
  float* center;              // [n_cl][kBndStride]
  float* cnorm;               // [n_cl][4] norms of the center's parts
  const uint32_t* bcl;        // [n_blocks] dense cluster of a flagged block, ~0u otherwise
  float* brad;                // [n_blocks][4] radii (upper bounds, +inf when a slot is not finite)
};
struct BoundScanArgs {
  const float* center;
  const float* cnorm;
  uint32_t n_cl;
  const uint32_t* bcl;
  const float* brad;
  uint64_t n_blocks;
  const mrl_query_plan* plans;
  const float* luts;
  uint32_t n_q;
  ScanParams sp;
  int32_t eden;               // prefix codec of the plans is EdenProd
  float* table;               // [n_cl][n_q] mean_ip + <center, c_q> + margin
  float* qn;                  // [n_q][4] norms of the column parts (prefix, S1, S4) raised by the margin
  const float* floor;         // [n_q] floors of the pass (null: the diagnostic)
  uint32_t n_pos;             // the pass's blocks: pos << shift for pos < n_pos
  uint32_t shift;
  uint32_t chunk;             // queries per block list (one list per chunk of queries)
  uint32_t* blist;            // [n_chunks][stride] blocks some query of the chunk can reach
  uint32_t* bcount;           // [n_chunks]
  uint32_t stride;
  float* out_bound;           // diagnostic [n_q][n_blocks] bounds (NaN: unbounded block), or null
};

// Launchers (mrl_kernels.hip).
// Optional start/stop events written by the dispatch itself (kernel-only
// duration, the same interval a kernel-trace profiler reports).
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

// Block bounds: centers and radii at upload; per scan the cluster x query
// table, then the block lists of a final pass (BoundScanArgs).
hipError_t launch_bound_build(const BoundBuildArgs& a, hipStream_t s);
hipError_t launch_bound_table(const BoundScanArgs& a, hipStream_t s, const LaunchEvents& ev = {});
hipError_t launch_block_select(const BoundScanArgs& a, hipStream_t s, const LaunchEvents& ev = {});

// to_device also writes each slot's record (recs, may be null).
hipError_t launch_relayout(const uint8_t* src, uint8_t* dst, uint64_t n_blocks, bool to_device, hipStream_t s,
                           uint4* recs = nullptr);
hipError_t launch_plan(const PlanArgs& a, hipStream_t s, const LaunchEvents& ev = {});
int scan_query_tile(uint32_t n_q);  // queries per workgroup of the non-tile kernels
uint32_t scan_grid(const ScanArgs& a, bool diag);
hipError_t launch_scan(const ScanArgs& a, bool diag, hipStream_t s, const LaunchEvents& ev = {});
hipError_t launch_select(const SelectArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev = {});
// Sets n words at p to v (a kernel, so that a caller may capture it in a graph).
hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t s);
// Reads n uint4 at p (evicts the caches; the loads are kept alive by a store
// whose condition never holds for the data written by launch_fill_u32).
hipError_t launch_read_sweep(uint4* p, uint64_t n, hipStream_t s);
// MFMA path: mode 0 samples (lower bounds into the histogram), 1 appends the
// pairs whose upper bound reaches the floor in a.tau, 2 appends every active pair.
hipError_t launch_mma_prep(const MmaPrepArgs& a, hipStream_t s, const LaunchEvents& ev = {});
// k_plan then k_mma_prep for every query of the batch, in one launch (pa.n_q == ma.n_q)
hipError_t launch_plan_mma_prep(const PlanArgs& pa, const MmaPrepArgs& ma, hipStream_t s, const LaunchEvents& ev = {});
uint32_t mma_scan_grid(const ScanArgs& a);
hipError_t launch_scan_mma(const ScanArgs& a, int mode, hipStream_t s, const LaunchEvents& ev = {});
// Floors of a sampling stage from its histogram (which is then cleared): rank
// `rank` into floor_out and rank safe_rank into safe_out, each raised to the
// previous stage's value when `prev` is set (those arrays hold it on entry).
hipError_t launch_mma_floors(uint32_t* hist, const float* luts, uint32_t n_q, uint32_t rank, uint32_t safe_rank,
                             float* floor_out, float* safe_out, bool prev, hipStream_t s, const LaunchEvents& ev = {});
// The floors of a first sampling stage that stored its lower bounds (n_s per
// query, rows of lbuf_stride floats) instead of counting them.
hipError_t launch_mma_floors_lb(const float* lbuf, uint32_t lbuf_stride, uint32_t n_s, const float* luts,
                                uint32_t n_q, uint32_t rank, uint32_t safe_rank, float* floor_out, float* safe_out,
                                hipStream_t s, const LaunchEvents& ev = {});
// Floors of a later sampling stage that listed its counted lower bounds per
// workgroup (ScanArgs::lcount): the query's histogram from its n_wg lists
// and the global histogram (left zeroed), floors at rank and safe_rank, each
// at least the previous stage's.
hipError_t launch_mma_floors_seg(const float* lbuf, const uint32_t* lcount, uint32_t lbuf_stride, uint32_t n_wg,
                                 uint32_t lcap, uint32_t* hist, const float* luts, uint32_t n_q, uint32_t rank,
                                 uint32_t safe_rank, float* floor_out, float* safe_out, hipStream_t s,
                                 const LaunchEvents& ev = {});
hipError_t launch_finish(const FinishArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev = {});
hipError_t launch_exact(const FinishArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev = {});

// mrl_rerank.hip: build a 768-dim store from f32 rows; score + sort.
hipError_t launch_rerank_store(const float* rows, uint64_t n_rows, int precision, void* data, uint16_t* scales,
                               hipStream_t s);
hipError_t launch_rerank(const RerankArgs& a, hipStream_t s, const LaunchEvents& ev_score = {},
                         const LaunchEvents& ev_sort = {});
hipError_t launch_ring_merge(const RingMergeArgs& a, hipStream_t s, const LaunchEvents& ev = {});

}  // namespace mrl
