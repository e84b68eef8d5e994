// mrl_api.cpp -- C ABI runtime of the MI355X scan (contexts, device index,
// plans, the multi-pass scan driver, diagnostics, ingest helpers).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <map>
#include <memory>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mrl_scan.h"
#include "../../include/mrl_synth.h"
#include "mrl_codec.h"
#include "mrl_internal.h"

using namespace mrl;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_err;

static int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define HIP_TRY(expr)                                                                          \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess) return fail(MRL_ERR_HIP, std::string(#expr ": ") + hipGetErrorString(e_)); \
  } while (0)

extern "C" const char* mrl_last_error(void) { return g_err.c_str(); }
extern "C" int mrl_abi_version(void) { return MRL_ABI_VERSION; }
extern "C" size_t mrl_query_plan_size(void) { return sizeof(mrl_query_plan); }

// ---------------------------------------------------------------------------
// objects
// ---------------------------------------------------------------------------
// Pass p scans blocks b = pos << shift (pos < n_pos) that no earlier pass
// scanned (b not a multiple of 1 << prev_shift); n_new of them.
struct Pass {
  uint32_t shift;
  int32_t prev_shift;
  uint32_t n_pos;
  uint32_t n_new;
};
struct LevelPlan {
  std::vector<Pass> passes;
};

struct ProfRecord {
  hipEvent_t start, stop;
  mrl_kernel_time info;
};

struct mrl_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  float* d_flag_tabs = nullptr;
  PlanConsts consts;
  bool profiling = false;
  int s4_policy = MRL_S4_BOUND_AUTO;  // mrl_ctx_set_s4_bound
  std::vector<ProfRecord> prof;       // recorded, not yet collected
  std::vector<hipEvent_t> event_pool; // reusable events
  uint32_t* d_crc = nullptr;          // encoder CRC tables: [256] byte table, then [64][32] carry map
  uint8_t* d_evict = nullptr;         // cache-eviction buffer (mrl_ctx_evict_caches), zero-filled
  uint64_t evict_bytes = 0;
  uint32_t crc_const = 0;
  void* h_stage = nullptr;            // pinned host staging for result read-back
  size_t h_stage_cap = 0;
  mrl_results* spare = nullptr;       // result buffers kept between synchronous mrl_scan calls
  uint8_t* scratch = nullptr;         // this device's copy of `scratch` (mrl_scan_noalloc); null: lookup failed
  // per-scan scratch of the block selection (grown on demand): the cluster x
  // query table, query norms, block lists and counts of this context's scans
  uint8_t* d_bsel = nullptr;
  size_t bsel_bytes = 0;
  // The caller's handle plus one per live object made on this context (index,
  // plans, results, rerank store).  Each of those reaches the context through
  // its `ctx` member when it is destroyed, so the context's stream and
  // buffers are freed when the last reference goes, in whatever order the
  // caller destroys the handles.
  std::atomic<uint32_t> refs{1};
};

static void ctx_free(mrl_ctx* ctx);

// The context of the last MFMA final pass enqueued on each device, and when.
// A final pass whose predecessor on the device came from another context
// less than 2 ms earlier runs beside that context's work, and may leave room
// for the other's small launches (ScanArgs::leave_room).  One context alone
// keeps the whole GPU.
struct RecentPass {
  std::atomic<uintptr_t> ctx{0};
  std::atomic<int64_t> t_ns{0};
};
static RecentPass g_recent_pass[64];
static bool other_context_active(const mrl_ctx* ctx) {
  if (ctx->device < 0 || ctx->device >= 64) return false;
  RecentPass& r = g_recent_pass[ctx->device];
  const int64_t now =
      std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
          .count();
  const uintptr_t prev = r.ctx.exchange((uintptr_t)ctx);
  const int64_t t_prev = r.t_ns.exchange(now);
  return prev != 0 && prev != (uintptr_t)ctx && now - t_prev < 2000000;
}
static void ctx_retain(mrl_ctx* ctx) { ctx->refs.fetch_add(1, std::memory_order_relaxed); }
static void ctx_release(mrl_ctx* ctx) {
  if (ctx->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) ctx_free(ctx);
}

// ---------------------------------------------------------------------------
// scratch of the allocation-free scan (mrl_scan_noalloc)
// ---------------------------------------------------------------------------
// A fixed array in the library's code object: each GPU the library runs on
// holds its own copy, at its own address, until the process ends.  In host
// code its name is only a stand-in for the symbol, never a device address:
// host code uses the address hipGetSymbolAddress gives for the device
// (looked up once per device, when a context is created on it).
constexpr size_t kNaScratchBytes = (size_t)13 << 20;  // 13 MiB
static __device__ __align__(256) uint8_t scratch[kNaScratchBytes];

static std::mutex g_scratch_mu;
static std::vector<uint8_t*> g_scratch_ptr;  // per device id

// The device address of `scratch` on `device`, which is current.
static int scratch_address(int device, uint8_t** out) {
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if ((size_t)device >= g_scratch_ptr.size()) g_scratch_ptr.resize((size_t)device + 1, nullptr);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MRL_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[device] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[device];
  return MRL_OK;
}

// Pinned host buffer of at least `bytes` (grown on demand; every read-back
// into it is waited for before the call returns).  Caller holds the lock.
static uint8_t* host_stage(mrl_ctx* c, size_t bytes) {
  if (bytes > c->h_stage_cap) {
    if (c->h_stage) (void)hipHostFree(c->h_stage);
    c->h_stage = nullptr;
    c->h_stage_cap = 0;
    const size_t cap = std::max<size_t>(bytes, (size_t)1 << 20);
    if (hipHostMalloc(&c->h_stage, cap, hipHostMallocDefault) != hipSuccess) {
      c->h_stage = nullptr;
      return nullptr;
    }
    c->h_stage_cap = cap;
  }
  return static_cast<uint8_t*>(c->h_stage);
}

static hipEvent_t pool_event(mrl_ctx* c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Supplies dispatch-recorded start/stop events to one launch when profiling
// is on; the record is kept once the launch was enqueued (commit()).
struct ProfScope {
  mrl_ctx* c;
  ProfRecord r{};
  bool on;
  ProfScope(mrl_ctx* ctx, int kind, int pass, uint32_t n_blocks, uint32_t n_q) : c(ctx), on(ctx->profiling) {
    if (!on) return;
    r.start = pool_event(c);
    r.stop = pool_event(c);
    r.info = mrl_kernel_time{kind, pass, n_blocks, n_q, 0.0f, 0u};
    if (!r.start || !r.stop) {
      if (r.start) c->event_pool.push_back(r.start);
      if (r.stop) c->event_pool.push_back(r.stop);
      on = false;
    }
  }
  LaunchEvents ev() const {
    LaunchEvents e;
    if (on) {
      e.start = r.start;
      e.stop = r.stop;
    }
    return e;
  }
  // Called after a successful enqueue; events of a launch that was skipped
  // (empty work) are returned to the pool instead.
  void commit(bool launched) {
    if (!on) return;
    if (launched) {
      c->prof.push_back(r);
    } else {
      c->event_pool.push_back(r.start);
      c->event_pool.push_back(r.stop);
    }
    on = false;
  }
  ~ProfScope() {
    if (on) {  // enqueue failed: recycle the events
      c->event_pool.push_back(r.start);
      c->event_pool.push_back(r.stop);
    }
  }
};

struct mrl_index {
  mrl_ctx* ctx = nullptr;
  uint8_t* d_blocks = nullptr;
  uint4* d_recs = nullptr;  // each slot's 64-byte record (kRecWords uint4, slot-major)
  uint64_t n_blocks = 0;
  const uint4* recs() const { return d_recs; }
  // Pass schedules by K, shared by every context that scans the index.
  std::mutex levels_mu;
  std::map<uint32_t, LevelPlan> levels;
  // Block bounds (blocks with MRL_BLOCK_FLAG_ONE_CLUSTER): one allocation
  // holding the cluster centers [n_cl][kBndStride], their part norms
  // [n_cl][4], each block's dense cluster (~0u: unbounded) and radii [4].
  uint32_t n_cl = 0;
  uint8_t* d_bounds = nullptr;
  float* d_center = nullptr;
  float* d_cnorm = nullptr;
  uint32_t* d_bcl = nullptr;
  float* d_brad = nullptr;
};

// An index is read-only once uploaded, so any context on its device may scan
// it (each context's scans run on that context's own stream).
static bool index_usable(const mrl_index* ix, const mrl_ctx* ctx) { return ix->ctx->device == ctx->device; }

struct mrl_plans {
  mrl_ctx* ctx = nullptr;
  mrl_query_plan* d_plans = nullptr;
  uint32_t n_q = 0;
  uint32_t dims = 0;
  int prefix_codec = 0;
  int mid_codec = 0;
  float* d_eden_mean = nullptr;
  uint64_t eden_seed = 0;
  float* d_mid_mean = nullptr;
  uint64_t mid_seed = 0;
  float* d_queries = nullptr;  // owned copy, n_q * dims
  float* d_luts = nullptr;     // n_q * kQData scan constants written by the plan kernel
  uint8_t* d_block = nullptr;  // one allocation holding all of the above
  // The plans are built lazily: by the next call that reads them (flush_plans),
  // or inside a one-query sampling pass (k_scan's fused plan).
  mutable bool pending = false;
};

// The per-query outputs sit in one device block, read back with one copy:
// status u32[n_q], counts u32[n_q], stats u64[kStatCopies][kStatCount] (summed
// over the copies when read), ids u64[n_q][k], scores f32[n_q][k].
struct mrl_results {
  mrl_ctx* ctx = nullptr;
  uint32_t n_q = 0, k = 0, seg_cap = 0;
  uint8_t* d_out = nullptr;
  size_t out_bytes = 0;
  uint64_t* d_ids = nullptr;
  float* d_scores = nullptr;
  uint32_t* d_counts = nullptr;
  float* d_cand_score = nullptr;   // [n_q][kSegs][seg_cap]
  uint32_t* d_cand_row = nullptr;
  float* d_cand_lower = nullptr;   // [n_q][kSegs][seg_cap] lower bounds of the MFMA path's appends
  uint8_t* d_mma = nullptr;        // MFMA path: query operands [n_q][kMmaSteps][2] uint4, then constants
  uint32_t* d_seg_count = nullptr; // [n_q][kMaxSegs] (a scan uses [n_q][nseg]), zero between scans
  float* d_tau = nullptr;
  float* d_tau_hi = nullptr;       // [n_q] floor of the final pass
  uint32_t* d_hist = nullptr;      // [n_q][kHistBins] sampling-pass score counts, zero between scans
  uint32_t* d_err = nullptr;       // [n_q], zero between scans
  uint32_t* d_status = nullptr;    // [n_q]
  unsigned long long* d_stats = nullptr;
  unsigned long long stats_seen[kStatCount] = {0};
  // the last enqueued scan, re-run densely for queries whose candidate list overflowed
  const mrl_index* last_index = nullptr;
  const mrl_plans* last_plans = nullptr;
  mrl_scan_config last_cfg{};
  mrl_time_range last_time{};
  bool pending = false;
  // per query of the last scan, the floor its list was selected at:
  // 0 none (-inf), 1 the final floor (d_tau_hi), 2 the safe floor (d_tau)
  std::vector<uint8_t> floor_kind;
  // rerank of the shortlists (allocated by the first mrl_results_rerank):
  // scores/rows scratch, sorted rows/scores, status
  void* d_rr = nullptr;
};

struct mrl_rerank_store {
  mrl_ctx* ctx = nullptr;
  int precision = 0;
  uint64_t n_rows = 0;
  uint32_t dims = 0;
  void* d_data = nullptr;       // 768 dims: accumulator-major rows; else row-major f32
  uint16_t* d_scales = nullptr; // int8: f16 scale bits per row
};

static int build_bounds(mrl_ctx* ctx, mrl_index* ix);

static void dev_free(void* p) {
  if (p) (void)hipFree(p);
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
extern "C" int mrl_ctx_create(int device, mrl_ctx** out) {
  if (!out) return fail(MRL_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(MRL_ERR_NO_DEVICE, "no HIP device");
  if (device < 0 || device >= n) return fail(MRL_ERR_INVALID_ARG, "device index out of range");
  HIP_TRY(hipSetDevice(device));
  std::unique_ptr<mrl_ctx> c(new mrl_ctx());
  c->device = device;
  HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
  // IEEE constants the reference computes with the same f32 operations.
  c->consts.inv_sqrt64 = 1.0f / sqrtf(64.0f);
  c->consts.inv_sqrt128 = 1.0f / sqrtf(128.0f);
  c->consts.rabitq_scale = sqrtf(2.0f / (float)M_PI) / sqrtf(128.0f);    // rotate.rs:46-49
  c->consts.tail_fold_scale = sqrtf(2.0f / (float)M_PI) / sqrtf(64.0f);  // rotate.rs:124-126
  int nb;
  const float* cb4 = lloyd_max(4, &nb);
  for (int i = 0; i < 16; ++i) c->consts.eden_codebook[i] = cb4[i];
  const float* cb1 = lloyd_max(1, &nb);
  c->consts.eden_mid_codebook[0] = cb1[0];
  c->consts.eden_mid_codebook[1] = cb1[1];
  // VectorMeta::rho_ratio and the sqrt factor of mid_norm_f32 per flags byte (block.rs:74-84)
  float tabs[512];
  for (int f = 0; f < 256; ++f) {
    float r = (float)f / 255.0f;
    tabs[f] = r;
    float rc = r < 0.0f ? 0.0f : (r > 1.0f ? 1.0f : r);
    tabs[256 + f] = sqrtf(fmaxf(1.0f - rc * rc, 0.0f));
  }
  HIP_TRY(hipMalloc(&c->d_flag_tabs, sizeof(tabs)));
  HIP_TRY(hipMemcpy(c->d_flag_tabs, tabs, sizeof(tabs), hipMemcpyHostToDevice));
  // The scan entry points other than mrl_scan_noalloc do not need the
  // scratch address: a failed lookup only makes that one entry point fail.
  if (scratch_address(device, &c->scratch)) c->scratch = nullptr;
  g_err.clear();
  *out = c.release();
  return MRL_OK;
}

static void results_release(mrl_results* r);

extern "C" void mrl_ctx_destroy(mrl_ctx* ctx) {
  if (ctx) ctx_release(ctx);
}

static void ctx_free(mrl_ctx* ctx) {
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  results_release(ctx->spare);
  dev_free(ctx->d_flag_tabs);
  dev_free(ctx->d_crc);
  dev_free(ctx->d_evict);
  dev_free(ctx->d_bsel);
  for (auto& r : ctx->prof) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
  if (ctx->h_stage) (void)hipHostFree(ctx->h_stage);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" int mrl_ctx_synchronize(mrl_ctx* ctx) {
  if (!ctx) return fail(MRL_ERR_INVALID_ARG, "ctx is null");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MRL_OK;
}

extern "C" int mrl_ctx_set_profiling(mrl_ctx* ctx, int enable) {
  if (!ctx) return fail(MRL_ERR_INVALID_ARG, "ctx is null");
  std::lock_guard<std::mutex> g(ctx->mu);
  ctx->profiling = enable != 0;
  return MRL_OK;
}

extern "C" int mrl_ctx_set_s4_bound(mrl_ctx* ctx, int policy) {
  if (!ctx) return fail(MRL_ERR_INVALID_ARG, "ctx is null");
  if (policy != MRL_S4_BOUND_AUTO && policy != MRL_S4_BOUND_ALWAYS && policy != MRL_S4_BOUND_NEVER)
    return fail(MRL_ERR_INVALID_ARG, "unknown S4 bound policy");
  std::lock_guard<std::mutex> g(ctx->mu);
  ctx->s4_policy = policy;
  return MRL_OK;
}

extern "C" int mrl_ctx_evict_caches(mrl_ctx* ctx, uint64_t bytes) {
  if (!ctx) return fail(MRL_ERR_INVALID_ARG, "ctx is null");
  if (bytes > ((uint64_t)4 << 30)) return fail(MRL_ERR_INVALID_ARG, "at most 4 GiB");
  bytes = (bytes + 15) & ~(uint64_t)15;
  if (!bytes) return MRL_OK;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (bytes > ctx->evict_bytes) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    dev_free(ctx->d_evict);
    ctx->d_evict = nullptr;
    ctx->evict_bytes = 0;
    if (hipMalloc(&ctx->d_evict, bytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "eviction buffer");
    ctx->evict_bytes = bytes;
    HIP_TRY(launch_fill_u32(reinterpret_cast<uint32_t*>(ctx->d_evict), bytes / 4, 0u, ctx->stream));
  }
  HIP_TRY(launch_read_sweep(reinterpret_cast<uint4*>(ctx->d_evict), bytes / 16, ctx->stream));
  return MRL_OK;
}

extern "C" int mrl_ctx_profile_collect(mrl_ctx* ctx, mrl_kernel_time* out, uint32_t max, uint32_t* n_recorded) {
  if (!ctx || (max && !out)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  uint32_t i = 0;
  for (auto& r : ctx->prof) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) {
      ms = -1.0f;
      (void)hipGetLastError();  // do not leave the failure for the next launch check
    }
    if (i < max) {
      out[i] = r.info;
      out[i].ms = ms;
    }
    ++i;
    ctx->event_pool.push_back(r.start);
    ctx->event_pool.push_back(r.stop);
  }
  if (n_recorded) *n_recorded = (uint32_t)ctx->prof.size();
  ctx->prof.clear();
  return MRL_OK;
}

// ---------------------------------------------------------------------------
// index
// ---------------------------------------------------------------------------
// CRC check of n_blocks blocks whose first is block `first` of the index (for the message).
static int verify_crcs(const uint8_t* blocks, uint64_t n_blocks, uint64_t first = 0) {
  std::atomic<int64_t> bad{-1};
  parallel_for(n_blocks, 0, [&](uint64_t b0, uint64_t b1) {
    for (uint64_t b = b0; b < b1; ++b)
      if (!block_crc_ok(blocks + b * kBlockBytes)) {
        int64_t expect = -1;
        bad.compare_exchange_strong(expect, (int64_t)b);
      }
  });
  return bad.load() < 0 ? MRL_OK
                        : fail(MRL_ERR_CORRUPT, "crc32 mismatch in block " + std::to_string(first + bad.load()));
}

extern "C" int mrl_index_upload(mrl_ctx* ctx, const void* blocks, uint64_t n_blocks, int verify_crc,
                                mrl_index** out) {
  if (!ctx || !out || (n_blocks && !blocks)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (n_blocks > (1ull << 26)) return fail(MRL_ERR_INVALID_ARG, "n_blocks exceeds 2^26 (32-bit row ids)");
  *out = nullptr;
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  if (verify_crc) {
    int rc = verify_crcs(src, n_blocks);
    if (rc) return rc;
  }
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  std::unique_ptr<mrl_index> ix(new mrl_index());
  ix->ctx = ctx;
  ix->n_blocks = n_blocks;
  if (n_blocks) {
    const size_t bytes = (size_t)n_blocks * kBlockBytes;
    uint8_t* staging = nullptr;
    if (hipMalloc(&ix->d_blocks, bytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc index");
    if (hipMalloc(&ix->d_recs, (size_t)n_blocks * 64 * kRecWords * 16) != hipSuccess) {
      dev_free(ix->d_blocks);
      return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc index records");
    }
    // stage in chunks of at most 256 MiB so the transient copy stays small
    const uint64_t chunk = std::min<uint64_t>(n_blocks, 65536);
    if (hipMalloc(&staging, chunk * kBlockBytes) != hipSuccess) {
      dev_free(ix->d_blocks);
      dev_free(ix->d_recs);
      return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc staging");
    }
    for (uint64_t b = 0; b < n_blocks; b += chunk) {
      uint64_t nb = std::min(chunk, n_blocks - b);
      hipError_t e = hipMemcpyAsync(staging, src + b * kBlockBytes, nb * kBlockBytes, hipMemcpyHostToDevice,
                                    ctx->stream);
      if (e == hipSuccess)
        e = launch_relayout(staging, ix->d_blocks + b * kBlockBytes, nb, true, ctx->stream,
                            ix->d_recs + b * 64 * kRecWords);
      if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
      if (e != hipSuccess) {
        dev_free(staging);
        dev_free(ix->d_blocks);
        dev_free(ix->d_recs);
        return fail(MRL_ERR_HIP, std::string("upload: ") + hipGetErrorString(e));
      }
    }
    dev_free(staging);
    int rc = build_bounds(ctx, ix.get());
    if (rc) {
      dev_free(ix->d_blocks);
      dev_free(ix->d_recs);
      return rc;
    }
  }
  ctx_retain(ctx);
  *out = ix.release();
  return MRL_OK;
}

// Segment blocks per staging chunk of mrl_index_open_segment (16 MiB).
static const uint64_t kSegChunkBlocks = 4096;

extern "C" int mrl_index_open_segment(mrl_ctx* ctx, const char* path, int verify_crc, mrl_index** out) {
  if (!ctx || !path || !out) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  if (!f) return mrl_index_upload(ctx, nullptr, 0, 0, out);  // segment.rs:94-101: absent file = empty
  if (fseek(f, 0, SEEK_END) != 0) {
    fclose(f);
    return fail(MRL_ERR_IO, "seek failed");
  }
  long len = ftell(f);
  if (len < 0) {
    fclose(f);
    return fail(MRL_ERR_IO, "ftell failed");
  }
  if (len % kBlockBytes != 0) {  // segment.rs:101-103
    fclose(f);
    return fail(MRL_ERR_CORRUPT, "corrupt segment size " + std::to_string(len) + " (not multiple of 4096)");
  }
  const uint64_t n_blocks = (uint64_t)len / kBlockBytes;
  if (n_blocks == 0) {
    fclose(f);
    return mrl_index_upload(ctx, nullptr, 0, 0, out);
  }
  if (n_blocks > (1ull << 26)) {
    fclose(f);
    return fail(MRL_ERR_INVALID_ARG, "n_blocks exceeds 2^26 (32-bit row ids)");
  }
  fseek(f, 0, SEEK_SET);
  // The file streams through two pinned host chunks: while the GPU copies
  // chunk i and re-lays it out into the index, the host reads (and checks)
  // chunk i + 1.  No whole-file host copy is made.
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  std::unique_ptr<mrl_index> ix(new mrl_index());
  ix->ctx = ctx;
  ix->n_blocks = n_blocks;
  const uint64_t chunk = std::min<uint64_t>(n_blocks, kSegChunkBlocks);
  uint8_t* host[2] = {nullptr, nullptr};
  uint8_t* dstage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  auto cleanup = [&](bool keep_index) {
    (void)hipStreamSynchronize(ctx->stream);  // nothing may still read the staging
    for (int k = 0; k < 2; ++k) {
      if (host[k]) (void)hipHostFree(host[k]);
      dev_free(dstage[k]);
      if (done[k]) (void)hipEventDestroy(done[k]);
    }
    if (!keep_index) {
      dev_free(ix->d_blocks);
      dev_free(ix->d_recs);
    }
    fclose(f);
  };
  int rc = MRL_OK;
  std::string msg;
  if (hipMalloc(&ix->d_blocks, (size_t)n_blocks * kBlockBytes) != hipSuccess ||
      hipMalloc(&ix->d_recs, (size_t)n_blocks * 64 * kRecWords * 16) != hipSuccess) {
    rc = MRL_ERR_OUT_OF_MEMORY;
    msg = "hipMalloc index";
  }
  for (int k = 0; k < 2 && !rc; ++k) {
    if (hipHostMalloc((void**)&host[k], chunk * kBlockBytes, hipHostMallocDefault) != hipSuccess ||
        hipMalloc(&dstage[k], chunk * kBlockBytes) != hipSuccess ||
        hipEventCreateWithFlags(&done[k], hipEventDisableTiming) != hipSuccess) {
      rc = MRL_ERR_OUT_OF_MEMORY;
      msg = "segment staging";
    }
  }
  for (uint64_t b = 0, i = 0; b < n_blocks && !rc; b += chunk, ++i) {
    const int k = (int)(i & 1u);
    const uint64_t nb = std::min(chunk, n_blocks - b);
    if (i >= 2 && hipEventSynchronize(done[k]) != hipSuccess) {  // chunk i - 2 left these buffers
      rc = MRL_ERR_HIP;
      msg = "segment staging wait";
      break;
    }
    if (fread(host[k], 1, nb * kBlockBytes, f) != nb * kBlockBytes) {
      rc = MRL_ERR_IO;
      msg = "short read";
      break;
    }
    if (verify_crc) {
      rc = verify_crcs(host[k], nb, b);
      if (rc) break;
    }
    hipError_t e = hipMemcpyAsync(dstage[k], host[k], nb * kBlockBytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
      e = launch_relayout(dstage[k], ix->d_blocks + b * kBlockBytes, nb, true, ctx->stream,
                          ix->d_recs + b * 64 * kRecWords);
    if (e == hipSuccess) e = hipEventRecord(done[k], ctx->stream);
    if (e != hipSuccess) {
      rc = MRL_ERR_HIP;
      msg = std::string("segment upload: ") + hipGetErrorString(e);
    }
  }
  if (!rc && hipStreamSynchronize(ctx->stream) != hipSuccess) {
    rc = MRL_ERR_HIP;
    msg = "segment upload";
  }
  if (rc) {
    cleanup(false);
    return msg.empty() ? rc : fail(rc, msg);  // verify_crcs has set its own message
  }
  cleanup(true);
  rc = build_bounds(ctx, ix.get());
  if (rc) {
    dev_free(ix->d_blocks);
    dev_free(ix->d_recs);
    return rc;
  }
  ctx_retain(ctx);
  *out = ix.release();
  return MRL_OK;
}

extern "C" int mrl_index_block_count(const mrl_index* index, uint64_t* out) {
  if (!index || !out) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = index->n_blocks;
  return MRL_OK;
}

extern "C" int mrl_index_download(mrl_ctx* ctx, const mrl_index* index, void* out_blocks) {
  if (!ctx || !index || (index->n_blocks && !out_blocks)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (!index->n_blocks) return MRL_OK;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  uint8_t* staging = nullptr;
  const uint64_t chunk = std::min<uint64_t>(index->n_blocks, 65536);
  if (hipMalloc(&staging, chunk * kBlockBytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc staging");
  uint8_t* dst = static_cast<uint8_t*>(out_blocks);
  for (uint64_t b = 0; b < index->n_blocks; b += chunk) {
    uint64_t nb = std::min(chunk, index->n_blocks - b);
    hipError_t e = launch_relayout(index->d_blocks + b * kBlockBytes, staging, nb, false, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(dst + b * kBlockBytes, staging, nb * kBlockBytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      dev_free(staging);
      return fail(MRL_ERR_HIP, std::string("download: ") + hipGetErrorString(e));
    }
  }
  dev_free(staging);
  return MRL_OK;
}

extern "C" void mrl_index_destroy(mrl_index* index) {
  if (!index) return;
  mrl_ctx* ctx = index->ctx;
  (void)hipSetDevice(ctx->device);
  // other contexts' streams may still read it
  (void)hipDeviceSynchronize();
  dev_free(index->d_blocks);
  dev_free(index->d_recs);
  dev_free(index->d_bounds);
  delete index;
  ctx_release(ctx);
}

// Block bounds of an uploaded index: every block whose header carries
// MRL_BLOCK_FLAG_ONE_CLUSTER belongs to the cluster in coarse_cluster_id
// (header dword 3 = coarse_cluster_id | block_flags << 16, src/block.rs:38-39).
// Builds the centers and radii on the device (k_bound_centers,
// k_bound_radii); no flagged block: no bounds.  Caller holds the lock.
static int build_bounds(mrl_ctx* ctx, mrl_index* ix) {
  const uint64_t B = ix->n_blocks;
  if (!B) return MRL_OK;
  std::vector<uint32_t> h3(B);
  HIP_TRY(hipMemcpy2DAsync(h3.data(), 4, ix->d_blocks + 12, kBlockBytes, 4, B, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  std::map<uint32_t, uint32_t> dense;
  std::vector<uint32_t> bcl(B, ~0u);
  for (uint64_t b = 0; b < B; ++b)
    if ((h3[b] >> 16) & kBlockFlagOneCluster) {
      auto it = dense.emplace(h3[b] & 0xffffu, (uint32_t)dense.size()).first;
      bcl[b] = it->second;
    }
  const uint32_t n_cl = (uint32_t)dense.size();
  if (!n_cl) return MRL_OK;
  std::vector<uint32_t> start(n_cl + 1, 0), blocks;
  for (uint64_t b = 0; b < B; ++b)
    if (bcl[b] != ~0u) ++start[bcl[b] + 1];
  for (uint32_t c = 0; c < n_cl; ++c) start[c + 1] += start[c];
  blocks.resize(start[n_cl]);
  {
    std::vector<uint32_t> fill(start.begin(), start.end() - 1);
    for (uint64_t b = 0; b < B; ++b)
      if (bcl[b] != ~0u) blocks[fill[bcl[b]]++] = (uint32_t)b;
  }
  const size_t center_bytes = (size_t)n_cl * kBndStride * 4, cnorm_bytes = (size_t)n_cl * 16;
  const size_t bcl_bytes = ((B * 4 + 15) / 16) * 16, brad_bytes = B * 16;
  const size_t bytes = center_bytes + cnorm_bytes + bcl_bytes + brad_bytes;
  uint32_t* d_csr = nullptr;
  if (hipMalloc(&ix->d_bounds, bytes) != hipSuccess) {
    ix->d_bounds = nullptr;
    return fail(MRL_ERR_OUT_OF_MEMORY, "block bounds");
  }
  if (hipMalloc(&d_csr, (start.size() + blocks.size()) * 4) != hipSuccess) {
    dev_free(ix->d_bounds);
    ix->d_bounds = nullptr;
    return fail(MRL_ERR_OUT_OF_MEMORY, "block bounds");
  }
  ix->d_center = reinterpret_cast<float*>(ix->d_bounds);
  ix->d_cnorm = reinterpret_cast<float*>(ix->d_bounds + center_bytes);
  ix->d_bcl = reinterpret_cast<uint32_t*>(ix->d_bounds + center_bytes + cnorm_bytes);
  ix->d_brad = reinterpret_cast<float*>(ix->d_bounds + center_bytes + cnorm_bytes + bcl_bytes);
  hipError_t e = hipMemcpyAsync(ix->d_bcl, bcl.data(), B * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d_csr, start.data(), start.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d_csr + start.size(), blocks.data(), blocks.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  BoundBuildArgs a{};
  a.idx = ix->d_blocks;
  a.recs = ix->recs();
  a.n_blocks = B;
  a.cl_start = d_csr;
  a.cl_blocks = d_csr + start.size();
  a.n_cl = n_cl;
  a.flag_tabs = ctx->d_flag_tabs;
  for (int i = 0; i < 16; ++i) a.cb[i] = ctx->consts.eden_codebook[i];
  a.center = ix->d_center;
  a.cnorm = ix->d_cnorm;
  a.bcl = ix->d_bcl;
  a.brad = ix->d_brad;
  if (e == hipSuccess) e = launch_bound_build(a, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  dev_free(d_csr);
  if (e != hipSuccess) {
    dev_free(ix->d_bounds);
    ix->d_bounds = nullptr;
    return fail(MRL_ERR_HIP, std::string("block bounds: ") + hipGetErrorString(e));
  }
  ix->n_cl = n_cl;
  return MRL_OK;
}

// Pass schedule (the same for every K).  When the index has more than 256
// blocks, a sampling pass first scores every S0-th block (S0 the smallest
// power of two leaving at most 256 blocks), with no threshold; the final pass
// then scores every block.  Block ids are arithmetic, so a pass needs no
// index list.
static int get_levels(mrl_index* ix, uint32_t K, LevelPlan** out) {
  std::lock_guard<std::mutex> g(ix->levels_mu);  // map nodes stay put: the pointer outlives the lock
  auto it = ix->levels.find(K);
  if (it != ix->levels.end()) {
    *out = &it->second;
    return MRL_OK;
  }
  const uint64_t B = ix->n_blocks;
  LevelPlan lp;
  uint32_t s0 = 0;
  while (((B + (1ull << s0) - 1) >> s0) > 256) ++s0;
  if (s0 > 0) {
    Pass p;
    p.shift = s0;
    p.prev_shift = -1;
    p.n_pos = (uint32_t)((B + (1ull << s0) - 1) >> s0);
    p.n_new = p.n_pos;
    lp.passes.push_back(p);
  }
  Pass f;
  f.shift = 0;
  f.prev_shift = -1;
  f.n_pos = (uint32_t)B;
  f.n_new = (uint32_t)B;
  lp.passes.push_back(f);
  auto res = ix->levels.emplace(K, std::move(lp));
  *out = &res.first->second;
  return MRL_OK;
}

// ---------------------------------------------------------------------------
// plans
// ---------------------------------------------------------------------------
static int check_fit(const mrl_eden_fit* f, uint32_t dim, uint32_t bits, const char* what) {
  if (!f) return fail(MRL_ERR_INVALID_ARG, std::string(what) + " requires an EdenFit");
  if (f->dim != dim || f->bits != bits || !f->mean)
    return fail(MRL_ERR_INVALID_ARG, std::string(what) + " fit must have dim " + std::to_string(dim) + ", bits " +
                                         std::to_string(bits));
  return MRL_OK;
}

// Plan kernel over the plan set's resident queries.  Caller holds the lock.
static PlanArgs plan_args(const mrl_ctx* ctx, const mrl_plans* p) {
  PlanArgs a;
  a.queries = p->d_queries;
  a.n_q = p->n_q;
  a.dims = p->dims;
  a.prefix_codec = p->prefix_codec;
  a.mid_codec = p->mid_codec;
  a.eden_mean = p->d_eden_mean;
  a.eden_seed = p->eden_seed;
  a.mid_mean = p->d_mid_mean;
  a.mid_seed = p->mid_seed;
  a.c = ctx->consts;
  a.out = p->d_plans;
  a.luts = p->d_luts;
  return a;
}

static int enqueue_plan(mrl_ctx* ctx, mrl_plans* p) {
  if (!p->n_q) return MRL_OK;
  const PlanArgs a = plan_args(ctx, p);
  ProfScope ps(ctx, MRL_KERNEL_PLAN, 0, 0, p->n_q);
  HIP_TRY(launch_plan(a, ctx->stream, ps.ev()));
  ps.commit(p->n_q != 0);
  return MRL_OK;
}

// Builds plans whose build is still pending (the lazy build of
// mrl_plans_build / _rebuild).  Caller holds the lock.
static int flush_plans(mrl_ctx* ctx, const mrl_plans* plans) {
  if (!plans || !plans->pending) return MRL_OK;
  int rc = enqueue_plan(ctx, const_cast<mrl_plans*>(plans));
  if (!rc) plans->pending = false;
  return rc;
}

static int plans_build_impl(mrl_ctx* ctx, const float* queries, bool on_device, uint32_t n_q, uint32_t dims,
                            int prefix_codec, int mid_codec, const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                            mrl_plans** out) {
  if (!ctx || !out || (n_q && !queries)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  if (dims < (uint32_t)(kPrefixDims + kRabitqDims)) return fail(MRL_ERR_INVALID_ARG, "dims must be >= 192");  // scan.rs:114
  if (dims > MRL_MAX_DIMS) return fail(MRL_ERR_INVALID_ARG, "dims above MRL_MAX_DIMS");
  if (prefix_codec != MRL_PREFIX_MINMAX4 && prefix_codec != MRL_PREFIX_EDEN_PROD)
    return fail(MRL_ERR_INVALID_ARG, "unknown prefix codec");
  if (mid_codec != MRL_MID_RABITQ && mid_codec != MRL_MID_EDEN_B1) return fail(MRL_ERR_INVALID_ARG, "unknown mid codec");
  int rc;
  if (prefix_codec == MRL_PREFIX_EDEN_PROD && (rc = check_fit(eden, 64, 4, "EdenProd"))) return rc;  // scan.rs:115-119
  if (mid_codec == MRL_MID_EDEN_B1 && (rc = check_fit(eden_mid, 128, 1, "EdenB1 mid"))) return rc;  // scan.rs:120-124
  if (eden && (rc = check_fit(eden, 64, 4, "prefix"))) return rc;
  if (eden_mid && (rc = check_fit(eden_mid, 128, 1, "mid"))) return rc;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  std::unique_ptr<mrl_plans> p(new mrl_plans());
  p->ctx = ctx;
  p->n_q = n_q;
  p->dims = dims;
  p->prefix_codec = prefix_codec;
  p->mid_codec = mid_codec;
  // One device block: plans, LUTs, then the inputs [eden mean 64][mid mean
  // 128][queries], which arrive with one copy (host inputs staged in pinned
  // memory).
  const size_t nq = std::max<uint32_t>(n_q, 1);
  const size_t plan_bytes = sizeof(mrl_query_plan) * nq, lut_bytes = sizeof(float) * kQData * nq;
  const size_t qbytes = (size_t)n_q * dims * sizeof(float);
  const size_t in_bytes = (64 + 128) * sizeof(float) + qbytes;
  if (hipMalloc(&p->d_block, plan_bytes + lut_bytes + in_bytes) != hipSuccess)
    return fail(MRL_ERR_OUT_OF_MEMORY, "plans");
  p->d_plans = reinterpret_cast<mrl_query_plan*>(p->d_block);
  p->d_luts = reinterpret_cast<float*>(p->d_block + plan_bytes);
  float* d_in = reinterpret_cast<float*>(p->d_block + plan_bytes + lut_bytes);
  if (eden) {
    p->eden_seed = eden->seed;
    p->d_eden_mean = d_in;
  }
  if (eden_mid) {
    p->mid_seed = eden_mid->seed;
    p->d_mid_mean = d_in + 64;
  }
  if (n_q) p->d_queries = d_in + 192;
  hipError_t e = hipSuccess;
  if (!on_device) {
    uint8_t* h = host_stage(ctx, in_bytes);
    if (!h) {
      dev_free(p->d_block);
      return fail(MRL_ERR_OUT_OF_MEMORY, "pinned staging buffer");
    }
    float* hf = reinterpret_cast<float*>(h);
    if (eden) memcpy(hf, eden->mean, 64 * sizeof(float));
    if (eden_mid) memcpy(hf + 64, eden_mid->mean, 128 * sizeof(float));
    if (n_q) memcpy(hf + 192, queries, qbytes);
    e = hipMemcpyAsync(d_in, h, in_bytes, hipMemcpyHostToDevice, ctx->stream);
  } else {
    float means[192] = {0};
    if (eden) memcpy(means, eden->mean, 64 * sizeof(float));
    if (eden_mid) memcpy(means + 64, eden_mid->mean, 128 * sizeof(float));
    e = hipMemcpy(d_in, means, sizeof(means), hipMemcpyHostToDevice);
    if (e == hipSuccess && n_q) e = hipMemcpyAsync(d_in + 192, queries, qbytes, hipMemcpyDeviceToDevice, ctx->stream);
  }
  if (e != hipSuccess) {
    dev_free(p->d_block);
    return fail(MRL_ERR_HIP, "plan inputs copy");
  }
  int rc2 = MRL_OK;
  p->pending = true;  // built by the first call that reads the plans
  // The pinned inputs are reused by the next call: wait for the copy (host path).
  if (!rc2 && !on_device && hipStreamSynchronize(ctx->stream) != hipSuccess) rc2 = fail(MRL_ERR_HIP, "plan build");
  if (rc2) {
    (void)hipStreamSynchronize(ctx->stream);
    dev_free(p->d_block);
    return rc2;
  }
  ctx_retain(ctx);
  *out = p.release();
  return MRL_OK;
}

extern "C" int mrl_plans_build(mrl_ctx* ctx, const float* queries, uint32_t n_q, uint32_t dims, int prefix_codec,
                               int mid_codec, const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                               mrl_plans** out) {
  return plans_build_impl(ctx, queries, false, n_q, dims, prefix_codec, mid_codec, eden, eden_mid, out);
}

extern "C" int mrl_plans_build_device(mrl_ctx* ctx, const float* d_queries, uint32_t n_q, uint32_t dims,
                                      int prefix_codec, int mid_codec, const mrl_eden_fit* eden,
                                      const mrl_eden_fit* eden_mid, mrl_plans** out) {
  return plans_build_impl(ctx, d_queries, true, n_q, dims, prefix_codec, mid_codec, eden, eden_mid, out);
}

extern "C" int mrl_plans_rebuild(mrl_ctx* ctx, mrl_plans* plans) {
  if (!ctx || !plans) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (plans->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "plans belong to another context");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  plans->pending = true;  // built by the next call that reads the plans
  return MRL_OK;
}

extern "C" int mrl_plans_count(const mrl_plans* plans, uint32_t* out) {
  if (!plans || !out) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = plans->n_q;
  return MRL_OK;
}

extern "C" int mrl_plans_export(mrl_ctx* ctx, const mrl_plans* plans, uint32_t first, uint32_t count,
                                mrl_query_plan* out) {
  if (!ctx || !plans || (count && !out)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if ((uint64_t)first + count > plans->n_q) return fail(MRL_ERR_INVALID_ARG, "plan range out of bounds");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  int rc = flush_plans(ctx, plans);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  if (count) HIP_TRY(hipMemcpy(out, plans->d_plans + first, sizeof(mrl_query_plan) * count, hipMemcpyDeviceToHost));
  return MRL_OK;
}

extern "C" void mrl_plans_destroy(mrl_plans* plans) {
  if (!plans) return;
  mrl_ctx* ctx = plans->ctx;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  dev_free(plans->d_block);
  delete plans;
  ctx_release(ctx);
}

// ---------------------------------------------------------------------------
// scan
// ---------------------------------------------------------------------------
static int check_cfg(const mrl_scan_config* cfg, uint32_t* k_eff) {
  if (!cfg) return fail(MRL_ERR_INVALID_ARG, "cfg is null");
  if (cfg->strata_depth < MRL_STRATA_L0_ONLY || cfg->strata_depth > MRL_STRATA_FULL64B)
    return fail(MRL_ERR_INVALID_ARG, "unknown strata_depth");
  if (cfg->shortlist_cand > MRL_MAX_SHORTLIST) return fail(MRL_ERR_INVALID_ARG, "shortlist_cand above 4096");
  *k_eff = std::max<uint32_t>(cfg->shortlist_cand, 1);  // Shortlist::new: capacity.max(1)
  return MRL_OK;
}

static ScanParams make_params(const mrl_scan_config* cfg, const mrl_time_range* t) {
  ScanParams sp{};
  sp.alpha = cfg->cs_tolerance;
  sp.w_s4 = cfg->stratum4_weight;
  sp.strata = cfg->strata_depth;
  sp.temporal = cfg->temporal_filter_enable ? 1 : 0;
  sp.has_lo = t && t->has_lo;
  sp.lo = t ? t->lo : 0;
  sp.has_hi = t && t->has_hi;
  sp.hi = t ? t->hi : 0;
  sp.exhaustive = cfg->exhaustive ? 1 : 0;
  return sp;
}

static void results_free(mrl_results* r) {
  dev_free(r->d_out);
  dev_free(r->d_cand_score);
  dev_free(r->d_cand_row);
  dev_free(r->d_cand_lower);
  dev_free(r->d_mma);
  dev_free(r->d_seg_count);
  dev_free(r->d_tau);
  dev_free(r->d_tau_hi);
  dev_free(r->d_hist);
  dev_free(r->d_err);
  dev_free(r->d_rr);
}

static void results_release(mrl_results* r) {
  if (!r) return;
  results_free(r);
  delete r;
}

static size_t results_head_bytes(uint32_t n_q) { return (size_t)n_q * 8 + kStatCopies * kStatCount * 8; }

static const uint32_t kSegCap = 4096;  // kSegs * kSegCap = 65536 candidates per query and scan

// MFMA path, per query: query operands, kMcCount constants and k_exact's
// work items (kFinCap / kExactItem), plus 16 bytes for the work list's head.
static size_t mma_bytes_per_query() { return (size_t)2 * kMmaSteps * 16 + kMcCount * 4 + kFinCap / kExactItem * 4; }
static size_t mma_bytes(uint32_t n_q) { return (size_t)std::max<uint32_t>(n_q, 1) * mma_bytes_per_query() + 16; }

// A results object that holds no reference to its context (the context's
// own spare, kept for mrl_scan); mrl_results_create adds the reference.
static int results_create(mrl_ctx* ctx, uint32_t n_q, uint32_t k, mrl_results** out) {
  if (!ctx || !out) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (k == 0 || k > MRL_MAX_SHORTLIST) return fail(MRL_ERR_INVALID_ARG, "k must be in [1, 4096]");
  *out = nullptr;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  std::unique_ptr<mrl_results> r(new mrl_results());
  r->ctx = ctx;
  r->n_q = n_q;
  r->k = k;
  r->seg_cap = kSegCap;
  const size_t nq = std::max<uint32_t>(n_q, 1);
  const size_t cands = nq * kSegs * (size_t)kSegCap;
  const size_t head = results_head_bytes((uint32_t)nq);
  r->out_bytes = head + nq * k * 12;
  bool ok = hipMalloc(&r->d_out, r->out_bytes) == hipSuccess;
  if (ok) {
    r->d_status = reinterpret_cast<uint32_t*>(r->d_out);
    r->d_counts = r->d_status + nq;
    r->d_stats = reinterpret_cast<unsigned long long*>(r->d_out + nq * 8);
    r->d_ids = reinterpret_cast<uint64_t*>(r->d_out + head);
    r->d_scores = reinterpret_cast<float*>(r->d_out + head + nq * k * 8);
  }
  ok = ok && hipMalloc(&r->d_cand_score, cands * sizeof(float)) == hipSuccess &&
            hipMalloc(&r->d_cand_row, cands * sizeof(uint32_t)) == hipSuccess &&
            hipMalloc(&r->d_cand_lower, cands * sizeof(float)) == hipSuccess &&
            hipMalloc(&r->d_mma, mma_bytes((uint32_t)nq)) == hipSuccess &&
            hipMalloc(&r->d_seg_count, nq * kMaxSegs * sizeof(uint32_t)) == hipSuccess &&
            hipMalloc(&r->d_tau, nq * sizeof(float)) == hipSuccess &&
            hipMalloc(&r->d_tau_hi, nq * sizeof(float)) == hipSuccess &&
            hipMalloc(&r->d_hist, nq * kHistBins * sizeof(uint32_t)) == hipSuccess &&
            hipMalloc(&r->d_err, nq * sizeof(uint32_t)) == hipSuccess;
  if (!ok) {
    results_free(r.get());
    return fail(MRL_ERR_OUT_OF_MEMORY, "results buffers");
  }
  // Pass state starts zeroed; each final selection leaves it zeroed again.
  ok = hipMemset(r->d_seg_count, 0, nq * kMaxSegs * sizeof(uint32_t)) == hipSuccess &&
       hipMemset(r->d_err, 0, nq * sizeof(uint32_t)) == hipSuccess &&
       hipMemset(r->d_out, 0, head) == hipSuccess &&
       hipMemset(r->d_hist, 0, nq * kHistBins * sizeof(uint32_t)) == hipSuccess &&
       hipDeviceSynchronize() == hipSuccess;
  if (!ok) {
    results_free(r.get());
    return fail(MRL_ERR_HIP, "results init");
  }
  *out = r.release();
  return MRL_OK;
}

extern "C" int mrl_results_create(mrl_ctx* ctx, uint32_t n_q, uint32_t k, mrl_results** out) {
  const int rc = results_create(ctx, n_q, k, out);
  if (rc == MRL_OK) ctx_retain(ctx);
  return rc;
}

// Frees a results object without touching its context's reference count.
static void results_destroy(mrl_results* res) {
  (void)hipSetDevice(res->ctx->device);
  (void)hipStreamSynchronize(res->ctx->stream);
  results_free(res);
  delete res;
}

extern "C" void mrl_results_destroy(mrl_results* res) {
  if (!res) return;
  mrl_ctx* ctx = res->ctx;
  results_destroy(res);
  ctx_release(ctx);
}

// Buffers one scan writes its candidates into.
struct PassBuffers {
  float* cand_score;
  uint32_t* cand_row;
  float* cand_lower = nullptr;    // MFMA path (null: the exact kernels only)
  uint4* mma_ops = nullptr;
  float* mma_consts = nullptr;
  uint32_t* mma_work = nullptr;
  uint32_t* seg_count;
  uint32_t nseg;
  uint32_t seg_cap;
  uint32_t* err;
  float* tau;
  float* tau_hi;
  uint32_t* hist;
  uint32_t* status;
  uint64_t* out_ids;
  float* out_scores;
  uint32_t* out_counts;
  bool block_lists = true;  // false: never skip blocks (the block selection allocates its scratch)
};

// Floor rank for the final pass: the rank-th best score of a sample of n_s
// of the index's n blocks.  The number of sampled vectors above the true
// K-th score is about Poisson(lambda = K * n_s / n); the final floor is too
// high only if at least `rank` of them are, and rank = lambda + 4 sqrt(lambda)
// + 6 leaves a tail of ~1e-6 or less (then the query is re-run at the safe
// floor) while the final pass keeps about rank * n / n_s candidates.  Never
// above K (then the floor is the safe one).
static uint32_t final_rank(uint32_t K, uint64_t n_s, uint64_t n) {
  const double lambda = (double)K * (double)n_s / (double)std::max<uint64_t>(n, 1);
  const double r = std::ceil(lambda + 4.0 * std::sqrt(lambda) + 6.0);
  return (uint32_t)std::min<double>((double)K, std::max(1.0, r));
}

// The one-query kernel's final pass gives each workgroup a candidate segment
// of its own (no atomic reservation) when the results hold kSegs segments per
// query; an append count past the room flags the query for the dense re-run.
static const uint32_t kExclCap = 1024;  // the kernel's per-workgroup staging room
static bool excl_ok(const PassBuffers& pb, uint32_t n_q, const ScanParams& sp) {
  return pb.nseg == (uint32_t)kSegs && scan_query_tile(n_q) == 1 && sp.strata != MRL_STRATA_L0_ONLY;
}

// Enqueue a scan of n_q plans starting at plans_first.  The sampling pass
// (when the index has more than 256 blocks) scores a strided sample of
// blocks with no candidate appends and counts the survivors' exact scores
// per query.  The final pass scores every block; its workgroups take the
// floor from those counts at rank final_rank, prune and append at it, and
// k_select emits the top K (and flags a query whose floor left fewer than K
// candidates).  rerun_safe: the final pass alone at the safe floor k_select
// kept (rank K).  Caller holds the context lock.
// The MFMA-bounded path serves batches under the settings where the
// reference's top K is the top K by full score (the conditions tight_coef()
// checks on the device) and the RaBitQ mid-band.
static bool mma_ok(const mrl_plans* plans, uint32_t n_q, const ScanParams& sp, const PassBuffers& pb) {
  return pb.cand_lower && n_q >= (uint32_t)kMmaMinQ && plans->mid_codec == MRL_MID_RABITQ &&
         sp.strata != MRL_STRATA_L0_ONLY && sp.alpha >= 1.0f && sp.w_s4 >= 0.0f && 2.4f * sp.w_s4 <= sp.alpha;
}

// Sampling stages of the MFMA path: blocks b = pos << shift, pos < n_pos.
// Above 256 blocks a first stage scores 16..128 blocks (fewer for larger
// batches); when that is at most 1/128 of the index, a second stage scores
// every 64th block (every 32nd when the index has fewer than 32 K blocks, or
// the first stage is at most 1/64 of it) but counts only lower bounds at or
// above the first stage's floor, so its histogram stays small while its
// floor (rank final_rank of a much larger sample) is much tighter.  A
// sparser second stage costs less but leaves a looser floor, so more pairs
// are appended in the final pass; on the benchmark indexes every 64th block
// paid when the index holds 32 K blocks or more (8.8M vectors, K 256:
// 0.418 -> 0.413 ms per step; 1M, K 256: -1.5 us) and lost below
// (1M, K 1024: +5 us), and every 16th block cost more than it saved.
// Per-workgroup list room below which a later sampling stage counts into the
// global histogram instead.
static const uint32_t kMinListCap = 16;
struct MmaStage {
  uint32_t shift;
  uint32_t n_pos;
};
// One sampling stage that stores every pair's lower bound serves an index
// without block bounds when its stride is at least 1/16 and its block-query
// pairs stay under kOneStageBudget (8.8M vectors x 64 queries: every 256th
// block, 34,368 bounds per query); config 4: 0.406 -> 0.397 ms per step.  Over
// block lists such a sample misses the queries' clusters and the floor is too
// loose to skip blocks (0.165 -> 0.424 ms), so those keep two stages.
static const uint64_t kOneStageBudget = 40000;

// one_stage_room: the lower bounds a query's row holds (0: two stages).
static std::vector<MmaStage> mma_stages(uint64_t B, uint32_t n_q, uint32_t K, uint32_t one_stage_room) {
  std::vector<MmaStage> st;
  if (B <= 256) return st;
  if (one_stage_room) {
    uint32_t s = 0;
    while (((B + (1ull << s) - 1) >> s) * 64ull > one_stage_room) ++s;
    const uint64_t n_pos = (B + (1ull << s) - 1) >> s;
    if (s >= 4 && n_pos * n_q <= kOneStageBudget) {
      st.push_back(MmaStage{s, (uint32_t)n_pos});
      return st;
    }
  }
  // the first stage counts every pair: keep it near 4096 x 64 block-queries
  const uint64_t cap = std::min<uint64_t>(128, std::max<uint64_t>(16, 4096 / std::max<uint32_t>(n_q, 1)));
  uint32_t s1 = 0;
  while (((B + (1ull << s1) - 1) >> s1) > cap) ++s1;
  st.push_back(MmaStage{s1, (uint32_t)((B + (1ull << s1) - 1) >> s1)});
  // the second stage holds at least twice the first stage's blocks
  const uint32_t s2 = B >= 32ull * K && s1 >= 7 ? 6u : 5u;
  if (s1 >= s2 + 1) st.push_back(MmaStage{s2, (uint32_t)((B + (1ull << s2) - 1) >> s2)});
  return st;
}

// Block bounds apply to scans whose score is the code-space dot product the
// bounds were built for: the RaBitQ mid-band, an S1 stage, and pruning on.
static bool bounds_ok(const mrl_index* ix, const mrl_plans* plans, const ScanParams& sp, const PassBuffers& pb) {
  return pb.block_lists && ix->n_cl != 0 && plans->mid_codec == MRL_MID_RABITQ &&
         (sp.strata == MRL_STRATA_L1_RABITQ || sp.strata == MRL_STRATA_FULL64B) && !sp.exhaustive;
}

// Scratch of the block selection of one scan, in the index (grown on demand):
// the cluster x query table, the query norms, two count arrays (one per
// block list of the scan) and the block lists, n_chunks of n_blocks each.
struct BoundSel {
  float* table;
  float* qn;
  uint32_t* bcount;  // [2][n_chunks]
  uint32_t* blist;
  uint32_t n_chunks;
  uint32_t chunk;
};

// The cluster x query table of a scan whose workgroups take `chunk` queries
// each; clears both count arrays.  Caller holds the lock.
static int enqueue_bound_table(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t plans_first,
                               uint32_t n_q, const ScanParams& sp, uint32_t chunk, BoundSel* sel) {
  if (int rc = flush_plans(ctx, plans)) return rc;
  const uint32_t n_chunks = (n_q + chunk - 1) / chunk;
  const size_t table_bytes = ((size_t)ix->n_cl * n_q * 4 + 255) & ~(size_t)255;
  const size_t qn_bytes = ((size_t)n_q * 16 + 255) & ~(size_t)255;
  const size_t count_bytes = ((size_t)2 * n_chunks * 4 + 255) & ~(size_t)255;
  const size_t need = table_bytes + qn_bytes + count_bytes + (size_t)n_chunks * ix->n_blocks * 4;
  if (need > ctx->bsel_bytes) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));  // an earlier scan may still read the old lists
    dev_free(ctx->d_bsel);
    ctx->d_bsel = nullptr;
    ctx->bsel_bytes = 0;
    if (hipMalloc(&ctx->d_bsel, need) != hipSuccess) {
      ctx->d_bsel = nullptr;
      return fail(MRL_ERR_OUT_OF_MEMORY, "block selection");
    }
    ctx->bsel_bytes = need;
  }
  sel->table = reinterpret_cast<float*>(ctx->d_bsel);
  sel->qn = reinterpret_cast<float*>(ctx->d_bsel + table_bytes);
  sel->bcount = reinterpret_cast<uint32_t*>(ctx->d_bsel + table_bytes + qn_bytes);
  sel->blist = reinterpret_cast<uint32_t*>(ctx->d_bsel + table_bytes + qn_bytes + count_bytes);
  sel->n_chunks = n_chunks;
  sel->chunk = chunk;
  BoundScanArgs b{};
  b.center = ix->d_center;
  b.cnorm = ix->d_cnorm;
  b.n_cl = ix->n_cl;
  b.n_q = n_q;
  b.plans = plans->d_plans + plans_first;
  b.luts = plans->d_luts + (size_t)plans_first * kQData;
  b.sp = sp;
  b.eden = plans->prefix_codec == MRL_PREFIX_EDEN_PROD;
  b.table = sel->table;
  b.qn = sel->qn;
  b.bcount = sel->bcount;
  b.chunk = chunk;
  ProfScope ps(ctx, MRL_KERNEL_BOUNDS, 0, 0, n_q);
  HIP_TRY(launch_bound_table(b, ctx->stream, ps.ev()));
  ps.commit(true);
  return MRL_OK;
}

// Block list `which` (0 or 1) of the pass over blocks pos << shift, pos <
// n_pos, at the floors in `floor`; points the block-list fields of *a at it.
// Caller holds the lock.
static int enqueue_block_select(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t n_q,
                                const BoundSel& sel, int which, const float* floor, uint32_t n_pos, uint32_t shift,
                                ScanArgs* a) {
  BoundScanArgs b{};
  b.n_cl = ix->n_cl;
  b.bcl = ix->d_bcl;
  b.brad = ix->d_brad;
  b.n_blocks = ix->n_blocks;
  b.n_q = n_q;
  b.eden = plans->prefix_codec == MRL_PREFIX_EDEN_PROD;
  b.table = sel.table;
  b.qn = sel.qn;
  b.floor = floor;
  b.n_pos = n_pos;
  b.shift = shift;
  b.chunk = sel.chunk;
  b.bcount = sel.bcount + (size_t)which * sel.n_chunks;
  b.blist = sel.blist;
  b.stride = (uint32_t)ix->n_blocks;
  ProfScope ps(ctx, MRL_KERNEL_BOUNDS, 1 + which, n_pos, n_q);
  HIP_TRY(launch_block_select(b, ctx->stream, ps.ev()));
  ps.commit(n_pos != 0);
  a->blist = b.blist;
  a->bcount = b.bcount;
  a->blist_stride = b.stride;
  return MRL_OK;
}

// MFMA-bounded scan of n_q plans: operands (k_mma_prep); the sampling stages,
// each followed by k_mma_floors (final floor at rank final_rank, safe floor
// at rank K); the final pass, which appends (upper, lower, row) for the pairs
// whose upper bound reaches the floor (every active pair when the index has
// no sampling stage); k_finish lists the candidates whose upper bound reaches
// the K-th best lower bound; k_exact scores them exactly; k_select emits the
// top K.  rerun_safe: the final pass alone at the safe floor.
static int enqueue_scan_mma(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t plans_first, uint32_t n_q,
                            const ScanParams& sp, uint32_t K, const PassBuffers& pb, unsigned long long* stats,
                            bool rerun_safe, bool fuse_prep = false) {
  hipStream_t s = ctx->stream;
  const uint64_t B = ix->n_blocks;
  const std::vector<MmaStage> stages =
      rerun_safe ? std::vector<MmaStage>() : mma_stages(B, n_q, K, bounds_ok(ix, plans, sp, pb) ? 0u : pb.nseg * pb.seg_cap);
  const bool sampled = !stages.empty();
  {
    MmaPrepArgs pa{};
    pa.plans = plans->d_plans + plans_first;
    pa.luts = plans->d_luts + (size_t)plans_first * kQData;
    pa.n_q = n_q;
    pa.sp = sp;
    pa.ops = pb.mma_ops;
    pa.consts = pb.mma_consts;
    pa.work = pb.mma_work;
    if (fuse_prep) {  // the batch's pending plans first, in the same launch
      ProfScope ps(ctx, MRL_KERNEL_PLAN_PREP, 0, 0, n_q);
      HIP_TRY(launch_plan_mma_prep(plan_args(ctx, plans), pa, s, ps.ev()));
      ps.commit(n_q != 0);
      plans->pending = false;
    } else {
      ProfScope ps(ctx, MRL_KERNEL_MMA_PREP, 0, 0, n_q);
      HIP_TRY(launch_mma_prep(pa, s, ps.ev()));
      ps.commit(n_q != 0);
    }
  }
  ScanArgs a{};
  a.idx = ix->d_blocks;
  a.recs = ix->recs();
  a.n_blocks = B;
  a.prev_shift = -1;
  a.plans = plans->d_plans + plans_first;
  a.luts = plans->d_luts + (size_t)plans_first * kQData;
  a.n_q = n_q;
  a.flag_tabs = ctx->d_flag_tabs;
  a.sp = sp;
  a.cand_score = pb.cand_score;
  a.cand_row = pb.cand_row;
  a.cand_lower = pb.cand_lower;
  a.seg_count = pb.seg_count;
  a.nseg = pb.nseg;
  a.seg_cap = pb.seg_cap;
  a.err = pb.err;
  a.mma_ops = pb.mma_ops;
  a.mma_consts = pb.mma_consts;
  // block bounds: the table once; a block list for every stage with a floor
  const bool bounded = sampled && bounds_ok(ix, plans, sp, pb);
  BoundSel sel{};
  int rc;
  if (bounded && (rc = enqueue_bound_table(ctx, ix, plans, plans_first, n_q, sp, kMmaQ, &sel))) return rc;
  for (size_t si = 0; si < stages.size(); ++si) {
    a.n_pos = stages[si].n_pos;
    a.shift = stages[si].shift;
    a.tau = si ? pb.tau_hi : nullptr;  // count only lower bounds at or above the previous floor
    a.hist = pb.hist;
    a.stats = nullptr;
    a.blist = nullptr;
    a.bcount = nullptr;
    // a block whose bound lies below the previous floor adds no count
    if (si && bounded &&
        (rc = enqueue_block_select(ctx, ix, plans, n_q, sel, 0, pb.tau_hi, a.n_pos, a.shift, &a)))
      return rc;
    // The first stage (no previous floor) counts every pair: it stores the
    // lower bounds in the MFMA lower-bound area (free until the final pass)
    // and the floors kernel builds the histograms, instead of contended
    // global histogram atomics.
    // A later stage over block lists (counting only the bounds at or above
    // the previous floor, which on a cluster-grouped index concentrates them
    // on a few histogram bins) lists them per workgroup in the same area, the
    // list lengths in the candidate-row area (also free until the final
    // pass), when every workgroup's list gets kMinListCap entries or more.
    // (Without block lists the global histogram atomics cost no more than
    // the lists: 1M..8.8M-vector benchmark indexes, batches 64..1024.)
    const uint32_t lb_stride = pb.nseg * pb.seg_cap;
    const bool store = si == 0 && (uint64_t)stages[si].n_pos * 64u <= lb_stride;
    const uint32_t n_wg = mma_scan_grid(a);
    const uint32_t lcap = n_wg ? lb_stride / n_wg : 0u;
    const bool lists = si != 0 && a.blist && lcap >= kMinListCap && n_wg <= (uint32_t)kMaxListWg;
    a.lbuf = store || lists ? pb.cand_lower : nullptr;
    a.lbuf_stride = store || lists ? lb_stride : 0u;
    a.lcount = lists ? pb.cand_row : nullptr;
    a.lcap = lists ? lcap : 0u;
    ProfScope ps(ctx, MRL_KERNEL_SCAN, (int)si, stages[si].n_pos, n_q);
    HIP_TRY(launch_scan_mma(a, 0, s, ps.ev()));
    ps.commit(a.n_pos != 0 && n_q != 0);
    ProfScope pt(ctx, MRL_KERNEL_THRESH, (int)si, 0, n_q);
    if (store)
      HIP_TRY(launch_mma_floors_lb(pb.cand_lower, lb_stride, stages[si].n_pos * 64u, a.luts, n_q,
                                   final_rank(K, stages[si].n_pos, B), K, pb.tau_hi, pb.tau, s, pt.ev()));
    else if (lists)
      HIP_TRY(launch_mma_floors_seg(pb.cand_lower, pb.cand_row, lb_stride, n_wg, lcap, pb.hist, a.luts, n_q,
                                    final_rank(K, stages[si].n_pos, B), K, pb.tau_hi, pb.tau, s, pt.ev()));
    else
      HIP_TRY(launch_mma_floors(pb.hist, a.luts, n_q, final_rank(K, stages[si].n_pos, B), K, pb.tau_hi, pb.tau,
                                si != 0, s, pt.ev()));
    pt.commit(n_q != 0);
    a.lbuf = nullptr;
    a.lbuf_stride = 0u;
    a.lcount = nullptr;
    a.lcap = 0u;
  }
  const int final_pass = (int)stages.size();
  const float* floor = rerun_safe ? pb.tau : (sampled ? pb.tau_hi : nullptr);
  a.n_pos = (uint32_t)B;
  a.shift = 0;
  a.tau = floor;
  a.hist = nullptr;
  a.stats = stats;
  a.blist = nullptr;
  a.bcount = nullptr;
  if (bounded && (rc = enqueue_block_select(ctx, ix, plans, n_q, sel, 1, floor, (uint32_t)B, 0u, &a))) return rc;
  // The final pass bounds the S4 stage instead of running its four K-steps
  // when it is expected to append few pairs.  The last sample's floor, at
  // rank r of its n_pos blocks, leaves about r B / n_pos vectors per query
  // with a lower bound above it, and about twice that many with an upper
  // bound above it: 64 r / n_pos appends per 32-vector tile of 64 queries.
  // The S4 bound lets more pairs through, and past about 2 appends per tile
  // their epilogue and exact S4 sums cost more than the four K-steps save
  // (config 4: 1.3, kept; config 3: 3.3, not kept).  On block lists (a
  // cluster-grouped index) the listed blocks hold the pairs near the floor,
  // and a re-run at the safe floor appends more: both keep the full tiles.
  // A wide pass's wave whose appends pass 2 per 1024 pairs (4 per tile of
  // 64 queries, plus kMmaWideSlack) runs the full tiles for the rest of it.
  // (mrl_ctx_set_s4_bound: ALWAYS / NEVER override the estimate.)
  {
    const uint32_t n_last = stages.empty() ? 0u : stages.back().n_pos;
    const double per_tile = n_last ? 64.0 * final_rank(K, n_last, B) / n_last : 1e30;
    const bool cheap = !rerun_safe && !bounded && per_tile < 2.0;
    const bool fits = sp.strata != MRL_STRATA_FULL64B || sp.w_s4 <= kMmaWideMaxWs4;
    const int pol = ctx->s4_policy;
    a.mma_wide = floor && fits && pol != MRL_S4_BOUND_NEVER && (cheap || pol == MRL_S4_BOUND_ALWAYS) ? 1u : 0u;
    a.wide_lim = 2u;
  }
  // Room is left for batches of up to 256 queries, whose other launches are
  // latency-bound (a few workgroups per query); a larger batch's exact
  // scoring and selection fill the GPU themselves (config 4: 0.310 ->
  // 0.303 ms per step over three contexts, config 3 0.189 -> 0.186;
  // config 5, 1024 queries: 0.787 -> 0.812 with the room, so not there).
  const bool other = other_context_active(ctx);
  a.leave_room = other && n_q <= 256u ? 1u : 0u;
  a.lmax = reinterpret_cast<uint32_t*>(pb.mma_consts) + kMcLMax;
  {
    ProfScope ps(ctx, MRL_KERNEL_SCAN, final_pass, (uint32_t)B, n_q);
    ps.r.info.flags = a.mma_wide ? MRL_KT_S4_BOUNDED : 0u;
    HIP_TRY(launch_scan_mma(a, floor ? 1 : 2, s, ps.ev()));
    ps.commit(a.n_pos != 0 && n_q != 0);
  }
  FinishArgs fa{};
  fa.idx = ix->d_blocks;
  fa.n_blocks = B;
  fa.recs = ix->recs();
  fa.plans = plans->d_plans + plans_first;
  fa.luts = plans->d_luts + (size_t)plans_first * kQData;
  fa.mma_consts = pb.mma_consts;
  fa.sp = sp;
  fa.k = K;
  fa.cand_score = pb.cand_score;
  fa.cand_lower = pb.cand_lower;
  fa.cand_row = pb.cand_row;
  fa.seg_count = pb.seg_count;
  fa.nseg = pb.nseg;
  fa.seg_cap = pb.seg_cap;
  fa.tau_final = floor;
  fa.err = pb.err;
  fa.stats = stats;
  fa.n_q = n_q;
  fa.work = pb.mma_work;
  {
    ProfScope ps(ctx, MRL_KERNEL_FINISH, final_pass, 0, n_q);
    HIP_TRY(launch_finish(fa, n_q, s, ps.ev()));
    ps.commit(n_q != 0);
  }
  {
    ProfScope ps(ctx, MRL_KERNEL_EXACT, final_pass, 0, n_q);
    HIP_TRY(launch_exact(fa, n_q, s, ps.ev()));
    ps.commit(n_q != 0);
  }
  SelectArgs sa{};
  sa.luts = plans->d_luts + (size_t)plans_first * kQData;
  sa.cand_score = pb.cand_score;
  sa.cand_row = pb.cand_row;
  sa.seg_count = pb.seg_count;
  sa.nseg = pb.nseg;
  sa.seg_cap = pb.seg_cap;
  sa.err = pb.err;
  sa.k = K;
  sa.status = pb.status;
  sa.out_ids = pb.out_ids;
  sa.out_scores = pb.out_scores;
  sa.out_counts = pb.out_counts;
  sa.stats = stats;
  sa.hist = sampled ? pb.hist : nullptr;
  sa.tau_final = pb.tau_hi;
  sa.tau_safe = pb.tau;
  sa.tau_used = floor;
  ProfScope ps(ctx, MRL_KERNEL_SELECT, final_pass, 0, n_q);
  HIP_TRY(launch_select(sa, n_q, s, ps.ev()));
  ps.commit(n_q != 0);
  return MRL_OK;
}

static int enqueue_scan(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t plans_first, uint32_t n_q,
                        const ScanParams& sp, uint32_t K, const LevelPlan& lp, const PassBuffers& pb,
                        unsigned long long* stats, bool rerun_safe = false) {
  // A pending plan build of one query goes into its sampling pass (the fused
  // k_scan); otherwise the plans are built first.
  const bool mma = mma_ok(plans, n_q, sp, pb);
  const bool fuse = plans->pending && n_q == 1 && plans_first == 0 && plans->n_q == 1 && !rerun_safe &&
                    lp.passes.size() > 1 && sp.strata != MRL_STRATA_L0_ONLY && plans->dims <= (uint32_t)kFuseMaxDims &&
                    !mma;
  // the MFMA path builds a pending plan of the whole batch with the query
  // operands (up to one workgroup per CU: larger batches run the plan kernel
  // and the lighter operand kernel at their own occupancies)
  const bool fuse_prep = mma && plans->pending && plans_first == 0 && n_q == plans->n_q && n_q <= 256u;
  if (!fuse && !fuse_prep) {
    int rc = flush_plans(ctx, plans);
    if (rc) return rc;
  }
  if (mma) return enqueue_scan_mma(ctx, ix, plans, plans_first, n_q, sp, K, pb, stats, rerun_safe, fuse_prep);
  hipStream_t s = ctx->stream;
  const size_t np = lp.passes.size();
  const bool sampled = np > 1 && !rerun_safe;
  // Beside another context's scan, the one-query passes run 384 of their 512
  // workgroups, leaving room for that context's launches (config 2 over three
  // contexts 0.0224 -> 0.0211 ms per step; alone the final pass would take
  // 19.6 -> 22.1 us, so only then).
  const bool beside = other_context_active(ctx) && n_q < (uint32_t)kMmaMinQ;
  uint32_t nseg_final = pb.nseg, cap_final = pb.seg_cap;
  const uint32_t rank = np > 1 ? final_rank(K, lp.passes[0].n_pos, ix->n_blocks) : K;
  for (size_t pi = 0; pi < np; ++pi) {
    const bool last = pi + 1 == np;
    if (rerun_safe && !last) continue;
    ScanArgs a{};
    a.idx = ix->d_blocks;
    a.recs = ix->recs();
    a.n_blocks = ix->n_blocks;
    a.n_pos = lp.passes[pi].n_pos;
    a.shift = lp.passes[pi].shift;
    a.prev_shift = lp.passes[pi].prev_shift;
    a.plans = plans->d_plans + plans_first;
    a.luts = plans->d_luts + (size_t)plans_first * kQData;
    a.n_q = n_q;
    a.flag_tabs = ctx->d_flag_tabs;
    a.sp = sp;
    a.tau = (last && rerun_safe) ? pb.tau : nullptr;
    a.hist = last ? nullptr : pb.hist;
    a.floor_hist = (last && sampled) ? pb.hist : nullptr;
    a.floor_rank = rank;
    a.safe_rank = K;
    a.floor_out = pb.tau_hi;
    a.safe_out = pb.tau;
    a.cand_score = pb.cand_score;
    a.cand_row = pb.cand_row;
    a.seg_count = pb.seg_count;
    a.nseg = pb.nseg;
    a.seg_cap = pb.seg_cap;
    a.leave_room = beside ? 1u : 0u;
    if (last && excl_ok(pb, n_q, sp)) {
      // one segment per workgroup of the final pass, the same candidate room per query
      a.excl = 1;
      const uint32_t g = scan_grid(a, false);
      if (g >= 1 && g <= (uint32_t)kMaxSegs) {
        a.nseg = g;
        a.seg_cap = std::min<uint32_t>(pb.nseg * pb.seg_cap / g, kExclCap);
        nseg_final = a.nseg;
        cap_final = a.seg_cap;
      } else {
        a.excl = 0;
      }
    }
    a.stats = last ? stats : nullptr;
    a.err = pb.err;
    if (last && sampled && bounds_ok(ix, plans, sp, pb)) {
      // floors from the sampling counts first (as take_floors would), then
      // the blocks some query of a workgroup's tile can reach
      ProfScope pt(ctx, MRL_KERNEL_THRESH, (int)pi, 0, n_q);
      HIP_TRY(launch_mma_floors(pb.hist, a.luts, n_q, rank, K, pb.tau_hi, pb.tau, false, s, pt.ev()));
      pt.commit(n_q != 0);
      a.floor_hist = nullptr;
      a.tau = pb.tau_hi;
      const uint32_t chunk = n_q >= 8 ? (uint32_t)kTileQ : (uint32_t)scan_query_tile(n_q);
      BoundSel sel{};
      int rc = enqueue_bound_table(ctx, ix, plans, plans_first, n_q, sp, chunk, &sel);
      if (!rc) rc = enqueue_block_select(ctx, ix, plans, n_q, sel, 1, pb.tau_hi, (uint32_t)ix->n_blocks, 0u, &a);
      if (rc) return rc;
    }
    if (fuse && pi == 0) {
      a.fuse_plan = 1;
      a.plan = plan_args(ctx, plans);
    }
    ProfScope ps(ctx, a.fuse_plan ? MRL_KERNEL_PLAN_SCAN : MRL_KERNEL_SCAN, (int)pi, lp.passes[pi].n_new, n_q);
    HIP_TRY(launch_scan(a, false, s, ps.ev()));
    ps.commit(a.n_pos != 0 && n_q != 0);
    if (a.fuse_plan) plans->pending = false;
  }
  SelectArgs sa{};
  sa.luts = plans->d_luts + (size_t)plans_first * kQData;
  sa.cand_score = pb.cand_score;
  sa.cand_row = pb.cand_row;
  sa.seg_count = pb.seg_count;
  sa.nseg = nseg_final;
  sa.seg_cap = cap_final;
  sa.err = pb.err;
  sa.k = K;
  sa.status = pb.status;
  sa.out_ids = pb.out_ids;
  sa.out_scores = pb.out_scores;
  sa.out_counts = pb.out_counts;
  sa.stats = stats;
  sa.hist = sampled ? pb.hist : nullptr;
  sa.tau_final = pb.tau_hi;
  sa.tau_safe = pb.tau;
  sa.tau_used = rerun_safe ? pb.tau : (sampled ? pb.tau_hi : nullptr);
  ProfScope ps(ctx, MRL_KERNEL_SELECT, (int)np - 1, 0, n_q);
  HIP_TRY(launch_select(sa, n_q, s, ps.ev()));
  ps.commit(n_q != 0);
  return MRL_OK;
}

static PassBuffers results_buffers(mrl_results* r) {
  PassBuffers pb;
  pb.cand_score = r->d_cand_score;
  pb.cand_row = r->d_cand_row;
  pb.cand_lower = r->d_cand_lower;
  pb.mma_ops = reinterpret_cast<uint4*>(r->d_mma);
  const size_t nq = std::max<uint32_t>(r->n_q, 1);
  pb.mma_consts = reinterpret_cast<float*>(r->d_mma + nq * 2 * kMmaSteps * 16);
  pb.mma_work = reinterpret_cast<uint32_t*>(r->d_mma + nq * (2 * kMmaSteps * 16 + kMcCount * 4));
  pb.seg_count = r->d_seg_count;
  pb.nseg = kSegs;
  pb.seg_cap = r->seg_cap;
  pb.err = r->d_err;
  pb.tau = r->d_tau;
  pb.tau_hi = r->d_tau_hi;
  pb.hist = r->d_hist;
  pb.status = r->d_status;
  pb.out_ids = r->d_ids;
  pb.out_scores = r->d_scores;
  pb.out_counts = r->d_counts;
  return pb;
}

static int enqueue_gated_rerun(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t n_q,
                               const ScanParams& sp, uint32_t K, const PassBuffers& pb);

extern "C" int mrl_scan_async(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans,
                              const mrl_scan_config* cfg, const mrl_time_range* time, mrl_results* res) {
  if (!ctx || !index || !plans || !res) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (plans->ctx != ctx || res->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  if (K != res->k) return fail(MRL_ERR_INVALID_ARG, "results were created for another K");
  if (plans->n_q > res->n_q) return fail(MRL_ERR_INVALID_ARG, "results hold fewer queries than plans");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  mrl_index* ix = const_cast<mrl_index*>(index);
  const ScanParams sp = make_params(cfg, time);
  res->last_index = index;
  res->last_plans = plans;
  res->last_cfg = *cfg;
  res->last_time = time ? *time : mrl_time_range{0, 0, 0, 0};
  res->pending = true;
  res->floor_kind.assign(plans->n_q, 0);
  if (plans->n_q == 0) return MRL_OK;
  if (ix->n_blocks == 0) {
    HIP_TRY(hipMemsetAsync(res->d_counts, 0, plans->n_q * sizeof(uint32_t), ctx->stream));
    HIP_TRY(hipMemsetAsync(res->d_status, 0, plans->n_q * sizeof(uint32_t), ctx->stream));
    return MRL_OK;
  }
  LevelPlan* lp;
  if ((rc = get_levels(ix, K, &lp))) return rc;
  const PassBuffers pb = results_buffers(res);
  const bool sampled = mma_ok(plans, plans->n_q, sp, pb) ? !mma_stages(ix->n_blocks, plans->n_q, K, 0u).empty()
                                                         : lp->passes.size() > 1;
  res->floor_kind.assign(plans->n_q, sampled ? 1 : 0);
  if ((rc = enqueue_scan(ctx, ix, plans, 0, plans->n_q, sp, K, *lp, pb, res->d_stats))) return rc;
  // A query its selection left short of K above the sample's final floor is
  // re-run on the device at the safe floor (two launches that end at once for
  // every other query), so the step is complete when the stream is; only an
  // overflowed list (or a shortfall at the safe floor) is left to
  // mrl_results_fetch, which re-runs it with no floor.
  return sampled ? enqueue_gated_rerun(ctx, ix, plans, plans->n_q, sp, K, pb) : MRL_OK;
}

// Exhaustive single pass for one query whose candidate list overflowed
// (massive score ties or a threshold that could not tighten): every scored
// vector becomes a candidate in one large segment, then one exact selection
// written into the query's result row.
static int dense_rerun(mrl_ctx* ctx, mrl_results* r, uint32_t q) {
  mrl_index* ix = const_cast<mrl_index*>(r->last_index);
  const uint64_t n_vec = ix->n_blocks * 64;
  if (n_vec > 0xffffffffull) return fail(MRL_ERR_INVALID_ARG, "index too large for the dense fallback");
  float* sc = nullptr;
  uint32_t *rw = nullptr, *small = nullptr;
  if (hipMalloc(&sc, n_vec * sizeof(float)) != hipSuccess || hipMalloc(&rw, n_vec * sizeof(uint32_t)) != hipSuccess ||
      hipMalloc(&small, (kHistBins + 4) * sizeof(uint32_t)) != hipSuccess) {
    dev_free(sc);
    dev_free(rw);
    dev_free(small);
    return fail(MRL_ERR_OUT_OF_MEMORY, "dense fallback buffers");
  }
  LevelPlan lp;
  lp.passes.push_back(Pass{0u, -1, (uint32_t)ix->n_blocks, (uint32_t)ix->n_blocks});
  PassBuffers pb;
  pb.cand_score = sc;
  pb.cand_row = rw;
  pb.seg_count = small + kHistBins;
  pb.err = small + kHistBins + 1;
  pb.status = small + kHistBins + 2;
  pb.nseg = 1;
  pb.seg_cap = (uint32_t)n_vec;
  pb.tau = r->d_tau + q;
  pb.tau_hi = r->d_tau_hi + q;
  pb.hist = nullptr;
  pb.out_ids = r->d_ids + (size_t)q * r->k;
  pb.out_scores = r->d_scores + (size_t)q * r->k;
  pb.out_counts = r->d_counts + q;
  ScanParams sp = make_params(&r->last_cfg, &r->last_time);
  uint32_t st = 0;
  hipError_t e = hipMemsetAsync(small, 0, (kHistBins + 4) * sizeof(uint32_t), ctx->stream);
  int rc = e == hipSuccess ? enqueue_scan(ctx, ix, r->last_plans, q, 1, sp, r->k, lp, pb, nullptr) : MRL_ERR_HIP;
  if (e == hipSuccess) e = hipMemcpyAsync(&st, pb.status, sizeof(st), hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  dev_free(sc);
  dev_free(rw);
  dev_free(small);
  if (rc) return rc;
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("dense rerun: ") + hipGetErrorString(e));
  if (st & 2u) return fail(MRL_ERR_HIP, "dense rerun overflowed");
  return (st & 1u) ? fail(MRL_ERR_NAN, "NaN score among scan survivors (Shortlist::into_sorted would panic)")
                   : MRL_OK;
}

// The final pass alone, at the safe floor, for query q of the last scan (its
// final floor left fewer than K candidates); rewrites the query's result row.
// *st receives the new status.  Caller holds the lock.
static int safe_rerun(mrl_ctx* ctx, mrl_results* r, uint32_t q, uint32_t* st) {
  mrl_index* ix = const_cast<mrl_index*>(r->last_index);
  LevelPlan* lp;
  int rc = get_levels(ix, r->k, &lp);
  if (rc) return rc;
  PassBuffers pb = results_buffers(r);
  const size_t cand = (size_t)q * kSegs * r->seg_cap;
  pb.cand_score += cand;
  pb.cand_row += cand;
  pb.cand_lower = nullptr;  // one query: the exact kernels
  pb.seg_count += (size_t)q * kMaxSegs;
  pb.err += q;
  pb.tau += q;
  pb.tau_hi += q;
  pb.hist += (size_t)q * kHistBins;
  pb.status += q;
  pb.out_ids += (size_t)q * r->k;
  pb.out_scores += (size_t)q * r->k;
  pb.out_counts += q;
  const ScanParams sp = make_params(&r->last_cfg, &r->last_time);
  if ((rc = enqueue_scan(ctx, ix, r->last_plans, q, 1, sp, r->k, *lp, pb, nullptr, true))) return rc;
  HIP_TRY(hipMemcpyAsync(st, pb.status, sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MRL_OK;
}

// Acts on one query's scan status: bit 2 (final floor too high) re-runs the
// final pass at the safe floor; bit 1 (a segment overflowed) or bit 3 (short
// of K at a floor no tighter than the safe one: bounds that are not
// admissible) re-runs densely, with no floor; bit 0 (NaN) sets *nan.  *rerun
// is set if anything ran.  Caller holds the lock.
static int rerun_query(mrl_ctx* ctx, mrl_results* r, uint32_t q, uint32_t status, bool* nan, bool* rerun) {
  int rc;
  if (status & 4u) {
    if ((rc = safe_rerun(ctx, r, q, &status))) return rc;
    if (q < r->floor_kind.size()) r->floor_kind[q] = 2;
    *rerun = true;
  }
  if (status & 1u) *nan = true;
  if (status & 10u) {
    if (q < r->floor_kind.size()) r->floor_kind[q] = 0;
    rc = dense_rerun(ctx, r, q);
    if (rc == MRL_ERR_NAN) *nan = true;
    else if (rc) return rc;
    *rerun = true;
  }
  return MRL_OK;
}

// Waits for the last scan on res; queries whose candidate lists overflowed are
// re-run densely.  MRL_ERR_NAN if any query saw a NaN survivor.  Caller holds
// the context lock.
static int resolve_pending(mrl_ctx* ctx, mrl_results* res) {
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  const uint32_t n_q = res->last_plans ? res->last_plans->n_q : 0;
  bool nan = false;
  if (res->pending && n_q && res->last_index && res->last_index->n_blocks) {
    std::vector<uint32_t> status(n_q);
    HIP_TRY(hipMemcpy(status.data(), res->d_status, n_q * sizeof(uint32_t), hipMemcpyDeviceToHost));
    bool rerun = false;
    for (uint32_t q = 0; q < n_q; ++q) {
      int rc = rerun_query(ctx, res, q, status[q], &nan, &rerun);
      if (rc) return rc;
    }
  }
  res->pending = false;
  if (nan) return fail(MRL_ERR_NAN, "NaN score among scan survivors (Shortlist::into_sorted would panic)");
  return MRL_OK;
}

// One read-back of the results block into pinned memory: the head (status,
// counts, stats) and the ids / scores rows of the first n_q queries.  Caller
// holds the lock.
static int read_back(mrl_ctx* ctx, mrl_results* res, uint32_t n_q, uint8_t** out) {
  const size_t nq = std::max<uint32_t>(res->n_q, 1), K = res->k;
  const size_t head = results_head_bytes((uint32_t)nq);
  uint8_t* h = host_stage(ctx, res->out_bytes);
  if (!h) return fail(MRL_ERR_OUT_OF_MEMORY, "pinned staging buffer");
  if (n_q == nq) {
    HIP_TRY(hipMemcpyAsync(h, res->d_out, res->out_bytes, hipMemcpyDeviceToHost, ctx->stream));
  } else {
    HIP_TRY(hipMemcpyAsync(h, res->d_out, head + n_q * K * 8, hipMemcpyDeviceToHost, ctx->stream));
    if (n_q)
      HIP_TRY(hipMemcpyAsync(h + head + nq * K * 8, res->d_out + head + nq * K * 8, n_q * K * 4,
                             hipMemcpyDeviceToHost, ctx->stream));
  }
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  *out = h;
  return MRL_OK;
}

// Pending-scan statuses read back: dense re-run of overflowed queries; true
// in *rerun if any ran.  Caller holds the lock.
static int handle_scan_status(mrl_ctx* ctx, mrl_results* res, const uint32_t* status, uint32_t n_q, bool* rerun) {
  *rerun = false;
  bool nan = false;
  if (res->pending && n_q && res->last_index && res->last_index->n_blocks) {
    for (uint32_t q = 0; q < n_q; ++q) {
      int rc = rerun_query(ctx, res, q, status[q], &nan, rerun);
      if (rc) return rc;
    }
  }
  res->pending = false;
  if (nan) return fail(MRL_ERR_NAN, "NaN score among scan survivors (Shortlist::into_sorted would panic)");
  return MRL_OK;
}

extern "C" int mrl_results_fetch(mrl_ctx* ctx, mrl_results* res, uint64_t* out_ids, float* out_scores,
                                 uint32_t* out_counts, mrl_scan_stats* stats) {
  if (!ctx || !res) return fail(MRL_ERR_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  const uint32_t n_q = res->last_plans ? res->last_plans->n_q : 0;
  uint8_t* h = nullptr;
  int rc = read_back(ctx, res, n_q, &h);
  if (rc) return rc;
  bool rerun = false;
  if ((rc = handle_scan_status(ctx, res, reinterpret_cast<const uint32_t*>(h), n_q, &rerun))) return rc;
  if (rerun && (rc = read_back(ctx, res, n_q, &h))) return rc;
  const size_t nq = std::max<uint32_t>(res->n_q, 1), K = res->k;
  const size_t head = results_head_bytes((uint32_t)nq);
  if (out_ids && n_q) memcpy(out_ids, h + head, n_q * K * 8);
  if (out_scores && n_q) memcpy(out_scores, h + head + nq * K * 8, n_q * K * 4);
  if (out_counts && n_q) memcpy(out_counts, h + nq * 4, (size_t)n_q * 4);
  unsigned long long st[kStatCount] = {0};
  for (int c = 0; c < kStatCopies; ++c) {
    unsigned long long part[kStatCount];
    memcpy(part, h + nq * 8 + (size_t)c * sizeof(part), sizeof(part));
    for (int i = 0; i < kStatCount; ++i) st[i] += part[i];
  }
  if (stats) {  // counters accumulated since the previous fetch
    stats->blocks = st[kStatBlocks] - res->stats_seen[kStatBlocks];
    stats->active_vecs = st[kStatActive] - res->stats_seen[kStatActive];
    stats->after_prefix = st[kStatPrefix] - res->stats_seen[kStatPrefix];
    stats->after_s1 = st[kStatS1] - res->stats_seen[kStatS1];
    stats->after_s4_budget = st[kStatS4Budget] - res->stats_seen[kStatS4Budget];
    stats->pushed = st[kStatPushed] - res->stats_seen[kStatPushed];
    stats->reruns_safe = st[kStatRerunSafe] - res->stats_seen[kStatRerunSafe];
    stats->reruns_dense = st[kStatRerunDense] - res->stats_seen[kStatRerunDense];
  }
  memcpy(res->stats_seen, st, sizeof(st));
  return MRL_OK;
}

extern "C" int mrl_results_floors(mrl_ctx* ctx, mrl_results* res, float* out_floors) {
  if (!ctx || !res || !out_floors) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (res->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "results belong to another context");
  std::lock_guard<std::mutex> g(ctx->mu);
  if (res->pending) return fail(MRL_ERR_INVALID_ARG, "the last scan on these results has not been fetched");
  HIP_TRY(hipSetDevice(ctx->device));
  const size_t n = res->floor_kind.size();
  if (!n) return MRL_OK;
  std::vector<float> fin(n), safe(n);
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  HIP_TRY(hipMemcpy(fin.data(), res->d_tau_hi, n * sizeof(float), hipMemcpyDeviceToHost));
  HIP_TRY(hipMemcpy(safe.data(), res->d_tau, n * sizeof(float), hipMemcpyDeviceToHost));
  for (size_t q = 0; q < n; ++q) {
    const uint8_t k = res->floor_kind[q];
    out_floors[q] = k == 1 ? fin[q] : (k == 2 ? safe[q] : -INFINITY);
  }
  return MRL_OK;
}

extern "C" int mrl_scan(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans, const mrl_scan_config* cfg,
                        const mrl_time_range* time, uint64_t* out_ids, float* out_scores, uint32_t* out_counts,
                        mrl_scan_stats* stats) {
  if (!ctx || !index || !plans) return fail(MRL_ERR_INVALID_ARG, "null argument");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  // Result buffers of the same K and at least n_q rows are reused from the
  // previous call (every selection leaves the pass state zeroed again).
  mrl_results* res = nullptr;
  {
    std::lock_guard<std::mutex> g(ctx->mu);
    if (ctx->spare && ctx->spare->k == K && ctx->spare->n_q >= plans->n_q) {
      res = ctx->spare;
      ctx->spare = nullptr;
    }
  }
  if (!res && (rc = results_create(ctx, plans->n_q, K, &res))) return rc;
  rc = mrl_scan_async(ctx, index, plans, cfg, time, res);
  if (!rc) rc = mrl_results_fetch(ctx, res, out_ids, out_scores, out_counts, stats);
  if (rc) {  // a failed scan may leave pass state behind: do not keep these buffers
    std::string msg = g_err;
    results_destroy(res);
    g_err = msg;
    return rc;
  }
  res->last_plans = nullptr;  // the caller may free the plans and index now
  res->last_index = nullptr;
  mrl_results* old = nullptr;
  {
    std::lock_guard<std::mutex> g(ctx->mu);
    old = ctx->spare;
    ctx->spare = res;
  }
  if (old) results_destroy(old);
  return rc;
}

// ---------------------------------------------------------------------------
// allocation-free scan
// ---------------------------------------------------------------------------
// Buffers of one mrl_scan_noalloc call inside the device's scratch array.
// The candidate room per query shrinks with the batch: 16 segments of 4096
// entries up to 16 queries (the room mrl_results gives), 2048 up to 32,
// 1024 up to MRL_NOALLOC_MAX_QUERIES.
struct NaLayout {
  uint32_t seg_cap;
  float *cand_score, *cand_lower;
  uint32_t *cand_row, *seg_count, *hist, *err;
  float *tau, *tau_hi;
  uint8_t* mma;
  uint32_t* zero_begin;  // seg_count .. err: the words a call clears first
  uint64_t zero_words;
  size_t bytes;          // end of the last buffer
};
static NaLayout na_layout(uint32_t n_q, uint8_t* base) {
  NaLayout L{};
  L.seg_cap = n_q <= 16 ? 4096u : (n_q <= 32 ? 2048u : 1024u);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base + off;
    off += (bytes + 255) & ~(size_t)255;
    return p;
  };
  const size_t cands = (size_t)n_q * kSegs * L.seg_cap;
  L.cand_score = reinterpret_cast<float*>(take(cands * 4));
  L.cand_lower = reinterpret_cast<float*>(take(cands * 4));
  L.cand_row = reinterpret_cast<uint32_t*>(take(cands * 4));
  // seg_count, hist and err are contiguous (their sizes are multiples of 256 B
  // except err's, which comes last): one fill clears them
  L.seg_count = reinterpret_cast<uint32_t*>(take((size_t)n_q * kMaxSegs * 4));
  L.hist = reinterpret_cast<uint32_t*>(take((size_t)n_q * kHistBins * 4));
  L.err = reinterpret_cast<uint32_t*>(take((size_t)n_q * 4));
  L.zero_begin = L.seg_count;
  L.zero_words = (uint64_t)n_q * (kMaxSegs + kHistBins + 1);
  L.tau = reinterpret_cast<float*>(take((size_t)n_q * 4));
  L.tau_hi = reinterpret_cast<float*>(take((size_t)n_q * 4));
  L.mma = take(mma_bytes(n_q));
  L.bytes = off;
  return L;
}

// Safe-floor re-run decided on the device: the final pass at the safe floor
// for every query whose selection flagged a shortfall (bit 2 of its status),
// then its selection; both launches exit at once for every other query.
// Caller holds the lock.
static int enqueue_gated_rerun(mrl_ctx* ctx, mrl_index* ix, const mrl_plans* plans, uint32_t n_q,
                               const ScanParams& sp, uint32_t K, const PassBuffers& pb) {
  if (int rc = flush_plans(ctx, plans)) return rc;
  ScanArgs a{};
  a.idx = ix->d_blocks;
  a.recs = ix->recs();
  a.n_blocks = ix->n_blocks;
  a.n_pos = (uint32_t)ix->n_blocks;
  a.shift = 0;
  a.prev_shift = -1;
  a.plans = plans->d_plans;
  a.luts = plans->d_luts;
  a.n_q = n_q;
  a.flag_tabs = ctx->d_flag_tabs;
  a.sp = sp;
  a.tau = pb.tau;  // the safe floors
  a.floor_out = pb.tau_hi;
  a.safe_out = pb.tau;
  a.cand_score = pb.cand_score;
  a.cand_row = pb.cand_row;
  a.seg_count = pb.seg_count;
  a.nseg = pb.nseg;
  a.seg_cap = pb.seg_cap;
  a.err = pb.err;
  a.gate = pb.status;
  if (sp.strata != MRL_STRATA_L0_ONLY) {
    a.excl = 1;
    const uint32_t g = scan_grid(a, false);
    if (g >= 1 && g <= (uint32_t)kMaxSegs) {
      a.nseg = g;
      a.seg_cap = std::min<uint32_t>(pb.nseg * pb.seg_cap / g, kExclCap);
    } else {
      a.excl = 0;
    }
  }
  {
    ProfScope ps(ctx, MRL_KERNEL_SCAN, -1, (uint32_t)ix->n_blocks, n_q);
    HIP_TRY(launch_scan(a, false, ctx->stream, ps.ev()));
    ps.commit(true);
  }
  SelectArgs sa{};
  sa.luts = plans->d_luts;
  sa.cand_score = pb.cand_score;
  sa.cand_row = pb.cand_row;
  sa.seg_count = pb.seg_count;
  sa.nseg = a.nseg;
  sa.seg_cap = a.seg_cap;
  sa.err = pb.err;
  sa.k = K;
  sa.status = pb.status;
  sa.out_ids = pb.out_ids;
  sa.out_scores = pb.out_scores;
  sa.out_counts = pb.out_counts;
  sa.tau_final = pb.tau_hi;
  sa.tau_safe = pb.tau;
  sa.tau_used = pb.tau;
  sa.floor_record = pb.tau_hi;  // a re-run query's list now stands at the safe floor
  sa.gate = pb.status;
  ProfScope ps(ctx, MRL_KERNEL_SELECT, -1, 0, n_q);
  HIP_TRY(launch_select(sa, n_q, ctx->stream, ps.ev()));
  ps.commit(true);
  return MRL_OK;
}

extern "C" int mrl_scan_noalloc(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans,
                                const mrl_scan_config* cfg, const mrl_time_range* time, uint64_t* d_out_ids,
                                float* d_out_scores, uint32_t* d_out_counts, uint32_t* d_out_status) {
  if (!ctx || !index || !plans) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (plans->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  const uint32_t n_q = plans->n_q;
  if (n_q > MRL_NOALLOC_MAX_QUERIES)
    return fail(MRL_ERR_INVALID_ARG, "mrl_scan_noalloc takes at most " + std::to_string(MRL_NOALLOC_MAX_QUERIES) +
                                         " queries per call (its scratch has a fixed size)");
  if (n_q && (!d_out_ids || !d_out_scores || !d_out_counts || !d_out_status))
    return fail(MRL_ERR_INVALID_ARG, "null output");
  if (!n_q) return MRL_OK;
  if (!ctx->scratch) return fail(MRL_ERR_HIP, "no scratch address for this device");
  const NaLayout L = na_layout(n_q, ctx->scratch);
  if (L.bytes > kNaScratchBytes) return fail(MRL_ERR_INVALID_ARG, "batch exceeds the scratch array");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  hipStream_t s = ctx->stream;
  mrl_index* ix = const_cast<mrl_index*>(index);
  // The array keeps the previous call's contents: the pass state starts from zero.
  HIP_TRY(launch_fill_u32(L.zero_begin, L.zero_words, 0u, s));
  if (ix->n_blocks == 0) {
    HIP_TRY(launch_fill_u32(d_out_counts, n_q, 0u, s));
    HIP_TRY(launch_fill_u32(d_out_status, n_q, 0u, s));
    return MRL_OK;
  }
  PassBuffers pb;
  pb.cand_score = L.cand_score;
  pb.cand_row = L.cand_row;
  pb.cand_lower = L.cand_lower;
  pb.mma_ops = reinterpret_cast<uint4*>(L.mma);
  pb.mma_consts = reinterpret_cast<float*>(L.mma + (size_t)n_q * 2 * kMmaSteps * 16);
  pb.mma_work = reinterpret_cast<uint32_t*>(L.mma + (size_t)n_q * (2 * kMmaSteps * 16 + kMcCount * 4));
  pb.seg_count = L.seg_count;
  pb.nseg = kSegs;
  pb.seg_cap = L.seg_cap;
  pb.err = L.err;
  pb.tau = L.tau;
  pb.tau_hi = L.tau_hi;
  pb.hist = L.hist;
  pb.status = d_out_status;
  pb.out_ids = d_out_ids;
  pb.out_scores = d_out_scores;
  pb.out_counts = d_out_counts;
  pb.block_lists = false;
  const ScanParams sp = make_params(cfg, time);
  LevelPlan* lp;
  if ((rc = get_levels(ix, K, &lp))) return rc;
  const bool sampled =
      mma_ok(plans, n_q, sp, pb) ? !mma_stages(ix->n_blocks, n_q, K, 0u).empty() : lp->passes.size() > 1;
  if ((rc = enqueue_scan(ctx, ix, plans, 0, n_q, sp, K, *lp, pb, nullptr))) return rc;
  // without a sampling pass no query can be flagged
  if (sampled && (rc = enqueue_gated_rerun(ctx, ix, plans, n_q, sp, K, pb))) return rc;
  return MRL_OK;
}

extern "C" int mrl_scan_fixed_tau(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans,
                                  const mrl_scan_config* cfg, const mrl_time_range* time, const float* tau,
                                  uint64_t* out_masks, float* out_prefix_ip, float* out_scores) {
  if (!ctx || !index || !plans || !tau) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (plans->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  const uint64_t nq = plans->n_q, B = index->n_blocks;
  if (!nq || !B) return MRL_OK;
  if (!out_masks || !out_prefix_ip || !out_scores) return fail(MRL_ERR_INVALID_ARG, "null output");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (int rc = flush_plans(ctx, plans)) return rc;
  float* d_tau = nullptr;
  uint64_t* d_masks = nullptr;
  float *d_prefix = nullptr, *d_score = nullptr;
  auto cleanup = [&]() {
    dev_free(d_tau);
    dev_free(d_masks);
    dev_free(d_prefix);
    dev_free(d_score);
  };
  if (hipMalloc(&d_tau, nq * sizeof(float)) != hipSuccess || hipMalloc(&d_masks, nq * B * 5 * 8) != hipSuccess ||
      hipMalloc(&d_prefix, nq * B * 64 * 4) != hipSuccess || hipMalloc(&d_score, nq * B * 64 * 4) != hipSuccess) {
    cleanup();
    return fail(MRL_ERR_OUT_OF_MEMORY, "diagnostic buffers");
  }
  ScanArgs a{};
  a.idx = index->d_blocks;
  a.n_blocks = B;
  a.n_pos = (uint32_t)B;
  a.shift = 0;
  a.prev_shift = -1;
  a.plans = plans->d_plans;
  a.luts = plans->d_luts;
  a.n_q = (uint32_t)nq;
  a.flag_tabs = ctx->d_flag_tabs;
  a.sp = make_params(cfg, time);
  a.tau = d_tau;
  a.nseg = 1;
  a.d_masks = d_masks;
  a.d_prefix = d_prefix;
  a.d_score = d_score;
  hipError_t e = hipMemcpyAsync(d_tau, tau, nq * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = launch_scan(a, true, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_masks, d_masks, nq * B * 5 * 8, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_prefix_ip, d_prefix, nq * B * 64 * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_scores, d_score, nq * B * 64 * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  cleanup();
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("fixed-tau scan: ") + hipGetErrorString(e));
  return MRL_OK;
}

// Every (query, slot) pair's MFMA bounds: k_mma_prep, then the single-pass
// k_scan_mma (every active pair appended with its upper and lower bound) into
// one segment per query with room for every slot; the host scatters the
// appended pairs to out[q][row].  Pairs not appended (inactive slots, queries
// with unusable operands) read NaN.
extern "C" int mrl_index_block_bounds(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans,
                                      const mrl_scan_config* cfg, float* out_bounds) {
  if (!ctx || !index || !plans) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (plans->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  ScanParams sp = make_params(cfg, nullptr);
  if (plans->mid_codec != MRL_MID_RABITQ || sp.strata == MRL_STRATA_L0_ONLY)
    return fail(MRL_ERR_INVALID_ARG, "block bounds need the RaBitQ mid-band and an S1 stage");
  const uint64_t nq = plans->n_q, B = index->n_blocks;
  if (!nq || !B) return MRL_OK;
  if (!out_bounds) return fail(MRL_ERR_INVALID_ARG, "null output");
  const float nan = std::numeric_limits<float>::quiet_NaN();
  if (!index->n_cl) {
    std::fill(out_bounds, out_bounds + nq * B, nan);
    return MRL_OK;
  }
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (int rc = flush_plans(ctx, plans)) return rc;
  float *d_table = nullptr, *d_qn = nullptr, *d_out = nullptr;
  auto cleanup = [&]() {
    dev_free(d_table);
    dev_free(d_qn);
    dev_free(d_out);
  };
  if (hipMalloc(&d_table, (size_t)index->n_cl * nq * 4) != hipSuccess || hipMalloc(&d_qn, nq * 16) != hipSuccess ||
      hipMalloc(&d_out, nq * B * 4) != hipSuccess) {
    cleanup();
    return fail(MRL_ERR_OUT_OF_MEMORY, "bounds buffers");
  }
  sp.exhaustive = 0;
  BoundScanArgs b{};
  b.center = index->d_center;
  b.cnorm = index->d_cnorm;
  b.n_cl = index->n_cl;
  b.bcl = index->d_bcl;
  b.brad = index->d_brad;
  b.n_blocks = B;
  b.plans = plans->d_plans;
  b.luts = plans->d_luts;
  b.n_q = (uint32_t)nq;
  b.sp = sp;
  b.eden = plans->prefix_codec == MRL_PREFIX_EDEN_PROD;
  b.table = d_table;
  b.qn = d_qn;
  b.chunk = 64;
  b.n_pos = (uint32_t)B;
  b.shift = 0;
  b.out_bound = d_out;
  hipError_t e = launch_bound_table(b, ctx->stream);
  if (e == hipSuccess) e = launch_block_select(b, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out_bounds, d_out, nq * B * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  cleanup();
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("block bounds: ") + hipGetErrorString(e));
  return MRL_OK;
}

extern "C" int mrl_scan_mma_bounds(mrl_ctx* ctx, const mrl_index* index, const mrl_plans* plans,
                                   const mrl_scan_config* cfg, const mrl_time_range* time, float* out_upper,
                                   float* out_lower) {
  if (!ctx || !index || !plans) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (!index_usable(index, ctx)) return fail(MRL_ERR_INVALID_ARG, "index lives on another device");
  if (plans->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  uint32_t K;
  int rc = check_cfg(cfg, &K);
  if (rc) return rc;
  const ScanParams sp = make_params(cfg, time);
  if (plans->mid_codec != MRL_MID_RABITQ || sp.strata == MRL_STRATA_L0_ONLY)
    return fail(MRL_ERR_INVALID_ARG, "MFMA bounds need the RaBitQ mid-band and an S1 stage");
  const uint64_t nq = plans->n_q, B = index->n_blocks, N = B * 64;
  if (!nq || !B) return MRL_OK;
  if (!out_upper || !out_lower) return fail(MRL_ERR_INVALID_ARG, "null output");
  if (N > (1ull << 24)) return fail(MRL_ERR_INVALID_ARG, "MFMA bounds dump is limited to 2^24 slots");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (int rc = flush_plans(ctx, plans)) return rc;
  float *d_u = nullptr, *d_l = nullptr, *d_consts = nullptr, *d_tau = nullptr;
  uint32_t *d_row = nullptr, *d_cnt = nullptr, *d_work = nullptr;
  uint4* d_ops = nullptr;
  auto cleanup = [&]() {
    dev_free(d_tau);
    dev_free(d_u);
    dev_free(d_l);
    dev_free(d_row);
    dev_free(d_cnt);
    dev_free(d_ops);
    dev_free(d_consts);
    dev_free(d_work);
  };
  if (hipMalloc(&d_u, nq * N * 4) != hipSuccess || hipMalloc(&d_l, nq * N * 4) != hipSuccess ||
      hipMalloc(&d_row, nq * N * 4) != hipSuccess || hipMalloc(&d_cnt, nq * 4) != hipSuccess ||
      hipMalloc(&d_ops, nq * 2 * kMmaSteps * 16) != hipSuccess ||
      hipMalloc(&d_consts, nq * kMcCount * 4) != hipSuccess || hipMalloc(&d_work, 16) != hipSuccess) {
    cleanup();
    return fail(MRL_ERR_OUT_OF_MEMORY, "bounds buffers");
  }
  MmaPrepArgs pa{};
  pa.plans = plans->d_plans;
  pa.luts = plans->d_luts;
  pa.n_q = (uint32_t)nq;
  pa.sp = sp;
  pa.ops = d_ops;
  pa.consts = d_consts;
  pa.work = d_work;
  ScanArgs a{};
  a.idx = index->d_blocks;
  a.recs = index->recs();
  a.n_blocks = B;
  a.n_pos = (uint32_t)B;
  a.shift = 0;
  a.prev_shift = -1;
  a.plans = plans->d_plans;
  a.luts = plans->d_luts;
  a.n_q = (uint32_t)nq;
  a.flag_tabs = ctx->d_flag_tabs;
  a.sp = sp;
  a.cand_score = d_u;
  a.cand_lower = d_l;
  a.cand_row = d_row;
  a.seg_count = d_cnt;
  a.nseg = 1;
  a.seg_cap = (uint32_t)N;
  a.mma_ops = d_ops;
  a.mma_consts = d_consts;
  std::vector<uint32_t> cnt(nq);
  std::vector<float> u(nq * N), l(nq * N);
  std::vector<uint32_t> row(nq * N);
  hipError_t e = hipMemsetAsync(d_cnt, 0, nq * 4, ctx->stream);
  if (e == hipSuccess) e = launch_mma_prep(pa, ctx->stream);
  if (e == hipSuccess) e = launch_scan_mma(a, 2, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(cnt.data(), d_cnt, nq * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(u.data(), d_u, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(l.data(), d_l, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(row.data(), d_row, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  // ALWAYS: the S4-bounded final pass, at a floor one below every pair's
  // lower bound so that every active pair passes it and is made exact.  At
  // most 4 queries per launch: a 32-vector tile then appends at most 128
  // pairs, which the wave's staging region holds (no pair is written out
  // straight with the bound still in it).
  const bool wide = ctx->s4_policy == MRL_S4_BOUND_ALWAYS &&
                    (sp.strata != MRL_STRATA_FULL64B || sp.w_s4 <= kMmaWideMaxWs4);
  if (wide && e == hipSuccess) {
    std::vector<float> tau(nq);
    for (uint64_t q = 0; q < nq; ++q) {
      float mn = std::numeric_limits<float>::infinity();
      for (uint64_t i = 0; i < std::min<uint64_t>(cnt[q], N); ++i)
        if (std::isfinite(l[q * N + i])) mn = std::min(mn, l[q * N + i]);
      tau[q] = std::isfinite(mn) ? mn - 1.0f : -1.0f;
    }
    e = hipMalloc(&d_tau, nq * 4);
    if (e == hipSuccess) e = hipMemcpyAsync(d_tau, tau.data(), nq * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(d_cnt, 0, nq * 4, ctx->stream);
    for (uint64_t g0 = 0; g0 < nq && e == hipSuccess; g0 += 4) {
      ScanArgs w = a;
      w.plans = plans->d_plans + g0;
      w.luts = plans->d_luts + g0 * kQData;
      w.n_q = (uint32_t)std::min<uint64_t>(4, nq - g0);
      w.mma_ops = d_ops + g0 * 2 * kMmaSteps;
      w.mma_consts = d_consts + g0 * kMcCount;
      w.tau = d_tau + g0;
      w.cand_score = d_u + g0 * N;
      w.cand_lower = d_l + g0 * N;
      w.cand_row = d_row + g0 * N;
      w.seg_count = d_cnt + g0;
      w.mma_wide = 1u;
      w.wide_lim = 1u << 20;  // no wave returns to the full tiles
      e = launch_scan_mma(w, 1, ctx->stream);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(cnt.data(), d_cnt, nq * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(u.data(), d_u, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(l.data(), d_l, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(row.data(), d_row, nq * N * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  }
  cleanup();
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("MFMA bounds: ") + hipGetErrorString(e));
  const float nan = std::numeric_limits<float>::quiet_NaN();
  std::fill(out_upper, out_upper + nq * N, nan);
  std::fill(out_lower, out_lower + nq * N, nan);
  for (uint64_t q = 0; q < nq; ++q) {
    if (cnt[q] > N) return fail(MRL_ERR_HIP, "MFMA bounds: more appends than slots");
    for (uint64_t i = 0; i < cnt[q]; ++i) {
      const uint32_t r = row[q * N + i];
      if (r >= N) return fail(MRL_ERR_HIP, "MFMA bounds: row out of range");
      out_upper[q * N + r] = u[q * N + i];
      out_lower[q * N + r] = l[q * N + i];
    }
  }
  return MRL_OK;
}

// ---------------------------------------------------------------------------
// post-scan rerank
// ---------------------------------------------------------------------------
static size_t store_row_bytes(int precision, uint32_t dims) {
  return precision == MRL_RERANK_FP32 ? (size_t)dims * 4 : precision == MRL_RERANK_FP16 ? 768 * 2 : 768;
}

// Builds a store; caller holds the context lock and has set the device.
static int store_create_locked(mrl_ctx* ctx, const float* rows, int rows_on_device, uint64_t n_rows, uint32_t dims,
                               int precision, mrl_rerank_store** out) {
  *out = nullptr;
  std::unique_ptr<mrl_rerank_store> st(new mrl_rerank_store());
  st->ctx = ctx;
  st->precision = precision;
  st->n_rows = n_rows;
  st->dims = dims;
  const size_t rb = store_row_bytes(precision, dims);
  float* staging = nullptr;
  auto cleanup = [&]() {
    dev_free(st->d_data);
    dev_free(st->d_scales);
    dev_free(staging);
  };
  if (hipMalloc(&st->d_data, std::max<size_t>(n_rows * rb, 16)) != hipSuccess ||
      (precision == MRL_RERANK_INT8 &&
       hipMalloc(&st->d_scales, std::max<size_t>(n_rows * 2, 16)) != hipSuccess)) {
    cleanup();
    return fail(MRL_ERR_OUT_OF_MEMORY, "rerank store");
  }
  hipError_t e = hipSuccess;
  if (dims != 768) {  // fp32 rows kept row-major
    if (n_rows)
      e = hipMemcpyAsync(st->d_data, rows, n_rows * rb,
                         rows_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream);
  } else if (rows_on_device) {
    e = launch_rerank_store(rows, n_rows, precision, st->d_data, st->d_scales, ctx->stream);
  } else if (n_rows) {
    // host rows go through a bounded device staging buffer
    const uint64_t chunk = std::min<uint64_t>(n_rows, 1ull << 16);
    if (hipMalloc(&staging, chunk * 768 * sizeof(float)) != hipSuccess) {
      cleanup();
      return fail(MRL_ERR_OUT_OF_MEMORY, "rerank store staging");
    }
    for (uint64_t r = 0; r < n_rows && e == hipSuccess; r += chunk) {
      const uint64_t nr = std::min(chunk, n_rows - r);
      e = hipMemcpyAsync(staging, rows + r * 768, nr * 768 * sizeof(float), hipMemcpyHostToDevice, ctx->stream);
      if (e == hipSuccess)
        e = launch_rerank_store(staging, nr, precision, static_cast<uint8_t*>(st->d_data) + r * rb,
                                st->d_scales ? st->d_scales + r : nullptr, ctx->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);  // staging is reused
    }
  }
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    cleanup();
    return fail(MRL_ERR_HIP, std::string("rerank store: ") + hipGetErrorString(e));
  }
  dev_free(staging);
  *out = st.release();
  return MRL_OK;
}

static void store_free(mrl_rerank_store* st) {
  if (!st) return;
  dev_free(st->d_data);
  dev_free(st->d_scales);
  delete st;
}

extern "C" int mrl_rerank_store_create(mrl_ctx* ctx, const float* rows, int rows_on_device, uint64_t n_rows,
                                       uint32_t dims, int precision, mrl_rerank_store** out) {
  if (!ctx || !out || (n_rows && !rows)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  if (precision != MRL_RERANK_FP32 && precision != MRL_RERANK_FP16 && precision != MRL_RERANK_INT8)
    return fail(MRL_ERR_INVALID_ARG, "unknown rerank precision");
  if (dims == 0 || dims > MRL_MAX_DIMS) return fail(MRL_ERR_INVALID_ARG, "dims must be in [1, MRL_MAX_DIMS]");
  if (precision != MRL_RERANK_FP32 && dims != 768)
    return fail(MRL_ERR_INVALID_ARG, "fp16 / int8 rerank rows need 768 dims");  // lowprec.rs:50,73
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  const int rc = store_create_locked(ctx, rows, rows_on_device, n_rows, dims, precision, out);
  if (rc == MRL_OK) ctx_retain(ctx);
  return rc;
}

extern "C" void mrl_rerank_store_destroy(mrl_rerank_store* store) {
  if (!store) return;
  mrl_ctx* ctx = store->ctx;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  store_free(store);
  ctx_release(ctx);
}

extern "C" int mrl_rerank_store_download(mrl_ctx* ctx, const mrl_rerank_store* store, void* out_rows,
                                         uint16_t* out_scales) {
  if (!ctx || !store || (store->n_rows && !out_rows)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (store->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "store belongs to another context");
  if (store->precision == MRL_RERANK_INT8 && store->n_rows && !out_scales)
    return fail(MRL_ERR_INVALID_ARG, "int8 store needs out_scales");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  const size_t rb = store_row_bytes(store->precision, store->dims);
  if (store->dims != 768) {
    HIP_TRY(hipMemcpy(out_rows, store->d_data, store->n_rows * rb, hipMemcpyDeviceToHost));
    return MRL_OK;
  }
  // accumulator-major (element 8t + j at 96j + t) back to row-major
  const size_t es = rb / 768;
  const uint64_t chunk = 4096;
  std::vector<uint8_t> buf(chunk * rb);
  uint8_t* dst = static_cast<uint8_t*>(out_rows);
  for (uint64_t r = 0; r < store->n_rows; r += chunk) {
    const uint64_t nr = std::min(chunk, store->n_rows - r);
    HIP_TRY(hipMemcpy(buf.data(), static_cast<const uint8_t*>(store->d_data) + r * rb, nr * rb,
                      hipMemcpyDeviceToHost));
    for (uint64_t k = 0; k < nr; ++k)
      for (uint32_t i = 0; i < 768; ++i)
        memcpy(dst + (r + k) * rb + i * es, buf.data() + k * rb + ((i & 7u) * 96u + (i >> 3)) * es, es);
  }
  if (store->precision == MRL_RERANK_INT8)
    HIP_TRY(hipMemcpy(out_scales, store->d_scales, store->n_rows * 2, hipMemcpyDeviceToHost));
  return MRL_OK;
}

// Rerank buffers for n_q lists of `stride` entries, carved from one
// allocation.  The outputs come first so one copy reads them back: status
// u32[n_q], counts u32[n_q], out_rows u64[n], out_scores f32[n]; then the
// scratch row u64[n] and score f32[n] (n = n_q * stride).
struct RerankBuffers {
  float* score;
  uint64_t* row;
  uint64_t* out_rows;
  float* out_scores;
  uint32_t* status;
  uint32_t* counts;
};
static size_t rerank_out_bytes(uint32_t n_q, uint32_t stride) {
  return (size_t)n_q * 8 + (size_t)n_q * stride * 12;
}
static size_t rerank_bytes(uint32_t n_q, uint32_t stride) {
  return ((rerank_out_bytes(n_q, stride) + 15) & ~(size_t)15) + (size_t)n_q * stride * 12 + 64;
}
static RerankBuffers rerank_carve(void* base, uint32_t n_q, uint32_t stride) {
  const size_t n = (size_t)n_q * stride;
  uint8_t* p = static_cast<uint8_t*>(base);
  RerankBuffers b;
  b.status = reinterpret_cast<uint32_t*>(p);
  b.counts = b.status + n_q;
  b.out_rows = reinterpret_cast<uint64_t*>(p + (size_t)n_q * 8);
  b.out_scores = reinterpret_cast<float*>(p + (size_t)n_q * 8 + n * 8);
  uint8_t* scratch = p + ((rerank_out_bytes(n_q, stride) + 15) & ~(size_t)15);
  b.row = reinterpret_cast<uint64_t*>(scratch);
  b.score = reinterpret_cast<float*>(scratch + n * 8);
  return b;
}

static int status_error(const uint32_t* st, uint32_t n) {
  uint32_t all = 0;
  for (uint32_t i = 0; i < n; ++i) all |= st[i] & 0xffu;
  if (all & 2u) return fail(MRL_ERR_INVALID_ARG, "candidate row out of range of the rerank store");
  if (all & 1u) return fail(MRL_ERR_NAN, "NaN rerank score (partial_cmp().unwrap() would panic)");
  return MRL_OK;
}

// Enqueue score + sort.  Caller holds the lock.
static int enqueue_rerank(mrl_ctx* ctx, const mrl_rerank_store* st, const float* d_queries, uint32_t n_q,
                          const uint64_t* d_cand, int cand_ids, const uint32_t* d_counts, uint32_t stride,
                          const RerankBuffers& b, const uint32_t* d_scan_status = nullptr) {
  RerankArgs a{};
  a.data = st->d_data;
  a.scales = st->d_scales;
  a.n_rows = st->n_rows;
  a.dims = st->dims;
  a.precision = st->precision;
  a.queries = d_queries;
  a.cand = d_cand;
  a.counts = d_counts;
  a.stride = stride;
  a.n_q = n_q;
  a.cand_ids = cand_ids;
  a.score = b.score;
  a.row = b.row;
  a.out_rows = b.out_rows;
  a.out_scores = b.out_scores;
  a.status = b.status;
  a.out_counts = b.counts;
  a.scan_status = d_scan_status;
  ProfScope p1(ctx, MRL_KERNEL_RERANK, 0, 0, n_q);
  ProfScope p2(ctx, MRL_KERNEL_RERANK_SORT, 0, 0, n_q);
  HIP_TRY(launch_rerank(a, ctx->stream, p1.ev(), p2.ev()));
  p1.commit(n_q != 0 && stride != 0);
  p2.commit(n_q != 0 && stride != 0);
  return MRL_OK;
}

extern "C" int mrl_rerank_rows(mrl_ctx* ctx, const mrl_rerank_store* store, const float* queries, uint32_t n_q,
                               uint32_t dims, const uint64_t* cand_rows, const uint32_t* counts, uint32_t stride,
                               uint64_t* out_rows, float* out_scores) {
  if (!ctx || !store) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (store->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "store belongs to another context");
  if (dims != store->dims) return fail(MRL_ERR_INVALID_ARG, "query dims differ from the store's");
  if (stride > MRL_MAX_SHORTLIST) return fail(MRL_ERR_INVALID_ARG, "stride above MRL_MAX_SHORTLIST");
  if (n_q == 0 || stride == 0) return MRL_OK;
  if (!queries || !cand_rows || !counts || !out_rows || !out_scores) return fail(MRL_ERR_INVALID_ARG, "null buffer");
  for (uint32_t q = 0; q < n_q; ++q) {
    if (counts[q] > stride) return fail(MRL_ERR_INVALID_ARG, "count above stride");
    for (uint32_t i = 0; i < counts[q]; ++i)
      if (cand_rows[(size_t)q * stride + i] >= store->n_rows)
        return fail(MRL_ERR_INVALID_ARG, "candidate row out of range of the rerank store");
  }
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  const size_t nc = (size_t)n_q * stride;
  const size_t qbytes = (size_t)n_q * dims * 4;
  const size_t bytes = rerank_bytes(n_q, stride) + qbytes + nc * 8 + (size_t)n_q * 4 + 64;
  uint8_t* base = nullptr;
  if (hipMalloc(&base, bytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "rerank buffers");
  const RerankBuffers b = rerank_carve(base, n_q, stride);
  uint8_t* p = base + ((rerank_bytes(n_q, stride) + 15) & ~(size_t)15);
  uint64_t* d_cand = reinterpret_cast<uint64_t*>(p);
  float* d_q = reinterpret_cast<float*>(p + nc * 8);
  uint32_t* d_counts = reinterpret_cast<uint32_t*>(p + nc * 8 + qbytes);
  hipError_t e = hipMemcpyAsync(d_cand, cand_rows, nc * 8, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(d_q, queries, qbytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(d_counts, counts, (size_t)n_q * 4, hipMemcpyHostToDevice, ctx->stream);
  int rc = MRL_OK;
  if (e == hipSuccess) rc = enqueue_rerank(ctx, store, d_q, n_q, d_cand, 0, d_counts, stride, b);
  std::vector<uint32_t> st(n_q);
  if (e == hipSuccess && !rc) e = hipMemcpyAsync(out_rows, b.out_rows, nc * 8, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess && !rc) e = hipMemcpyAsync(out_scores, b.out_scores, nc * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess && !rc) e = hipMemcpyAsync(st.data(), b.status, (size_t)n_q * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  dev_free(base);
  if (rc) return rc;
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("rerank: ") + hipGetErrorString(e));
  return status_error(st.data(), (uint32_t)st.size());
}

extern "C" int mrl_results_rerank(mrl_ctx* ctx, mrl_results* res, const mrl_rerank_store* store, uint64_t* out_rows,
                                  float* out_scores, uint32_t* out_counts) {
  if (!ctx || !res || !store) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (res->ctx != ctx || store->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "objects belong to another context");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  const mrl_plans* plans = res->last_plans;
  if (!plans) return fail(MRL_ERR_INVALID_ARG, "no scan was enqueued on these results");
  if (plans->dims != store->dims) return fail(MRL_ERR_INVALID_ARG, "query dims differ from the store's");
  const uint32_t n_q = plans->n_q, K = res->k, nq = std::max<uint32_t>(res->n_q, 1);
  if (n_q == 0) {
    res->pending = false;
    return MRL_OK;
  }
  if (!res->d_rr && hipMalloc(&res->d_rr, rerank_bytes(nq, K)) != hipSuccess) {
    res->d_rr = nullptr;
    return fail(MRL_ERR_OUT_OF_MEMORY, "rerank buffers");
  }
  const RerankBuffers b = rerank_carve(res->d_rr, nq, K);
  const size_t n = (size_t)nq * K;
  uint8_t* h = host_stage(ctx, rerank_out_bytes(nq, K));
  if (!h) return fail(MRL_ERR_OUT_OF_MEMORY, "pinned staging buffer");
  // The rerank is enqueued right behind the scan; the scan's status rides
  // along in bits 8.. of the rerank status, so one read-back serves both.
  auto run = [&](const uint32_t* scan_status) -> int {
    int rc = enqueue_rerank(ctx, store, plans->d_queries, n_q, res->d_ids, 1, res->d_counts, K, b, scan_status);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(h, b.status, (size_t)nq * 8 + (size_t)n_q * K * 8, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipMemcpyAsync(h + (size_t)nq * 8 + n * 8, b.out_scores, (size_t)n_q * K * 4, hipMemcpyDeviceToHost,
                           ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    return MRL_OK;
  };
  const bool pend = res->pending && res->last_index && res->last_index->n_blocks;
  int rc = run(pend ? res->d_status : nullptr);
  if (rc) return rc;
  const uint32_t* st = reinterpret_cast<const uint32_t*>(h);
  std::vector<uint32_t> scan_st(n_q);
  for (uint32_t q = 0; q < n_q; ++q) scan_st[q] = st[q] >> 8;
  bool rerun = false;
  if ((rc = handle_scan_status(ctx, res, scan_st.data(), n_q, &rerun))) return rc;
  if (rerun && (rc = run(nullptr))) return rc;
  if ((rc = status_error(st, n_q))) return rc;
  if (out_rows) memcpy(out_rows, h + (size_t)nq * 8, (size_t)n_q * K * 8);
  if (out_scores) memcpy(out_scores, h + (size_t)nq * 8 + n * 8, (size_t)n_q * K * 4);
  if (out_counts) memcpy(out_counts, h + (size_t)nq * 4, (size_t)n_q * 4);
  return MRL_OK;
}

// Ring search of n_q queries (device) over n_pending host rows: a transient
// fp32 store, every row a candidate, rerank buffers carved from *scratch
// (caller frees).  Caller holds the lock.
static int ring_search_enqueue(mrl_ctx* ctx, const float* pending, uint32_t n_pending, uint32_t dims,
                               const float* d_queries, uint32_t n_q, mrl_rerank_store** store, void** scratch,
                               RerankBuffers* b) {
  int rc = store_create_locked(ctx, pending, 0, n_pending, dims, MRL_RERANK_FP32, store);
  if (rc) return rc;
  if (hipMalloc(scratch, rerank_bytes(n_q, n_pending)) != hipSuccess) {
    *scratch = nullptr;
    return fail(MRL_ERR_OUT_OF_MEMORY, "ring search buffers");
  }
  *b = rerank_carve(*scratch, n_q, n_pending);
  return enqueue_rerank(ctx, *store, d_queries, n_q, nullptr, 0, nullptr, n_pending, *b);
}

static int check_ring_args(const float* pending, uint32_t n_pending, uint32_t dims) {
  if (n_pending && !pending) return fail(MRL_ERR_INVALID_ARG, "null pending rows");
  if (n_pending > MRL_MAX_SHORTLIST) return fail(MRL_ERR_INVALID_ARG, "more than MRL_MAX_SHORTLIST pending rows");
  if (dims == 0 || dims > MRL_MAX_DIMS) return fail(MRL_ERR_INVALID_ARG, "dims must be in [1, MRL_MAX_DIMS]");
  return MRL_OK;
}

extern "C" int mrl_ring_search(mrl_ctx* ctx, const float* pending, uint32_t n_pending, uint32_t dims,
                               const float* queries, uint32_t n_q, uint32_t top_k, uint64_t* out_local,
                               float* out_scores, uint32_t* out_counts) {
  if (!ctx) return fail(MRL_ERR_INVALID_ARG, "null argument");
  int rc = check_ring_args(pending, n_pending, dims);
  if (rc) return rc;
  if (n_q && (!queries || !out_counts || (top_k && (!out_local || !out_scores))))
    return fail(MRL_ERR_INVALID_ARG, "null buffer");
  const uint32_t keep = std::min(top_k, n_pending);
  if (n_q == 0) return MRL_OK;
  if (keep == 0) {
    memset(out_counts, 0, (size_t)n_q * 4);
    return MRL_OK;
  }
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  float* d_q = nullptr;
  mrl_rerank_store* store = nullptr;
  void* scratch = nullptr;
  RerankBuffers b{};
  const size_t qbytes = (size_t)n_q * dims * 4;
  if (hipMalloc(&d_q, qbytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "ring queries");
  hipError_t e = hipMemcpyAsync(d_q, queries, qbytes, hipMemcpyHostToDevice, ctx->stream);
  rc = e == hipSuccess ? ring_search_enqueue(ctx, pending, n_pending, dims, d_q, n_q, &store, &scratch, &b)
                       : fail(MRL_ERR_HIP, "ring query copy");
  std::vector<uint32_t> st(n_q);
  if (!rc) {
    // search_exact's truncate(top_k): the first `keep` of each sorted row
    e = hipMemcpy2DAsync(out_local, keep * 8, b.out_rows, (size_t)n_pending * 8, keep * 8, n_q,
                         hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess)
      e = hipMemcpy2DAsync(out_scores, keep * 4, b.out_scores, (size_t)n_pending * 4, keep * 4, n_q,
                           hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(st.data(), b.status, (size_t)n_q * 4, hipMemcpyDeviceToHost, ctx->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  dev_free(d_q);
  dev_free(scratch);
  store_free(store);
  if (rc) return rc;
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("ring search: ") + hipGetErrorString(e));
  for (uint32_t q = 0; q < n_q; ++q) out_counts[q] = keep;
  return status_error(st.data(), (uint32_t)st.size());
}

extern "C" int mrl_results_merge_ring(mrl_ctx* ctx, mrl_results* res, const float* pending, uint32_t n_pending,
                                      uint32_t dims) {
  if (!ctx || !res) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (res->ctx != ctx) return fail(MRL_ERR_INVALID_ARG, "results belong to another context");
  int rc = check_ring_args(pending, n_pending, dims);
  if (rc) return rc;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  const mrl_plans* plans = res->last_plans;
  if (!plans) return fail(MRL_ERR_INVALID_ARG, "no scan was enqueued on these results");
  if (plans->dims != dims) return fail(MRL_ERR_INVALID_ARG, "pending rows have other dims than the queries");
  if ((rc = resolve_pending(ctx, res))) return rc;
  const uint32_t n_q = plans->n_q, K = res->k;
  if (n_q == 0 || n_pending == 0) return MRL_OK;
  mrl_rerank_store* store = nullptr;
  void* scratch = nullptr;
  uint8_t* merged = nullptr;
  RerankBuffers b{};
  const size_t nc = (size_t)n_q * K;
  auto cleanup = [&]() {
    dev_free(scratch);
    dev_free(merged);
    store_free(store);
  };
  if (hipMalloc(&merged, nc * 12 + (size_t)n_q * 4) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "ring merge");
  rc = ring_search_enqueue(ctx, pending, n_pending, dims, plans->d_queries, n_q, &store, &scratch, &b);
  if (rc) {
    cleanup();
    return rc;
  }
  RingMergeArgs ma{};
  ma.ids = res->d_ids;
  ma.scores = res->d_scores;
  ma.counts = res->d_counts;
  ma.ring_rows = b.out_rows;
  ma.ring_scores = b.out_scores;
  ma.ring_status = b.status;
  ma.n_ring = n_pending;
  ma.k = K;
  ma.n_q = n_q;
  ma.out_ids = reinterpret_cast<uint64_t*>(merged);
  ma.out_scores = reinterpret_cast<float*>(merged + nc * 8);
  ma.out_counts = reinterpret_cast<uint32_t*>(merged + nc * 12);
  std::vector<uint32_t> st(n_q);
  hipError_t e = launch_ring_merge(ma, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(res->d_ids, ma.out_ids, nc * 8, hipMemcpyDeviceToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(res->d_scores, ma.out_scores, nc * 4, hipMemcpyDeviceToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(res->d_counts, ma.out_counts, (size_t)n_q * 4, hipMemcpyDeviceToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(st.data(), b.status, (size_t)n_q * 4, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  cleanup();
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("ring merge: ") + hipGetErrorString(e));
  return status_error(st.data(), (uint32_t)st.size());
}

// ---------------------------------------------------------------------------
// ingest helpers
// ---------------------------------------------------------------------------
static bool fit_view(const mrl_eden_fit* f, EdenFitView* v) {
  if (!f) return false;
  v->dim = f->dim;
  v->bits = f->bits;
  v->seed = f->seed;
  v->mean = f->mean;
  return true;
}

extern "C" int mrl_encode_block(const float* vectors, uint32_t n, uint32_t dims, const uint32_t* timestamps,
                                const uint32_t* sources, const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                                void* out_block) {
  if (!vectors || !timestamps || !sources || !out_block) return fail(MRL_ERR_INVALID_ARG, "null argument");
  EdenFitView e, m;
  int rc = encode_block(vectors, n, dims, timestamps, sources, fit_view(eden, &e) ? &e : nullptr,
                        fit_view(eden_mid, &m) ? &m : nullptr, static_cast<uint8_t*>(out_block));
  return rc ? fail(rc, "encode_block: invalid arguments (n in 1..64, dims >= 192, fit shapes)") : MRL_OK;
}

extern "C" int mrl_encode_corpus(const float* matrix, uint64_t n, uint32_t dims, uint32_t default_source,
                                 const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid, int n_threads,
                                 void* out_blocks) {
  if ((n && (!matrix || !out_blocks))) return fail(MRL_ERR_INVALID_ARG, "null argument");
  EdenFitView e, m;
  int rc = encode_corpus(matrix, n, dims, default_source, fit_view(eden, &e) ? &e : nullptr,
                         fit_view(eden_mid, &m) ? &m : nullptr, n_threads, static_cast<uint8_t*>(out_blocks));
  return rc ? fail(rc, "encode_corpus: invalid arguments") : MRL_OK;
}

extern "C" int mrl_encode_corpus_clustered(const float* matrix, uint64_t n, uint32_t dims, const uint32_t* cluster,
                                           uint32_t default_source, const mrl_eden_fit* eden,
                                           const mrl_eden_fit* eden_mid, int n_threads, void* out_blocks) {
  if ((n && (!matrix || !out_blocks || !cluster))) return fail(MRL_ERR_INVALID_ARG, "null argument");
  EdenFitView e, m;
  int rc = encode_corpus(matrix, n, dims, default_source, fit_view(eden, &e) ? &e : nullptr,
                         fit_view(eden_mid, &m) ? &m : nullptr, n_threads, static_cast<uint8_t*>(out_blocks),
                         cluster);
  return rc ? fail(rc, "encode_corpus: invalid arguments") : MRL_OK;
}


// CRC-32 tables for the GPU encoder.  raw(c, M) is the reflected CRC register
// after bytes M starting from register c (no initial or final xor); it is
// linear in c and M over GF(2), so
//   CRC(M) = raw(~0, 0^4096) ^ xor_k carry(raw(0, M_k), 64 * (63 - k)) ^ ~0
// for the 64-byte chunks M_k, with carry(c, L) = raw(c, 0^L) = xor over the
// set bits i of c of carry(1 << i, L).
struct CrcTables {
  uint32_t tab[256 + 64 * 32];
  uint32_t konst;
};
static const CrcTables& crc_tables() {
  static const CrcTables t = [] {
    CrcTables r{};
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      r.tab[i] = c;
    }
    auto zeros = [&](uint32_t c, uint32_t nbytes) {
      for (uint32_t j = 0; j < nbytes; ++j) c = r.tab[c & 0xffu] ^ (c >> 8);
      return c;
    };
    for (uint32_t k = 0; k < 64; ++k)
      for (uint32_t i = 0; i < 32; ++i) r.tab[256 + 32 * k + i] = zeros(1u << i, 64u * (63u - k));
    r.konst = zeros(0xffffffffu, kBlockBytes) ^ 0xffffffffu;
    return r;
  }();
  return t;
}

static int encode_device(mrl_ctx* ctx, const float* d_matrix, uint64_t n, uint32_t dims, const uint32_t* d_cluster,
                         uint32_t default_source, const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                         void* d_out_blocks) {
  if (!ctx || (n && (!d_matrix || !d_out_blocks))) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (dims < (uint32_t)(kPrefixDims + kRabitqDims)) return fail(MRL_ERR_INVALID_ARG, "dims < 192");
  if (eden && (eden->dim != 64 || eden->bits != 4 || !eden->mean))
    return fail(MRL_ERR_INVALID_ARG, "EdenProd prefix needs a 64-d 4-bit fit");
  if (eden_mid && (!eden || eden_mid->dim != 128 || eden_mid->bits != 1 || !eden_mid->mean))
    return fail(MRL_ERR_INVALID_ARG, "EdenB1 mid-band needs a 128-d 1-bit fit and an EdenProd prefix");
  if (n == 0) return MRL_OK;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (!ctx->d_crc) {
    const CrcTables& t = crc_tables();
    if (hipMalloc(&ctx->d_crc, sizeof(t.tab)) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "crc tables");
    HIP_TRY(hipMemcpy(ctx->d_crc, t.tab, sizeof(t.tab), hipMemcpyHostToDevice));
    ctx->crc_const = t.konst;
  }
  float* d_means = nullptr;
  if (hipMalloc(&d_means, 192 * sizeof(float)) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "fit means");
  hipError_t e = hipSuccess;
  if (eden) e = hipMemcpy(d_means, eden->mean, 64 * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess && eden_mid) e = hipMemcpy(d_means + 64, eden_mid->mean, 128 * sizeof(float), hipMemcpyHostToDevice);
  EncodeArgs a{};
  a.x = d_matrix;
  a.n = n;
  a.dims = dims;
  a.cluster = d_cluster;
  a.source = default_source;
  a.eden_mean = eden ? d_means : nullptr;
  a.eden_seed = eden ? eden->seed : 0;
  a.mid_mean = eden_mid ? d_means + 64 : nullptr;
  a.mid_seed = eden_mid ? eden_mid->seed : 0;
  a.crc_tab = ctx->d_crc;
  a.crc_zt = ctx->d_crc + 256;
  a.crc_const = ctx->crc_const;
  a.c = ctx->consts;
  a.sqrt64 = sqrtf(64.0f);
  a.sqrt128 = sqrtf(128.0f);
  a.out = static_cast<uint8_t*>(d_out_blocks);
  a.n_blocks = (n + 63) / 64;
  if (e == hipSuccess) e = launch_encode(a, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  dev_free(d_means);
  if (e != hipSuccess) return fail(MRL_ERR_HIP, std::string("encode: ") + hipGetErrorString(e));
  return MRL_OK;
}

extern "C" int mrl_encode_corpus_device(mrl_ctx* ctx, const float* d_matrix, uint64_t n, uint32_t dims,
                                        uint32_t default_source, const mrl_eden_fit* eden,
                                        const mrl_eden_fit* eden_mid, void* d_out_blocks) {
  return encode_device(ctx, d_matrix, n, dims, nullptr, default_source, eden, eden_mid, d_out_blocks);
}

extern "C" int mrl_encode_corpus_device_clustered(mrl_ctx* ctx, const float* d_matrix, uint64_t n, uint32_t dims,
                                                  const uint32_t* d_cluster, uint32_t default_source,
                                                  const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                                                  void* d_out_blocks) {
  if (n && !d_cluster) return fail(MRL_ERR_INVALID_ARG, "null argument");
  return encode_device(ctx, d_matrix, n, dims, d_cluster, default_source, eden, eden_mid, d_out_blocks);
}

// Device memory for callers without a HIP allocator of their own (plain
// pointers in and out; copies are synchronous on the context stream).
extern "C" int mrl_device_alloc(mrl_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return fail(MRL_ERR_INVALID_ARG, "null argument");
  *out = nullptr;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  if (bytes && hipMalloc(out, bytes) != hipSuccess) return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc");
  return MRL_OK;
}

extern "C" void mrl_device_free(mrl_ctx* ctx, void* d_ptr) {
  if (!ctx || !d_ptr) return;
  std::lock_guard<std::mutex> g(ctx->mu);
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipFree(d_ptr);
}

extern "C" int mrl_device_mem_info(mrl_ctx* ctx, uint64_t* free_bytes, uint64_t* total_bytes) {
  if (!ctx || !free_bytes || !total_bytes) return fail(MRL_ERR_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  size_t f = 0, t = 0;
  HIP_TRY(hipMemGetInfo(&f, &t));
  *free_bytes = f;
  *total_bytes = t;
  return MRL_OK;
}

extern "C" int mrl_copy_to_device(mrl_ctx* ctx, void* d_dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!d_dst || !src))) return fail(MRL_ERR_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MRL_OK;
}

extern "C" int mrl_copy_to_host(mrl_ctx* ctx, void* dst, const void* d_src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !d_src))) return fail(MRL_ERR_INVALID_ARG, "null argument");
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return MRL_OK;
}

extern "C" int mrl_index_from_device(mrl_ctx* ctx, const void* d_blocks, uint64_t n_blocks, mrl_index** out) {
  if (!ctx || !out || (n_blocks && !d_blocks)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (n_blocks > (1ull << 26)) return fail(MRL_ERR_INVALID_ARG, "n_blocks exceeds 2^26 (32-bit row ids)");
  *out = nullptr;
  std::lock_guard<std::mutex> g(ctx->mu);
  HIP_TRY(hipSetDevice(ctx->device));
  std::unique_ptr<mrl_index> ix(new mrl_index());
  ix->ctx = ctx;
  ix->n_blocks = n_blocks;
  if (n_blocks) {
    if (hipMalloc(&ix->d_blocks, (size_t)n_blocks * kBlockBytes) != hipSuccess)
      return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc index");
    if (hipMalloc(&ix->d_recs, (size_t)n_blocks * 64 * kRecWords * 16) != hipSuccess) {
      dev_free(ix->d_blocks);
      return fail(MRL_ERR_OUT_OF_MEMORY, "hipMalloc index records");
    }
    hipError_t e = launch_relayout(static_cast<const uint8_t*>(d_blocks), ix->d_blocks, n_blocks, true, ctx->stream,
                                   ix->d_recs);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      dev_free(ix->d_blocks);
      dev_free(ix->d_recs);
      return fail(MRL_ERR_HIP, std::string("index from device: ") + hipGetErrorString(e));
    }
    int rc = build_bounds(ctx, ix.get());
    if (rc) {
      dev_free(ix->d_blocks);
      dev_free(ix->d_recs);
      return rc;
    }
  }
  ctx_retain(ctx);
  *out = ix.release();
  return MRL_OK;
}

extern "C" int mrl_eden_fit_band(const float* rows, uint64_t n_rows, uint32_t row_stride, uint32_t start, uint32_t dim,
                                 float* out_mean) {
  if (!rows || !out_mean) return fail(MRL_ERR_INVALID_ARG, "null argument");
  if (start + dim > row_stride) return fail(MRL_ERR_INVALID_ARG, "band exceeds the row");
  int rc = eden_fit_band(rows, n_rows, row_stride, start, dim, out_mean);
  return rc ? fail(rc, "empty corpus for EdenFit") : MRL_OK;
}

// ---------------------------------------------------------------------------
// synthetic workloads (benchmark inputs)
// ---------------------------------------------------------------------------
static SynthSpec to_spec(const mrl_synth_spec* s) {
  SynthSpec o;
  o.n_docs = s->n_docs;
  o.dims = s->dims;
  o.mean_offset = s->mean_offset;
  o.seed = s->seed;
  o.n_centroids = s->n_centroids;
  o.seed_centroids = s->seed_centroids;
  o.seed_assign = s->seed_assign;
  o.noise_sigma = s->noise_sigma;
  return o;
}

extern "C" int mrl_synth_docs(const mrl_synth_spec* spec, uint64_t first_row, uint64_t n_rows, int n_threads,
                              float* out) {
  if (!spec || (n_rows && !out)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  SynthSpec s = to_spec(spec);
  parallel_for(n_rows, n_threads, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t r = r0; r < r1; ++r) synth_doc(s, first_row + r, out + r * s.dims);
  });
  return MRL_OK;
}

extern "C" int mrl_synth_queries(const mrl_synth_spec* spec, uint64_t seed_q, float noise_sigma, int fresh,
                                 uint32_t n_q, float* out, uint64_t* out_src_rows) {
  if (!spec || (n_q && !out)) return fail(MRL_ERR_INVALID_ARG, "null argument");
  SynthSpec s = to_spec(spec);
  for (uint32_t q = 0; q < n_q; ++q)
    synth_query(s, seed_q, noise_sigma, fresh, q, out + (size_t)q * s.dims, out_src_rows ? out_src_rows + q : nullptr);
  return MRL_OK;
}

extern "C" int mrl_synth_eden_fit(const mrl_synth_spec* spec, uint64_t n_rows, float* out_mean64) {
  if (!spec || !out_mean64) return fail(MRL_ERR_INVALID_ARG, "null argument");
  SynthSpec s = to_spec(spec);
  n_rows = std::min<uint64_t>(n_rows, s.n_docs);
  if (!n_rows) return fail(MRL_ERR_INVALID_ARG, "empty corpus for EdenFit");
  std::vector<float> rows(n_rows * s.dims);
  parallel_for(n_rows, 0, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t r = r0; r < r1; ++r) synth_doc(s, r, rows.data() + r * s.dims);
  });
  return eden_fit_band(rows.data(), n_rows, s.dims, 0, 64, out_mean64);
}

extern "C" int mrl_synth_encode(const mrl_synth_spec* spec, const mrl_eden_fit* eden, const mrl_eden_fit* eden_mid,
                                uint32_t default_source, int n_threads, void* out_blocks) {
  if (!spec || !out_blocks) return fail(MRL_ERR_INVALID_ARG, "null argument");
  SynthSpec s = to_spec(spec);
  EdenFitView e, m;
  const EdenFitView* ep = fit_view(eden, &e) ? &e : nullptr;
  const EdenFitView* mp = fit_view(eden_mid, &m) ? &m : nullptr;
  const uint64_t n_blocks = (s.n_docs + 63) / 64;
  std::atomic<int> status{MRL_OK};
  uint8_t* out = static_cast<uint8_t*>(out_blocks);
  parallel_for(n_blocks, n_threads, [&](uint64_t b0, uint64_t b1) {
    std::vector<float> rows(64 * (size_t)s.dims);
    uint32_t ts[64], src[64];
    for (uint64_t b = b0; b < b1; ++b) {
      const uint64_t start = b * 64, end = std::min(s.n_docs, start + 64);
      for (uint64_t r = start; r < end; ++r) {
        synth_doc(s, r, rows.data() + (r - start) * s.dims);
        ts[r - start] = (uint32_t)r;
        src[r - start] = default_source;
      }
      int rc = encode_block(rows.data(), (uint32_t)(end - start), s.dims, ts, src, ep, mp, out + b * kBlockBytes);
      if (rc) status.store(rc);
    }
  });
  return status.load() ? fail(status.load(), "synth encode failed") : MRL_OK;
}

extern "C" int mrl_synth_encode_clustered(const mrl_synth_spec* spec, const mrl_eden_fit* eden,
                                          const mrl_eden_fit* eden_mid, uint32_t default_source, int n_threads,
                                          void* out_blocks, uint64_t* out_rows) {
  if (!spec || !out_blocks) return fail(MRL_ERR_INVALID_ARG, "null argument");
  SynthSpec s = to_spec(spec);
  if (s.n_centroids == 0) return fail(MRL_ERR_INVALID_ARG, "the corpus has no clusters");
  // rows in (cluster, row) order: a counting sort of the row clusters
  std::vector<uint32_t> cl(s.n_docs);
  parallel_for(s.n_docs, n_threads, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t r = r0; r < r1; ++r) cl[r] = synth_cluster(s, r);
  });
  std::vector<uint64_t> start(s.n_centroids + 1, 0);
  for (uint64_t r = 0; r < s.n_docs; ++r) ++start[cl[r] + 1];
  for (uint32_t c = 0; c < s.n_centroids; ++c) start[c + 1] += start[c];
  std::vector<uint64_t> order(s.n_docs);
  for (uint64_t r = 0; r < s.n_docs; ++r) order[start[cl[r]]++] = r;
  if (out_rows) memcpy(out_rows, order.data(), s.n_docs * sizeof(uint64_t));
  EdenFitView e, m;
  const EdenFitView* ep = fit_view(eden, &e) ? &e : nullptr;
  const EdenFitView* mp = fit_view(eden_mid, &m) ? &m : nullptr;
  const uint64_t n_blocks = (s.n_docs + 63) / 64;
  std::atomic<int> status{MRL_OK};
  uint8_t* out = static_cast<uint8_t*>(out_blocks);
  parallel_for(n_blocks, n_threads, [&](uint64_t b0, uint64_t b1) {
    std::vector<float> rows(64 * (size_t)s.dims);
    uint32_t ts[64], src[64], bc[64];
    for (uint64_t b = b0; b < b1; ++b) {
      const uint64_t start_p = b * 64, end = std::min(s.n_docs, start_p + 64);
      for (uint64_t p = start_p; p < end; ++p) {
        synth_doc(s, order[p], rows.data() + (p - start_p) * s.dims);
        ts[p - start_p] = (uint32_t)p;  // the row's position in the encoded order (encoder.rs:184-189)
        src[p - start_p] = default_source;
        bc[p - start_p] = cl[order[p]];
      }
      int rc = encode_block(rows.data(), (uint32_t)(end - start_p), s.dims, ts, src, ep, mp, out + b * kBlockBytes,
                            block_cluster(bc, end - start_p));
      if (rc) status.store(rc);
    }
  });
  return status.load() ? fail(status.load(), "synth encode failed") : MRL_OK;
}
