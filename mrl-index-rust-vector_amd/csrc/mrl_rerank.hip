// mrl_rerank.hip -- gfx950 post-scan rerank: every candidate row of a shortlist is
// scored against the full f32 query, then the list is stably sorted by score,
// descending.  This is QueryPipeline::rerank_exact_rows (src/pipeline.rs:157-169)
// and the precision loop of the retrieval bench (src/retrieval_bench.rs:739-745)
// over rerank_dot (src/lowprec.rs:103-121).
//
// Numerics match the reference bit for bit:
//  - 768 dims: dot_768 / dot_f16_768 / dot_i8_768 (src/embed.rs:130-206) run eight
//    accumulators, accumulator j summing the products of the elements i = j mod 8
//    in index order from +0.0; the result is acc0 + acc1 + ... + acc7, left to
//    right (times the f16 scale for int8).  Here lane j of an 8-lane group runs
//    accumulator j of one candidate, so the 96 dependent adds of a chain stay
//    sequential and the eight chains run side by side.
//  - other dims (fp32 only): the sequential sum of a[i]*b[i] from -0.0
//    (src/embed.rs:123), one lane per candidate.
//  - the sort is stable: ties (including +0.0 against -0.0, which partial_cmp
//    calls equal) keep the candidates' input order.
//
// Store layout (768 dims).  A row's elements are kept "accumulator-major":
// element i = 8t + j sits at position 96j + t, so accumulator j reads one
// contiguous run of 96 elements with 16-byte loads (24 for f32, 12 for f16, 6
// for int8) instead of 96 strided scalar loads.  The stores for f16 and int8 are
// built here from f32 rows with the reference's conversions
// (Fp16Vec768::from_f32, Int8Vec768::from_f32, src/lowprec.rs:49-94).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mrl_half.h"
#include "mrl_internal.h"

namespace mrl {

namespace {

constexpr int kStoreThreads = 256;  // four rows per workgroup, one per wave
constexpr int kScoreThreads = 256;  // 768 dims: 32 candidates per workgroup (8 lanes each)
constexpr int kSortThreads = 256;
constexpr int kSortCap = MRL_MAX_SHORTLIST;
constexpr int kRankMax = 512;
constexpr int kQStride = 100;       // LDS row of one accumulator's 96 query values (bank spread)

__device__ __forceinline__ float zero_acc() {
  float z = 0.0f;
  asm volatile("" : "+v"(z));
  return z;
}

__device__ __forceinline__ uint32_t store_pos(uint32_t i) { return (i & 7u) * 96u + (i >> 3); }

// Order-preserving map f32 -> u32 (larger score -> larger key); -0 == +0.
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  if ((u << 1) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Int8Vec768::from_f32 code of one element (src/lowprec.rs:83-86):
// round half away from zero, clamp (NaN passes), `as i32` (NaN -> 0).
__device__ __forceinline__ uint32_t int8_code(float v, float inv) {
  float q = roundf(v * inv);
  if (q < -127.0f) q = -127.0f;
  if (q > 127.0f) q = 127.0f;
  const int32_t i = (q == q) ? (int32_t)q : 0;
  return (uint32_t)i & 0xffu;
}

// ---------------------------------------------------------------------------
// store build: f32 rows (row-major, 768 dims) -> accumulator-major rows
// ---------------------------------------------------------------------------
template <int P>
__global__ __launch_bounds__(kStoreThreads) void k_store768(const float* __restrict__ x, uint8_t* __restrict__ data,
                                                            uint16_t* __restrict__ scales, uint64_t n_rows) {
  constexpr uint32_t kRowBytes = P == MRL_RERANK_FP32 ? 3072u : P == MRL_RERANK_FP16 ? 1536u : 768u;
  __shared__ __align__(16) uint8_t s_row[kStoreThreads / 64][3072];
  const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  uint8_t* sb = s_row[w];
  for (uint64_t r0 = (uint64_t)blockIdx.x * 4u; r0 < n_rows; r0 += (uint64_t)gridDim.x * 4u) {
    const uint64_t r = r0 + w;
    const bool live = r < n_rows;
    float v[12];
    if (live) {
      const float4* src = reinterpret_cast<const float4*>(x + r * 768u);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float4 f = src[lane + 64u * k];
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 12; ++e) v[e] = 0.0f;
    }
    float inv = 0.0f;
    if (P == MRL_RERANK_INT8) {
      // max_abs = fold of f32::max over |x| from 0.0 (NaN ignored); max is exact,
      // so the wave reduction order does not matter.
      float m = 0.0f;
#pragma unroll
      for (int e = 0; e < 12; ++e) m = fmaxf(m, fabsf(v[e]));
#pragma unroll
      for (int h = 1; h < 64; h <<= 1) m = fmaxf(m, __shfl_xor(m, h));
      const float scale = m < 1e-12f ? 0.0f : m / 127.0f;
      inv = scale > 0.0f ? 1.0f / scale : 0.0f;
      if (live && lane == 0) scales[r] = (uint16_t)f32_to_f16(scale);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t i = 4u * lane + 256u * k + e;
        const uint32_t p = store_pos(i);
        const float f = v[4 * k + e];
        if (P == MRL_RERANK_FP32) reinterpret_cast<float*>(sb)[p] = f;
        else if (P == MRL_RERANK_FP16) reinterpret_cast<uint16_t*>(sb)[p] = (uint16_t)f32_to_f16(f);
        else sb[p] = (uint8_t)int8_code(f, inv);
      }
    }
    __syncthreads();
    if (live) {
      uint4* dst = reinterpret_cast<uint4*>(data + r * kRowBytes);
      const uint4* s4 = reinterpret_cast<const uint4*>(sb);
      for (uint32_t c = lane; c < kRowBytes / 16u; c += 64u) dst[c] = s4[c];
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// scoring
// ---------------------------------------------------------------------------
// Row markers in the scratch row array: a row outside the store, and a ring
// hit that scored_hits_to_row_ids drops.
constexpr uint64_t kRowBad = ~0ull;
constexpr uint64_t kRowSkip = ~0ull - 1u;

__device__ __forceinline__ uint32_t count_of(const RerankArgs& a, uint32_t q) {
  return a.counts ? a.counts[q] : a.stride;
}

// Candidate c of query q -> store row.  *ok false: no row to score (*row says why).
__device__ __forceinline__ void resolve_row(const RerankArgs& a, uint32_t q, uint32_t c, uint64_t* row, bool* ok) {
  if (!a.cand) {
    *row = c;
    *ok = c < a.n_rows;
    if (!*ok) *row = kRowBad;
    return;
  }
  const uint64_t id = a.cand[(uint64_t)q * a.stride + c];
  if (a.cand_ids && (id >> 16) == 0xffffffffull) {  // ring sentinel (block == u32::MAX): skipped
    *row = kRowSkip;
    *ok = false;
    return;
  }
  // scored_hits_to_row_ids (src/pipeline.rs:175-180): block * 64 + slot
  const uint64_t r = a.cand_ids ? (id >> 16) * 64u + (id & 0xffffu) : id;
  *ok = r < a.n_rows;
  *row = *ok ? r : kRowBad;
}

// Accumulator j of one candidate over its 96 stored elements.
template <int P>
__device__ __forceinline__ float chain768(const RerankArgs& a, uint64_t row, uint32_t j, const float* qj) {
  float acc = zero_acc();
  if (P == MRL_RERANK_FP32) {
    const float4* r4 = reinterpret_cast<const float4*>(static_cast<const float*>(a.data) + row * 768u + j * 96u);
    float4 b[24];
#pragma unroll
    for (int u = 0; u < 24; ++u) b[u] = r4[u];
#pragma unroll
    for (int u = 0; u < 24; ++u) {
      const float4 qv = reinterpret_cast<const float4*>(qj)[u];
      acc = acc + qv.x * b[u].x;
      acc = acc + qv.y * b[u].y;
      acc = acc + qv.z * b[u].z;
      acc = acc + qv.w * b[u].w;
    }
  } else if (P == MRL_RERANK_FP16) {
    const uint4* r4 = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.data) + row * 768u + j * 96u);
    uint4 b[12];
#pragma unroll
    for (int u = 0; u < 12; ++u) b[u] = r4[u];
#pragma unroll
    for (int u = 0; u < 12; ++u) {
      const uint32_t wd[4] = {b[u].x, b[u].y, b[u].z, b[u].w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float lo = h2f((uint16_t)(wd[h] & 0xffffu));
        const float hi = h2f((uint16_t)(wd[h] >> 16));
        acc = acc + qj[8 * u + 2 * h] * lo;
        acc = acc + qj[8 * u + 2 * h + 1] * hi;
      }
    }
  } else {
    const uint4* r4 = reinterpret_cast<const uint4*>(static_cast<const int8_t*>(a.data) + row * 768u + j * 96u);
    uint4 b[6];
#pragma unroll
    for (int u = 0; u < 6; ++u) b[u] = r4[u];
#pragma unroll
    for (int u = 0; u < 6; ++u) {
      const uint32_t wd[4] = {b[u].x, b[u].y, b[u].z, b[u].w};
#pragma unroll
      for (int h = 0; h < 4; ++h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float c = (float)(int8_t)((wd[h] >> (8 * e)) & 0xffu);
          acc = acc + qj[16 * u + 4 * h + e] * c;
        }
      }
    }
  }
  return acc;
}

template <int P>
__global__ __launch_bounds__(kScoreThreads) void k_score768(RerankArgs a, uint32_t n_chunks) {
  __shared__ __align__(16) float s_q[8 * kQStride];
  const uint32_t q = blockIdx.x / n_chunks;
  const uint32_t base = (blockIdx.x % n_chunks) * (kScoreThreads / 8);
  const uint32_t cnt = count_of(a, q);
  if (base >= cnt) return;  // uniform over the workgroup
  // query element i = 8t + j at s_q[kQStride*j + t]
  const float* qv = a.queries + (uint64_t)q * 768u;
  for (uint32_t i = threadIdx.x; i < 768u; i += kScoreThreads) s_q[kQStride * (i & 7u) + (i >> 3)] = qv[i];
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u, j = lane & 7u;
  const uint32_t c = base + threadIdx.x / 8u;
  uint64_t row = ~0ull;
  bool ok = false;
  if (c < cnt) resolve_row(a, q, c, &row, &ok);
  float acc = 0.0f;
  if (ok) acc = chain768<P>(a, row, j, s_q + kQStride * j);
  // acc0 + acc1 + ... + acc7, left to right, in lane j == 0 of the group
  const uint32_t g0 = lane & ~7u;
  float part[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) part[k] = __shfl(acc, (int)(g0 + k));
  if (j == 0 && c < cnt) {
    float s = part[0] + part[1];
#pragma unroll
    for (int k = 2; k < 8; ++k) s = s + part[k];
    if (P == MRL_RERANK_INT8 && ok) s = s * h2f(a.scales[row]);
    const uint64_t o = (uint64_t)q * a.stride + c;
    a.score[o] = ok ? s : 0.0f;
    a.row[o] = row;
  }
}

// fp32 at dims != 768: one lane per candidate, sequential from -0.0.
__global__ __launch_bounds__(kScoreThreads) void k_score_seq(RerankArgs a, uint32_t n_chunks) {
  __shared__ float s_q[MRL_MAX_DIMS];
  const uint32_t q = blockIdx.x / n_chunks;
  const uint32_t base = (blockIdx.x % n_chunks) * kScoreThreads;
  const uint32_t cnt = count_of(a, q);
  if (base >= cnt) return;
  const uint32_t dims = a.dims;
  const float* qv = a.queries + (uint64_t)q * dims;
  for (uint32_t i = threadIdx.x; i < dims; i += kScoreThreads) s_q[i] = qv[i];
  __syncthreads();
  const uint32_t c = base + threadIdx.x;
  if (c >= cnt) return;
  uint64_t row;
  bool ok;
  resolve_row(a, q, c, &row, &ok);
  float s = -0.0f;
  if (ok) {
    const float* r = static_cast<const float*>(a.data) + row * dims;
    for (uint32_t i = 0; i < dims; ++i) s = s + s_q[i] * r[i];
  }
  const uint64_t o = (uint64_t)q * a.stride + c;
  a.score[o] = ok ? s : 0.0f;
  a.row[o] = row;
}

// ---------------------------------------------------------------------------
// stable descending sort of one query's scored candidates
// ---------------------------------------------------------------------------
__device__ void bitonic_desc(uint64_t* s, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < n2 / 2; i += blockDim.x) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = s[lo], y = s[hi];
        if (desc ? (x < y) : (x > y)) {
          s[lo] = y;
          s[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Key = (score key, ~position): descending keys give score descending, then
// input position ascending -- the order of a stable sort.  Keys are distinct;
// skipped ring hits get a zero score key, below every scored entry (the
// smallest score key, that of -inf, is 0x007fffff), and are not emitted.
__global__ __launch_bounds__(kSortThreads) void k_rerank_sort(RerankArgs a) {
  __shared__ uint64_t s_key[kSortCap];
  __shared__ uint32_t s_bad, s_skip;
  const uint32_t q = blockIdx.x, tid = threadIdx.x;
  const uint32_t m = count_of(a, q);
  const uint64_t base = (uint64_t)q * a.stride;
  if (tid == 0) {
    s_bad = 0u;
    s_skip = 0u;
  }
  __syncthreads();
  uint32_t bad = 0u, skip = 0u;
  for (uint32_t i = tid; i < m; i += kSortThreads) {
    const float s = a.score[base + i];
    const uint64_t r = a.row[base + i];
    uint32_t key = score_key(s);
    if (r == kRowSkip) {
      key = 0u;
      ++skip;
    } else {
      if (!(s == s)) bad |= 1u;     // partial_cmp(..).unwrap() panics
      if (r == kRowBad) bad |= 2u;  // row index out of range
    }
    s_key[i] = ((uint64_t)key << 32) | (uint64_t)(~i);
  }
  if (bad) atomicOr(&s_bad, bad);
  if (skip) atomicAdd(&s_skip, skip);
  __syncthreads();
  auto emit = [&](uint32_t r, uint64_t key) {
    const uint32_t i = ~(uint32_t)key;
    a.out_rows[base + r] = a.row[base + i];
    a.out_scores[base + r] = a.score[base + i];
  };
  if (m <= (uint32_t)kRankMax) {
    for (uint32_t i = tid; i < m; i += kSortThreads) {
      const uint64_t key = s_key[i];
      uint32_t r = 0;
      for (uint32_t k = 0; k < m; ++k) r += s_key[k] > key ? 1u : 0u;
      emit(r, key);
    }
  } else {
    int n2 = 1;
    while ((uint32_t)n2 < m) n2 <<= 1;
    for (uint32_t i = m + tid; i < (uint32_t)n2; i += kSortThreads) s_key[i] = 0ull;
    __syncthreads();
    bitonic_desc(s_key, n2);
    for (uint32_t i = tid; i < m; i += kSortThreads) emit(i, s_key[i]);
  }
  if (tid == 0) {
    a.status[q] = s_bad | (a.scan_status ? (a.scan_status[q] & 7u) << 8 : 0u);
    if (a.out_counts) a.out_counts[q] = m - s_skip;
  }
}

// IndexEngine::query_filtered's ring merge (src/engine.rs:584-594): the ring
// hits, sorted descending, are pushed one by one into the query's Shortlist
// holding the scan hits (Shortlist::push, src/scan.rs:351-369), then
// into_sorted.  Pushing a descending sequence keeps the K largest of both
// lists where a ring hit never displaces an entry of equal score (push
// replaces the minimum only if strictly greater; below capacity it appends).
// So the result is the merge of the two sorted lists with the scan entry first
// on equal scores, cut at K.  Entry positions come from binary searches:
// scan entry i lands at i + #(ring > s_i), ring entry j at j + #(scan >= r_j).
__device__ __forceinline__ uint32_t count_greater(const float* v, uint32_t n, float x, bool or_equal) {
  uint32_t lo = 0, hi = n;  // v descending: first index whose value fails the test
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    const bool pass = or_equal ? (v[mid] >= x) : (v[mid] > x);
    if (pass) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kSortThreads) void k_ring_merge(RingMergeArgs a) {
  const uint32_t q = blockIdx.x;
  const uint64_t sb = (uint64_t)q * a.k, rb = (uint64_t)q * a.n_ring;
  const uint32_t c = a.counts[q];
  const bool ok = a.ring_status[q] == 0u;
  const uint32_t r = ok ? (a.n_ring < a.k ? a.n_ring : a.k) : 0u;  // search_exact truncates to top_k
  const float* ss = a.scores + sb;
  const float* rs = a.ring_scores + rb;
  for (uint32_t i = threadIdx.x; i < c; i += kSortThreads) {
    const uint32_t pos = i + count_greater(rs, r, ss[i], false);
    if (pos < a.k) {
      a.out_ids[sb + pos] = a.ids[sb + i];
      a.out_scores[sb + pos] = ss[i];
    }
  }
  for (uint32_t j = threadIdx.x; j < r; j += kSortThreads) {
    const uint32_t pos = j + count_greater(ss, c, rs[j], true);
    if (pos < a.k) {
      // VectorId::new(u32::MAX, local_i as u16)
      a.out_ids[sb + pos] = (0xffffffffull << 16) | (a.ring_rows[rb + j] & 0xffffull);
      a.out_scores[sb + pos] = rs[j];
    }
  }
  if (threadIdx.x == 0) a.out_counts[q] = (c + r < a.k) ? c + r : a.k;
}

template <typename K, typename... Args>
void launch(K kernel, dim3 grid, dim3 block, hipStream_t s, const LaunchEvents& ev, Args... args) {
  if (ev.start) hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ev.start, ev.stop, 0u, args...);
  else hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

}  // namespace

hipError_t launch_rerank_store(const float* rows, uint64_t n_rows, int precision, void* data, uint16_t* scales,
                               hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  const uint64_t wgs = (n_rows + 3) / 4;
  const dim3 grid((uint32_t)(wgs < 65536 ? wgs : 65536));
  uint8_t* d = static_cast<uint8_t*>(data);
  if (precision == MRL_RERANK_FP32)
    hipLaunchKernelGGL(k_store768<MRL_RERANK_FP32>, grid, dim3(kStoreThreads), 0, s, rows, d, scales, n_rows);
  else if (precision == MRL_RERANK_FP16)
    hipLaunchKernelGGL(k_store768<MRL_RERANK_FP16>, grid, dim3(kStoreThreads), 0, s, rows, d, scales, n_rows);
  else
    hipLaunchKernelGGL(k_store768<MRL_RERANK_INT8>, grid, dim3(kStoreThreads), 0, s, rows, d, scales, n_rows);
  return hipGetLastError();
}

hipError_t launch_ring_merge(const RingMergeArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_q == 0) return hipSuccess;
  launch(k_ring_merge, dim3(a.n_q), dim3(kSortThreads), s, ev, a);
  return hipGetLastError();
}

hipError_t launch_rerank(const RerankArgs& a, hipStream_t s, const LaunchEvents& ev_score,
                         const LaunchEvents& ev_sort) {
  if (a.n_q == 0 || a.stride == 0) return hipSuccess;
  if (a.dims == 768) {
    const uint32_t per = kScoreThreads / 8;
    const uint32_t n_chunks = (a.stride + per - 1) / per;
    const dim3 grid(n_chunks * a.n_q);
    if (a.precision == MRL_RERANK_FP32)
      launch(k_score768<MRL_RERANK_FP32>, grid, dim3(kScoreThreads), s, ev_score, a, n_chunks);
    else if (a.precision == MRL_RERANK_FP16)
      launch(k_score768<MRL_RERANK_FP16>, grid, dim3(kScoreThreads), s, ev_score, a, n_chunks);
    else
      launch(k_score768<MRL_RERANK_INT8>, grid, dim3(kScoreThreads), s, ev_score, a, n_chunks);
  } else {
    const uint32_t n_chunks = (a.stride + kScoreThreads - 1) / kScoreThreads;
    launch(k_score_seq, dim3(n_chunks * a.n_q), dim3(kScoreThreads), s, ev_score, a, n_chunks);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch(k_rerank_sort, dim3(a.n_q), dim3(kSortThreads), s, ev_sort, a);
  return hipGetLastError();
}

}  // namespace mrl
