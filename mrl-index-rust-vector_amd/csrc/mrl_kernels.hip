// mrl_kernels.hip -- gfx950 kernels for the PaxBlock64 progressive bitplane scan.
//
// Numerics: every f32 expression keeps the reference's operand order and is
// compiled with -ffp-contract=off (no fused multiply-add), correctly rounded
// division/sqrt and IEEE denormals, so per-vector scores are bit-identical to
// src/scan.rs.  Wave64 is the natural unit: the 64 slots of a PaxBlock64 map
// to the 64 lanes of a wavefront and a bitplane word is a lane mask.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mrl_half.h"
#include "mrl_internal.h"

#ifndef MRL_SCAN_AHEAD
#define MRL_SCAN_AHEAD 2  // blocks in flight per wave, one-query scan
#endif
constexpr uint32_t kRerunWorkgroups = 2048;  // total workgroups of a gated re-run launch
#ifndef MRL_SCAN_GRID1
#define MRL_SCAN_GRID1 512u  // workgroups of the one-query scan
#endif

namespace mrl {

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ bool lane_in(uint64_t mask) {
  return __builtin_amdgcn_inverse_ballot_w64(mask);
}

// Order-preserving map f32 -> u32 (larger score -> larger key); -0 == +0.
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  if ((u << 1) == 0u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_score(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// A +0.0f the optimiser cannot see through.  The AMDGPU backend folds
// `0 - x` into `-x` and `0 + x` into `x`, which differ from IEEE when x is a
// signed zero; every accumulator that the reference starts at 0.0 starts here.
__device__ __forceinline__ float zero_acc() {
  float z = 0.0f;
  asm volatile("" : "+v"(z));
  return z;
}

// SplitMix-style sign used by rotate.rs:53-67 (tail_rademacher) and
// eden.rs:75-88 (rademacher_diag).
__device__ __forceinline__ float mix_sign(uint64_t a, uint64_t i) {
  uint64_t x = (a * 0x9E3779B97F4A7C15ull + i) * 0xBF58476D1CE4E5B9ull;
  x ^= x >> 30;
  x = x * 0x94D049BB133111EBull;
  x ^= x >> 27;
  return (x & 1ull) == 0 ? 1.0f : -1.0f;
}

// Read-only views in the constant address space: uniform loads through them
// become scalar (SMEM) loads.  Only memory no kernel writes during a scan
// (device blocks, query plans) is read this way.
#define CONST_AS __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ const CONST_AS T* cview(const void* p) {
  return (const CONST_AS T*)(p);
}

struct Chunk8 {
  uint64_t p[8];
  float w[8];
};

// Plane words come from the block (scalar loads); weights from the LDS copy
// of the query's plan (every lane reads the same address).
__device__ __forceinline__ Chunk8 load_chunk8(const CONST_AS uint64_t* pl, const float* w) {
  Chunk8 c;
#pragma unroll
  for (int i = 0; i < 8; ++i) c.p[i] = pl[i];
  const float4* w4 = reinterpret_cast<const float4*>(w);
  const float4 a = w4[0], b = w4[1];
  c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
  c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
  return c;
}

// s += w[i] on the lanes whose bit is set in p[i] & m, for i = 0..7 in order
// (the asm saves and restores exec, so its only effect is its output and it
// is not volatile: loads of later chunks may be scheduled ahead of it):
// the reference's set-bit accumulation (scan.rs:553-562, 534-542, 618-627)
// with the bitplane word used directly as the wavefront's execution mask.
// Lanes not set keep s unchanged.  m is first restricted to the incoming
// exec mask, so no lane that was inactive on entry is ever enabled.
__device__ __forceinline__ float masked_add8(float s, uint64_t m, const Chunk8& c) {
  uint64_t sv, mm;
  asm(
      "s_mov_b64 %[sv], exec\n\t"
      "s_and_b64 %[mm], %[m], %[sv]\n\t"
      "s_and_b64 exec, %[p0], %[mm]\n\tv_add_f32 %[s], %[w0], %[s]\n\t"
      "s_and_b64 exec, %[p1], %[mm]\n\tv_add_f32 %[s], %[w1], %[s]\n\t"
      "s_and_b64 exec, %[p2], %[mm]\n\tv_add_f32 %[s], %[w2], %[s]\n\t"
      "s_and_b64 exec, %[p3], %[mm]\n\tv_add_f32 %[s], %[w3], %[s]\n\t"
      "s_and_b64 exec, %[p4], %[mm]\n\tv_add_f32 %[s], %[w4], %[s]\n\t"
      "s_and_b64 exec, %[p5], %[mm]\n\tv_add_f32 %[s], %[w5], %[s]\n\t"
      "s_and_b64 exec, %[p6], %[mm]\n\tv_add_f32 %[s], %[w6], %[s]\n\t"
      "s_and_b64 exec, %[p7], %[mm]\n\tv_add_f32 %[s], %[w7], %[s]\n\t"
      "s_mov_b64 exec, %[sv]"
      : [s] "+v"(s), [sv] "=&s"(sv), [mm] "=&s"(mm)
      : [m] "s"(m), [p0] "s"(c.p[0]), [p1] "s"(c.p[1]), [p2] "s"(c.p[2]), [p3] "s"(c.p[3]), [p4] "s"(c.p[4]),
        [p5] "s"(c.p[5]), [p6] "s"(c.p[6]), [p7] "s"(c.p[7]), [w0] "v"(c.w[0]), [w1] "v"(c.w[1]),
        [w2] "v"(c.w[2]), [w3] "v"(c.w[3]), [w4] "v"(c.w[4]), [w5] "v"(c.w[5]), [w6] "v"(c.w[6]),
        [w7] "v"(c.w[7])
      : "scc");
  return s;
}

// Sum over NCHUNK*8 dims with the next chunk's loads issued before the
// current chunk's adds.
template <int NCHUNK>
__device__ __forceinline__ float masked_accumulate(float s, uint64_t m, const CONST_AS uint64_t* planes,
                                                   const float* w) {
  Chunk8 cur = load_chunk8(planes, w);
#pragma unroll
  for (int c = 0; c < NCHUNK; ++c) {
    Chunk8 nxt;
    if (c + 1 < NCHUNK) nxt = load_chunk8(planes + 8 * (c + 1), w + 8 * (c + 1));
    s = masked_add8(s, m, cur);
    if (c + 1 < NCHUNK) cur = nxt;
  }
  return s;
}

// ---------------------------------------------------------------------------
// block re-layout (upload) and its inverse (download)
// one 64-lane workgroup per block; lane v owns slot v
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_relayout_to_device(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ dst, uint64_t n_blocks,
                                                          uint4* __restrict__ recs) {
  const uint32_t v = threadIdx.x;
  for (uint64_t b = blockIdx.x; b < n_blocks; b += gridDim.x) {
    const uint8_t* s = src + b * kBlockBytes;
    uint8_t* d = dst + b * kBlockBytes;
    if (v < 16) reinterpret_cast<uint32_t*>(d)[v] = reinterpret_cast<const uint32_t*>(s)[v];
    const uint8_t* m = s + kOrigMeta + 7 * v;
    reinterpret_cast<uint16_t*>(d + kDevScale)[v] = (uint16_t)(m[0] | (m[1] << 8));
    reinterpret_cast<uint16_t*>(d + kDevOffset)[v] = (uint16_t)(m[2] | (m[3] << 8));
    reinterpret_cast<uint16_t*>(d + kDevTail)[v] = (uint16_t)(m[4] | (m[5] << 8));
    d[kDevFlags + v] = m[6];
    const uint64_t* s0 = reinterpret_cast<const uint64_t*>(s + kOrigS0);
    const uint64_t* s2 = reinterpret_cast<const uint64_t*>(s + kOrigS2);
    const uint64_t* s3 = reinterpret_cast<const uint64_t*>(s + kOrigS3);
    const uint64_t* s5 = reinterpret_cast<const uint64_t*>(s + kOrigS5);
    uint32_t lw[8];
    for (int j = 0; j < 8; ++j) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i) {
        int dim = 8 * j + i;
        uint32_t lvl = (uint32_t)((s5[dim] >> v) & 1u) | ((uint32_t)((s3[dim] >> v) & 1u) << 1) |
                       ((uint32_t)((s2[dim] >> v) & 1u) << 2) | ((uint32_t)((s0[dim] >> v) & 1u) << 3);
        w |= lvl << (4 * i);
      }
      lw[j] = w;
      reinterpret_cast<uint32_t*>(d + kDevNibbles)[8 * v + j] = w;
    }
    const uint64_t* s1 = reinterpret_cast<const uint64_t*>(s + kOrigS1);
    const uint64_t* s4 = reinterpret_cast<const uint64_t*>(s + kOrigS4);
    uint64_t* d1 = reinterpret_cast<uint64_t*>(d + kDevS1);
    uint64_t* d4 = reinterpret_cast<uint64_t*>(d + kDevS4);
    d1[v] = s1[v];
    d1[v + 64] = s1[v + 64];
    d4[v] = s4[v];
    if (recs) {
      // slot v's record: its level words, then its own S1 / S4 bits (dword k
      // holds dims 32k..32k+31, bit i = dim 32k + i), then its meta
      uint32_t r[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const uint64_t* pl = k < 4 ? s1 + 32 * k : s4 + 32 * (k - 4);
        uint32_t w = 0;
        for (int i = 0; i < 32; ++i) w |= (uint32_t)((pl[i] >> v) & 1u) << i;
        r[k] = w;
      }
      uint4* rec = recs + (b * 64 + v) * kRecWords;
      rec[kRecLev0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
      rec[kRecLev1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
      rec[kRecS1] = make_uint4(r[0], r[1], r[2], r[3]);
      rec[kRecS4Meta] = make_uint4(r[4], r[5], (uint32_t)(m[0] | (m[1] << 8)) | ((uint32_t)(m[2] | (m[3] << 8)) << 16),
                                   (uint32_t)(m[4] | (m[5] << 8)) | ((uint32_t)m[6] << 16));
    }
  }
}

__global__ __launch_bounds__(64) void k_relayout_to_host(const uint8_t* __restrict__ src,
                                                        uint8_t* __restrict__ dst, uint64_t n_blocks) {
  const uint32_t v = threadIdx.x;
  for (uint64_t b = blockIdx.x; b < n_blocks; b += gridDim.x) {
    const uint8_t* s = src + b * kBlockBytes;
    uint8_t* d = dst + b * kBlockBytes;
    if (v < 16) reinterpret_cast<uint32_t*>(d)[v] = reinterpret_cast<const uint32_t*>(s)[v];
    uint16_t sc = reinterpret_cast<const uint16_t*>(s + kDevScale)[v];
    uint16_t of = reinterpret_cast<const uint16_t*>(s + kDevOffset)[v];
    uint16_t tl = reinterpret_cast<const uint16_t*>(s + kDevTail)[v];
    uint8_t* m = d + kOrigMeta + 7 * v;
    m[0] = (uint8_t)sc;
    m[1] = (uint8_t)(sc >> 8);
    m[2] = (uint8_t)of;
    m[3] = (uint8_t)(of >> 8);
    m[4] = (uint8_t)tl;
    m[5] = (uint8_t)(tl >> 8);
    m[6] = s[kDevFlags + v];
    // lane v rebuilds plane word `dim = v` of S0/S2/S3/S5 from the 64 slots
    const uint32_t* nib = reinterpret_cast<const uint32_t*>(s + kDevNibbles);
    const int dim = (int)v;
    uint64_t w0 = 0, w2 = 0, w3 = 0, w5 = 0;
    for (int slot = 0; slot < 64; ++slot) {
      uint32_t lvl = (nib[8 * slot + (dim >> 3)] >> (4 * (dim & 7))) & 15u;
      w5 |= (uint64_t)(lvl & 1u) << slot;
      w3 |= (uint64_t)((lvl >> 1) & 1u) << slot;
      w2 |= (uint64_t)((lvl >> 2) & 1u) << slot;
      w0 |= (uint64_t)((lvl >> 3) & 1u) << slot;
    }
    reinterpret_cast<uint64_t*>(d + kOrigS0)[dim] = w0;
    reinterpret_cast<uint64_t*>(d + kOrigS2)[dim] = w2;
    reinterpret_cast<uint64_t*>(d + kOrigS3)[dim] = w3;
    reinterpret_cast<uint64_t*>(d + kOrigS5)[dim] = w5;
    const uint64_t* s1 = reinterpret_cast<const uint64_t*>(s + kDevS1);
    const uint64_t* s4 = reinterpret_cast<const uint64_t*>(s + kDevS4);
    uint64_t* d1 = reinterpret_cast<uint64_t*>(d + kOrigS1);
    uint64_t* d4 = reinterpret_cast<uint64_t*>(d + kOrigS4);
    d1[v] = s1[v];
    d1[v + 64] = s1[v + 64];
    d4[v] = s4[v];
  }
}

// ---------------------------------------------------------------------------
// batched query plan: QueryPlan::from_query_codec (src/scan.rs:105-266)
// one 192-thread workgroup per query
// ---------------------------------------------------------------------------

// One FWHT butterfly stage of stride h < 64 (fwht_inplace, rotate.rs:13-33)
// over a vector held one element per lane: x + y at the lower index, x - y
// at the upper, the same f32 operations as the in-place loop.
__device__ __forceinline__ float fwht_lane(float v, int h, uint32_t lane) {
  const float o = __shfl_xor(v, h);
  return (lane & (uint32_t)h) ? o - v : v + o;
}

// acc + f(src[0]) + f(src[1]) + ... + f(src[n-1]), one f32 addition at a
// time in index order.  Two 16-term buffers alternate: the LDS reads of one
// go out before the additions of the other, so the chain runs at the adder's
// pace.  src is 16-byte aligned.
template <typename F>
__device__ __forceinline__ void add16(float& acc, const float4 (&c)[4], F f) {
#pragma unroll
  for (int u = 0; u < 4; ++u) acc = (((acc + f(c[u].x)) + f(c[u].y)) + f(c[u].z)) + f(c[u].w);
}
template <typename F>
__device__ __forceinline__ float chain_sum(float acc, const float* __restrict__ src, int n, F f) {
  const float4* s4 = reinterpret_cast<const float4*>(src);
  int i = 0;
  if (n >= 16) {
    float4 A[4], B[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) A[u] = s4[u];
#pragma unroll 1
    for (; i + 32 <= n; i += 32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) B[u] = s4[((i + 16) >> 2) + u];
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the additions
      add16(acc, A, f);
      // the chunk after B, or chunk 0 again (unused) past the last full one
      const int na = i + 48 <= n ? i + 32 : 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) A[u] = s4[(na >> 2) + u];
      __builtin_amdgcn_sched_barrier(0);
      add16(acc, B, f);
    }
    if (i + 16 <= n) {
      add16(acc, A, f);
      i += 16;
    }
  }
  for (; i < n; ++i) acc = acc + f(src[i]);
  return acc;
}

// Makes this wave's LDS writes visible to its own later reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Three waves per query, each on its own part after the query is in LDS
// (rotations are FWHTs across lanes with shuffles):
//  wave 0: the mid-band and folded-tail rotations, their fields and tables,
//          the sums over them and the S1 / S4 scan constants;
//  wave 1: q_tail_sq, the one long sum (dims - 192 terms);
//  wave 2: the prefix rotation, the prefix fields and LUT, the sums over the
//          raw query and the scalar fields.
// Each sum is a chain of f32 additions in the reference's order (scan.rs:
// 132-233, 528-531) whose terms are the reference's single rounded f32
// operations; `x -= y` is accumulated as `x + (-y)`, the same IEEE operation.
// The LDS of one query's plan for queries of at most MAXD dims.
template <int MAXD>
struct PlanLds {
  __align__(16) float q[MAXD];
  __align__(16) float sq[MAXD - kTailStart];
  __align__(16) float mid[128];
  __align__(16) float eden[64];
  __align__(16) float terms[9][128];
  float sums[11];
};

// One query's plan (plan record and scan constants) by threads 0..191 of the
// workgroup; every thread of the workgroup must call it (it has barriers).
template <int MAXD>
__device__ __forceinline__ void plan_body(const PlanArgs& a, uint32_t q, PlanLds<MAXD>& sh) {
  float* s_q = sh.q;
  float* s_sq = sh.sq;
  float* s_mid = sh.mid;
  float* s_eden = sh.eden;
  float (*s_terms)[128] = sh.terms;
  float* s_sums = sh.sums;
  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t lane = (uint32_t)t & 63u;
  const uint32_t dims = a.dims;
  const float* x = a.queries + (uint64_t)q * dims;
  mrl_query_plan* p = a.out + q;
  float* qd = a.luts + (uint64_t)q * kQData;
  const bool has_eden = a.eden_mean != nullptr;
  const bool has_mid = a.mid_mean != nullptr;
  const bool eden_codec = a.prefix_codec == MRL_PREFIX_EDEN_PROD;
  const bool has_tail = dims > (uint32_t)kTailStart;
  const int tail_n = has_tail ? (int)dims - kTailStart : 0;
  const float rs = a.c.rabitq_scale;
  const float ts = a.c.tail_fold_scale;
  const float c0 = has_mid ? a.c.eden_mid_codebook[0] : 0.0f;
  const float c1 = has_mid ? a.c.eden_mid_codebook[1] : 0.0f;

  // four loads in flight per thread (index clamped), then the stores
  for (uint32_t i0 = t; t < 192 && i0 < dims; i0 += 4u * 192u) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t i = i0 + 192u * (uint32_t)k;
      v[k] = x[i < dims ? i : dims - 1u];
    }
    // (the empty asm keeps the compiler from sinking a load into its store's branch)
#pragma unroll
    for (int k = 0; k < 4; ++k) asm volatile("" : "+v"(v[k]));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t i = i0 + 192u * (uint32_t)k;
      if (i < dims) s_q[i] = v[k];
    }
  }
  __syncthreads();

  if (wave >= 3) {
    // (a wider workgroup's other waves only meet the barriers)
  } else if (wave == 1) {
    // q_tail_sq: the squares formed by every lane, then the chain on one
    for (int i = (int)lane; i < tail_n; i += 64) s_sq[i] = s_q[kTailStart + i] * s_q[kTailStart + i];
    wave_lds_sync();
    if (lane == 0) s_sums[4] = chain_sum(zero_acc(), s_sq, tail_n, [](float v) { return v; });
  } else if (wave == 2) {
    // rotate_query of the prefix (eden.rs:91-98, 275-281)
    const float v = s_q[lane];
    float d = has_eden ? v * mix_sign(a.eden_seed, (uint64_t)lane) : 0.0f;
#pragma unroll
    for (int h = 1; h < 64; h *= 2) d = fwht_lane(d, h, lane);
    d *= a.c.inv_sqrt64;
    s_eden[lane] = d;
    p->prefix[lane] = v;
    p->bit_weights[lane][0] = v * 1.0f;
    p->bit_weights[lane][1] = v * 2.0f;
    p->bit_weights[lane][2] = v * 4.0f;
    p->bit_weights[lane][3] = v * 8.0f;
    p->eden_q_rot[lane] = d;
    p->prefix_weight[lane] = eden_codec ? d * a.c.inv_sqrt64 : v;  // scan.rs:457-461
    // terms of prefix_l1, prefix_sum, eden_mean_ip (64) and eden_mid_mean_ip, q_mid_sq (128)
    const float em = has_eden ? a.eden_mean[lane] : 0.0f;
    const float mm0 = has_mid ? a.mid_mean[lane] : 0.0f;
    const float mm1 = has_mid ? a.mid_mean[64 + lane] : 0.0f;
    const float mv0 = s_q[64 + lane], mv1 = s_q[128 + lane];
    s_terms[0][lane] = fabsf(v);
    s_terms[1][lane] = v;
    s_terms[2][lane] = has_eden ? v * em : 0.0f;
    s_terms[3][lane] = has_mid ? mv0 * mm0 : 0.0f;
    s_terms[3][64 + lane] = has_mid ? mv1 * mm1 : 0.0f;
    s_terms[4][lane] = mv0 * mv0;
    s_terms[4][64 + lane] = mv1 * mv1;
    // squared prefix norm, for the histogram scale only (any summation order)
    float psq = v * v;
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) psq += __shfl_xor(psq, h);
    if (lane == 0) s_sums[10] = psq;
    if (lane < 16) p->eden_codebook[lane] = has_eden ? a.c.eden_codebook[lane] : 0.0f;
    if (lane < 27) p->pad[lane] = 0.0f;
    if (lane == 0) {
      p->dims = dims;
      p->prefix_codec = a.prefix_codec;
      p->mid_codec = a.mid_codec;
      p->has_tail_fold = has_tail ? 1u : 0u;
      p->eden_inv_sqrt_d = a.c.inv_sqrt64;
      p->eden_mid_inv_sqrt_d = a.c.inv_sqrt128;
      p->eden_mid_codebook[0] = c0;
      p->eden_mid_codebook[1] = c1;
      p->rabitq_scale = rs;
    }
    // the unused tail; every address is written once, with its final value,
    // so a fused pass may read it while other workgroups still write it
    static_assert(kQdHistInv == kQdU4 + 1 && kQdHistScale == kQdU4 + 2, "scan constant layout");
    for (int e = kQdHistScale + 1 + (int)lane; e < kQData; e += 64) qd[e] = 0.0f;
    wave_lds_sync();
    // Prefix LUT: lut[d*16 + level] = codebook[level] * weight[d] (or
    // level * weight[d]), the product scan.rs:476-484 forms per (d, level).
    // Entry e = lane + 64 k has level lane & 15 for every k: one codebook
    // read per lane (an indexed read of the kernel argument array).
    const float cb = eden_codec ? a.c.eden_codebook[lane & 15u] : (float)(lane & 15u);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int dd = (int)(lane >> 4) + 4 * k;
      const float w = eden_codec ? s_eden[dd] * a.c.inv_sqrt64 : s_q[dd];
      qd[kQdLut + (int)lane + 64 * k] = cb * w;
    }
    if (lane < 5) {
      const int n = lane < 3 ? 64 : 128;
      const float sum = chain_sum(zero_acc(), s_terms[lane], n, [](float v) { return v; });
      s_sums[lane < 4 ? lane : 5] = sum;  // q_mid_sq is sum 5
    }
  } else {
    // rotate_query = diag(+-1) then FWHT (eden.rs:91-98, 275-281); fold_tail
    // (rotate.rs:73-93).  Lane l holds elements l and l + 64 of the 128-dim
    // rotations and element l of the folded tail.
    float m0 = s_q[64 + lane], m1 = s_q[128 + lane];
    float e0 = has_mid ? m0 * mix_sign(a.mid_seed, (uint64_t)lane) : 0.0f;
    float e1 = has_mid ? m1 * mix_sign(a.mid_seed, (uint64_t)lane + 64u) : 0.0f;
    float u = zero_acc();
    if (has_tail) {
      int nb = tail_n / 64;
      if (nb > kTailFoldBlocks) nb = kTailFoldBlocks;
      for (int b = 0; b < nb; ++b) u += mix_sign((uint64_t)b, (uint64_t)lane) * s_q[kTailStart + 64 * b + lane];
    }
#pragma unroll
    for (int h = 1; h < 64; h *= 2) {
      m0 = fwht_lane(m0, h, lane);
      m1 = fwht_lane(m1, h, lane);
      e0 = fwht_lane(e0, h, lane);
      e1 = fwht_lane(e1, h, lane);
      u = fwht_lane(u, h, lane);
    }
    {
      const float a0 = m0, b0 = e0;
      m0 = a0 + m1;
      m1 = a0 - m1;
      e0 = b0 + e1;
      e1 = b0 - e1;
    }
    m0 *= a.c.inv_sqrt128;
    m1 *= a.c.inv_sqrt128;
    e0 *= a.c.inv_sqrt128;
    e1 *= a.c.inv_sqrt128;
    u *= a.c.inv_sqrt64;
    s_mid[lane] = m0;
    s_mid[64 + lane] = m1;

    // elementwise fields
    const float tq = has_tail ? u : 0.0f;
    p->tail_fold_q[lane] = tq;
    const float w4 = has_tail ? 2.0f * (tq * ts) : 0.0f;
    p->tail_fold_weights2[lane] = w4;
    qd[kQdW4 + lane] = w4;
    float w1[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t i = lane + 64u * r;
      const float rq = r ? m1 : m0, eq = r ? e1 : e0;
      p->rabitq_q[i] = rq;
      p->rabitq_weights2[i] = 2.0f * (rq * rs);
      p->eden_mid_q_rot[i] = eq;
      // scan.rs:528-532 (deltas) with eden_mid_inv_sqrt_d = 1/sqrt(128)
      const float dl = (c1 - c0) * (eq * a.c.inv_sqrt128);
      p->eden_mid_deltas[i] = dl;
      w1[r] = a.mid_codec == MRL_MID_EDEN_B1 ? dl : 2.0f * (rq * rs);
      qd[kQdW1 + i] = w1[r];
      s_terms[5][i] = -(rq * rs);                          // rabitq_base
      s_terms[8][i] = c0 * (eq * a.c.inv_sqrt128);         // eden_mid_base
    }
    const float pos = u * ts;
    s_terms[6][lane] = has_tail ? -pos : 0.0f;             // tail_fold_base
    s_terms[7][lane] = has_tail ? fabsf(pos) : 0.0f;       // s4_abs_budget
    wave_lds_sync();
    // rabitq_lut (scan.rs:188-201): 512 entries
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = (int)lane + 64 * k;
      const int g = e >> 4, mask = e & 15;
      const float p0 = s_mid[4 * g] * rs, p1 = s_mid[4 * g + 1] * rs;
      const float p2 = s_mid[4 * g + 2] * rs, p3 = s_mid[4 * g + 3] * rs;
      const float v0 = (mask & 1) ? p0 : -p0;
      const float v1 = (mask & 2) ? p1 : -p1;
      const float v2 = (mask & 4) ? p2 : -p2;
      const float v3 = (mask & 8) ? p3 : -p3;
      p->rabitq_lut[g][mask] = v0 + v1 + v2 + v3;
    }
    // rabitq_base, tail_fold_base, s4_abs_budget, eden_mid_base on lanes 0..3
    float sum = 0.0f;
    if (lane < 4) {
      const int row = 5 + (int)lane;
      sum = chain_sum(zero_acc(), s_terms[row], lane == 1 || lane == 2 ? 64 : 128, [](float v) { return v; });
      s_sums[6 + lane] = sum;
    }
    // upper ends of the S1 / S4 sums: base + positive weights
    float pw1 = fmaxf(w1[0], 0.0f) + fmaxf(w1[1], 0.0f);
    float pw4 = fmaxf(w4, 0.0f);
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
      pw1 += __shfl_xor(pw1, h);
      pw4 += __shfl_xor(pw4, h);
    }
    const float base1 = __shfl(sum, 0), base4 = __shfl(sum, 1);
    if (lane == 0) {
      qd[kQdU1] = base1 + pw1;  // rabitq_base + positive rabitq_weights2
      qd[kQdU4] = base4 + pw4;  // tail_fold_base + positive tail weights
    }
  }
  __syncthreads();
  if (t == 0) {
    p->prefix_l1 = s_sums[0];
    p->prefix_sum = s_sums[1];
    p->eden_mean_ip = s_sums[2];
    p->eden_mid_mean_ip = s_sums[3];
    p->rabitq_base = s_sums[6];
    p->tail_fold_base = s_sums[7];
    p->s4_abs_budget = s_sums[8];
    p->eden_mid_base = s_sums[9];
    const float tail_sq = s_sums[4], mid_sq = s_sums[5];
    const float qt = sqrtf(tail_sq);
    p->q_tail_norm = qt;
    p->q_mid_norm = sqrtf(mid_sq);
    p->q_after_prefix = sqrtf(mid_sq + tail_sq);
    p->q_after_s1 = qt;
    // histogram scale: e = round(log2 |q|), clamped to [-60, 60]
    const float nrm = sqrtf(s_sums[10] + mid_sq + tail_sq);
    int e = 0;
    if (nrm > 0.0f && nrm - nrm == 0.0f) {
      int ex;
      const float mant = frexpf(nrm, &ex);  // nrm = mant * 2^ex, mant in [0.5, 1)
      e = mant >= 0.70710678f ? ex : ex - 1;
      e = e < -60 ? -60 : (e > 60 ? 60 : e);
    }
    qd[kQdHistInv] = ldexpf(1.0f, -e);
    qd[kQdHistScale] = ldexpf(1.0f, e);
  }
}

__global__ __launch_bounds__(192) void k_plan(PlanArgs a) {
  __shared__ PlanLds<MRL_MAX_DIMS> sh;
  plan_body<MRL_MAX_DIMS>(a, blockIdx.x, sh);
}

// ---------------------------------------------------------------------------
// strata scan
// ---------------------------------------------------------------------------

struct LaneBlock {
  float scale, offset, tail, mid_n, high_n;
  uint32_t nib[8];
};

// L0Only (src/scan.rs:753-790): the sign plane alone (bit 3 of every level),
// then the MinMax4 prefix formula whatever the codec.  accum_plane skips
// weight == 0, and adding a zero weight never changes a sum that started at +0.
__device__ __forceinline__ uint64_t eval_block_l0(uint64_t active, const LaneBlock& m,
                                                 const CONST_AS mrl_query_plan* p, const ScanParams& sp,
                                                 float tau, float& prefix_ip_out, float& score_out,
                                                 uint64_t* masks) {
  float cd = zero_acc();
#pragma unroll
  for (int d = 0; d < 64; ++d) {
    float w = p->bit_weights[d][3];
    bool bit = (m.nib[d >> 3] >> (4 * (d & 7) + 3)) & 1u;
    float nx = cd + w;
    cd = bit ? nx : cd;
  }
  float prefix_ip = cd * m.scale + m.offset * p->prefix_sum;
  float x_rest = fmaxf(m.tail, 0.0f);
  float ub = prefix_ip + sp.alpha * p->q_after_prefix * x_rest;
  uint64_t surv = ballot(ub >= tau) & active;
  masks[1] = masks[2] = masks[3] = masks[4] = surv;
  prefix_ip_out = prefix_ip;
  score_out = prefix_ip;
  return surv;
}

// Byte offset of the LUT entry of dim 8j+i inside dim-group j's 16 entries:
// level * 4.  From w2 = w << 2 and w3 = w >> 2, byte k of w2 holds level 2k
// in bits 2..5 and byte k of w3 holds level 2k+1 there, so each offset is one
// byte extract and mask.
// byte B of w, masked with m: one SDWA v_and_b32 (byte select of src0).
template <int B>
__device__ __forceinline__ uint32_t and_byte(uint32_t w, uint32_t m) {
  uint32_t r;
  if constexpr (B == 0)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
        : "=v"(r) : "v"(w), "v"(m));
  else if constexpr (B == 1)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:DWORD"
        : "=v"(r) : "v"(w), "v"(m));
  else if constexpr (B == 2)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:DWORD"
        : "=v"(r) : "v"(w), "v"(m));
  else
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:DWORD"
        : "=v"(r) : "v"(w), "v"(m));
  return r;
}

template <int I>
__device__ __forceinline__ uint32_t lut_off(uint32_t w2, uint32_t w3, uint32_t m) {
  return and_byte<I / 2>((I & 1) ? w3 : w2, m);
}

// Tighter admissible bounds for the stage checks.  When the reference's own
// bounds are admissible (alpha >= 1 and 2.4 * w_s4 <= alpha: every bound then
// dominates the score still to come, so its top K is the exact top K by full
// score), any bound on the full score gives the same top K.  The RaBitQ sum
// s1 = base + (set weights) lies in [base + negative weights, base + positive
// weights], and likewise the folded-tail sum, so with mid_n > 0 and hn > 0
//   full score <= prefix_ip + U1 * mid_n + U4 * w_s4 * hn   (U = base + positive weights),
// and after S1, score <= score + U4 * w_s4 * hn.  The float evaluation is
// covered by a relative margin of 2^-8 on the remainder and 2^-20 * (|x| + 1)
// on the sum (the sums run over at most 128 terms).  tight_coef() returns,
// from the plan kernel's U1 and U4, A = U1 (1 + 2^-8) and B = U4 w_s4 (1 + 2^-8)
// (B = 0 without a tail stage),
// or A = NaN where the reference's checks are kept: EdenB1 mid-band, other
// alpha / w_s4, or non-finite coefficients.
constexpr float kTightMargin = 1.0f / 1048576.0f;

__device__ __forceinline__ void tight_coef(float u1_raw, float u4_raw, bool eden_b1, bool has_tail, bool full,
                                           const ScanParams& sp, float* A, float* B) {
  const float u1 = u1_raw * (1.0f + 1.0f / 256.0f);
  const float u4 = (full && has_tail) ? u4_raw * sp.w_s4 * (1.0f + 1.0f / 256.0f) : 0.0f;
  const bool ok = !eden_b1 && sp.alpha >= 1.0f && sp.w_s4 >= 0.0f && 2.4f * sp.w_s4 <= sp.alpha &&
                  sp.strata != MRL_STRATA_L0_ONLY && u1 - u1 == 0.0f && u4 - u4 == 0.0f;
  *A = ok ? fmaxf(u1, 0.0f) : __builtin_nanf("");
  *B = fmaxf(u4, 0.0f);
}

// Bound before the S1 stage: the tight one when A is a number, else the reference's.
__device__ __forceinline__ float prefix_bound(float prefix_ip, float mid_n, float high_n, float A, float B,
                                              float alpha, float q_mid, float q_tail) {
  const float hn = fmaxf(high_n, 1e-6f);
  return A == A ? prefix_ip + (A * mid_n + B * hn) + kTightMargin * (fabsf(prefix_ip) + 1.0f)
                : prefix_ip + alpha * (q_mid * mid_n + q_tail * high_n);
}
__device__ __forceinline__ float s1_bound(float score, float high_n, float A, float B, float alpha, float q_after) {
  const float hn = fmaxf(high_n, 1e-6f);
  return A == A ? score + B * hn + kTightMargin * (fabsf(score) + 1.0f) : score + alpha * q_after * high_n;
}

// Stage: 4-bit prefix IP (scan.rs:453-517).  lut[d*16 + level] holds the
// reference's product codebook[level] * weight (or level * weight), so the
// per-vector sum over d is the same sequence of f32 additions.
template <bool READS_FIRST = false>
__device__ __forceinline__ float prefix_acc(const LaneBlock& m, const float* __restrict__ lut) {
  float acc = zero_acc();
  const char* lutb = reinterpret_cast<const char*>(lut);
  const uint32_t mask = 0x3Cu;
  auto ld = [&](int d, uint32_t off) { return *reinterpret_cast<const float*>(lutb + d * 64 + off); };
  if constexpr (!READS_FIRST) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w2 = m.nib[j] << 2, w3 = m.nib[j] >> 2;
      acc = acc + ld(8 * j + 0, lut_off<0>(w2, w3, mask));
      acc = acc + ld(8 * j + 1, lut_off<1>(w2, w3, mask));
      acc = acc + ld(8 * j + 2, lut_off<2>(w2, w3, mask));
      acc = acc + ld(8 * j + 3, lut_off<3>(w2, w3, mask));
      acc = acc + ld(8 * j + 4, lut_off<4>(w2, w3, mask));
      acc = acc + ld(8 * j + 5, lut_off<5>(w2, w3, mask));
      acc = acc + ld(8 * j + 6, lut_off<6>(w2, w3, mask));
      acc = acc + ld(8 * j + 7, lut_off<7>(w2, w3, mask));
    }
    return acc;
  }
  // All 64 table reads are independent: issue them before the first
  // addition so their LDS latency overlaps (the additions keep their order).
  // Costs ~36 VGPRs, which only the one-query kernel (two waves per SIMD)
  // can spare.
  float v[64];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w2 = m.nib[j] << 2, w3 = m.nib[j] >> 2;
    v[8 * j + 0] = ld(8 * j + 0, lut_off<0>(w2, w3, mask));
    v[8 * j + 1] = ld(8 * j + 1, lut_off<1>(w2, w3, mask));
    v[8 * j + 2] = ld(8 * j + 2, lut_off<2>(w2, w3, mask));
    v[8 * j + 3] = ld(8 * j + 3, lut_off<3>(w2, w3, mask));
    v[8 * j + 4] = ld(8 * j + 4, lut_off<4>(w2, w3, mask));
    v[8 * j + 5] = ld(8 * j + 5, lut_off<5>(w2, w3, mask));
    v[8 * j + 6] = ld(8 * j + 6, lut_off<6>(w2, w3, mask));
    v[8 * j + 7] = ld(8 * j + 7, lut_off<7>(w2, w3, mask));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < 64; ++d) acc = acc + v[d];
  return acc;
}

// One (block, query) evaluation: the stage functions of src/scan.rs:453-634
// composed as run_default_scan_kernel (654-691).  Returns the pushed-survivor
// mask; score/prefix_ip are this lane's values.
__device__ __forceinline__ uint64_t eval_block(const CONST_AS uint8_t* blk, uint64_t active,
                                              const LaneBlock& m, const float* __restrict__ lut,
                                              const float* __restrict__ w_mid, const float* __restrict__ w_tail,
                                              const CONST_AS mrl_query_plan* p, const ScanParams& sp,
                                              float tau, float& prefix_ip_out, float& score_out,
                                              uint64_t* masks, float tA, float tB) {
  const float alpha = sp.alpha;
  const float acc = prefix_acc(m, lut);
  const bool eden = p->prefix_codec == MRL_PREFIX_EDEN_PROD;
  float prefix_ip = eden ? p->eden_mean_ip + m.scale * acc : acc * m.scale + m.offset * p->prefix_sum;
  float score = prefix_ip;
  float ub = prefix_bound(prefix_ip, m.mid_n, m.high_n, tA, tB, alpha, p->q_mid_norm, p->q_tail_norm);
  uint64_t surv = ballot(ub >= tau) & active;
  masks[1] = masks[2] = masks[3] = surv;
  prefix_ip_out = prefix_ip;

  const bool rabitq = sp.strata == MRL_STRATA_L1_RABITQ || sp.strata == MRL_STRATA_FULL64B;
  const bool full = sp.strata == MRL_STRATA_FULL64B;
  if (surv != 0 && rabitq) {
    // Stage: mid-band 1-bit IP (scan.rs:520-569), set bits added in d order.
    const CONST_AS uint64_t* s1p = (const CONST_AS uint64_t*)(blk + kDevS1);
    const bool b1 = p->mid_codec == MRL_MID_EDEN_B1;
    float s1 = masked_accumulate<16>(b1 ? p->eden_mid_base : p->rabitq_base, surv, s1p, w_mid);
    score = b1 ? score + (p->eden_mid_mean_ip + m.offset * s1) : score + s1 * m.mid_n;
    // Stage: post-S1 CS (scan.rs:572-584)
    float ub2 = s1_bound(score, m.high_n, tA, tB, alpha, p->q_after_s1);
    surv &= ballot(ub2 >= tau);
    masks[2] = masks[3] = surv;
  }
  if (surv != 0 && full) {
    const float hn = fmaxf(m.high_n, 1e-6f);
    const float w_s4 = sp.w_s4;
    // Stage: S4 abs-budget prune (scan.rs:587-607)
    if (p->has_tail_fold && p->s4_abs_budget > 0.0f) {
      float ub3 = score + alpha * hn * w_s4 * p->s4_abs_budget;
      surv &= ballot(ub3 >= tau);
    }
    masks[3] = surv;
    // Stage: folded-tail 1-bit IP (scan.rs:610-634)
    if (surv != 0 && p->has_tail_fold) {
      const CONST_AS uint64_t* s4p = (const CONST_AS uint64_t*)(blk + kDevS4);
      float s4 = masked_accumulate<8>(p->tail_fold_base, surv, s4p, w_tail);
      score = score + s4 * hn * w_s4;
    }
  }
  masks[4] = surv;
  score_out = score;
  return surv;
}

// Histogram bin of an appended score (monotone non-decreasing in s): the
// score times the query's power-of-two histogram scale inv = 2^-e (exact
// unless it underflows, and monotone either way), then 512 bins per unit over
// [-2, 2).
__device__ __forceinline__ uint32_t hist_bin(float s, float inv) {
  float x = (s * inv + 2.0f) * 512.0f;
  x = fminf(fmaxf(x, 0.0f), (float)(kHistBins - 1));
  return (uint32_t)x;
}

// A float t with: hist_bin(s) >= b  implies  s >= t.  (For b >= 1, the
// rounding of s + 2 near the edge is below 2^-22, far inside the 1e-6 margin.)
__device__ __forceinline__ float bin_floor(uint32_t b) {
  if (b == 0) return -INFINITY;
  const double t = (double)b / 512.0 - 2.0 - 1e-6;
  float f = (float)t;
  if ((double)f > t) {  // one ulp toward -inf
    uint32_t u = __float_as_uint(f);
    if (f > 0.0f) u -= 1u;
    else if (f == 0.0f) u = 0x80000001u;
    else u += 1u;
    f = __uint_as_float(u);
  }
  return f;
}
// The floor of bin b for a query of histogram scale 2^e (scale = 2^e): an
// exact power-of-two multiple of bin_floor(b), whose magnitude stays in the
// normal range for |e| <= 60.  hist_bin(s, 2^-e) >= b implies s * 2^-e >=
// bin_floor(b) (when s * 2^-e underflows, |s * 2^-e| < 2^-126 lies above
// every finite bin floor), so s >= bin_floor(b) * 2^e.
__device__ __forceinline__ float bin_floor(uint32_t b, float scale) { return bin_floor(b) * scale; }

// One wave: the bin floor of the need-th best count of a histogram (-inf
// when it holds fewer than need).  Lane l holds bins 32(63-l) .. +31, so the
// lane order is descending in score.
struct HistRow {
  uint4 v[8];
};
__device__ __forceinline__ HistRow hist_row(const uint32_t* h) {
  const uint4* p = reinterpret_cast<const uint4*>(h + (63u - __lane_id()) * 32u);
  HistRow r;
#pragma unroll
  for (int k = 0; k < 8; ++k) r.v[k] = p[k];
  return r;
}
__device__ float floor_of(const HistRow& r, uint32_t need) {
  const uint32_t lane = __lane_id();
  const uint32_t seg = 63u - lane;
  uint32_t c[32];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    c[4 * k] = r.v[k].x;
    c[4 * k + 1] = r.v[k].y;
    c[4 * k + 2] = r.v[k].z;
    c[4 * k + 3] = r.v[k].w;
  }
  uint32_t part = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) part += c[i];
  uint32_t incl = part;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off);
    if ((int)lane >= off) incl += o;
  }
  const uint32_t excl = incl - part;
  const uint64_t hm = __ballot(excl < need && incl >= need);
  if (hm == 0) return -INFINITY;
  const uint32_t src = (uint32_t)__ffsll((long long)hm) - 1;
  uint32_t bin = 0, before = excl;
  bool found = false;
#pragma unroll
  for (int i = 31; i >= 0; --i) {
    before += c[i];
    if (!found && before >= need) {
      bin = seg * 32u + (uint32_t)i;
      found = true;
    }
  }
  bin = __shfl(bin, (int)src);
  return bin_floor(bin);
}
__device__ float wave_floor(const uint32_t* h, uint32_t need) { return floor_of(hist_row(h), need); }

// Per-lane raw inputs of one block, loaded one block ahead.  Lane l < 4 of
// `hdr` holds header dword {0, 1, 4, 5}[l]: min_ts, max_ts and the two halves
// of the tombstone mask.  t14 holds this lane's 24 bytes of the S1/S4 planes;
// the scan reads those planes with scalar loads, the vector loads here only
// bring them into L2 ahead of use.
struct RawLane {
  uint16_t scale, offset, tail;
  uint32_t flags;
  uint32_t nib[8];
  uint32_t hdr;
  uint4 t1;
  uint2 t4;
};

template <bool PLANES = true>
__device__ __forceinline__ RawLane load_raw(const uint8_t* blk) {
  RawLane r;
  const uint32_t lane = __lane_id();
  r.scale = reinterpret_cast<const uint16_t*>(blk + kDevScale)[lane];
  r.offset = reinterpret_cast<const uint16_t*>(blk + kDevOffset)[lane];
  r.tail = reinterpret_cast<const uint16_t*>(blk + kDevTail)[lane];
  r.flags = blk[kDevFlags + lane];
  const uint4* nibq = reinterpret_cast<const uint4*>(blk + kDevNibbles) + 2 * lane;
  const uint4 n0 = nibq[0], n1 = nibq[1];
  r.nib[0] = n0.x;
  r.nib[1] = n0.y;
  r.nib[2] = n0.z;
  r.nib[3] = n0.w;
  r.nib[4] = n1.x;
  r.nib[5] = n1.y;
  r.nib[6] = n1.z;
  r.nib[7] = n1.w;
  const uint32_t hw = lane < 2 ? lane : (lane < 4 ? lane + 2 : 0);
  r.hdr = reinterpret_cast<const uint32_t*>(blk)[hw];
  if constexpr (PLANES) {
    r.t1 = reinterpret_cast<const uint4*>(blk + kDevS1)[lane];
    r.t4 = reinterpret_cast<const uint2*>(blk + kDevS4)[lane];
  } else {
    r.t1 = make_uint4(0u, 0u, 0u, 0u);
    r.t4 = make_uint2(0u, 0u);
  }
  return r;
}

// Keeps the L2 warm-up loads alive without using their values.
__device__ __forceinline__ void retire_touch(const RawLane& r) {
  asm volatile("" ::"v"(r.t1.x), "v"(r.t1.y), "v"(r.t1.z), "v"(r.t1.w), "v"(r.t4.x), "v"(r.t4.y));
}

// Prologue of a scan workgroup: the floor of each of its queries.  In the
// final pass it comes from the sampling histogram at floor_rank; the safe
// floor (rank safe_rank) is taken too, and workgroup x = 0 of each query tile
// writes both out for k_select.  Otherwise it is tau (or -inf).  Wave w
// takes work items w, w + 4, ... (two per query).
// The histogram row of a wave's first item, loaded at the start of the prologue.
__device__ __forceinline__ HistRow floor_prefetch(const ScanArgs& a, uint32_t q0, int nq, int wave) {
  HistRow r{};
  if (a.floor_hist && wave < 2 * nq) r = hist_row(a.floor_hist + (uint64_t)(q0 + (wave >> 1)) * kHistBins);
  return r;
}

template <int QT>
__device__ __forceinline__ void take_floors(const ScanArgs& a, uint32_t q0, int nq, int wave, uint32_t lane,
                                            float* s_floor, const HistRow& first) {
  if (a.floor_hist) {
    for (int it = wave; it < 2 * nq; it += 4) {
      const int qi = it >> 1;
      const bool safe = it & 1;
      const uint32_t need = safe ? a.safe_rank : a.floor_rank;
      const float sc = a.luts[(uint64_t)(q0 + qi) * kQData + kQdHistScale];
      const float f = (it == wave ? floor_of(first, need)
                                  : wave_floor(a.floor_hist + (uint64_t)(q0 + qi) * kHistBins, need)) * sc;
      if (lane == 0) {
        if (!safe) s_floor[qi] = f;
        if (blockIdx.x == 0) (safe ? a.safe_out : a.floor_out)[q0 + qi] = f;
      }
    }
  } else if ((int)threadIdx.x < nq) {
    s_floor[threadIdx.x] = a.tau ? a.tau[q0 + threadIdx.x] : -INFINITY;
  }
}

// Appends of one workgroup are staged here per query and flushed at the end.
template <int QT>
struct Staging {
  static constexpr int kCap = QT == 1 ? 1024 : 1024 / QT;
  float score[QT][kCap];
  uint32_t row[QT][kCap];
  uint32_t n[QT];
  uint32_t gbase[QT];
};

// Appends (score, row) for the lanes in pm: into the LDS staging area while
// it has room, directly into the query's global segment otherwise (one
// global atomic per wave for the lanes that overflow).
template <int QT>
__device__ __forceinline__ void stage_append(Staging<QT>& st, const ScanArgs& a, int qi, uint32_t q, uint32_t seg,
                                             uint64_t pm, float score, uint32_t row) {
  const uint32_t lane = __lane_id();
  const uint32_t lead = (uint32_t)__ffsll((long long)pm) - 1;
  uint32_t base = 0;
  if (lane == lead) base = atomicAdd(&st.n[qi], (uint32_t)__popcll(pm));
  base = __shfl(base, (int)lead);
  const bool mine = (pm >> lane) & 1ull;
  const uint32_t slot = base + lanes_below(pm);
  if (mine && slot < (uint32_t)Staging<QT>::kCap) {
    st.score[qi][slot] = score;
    st.row[qi][slot] = row;
  }
  const uint64_t om = ballot(mine && slot >= (uint32_t)Staging<QT>::kCap);
  if (om != 0 && !a.excl) {  // an exclusive segment only counts them (its count then overflows)
    const uint64_t sq = (uint64_t)q * a.nseg + seg;
    const uint32_t olead = (uint32_t)__ffsll((long long)om) - 1;
    uint32_t g0 = 0;
    if (lane == olead) g0 = atomicAdd(a.seg_count + sq, (uint32_t)__popcll(om));
    g0 = __shfl(g0, (int)olead);
    const uint32_t g = g0 + lanes_below(om);
    if (((om >> lane) & 1ull) && g < a.seg_cap) {
      a.cand_score[sq * a.seg_cap + g] = score;
      a.cand_row[sq * a.seg_cap + g] = row;
    }
  }
}

// End of a scan workgroup: one global atomic per (workgroup, query) reserves
// space in the query's segment, then the staged appends are copied out.
template <int QT, bool DIAG>
__device__ __forceinline__ void flush_appends(Staging<DIAG ? 1 : QT>& st, const ScanArgs& a, uint32_t q0, int nq,
                                              uint32_t seg, const unsigned int* s_stats) {
  if constexpr (!DIAG) {
    const int tid = threadIdx.x;
    __syncthreads();
    if (tid < nq) {
      const uint32_t n = min(st.n[tid], (uint32_t)Staging<QT>::kCap);
      const uint64_t sq = (uint64_t)(q0 + tid) * a.nseg + seg;
      if (a.excl) {  // this workgroup's own segment: every append counted, from 0
        a.seg_count[sq] = st.n[tid];
        st.gbase[tid] = 0u;
      } else {
        st.gbase[tid] = n ? atomicAdd(a.seg_count + sq, n) : 0u;
      }
    }
    if (a.stats && tid < kStatCount && s_stats[tid]) {
      const uint32_t copy = (blockIdx.x + blockIdx.y * gridDim.x) % (uint32_t)kStatCopies;
      atomicAdd(a.stats + copy * kStatCount + tid, (unsigned long long)s_stats[tid]);
    }
    __syncthreads();
    for (int qi = 0; qi < nq; ++qi) {
      const uint32_t n = min(st.n[qi], (uint32_t)Staging<QT>::kCap);
      const uint32_t g0 = st.gbase[qi];
      const uint64_t sq = (uint64_t)(q0 + qi) * a.nseg + seg;
      for (uint32_t i = tid; i < n; i += 256) {
        const uint32_t g = g0 + i;
        if (g < a.seg_cap) {
          a.cand_score[sq * a.seg_cap + g] = st.score[qi][i];
          a.cand_row[sq * a.seg_cap + g] = st.row[qi][i];
        }
      }
    }
  }
}

// One-query scans defer the S1 / S4 stages: the prefix stage's survivors of
// each block wait in a per-wave queue, and once 64 are queued they are
// finished together with lane = survivor, from each slot's own S1 / S4 bits
// (its record).  A survivor's stage sums are the same additions in the same
// order as the exec-masked form (a clear bit adds -0.0, which leaves every
// value unchanged, as skipping it does).
struct DeferQ {
  uint32_t row[64];
  float score[64];  // prefix_ip
  float mid_n[64];
  float high_n[64];
  float offset[64];
};

// w where bit k of word is set, else -0.0
__device__ __forceinline__ float bit_weight(uint32_t word, int k, float w) {
  const uint32_t m = (uint32_t)((int32_t)(word << (31 - k)) >> 31);
  return __uint_as_float((__float_as_uint(w) & m) | (0x80000000u & ~m));
}

// s + the weights of the set bits of a row, in dim order (NW dwords = 32 NW dims)
template <int NW>
__device__ __forceinline__ float row_sum(float s, const uint32_t (&bits)[NW], const float* __restrict__ w) {
#pragma unroll
  for (int c = 0; c < NW * 8; ++c) {
    const float4 w4 = reinterpret_cast<const float4*>(w)[c];
    const uint32_t word = bits[c >> 3];
    const int k0 = (c & 7) * 4;
    s = s + bit_weight(word, k0, w4.x);
    s = s + bit_weight(word, k0 + 1, w4.y);
    s = s + bit_weight(word, k0 + 2, w4.z);
    s = s + bit_weight(word, k0 + 3, w4.w);
  }
  return s;
}

// Finishes the qn queued survivors of this wave: S1, post-S1 check, S4
// budget and S4 (scan.rs:520-634), then the push (or, in a sampling pass,
// the score count).
__device__ __forceinline__ void defer_flush(const DeferQ& dq, uint32_t qn, const ScanArgs& a,
                                         const CONST_AS mrl_query_plan* p, const float* __restrict__ w1,
                                         const float* __restrict__ w4, float tA, float tB, float tq, float tau,
                                         Staging<1>& st, uint32_t q, uint32_t seg, uint32_t* s_hist,
                                         unsigned int* s_stats, float hinv) {
  const uint32_t lane = __lane_id();
  const ScanParams& sp = a.sp;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool have = lane < qn;
  uint32_t row = 0;
  float score = 0.0f, mid_n = 1e-6f, high_n = 0.0f, offset = 0.0f;
  uint4 r1 = make_uint4(0u, 0u, 0u, 0u);
  uint2 r4 = make_uint2(0u, 0u);
  if (have) {
    row = dq.row[lane];
    score = dq.score[lane];
    mid_n = dq.mid_n[lane];
    high_n = dq.high_n[lane];
    offset = dq.offset[lane];
    const uint4* rec = a.recs + (uint64_t)row * kRecWords;
    r1 = rec[kRecS1];
    const uint4 x = rec[kRecS4Meta];
    r4 = make_uint2(x.x, x.y);
  }
  const bool b1 = p->mid_codec == MRL_MID_EDEN_B1;
  const uint32_t bits1[4] = {r1.x, r1.y, r1.z, r1.w};
  const float s1 = row_sum<4>(b1 ? p->eden_mid_base : p->rabitq_base, bits1, w1);
  score = b1 ? score + (p->eden_mid_mean_ip + offset * s1) : score + s1 * mid_n;
  // Stage: post-S1 CS (scan.rs:572-584)
  bool keep = have && s1_bound(score, high_n, tA, tB, sp.alpha, p->q_after_s1) >= tau;
  const uint64_t k1 = ballot(keep);
  uint64_t k3 = k1;
  if (sp.strata == MRL_STRATA_FULL64B && k1 != 0) {
    const float hn = fmaxf(high_n, 1e-6f);
    // Stage: S4 abs-budget prune (scan.rs:587-607)
    if (p->has_tail_fold && p->s4_abs_budget > 0.0f)
      keep = keep && score + sp.alpha * hn * sp.w_s4 * p->s4_abs_budget >= tau;
    k3 = ballot(keep);
    // Stage: folded-tail 1-bit IP (scan.rs:610-634)
    if (k3 != 0 && p->has_tail_fold) {
      const uint32_t bits4[2] = {r4.x, r4.y};
      const float s4 = row_sum<2>(p->tail_fold_base, bits4, w4);
      score = keep ? score + s4 * hn * sp.w_s4 : score;
    }
  }
  if (a.stats && lane == 0) {
    atomicAdd(&s_stats[kStatS1], (unsigned)__popcll(k1));
    atomicAdd(&s_stats[kStatS4Budget], (unsigned)__popcll(k3));
    atomicAdd(&s_stats[kStatPushed], (unsigned)__popcll(k3));
  }
  if (a.hist) {
    if (keep) atomicAdd(&s_hist[hist_bin(score, hinv)], 1u);
  } else {
    if (ballot(keep && score != score) != 0 && lane == 0) atomicOr(a.err + q, 1u);
    const uint64_t pm = ballot(keep && score >= tq);
    if (pm != 0) stage_append<1>(st, a, 0, q, seg, pm, score, row);
  }
}

// One pass of the strata scan.  Workgroup = 4 waves; wave = one block at a
// time (lane v = slot v), blocks pos = first + k * stride of the pass order.
// QT queries share each block's loads.  L0 selects the L0Only stage set.
// FUSE (one query, a sampling pass): the workgroup first builds the query's
// plan itself (plan_body, the work of k_plan); every workgroup writes the same
// plan record and scan constants, and each reads them only after its own
// writes, so the pass needs no separate plan launch.
template <int QT, bool DIAG, bool L0, bool FUSE = false>
__global__ __launch_bounds__(256) void k_scan(ScanArgs a) {
  static_assert(!FUSE || (QT == 1 && !DIAG && !L0), "the plan is fused into one-query scans only");
  if constexpr (FUSE) {
    __shared__ PlanLds<kFuseMaxDims> s_pl;
    plan_body<kFuseMaxDims>(a.plan, blockIdx.y, s_pl);
    __syncthreads();
  }
  __shared__ __align__(16) float s_qd[L0 ? 1 : QT * kQData];  // scan constants of each query
  __shared__ float s_rho[256];
  __shared__ float s_midf[256];
  __shared__ unsigned int s_stats[kStatCount];
  __shared__ Staging<DIAG ? 1 : QT> s_app;
  constexpr bool kLdsHist = QT == 1 && !DIAG;  // sampling-pass counts gathered per workgroup
  __shared__ uint32_t s_hist[kLdsHist ? kHistBins : 1];
  __shared__ float s_floor[QT];
  __shared__ float s_hinv[QT];  // histogram scale of each query (2^-e)
  __shared__ float s_tight[QT][2];
  constexpr bool DEFER = QT == 1 && !DIAG && !L0;  // S1 / S4 through the per-wave survivor queue
  __shared__ DeferQ s_dq[DEFER ? 4 : 1];

  const int tid = threadIdx.x;
  const uint32_t q0 = blockIdx.y * QT;
  const int nq = (int)min((uint32_t)QT, a.n_q - q0);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lane = lane_id();
  // gated re-run (QT == 1): only a query its final selection flagged
  if (QT == 1 && a.gate && (a.gate[q0] & 4u) == 0u) return;

  // This wave's blocks: positions pos = first + k * stride of the pass.  The
  // stride is odd (one wave of the grid stays idle), so the positions of a
  // wave run through every residue modulo the power-of-two pass ratio and the
  // blocks an earlier pass already scored are spread evenly over the waves.
  // The first block's loads are issued before the LDS set-up below.
  const uint32_t stride = gridDim.x * 4 - 1;
  const uint32_t first = blockIdx.x * 4 + wave;
  const uint32_t cover = a.prev_shift >= 0 ? (1u << a.prev_shift) - 1u : 0u;
  // position -> block: pos << shift, or this query tile's block list
  const uint32_t* bl = a.blist ? a.blist + (uint64_t)blockIdx.y * a.blist_stride : nullptr;
  const uint32_t n_pos = first < stride ? (bl ? a.bcount[blockIdx.y] : a.n_pos) : 0u;
  auto block_of = [&](uint32_t pos) -> uint32_t { return bl ? bl[pos] : pos << a.shift; };
  uint32_t b_cur = first < n_pos ? block_of(first) : 0u;
  RawLane cur;
  // The set-up's reads go out first (memory returns loads in order, so the
  // set-up below then waits for them alone), then the first blocks' loads.
  const HistRow fl = floor_prefetch(a, q0, nq, wave);
  constexpr int kQdPer = L0 ? 1 : (QT * (kQData / 4) + 255) / 256;  // float4 per thread
  float4 qdv[kQdPer];
  if (!L0) {
    // unconditional loads (the index clamped to the last element): the
    // values stay in registers and no wait lands before the block loads
    const float4* src = reinterpret_cast<const float4*>(a.luts + (uint64_t)q0 * kQData);
    const int lim = nq * (kQData / 4);
#pragma unroll
    for (int k = 0; k < kQdPer; ++k) {
      const int e = tid + 256 * k;
      qdv[k] = src[e < lim ? e : lim - 1];
    }
  }
  const float fr0 = a.flag_tabs[tid], fr1 = a.flag_tabs[256 + tid];
  float tu1 = 0.0f, tu4 = 0.0f, hinv = 1.0f;
  int t_b1 = 0, t_tail = 0;
  if (!DIAG && tid < nq) hinv = a.luts[(uint64_t)(q0 + tid) * kQData + kQdHistInv];
  if (!DIAG && !L0 && tid < nq) {
    const float* qd = a.luts + (uint64_t)(q0 + tid) * kQData;
    const mrl_query_plan* pq = a.plans + q0 + tid;
    tu1 = qd[kQdU1];
    tu4 = qd[kQdU4];
    t_b1 = pq->mid_codec == MRL_MID_EDEN_B1;
    t_tail = pq->has_tail_fold != 0;
  }
  if (first < n_pos) cur = load_raw<!DEFER>(a.idx + (uint64_t)b_cur * kBlockBytes);
  // DEFER keeps kAhead blocks in flight: the loads of the following ones go out now too
  constexpr int kAhead = DEFER ? MRL_SCAN_AHEAD : 1;
  uint32_t b_pf[kAhead > 1 ? kAhead - 1 : 1];
  RawLane pf[kAhead > 1 ? kAhead - 1 : 1];
#pragma unroll
  for (int k = 0; k + 1 < kAhead; ++k) {
    const uint32_t pk = first + (uint32_t)(k + 1) * stride;
    b_pf[k] = pk < n_pos ? block_of(pk) : b_cur;
    if (first < n_pos) pf[k] = load_raw<false>(a.idx + (uint64_t)b_pf[k] * kBlockBytes);
  }

  if (tid < kStatCount) s_stats[tid] = 0u;
  if (tid < QT) s_app.n[tid] = 0u;
  if (!L0) {  // one contiguous copy of each query's scan constants
    float4* dst = reinterpret_cast<float4*>(s_qd);
#pragma unroll
    for (int k = 0; k < kQdPer; ++k) {
      const int e = tid + 256 * k;
      if (e < nq * (kQData / 4)) dst[e] = qdv[k];
    }
  }
  s_rho[tid] = fr0;
  s_midf[tid] = fr1;
  if (tid < nq) s_hinv[tid] = hinv;
  if (kLdsHist && a.hist)
    for (int i = tid; i < kHistBins; i += 256) s_hist[i] = 0u;
  if (!DIAG && !L0 && tid < nq) {  // diagnostic scans keep the reference's checks
    float A, B;
    tight_coef(tu1, tu4, t_b1, t_tail, a.sp.strata == MRL_STRATA_FULL64B, a.sp, &A, &B);
    s_tight[tid][0] = A;
    s_tight[tid][1] = B;
  }
  // Per-query floor: from the sampling histogram (final pass), else tau.
  take_floors<QT>(a, q0, nq, wave, lane, s_floor, fl);
  __syncthreads();

  const ScanParams sp = a.sp;
  const uint32_t seg = blockIdx.x % a.nseg;
  uint32_t qn = 0;  // survivors in this wave's queue (DEFER)
  // The one-query prefix stage's constants, read once before the block loop
  // (the loop's stores would otherwise make the compiler reload them per block).
  bool d_eden = false;
  float d_mean = 0.0f, d_psum = 0.0f, d_qmid = 0.0f, d_qtail = 0.0f, d_tq = 0.0f, d_tA = 0.0f, d_tB = 0.0f;
  float d_hinv = 1.0f;
  if constexpr (DEFER) {
    const CONST_AS mrl_query_plan* p = cview<mrl_query_plan>(a.plans + q0);
    d_eden = p->prefix_codec == MRL_PREFIX_EDEN_PROD;
    d_mean = p->eden_mean_ip;
    d_psum = p->prefix_sum;
    d_qmid = p->q_mid_norm;
    d_qtail = p->q_tail_norm;
    d_tq = s_floor[0];
    d_tA = s_tight[0][0];
    d_tB = s_tight[0][1];
    d_hinv = s_hinv[0];
    // (through an empty asm: held in registers, not re-read from the plan)
    asm volatile("" : "+s"(d_mean), "+s"(d_psum), "+s"(d_qmid), "+s"(d_qtail));
  }

  // Every wave reaches the flush barrier below, also one with no block.
  for (uint32_t pos = first; pos < n_pos; pos += stride) {
    // Prefetch the next block of this wave.  Past the end the current block
    // is loaded again, so the loads are unconditional and the wait before
    // this block's compute covers only this block's own loads.
    const uint32_t ahead = (uint32_t)kAhead * stride;
    const uint32_t b_nxt = pos + ahead < n_pos ? block_of(pos + ahead) : b_cur;
    const RawLane nxt = load_raw<!DEFER>(a.idx + (uint64_t)b_nxt * kBlockBytes);

    const uint32_t b = b_cur;
    const CONST_AS uint8_t* blk = cview<uint8_t>(a.idx + (uint64_t)b * kBlockBytes);
    // readlane returns int: widen through uint32_t (no sign extension)
    const uint32_t min_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 0);
    const uint32_t max_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 1);
    const uint64_t tomb = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 3) << 32) |
                          (uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 2);
    bool skip = false;
    if (sp.temporal) {  // scan.rs:719-730
      if (sp.has_lo && max_ts < sp.lo) skip = true;
      if (sp.has_hi && min_ts > sp.hi) skip = true;
    }
    const uint64_t active = ~tomb;
    const bool covered = a.prev_shift >= 0 && (b & cover) == 0u;  // scanned by an earlier pass
    if (covered) {
      // the block belongs to an earlier pass
    } else if (skip || active == 0) {
      if (DIAG) {
        for (int qi = 0; qi < nq; ++qi) {
          uint64_t o = ((uint64_t)(q0 + qi) * a.n_blocks + b);
          if (lane < 5) a.d_masks[o * 5 + lane] = 0;
          a.d_prefix[o * 64 + lane] = 0.0f;
          a.d_score[o * 64 + lane] = 0.0f;
        }
      }
    } else {
      // per-lane meta decode (block.rs:61-99)
      LaneBlock m;
      m.scale = h2f(cur.scale);
      m.offset = h2f(cur.offset);
      m.tail = h2f(cur.tail);
      const float t = fmaxf(m.tail, 0.0f);
      m.mid_n = fmaxf(s_midf[cur.flags] * t, 1e-6f);
      m.high_n = fmaxf(s_rho[cur.flags] * t, 0.0f);
#pragma unroll
      for (int j = 0; j < 8; ++j) m.nib[j] = cur.nib[j];

      const uint32_t n_active = (uint32_t)__popcll(active);
      if constexpr (DEFER) {
        // prefix stage here; survivors join the queue for S1 / S4
        const CONST_AS mrl_query_plan* p = cview<mrl_query_plan>(a.plans + q0);
        const float tq = d_tq;
        const float tau = sp.exhaustive ? -INFINITY : tq;
        const float acc = prefix_acc<true>(m, s_qd + kQdLut);
        const float prefix_ip = d_eden ? d_mean + m.scale * acc : acc * m.scale + m.offset * d_psum;
        const float ub = prefix_bound(prefix_ip, m.mid_n, m.high_n, d_tA, d_tB, sp.alpha, d_qmid, d_qtail);
        const uint64_t surv = ballot(ub >= tau) & active;
        if (a.stats && lane == 0) {
          atomicAdd(&s_stats[kStatBlocks], 1u);
          atomicAdd(&s_stats[kStatActive], n_active);
          atomicAdd(&s_stats[kStatPrefix], (unsigned)__popcll(surv));
        }
        if (surv != 0) {
          const uint32_t n = (uint32_t)__popcll(surv);
          if (qn + n > 64u) {
            defer_flush(s_dq[wave], qn, a, p, s_qd + kQdW1, s_qd + kQdW4, d_tA, d_tB, tq, tau, s_app, q0, seg,
                        s_hist, s_stats, d_hinv);
            qn = 0;
          }
          if ((surv >> lane) & 1ull) {
            const uint32_t slot = qn + lanes_below(surv);
            DeferQ& dq = s_dq[wave];
            dq.row[slot] = b * 64u + lane;
            dq.score[slot] = prefix_ip;
            dq.mid_n[slot] = m.mid_n;
            dq.high_n[slot] = m.high_n;
            dq.offset[slot] = m.offset;
          }
          qn += n;
        }
      } else
#pragma unroll 1
      for (int qi = 0; qi < nq; ++qi) {
        const uint32_t q = q0 + qi;
        const CONST_AS mrl_query_plan* p = cview<mrl_query_plan>(a.plans + q);
        const float tq = s_floor[qi];
        const float tau = sp.exhaustive ? -INFINITY : tq;
        uint64_t masks[5];
        masks[0] = active;
        float prefix_ip, score;
        uint64_t surv;
        if constexpr (L0) {
          surv = eval_block_l0(active, m, p, sp, tau, prefix_ip, score, masks);
        } else {
          // Re-derive the block pointer opaquely per query so the plane-word
          // loads stay inside this loop (hoisted, 192 words would not fit in SGPRs).
          uint64_t blk_bits = (uint64_t)blk;
          asm volatile("" : "+s"(blk_bits));
          const CONST_AS uint8_t* blk_q = (const CONST_AS uint8_t*)blk_bits;
          // the diagnostic path keeps the reference's checks (its masks are compared)
          const float tA = DIAG ? __builtin_nanf("") : s_tight[qi][0];
          const float tB = DIAG ? 0.0f : s_tight[qi][1];
          const float* qd = s_qd + qi * kQData;
          surv = eval_block(blk_q, active, m, qd + kQdLut, qd + kQdW1, qd + kQdW4, p, sp, tau, prefix_ip, score, masks,
                            tA, tB);
        }
        if constexpr (DIAG) {
          uint64_t o = ((uint64_t)q * a.n_blocks + b);
          if (lane < 5) {
            uint64_t mv = lane == 0 ? masks[0] : lane == 1 ? masks[1] : lane == 2 ? masks[2] : lane == 3 ? masks[3] : masks[4];
            a.d_masks[o * 5 + lane] = mv;
          }
          a.d_prefix[o * 64 + lane] = prefix_ip;
          a.d_score[o * 64 + lane] = score;
        } else {
          if (a.stats && lane == 0) {
            atomicAdd(&s_stats[kStatBlocks], 1u);
            atomicAdd(&s_stats[kStatActive], n_active);
            atomicAdd(&s_stats[kStatPrefix], (unsigned)__popcll(masks[1]));
            atomicAdd(&s_stats[kStatS1], (unsigned)__popcll(masks[2]));
            atomicAdd(&s_stats[kStatS4Budget], (unsigned)__popcll(masks[3]));
            atomicAdd(&s_stats[kStatPushed], (unsigned)__popcll(surv));
          }
          const bool mine = (surv >> lane) & 1ull;
          if (a.hist) {
            // sampling pass: count the survivors' exact scores
            if (mine) {
              if constexpr (kLdsHist) atomicAdd(&s_hist[hist_bin(score, s_hinv[qi])], 1u);
              else atomicAdd(a.hist + (uint64_t)q * kHistBins + hist_bin(score, s_hinv[qi]), 1u);
            }
          } else {
            if (ballot(mine && score != score) != 0 && lane == 0) atomicOr(a.err + q, 1u);
            // Append survivors whose score can still reach the top K.
            const uint64_t pm = ballot(mine && score >= tq);
            if (pm != 0) stage_append<QT>(s_app, a, qi, q, seg, pm, score, b * 64u + lane);
          }
        }
      }
    }
    if constexpr (!DEFER) retire_touch(cur);
    if constexpr (kAhead > 1) {
      cur = pf[0];
      b_cur = b_pf[0];
#pragma unroll
      for (int k = 0; k + 2 < kAhead; ++k) {
        pf[k] = pf[k + 1];
        b_pf[k] = b_pf[k + 1];
      }
      pf[kAhead - 2] = nxt;
      b_pf[kAhead - 2] = b_nxt;
    } else {
      cur = nxt;
      b_cur = b_nxt;
    }
  }
  if constexpr (DEFER) {
    if (qn != 0)
      defer_flush(s_dq[wave], qn, a, cview<mrl_query_plan>(a.plans + q0), s_qd + kQdW1, s_qd + kQdW4, s_tight[0][0],
                  s_tight[0][1], s_floor[0], sp.exhaustive ? -INFINITY : s_floor[0], s_app, q0, seg, s_hist, s_stats,
                  s_hinv[0]);
  }
  flush_appends<QT, DIAG>(s_app, a, q0, nq, seg, s_stats);
  if (kLdsHist && a.hist) {
    __syncthreads();
    for (int i = tid; i < kHistBins; i += 256) {
      const uint32_t c = s_hist[i];
      if (c) atomicAdd(a.hist + (uint64_t)q0 * kHistBins + i, c);
    }
  }
}

// ---------------------------------------------------------------------------
// batched scan: one block against a tile of QT queries at a time
// ---------------------------------------------------------------------------
// The stages of src/scan.rs:453-634 for QT (4 or 8) queries per block,
// ordered dim outer / query inner so that each per-lane load or mask is
// shared by the tile's queries.  Every sum keeps the reference's order per
// (vector, query):
//  - prefix: one byte extract gives the level offset of a dim; the LUT holds
//    the tile's products of that (dim, level) side by side, read as 16-byte
//    LDS loads of 4 queries;
//  - S1/S4: the plane word of a dim (from the block's prefetched plane words)
//    becomes the execution mask and the tile's weights are added under it.  These sums run for every active lane; a lane takes part in a
//    query's stage only through that query's survivor mask, so a survivor's
//    sum is the reference's and other lanes are never pushed.

// s[i] += w[i] on the lanes set in p (and in the incoming execution mask).
__device__ __forceinline__ void masked_add_tile(float (&s)[8], uint64_t p, const float4* w) {
  uint64_t sv;
  const float4 wa = w[0], wb = w[1];
  asm(
      "s_mov_b64 %[sv], exec\n\t"
      "s_and_b64 exec, %[p], %[sv]\n\t"
      "v_add_f32 %[s0], %[w0], %[s0]\n\t"
      "v_add_f32 %[s1], %[w1], %[s1]\n\t"
      "v_add_f32 %[s2], %[w2], %[s2]\n\t"
      "v_add_f32 %[s3], %[w3], %[s3]\n\t"
      "v_add_f32 %[s4], %[w4], %[s4]\n\t"
      "v_add_f32 %[s5], %[w5], %[s5]\n\t"
      "v_add_f32 %[s6], %[w6], %[s6]\n\t"
      "v_add_f32 %[s7], %[w7], %[s7]\n\t"
      "s_mov_b64 exec, %[sv]"
      : [s0] "+v"(s[0]), [s1] "+v"(s[1]), [s2] "+v"(s[2]), [s3] "+v"(s[3]), [s4] "+v"(s[4]), [s5] "+v"(s[5]),
        [s6] "+v"(s[6]), [s7] "+v"(s[7]), [sv] "=&s"(sv)
      : [p] "s"(p), [w0] "v"(wa.x), [w1] "v"(wa.y), [w2] "v"(wa.z), [w3] "v"(wa.w), [w4] "v"(wb.x),
        [w5] "v"(wb.y), [w6] "v"(wb.z), [w7] "v"(wb.w)
      : "scc");
}
__device__ __forceinline__ void masked_add_tile(float (&s)[4], uint64_t p, const float4* w) {
  uint64_t sv;
  const float4 wa = w[0];
  asm(
      "s_mov_b64 %[sv], exec\n\t"
      "s_and_b64 exec, %[p], %[sv]\n\t"
      "v_add_f32 %[s0], %[w0], %[s0]\n\t"
      "v_add_f32 %[s1], %[w1], %[s1]\n\t"
      "v_add_f32 %[s2], %[w2], %[s2]\n\t"
      "v_add_f32 %[s3], %[w3], %[s3]\n\t"
      "s_mov_b64 exec, %[sv]"
      : [s0] "+v"(s[0]), [s1] "+v"(s[1]), [s2] "+v"(s[2]), [s3] "+v"(s[3]), [sv] "=&s"(sv)
      : [p] "s"(p), [w0] "v"(wa.x), [w1] "v"(wa.y), [w2] "v"(wa.z), [w3] "v"(wa.w)
      : "scc");
}

// Plane word d of a 128-word plane held as uint4 per lane (lane l: dwords
// 4l..4l+3), or of a 64-word plane held as uint2 per lane.
__device__ __forceinline__ uint64_t plane_word128(const uint4& t, int d) {
  const int l = d >> 1;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((d & 1) ? t.z : t.x, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((d & 1) ? t.w : t.y, l);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t plane_word64(const uint2& t, int d) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane(t.x, d);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane(t.y, d);
  return ((uint64_t)hi << 32) | lo;
}

// Per-query constants of the tile kernel, one 16-float record per query in
// LDS (read as broadcasts, so they occupy no scalar registers).
enum {
  kQcEden = 0,      // prefix codec is EdenProd (1.0) or MinMax4 (0.0)
  kQcMeanIp,        // eden_mean_ip
  kQcPrefixSum,     // prefix_sum
  kQcMidNorm,       // q_mid_norm
  kQcTailNorm,      // q_tail_norm
  kQcTauPrune,      // pruning threshold (-inf when exhaustive)
  kQcTauPush,       // candidate floor
  kQcB1,            // mid codec is EdenB1 (1.0)
  kQcS1Base,        // eden_mid_base or rabitq_base
  kQcMidMeanIp,     // eden_mid_mean_ip
  kQcAfterS1,       // q_after_s1
  kQcHasTail,       // has_tail_fold (1.0)
  kQcBudget,        // s4_abs_budget
  kQcTailBase,      // tail_fold_base
  kQcTightA,        // tight bound coefficients (NaN: the reference's checks)
  kQcTightB,
  kQcCount = 16
};

template <int QT, bool FULL>
__global__ __launch_bounds__(256) void k_scan_tile(ScanArgs a) {
  static_assert(QT == 4 || QT == 8, "tile of 4 or 8 queries");
  constexpr int NG = QT / 4;  // float4 groups per (dim, level)
  // LUT: ((g * 64 + d) * 16 + level) * 4 + j holds query 4g + j's entry of (d, level)
  __shared__ __align__(16) float s_lut[QT * 1024];
  __shared__ __align__(16) float s_w1[128 * QT];  // [d][q]: rabitq_weights2 or eden_mid_deltas
  __shared__ __align__(16) float s_w4[64 * QT];   // [d][q]: tail_fold_weights2
  __shared__ __align__(16) float s_qc[QT * kQcCount];
  __shared__ unsigned int s_stats[kStatCount];
  __shared__ Staging<QT> s_app;
  __shared__ float s_floor[QT];
  __shared__ float s_hinv[QT];  // histogram scale of each query (2^-e)

  const int tid = threadIdx.x;
  const uint32_t q0 = blockIdx.y * QT;
  const int nq = (int)min((uint32_t)QT, a.n_q - q0);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lane = lane_id();

  const uint32_t stride = gridDim.x * 4 - 1;  // odd: see k_scan
  const uint32_t first = blockIdx.x * 4 + wave;
  const uint32_t cover = a.prev_shift >= 0 ? (1u << a.prev_shift) - 1u : 0u;
  const uint32_t* bl = a.blist ? a.blist + (uint64_t)blockIdx.y * a.blist_stride : nullptr;
  const uint32_t n_pos = first < stride ? (bl ? a.bcount[blockIdx.y] : a.n_pos) : 0u;
  auto block_of = [&](uint32_t pos) -> uint32_t { return bl ? bl[pos] : pos << a.shift; };
  uint32_t b_cur = first < n_pos ? block_of(first) : 0u;
  RawLane cur;
  if (first < n_pos) cur = load_raw(a.idx + (uint64_t)b_cur * kBlockBytes);
  const HistRow fl = floor_prefetch(a, q0, nq, wave);

  const ScanParams sp = a.sp;
  if (tid < kStatCount) s_stats[tid] = 0u;
  if (tid < QT) s_app.n[tid] = 0u;
  for (int e = tid; e < QT * 1024; e += 256) {
    const int j = e & 3, l = (e >> 2) & 15, d = (e >> 6) & 63, g = e >> 12;
    const int qi = 4 * g + j;
    s_lut[e] = qi < nq ? a.luts[(uint64_t)(q0 + qi) * kQData + kQdLut + d * 16 + l] : 0.0f;
  }
  for (int e = tid; e < 192 * QT; e += 256) {
    const int qi = e % QT, d = e / QT;
    float w = 0.0f;
    if (qi < nq) w = a.luts[(uint64_t)(q0 + qi) * kQData + (d < 128 ? kQdW1 + d : kQdW4 + d - 128)];
    if (d < 128) s_w1[e] = w;
    else s_w4[e - 128 * QT] = w;
  }
  if (tid < nq) s_hinv[tid] = a.luts[(uint64_t)(q0 + tid) * kQData + kQdHistInv];
  take_floors<QT>(a, q0, nq, wave, lane, s_floor, fl);
  __syncthreads();
  if (tid < QT) {
    const int qi = tid;
    float* c = s_qc + qi * kQcCount;
    // the tight-bound slots of present queries are written by the loop below
    for (int i = 0; i < kQcCount; ++i)
      if (qi >= nq || (i != kQcTightA && i != kQcTightB)) c[i] = 0.0f;
    c[kQcTauPrune] = __builtin_nanf("");  // absent query: no lane ever survives
    if (qi < nq) {
      const mrl_query_plan* pq = a.plans + q0 + qi;
      const float tq = s_floor[qi];
      const bool b1 = pq->mid_codec == MRL_MID_EDEN_B1;
      c[kQcEden] = pq->prefix_codec == MRL_PREFIX_EDEN_PROD ? 1.0f : 0.0f;
      c[kQcMeanIp] = pq->eden_mean_ip;
      c[kQcPrefixSum] = pq->prefix_sum;
      c[kQcMidNorm] = pq->q_mid_norm;
      c[kQcTailNorm] = pq->q_tail_norm;
      c[kQcTauPrune] = sp.exhaustive ? -INFINITY : tq;
      c[kQcTauPush] = tq;
      c[kQcB1] = b1 ? 1.0f : 0.0f;
      c[kQcS1Base] = b1 ? pq->eden_mid_base : pq->rabitq_base;
      c[kQcMidMeanIp] = pq->eden_mid_mean_ip;
      c[kQcAfterS1] = pq->q_after_s1;
      c[kQcHasTail] = pq->has_tail_fold ? 1.0f : 0.0f;
      c[kQcBudget] = pq->s4_abs_budget;
      c[kQcTailBase] = pq->tail_fold_base;
    }
  }
  if (tid < nq) {
    const float* qd = a.luts + (uint64_t)(q0 + tid) * kQData;
    const mrl_query_plan* pq = a.plans + q0 + tid;
    float A, B;
    tight_coef(qd[kQdU1], qd[kQdU4], pq->mid_codec == MRL_MID_EDEN_B1, pq->has_tail_fold != 0, FULL, a.sp, &A, &B);
    s_qc[tid * kQcCount + kQcTightA] = A;
    s_qc[tid * kQcCount + kQcTightB] = B;
  }
  __syncthreads();

  const float alpha = sp.alpha;
  const uint32_t seg = blockIdx.x % a.nseg;
  const char* lutb = reinterpret_cast<const char*>(s_lut);
  const float4* w1 = reinterpret_cast<const float4*>(s_w1);
  const float4* w4 = reinterpret_cast<const float4*>(s_w4);
  const float4* qc4 = reinterpret_cast<const float4*>(s_qc);
  // ScanStats of this wave, summed over its blocks and the tile's queries
  uint32_t c_blocks = 0, c_active = 0, c_prefix = 0, c_s1 = 0, c_s4b = 0;

  for (uint32_t pos = first; pos < n_pos; pos += stride) {
    const uint32_t b_nxt = pos + stride < n_pos ? block_of(pos + stride) : b_cur;
    const RawLane nxt = load_raw(a.idx + (uint64_t)b_nxt * kBlockBytes);
    const uint32_t b = b_cur;
    const uint32_t min_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 0);
    const uint32_t max_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 1);
    const uint64_t tomb = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 3) << 32) |
                          (uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 2);
    bool skip = false;
    if (sp.temporal) {  // scan.rs:719-730
      if (sp.has_lo && max_ts < sp.lo) skip = true;
      if (sp.has_hi && min_ts > sp.hi) skip = true;
    }
    const uint64_t active = ~tomb;
    const bool covered = a.prev_shift >= 0 && (b & cover) == 0u;
    if (!covered && !skip && active != 0) {
      // per-lane meta decode (block.rs:61-99)
      // rho = flags / 255 and sqrt(max(1 - rho^2, 0)) (block.rs:74-84), correctly rounded
      const float m_scale = h2f(cur.scale), m_offset = h2f(cur.offset), m_tail = h2f(cur.tail);
      const float t = fmaxf(m_tail, 0.0f);
      const float rho = (float)cur.flags / 255.0f;
      const float rc = rho > 1.0f ? 1.0f : rho;
      const float mid_n = fmaxf(sqrtf(fmaxf(1.0f - rc * rc, 0.0f)) * t, 1e-6f);
      const float high_n = fmaxf(rho * t, 0.0f);

      // Stage: 4-bit prefix IP (scan.rs:453-517), all queries
      float acc[QT];
#pragma unroll
      for (int qi = 0; qi < QT; ++qi) acc[qi] = zero_acc();
      const uint32_t mask = 0xF0u;
#pragma unroll 1
      for (int j = 0; j < 8; ++j) {
        // one 8-dim group per iteration; the level word is picked by selects
        // (a run-time index into the per-lane array would place it in scratch)
        uint32_t w = cur.nib[7];
#pragma unroll
        for (int u = 6; u >= 0; --u) w = j == u ? cur.nib[u] : w;
        const uint32_t w4s = w << 4;
        const char* lj = lutb + j * 8 * 256;
        uint32_t off[8];
        // level * 16: even dims from w << 4, odd dims from w (high nibble of each byte)
        off[0] = and_byte<0>(w4s, mask);
        off[1] = and_byte<0>(w, mask);
        off[2] = and_byte<1>(w4s, mask);
        off[3] = and_byte<1>(w, mask);
        off[4] = and_byte<2>(w4s, mask);
        off[5] = and_byte<2>(w, mask);
        off[6] = and_byte<3>(w4s, mask);
        off[7] = and_byte<3>(w, mask);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const float4 v = *reinterpret_cast<const float4*>(lj + g * 64 * 256 + i * 256 + off[i]);
            acc[4 * g + 0] = acc[4 * g + 0] + v.x;
            acc[4 * g + 1] = acc[4 * g + 1] + v.y;
            acc[4 * g + 2] = acc[4 * g + 2] + v.z;
            acc[4 * g + 3] = acc[4 * g + 3] + v.w;
          }
        }
      }
      // survivors: bit qi of sv = this lane survives query qi's stages so far
      const bool act = lane_in(active);
      float score[QT];
      uint32_t sv = 0;
#pragma unroll
      for (int qi = 0; qi < QT; ++qi) {
        const float4 c0 = qc4[qi * 4 + 0], c1 = qc4[qi * 4 + 1];
        // c0 = {eden, mean_ip, prefix_sum, mid_norm}, c1 = {tail_norm, tau_prune, tau_push, b1}
        const float prefix_ip = c0.x != 0.0f ? c0.y + m_scale * acc[qi] : acc[qi] * m_scale + m_offset * c0.z;
        score[qi] = prefix_ip;
        const float4 c3 = qc4[qi * 4 + 3];
        const float ub = prefix_bound(prefix_ip, mid_n, high_n, c3.z, c3.w, alpha, c0.w, c1.x);
        sv |= (act && ub >= c1.y) ? (1u << qi) : 0u;
      }
      if (a.stats) {
#pragma unroll
        for (int qi = 0; qi < QT; ++qi) c_prefix += (uint32_t)__popcll(ballot((sv >> qi) & 1u));
      }

      if (ballot(sv != 0u) != 0) {
        // Stage: mid-band 1-bit IP (scan.rs:520-569), all queries
        float s1[QT];
#pragma unroll
        for (int qi = 0; qi < QT; ++qi) s1[qi] = s_qc[qi * kQcCount + kQcS1Base];
#pragma unroll 4
        for (int d = 0; d < 128; ++d) {
          const uint64_t pw = plane_word128(cur.t1, d);
          masked_add_tile(s1, pw & active, w1 + NG * d);
        }
        bool any3 = false;
#pragma unroll
        for (int qi = 0; qi < QT; ++qi) {
          const float4 c1 = qc4[qi * 4 + 1], c2 = qc4[qi * 4 + 2], c3 = qc4[qi * 4 + 3];
          // c1 = {tail_norm, tau_prune, tau_push, b1}, c2 = {s1base, mid_mean_ip, after_s1, has_tail},
          // c3 = {budget, tail_base, -, -}
          const bool in = (sv >> qi) & 1u;
          const float sc = c1.w != 0.0f ? score[qi] + (c2.y + m_offset * s1[qi]) : score[qi] + s1[qi] * mid_n;
          score[qi] = in ? sc : score[qi];
          // Stage: post-S1 CS (scan.rs:572-584)
          const float ub2 = s1_bound(score[qi], high_n, c3.z, c3.w, alpha, c2.z);
          bool keep = in && ub2 >= c1.y;
          if (a.stats) c_s1 += (uint32_t)__popcll(ballot(keep));
          if (FULL) {
            // Stage: S4 abs-budget prune (scan.rs:587-607), when has_tail_fold and budget > 0
            const float hn = fmaxf(high_n, 1e-6f);
            const float ub3 = score[qi] + alpha * hn * sp.w_s4 * c3.x;
            const bool gate = c2.w != 0.0f && c3.x > 0.0f;
            keep = keep && (!gate || ub3 >= c1.y);
            any3 = any3 || (keep && c2.w != 0.0f);
          }
          sv = keep ? (sv | (1u << qi)) : (sv & ~(1u << qi));
        }
        if (FULL && ballot(any3) != 0) {
          // Stage: folded-tail 1-bit IP (scan.rs:610-634), all queries
          float s4[QT];
#pragma unroll
          for (int qi = 0; qi < QT; ++qi) s4[qi] = s_qc[qi * kQcCount + kQcTailBase];
#pragma unroll 4
          for (int d = 0; d < 64; ++d) {
            const uint64_t pw = plane_word64(cur.t4, d);
            masked_add_tile(s4, pw & active, w4 + NG * d);
          }
          const float hn = fmaxf(high_n, 1e-6f);
#pragma unroll
          for (int qi = 0; qi < QT; ++qi) {
            const float sc = score[qi] + s4[qi] * hn * sp.w_s4;
            score[qi] = (s_qc[qi * kQcCount + kQcHasTail] != 0.0f && ((sv >> qi) & 1u)) ? sc : score[qi];
          }
        }
      } else if (a.stats) {
#pragma unroll
        for (int qi = 0; qi < QT; ++qi) c_s1 += (uint32_t)__popcll(ballot((sv >> qi) & 1u));
      }
      // push / append, per query
      c_blocks += (uint32_t)nq;
      c_active += (uint32_t)nq * (uint32_t)__popcll(active);
#pragma unroll
      for (int qi = 0; qi < QT; ++qi) {
        const uint32_t q = q0 + qi;
        const bool mine = (sv >> qi) & 1u;
        const uint64_t pushed = ballot(mine);
        if (a.stats) c_s4b += (uint32_t)__popcll(pushed);
        if (pushed == 0) continue;
        if (a.hist) {
          if (mine) atomicAdd(a.hist + (uint64_t)q * kHistBins + hist_bin(score[qi], s_hinv[qi]), 1u);
          continue;
        }
        const float tq = s_qc[qi * kQcCount + kQcTauPush];
        if (ballot(mine && score[qi] != score[qi]) != 0 && lane == 0) atomicOr(a.err + q, 1u);
        const uint64_t pm = ballot(mine && score[qi] >= tq);
        if (pm != 0) stage_append<QT>(s_app, a, qi, q, seg, pm, score[qi], b * 64u + lane);
      }
    }
    retire_touch(cur);
    cur = nxt;
    b_cur = b_nxt;
  }
  if (a.stats && lane == 0) {
    atomicAdd(&s_stats[kStatBlocks], c_blocks);
    atomicAdd(&s_stats[kStatActive], c_active);
    atomicAdd(&s_stats[kStatPrefix], c_prefix);
    atomicAdd(&s_stats[kStatS1], c_s1);
    atomicAdd(&s_stats[kStatS4Budget], c_s4b);
    atomicAdd(&s_stats[kStatPushed], c_s4b);
  }
  flush_appends<QT, false>(s_app, a, q0, nq, seg, s_stats);
}

// ---------------------------------------------------------------------------
// thresholds and top-K selection
// Order: score descending, then row ascending (a total order, so the best K
// under it is unique and can be assembled from any superset).
// ---------------------------------------------------------------------------
constexpr int kSortCap = 8192;
constexpr int kSelCap = 2048;   // entries at or above the K-th bin floor kept for the final sort
constexpr int kSelThreads = 1024;
constexpr int kRankMax = 512;  // up to this many gathered entries are rank-sorted

// Block-wide exclusive prefix sum of one value per thread; *total gets the
// sum over the block.  ws: blockDim.x / 64 words of LDS, free until the
// caller's next barrier.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* ws, uint32_t* total) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6, nw = blockDim.x >> 6;
  uint32_t incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t x = __shfl_up(incl, o);
    if ((int)lane >= o) incl += x;
  }
  if (lane == 63) ws[w] = incl;
  __syncthreads();
  uint32_t base = 0, all = 0;
  for (uint32_t u = 0; u < nw; ++u) {
    const uint32_t x = ws[u];
    base += u < w ? x : 0u;
    all += x;
  }
  *total = all;
  return base + incl - v;
}

// Block-wide: the bin holding the need-th largest entry of a scan of `hist`
// (nb = blockDim.x or 2 * blockDim.x bins) from the top (desc) or the
// bottom.  Writes the bin and the count strictly before it in the scan to
// LDS outputs (read after the caller's barrier); bin 0 (desc) or nb - 1
// when the histogram holds fewer than `need`.  Thread t takes scan
// positions per*t .. per*t + per - 1, so neighbouring lanes read
// neighbouring bins.
__device__ __forceinline__ void find_boundary(const uint32_t* hist, uint32_t nb, uint32_t need, bool desc,
                              uint32_t* out_bin, uint32_t* out_before, uint32_t* ws) {
  const uint32_t t = threadIdx.x, per = nb / blockDim.x;
  auto bin_at = [&](uint32_t pos) { return desc ? nb - 1 - pos : pos; };
  const uint32_t c0 = hist[bin_at(per * t)];
  const uint32_t c1 = per == 2 ? hist[bin_at(per * t + 1)] : 0u;
  uint32_t total;
  const uint32_t excl = block_excl_scan(c0 + c1, ws, &total);
  if (excl < need && excl + c0 + c1 >= need) {
    const bool first = excl + c0 >= need;
    *out_bin = bin_at(per * t + (first ? 0u : 1u));
    *out_before = first ? excl : excl + c0;
  }
  if (t == 0 && (total < need || need == 0)) {  // no bin holds the need-th entry
    *out_bin = desc ? 0u : nb - 1;
    *out_before = total;
  }
}

// Walk over a query's candidate segments in work items of kChunk entries of
// one segment: item c lies in segment s with coff[s] <= c < coff[s+1].  A
// wave takes items c = wave, wave + nwaves, ...; lane l loads entries
// base + 64u + l (u < kWalk) of its item, all before any is used, so the
// loads are coalesced and kWalk of them are in flight per lane (with 16
// waves, up to 32K candidates take one round of memory latency).
constexpr int kWalk = 32;
constexpr uint32_t kChunk = 64u * kWalk;  // entries of a work item
struct CandView {
  const float* sc;
  const uint32_t* rw;
  uint32_t seg_cap;
  uint32_t nseg;
  const uint32_t* off;   // LDS, nseg + 1 prefix offsets of the capped counts
  const uint32_t* coff;  // LDS, nseg + 1 prefix offsets of the item counts
};

// W (<= kWalk) loads per lane at a time; an item is walked in kWalk / W steps.
template <int W = kWalk, typename F>
__device__ __forceinline__ void for_each_cand(const CandView& v, F&& fn) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const uint32_t items = v.coff[v.nseg];
  uint32_t s = 0;
  for (uint32_t c = wave; c < items; c += nwaves) {
    while (v.coff[s + 1] <= c) ++s;
    const uint32_t base = (c - v.coff[s]) * kChunk;
    const uint32_t cnt = v.off[s + 1] - v.off[s];
    const uint32_t lim = cnt > base ? cnt - base : 0u;  // entries of the item (may exceed kChunk)
    for (int h = 0; h < kWalk / W; ++h) {
      const uint32_t i0 = s * v.seg_cap + base + (uint32_t)h * 64u * W + lane;
      const uint32_t lh = lim > (uint32_t)h * 64u * W ? lim - (uint32_t)h * 64u * W : 0u;
      float sc[W];
#pragma unroll
      for (int u = 0; u < W; ++u)
        if (64u * u + lane < lh) sc[u] = v.sc[i0 + 64u * u];
#pragma unroll
      for (int u = 0; u < W; ++u)
        if (64u * u + lane < lh) fn(sc[u], i0 + 64u * u);
    }
  }
}

// The same walk, loading each entry's score and row together; fn also gets
// the entry's dense position (its index among all of the query's entries,
// segments in order).
template <typename F>
__device__ __forceinline__ void for_each_pair(const CandView& v, F&& fn) {
  constexpr int W = kWalk / 2;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const uint32_t items = v.coff[v.nseg];
  uint32_t s = 0;
  for (uint32_t c = wave; c < items; c += nwaves) {
    while (v.coff[s + 1] <= c) ++s;
    const uint32_t base = (c - v.coff[s]) * kChunk;
    const uint32_t cnt = v.off[s + 1] - v.off[s];
    const uint32_t lim = cnt > base ? cnt - base : 0u;
    for (int h = 0; h < kWalk / W; ++h) {
      const uint32_t i0 = s * v.seg_cap + base + (uint32_t)h * 64u * W + lane;
      const uint32_t d0 = v.off[s] + base + (uint32_t)h * 64u * W + lane;
      const uint32_t lh = lim > (uint32_t)h * 64u * W ? lim - (uint32_t)h * 64u * W : 0u;
      float sc[W];
      uint32_t rw[W];
#pragma unroll
      for (int u = 0; u < W; ++u)
        if (64u * u + lane < lh) {
          sc[u] = v.sc[i0 + 64u * u];
          rw[u] = v.rw[i0 + 64u * u];
        }
#pragma unroll
      for (int u = 0; u < W; ++u)
        if (64u * u + lane < lh) fn(sc[u], rw[u], d0 + 64u * u);
    }
  }
}

// Prefix offsets of the (capped) segment counts into off[0..nseg] and of
// their item counts into coff[0..nseg] (nseg <= blockDim.x): thread t holds
// counter t (`count`, 0 past nseg); wave scans, then a scan of the wave
// totals (ws: 2 * 16 words).
__device__ __forceinline__ void seg_offsets(uint32_t count, uint32_t nseg, uint32_t seg_cap, uint32_t* off, uint32_t* coff,
                            uint32_t* ws) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  const uint32_t c = count < seg_cap ? count : seg_cap;
  uint32_t ic = c, ii = (c + kChunk - 1) / kChunk;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t x = __shfl_up(ic, o), y = __shfl_up(ii, o);
    if ((int)lane >= o) {
      ic += x;
      ii += y;
    }
  }
  if (lane == 63) {
    ws[w] = ic;
    ws[16 + w] = ii;
  }
  __syncthreads();
  uint32_t bc = 0, bi = 0;
  for (uint32_t u = 0; u < w; ++u) {
    bc += ws[u];
    bi += ws[16 + u];
  }
  if (t < nseg) {
    off[t + 1] = bc + ic;
    coff[t + 1] = bi + ii;
  }
  if (t == 0) {
    off[0] = 0;
    coff[0] = 0;
  }
  __syncthreads();
}

// The walk of for_each_pair for many short segments (one per workgroup of
// the final pass, nseg <= blockDim.x): thread t takes segment t and loads up
// to kShortRound of its entries per round, all before any is used.
constexpr int kShortRound = 16;
// With a segment per workgroup of the final pass, a thread of k_select reads
// the first kShortPre entries of its segment together with the segment's
// count (segments hold at least that many), before the offsets are known.
constexpr int kShortPre = 8;
struct ShortPre {
  float sc[kShortPre];
  uint32_t rw[kShortPre];
};
template <typename F>
__device__ __forceinline__ void for_each_pair_short(const CandView& v, const ShortPre& pre, F&& fn) {
  const uint32_t t = threadIdx.x;
  if (t >= v.nseg) return;
  const uint32_t cnt = v.off[t + 1] - v.off[t];
  const uint64_t base = (uint64_t)t * v.seg_cap;
  // the first kShortPre entries were read with the segment's count
#pragma unroll
  for (int u = 0; u < kShortPre; ++u)
    if ((uint32_t)u < cnt) fn(pre.sc[u], pre.rw[u], v.off[t] + (uint32_t)u);
  for (uint32_t r = kShortPre; r < cnt; r += kShortRound) {
    float sc[kShortRound];
    uint32_t rw[kShortRound];
#pragma unroll
    for (int u = 0; u < kShortRound; ++u)
      if (r + u < cnt) {
        sc[u] = v.sc[base + r + u];
        rw[u] = v.rw[base + r + u];
      }
#pragma unroll
    for (int u = 0; u < kShortRound; ++u)
      if (r + u < cnt) fn(sc[u], rw[u], v.off[t] + r + u);
  }
}

// LDS histogram of the appended scores of one query (all segments).
__device__ __forceinline__ void build_hist(uint32_t* hist, const CandView& v, float hinv) {
  for (int i = threadIdx.x; i < kHistBins; i += blockDim.x) hist[i] = 0u;
  __syncthreads();
  for_each_cand(v, [&](float sc, uint32_t) { atomicAdd(&hist[hist_bin(sc, hinv)], 1u); });
  __syncthreads();
}

__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t row) {
  return ((uint64_t)key << 32) | (uint64_t)(~row);
}

// Descending bitonic sort of s[0..n2) (n2 a power of two).
__device__ __forceinline__ void bitonic_desc(uint64_t* s, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < n2 / 2; i += blockDim.x) {
        int lo = 2 * i - (i & (stride - 1));
        int hi = lo + stride;
        bool desc = ((lo & size) == 0);
        uint64_t x = s[lo], y = s[hi];
        bool swap = desc ? (x < y) : (x > y);
        if (swap) {
          s[lo] = y;
          s[hi] = x;
        }
      }
      __syncthreads();
    }
  }
}

// Final selection for one query: threshold from the histogram, gather the
// appended candidates at or above it (typically K plus one bin), sort, emit.
// Falls back to an exact radix select on the score key (then on the row for
// exact ties) when the gathered set exceeds the sort buffer.  Leaves the
// query's counters, histogram and error flag zeroed for the next scan.
__global__ __launch_bounds__(kSelThreads) void k_select(SelectArgs a) {
  __shared__ __align__(16) uint64_t s_buf[kSortCap];  // read as 16-byte pairs by the rank sort
  __shared__ __align__(16) uint64_t s_sel[kSelCap + 16];
  __shared__ uint32_t s_start[kHistBins];
  __shared__ uint32_t s_hist[2048];
  __shared__ uint32_t s_misc[8];
  __shared__ uint32_t s_off[kMaxSegs + 1];
  __shared__ uint32_t s_coff[kMaxSegs + 1];
  __shared__ uint32_t s_ws[32];

  __shared__ float s_fl[3];

  const uint32_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const uint32_t K = a.k;
  if (a.gate && (a.gate[q] & 4u) == 0u) return;  // gated re-run: only a flagged query
  const uint32_t* qcount = a.seg_count + (uint64_t)q * a.nseg;
  const CandView v{a.cand_score + (uint64_t)q * a.nseg * a.seg_cap, a.cand_row + (uint64_t)q * a.nseg * a.seg_cap,
                   a.seg_cap, a.nseg, s_off, s_coff};
  // The set-up's reads go out together: the final pass's floor and the safe
  // one (for the shortfall check below) and this thread's segment count.
  const bool short_segs = a.nseg > (uint32_t)kSegs;
  // the query's histogram scale (2^-e, 2^e)
  const float hinv = a.luts[(uint64_t)q * kQData + kQdHistInv];
  const float hscale = a.luts[(uint64_t)q * kQData + kQdHistScale];
  float fl_safe = 0.0f, fl_final = 0.0f, fl_used = -INFINITY;
  if (a.hist && tid == 0) {
    fl_safe = a.tau_safe[q];
    fl_final = a.tau_final[q];
  }
  if (a.tau_used && tid == 0) fl_used = a.tau_used[q];
  const uint32_t c_own = tid < (int)a.nseg ? qcount[tid] : 0u;
  ShortPre pre;
  if (short_segs && tid < (int)a.nseg && a.seg_cap >= (uint32_t)kShortPre) {
    const uint64_t base = (uint64_t)tid * a.seg_cap;
#pragma unroll
    for (int u = 0; u < kShortPre; ++u) {
      pre.sc[u] = v.sc[base + u];
      pre.rw[u] = v.rw[base + u];
    }
  }
  if (tid == 0) {
    s_misc[7] = 0;
    s_fl[0] = fl_safe;
    s_fl[1] = fl_final;
    s_fl[2] = fl_used;
  }
  __syncthreads();
  if (c_own > a.seg_cap) atomicOr(&s_misc[7], 2u);
  seg_offsets(c_own, a.nseg, a.seg_cap, s_off, s_coff, s_ws);
  const uint32_t total = s_off[a.nseg];
  uint32_t m;
  uint64_t* sb = s_buf;  // the entries the final sort reads
  if (total <= (uint32_t)kSelCap) {
    // Every entry fits the final sort: one walk loads (score, row) pairs
    // into LDS, and all of them are sorted (no histogram, no threshold).
    auto take = [&](float sc, uint32_t row, uint32_t dense) { s_sel[dense] = composite(score_key(sc), row); };
    if (short_segs && a.seg_cap >= (uint32_t)kShortPre) for_each_pair_short(v, pre, take);
    else for_each_pair(v, take);
    __syncthreads();
    m = total;
    sb = s_sel;
  } else if (total <= (uint32_t)kSortCap) {
    // Every entry fits in LDS: one walk loads (score, row) pairs and
    // histograms them; the entries at or above the K-th bin's floor are then
    // picked out of LDS.
    for (int i = tid; i < kHistBins; i += kSelThreads) s_hist[i] = 0u;
    __syncthreads();
    auto take = [&](float sc, uint32_t row, uint32_t dense) {
      atomicAdd(&s_hist[hist_bin(sc, hinv)], 1u);
      s_buf[dense] = composite(score_key(sc), row);
    };
    if (short_segs && a.seg_cap >= (uint32_t)kShortPre) for_each_pair_short(v, pre, take);
    else for_each_pair(v, take);
    __syncthreads();
    find_boundary(s_hist, kHistBins, K, true, &s_misc[0], &s_misc[1], s_ws);
    if (tid == 0) s_misc[2] = 0;
    __syncthreads();
    const uint32_t fkey = score_key(bin_floor(s_misc[0], hscale));
    for (uint32_t i = tid; i < total; i += kSelThreads) {
      const uint64_t c = s_buf[i];
      if ((uint32_t)(c >> 32) >= fkey) {
        const uint32_t slot = atomicAdd(&s_misc[2], 1u);
        if (slot < (uint32_t)kSelCap) s_sel[slot] = c;
      }
    }
    __syncthreads();
    m = s_misc[2];
    if (m <= (uint32_t)kSelCap) sb = s_sel;
    else m = total;  // sort every entry
  } else {
  build_hist(s_hist, v, hinv);
  find_boundary(s_hist, kHistBins, K, true, &s_misc[0], &s_misc[1], s_ws);
  __syncthreads();
  const float floor_t = bin_floor(s_misc[0], hscale);

  // entries >= floor_t as (score key, candidate index); the rows of the
  // gathered entries are then loaded all at once
  if (tid == 0) s_misc[2] = 0;
  __syncthreads();
  for_each_cand(v, [&](float sc, uint32_t idx) {
    if (sc >= floor_t) {
      const uint32_t slot = atomicAdd(&s_misc[2], 1u);
      if (slot < (uint32_t)kSortCap) s_buf[slot] = ((uint64_t)score_key(sc) << 32) | idx;
    }
  });
  __syncthreads();
  m = s_misc[2];
  if (m <= (uint32_t)kSortCap) {
    for (uint32_t i = tid; i < m; i += kSelThreads) {
      const uint64_t c = s_buf[i];
      s_buf[i] = composite((uint32_t)(c >> 32), v.rw[(uint32_t)c]);
    }
    __syncthreads();
  } else {
    // Radix select: the exact K-th key among entries >= floor_t, then the
    // smallest rows among its exact ties.
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    uint32_t prefix = 0, need = K;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass], wd = widths[pass];
      const uint32_t nb = 1u << wd;
      for (int i = tid; i < 2048; i += kSelThreads) s_hist[i] = 0;
      __syncthreads();
      for_each_cand<16>(v, [&](float sc, uint32_t) {
        if (!(sc >= floor_t)) return;
        const uint32_t key = score_key(sc);
        if (pass == 0 || (key >> (sh + wd)) == prefix) atomicAdd(&s_hist[(key >> sh) & (nb - 1)], 1u);
      });
      __syncthreads();
      find_boundary(s_hist, nb, need, true, &s_misc[3], &s_misc[4], s_ws);
      __syncthreads();
      need -= s_misc[4];
      prefix = (prefix << wd) | s_misc[3];
      __syncthreads();
    }
    const uint32_t tie_key = prefix;  // exact K-th key; `need` of its ties are kept
    uint32_t rprefix = 0, rneed = need;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass], wd = widths[pass];
      const uint32_t nb = 1u << wd;
      for (int i = tid; i < 2048; i += kSelThreads) s_hist[i] = 0;
      __syncthreads();
      for_each_cand<16>(v, [&](float sc, uint32_t idx) {
        if (!(sc >= floor_t) || score_key(sc) != tie_key) return;
        const uint32_t r = v.rw[idx];
        if (pass == 0 || (r >> (sh + wd)) == rprefix) atomicAdd(&s_hist[(r >> sh) & (nb - 1)], 1u);
      });
      __syncthreads();
      find_boundary(s_hist, nb, rneed, false, &s_misc[3], &s_misc[4], s_ws);
      __syncthreads();
      rneed -= s_misc[4];
      rprefix = (rprefix << wd) | s_misc[3];
      __syncthreads();
    }
    const uint32_t row_max = rprefix;
    if (tid == 0) s_misc[2] = 0;
    __syncthreads();
    for_each_cand<16>(v, [&](float sc, uint32_t idx) {
      if (!(sc >= floor_t)) return;
      const uint32_t key = score_key(sc);
      const uint32_t r = v.rw[idx];
      if (key > tie_key || (key == tie_key && r <= row_max)) {
        const uint32_t slot = atomicAdd(&s_misc[2], 1u);
        if (slot < (uint32_t)kSortCap) s_buf[slot] = composite(key, r);
      }
    });
    __syncthreads();
    m = s_misc[2];  // == K
    if (m > (uint32_t)kSortCap) m = kSortCap;
  }
  }
  const uint32_t keep = m < K ? m : K;
  auto emit = [&](uint32_t r, uint64_t c) {
    const uint32_t row = ~(uint32_t)c;
    a.out_ids[(uint64_t)q * K + r] = ((uint64_t)(row >> 6) << 16) | (uint64_t)(row & 63u);
    a.out_scores[(uint64_t)q * K + r] = key_score((uint32_t)(c >> 32));
  };
  if (sb == s_sel) {
    // Counting sort by bin, descending: an entry's position is the number of
    // selected entries in higher bins plus the number of larger keys in its
    // own bin (keys are distinct).  The bins split the selected entries' own
    // score range [smin, smax] evenly (never wider than the sampling
    // histogram's bins, and much finer when the selected scores crowd
    // together, as for a query among near-duplicates).  s_hist counts per
    // bin, then serves as the scatter cursor.  Only bins that start above
    // position keep are placed and ranked: an entry in a bin with `keep`
    // entries above it ranks at keep or lower.  These low bins are the
    // crowded ones (the scores thin out towards the top), so skipping them
    // also skips most same-bin LDS atomics.  s_misc[5]: the end of the bin
    // that holds position keep - 1, m when keep == m.
    if (tid == 0) {
      s_misc[3] = 0xFFFFFFFFu;
      s_misc[4] = 0u;
      s_misc[5] = m;
    }
    for (int i = tid; i < kHistBins; i += kSelThreads) s_hist[i] = 0u;
    __syncthreads();
    {  // the key range: per wave first, then one LDS atomic per wave
      uint32_t lo_k = 0xFFFFFFFFu, hi_k = 0u;
      for (uint32_t i = tid; i < m; i += kSelThreads) {
        const uint32_t k = (uint32_t)(sb[i] >> 32);
        lo_k = min(lo_k, k);
        hi_k = max(hi_k, k);
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        lo_k = min(lo_k, (uint32_t)__shfl_xor((int)lo_k, o));
        hi_k = max(hi_k, (uint32_t)__shfl_xor((int)hi_k, o));
      }
      if ((tid & 63) == 0 && lo_k <= hi_k) {
        atomicMin(&s_misc[3], lo_k);
        atomicMax(&s_misc[4], hi_k);
      }
    }
    __syncthreads();
    const float smin = key_score(s_misc[3]), smax = key_score(s_misc[4]);
    // (bounded, so every product below is finite: 0 when the range overflows)
    const float binv = m && smax > smin ? fminf((float)(kHistBins - 1) / (smax - smin), 1e30f) : 0.0f;
    // monotone in the score: a larger score never takes a lower bin
    auto lbin = [&](uint64_t c) -> uint32_t {
      const float b = fminf((key_score((uint32_t)(c >> 32)) - smin) * binv, (float)(kHistBins - 1));
      return (uint32_t)b;
    };
    for (uint32_t i = tid; i < m; i += kSelThreads) atomicAdd(&s_hist[lbin(sb[i])], 1u);
    __syncthreads();
    {  // start[b] = entries in bins above b; thread t owns bins 2047 - 2t and 2046 - 2t
      const uint32_t b0 = kHistBins - 1 - 2u * (uint32_t)tid, b1 = b0 - 1;
      const uint32_t c0 = s_hist[b0], c1 = s_hist[b1];
      uint32_t total;
      const uint32_t excl = block_excl_scan(c0 + c1, s_ws, &total);
      s_start[b0] = excl;
      s_start[b1] = excl + c0;
      s_hist[b0] = 0u;
      s_hist[b1] = 0u;
      // at most one bin holds position keep - 1 (empty bins hold none)
      if (excl < keep && excl + c0 >= keep) s_misc[5] = excl + c0;
      if (excl + c0 < keep && excl + c0 + c1 >= keep) s_misc[5] = excl + c0 + c1;
    }
    __syncthreads();
    for (uint32_t i = tid; i < m; i += kSelThreads) {
      const uint64_t c = sb[i];
      const uint32_t b = lbin(c);
      if (s_start[b] < keep) s_buf[s_start[b] + atomicAdd(&s_hist[b], 1u)] = c;
    }
    __syncthreads();
    const uint32_t placed = s_misc[5];
    for (uint32_t i = tid; i < placed; i += kSelThreads) {
      const uint64_t c = s_buf[i];
      const uint32_t b = lbin(c);
      const uint32_t lo = s_start[b], hi = lo + s_hist[b];
      uint32_t r = lo, j = lo;
      for (; j + 4 <= hi; j += 4) {  // four independent reads in flight
        const uint64_t x0 = s_buf[j], x1 = s_buf[j + 1], x2 = s_buf[j + 2], x3 = s_buf[j + 3];
        r += (x0 > c ? 1u : 0u) + (x1 > c ? 1u : 0u) + (x2 > c ? 1u : 0u) + (x3 > c ? 1u : 0u);
      }
      for (; j < hi; ++j) r += s_buf[j] > c ? 1u : 0u;
      if (r < keep) emit(r, c);
    }
  } else if (m <= (uint32_t)kRankMax) {
    // Rank sort: the composite keys are distinct, so an entry's position in
    // the descending order is the number of larger keys.  Every lane of a
    // wave reads the same key j at the same time (an LDS broadcast).
    // pad to a multiple of 16 with keys below every composite key
    for (uint32_t i = m + tid; i < ((m + 15u) & ~15u); i += kSelThreads) sb[i] = 0ull;
    __syncthreads();
    const uint32_t m16 = (m + 15u) & ~15u;
    const ulonglong2* b2 = reinterpret_cast<const ulonglong2*>(sb);
    for (uint32_t i = tid; i < m; i += kSelThreads) {
      const uint64_t key = sb[i];
      uint32_t r = 0;
      ulonglong2 nx[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) nx[u] = b2[u];
      for (uint32_t j = 8; j <= m16; j += 8) {
        ulonglong2 k4[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) k4[u] = nx[u];
        if (j < m16) {
#pragma unroll
          for (int u = 0; u < 4; ++u) nx[u] = b2[(j >> 1) + u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) r += (k4[u].x > key ? 1u : 0u) + (k4[u].y > key ? 1u : 0u);
      }
      if (r < keep) emit(r, key);
    }
  } else {
    int n2 = 1;
    while ((uint32_t)n2 < m) n2 <<= 1;
    for (int i = (int)m + tid; i < n2; i += kSelThreads) sb[i] = 0ull;
    __syncthreads();
    bitonic_desc(sb, n2);
    for (uint32_t i = tid; i < keep; i += kSelThreads) emit(i, sb[i]);
  }
  __syncthreads();
  // leave this query's pass state clean for the next scan
  if (tid < (int)a.nseg) a.seg_count[(uint64_t)q * a.nseg + tid] = 0u;
  if (a.hist)
    for (int i = tid; i < kHistBins; i += kSelThreads) a.hist[(uint64_t)q * kHistBins + i] = 0u;
  if (tid == 0) {
    // Fewer than K candidates above a floor tighter than the safe one: the
    // top K may lie below it, so the final pass is re-run at the safe floor.
    // Fewer than K above a finite floor no tighter than the safe one happens
    // only when the stage bounds are not admissible (vectors above the floor
    // were rejected): the query is re-run with no floor, as the reference's
    // shortlist, whose threshold stays at -inf until it holds K, keeps
    // min(K, active) hits.
    const uint32_t short_k = (a.hist && keep < K && s_fl[1] > s_fl[0]) ? 4u : 0u;
    const uint32_t short_f = (!short_k && keep < K && s_fl[2] > -INFINITY) ? 8u : 0u;
    a.out_counts[q] = keep;
    if (a.floor_record) a.floor_record[q] = s_fl[2];
    a.status[q] = (a.err[q] & 1u) | s_misc[7] | short_k | short_f;
    a.err[q] = 0u;
    if (a.stats && (short_k | short_f | s_misc[7])) {
      unsigned long long* st = a.stats + (q % (uint32_t)kStatCopies) * kStatCount;
      if (short_k) atomicAdd(st + kStatRerunSafe, 1ull);
      if ((s_misc[7] & 2u) || short_f) atomicAdd(st + kStatRerunDense, 1ull);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA-bounded batched scan
// ---------------------------------------------------------------------------
// In real arithmetic the reference's full score of a vector for a query
// (scan.rs:453-634, every stage run; mid_n = max(mid_norm, 1e-6),
// hn = max(high_n, 1e-6)) is
//   P + mid_n * S1 + hn * w_s4 * S4,
//   P  = mean_ip + scale * sum_d cb[l_d] w_d     (EdenProd; the LUT is cb * w)
//      = scale * sum_d l_d q_d + offset * prefix_sum   (MinMax4),
//   S1 = sum_d pos_d (2 b_d - 1)   (rabitq_base = -sum pos, weights2 = 2 pos),
//   S4 = the same over the folded tail,
// a dot product of a 261-value row per vector with a column per query.
// k_scan_mma evaluates it for 32 queries x 32 vectors per f16 MFMA tile
// (v_mfma_f32_32x32x16_f16, 17 K-steps): queries are the A operand, scaled
// by a power of two s; vectors are the B operand, built from the block:
// scale * cb[level] (a byte -> two-f16 LDS table, then a packed multiply),
// +-mid_n / 2 and +-hn w_s4 / 2 from the sign of each S1 / S4 bit, and a last
// step of error columns.  The accumulator starts at C = s (mean_ip - tau + e0).
//   E(v, q) = |scale| eP + mid_n e1 + hn e4 + |offset| eO + e0
// bounds |tile value / s - (reference's f32 score - tau)|.  With u = 2^-11
// (f16 rounding, relative; 2^-25 absolute below the normal range, covered by
// the t25 terms and e0) and M the summed magnitudes of a part's products:
//  - prefix: a query weight rounded once, scale * cb rounded twice (cb, then
//    the packed product): <= (3u + 3u^2 + u^3) M, M <= |scale| cbm l1w;
//  - S1 / S4 / offset * prefix_sum: two roundings (one for the offset):
//    <= (2u + u^2) M, M = mid_n l1w2 / 2, hn w_s4 l1w4 / 2, |offset psum|;
//  - the MFMA's f32 accumulation of the 272 products and the start value C,
//    in any order, each addition rounding to nearest or truncating:
//    <= gamma_273 ~ 2^-14.9 of all the magnitudes;
//  - the reference's own sequential f32 sums (at most 128 terms each):
//    <= gamma_128 ~ 2^-17 of their magnitudes.
// eP = cbm l1w / 600 (needs 1 / 664), e1 = l1w2 / 1800 (needs 1 / 1966),
// e4 = w_s4 l1w4 / 1800, eO = |psum| / 1700 (needs 1 / 1892), each times
// 1 + 2^-10 for its own f32 evaluation; C's share is in e0 (|mean_ip| /
// 16384, |tau| / 16384).  With the error columns added the tile holds
// s (U - tau), U = approximation + E >= score; the sampling pass subtracts
// them and gets s L, L = approximation - E <= score.  Under the settings
// tight_coef() accepts, the reference's top K is the top K by full score, so
// dropping pairs with U < tau (tau <= the K-th best score) is exact, and so
// is scoring exactly only the pairs whose U reaches the K-th best L
// (k_finish).
typedef _Float16 mma_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mma_h2 __attribute__((ext_vector_type(2)));
typedef float mma_f16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ mma_h8 as_h8(uint4 u) { return __builtin_bit_cast(mma_h8, u); }

// Dimension of the query weight behind element e (0..7) of K-half kh at
// K-step st < 16.  Prefix step st: level word 4 kh + st, element e = nibble e.
// S1 step 4 + t: dword 2 kh + t / 4 of the slot's S1 row, element 2 j + p =
// bit 4 (t % 4) + j + 16 p.  S4 step 12 + t: dword kh of the S4 row, element
// 2 j + p = bit 4 t + j + 16 p.  k_scan_mma builds the vector operand in the
// same order.
__device__ __forceinline__ int mma_dim(int st, int kh, int e) {
  if (st < 4) return 8 * (4 * kh + st) + e;
  const int j = e >> 1, p = e & 1;
  if (st < 12) {
    const int t = st - 4;
    return 64 * kh + 32 * (t >> 2) + 4 * (t & 3) + j + 16 * p;
  }
  return 32 * kh + 4 * (st - 12) + j + 16 * p;
}

// f16 bits of x, rounded to nearest (the hardware conversion).
__device__ __forceinline__ uint32_t f16_bits(float x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

// f16 bits of x >= 0 with a magnitude no smaller than x: the nearest f16,
// one ulp up when that lies below x.
__device__ __forceinline__ uint32_t f16_up(float x) {
  uint32_t h = f16_bits(x);
  if (h2f((uint16_t)h) < x) h += 1u;
  return h;
}

// Query operands and error coefficients of query q, by the first wave of
// the workgroup (threads 0..63; the other waves have nothing to do).
struct MmaPrepLds {
  float w[64], w1[128], w4[64], ex[8];
};
__device__ __forceinline__ void mma_prep_body(const MmaPrepArgs& a, uint32_t q, MmaPrepLds& sh) {
  float* s_w = sh.w;
  float* s_w1 = sh.w1;
  float* s_w4 = sh.w4;
  float* s_ex = sh.ex;
  const uint32_t lane = threadIdx.x;
  float s = 0.0f, psum = 0.0f;  // operand scale and prefix_sum, for the operand step below
  float s4b = 0.0f;             // bound on |S4 stage score| per unit high_n (score units)
  float s1b = 0.0f;             // bound on |S1| (the S1 stage's score per unit mid_n)
  if (lane < 64) {
    const mrl_query_plan* p = a.plans + q;
    const float* qd = a.luts + (uint64_t)q * kQData;
    const bool eden = p->prefix_codec == MRL_PREFIX_EDEN_PROD;
    const bool s1on = a.sp.strata != MRL_STRATA_L0_ONLY;
    const bool tail = a.sp.strata == MRL_STRATA_FULL64B && p->has_tail_fold != 0;
    const float w = p->prefix_weight[lane];
    const float w1a = s1on ? qd[kQdW1 + lane] : 0.0f, w1b = s1on ? qd[kQdW1 + 64 + lane] : 0.0f;
    const float w4 = tail ? qd[kQdW4 + lane] : 0.0f;
    s_w[lane] = w;
    s_w1[lane] = w1a;
    s_w1[64 + lane] = w1b;
    s_w4[lane] = w4;
    const float cbv = lane < 16 ? (eden ? fabsf(p->eden_codebook[lane]) : (float)lane) : 0.0f;
    float l1w = fabsf(w), l1w2 = fabsf(w1a) + fabsf(w1b), l1w4 = fabsf(w4), cbm = cbv;
    float mx = fmaxf(fmaxf(fabsf(w), fabsf(w4)), fmaxf(fabsf(w1a), fabsf(w1b)));
    const bool fin_l = w - w == 0.0f && w1a - w1a == 0.0f && w1b - w1b == 0.0f && w4 - w4 == 0.0f && cbv - cbv == 0.0f;
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
      l1w += __shfl_xor(l1w, h);
      l1w2 += __shfl_xor(l1w2, h);
      l1w4 += __shfl_xor(l1w4, h);
      mx = fmaxf(mx, __shfl_xor(mx, h));
      cbm = fmaxf(cbm, __shfl_xor(cbm, h));
    }
    const float mean = eden ? p->eden_mean_ip : 0.0f;
    psum = eden ? 0.0f : p->prefix_sum;
    const float ws4 = tail ? a.sp.w_s4 : 0.0f;
    // The f32 sums above run over at most 128 terms: relative error < 2^-17.
    const float up = 1.0f + 1.0f / 1024.0f;
    // s: every query-operand value times s stays below 2^14 in magnitude
    const float bm = fmaxf(mx, fabsf(psum));
    int ex = 0;
    if (bm > 0.0f && bm - bm == 0.0f) (void)frexpf(bm, &ex);
    ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
    s = ldexpf(1.0f, 14 - ex);
    const float inv_s = ldexpf(1.0f, ex - 14);
    const float t25 = 2.98023223876953125e-8f;  // 2^-25
    const float eP = (cbm * l1w * (1.0f / 600.0f) + t25 * (64.0f * cbm + 1.0f) * inv_s) * up;
    const float e1 = s1on ? (l1w2 * (1.0f / 1800.0f) + t25 * 65.0f * inv_s) * up : 0.0f;
    const float e4 = tail ? (ws4 * l1w4 * (1.0f / 1800.0f) + t25 * (32.0f * ws4 + 1.0f) * inv_s) * up : 0.0f;
    // |w_s4 * S4| <= w_s4 * sum|w4| / 2 (w4 = 2 pos, S4 = sum pos (2 b - 1)); raised by 2^-12 for the
    // f32 sum over 64 terms above and the reference's own rounding of S4 (sequential, 65 terms)
    // (the final pass bounds S4 only for w_s4 <= kMmaWideMaxWs4: then s * s4b / 64 < 2^15, a finite f16)
    s4b = tail && ws4 <= kMmaWideMaxWs4 ? ws4 * l1w4 * 0.5f * (1.0f + 1.0f / 4096.0f) : 0.0f;
    // |S1| <= sum |w1| / 2 (w1 = 2 pos, S1 = sum pos (2 b - 1)), raised by 2^-12 for the f32 sum above and
    // the reference's own rounding of S1 (sequential, 129 terms); s * s1b < 2^20 (every s |w1| < 2^14), so
    // s * s1b / 24 is a finite f16
    s1b = s1on ? l1w2 * 0.5f * (1.0f + 1.0f / 4096.0f) : 0.0f;
    const float eO = eden ? 0.0f : (fabsf(psum) * (1.0f / 1700.0f) + t25 * 2.0f * inv_s) * up;
    const float e0 =
        (fabsf(mean) * (1.0f / 16384.0f) + t25 * (l1w + l1w2 + l1w4 + fabsf(psum) + eP + e1 + e4 + eO)) * up +
        1e-18f;
    const float R = 2.0f * (fabsf(mean) +
                            kMmaSafe * (cbm * l1w + l1w2 + ws4 * l1w4 + fabsf(psum) + eP + e1 + e4 + eO) + e0 + 1.0f);
    const bool fin = ballot(!fin_l) == 0 && mean - mean == 0.0f && psum - psum == 0.0f && R - R == 0.0f;
    if (q == 0 && lane == 0) a.work[0] = 0u;  // k_exact's item count, filled by k_finish
    if (lane == 0) {
      s_ex[0] = eP;
      s_ex[1] = e1;
      s_ex[2] = e4;
      s_ex[3] = eO;
      float* mc = a.consts + (uint64_t)q * kMcCount;
      mc[kMcS] = s;
      mc[kMcInvS] = inv_s;
      mc[kMcMean] = mean;
      mc[kMcEP] = eP;
      mc[kMcE1] = e1;
      mc[kMcE4] = e4;
      mc[kMcEO] = eO;
      mc[kMcE0] = e0;
      mc[kMcR] = R;
      mc[kMcOk] = fin ? 1.0f : 0.0f;
      for (int i = kMcOk + 1; i < kMcCount; ++i) mc[i] = 0.0f;
    }
  }
  // The operands are read back from LDS by the same wave that wrote them
  // (no workgroup barrier: the coefficient stores above need not complete
  // first).  Each lane converts its 8 elements along one path: value, then
  // f16 rounding to nearest, rounded up for the error columns.
  if (lane >= 64) return;
  wave_lds_sync();
  if (lane < 2 * kMmaSteps) {
    const int st = (int)lane >> 1, kh = (int)lane & 1;
    const float* src = st < 4 ? s_w : (st < 12 ? s_w1 : s_w4);
    uint32_t hv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.0f;
      if (st < 16) v = src[mma_dim(st, kh, e)];
      else if (kh == 0 && e < 4) v = s_ex[e];   // error columns
      else if (kh == 0 && e == 4) v = psum;     // offset * prefix_sum
      else if (kh == 0) v = s1b * (1.0f / 24.0f);  // S1 bound, 3 columns (f16 of 8 mid_n, rounded up)
      else if (kh == 1) v = s4b * (1.0f / 64.0f);  // S4 bound, 8 columns (f16 of 8 high_n, rounded up)
      const float x = s * v;
      uint32_t h = f32_to_f16(x);
      if (st == 16 && (e != 4 || kh == 1) && h2f((uint16_t)h) < x) h += 1u;  // f16_up: magnitude no smaller than x
      hv[e] = h;
    }
    a.ops[(uint64_t)q * (2 * kMmaSteps) + lane] =
        make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
  }
}

__global__ __launch_bounds__(64) void k_mma_prep(MmaPrepArgs a) {
  __shared__ MmaPrepLds sh;
  mma_prep_body(a, blockIdx.x, sh);
}

// The plan of query blockIdx.x (k_plan's work), then its MFMA operands from
// that plan (k_mma_prep's): one launch where a batch's plan is still to be
// built.  The plan record and scan constants are written to global memory
// by this workgroup and read back after its barrier.
__global__ __launch_bounds__(192) void k_plan_mma_prep(PlanArgs pa, MmaPrepArgs ma) {
  __shared__ PlanLds<MRL_MAX_DIMS> sh;
  __shared__ MmaPrepLds sp;
  plan_body<MRL_MAX_DIMS>(pa, blockIdx.x, sh);
  __syncthreads();
  mma_prep_body(ma, blockIdx.x, sp);
}

// Floors of a sampling stage from its histogram, one wave per query: rank
// `rank` and the safe rank K, raised to the previous stage's floors when
// `prev` (a later stage counts only lower bounds at or above the previous
// floor, so its own floor is -inf when too few were counted).  The histogram
// is left zeroed for the next stage.
__global__ __launch_bounds__(64) void k_mma_floors(uint32_t* hist, const float* luts, uint32_t rank,
                                                   uint32_t safe_rank, float* floor_out, float* safe_out, int prev) {
  const uint32_t q = blockIdx.x, lane = __lane_id();
  uint32_t* h = hist + (uint64_t)q * kHistBins;
  const HistRow r = hist_row(h);
  const float sc = luts[(uint64_t)q * kQData + kQdHistScale];  // the query's histogram scale 2^e
  float f = floor_of(r, rank) * sc;
  float sf = floor_of(r, safe_rank) * sc;
  uint4* mine = reinterpret_cast<uint4*>(h + (63u - lane) * 32u);  // the bins hist_row gave this lane
#pragma unroll
  for (int k = 0; k < 8; ++k) mine[k] = make_uint4(0u, 0u, 0u, 0u);
  if (lane == 0) {
    if (prev) {
      f = fmaxf(f, floor_out[q]);
      sf = fmaxf(sf, safe_out[q]);
    }
    floor_out[q] = f;
    safe_out[q] = sf;
  }
}

// One 32-vector tile's per-lane inputs: lane l serves vector 32 h + l % 32
// of block b, half l / 32 of the K range.
struct MmaRaw {
  uint4 lev;      // level words 4 kh .. 4 kh + 3
  uint2 r1;       // S1 row dwords 2 kh, 2 kh + 1
  uint32_t r4;    // S4 row dword kh
  uint32_t meta;  // scale | offset << 16 (f16 bits)
  uint32_t tf;    // tail_norm | flags << 16
  uint32_t hdr;   // lanes 0..3: header dwords 0, 1, 4, 5
};

__device__ __forceinline__ MmaRaw mma_load(const uint8_t* idx, const uint4* recs, uint64_t b, uint32_t h) {
  const uint32_t lane = __lane_id(), kh = lane >> 5, v = 32u * h + (lane & 31u);
  const uint8_t* blk = idx + b * kBlockBytes;
  const uint4* rec = recs + (b * 64u + v) * kRecWords;
  MmaRaw r;
  r.lev = rec[kRecLev0 + kh];
  r.r1 = reinterpret_cast<const uint2*>(rec + kRecS1)[kh];
  const uint4 x = rec[kRecS4Meta];
  r.r4 = kh ? x.y : x.x;
  r.meta = x.z;
  r.tf = x.w;
  const uint32_t hw = lane < 2 ? lane : (lane < 4 ? lane + 2 : 0);
  r.hdr = reinterpret_cast<const uint32_t*>(blk)[hw];
  return r;
}

// Candidate appends of one workgroup, staged in LDS.  Each wave owns a
// region of CAP entries and keeps its fill count in a scalar register, so an
// append needs no atomic; a region is written out when nearly full
// (mma_wave_flush) and at the kernel's end (one global reservation per query
// for the workgroup).
template <int W, int CAP>
struct MmaStaging {
  static constexpr int kWaves = W;
  static constexpr int kCap = CAP;  // entries per wave
  uint32_t drop;            // wide entries dropped once made exact (taken off the append count)
  uint32_t lmax[kMmaQ];     // largest lower-bound key written per query (ScanArgs::lmax)
  uint32_t cnt[kMmaQ];      // final flush: entries per query of the workgroup
  uint32_t base[kMmaQ];
  uint32_t wcnt[W][kMmaQ];  // a wave's own flush: entries per query
  uint32_t wbase[W][kMmaQ];
  uint32_t row[W * CAP];
  float acc[W * CAP];       // tile value; the bounds are formed when the entry is written out
  uint8_t q[W * CAP];
};

// The meta values of a slot's record word kRecS4Meta as the tiles use them.
struct MmaMeta {
  float m_scale, m_offset, mid_n, hn;
  bool safe;  // every magnitude within the operand range
};
__device__ __forceinline__ MmaMeta mma_meta(const uint4 x, const float* s_flag) {
  MmaMeta m;
  m.m_scale = h2f((uint16_t)(x.z & 0xffffu));
  m.m_offset = h2f((uint16_t)(x.z >> 16));
  const float tn = fmaxf(h2f((uint16_t)(x.w & 0xffffu)), 0.0f);
  const uint32_t fl = (x.w >> 16) & 0xffu;
  m.mid_n = fmaxf(s_flag[256 + fl] * tn, 1e-6f);
  m.hn = fmaxf(fmaxf(s_flag[fl] * tn, 0.0f), 1e-6f);
  m.safe = fabsf(m.m_scale) <= kMmaSafe && m.mid_n <= kMmaSafe && m.hn <= kMmaSafe && fabsf(m.m_offset) <= kMmaSafe;
  return m;
}

// Bounds (U, L) of a staged pair from its tile value acc = s (U' - tau): the
// query's constants qk = {tau, 1/s, eP, e1, e4, eO, e0, ok} and the slot's
// record word x = kRecS4Meta.  A slot beyond the operand range gets (+inf, -inf).
// wpc != 0: the tile value still holds the stage bounds of a bounded final
// pass: 8 h8 wpc for S4 (wpc = the query's S4 bound column, h8 = 8 high_n
// rounded up to f16) and 3 m8 wpc1 for S1 (wpc1 = its S1 bound column, m8 =
// 8 mid_n rounded up): U stays, L drops by twice the bounds.
__device__ __forceinline__ void mma_bounds_x(float acc, const uint4 x, const float* qk, const float* s_flag, float* U,
                                             float* L, float wpc = 0.0f, float wpc1 = 0.0f) {
  const MmaMeta m = mma_meta(x, s_flag);
  float u = INFINITY, l = -INFINITY;
  if (m.safe) {
    const float4 k0 = *reinterpret_cast<const float4*>(qk);      // tau, 1/s, eP, e1
    const float4 k1 = *reinterpret_cast<const float4*>(qk + 4);  // e4, eO, e0, ok
    const float tau = k0.x;
    const float u0 = tau + acc * k0.y;
    const float E = fabsf(m.m_scale) * k0.z + m.mid_n * k0.w + m.hn * k1.x + fabsf(m.m_offset) * k1.y + k1.z;
    const float mg = (fabsf(u0) + fabsf(tau)) * (1.0f / 4194304.0f);
    const float W = (wpc != 0.0f ? (8.0f * h2f((uint16_t)f16_up(8.0f * m.hn))) * wpc * k0.y : 0.0f) +
                    (wpc1 != 0.0f ? (3.0f * h2f((uint16_t)f16_up(8.0f * m.mid_n))) * wpc1 * k0.y : 0.0f);
    u = u0 + mg;
    l = (u0 - 2.0f * (E + W) * (1.0f + 1.0f / 1048576.0f)) - mg;
    if (!(u == u)) u = INFINITY;
    if (!(l == l)) l = -INFINITY;
  }
  *U = u;
  *L = l;
}
__device__ __forceinline__ void mma_bounds(float acc, const uint4* recs, uint32_t row, const float* qk,
                                           const float* s_flag, float* U, float* L, float wpc = 0.0f,
                                           float wpc1 = 0.0f) {
  mma_bounds_x(acc, recs[(uint64_t)row * kRecWords + kRecS4Meta], qk, s_flag, U, L, wpc, wpc1);
}

// The tile value of a pair from a bounded final pass (see ScanArgs::mma_wide),
// made what the 17 K-steps would give with the e1 and e4 columns counted
// twice (mma_bounds takes 2 e1 and 2 e4 in such a pass).  The eight S4 bound
// columns 8 h8 * piece (h8 = 8 high_n rounded up to f16, piece = s * the
// query's S4 bound / 64 rounded up) are replaced by the S4 steps' sum,
// V4 * sum_d A4[d] (2 b_d - 1) with V4 = f16(high_n * w_s4 / 2) and A4 the
// query's S4 operands (in qa, steps 12..15, element order of mma_dim, bits b
// from the record word x); the three S1 bound columns 8 m8 * piece1 (m8 =
// 8 mid_n rounded up, piece1 = s * the query's S1 bound / 24 rounded up) by
// the S1 steps' sum, V1 * sum_d A1[d] (2 b_d - 1) with V1 = f16(mid_n / 2), A1
// the query's S1 operands (steps 4..11) and b the slot's S1 bits (record word
// x1).  The products are exact and the f32 roundings here (a few 2^-24 of the
// summed magnitudes) are far inside the second e1 / e4 columns.  A slot beyond
// the operand range keeps its value.  U: unroll factor of the operand loops.
// (float)lo + (float)hi of the two f16 halves of w, in one mixed-precision
// FMA (lo * 1 + hi, one rounding to f32: the same value bit for bit).
__device__ __forceinline__ float f16_pair_sum(uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(w));
  return r;
}

template <int U>
__device__ __forceinline__ float mma_tighten_x(float acc, const uint4 x, const uint4 x1, uint32_t qi,
                                               const uint4* qa, const float* s_flag, float ws4) {
  const MmaMeta m = mma_meta(x, s_flag);
  if (!m.safe) return acc;
  const float hn = m.hn;
  const uint32_t ln = qi & 31u;
  const uint4* qt = qa + (uint64_t)(qi >> 5) * (kMmaSteps * 64);
  const uint4 e0 = qt[16 * 64 + ln];  // the error step's query operand, K-half 0
  const float c1 = h2f((uint16_t)(e0.x >> 16));                          // e1 column (element 1)
  const float c4 = h2f((uint16_t)(e0.y & 0xffffu));                      // e4 column (element 2)
  const float pc1 = h2f((uint16_t)(e0.z >> 16));                         // S1 bound column (element 5)
  const float pc = h2f((uint16_t)(qt[16 * 64 + 32 + ln].x & 0xffffu));   // S4 bound column (K-half 1)
  const float hn16 = h2f((uint16_t)f16_bits(hn));
  const float h8 = h2f((uint16_t)f16_up(8.0f * hn));
  const float V = h2f((uint16_t)f16_bits(0.5f * hn * ws4));
  const float mid16 = h2f((uint16_t)f16_bits(m.mid_n));
  const float m8 = h2f((uint16_t)f16_up(8.0f * m.mid_n));
  const float V1 = h2f((uint16_t)f16_bits(0.5f * m.mid_n));
  float S = 0.0f, S1 = 0.0f;
#pragma unroll 1
  for (int kh = 0; kh < 2; ++kh) {
    const uint32_t bits = kh ? x.y : x.x;
#pragma unroll U
    for (int st = 0; st < 4; ++st) {
      const uint4 a4 = qt[(12 + st) * 64 + 32 * kh + ln];
      const uint32_t w[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // the operand pair with each sign flipped where its bit is clear (as the tiles' vector operand)
        const uint32_t sw = w[j] ^ ((~bits << (15 - 4 * st - j)) & 0x80008000u);
        S += f16_pair_sum(sw);
      }
    }
#pragma unroll U
    for (int t = 0; t < 8; ++t) {
      const uint32_t b1 = t < 4 ? (kh ? x1.z : x1.x) : (kh ? x1.w : x1.y);  // dword 2 kh + t / 4
      const uint4 a1 = qt[(4 + t) * 64 + 32 * kh + ln];
      const uint32_t w[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t sw = w[j] ^ ((~b1 << (15 - 4 * (t & 3) - j)) & 0x80008000u);
        S1 += f16_pair_sum(sw);
      }
    }
  }
  const float d = fmaf(hn16, c4, -((8.0f * h8) * pc)) + fmaf(mid16, c1, -((3.0f * m8) * pc1));
  return fmaf(V1, S1, fmaf(V, S, acc + d));
}

// Stages the pairs of pm (one query per lane: qi) as (row, tile value, query)
// in this wave's region; past its end they go straight to the query's
// segment, bounds formed here.  In a pass that bounded S4 (wide) a staged
// pair's query index carries kMmaWideFlag (the flush makes it exact); a
// wide pair written straight out keeps the bound, its lower bound widened
// by twice the bound.
template <typename ST>
__device__ __forceinline__ void mma_append(ST& st, const ScanArgs& a, const float (*s_qk)[8], const float* s_flag,
                                           int wave, uint32_t* fill, uint32_t q0, uint32_t qi, uint32_t seg,
                                           uint64_t pm, float acc, uint32_t row, bool wide, const uint4* qa,
                                           float ws4) {
  const uint32_t lane = __lane_id();
  const uint32_t base = *fill;
  *fill = base + (uint32_t)__popcll(pm);
  if (!((pm >> lane) & 1ull)) return;
  const uint32_t slot = base + lanes_below(pm);
  if (slot < (uint32_t)ST::kCap) {
    const uint32_t e = (uint32_t)wave * ST::kCap + slot;
    st.row[e] = row;
    st.acc[e] = acc;
    st.q[e] = (uint8_t)(wide ? (qi | kMmaWideFlag) : qi);
  } else {
    // (the query index passes through an empty asm so the compiler cannot
    // hoist this rare path's addresses out of the scan loop into registers)
    uint32_t qq = q0 + qi;
    asm volatile("" : "+v"(qq));
    const uint64_t sq = (uint64_t)qq * a.nseg + seg;
    const uint32_t g = atomicAdd(a.seg_count + sq, 1u);
    if (g < a.seg_cap) {
      float u, l;
      // a wide pair keeps the stage bounds: its lower bound is widened by them twice
      const uint4* qe = qa + (uint64_t)((qq - q0) >> 5) * (kMmaSteps * 64) + 16 * 64 + ((qq - q0) & 31u);
      const float wpc = wide ? h2f((uint16_t)(qe[32].x & 0xffffu)) : 0.0f;
      const float wpc1 = wide ? h2f((uint16_t)(qe[0].z >> 16)) : 0.0f;
      mma_bounds(acc, a.recs, row, s_qk[qq - q0], s_flag, &u, &l, wpc, wpc1);
      if (a.lmax) atomicMax(a.lmax + (uint64_t)qq * kMcCount, score_key(l));
      const uint64_t i = sq * a.seg_cap + g;
      a.cand_score[i] = u;
      a.cand_lower[i] = l;
      a.cand_row[i] = row;
    }
  }
}

// A staged entry of a pass that bounded S4 (flag kMmaWideFlag) is made
// exact (mma_tighten_x, x = its record word); one whose upper bound is then
// below the floor is marked kMmaDropped.
template <int U, typename ST>
__device__ __forceinline__ void mma_stage_tighten(ST& st, const float* s_flag, uint32_t i, const uint4 x,
                                                  const uint4 x1, const uint4* qa, float ws4) {
  const uint32_t q8 = st.q[i];
  if (!(q8 & kMmaWideFlag)) return;
  const float t = mma_tighten_x<U>(st.acc[i], x, x1, q8 & 0x7fu, qa, s_flag, ws4);
  st.acc[i] = t;
  if (t < 0.0f) {
    st.q[i] = kMmaDropped;
    atomicAdd(&st.drop, 1u);
  } else {
    st.q[i] = (uint8_t)(q8 & 0x7fu);
  }
}

// Writes out the n entries of this wave's region: a count per query in LDS,
// one global reservation per query with entries, then each entry's bounds
// (wide entries made exact first).  Every entry's record words are requested
// at once, and the bounds use the same words.
template <typename ST>
__device__ __forceinline__ void mma_wave_flush(ST& st, const ScanArgs& a, const float (*s_qk)[8],
                                               const float* s_flag, int wave, uint32_t n, uint32_t q0,
                                               uint32_t seg, bool wide, const uint4* qa, float ws4) {
  constexpr int kPer = ST::kCap / 64;
  const uint32_t lane = __lane_id();
  uint32_t* cnt = st.wcnt[wave];
  uint32_t* base = st.wbase[wave];
  cnt[lane] = 0u;
  uint4 xr[kPer], x1r[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t e = lane + 64u * (uint32_t)k;
    const uint4* rec = a.recs + (uint64_t)(e < n ? st.row[(uint32_t)wave * ST::kCap + e] : 0u) * kRecWords;
    xr[k] = e < n ? rec[kRecS4Meta] : make_uint4(0u, 0u, 0u, 0u);
    x1r[k] = wide && e < n ? rec[kRecS1] : make_uint4(0u, 0u, 0u, 0u);
  }
  if (wide) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const uint32_t e = lane + 64u * (uint32_t)k;
      if (e < n) mma_stage_tighten<4>(st, s_flag, (uint32_t)wave * ST::kCap + e, xr[k], x1r[k], qa, ws4);
    }
  }
  wave_lds_sync();
  uint32_t rk[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t e = lane + 64u * (uint32_t)k;
    const uint32_t q8 = e < n ? st.q[(uint32_t)wave * ST::kCap + e] : kMmaDropped;
    rk[k] = q8 != kMmaDropped ? atomicAdd(&cnt[q8], 1u) : 0u;
  }
  wave_lds_sync();
  const uint32_t c = cnt[lane];
  base[lane] = c ? atomicAdd(a.seg_count + (uint64_t)(q0 + lane) * a.nseg + seg, c) : 0u;
  wave_lds_sync();
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t e = lane + 64u * (uint32_t)k;
    const uint32_t i = (uint32_t)wave * ST::kCap + e;
    if (e < n && st.q[i] != kMmaDropped) {
      const uint32_t qi = st.q[i];
      const uint32_t g = base[qi] + rk[k];
      if (g < a.seg_cap) {
        const uint32_t row = st.row[i];
        float u, l;
        mma_bounds_x(st.acc[i], xr[k], s_qk[qi], s_flag, &u, &l);
        atomicMax(&st.lmax[qi], score_key(l));
        const uint64_t o = ((uint64_t)(q0 + qi) * a.nseg + seg) * a.seg_cap + g;
        a.cand_score[o] = u;
        a.cand_lower[o] = l;
        a.cand_row[o] = row;
      }
    }
  }
  wave_lds_sync();  // the region is read before it is refilled
}

// Floors of a first sampling stage that stored its lower bounds: the
// query's histogram is built in LDS from its n_s values (the bins and the
// values that count are those k_scan_mma's counting form would have added to
// the global histogram), then the floors at `rank` and the safe rank K.
constexpr int kFlbThreads = 1024;
constexpr int kFlbCopies = 4;  // histogram copies (wave % 4): fewer LDS atomics on one address
__global__ __launch_bounds__(kFlbThreads) void k_mma_floors_lb(const float* lbuf, uint32_t lbuf_stride, uint32_t n_s,
                                                              const float* luts, uint32_t rank, uint32_t safe_rank,
                                                              float* floor_out, float* safe_out) {
  __shared__ __align__(16) uint32_t s_h[kFlbCopies][kHistBins];
  const uint32_t q = blockIdx.x, tid = threadIdx.x;
  uint32_t* h = s_h[(tid >> 6) % kFlbCopies];
  const float hinv = luts[(uint64_t)q * kQData + kQdHistInv];
  const float sc = luts[(uint64_t)q * kQData + kQdHistScale];
  for (uint32_t i = tid; i < (uint32_t)(kFlbCopies * kHistBins); i += kFlbThreads) (&s_h[0][0])[i] = 0u;
  __syncthreads();
  const float* row = lbuf + (uint64_t)q * lbuf_stride;
  for (uint32_t i0 = 0; i0 < n_s; i0 += kFlbThreads * 8u) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t i = i0 + kFlbThreads * (uint32_t)u + tid;
      v[u] = i < n_s ? row[i] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (v[u] > -INFINITY) atomicAdd(&h[hist_bin(v[u], hinv)], 1u);
  }
  __syncthreads();
  for (uint32_t i = tid; i < (uint32_t)kHistBins; i += kFlbThreads) {
    uint32_t c = 0;
#pragma unroll
    for (int k = 0; k < kFlbCopies; ++k) c += s_h[k][i];
    s_h[0][i] = c;
  }
  __syncthreads();
  if (tid < 64) {
    const HistRow r = hist_row(s_h[0]);
    const float f = floor_of(r, rank) * sc;
    const float sf = floor_of(r, safe_rank) * sc;
    if (tid == 0) {
      floor_out[q] = f;
      safe_out[q] = sf;
    }
  }
}

// Floors of a later sampling stage that listed its counted lower bounds:
// the query's histogram is built in LDS from the global row (the bounds past
// a list's room; the row is then cleared) and the n_wg workgroup lists, then
// the floors at `rank` and the safe rank K, each at least the previous
// stage's (floor_out / safe_out hold it on entry).  The lists' lengths are
// scanned into offsets, so the threads take the entries of all lists
// together, kSegUnroll loads in flight per thread (entry e: the list whose
// offsets bracket it, by binary search in LDS).
constexpr int kSegThreads = 1024, kSegUnroll = 8;
__global__ __launch_bounds__(kSegThreads) void k_mma_floors_seg(const float* lbuf, const uint32_t* lcount,
                                                               uint32_t lbuf_stride, uint32_t n_wg, uint32_t lcap,
                                                               uint32_t* hist, const float* luts, uint32_t rank,
                                                               uint32_t safe_rank, float* floor_out,
                                                               float* safe_out) {
  static_assert(kMaxListWg == kSegThreads, "one list length per thread");
  __shared__ __align__(16) uint32_t s_h[kHistBins];
  __shared__ uint32_t s_off[2][kMaxListWg + 1];
  const uint32_t q = blockIdx.x, tid = threadIdx.x;
  const float hinv = luts[(uint64_t)q * kQData + kQdHistInv];
  const float sc = luts[(uint64_t)q * kQData + kQdHistScale];
  uint32_t* g = hist + (uint64_t)q * kHistBins;
  const float* row = lbuf + (uint64_t)q * lbuf_stride;
  const uint32_t len = tid < n_wg ? min(lcount[(uint64_t)q * lbuf_stride + tid], lcap) : 0u;
  for (uint32_t i = tid; i < (uint32_t)kHistBins; i += kSegThreads) {
    s_h[i] = g[i];
    g[i] = 0u;
  }
  // inclusive scan of the lengths at offsets 1.. (Hillis-Steele)
  s_off[0][tid + 1] = len;
  if (tid == 0) s_off[0][0] = s_off[1][0] = 0u;
  __syncthreads();
  int cur = 0;
  for (uint32_t d = 1; d < (uint32_t)kMaxListWg; d <<= 1) {
    s_off[cur ^ 1][tid + 1] = s_off[cur][tid + 1] + (tid >= d ? s_off[cur][tid + 1 - d] : 0u);
    cur ^= 1;
    __syncthreads();
  }
  const uint32_t* off = s_off[cur];  // off[w] = entries of lists before w
  const uint32_t total = off[n_wg];
  for (uint32_t e0 = 0; e0 < total; e0 += kSegThreads * kSegUnroll) {
    float v[kSegUnroll];
#pragma unroll
    for (int u = 0; u < kSegUnroll; ++u) {
      const uint32_t e = e0 + kSegThreads * (uint32_t)u + tid;
      v[u] = -INFINITY;
      if (e < total) {
        uint32_t lo = 0, hi = n_wg;  // the last w with off[w] <= e
        while (hi - lo > 1u) {
          const uint32_t mid = (lo + hi) >> 1;
          if (off[mid] <= e) lo = mid;
          else hi = mid;
        }
        v[u] = row[(uint64_t)lo * lcap + (e - off[lo])];
      }
    }
#pragma unroll
    for (int u = 0; u < kSegUnroll; ++u)
      if (v[u] > -INFINITY) atomicAdd(&s_h[hist_bin(v[u], hinv)], 1u);
  }
  __syncthreads();
  if (tid < 64) {
    const HistRow r = hist_row(s_h);
    const float f = floor_of(r, rank) * sc;
    const float sf = floor_of(r, safe_rank) * sc;
    if (tid == 0) {
      floor_out[q] = fmaxf(f, floor_out[q]);
      safe_out[q] = fmaxf(sf, safe_out[q]);
    }
  }
}

// One pass of the MFMA-bounded scan.  Workgroup = 8 waves over the same 64
// queries (blockIdx.y); a wave takes one 32-vector tile (half a block) at a
// time, items i = first + k * stride with block (i / 2) << shift and half
// i % 2; NQT 32-query tiles per wave.  The query operands sit in LDS and are
// read one K-step ahead of the MFMAs that use them, which keeps the register
// file small enough for four waves per SIMD.
// MODE 0: sampling pass, the lower bounds of every active pair go into the
// query's histogram; 3: the same pass storing every pair's lower bound at
// a.lbuf (-inf where it does not count) for k_mma_floors_lb; 4: the
// sampling pass listing the counted lower bounds per workgroup (a.lcount)
// for k_mma_floors_seg; 1: final pass,
// pairs with U >= the floor in a.tau are appended; 2: single pass, every
// active pair is appended.  WIDE (MODE 1): the final pass that bounds the
// S4 stage (ScanArgs::mma_wide).
template <int NQT, int MODE, bool WIDE = false>
__global__ __launch_bounds__(kMmaWaves * 64, 4) void k_scan_mma(ScanArgs a) {
  constexpr int WPG = kMmaWaves;  // waves per workgroup
  constexpr bool SAMPLE = MODE == 0 || MODE == 3 || MODE == 4;  // a sampling pass (lower bounds, no appends)
  using Staging = MmaStaging<WPG, 256>;
  __shared__ __align__(16) uint4 s_qa[NQT][kMmaSteps][64];
  __shared__ uint32_t s_tab[256];
  __shared__ float s_flag[512];      // rho = f / 255, then sqrt(max(1 - rho^2, 0))
  __shared__ __align__(16) float s_c[kMmaQ];
  __shared__ __align__(16) float s_qk[kMmaQ][8];  // tau, 1/s, eP, e1, e4, eO, e0 (with the tau term), ok
  __shared__ float s_hinv[kMmaQ];                 // histogram scale of each query (2^-e, sampling passes)
  __shared__ unsigned int s_stats[kStatCount];
  __shared__ uint32_t s_anyall;  // sampling: some query counts every lower bound
  __shared__ uint32_t s_next;    // final passes: the workgroup's next item number
  __shared__ Staging s_st;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lane = lane_id(), kh = lane >> 5, vl = lane & 31u;
  const uint32_t q0 = blockIdx.y * kMmaQ;
  const int nq = (int)min((uint32_t)kMmaQ, a.n_q - q0);
  if (tid == 0) {
    s_anyall = 0u;
    s_next = 0u;
  }
  __syncthreads();

  // item i: half i % 2 of the block at position i / 2 (pos << shift, or
  // this query chunk's block list)
  const uint32_t* bl = a.blist ? a.blist + (uint64_t)blockIdx.y * a.blist_stride : nullptr;
  const uint32_t n_items = 2u * (bl ? a.bcount[blockIdx.y] : a.n_pos);
  auto block_of = [&](uint32_t pos) -> uint64_t { return bl ? (uint64_t)bl[pos] : (uint64_t)pos << a.shift; };
  const uint32_t stride = gridDim.x * WPG - 1;  // odd: see k_scan
  // The final passes share a workgroup's items among its waves, each wave
  // taking the next from an LDS counter two items ahead (a wave slowed by
  // its appends then takes fewer).  The items: column col = blockIdx.x % n_col
  // (col + n_col j), j in this workgroup's part of the column: all of it,
  // or with ScanArgs::pair_cols (n_col = the CU count) the first
  // kMmaFirstShare / 256 of it for the CU's first workgroup and the rest for
  // its second (a third or later workgroup of a column: equal parts).  The
  // sampling passes keep the fixed stride.
  constexpr bool dyn = !SAMPLE;
  const uint32_t n_col = a.pair_cols ? min(a.pair_cols, gridDim.x) : gridDim.x;
  const uint32_t col = blockIdx.x % n_col, slot = blockIdx.x / n_col;
  const uint32_t n_slot = (gridDim.x - col + n_col - 1u) / n_col;  // workgroups of this column
  const uint32_t col_n = n_items > col ? (n_items - col - 1u) / n_col + 1u : 0u;  // items of this column
  auto cut = [&](uint32_t s) -> uint32_t {  // the column's items before slot s
    if (s >= n_slot) return col_n;
    if (n_slot == 2u) return s ? (uint32_t)(((uint64_t)col_n * kMmaFirstShare) >> 8) : 0u;
    return (uint32_t)((uint64_t)col_n * s / n_slot);
  };
  const uint32_t j_lo = cut(slot), j_n = cut(slot + 1u) - j_lo;
  auto grab = [&]() -> uint32_t {  // the next k (lane 0's value)
    uint32_t k = 0u;
    if (lane == 0u) k = atomicAdd(&s_next, 1u);
    return k;
  };
  auto item_of = [&](uint32_t k) -> uint32_t {  // n_items past the end
    const uint32_t kk = (uint32_t)__builtin_amdgcn_readfirstlane((int)k);
    return kk < j_n ? col + n_col * (j_lo + kk) : n_items;
  };
  uint32_t first = blockIdx.x * WPG + wave;
  uint32_t after = first + stride;  // the item after the current one (n_it or more: none)
  uint32_t pend = 0u;               // (dyn) the k of the item after that, requested one item early
  const uint32_t n_it = dyn || first < stride ? n_items : 0u;
  if (dyn) {
    first = item_of(grab());
    after = item_of(grab());
    pend = grab();
  }
  uint32_t it_cur = first;
  uint64_t b_cur = 0;
  MmaRaw cur{};
  if (first < n_it) {
    b_cur = block_of(first >> 1);
    cur = mma_load(a.idx, a.recs, b_cur, first & 1u);
  }

  if (tid < 256) {  // byte -> (f16 cb[low nibble], f16 cb[high nibble])
    const mrl_query_plan* p0 = a.plans + q0;
    const bool eden = p0->prefix_codec == MRL_PREFIX_EDEN_PROD;
    const uint32_t lo = (uint32_t)tid & 15u, hi = (uint32_t)tid >> 4;
    const float clo = eden ? p0->eden_codebook[lo] : (float)lo;
    const float chi = eden ? p0->eden_codebook[hi] : (float)hi;
    s_tab[tid] = f32_to_f16(clo) | (f32_to_f16(chi) << 16);
  }
  if (tid < 256) {
    s_flag[tid] = a.flag_tabs[tid];
    s_flag[256 + tid] = a.flag_tabs[256 + tid];
  }
  if (tid < kStatCount) s_stats[tid] = 0u;
  if (tid == 0) s_st.drop = 0u;
  if (tid < kMmaQ) s_st.lmax[tid] = 0u;
  if (tid < kMmaQ) {
    const int qi = tid;
    s_st.cnt[qi] = 0u;
    float C = -INFINITY, qk[8] = {0.0f, 1.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (qi < nq) {
      const float* mc = a.mma_consts + (uint64_t)(q0 + qi) * kMcCount;
      const float sc = mc[kMcS], mean = mc[kMcMean], R = mc[kMcR];
      const bool ok = mc[kMcOk] != 0.0f;
      // MODE 1: tau = the floor.  MODE 0: tau = the previous stage's floor;
      // only lower bounds at or above it are counted (all of them without one).
      float tau = 0.0f;
      bool all = false;
      if (MODE != 2) {
        tau = a.tau ? a.tau[q0 + qi] : -INFINITY;
        if (!(tau >= -R)) {
          all = SAMPLE;
          tau = SAMPLE ? 0.0f : -R;  // MODE 1 without a floor: below every score of a vector with safe magnitudes
        }
      }
      if (all) atomicOr(&s_anyall, 1u);
      const float e0q = mc[kMcE0] + fabsf(tau) * (1.0f / 16384.0f);
      if (ok) C = sc * ((mean - tau) + (SAMPLE ? -e0q : e0q));
      qk[0] = tau;
      qk[1] = mc[kMcInvS];
      qk[2] = mc[kMcEP];
      qk[3] = (MODE == 1 && WIDE) ? 2.0f * mc[kMcE1] : mc[kMcE1];  // mma_tighten's second e1 column
      qk[4] = (MODE == 1 && WIDE) ? 2.0f * mc[kMcE4] : mc[kMcE4];  // and second e4 column
      qk[5] = mc[kMcEO];
      qk[6] = e0q;
      qk[7] = ok ? 1.0f : 0.0f;
    }
    s_c[qi] = C;
#pragma unroll
    for (int i = 0; i < 8; ++i) s_qk[qi][i] = qk[i];
    s_hinv[qi] = (SAMPLE && qi < nq) ? a.luts[(uint64_t)(q0 + qi) * kQData + kQdHistInv] : 1.0f;
  }
  // Query operands, element e: tile t, K-step st, lane ln -> query
  // q0 + 32 t + ln % 32, K-half ln / 32.  Every thread's loads go out first (from a clamped query
  // index), then the stores, zeroed past the batch.
  constexpr int kQaN = NQT * kMmaSteps * 64, kQaPer = (kQaN + 64 * WPG - 1) / (64 * WPG);
  uint4 qav[kQaPer];
#pragma unroll
  for (int k = 0; k < kQaPer; ++k) {
    const int e = min(tid + 64 * WPG * k, kQaN - 1);
    const int t = e / (kMmaSteps * 64), st = (e / 64) % kMmaSteps, ln = e & 63;
    const int qi = 32 * t + (ln & 31), qc = qi < nq ? qi : nq - 1;
    qav[k] = a.mma_ops[(uint64_t)(q0 + qc) * (2 * kMmaSteps) + 2 * st + (ln >> 5)];
  }
#pragma unroll
  for (int k = 0; k < kQaPer; ++k) {
    const int e = tid + 64 * WPG * k;
    if (e < kQaN) {
      const int t = e / (kMmaSteps * 64), st = (e / 64) % kMmaSteps, ln = e & 63;
      uint4 v = 32 * t + (ln & 31) < nq ? qav[k] : make_uint4(0u, 0u, 0u, 0u);
      if (SAMPLE && (ln >> 5) == 0 && st == kMmaSteps - 1) {  // the sampling pass subtracts the error columns
        v.x ^= 0x80008000u;
        v.y ^= 0x80008000u;
      }
      s_qa[t][st][ln] = v;
    }
  }
  auto qa_raw = [&](int t, int st) -> uint4 { return s_qa[t][st][lane]; };
  __syncthreads();

  const float ws4 = a.sp.strata == MRL_STRATA_FULL64B ? a.sp.w_s4 : 0.0f;
  const uint32_t seg = blockIdx.x % a.nseg;
  uint32_t c_blocks = 0, c_active = 0, c_app = 0;
  // final pass bounding S4 (wave-uniform; off for good once the wave's
  // appends pass its allowance)
  constexpr bool wide_pass = MODE == 1 && WIDE;
  bool wide = wide_pass;
  uint32_t w_items = 0, w_app = 0;
  const uint32_t w_lim = (32u * (uint32_t)nq * a.wide_lim) >> 10;  // appends per item
  const uint4* qa = &s_qa[0][0][0];
  uint32_t fill = 0;  // entries of this wave's staging region (wave-uniform)
  // bit 16 t + r: register r of tile t belongs to a query of the batch with
  // usable operands (read only on the rare paths that force candidates)
  uint32_t okbits = 0u;
  if constexpr (!SAMPLE) {
#pragma unroll
    for (int t = 0; t < NQT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
        if (qi < nq && s_qk[qi][7] != 0.0f) okbits |= 1u << (16 * t + r);
      }
    asm volatile("" : "+v"(okbits));  // one register, not 32 hoisted masks
  }

  // On block lists, a final pass reads the block of the item after next one
  // item early, so the list read does not delay the record loads of the next
  // item.  (The sampling passes keep the register.)
  const bool pre = !SAMPLE && bl != nullptr;
  uint64_t b_pre = 0;
  if (pre && after < n_it) b_pre = block_of(after >> 1);
  for (uint32_t it = first; it < n_it;) {
    const uint32_t it_adv = after;  // the next item
    if (dyn) {
      after = item_of(pend);
      pend = grab();
    } else {
      after = it_adv + stride;
    }
    const uint32_t it_nxt = it_adv < n_it ? it_adv : it_cur;
    uint64_t b_nxt = b_cur;
    if (it_adv < n_it) b_nxt = pre ? b_pre : block_of(it_nxt >> 1);
    if (pre && after < n_it) b_pre = block_of(after >> 1);
    const MmaRaw nxt = mma_load(a.idx, a.recs, b_nxt, it_nxt & 1u);
    const uint32_t b = (uint32_t)b_cur, h = it_cur & 1u;
    const uint32_t min_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 0);
    const uint32_t max_ts = (uint32_t)__builtin_amdgcn_readlane(cur.hdr, 1);
    const uint64_t tomb = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 3) << 32) |
                          (uint64_t)(uint32_t)__builtin_amdgcn_readlane(cur.hdr, 2);
    bool skip = false;
    if (a.sp.temporal) {  // scan.rs:719-730
      if (a.sp.has_lo && max_ts < a.sp.lo) skip = true;
      if (a.sp.has_hi && min_ts > a.sp.hi) skip = true;
    }
    const uint32_t active = (uint32_t)(~tomb >> (32u * h));  // this tile's slots
    if (MODE == 3 && (skip || active == 0)) {
      // a skipped tile stores no lower bounds that count
      float* lrow = a.lbuf + (uint64_t)(q0 + 4u * kh) * a.lbuf_stride + 32u * it_cur + vl;
#pragma unroll
      for (int t = 0; t < NQT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
          if (qi < nq) lrow[(uint64_t)(32 * t + 8 * (r >> 2) + (r & 3)) * a.lbuf_stride] = -INFINITY;
        }
    }
    if (!skip && active != 0) {
      if (h == 0) {
        c_blocks += (uint32_t)nq;
        c_active += (uint32_t)nq * (uint32_t)__popcll(~tomb);
      }
      const uint32_t v = 32u * h + vl;
      const bool act = (active >> vl) & 1u;
      // meta (block.rs:61-99); flags / 255 and sqrt(max(1 - rho^2, 0)) from the context's tables
      const uint32_t sc_b = cur.meta & 0xffffu, of_b = cur.meta >> 16;
      const float m_scale = h2f((uint16_t)sc_b), m_offset = h2f((uint16_t)of_b);
      const float tn = fmaxf(h2f((uint16_t)(cur.tf & 0xffffu)), 0.0f);
      const uint32_t fl = cur.tf >> 16;
      const float mid_n = fmaxf(s_flag[256 + fl] * tn, 1e-6f);
      const float hn = fmaxf(fmaxf(s_flag[fl] * tn, 0.0f), 1e-6f);
      const bool safe = fabsf(m_scale) <= kMmaSafe && mid_n <= kMmaSafe && hn <= kMmaSafe &&
                        fabsf(m_offset) <= kMmaSafe;
      mma_f16 acc[NQT];
#pragma unroll
      for (int t = 0; t < NQT; ++t) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 c4 = *reinterpret_cast<const float4*>(&s_c[32 * t + 8 * g + 4 * (int)kh]);
          acc[t][4 * g + 0] = c4.x;
          acc[t][4 * g + 1] = c4.y;
          acc[t][4 * g + 2] = c4.z;
          acc[t][4 * g + 3] = c4.w;
        }
      }
      // The vector operand of K-step st: prefix scale * cb[level] (8 dims per
      // step, the 16 table reads issued together), S1 +-mid_n / 2 and S4
      // +-hn w_s4 / 2 by bit (zero without a tail stage), then the error
      // columns and offset * prefix_sum.
      const mma_h2 sc2 = __builtin_bit_cast(mma_h2, sc_b | (sc_b << 16));
      const uint32_t lw[4] = {cur.lev.x, cur.lev.y, cur.lev.z, cur.lev.w};
      uint32_t tv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) tv[i] = s_tab[(lw[i >> 2] >> (8 * (i & 3))) & 255u];
      const uint32_t hp1 = f16_bits(0.5f * mid_n) * 0x10001u;
      const uint32_t hp4 = f16_bits(0.5f * hn * ws4) * 0x10001u;
      auto vec_op = [&](int st) -> uint4 {
        uint32_t d[4];
        if (st < 4) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            d[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(mma_h2, tv[4 * st + j]) * sc2);
        } else if (st < 12) {
          const int tt = st - 4;
          const uint32_t nx = ~(tt < 4 ? cur.r1.x : cur.r1.y);
          const int jb = 4 * (tt & 3);
#pragma unroll
          for (int j = 0; j < 4; ++j) d[j] = hp1 | ((nx << (15 - jb - j)) & 0x80008000u);
        } else if (st < 16) {
          const int tt = st - 12;
          const uint32_t nx = ~cur.r4;
#pragma unroll
          for (int j = 0; j < 4; ++j) d[j] = hp4 | ((nx << (15 - 4 * tt - j)) & 0x80008000u);
        } else {
          // K-half 0: the error columns and the offset; K-half 1: zero.  In a
          // bounded pass K-half 0 also carries the S1 bound columns (elements
          // 5..7: 8 mid_n rounded up, 3 times) and K-half 1 the S4 bound
          // columns (8 high_n rounded up), as mma_tighten takes them.  Both
          // halves' words are formed and each lane takes its own (no branch
          // on the lane's half).
          uint32_t e2 = of_b, e3 = 0u, k1 = 0u;
          if (MODE == 1 && wide) {
            const uint32_t m8 = f16_up(8.0f * mid_n);
            e2 |= m8 << 16;
            e3 = m8 * 0x10001u;
            k1 = f16_up(8.0f * hn) * 0x10001u;
          }
          d[0] = kh ? k1 : (sc_b & 0x7fffu) | (f16_bits(mid_n) << 16);
          d[1] = kh ? k1 : f16_bits(hn) | ((of_b & 0x7fffu) << 16);
          d[2] = kh ? k1 : e2;
          d[3] = kh ? k1 : e3;
        }
        return make_uint4(d[0], d[1], d[2], d[3]);
      };
      // The query operands of step nst are requested before step st's
      // MFMAs, so their LDS latency overlaps the matrix work.  A final pass
      // raises the wave's issue priority while it feeds the matrix unit
      // (the other waves' epilogues and operand builds take the slots left).
      if constexpr (MODE == 1) __builtin_amdgcn_s_setprio(2);
      uint4 an[NQT];
#pragma unroll
      for (int t = 0; t < NQT; ++t) an[t] = qa_raw(t, 0);
      auto kstep = [&](int st, int nst) {
        uint4 ac[NQT];
#pragma unroll
        for (int t = 0; t < NQT; ++t) ac[t] = an[t];
        if (nst >= 0) {
#pragma unroll
          for (int t = 0; t < NQT; ++t) an[t] = qa_raw(t, nst);
        }
        // In the final passes the next step's reads stay ahead of this
        // step's MFMAs (left to itself the scheduler sinks each read to just
        // before its MFMA, which then waits out the LDS latency; the
        // sampling passes keep that order, which spills less there).
        if constexpr (!SAMPLE) __builtin_amdgcn_sched_barrier(0);
        const uint4 bo = vec_op(st);
#pragma unroll
        for (int t = 0; t < NQT; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_h8(ac[t]), as_h8(bo), acc[t], 0, 0, 0);
      };
      if constexpr (wide_pass) {
#pragma unroll
        for (int st = 0; st < 3; ++st) kstep(st, st + 1);
        kstep(3, wide ? 16 : 4);
        if (!wide) {  // else the S1 and S4 stages' scores are bounded in step 16
#pragma unroll
          for (int st = 4; st < 16; ++st) kstep(st, st + 1);
        }
        kstep(16, -1);
        static_assert(kMmaSteps == 17, "the step schedule above assumes prefix 4, S1 8, S4 4, error 1");
      } else {
#pragma unroll
        for (int st = 0; st < kMmaSteps; ++st) kstep(st, st + 1 < kMmaSteps ? st + 1 : -1);
      }
      if constexpr (MODE == 1) __builtin_amdgcn_s_setprio(0);
      // Register r of tile t holds query 32 t + 8 (r / 4) + 4 kh + r % 4.
      if constexpr (MODE == 3) {
        // store every pair's lower bound (sample 32 it + lane % 32 of the query)
        const bool cnt = act && safe;
        float* lrow = a.lbuf + (uint64_t)(q0 + 4u * kh) * a.lbuf_stride + 32u * it_cur + vl;
#pragma unroll
        for (int t = 0; t < NQT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
            if (qi >= nq) continue;
            const float2 k = *reinterpret_cast<const float2*>(&s_qk[qi][0]);  // tau, 1/s
            float L = k.x + acc[t][r] * k.y;
            L = L - (fabsf(L) + fabsf(k.x)) * (1.0f / 4194304.0f);
            if (!cnt || s_qk[qi][7] == 0.0f || !(acc[t][r] >= 0.0f || s_anyall != 0u)) L = -INFINITY;
            lrow[(uint64_t)(32 * t + 8 * (r >> 2) + (r & 3)) * a.lbuf_stride] = L;
          }
      } else if constexpr (MODE == 4) {
        // As MODE 0, but a counted lower bound joins this workgroup's list
        // for its query: one LDS reservation per half-wave (the two halves
        // hold different queries), then a plain store; past the list's room
        // it is counted in the global histogram instead.
        const uint64_t cm = ballot(act && safe);
        const bool all = s_anyall != 0u;
#pragma unroll
        for (int t = 0; t < NQT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            uint64_t pm = (all ? ~0ull : ballot(acc[t][r] >= 0.0f)) & cm;
            if (pm == 0) continue;
            const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
            pm &= ballot(qi < nq && s_qk[qi][7] != 0.0f);
            if (pm == 0) continue;
            const uint32_t n_lo = (uint32_t)__popcll(pm & 0xffffffffull), n_hi = (uint32_t)__popcll(pm >> 32);
            uint32_t qq = (uint32_t)qi;  // through an empty asm: no hoisted per-register addresses
            asm volatile("" : "+v"(qq));
            uint32_t base = 0u;
            if ((lane == 0u && n_lo != 0u) || (lane == 32u && n_hi != 0u))
              base = atomicAdd(&s_st.cnt[qq], kh ? n_hi : n_lo);
            const uint32_t b_lo = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
            const uint32_t b_hi = (uint32_t)__builtin_amdgcn_readlane((int)base, 32);
            if (!((pm >> lane) & 1ull)) continue;
            const uint32_t slot = (kh ? b_hi - n_lo : b_lo) + lanes_below(pm);
            const float2 k = *reinterpret_cast<const float2*>(&s_qk[qq][0]);  // tau, 1/s
            float L = k.x + acc[t][r] * k.y;
            L = L - (fabsf(L) + fabsf(k.x)) * (1.0f / 4194304.0f);
            const uint32_t q = q0 + qq;
            if (slot < a.lcap)
              a.lbuf[(uint64_t)q * a.lbuf_stride + blockIdx.x * a.lcap + slot] = L;
            else
              atomicAdd(a.hist + (uint64_t)q * kHistBins + hist_bin(L, s_hinv[qq]), 1u);
          }
      } else if constexpr (MODE == 0) {
        // Tile value = s (L - tau): the pairs at or above the previous floor
        // pass a compare; without one (some query counts all) every pair of
        // a present query is counted.  L = tau + value / s, less a margin
        // for that addition's rounding.
        const uint64_t cm = ballot(act && safe);
        const bool all = s_anyall != 0u;
#pragma unroll
        for (int t = 0; t < NQT; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const uint64_t pm = (all ? ~0ull : ballot(acc[t][r] >= 0.0f)) & cm;
            if (pm == 0 || !((pm >> lane) & 1ull)) continue;
            const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
            if (qi >= nq) continue;
            const float2 k = *reinterpret_cast<const float2*>(&s_qk[qi][0]);  // tau, 1/s
            if (s_qk[qi][7] == 0.0f) continue;
            float L = k.x + acc[t][r] * k.y;
            L = L - (fabsf(L) + fabsf(k.x)) * (1.0f / 4194304.0f);
            uint32_t qq = q0 + qi;  // through an empty asm: no hoisted per-register addresses
            asm volatile("" : "+v"(qq));
            atomicAdd(a.hist + (uint64_t)qq * kHistBins + hist_bin(L, s_hinv[qi]), 1u);
          }
      } else {
        // Absent queries and those with unusable operands start at C = -inf,
        // so acc >= 0 only holds for pairs of the batch.  A slot whose meta is
        // beyond the operand range is a candidate of every present query: its
        // registers are raised to +inf (its bounds are then taken as +-inf);
        // MODE 2 takes every present query's register as it is.
        const uint32_t c_app0 = c_app;
        const uint64_t actm = ballot(act);
        if (MODE == 1 && ballot(act && !safe) != 0) {
#pragma unroll
          for (int t = 0; t < NQT; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (!safe && ((okbits >> (16 * t + r)) & 1u)) acc[t][r] = INFINITY;
        }
        const uint32_t row = b * 64u + v;
#pragma unroll
        for (int t = 0; t < NQT; ++t)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            // MODE 1: one compare per group of four registers (four queries)
            // first.  The IEEE maximum (v_maximum3_f32, no quieting of its
            // inputs) is NaN where a register is: such a group is checked
            // register by register, so a group passes whenever a register
            // of it passes.
            if (MODE == 1) {
              const float m4 =
                  __builtin_elementwise_maximum(__builtin_elementwise_maximum(acc[t][4 * g], acc[t][4 * g + 1]),
                                                __builtin_elementwise_maximum(acc[t][4 * g + 2], acc[t][4 * g + 3]));
              if ((ballot(!(m4 < 0.0f)) & actm) == 0) continue;
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const int r = 4 * g + rr;
              const uint64_t pm =
                  (MODE == 2 ? ballot((okbits >> (16 * t + r)) & 1u) : ballot(acc[t][r] >= 0.0f)) & actm;
              if (pm == 0) continue;
              const int qi = 32 * t + 8 * (r >> 2) + 4 * (int)kh + (r & 3);
              c_app += (uint32_t)__popcll(pm);
              mma_append(s_st, a, s_qk, s_flag, wave, &fill, q0, (uint32_t)qi, seg, pm, acc[t][r], row,
                         MODE == 1 && wide, qa, ws4);
            }
          }
        if (MODE == 1 && wide) {
          ++w_items;
          w_app += c_app - c_app0;
          if (w_app > w_items * w_lim + kMmaWideSlack) wide = false;
        }
        // A region that may not hold the next tile's pairs is written out
        // now, while this tile's registers are free.  (Pairs past a region's
        // end go straight to their segments.)
        if (fill > (uint32_t)Staging::kCap - kMmaFlushRoom) {
          mma_wave_flush(s_st, a, s_qk, s_flag, wave, min(fill, (uint32_t)Staging::kCap), q0, seg, wide_pass, qa,
                         ws4);
          fill = 0u;
        }
      }
    }
    cur = nxt;
    it_cur = it_nxt;
    b_cur = b_nxt;
    it = it_adv;
  }
  if (a.stats && lane == 0) {
    atomicAdd(&s_stats[kStatBlocks], c_blocks);
    atomicAdd(&s_stats[kStatActive], c_active);
    atomicAdd(&s_stats[kStatPrefix], c_app);
  }
  if constexpr (MODE == 4) {  // the length of each query's list
    __syncthreads();
    if (tid < nq) a.lcount[(uint64_t)(q0 + tid) * a.lbuf_stride + blockIdx.x] = min(s_st.cnt[tid], a.lcap);
  }
  if constexpr (!SAMPLE) {
    // Each wave writes out its own region (entry lane + 64 k, as its flushes
    // in the loop): its record words requested at once, then (bounded pass)
    // the entries made exact and the survivors counted per query, without
    // waiting for the other waves; then one reservation per query for the
    // workgroup and each entry's bounds from the same record words.
    constexpr int kFl = Staging::kCap / 64;
    const uint32_t nf = min(fill, (uint32_t)Staging::kCap);
    const uint32_t r0 = (uint32_t)wave * Staging::kCap;
    uint4 xr[kFl];  // the record words with the meta / S4 bits
    {
      uint4 x1r[kFl];  // (bounded pass) the S1 bits
#pragma unroll
      for (int k = 0; k < kFl; ++k) {
        const uint32_t e = lane + 64u * (uint32_t)k;
        const uint4* rec = a.recs + (uint64_t)(e < nf ? s_st.row[r0 + e] : 0u) * kRecWords;
        xr[k] = e < nf ? rec[kRecS4Meta] : make_uint4(0u, 0u, 0u, 0u);
        x1r[k] = wide_pass && e < nf ? rec[kRecS1] : make_uint4(0u, 0u, 0u, 0u);
      }
      if (wide_pass) {
#pragma unroll
        for (int k = 0; k < kFl; ++k) {
          const uint32_t e = lane + 64u * (uint32_t)k;
          if (e < nf) mma_stage_tighten<8>(s_st, s_flag, r0 + e, xr[k], x1r[k], qa, ws4);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kFl; ++k) {
      const uint32_t e = lane + 64u * (uint32_t)k;
      if (e < nf && s_st.q[r0 + e] != kMmaDropped) atomicAdd(&s_st.cnt[s_st.q[r0 + e]], 1u);
    }
    __syncthreads();
    if (tid < nq) {
      const uint32_t c = s_st.cnt[tid];
      s_st.base[tid] = c ? atomicAdd(a.seg_count + (uint64_t)(q0 + tid) * a.nseg + seg, c) : 0u;
      s_st.cnt[tid] = 0u;
    }
    if (a.stats && tid < kStatCount) {
      // appends count the pairs whose bound reached the floor: less those a wide pass dropped
      const uint32_t v = s_stats[tid] - (tid == kStatPrefix ? s_st.drop : 0u);
      const uint32_t copy = (blockIdx.x + blockIdx.y * gridDim.x) % (uint32_t)kStatCopies;
      if (v) atomicAdd(a.stats + copy * kStatCount + tid, (unsigned long long)v);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kFl; ++k) {
      const uint32_t e = lane + 64u * (uint32_t)k, i = r0 + e;
      if (e >= nf) continue;
      const uint32_t qi = s_st.q[i];
      if (qi == kMmaDropped) continue;
      const uint32_t g = s_st.base[qi] + atomicAdd(&s_st.cnt[qi], 1u);
      if (g < a.seg_cap) {
        const uint64_t o = ((uint64_t)(q0 + qi) * a.nseg + seg) * a.seg_cap + g;
        const uint32_t row = s_st.row[i];
        float u, l;
        mma_bounds_x(s_st.acc[i], xr[k], s_qk[qi], s_flag, &u, &l);
        atomicMax(&s_st.lmax[qi], score_key(l));
        a.cand_score[o] = u;
        a.cand_lower[o] = l;
        a.cand_row[o] = row;
      }
    }
    if (a.lmax) {
      __syncthreads();
      if (tid < nq && s_st.lmax[tid]) atomicMax(a.lmax + (uint64_t)(q0 + tid) * kMcCount, s_st.lmax[tid]);
    }
  }
}

// The reference's full score of slot `row` for plan p (scan.rs:453-634, every
// stage run, the f32 operations of eval_block in their order).  False when a
// stage bound of the reference is NaN: NaN >= tau is false, so the reference
// drops such a vector before it is pushed.
__device__ bool exact_full(const FinishArgs& a, const mrl_query_plan* p, uint32_t row, const float* lut,
                           const float* w1, const float* w4, float* out) {
  // the slot's record: one 64-byte line holds every value the stages read
  const uint4* rec = a.recs + (uint64_t)row * kRecWords;
  const uint4 n0 = rec[kRecLev0], n1 = rec[kRecLev1], r1 = rec[kRecS1], x = rec[kRecS4Meta];
  LaneBlock m;
  m.scale = h2f((uint16_t)(x.z & 0xFFFFu));
  m.offset = h2f((uint16_t)(x.z >> 16));
  m.tail = h2f((uint16_t)(x.w & 0xFFFFu));
  const uint32_t flags = (x.w >> 16) & 0xFFu;
  m.nib[0] = n0.x;
  m.nib[1] = n0.y;
  m.nib[2] = n0.z;
  m.nib[3] = n0.w;
  m.nib[4] = n1.x;
  m.nib[5] = n1.y;
  m.nib[6] = n1.z;
  m.nib[7] = n1.w;
  const float t = fmaxf(m.tail, 0.0f);
  const float rho = (float)flags / 255.0f;
  const float rc = rho > 1.0f ? 1.0f : rho;
  const float mid_n = fmaxf(sqrtf(fmaxf(1.0f - rc * rc, 0.0f)) * t, 1e-6f);
  const float high_n = fmaxf(rho * t, 0.0f);
  const float acc = prefix_acc(m, lut);
  const bool eden = p->prefix_codec == MRL_PREFIX_EDEN_PROD;
  const float prefix_ip = eden ? p->eden_mean_ip + m.scale * acc : acc * m.scale + m.offset * p->prefix_sum;
  const float alpha = a.sp.alpha;
  const float ub1 = prefix_ip + alpha * (p->q_mid_norm * mid_n + p->q_tail_norm * high_n);  // scan.rs:499-505
  if (ub1 != ub1) return false;
  float score = prefix_ip;
  // Stage: mid-band 1-bit IP (scan.rs:553-568)
  const uint32_t bits1[4] = {r1.x, r1.y, r1.z, r1.w};
  const float s1 = row_sum<4>(p->rabitq_base, bits1, w1);
  score = score + s1 * mid_n;
  const float ub2 = score + alpha * p->q_after_s1 * high_n;  // scan.rs:572-584
  if (ub2 != ub2) return false;
  if (a.sp.strata == MRL_STRATA_FULL64B) {
    const float hn = fmaxf(high_n, 1e-6f);
    if (p->has_tail_fold && p->s4_abs_budget > 0.0f) {  // scan.rs:587-607
      const float ub3 = score + alpha * hn * a.sp.w_s4 * p->s4_abs_budget;
      if (ub3 != ub3) return false;
    }
    if (p->has_tail_fold) {  // scan.rs:610-634
      const uint32_t bits4[2] = {x.x, x.y};
      const float s4 = row_sum<2>(p->tail_fold_base, bits4, w4);
      score = score + s4 * hn * a.sp.w_s4;
    }
  }
  *out = score;
  return true;
}

constexpr int kFinThreads = 1024;

// Log-scale bin of a key distance d: d itself below 64, else 64 bins per
// octave (the leading bit's position and the 6 bits after it); monotone in d,
// bins 0..1727.
__device__ __forceinline__ uint32_t dist_bin(uint32_t d) {
  if (d < 64u) return d;
  const uint32_t e = 31u - (uint32_t)__clz((int)d);
  return ((e - 5u) << 6) | ((d >> (e - 6u)) & 63u);
}
// The largest distance in bin b.
__device__ __forceinline__ uint64_t dist_bin_top(uint32_t b) {
  if (b < 64u) return b;
  const uint32_t e = (b >> 6) + 5u, m = b & 63u;
  return ((uint64_t)(65u + m) << (e - 6u)) - 1u;
}

// One query: the K-th best lower bound among its candidates (exact radix
// select on the order-preserving key), the candidates whose upper bound
// reaches it, their exact scores, and those at or above the final floor
// written back as the query's candidate list (segments in order) for
// k_select.  A query whose candidate list overflowed, whose operands were
// not finite, or with more such candidates than its list room gets a count past
// the segment room, which k_select reports as an overflow (dense re-run).
__global__ __launch_bounds__(kFinThreads, 8) void k_finish(FinishArgs a) {
  __shared__ uint32_t s_hist[2048];
  __shared__ uint32_t s_off[kSegs + 1];
  __shared__ uint32_t s_coff[kSegs + 1];
  __shared__ uint32_t s_ws[32];
  __shared__ uint32_t s_misc[8];

  const uint32_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const uint32_t K = a.k;
  uint32_t* qcount = a.seg_count + (uint64_t)q * a.nseg;
  const uint32_t c_own = tid < (int)a.nseg ? qcount[tid] : 0u;
  const bool ok = a.mma_consts[(uint64_t)q * kMcCount + kMcOk] != 0.0f;
  const uint64_t qbase = (uint64_t)q * a.nseg * a.seg_cap;
  uint32_t* list = reinterpret_cast<uint32_t*>(a.cand_lower + qbase);  // written once the walks are done
  if (tid < 8) s_misc[tid] = 0u;
  __syncthreads();
  if (c_own > a.seg_cap || !ok) atomicOr(&s_misc[7], 1u);
  seg_offsets(c_own, a.nseg, a.seg_cap, s_off, s_coff, s_ws);
  if (s_misc[7]) {
    if (tid == 0) {
      qcount[0] = a.seg_cap + 1u;
      list[0] = 0u;
    }
    return;
  }
  const uint32_t total = s_off[a.nseg];

  // A key at or below the K-th largest lower-bound key (all candidates when
  // there are at most K): the largest key, then a histogram of each key's
  // distance below it on a log scale, so candidates crowded just under the
  // top spread over many bins.
  uint32_t tkey = 0u;
  if (total > K) {
    const CandView vl{a.cand_lower + qbase, a.cand_row + qbase, a.seg_cap, a.nseg, s_off, s_coff};
    // the largest key: the final pass kept it (kMcLMax), so no walk finds it
    // here.  A key above it (which the pass's own bookkeeping rules out)
    // would count at distance 0, which keeps the boundary below the K-th key.
    const uint32_t kmax = reinterpret_cast<const uint32_t*>(a.mma_consts)[(uint64_t)q * kMcCount + kMcLMax];
    for (int i = tid; i < 2048; i += kFinThreads) s_hist[i] = 0u;
    __syncthreads();
    for_each_cand<16>(vl, [&](float sc, uint32_t) {
      const uint32_t k = score_key(sc);
      atomicAdd(&s_hist[dist_bin(k < kmax ? kmax - k : 0u)], 1u);
    });
    __syncthreads();
    find_boundary(s_hist, 2048, K, false, &s_misc[3], &s_misc[4], s_ws);
    __syncthreads();
    const uint64_t dhi = dist_bin_top(s_misc[3]);
    tkey = dhi < (uint64_t)kmax ? kmax - (uint32_t)dhi : 0u;
  }
  // candidates whose upper bound reaches it, listed over the lower-bound area
  // (every read of it is done): count at list[0], rows from list[1], room
  // for fin_cap of them
  const uint32_t fin_cap = fin_room(a.nseg, a.seg_cap);
  const CandView vu{a.cand_score + qbase, a.cand_row + qbase, a.seg_cap, a.nseg, s_off, s_coff};
  for_each_pair(vu, [&](float u, uint32_t row, uint32_t) {
    if (score_key(u) >= tkey) {
      const uint32_t slot = atomicAdd(&s_misc[2], 1u);
      if (slot < fin_cap) list[1 + slot] = row;
    }
  });
  __syncthreads();
  const uint32_t nf = s_misc[2];
  if (nf > fin_cap) {
    if (tid == 0) {
      qcount[0] = a.seg_cap + 1u;
      list[0] = 0u;
    }
    return;
  }
  if (tid == 0) {
    list[0] = nf;
    // k_exact's work items of this query: (q, chunk) for every kExactItem entries
    const uint32_t items = (nf + kExactItem - 1) / kExactItem;
    s_misc[6] = items ? atomicAdd(a.work, items) : 0u;
  }
  __syncthreads();
  if ((uint32_t)tid < (nf + kExactItem - 1) / kExactItem) a.work[2 + s_misc[6] + tid] = (q << 8) | (uint32_t)tid;
  if (tid < (int)a.nseg) qcount[tid] = 0u;  // k_exact appends from zero
  if (a.stats && tid == 0 && nf) {
    const uint32_t copy = q % (uint32_t)kStatCopies;
    atomicAdd(a.stats + copy * kStatCount + kStatS1, (unsigned long long)nf);
    atomicAdd(a.stats + copy * kStatCount + kStatS4Budget, (unsigned long long)nf);
  }
}

// Exact scores of the listed candidates.  Work item = kExactItem entries of
// one query's list, one per thread; workgroups loop over the item list
// k_finish published (work[0] items at work[2..]).  Scores at or above
// the final floor are appended (one atomic per wave) to segment item % nseg
// of the query; a NaN score sets the query's error flag, as a NaN survivor
// does on the exact path.
__global__ __launch_bounds__(kExactItem) void k_exact(FinishArgs a) {
  // the query's LUT (1024 floats), then its S1 (128) and S4 (64) weights:
  // the first 1216 floats of its scan data, 304 float4
  __shared__ __align__(16) float4 s_qd4[(kQdW4 + 64) / 4];
  static_assert(kQdLut == 0 && kQdW1 == 1024 && kQdW4 == 1152, "scan data layout");
  const float* s_lut = reinterpret_cast<const float*>(s_qd4);
  const uint32_t n_items = a.work[0];
  const int tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  // A contiguous run of items per workgroup: the items of one query are
  // published together, so the query's tables are loaded once per run.
  const uint32_t per = (n_items + gridDim.x - 1) / gridDim.x;
  const uint32_t i0 = blockIdx.x * per, i1 = min(i0 + per, n_items);
  uint32_t q_have = ~0u;
  uint32_t wi = i0 < i1 ? a.work[2 + i0] : 0u;
  for (uint32_t item = i0; item < i1; ++item) {
    const uint32_t q = wi >> 8, c = wi & 255u;
    // next item's descriptor, in flight during this one
    wi = item + 1 < i1 ? a.work[2 + item + 1] : 0u;
    if (q >= a.n_q) continue;
    const uint64_t qbase = (uint64_t)q * a.nseg * a.seg_cap;
    const uint32_t* list = reinterpret_cast<const uint32_t*>(a.cand_lower + qbase);
    // the count, this thread's row (read whether or not it is below the
    // count: the list area holds 1 + fin_room entries), the floor and the
    // tables all go out together
    const uint32_t room = fin_room(a.nseg, a.seg_cap);
    const uint32_t i = c * (uint32_t)kExactItem + (uint32_t)tid;
    const uint32_t nf_raw = list[0];
    const uint32_t row_raw = list[1 + min(i, room - 1u)];
    const float floor_t = a.tau_final ? a.tau_final[q] : -INFINITY;
    if (q != q_have) {
      const float4* qd4 = reinterpret_cast<const float4*>(a.luts + (uint64_t)q * kQData);
      const float4 v0 = qd4[tid];
      const float4 v1 = qd4[kExactItem + (tid < 48 ? tid : 0)];
      __syncthreads();  // the previous query's table reads are done
      s_qd4[tid] = v0;
      if (tid < 48) s_qd4[kExactItem + tid] = v1;
      __syncthreads();
      q_have = q;
    }
    const uint32_t nf = min(nf_raw, room);
    if (c * (uint32_t)kExactItem >= nf) continue;
    bool keep = false;
    float sc = 0.0f;
    uint32_t row = 0u;
    if (i < nf) {
      row = row_raw;
      if ((uint64_t)(row >> 6) < a.n_blocks &&
          exact_full(a, a.plans + q, row, s_lut, s_lut + kQdW1, s_lut + kQdW4, &sc)) {
        if (sc != sc) atomicOr(a.err + q, 1u);
        else keep = sc >= floor_t;
      }
    }
    const uint64_t pm = ballot(keep);
    if (pm == 0) continue;
    const uint32_t seg = c % a.nseg;
    const uint64_t sq = (uint64_t)q * a.nseg + seg;
    const uint32_t lead = (uint32_t)__ffsll((long long)pm) - 1;
    uint32_t base = 0;
    if (lane == lead) {
      base = atomicAdd(a.seg_count + sq, (uint32_t)__popcll(pm));
      if (a.stats)
        atomicAdd(a.stats + (q % (uint32_t)kStatCopies) * kStatCount + kStatPushed, (unsigned long long)__popcll(pm));
    }
    base = __shfl(base, (int)lead);
    const uint32_t slot = base + lanes_below(pm);
    if (keep && slot < a.seg_cap) {
      a.cand_score[sq * a.seg_cap + slot] = sc;
      a.cand_row[sq * a.seg_cap + slot] = row;
    }
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <typename K, typename... Args>
static void launch(K kernel, dim3 grid, dim3 block, hipStream_t s, const LaunchEvents& ev, Args... args);

// ---------------------------------------------------------------------------
// block bounds (cluster-grouped indexes)
// ---------------------------------------------------------------------------
// One slot's meta as the scan decodes it (block.rs:61-99): scale, offset,
// mid_n = max(mid_norm, 1e-6), hn = max(high_n, 1e-6); false if one is not finite.
__device__ __forceinline__ bool slot_meta(uint4 x, const float* flag_tabs, float* scale, float* offset, float* mid_n,
                                          float* hn) {
  *scale = h2f((uint16_t)(x.z & 0xffffu));
  *offset = h2f((uint16_t)(x.z >> 16));
  const float t = fmaxf(h2f((uint16_t)(x.w & 0xffffu)), 0.0f);
  const uint32_t fl = (x.w >> 16) & 0xffu;
  *mid_n = fmaxf(flag_tabs[256 + fl] * t, 1e-6f);
  *hn = fmaxf(fmaxf(flag_tabs[fl] * t, 0.0f), 1e-6f);
  const float sum = *scale + *offset + *mid_n + *hn;
  return sum - sum == 0.0f;
}

// Record dword and bit position behind code-space dimension d (< kBndDims):
// prefix levels are nibbles of dwords 0..7, S1 bits of dwords 8..11, S4 bits
// of dwords 12..13 (the record layout of k_relayout_to_device).
__device__ __forceinline__ void bnd_source(int d, int* word, int* shift) {
  if (d < kBndOff) {
    const int dd = d & 63;
    *word = dd >> 3;
    *shift = 4 * (dd & 7);
  } else if (d == kBndOff) {
    *word = -1;
    *shift = 0;
  } else if (d < kBndS4) {
    const int k = d - kBndS1;
    *word = 8 + (k >> 5);
    *shift = k & 31;
  } else {
    const int k = d - kBndS4;
    *word = 12 + (k >> 5);
    *shift = k & 31;
  }
}

__device__ __forceinline__ float bnd_value(int d, uint32_t w, int shift, float scale, float offset, float mid_n,
                                           float hn, const float* cb) {
  if (d < kBndMm) return scale * cb[(w >> shift) & 15u];
  if (d < kBndOff) return scale * (float)((w >> shift) & 15u);
  if (d == kBndOff) return offset;
  const bool bit = (w >> shift) & 1u;
  if (d < kBndS4) return bit ? mid_n : -mid_n;
  return bit ? hn : -hn;
}

// Stage slot (0 EdenProd prefix, 1 MinMax4 prefix + offset, 2 S1, 3 S4) of dimension d.
__device__ __forceinline__ int bnd_stage(int d) {
  return d < kBndMm ? 0 : (d <= kBndOff ? 1 : (d < kBndS4 ? 2 : 3));
}

// Cluster centers: one workgroup per cluster, thread t owns dimensions t and
// t + 256; the sum runs over the cluster's blocks and active slots with
// finite meta in a fixed order (the center need not be exact: the radii are
// measured from the stored center).
__global__ __launch_bounds__(256) void k_bound_centers(BoundBuildArgs a) {
  __shared__ float s_cb[16];
  __shared__ float s_part[4][256];
  const uint32_t c = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid < 16) s_cb[tid] = a.cb[tid];
  __syncthreads();
  constexpr int kPer = 2;
  int word[kPer], shift[kPer];
  float sum[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int d = tid + 256 * k;
    bnd_source(d < kBndDims ? d : 0, &word[k], &shift[k]);
    sum[k] = 0.0f;
  }
  uint32_t count = 0;
  for (uint32_t i = a.cl_start[c]; i < a.cl_start[c + 1]; ++i) {
    const uint64_t b = a.cl_blocks[i];
    const uint8_t* blk = a.idx + b * kBlockBytes;
    const uint64_t tomb = *reinterpret_cast<const uint64_t*>(blk + kOrigTombstone);
    for (int v = 0; v < 64; ++v) {
      if ((tomb >> v) & 1ull) continue;
      const uint32_t* rw = reinterpret_cast<const uint32_t*>(a.recs + (b * 64u + (uint32_t)v) * kRecWords);
      const uint4 x = a.recs[(b * 64u + (uint32_t)v) * kRecWords + kRecS4Meta];
      float scale, offset, mid_n, hn;
      if (!slot_meta(x, a.flag_tabs, &scale, &offset, &mid_n, &hn)) continue;
      ++count;
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int d = tid + 256 * k;
        if (d < kBndDims) {
          const uint32_t w = word[k] >= 0 ? rw[word[k]] : 0u;
          sum[k] += bnd_value(d, w, shift[k], scale, offset, mid_n, hn, s_cb);
        }
      }
    }
  }
  const float inv = count ? 1.0f / (float)count : 0.0f;
  float* cen = a.center + (uint64_t)c * kBndStride;
  float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int d = tid + 256 * k;
    if (d < kBndStride) {
      const float m = d < kBndDims ? sum[k] * inv : 0.0f;
      cen[d] = m;
      if (d < kBndDims) part[bnd_stage(d)] += m * m;
    }
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) s_part[st][tid] = part[st];
  __syncthreads();
  if (tid < 4) {
    float t = 0.0f;
    for (int i = 0; i < 256; ++i) t += s_part[tid][i];
    a.cnorm[(uint64_t)c * 4 + tid] = sqrtf(t) * (1.0f + kBndMargin);
  }
}

// Per-block radii: one wave per block, lane = slot; the largest distance of
// an active slot's stage part from its cluster center's, raised by the
// margin; +inf when an active slot's meta is not finite.  Blocks without the
// one-cluster flag are left unbounded (+inf).
__global__ __launch_bounds__(256) void k_bound_radii(BoundBuildArgs a) {
  __shared__ float s_cb[16];
  const int tid = threadIdx.x;
  if (tid < 16) s_cb[tid] = a.cb[tid];
  __syncthreads();
  const uint64_t b = (uint64_t)blockIdx.x * 4 + (tid >> 6);
  const uint32_t lane = __lane_id();
  if (b >= a.n_blocks) return;
  const uint32_t cl = a.bcl[b];
  float r[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
  if (cl != ~0u) {
    const uint8_t* blk = a.idx + b * kBlockBytes;
    const uint64_t tomb = *reinterpret_cast<const uint64_t*>(blk + kOrigTombstone);
    const bool act = !((tomb >> lane) & 1ull);
    const uint4* rec = a.recs + (b * 64u + lane) * kRecWords;
    const uint4 q0 = rec[0], q1 = rec[1], q2 = rec[2], q3 = rec[3];
    const uint32_t rw[14] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w, q2.x, q2.y, q2.z, q2.w, q3.x, q3.y};
    float scale, offset, mid_n, hn;
    const bool fin = slot_meta(q3, a.flag_tabs, &scale, &offset, &mid_n, &hn);
    const float* cen = a.center + (uint64_t)cl * kBndStride;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int d = 0; d < kBndDims; ++d) {
      int w, sh;
      bnd_source(d, &w, &sh);
      const float x = bnd_value(d, w >= 0 ? rw[w] : 0u, sh, scale, offset, mid_n, hn, s_cb) - cen[d];
      acc[bnd_stage(d)] += x * x;
    }
    const bool bad = act && !fin;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      float v = act && fin ? acc[st] : 0.0f;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
      r[st] = sqrtf(v) * (1.0f + kBndMargin) + 1e-30f;
    }
    if (__ballot(bad) != 0) r[0] = r[1] = r[2] = r[3] = INFINITY;
  }
  if (lane < 4) a.brad[b * 4 + lane] = lane == 0 ? r[0] : lane == 1 ? r[1] : lane == 2 ? r[2] : r[3];
}

hipError_t launch_bound_build(const BoundBuildArgs& a, hipStream_t s) {
  if (a.n_cl) hipLaunchKernelGGL(k_bound_centers, dim3(a.n_cl), dim3(256), 0, s, a);
  if (a.n_blocks) hipLaunchKernelGGL(k_bound_radii, dim3((uint32_t)((a.n_blocks + 3) / 4)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// Query columns of the bound table, kBndCols per query: 65 prefix columns
// (EdenProd: prefix_weight and a zero; MinMax4: q_d and prefix_sum), 128 S1
// columns (rabitq_weights2 / 2), 64 S4 columns (w_s4 tail_fold_weights2 / 2).
// Column k multiplies center dimension bnd_center_dim(k).
constexpr int kBndCols = 65 + 128 + 64;
__device__ __forceinline__ int bnd_center_dim(int k, bool eden) {
  return k < 65 ? (eden ? k : kBndMm + k) : kBndS1 + (k - 65);
}

// Per (cluster, query): mean_ip + <center, c_q> + margin; per query the norms
// of its column parts (raised by the margin).  Grid (clusters / 4, queries /
// 64): a workgroup stages its 64 queries' columns (float4 loads of the S1 and
// S4 weights, all of a thread's loads in flight together) and its 4 clusters'
// centers in LDS, then each wave takes one cluster, lane = query.  Workgroup
// (0, 0) also clears the block-list counts.
constexpr int kBndTableClusters = 4;
constexpr int kBndColsPad = (kBndCols + 3) & ~3;  // columns past kBndCols are zero
static_assert(64 + 64 * (kBndColsPad - kBndCols) <= 256 && kQdW4 + 64 <= kQData, "table staging");
__global__ __launch_bounds__(256) void k_bound_table(BoundScanArgs a) {
  __shared__ float s_col[kBndColsPad][65];  // [column][query], padded: conflict-free both ways
  __shared__ __align__(16) float s_cen[kBndTableClusters][kBndColsPad];
  __shared__ float s_mean[64], s_ws4[64], s_s1[64];
  const int tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  const int wave = tid >> 6;
  const uint32_t q0 = blockIdx.y * 64;
  const uint32_t c0 = blockIdx.x * kBndTableClusters;
  const uint32_t nq = min(64u, a.n_q - q0);
  const bool eden = a.eden != 0;
  if (blockIdx.x == 0 && blockIdx.y == 0 && a.bcount) {
    // the counts of both block lists of a scan (a sampling stage's and the final pass's)
    const uint32_t n_chunks = (a.n_q + a.chunk - 1) / a.chunk;
    for (uint32_t i = (uint32_t)tid; i < 2 * n_chunks; i += 256) a.bcount[i] = 0u;
  }
  // per-query fields and column 64 (MinMax4: prefix_sum), then the rest
  if (tid < 64) {
    const bool have = (uint32_t)tid < nq;
    const mrl_query_plan* p = a.plans + q0 + (have ? tid : 0);
    const float ws4 = (a.sp.strata == MRL_STRATA_FULL64B && p->has_tail_fold) ? a.sp.w_s4 : 0.0f;
    s_ws4[tid] = have ? 0.5f * ws4 : 0.0f;
    s_s1[tid] = have && a.sp.strata != MRL_STRATA_L0_ONLY ? 0.5f : 0.0f;
    s_mean[tid] = have && eden ? p->eden_mean_ip : 0.0f;
    s_col[64][tid] = have && !eden ? p->prefix_sum : 0.0f;
  } else if (tid < 64 + 64 * (kBndColsPad - kBndCols)) {  // the zero rows past kBndCols
    const int i = tid - 64;
    s_col[kBndCols + (i >> 6)][i & 63] = 0.0f;
  }
  for (int i = tid; i < kBndTableClusters * kBndColsPad; i += 256) {
    const int j = i / kBndColsPad, k = i - j * kBndColsPad;
    const uint32_t c = c0 + (uint32_t)j;
    s_cen[j][k] = (c < a.n_cl && k < kBndCols) ? a.center[(uint64_t)c * kBndStride + bnd_center_dim(k, eden)] : 0.0f;
  }
  __syncthreads();
  // prefix columns 0..63: plan prefix_weight (one float per thread and query);
  // S1 columns 65..192 and S4 columns 193..256: 48 float4 per query
  {
    constexpr int kP = 64 * 64 / 256, kV = 64 * 48 / 256;
    float pv[kP];
    float4 wv[kV];
#pragma unroll
    for (int u = 0; u < kP; ++u) {
      const uint32_t i = (uint32_t)tid + 256u * u, qi = i >> 6, k = i & 63u;
      pv[u] = qi < nq ? a.plans[q0 + qi].prefix_weight[k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kV; ++u) {
      const uint32_t i = (uint32_t)tid + 256u * u, qi = i / 48u, k4 = i - qi * 48u;
      const float* qd = a.luts + (uint64_t)(q0 + (qi < nq ? qi : 0)) * kQData;
      wv[u] = qi < nq ? *reinterpret_cast<const float4*>(qd + (k4 < 32 ? kQdW1 + 4 * k4 : kQdW4 + 4 * (k4 - 32)))
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < kP; ++u) {
      const uint32_t i = (uint32_t)tid + 256u * u;
      s_col[i & 63u][i >> 6] = pv[u];
    }
#pragma unroll
    for (int u = 0; u < kV; ++u) {
      const uint32_t i = (uint32_t)tid + 256u * u, qi = i / 48u, k4 = i - qi * 48u;
      const float f = k4 < 32 ? s_s1[qi] : s_ws4[qi];
      const uint32_t k = 65u + 4u * k4;
      s_col[k][qi] = f * wv[u].x;
      s_col[k + 1][qi] = f * wv[u].y;
      s_col[k + 2][qi] = f * wv[u].z;
      s_col[k + 3][qi] = f * wv[u].w;
    }
  }
  __syncthreads();
  // lane = query: the norms of its column parts (raised by the margin)
  float n0 = 0.0f, n1 = 0.0f, n2 = 0.0f;
  for (int k = 0; k < 65; ++k) n0 += s_col[k][lane] * s_col[k][lane];
  for (int k = 65; k < 65 + 128; ++k) n1 += s_col[k][lane] * s_col[k][lane];
  for (int k = 65 + 128; k < kBndCols; ++k) n2 += s_col[k][lane] * s_col[k][lane];
  const float up = 1.0f + kBndMargin;
  const float nq0 = sqrtf(n0) * up, nq1 = sqrtf(n1) * up, nq2 = sqrtf(n2) * up, mean = s_mean[lane];
  const uint32_t q = q0 + lane;
  if (blockIdx.x == 0 && wave == 0 && q < a.n_q) {
    const float4 n = make_float4(nq0, nq1, nq2, 0.0f);
    *reinterpret_cast<float4*>(a.qn + (uint64_t)q * 4) = n;
  }
  const uint32_t c = c0 + (uint32_t)wave;
  if (c >= a.n_cl || q >= a.n_q) return;
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll 4
  for (int k = 0; k < kBndColsPad; k += 4) {
    const float4 cv = *reinterpret_cast<const float4*>(&s_cen[wave][k]);
    d0 += cv.x * s_col[k][lane] + cv.y * s_col[k + 1][lane];
    d1 += cv.z * s_col[k + 2][lane] + cv.w * s_col[k + 3][lane];
  }
  const float* cn = a.cnorm + (uint64_t)c * 4;
  const float margin = kBndMargin * (fabsf(mean) + (eden ? cn[0] : cn[1]) * nq0 + cn[2] * nq1 + cn[3] * nq2) + 1e-30f;
  a.table[(uint64_t)c * a.n_q + q] = (mean + (d0 + d1)) + margin;
}

hipError_t launch_bound_table(const BoundScanArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_cl == 0 || a.n_q == 0) return hipSuccess;
  launch(k_bound_table, dim3((a.n_cl + kBndTableClusters - 1) / kBndTableClusters, (a.n_q + 63) / 64), dim3(256), s,
         ev, a);
  return hipGetLastError();
}

// Block selection over the pass's blocks (pos << shift, pos < n_pos): a block
// is listed for a chunk of queries (at most 64) unless every query's bound on
// it lies below that query's floor (blocks without bounds are always listed).
// Lane = block; the chunk's query norms and floors sit in LDS; a workgroup
// reserves room for its listed blocks with one atomic and writes them in
// position order.  With out_bound (the diagnostic) every bound is written
// instead.
constexpr int kSelBlocksPerGroup = 256;
__global__ __launch_bounds__(256) void k_block_select(BoundScanArgs a) {
  __shared__ float4 s_q[64];  // norms of the column parts, floor
  __shared__ uint32_t s_wn[4], s_base;
  const int tid = threadIdx.x;
  const uint32_t lane = __lane_id();
  const int wave = tid >> 6;
  const uint32_t chunk = blockIdx.y;
  const uint32_t qc0 = chunk * a.chunk;
  const uint32_t nq = min(min(a.chunk, 64u), a.n_q - qc0);
  if ((uint32_t)tid < nq) {
    const float4 n = *reinterpret_cast<const float4*>(a.qn + (uint64_t)(qc0 + tid) * 4);
    s_q[tid] = make_float4(n.x, n.y, n.z, a.floor ? a.floor[qc0 + tid] : 0.0f);
  }
  __syncthreads();
  const uint32_t pos = blockIdx.x * kSelBlocksPerGroup + (uint32_t)tid;
  const bool have = pos < a.n_pos;
  const uint64_t b = (uint64_t)pos << a.shift;
  const uint32_t cl = have ? a.bcl[b] : ~0u;
  if (a.out_bound) {  // the diagnostic: every bound (NaN: unbounded block)
    if (!have) return;
    const float4 r = cl != ~0u ? *reinterpret_cast<const float4*>(a.brad + b * 4) : make_float4(0, 0, 0, 0);
    for (uint32_t i = 0; i < nq; ++i) {
      float bound = __builtin_nanf("");
      if (cl != ~0u) {
        const float4 qv = s_q[i];
        bound = a.table[(uint64_t)cl * a.n_q + qc0 + i] + ((a.eden ? r.x : r.y) * qv.x + r.z * qv.y + r.w * qv.z);
        if (!(bound == bound)) bound = INFINITY;
      }
      a.out_bound[(uint64_t)(qc0 + i) * a.n_blocks + b] = bound;
    }
    return;
  }
  bool need = have;
  if (cl != ~0u) {
    const float4 r = *reinterpret_cast<const float4*>(a.brad + b * 4);
    const float re = a.eden ? r.x : r.y;
    const float* trow = a.table + (uint64_t)cl * a.n_q + qc0;
    bool any = false;
    if (nq == 64u && (a.n_q & 3u) == 0u) {
      // a full chunk: its 64 table entries in one round of 16-byte loads
      // (the row is 16-byte aligned when n_q is a multiple of 4)
      const float4* tr4 = reinterpret_cast<const float4*>(trow);
      float4 t4[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) t4[u] = tr4[u];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float tv[4] = {t4[u].x, t4[u].y, t4[u].z, t4[u].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float4 qv = s_q[4 * u + c];
          const float bound = tv[c] + (re * qv.x + r.z * qv.y + r.w * qv.z);
          any |= !(bound < qv.w);  // NaN bounds keep the block
        }
      }
    } else {
      constexpr int kB = 16;  // table loads in flight together
      for (uint32_t i0 = 0; i0 < nq; i0 += kB) {
        float t[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) t[u] = i0 + u < nq ? trow[i0 + u] : -INFINITY;
#pragma unroll
        for (int u = 0; u < kB; ++u) {
          const float4 qv = s_q[min(i0 + (uint32_t)u, 63u)];
          const float bound = t[u] + (re * qv.x + r.z * qv.y + r.w * qv.z);
          // NaN bounds keep the block; past the chunk t = -inf
          any |= (i0 + u < nq) && !(bound < qv.w);
        }
      }
    }
    need = any;
  }
  const uint64_t m = __ballot(need);
  if (lane == 0) s_wn[wave] = (uint32_t)__popcll(m);
  __syncthreads();
  if (tid == 0) {
    const uint32_t cnt = s_wn[0] + s_wn[1] + s_wn[2] + s_wn[3];
    s_base = cnt ? atomicAdd(a.bcount + chunk, cnt) : 0u;
  }
  __syncthreads();
  if (need) {
    uint32_t off = s_base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) off += s_wn[w];
    a.blist[(uint64_t)chunk * a.stride + off] = (uint32_t)b;
  }
}

hipError_t launch_block_select(const BoundScanArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_pos == 0 || a.n_q == 0) return hipSuccess;
  const uint32_t chunks = (a.n_q + a.chunk - 1) / a.chunk;
  launch(k_block_select, dim3((a.n_pos + kSelBlocksPerGroup - 1) / kSelBlocksPerGroup, chunks), dim3(256), s, ev,
         a);
  return hipGetLastError();
}

hipError_t launch_relayout(const uint8_t* src, uint8_t* dst, uint64_t n_blocks, bool to_device,
                           hipStream_t s, uint4* recs) {
  if (n_blocks == 0) return hipSuccess;
  uint32_t grid = (uint32_t)(n_blocks < 65536 ? n_blocks : 65536);
  if (to_device)
    hipLaunchKernelGGL(k_relayout_to_device, dim3(grid), dim3(64), 0, s, src, dst, n_blocks, recs);
  else hipLaunchKernelGGL(k_relayout_to_host, dim3(grid), dim3(64), 0, s, src, dst, n_blocks);
  return hipGetLastError();
}

// Launch with the dispatch-recorded events when profiling, plainly otherwise.
template <typename K, typename... Args>
static void launch(K kernel, dim3 grid, dim3 block, hipStream_t s, const LaunchEvents& ev, Args... args) {
  if (ev.start) hipExtLaunchKernelGGL(kernel, grid, block, 0, s, ev.start, ev.stop, 0u, args...);
  else hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
}

hipError_t launch_plan(const PlanArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_q == 0) return hipSuccess;
  launch(k_plan, dim3(a.n_q), dim3(192), s, ev, a);
  return hipGetLastError();
}

int scan_query_tile(uint32_t n_q) { return n_q >= 8 ? 8 : 1; }

// Workgroups of `kernel` (of `threads` threads) resident at once on the current device.
template <typename K>
static uint32_t resident_groups_n(K kernel, int threads) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1024;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 1024;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  return (uint32_t)(cus * per_cu);
}
template <typename K>
static uint32_t resident_groups(K kernel) {
  return resident_groups_n(kernel, 256);
}

// Workgroups along x of a scan launch (the same for every query tile).
uint32_t scan_grid(const ScanArgs& a, bool diag) {
  const bool l0 = a.sp.strata == MRL_STRATA_L0_ONLY;
  const bool tile = a.n_q >= 8 && !diag && !l0 && !a.gate;
  const int qt = tile ? kTileQ : (a.gate ? 1 : scan_query_tile(a.n_q));
  const uint32_t tiles = (a.n_q + qt - 1) / qt;
  // One round of resident workgroups (each wave then loops over blocks),
  // but at least one workgroup per candidate segment of a query.
  static const uint32_t res1 = resident_groups(k_scan<1, false, false>);
  static const uint32_t res8 = resident_groups(k_scan<8, false, false>);
  static const uint32_t rest = resident_groups(k_scan_tile<kTileQ, true>);
  const uint32_t res = tile ? rest : (qt == 8 ? res8 : res1);
  uint32_t grid = (a.n_pos + 4) / 4;  // 4 * grid - 1 >= n_pos waves carry positions
  uint32_t max_grid = res / tiles;
  // A gated re-run scans for the few flagged queries only (the other
  // queries' workgroups exit at once): each query gets up to a quarter of
  // the one-query grid, not 1/n_q of the GPU, within a total of
  // kRerunWorkgroups so that the launch costs no more than an empty one
  // when no query is flagged (a grid of 131,072 empty workgroups took 37 us).
  if (a.gate) {
    const uint32_t g_one = (res1 < MRL_SCAN_GRID1 ? res1 : MRL_SCAN_GRID1) / 4u;
    const uint32_t g_budget = kRerunWorkgroups / tiles;
    uint32_t g = g_one < g_budget ? g_one : g_budget;
    if (g < 1u) g = 1u;
    if (max_grid < g) max_grid = g;
  }
  // (a one-query final pass beside another context's scan leaves a quarter
  // of its workgroups to that context's launches)
  const uint32_t grid1 = a.leave_room ? MRL_SCAN_GRID1 - MRL_SCAN_GRID1 / 4u : MRL_SCAN_GRID1;
  if (!tile && qt == 1 && !diag && !l0 && max_grid > grid1) max_grid = grid1;
  if (!a.excl && max_grid < a.nseg) max_grid = a.nseg;
  if (grid > max_grid) grid = max_grid;
  return grid;
}

hipError_t launch_scan(const ScanArgs& a, bool diag, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_pos == 0 || a.n_q == 0) return hipSuccess;
  const bool l0 = a.sp.strata == MRL_STRATA_L0_ONLY;
  // batched: the tile kernel; otherwise one query per workgroup, or the
  // 8-query workgroups of the diagnostic and L0Only paths
  const bool tile = a.n_q >= 8 && !diag && !l0 && !a.gate;
  const int qt = tile ? kTileQ : (a.gate ? 1 : scan_query_tile(a.n_q));
  if (a.gate && diag) return hipErrorInvalidValue;
  if (a.fuse_plan && (a.n_q != 1 || diag || l0 || a.gate || a.plan.dims > (uint32_t)kFuseMaxDims || a.plan.n_q != 1))
    return hipErrorInvalidValue;
  const uint32_t tiles = (a.n_q + qt - 1) / qt;
  const uint32_t grid = scan_grid(a, diag);
  // exclusive segments: the one-query kernel, one segment per workgroup
  if (a.excl && (tile || qt != 1 || diag || l0 || grid != a.nseg || a.nseg > (uint32_t)kMaxSegs ||
                 a.seg_cap > (uint32_t)Staging<1>::kCap))
    return hipErrorInvalidValue;
  dim3 g(grid, tiles);
  if (tile) {
    if (a.sp.strata == MRL_STRATA_FULL64B) launch(k_scan_tile<kTileQ, true>, g, dim3(256), s, ev, a);
    else launch(k_scan_tile<kTileQ, false>, g, dim3(256), s, ev, a);
  } else if (qt == 8) {
    if (l0) {
      if (diag) launch(k_scan<8, true, true>, g, dim3(256), s, ev, a);
      else launch(k_scan<8, false, true>, g, dim3(256), s, ev, a);
    } else {
      if (diag) launch(k_scan<8, true, false>, g, dim3(256), s, ev, a);
      else launch(k_scan<8, false, false>, g, dim3(256), s, ev, a);
    }
  } else {
    if (l0) {
      if (diag) launch(k_scan<1, true, true>, g, dim3(256), s, ev, a);
      else launch(k_scan<1, false, true>, g, dim3(256), s, ev, a);
    } else {
      if (diag) launch(k_scan<1, true, false>, g, dim3(256), s, ev, a);
      else if (a.fuse_plan) launch(k_scan<1, false, false, true>, g, dim3(256), s, ev, a);
      else launch(k_scan<1, false, false>, g, dim3(256), s, ev, a);
    }
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* p, uint64_t n, uint32_t v) {
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) p[i] = v;
}

hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t groups = (n + 255) / 256;
  hipLaunchKernelGGL(k_fill_u32, dim3((uint32_t)(groups < 2048 ? groups : 2048)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

// Cache eviction sweep: every thread xors its share of the buffer; the
// buffer holds zeros, so the final store never happens, but the compiler must
// keep the loads.
__global__ __launch_bounds__(256) void k_read_sweep(uint4* p, uint64_t n) {
  uint32_t x = 0u;
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u) {
    const uint4 v = p[i];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (x == 0x9e3779b9u) p[0].x = x;
}

hipError_t launch_read_sweep(uint4* p, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_read_sweep, dim3(4096), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

hipError_t launch_select(const SelectArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  launch(k_select, dim3(n_q), dim3(kSelThreads), s, ev, a);
  return hipGetLastError();
}

hipError_t launch_mma_prep(const MmaPrepArgs& a, hipStream_t s, const LaunchEvents& ev) {
  if (a.n_q == 0) return hipSuccess;
  launch(k_mma_prep, dim3(a.n_q), dim3(64), s, ev, a);
  return hipGetLastError();
}

hipError_t launch_plan_mma_prep(const PlanArgs& pa, const MmaPrepArgs& ma, hipStream_t s, const LaunchEvents& ev) {
  if (ma.n_q == 0) return hipSuccess;
  if (pa.n_q != ma.n_q) return hipErrorInvalidValue;
  launch(k_plan_mma_prep, dim3(ma.n_q), dim3(192), s, ev, pa, ma);
  return hipGetLastError();
}

// Workgroups along x of an MFMA scan launch: one round of resident
// workgroups over the query chunks, at most one block per wave.
uint32_t mma_scan_grid(const ScanArgs& a) {
  const uint32_t chunks = (a.n_q + kMmaQ - 1) / kMmaQ;
  static const uint32_t res = resident_groups_n(k_scan_mma<2, 1>, kMmaWaves * 64);
  const uint32_t wpg = kMmaWaves;
  uint32_t grid = (2u * a.n_pos + wpg) / wpg;  // items: two 32-vector tiles per block
  uint32_t max_grid = (a.leave_room ? res - res / 16u : res) / chunks;
  if (max_grid < 1) max_grid = 1;
  if (grid > max_grid) grid = max_grid;
  return grid;
}

hipError_t launch_scan_mma(const ScanArgs& args, int mode, hipStream_t s, const LaunchEvents& ev) {
  if (args.n_pos == 0 || args.n_q == 0) return hipSuccess;
  static const uint32_t cus = [] {
    int dev = 0, n = 0;
    return hipGetDevice(&dev) == hipSuccess &&
                   hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0
               ? (uint32_t)n
               : 0u;
  }();
  // A final pass that has the device to itself splits a CU's items between
  // its two workgroups.  (Beside another context's launches the
  // workgroups' placement is not known: config 4 over three contexts went
  // 0.1972 -> 0.2009 ms per step with the split, same box.)
  ScanArgs a = args;
  a.pair_cols = mode != 0 && !a.leave_room ? cus : 0u;
  const dim3 g(mma_scan_grid(a), (a.n_q + kMmaQ - 1) / kMmaQ), b(kMmaWaves * 64);
  const bool two = a.n_q > 32;  // one 32-query tile per wave suffices up to 32 queries
  if (mode == 0 && a.lbuf && a.lcount) {
    // every workgroup's list fits in its query's row
    if ((uint64_t)g.x * a.lcap > a.lbuf_stride || a.lcap == 0) return hipErrorInvalidValue;
    if (two) launch(k_scan_mma<2, 4>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 4>, g, b, s, ev, a);
  } else if (mode == 0 && a.lbuf) {
    if (two) launch(k_scan_mma<2, 3>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 3>, g, b, s, ev, a);
  } else if (mode == 0) {
    if (two) launch(k_scan_mma<2, 0>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 0>, g, b, s, ev, a);
  } else if (mode == 1 && a.mma_wide) {
    if (two) launch(k_scan_mma<2, 1, true>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 1, true>, g, b, s, ev, a);
  } else if (mode == 1) {
    if (two) launch(k_scan_mma<2, 1>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 1>, g, b, s, ev, a);
  } else {
    if (two) launch(k_scan_mma<2, 2>, g, b, s, ev, a);
    else launch(k_scan_mma<1, 2>, g, b, s, ev, a);
  }
  return hipGetLastError();
}

hipError_t launch_mma_floors_lb(const float* lbuf, uint32_t lbuf_stride, uint32_t n_s, const float* luts,
                                uint32_t n_q, uint32_t rank, uint32_t safe_rank, float* floor_out, float* safe_out,
                                hipStream_t s, const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  if (n_s > lbuf_stride) return hipErrorInvalidValue;
  launch(k_mma_floors_lb, dim3(n_q), dim3(kFlbThreads), s, ev, lbuf, lbuf_stride, n_s, luts, rank, safe_rank, floor_out,
         safe_out);
  return hipGetLastError();
}

hipError_t launch_mma_floors_seg(const float* lbuf, const uint32_t* lcount, uint32_t lbuf_stride, uint32_t n_wg,
                                 uint32_t lcap, uint32_t* hist, const float* luts, uint32_t n_q, uint32_t rank,
                                 uint32_t safe_rank, float* floor_out, float* safe_out, hipStream_t s,
                                 const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  if ((uint64_t)n_wg * lcap > lbuf_stride || n_wg > lbuf_stride || n_wg > (uint32_t)kMaxListWg)
    return hipErrorInvalidValue;
  launch(k_mma_floors_seg, dim3(n_q), dim3(kSegThreads), s, ev, lbuf, lcount, lbuf_stride, n_wg, lcap, hist, luts,
         rank, safe_rank, floor_out, safe_out);
  return hipGetLastError();
}

hipError_t launch_mma_floors(uint32_t* hist, const float* luts, uint32_t n_q, uint32_t rank, uint32_t safe_rank,
                             float* floor_out, float* safe_out, bool prev, hipStream_t s, const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  launch(k_mma_floors, dim3(n_q), dim3(64), s, ev, hist, luts, rank, safe_rank, floor_out, safe_out, prev ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_finish(const FinishArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  launch(k_finish, dim3(n_q), dim3(kFinThreads), s, ev, a);
  return hipGetLastError();
}

hipError_t launch_exact(const FinishArgs& a, uint32_t n_q, hipStream_t s, const LaunchEvents& ev) {
  if (n_q == 0) return hipSuccess;
  static const uint32_t res = resident_groups_n(k_exact, kExactItem);
  const uint32_t items = n_q * (uint32_t)(kFinCap / kExactItem);  // at most
  launch(k_exact, dim3(items < res ? items : res), dim3(kExactItem), s, ev, a);
  return hipGetLastError();
}

}  // namespace mrl
