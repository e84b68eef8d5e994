// mrl_kernels.hip -- gfx950 kernels for the PaxBlock64 progressive bitplane scan.
//
// Numerics: every f32 expression keeps the reference's operand order and is
// compiled with -ffp-contract=off (no fused multiply-add), correctly rounded
// division/sqrt and IEEE denormals, so per-vector scores are bit-identical to
// src/scan.rs.  Wave64 is the natural unit: the 64 slots of a PaxBlock64 map
// to the 64 lanes of a wavefront and a bitplane word is a lane mask.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mrl_internal.h"

namespace mrl {

// ---------------------------------------------------------------------------
// small helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, h);
  return (float)x;
}

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
// eden.rs:357-370 (rademacher_diag).
__device__ __forceinline__ float mix_sign(uint64_t a, uint64_t i) {
  uint64_t x = (a * 0x9E3779B97F4A7C15ull + i) * 0xBF58476D1CE4E5B9ull;
  x ^= x >> 30;
  x = x * 0x94D049BB133111EBull;
  x ^= x >> 27;
  return (x & 1ull) == 0 ? 1.0f : -1.0f;
}

// ---------------------------------------------------------------------------
// block re-layout (upload) and its inverse (download)
// one 64-lane workgroup per block; lane v owns slot v
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_relayout_to_device(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ dst, uint64_t n_blocks) {
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
    for (int j = 0; j < 8; ++j) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i) {
        int dim = 8 * j + i;
        uint32_t lvl = (uint32_t)((s5[dim] >> v) & 1u) | ((uint32_t)((s3[dim] >> v) & 1u) << 1) |
                       ((uint32_t)((s2[dim] >> v) & 1u) << 2) | ((uint32_t)((s0[dim] >> v) & 1u) << 3);
        w |= lvl << (4 * i);
      }
      reinterpret_cast<uint32_t*>(d + kDevNibbles)[64 * j + v] = w;
    }
    const uint64_t* s1 = reinterpret_cast<const uint64_t*>(s + kOrigS1);
    const uint64_t* s4 = reinterpret_cast<const uint64_t*>(s + kOrigS4);
    uint64_t* d1 = reinterpret_cast<uint64_t*>(d + kDevS1);
    uint64_t* d4 = reinterpret_cast<uint64_t*>(d + kDevS4);
    d1[v] = s1[v];
    d1[v + 64] = s1[v + 64];
    d4[v] = s4[v];
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
      uint32_t lvl = (nib[64 * (dim >> 3) + slot] >> (4 * (dim & 7))) & 15u;
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
// one 128-thread workgroup per query
// ---------------------------------------------------------------------------

// In-place FWHT butterflies over an LDS array (fwht_inplace, rotate.rs:13-33,
// without the final scale).  Each output of a stage is one add or subtract of
// two outputs of the previous stage, so the parallel order is bit-identical.
__device__ __forceinline__ void fwht_stage(float* a, int n, int h, int i) {
  if (i < n / 2) {
    int j = (i / h) * (2 * h) + (i % h);
    float x = a[j];
    float y = a[j + h];
    a[j] = x + y;
    a[j + h] = x - y;
  }
}

__global__ __launch_bounds__(128) void k_plan(PlanArgs a) {
  __shared__ float s_q[MRL_MAX_DIMS];
  __shared__ float s_mid[128];
  __shared__ float s_emid[128];
  __shared__ float s_eden[64];
  __shared__ float s_tail[64];
  __shared__ float s_sums[4];

  const uint32_t q = blockIdx.x;
  const int t = threadIdx.x;
  const uint32_t dims = a.dims;
  const float* x = a.queries + (uint64_t)q * dims;
  mrl_query_plan* p = a.out + q;
  const bool has_eden = a.eden_mean != nullptr;
  const bool has_mid = a.mid_mean != nullptr;
  const bool eden_codec = a.prefix_codec == MRL_PREFIX_EDEN_PROD;

  for (uint32_t i = t; i < dims; i += 128) s_q[i] = x[i];
  __syncthreads();

  // rotate_query = diag(+-1) then FWHT (eden.rs:91-98, 275-281); fold_tail (rotate.rs:73-93)
  s_mid[t] = s_q[64 + t];
  s_emid[t] = has_mid ? s_q[64 + t] * mix_sign(a.mid_seed, (uint64_t)t) : 0.0f;
  if (t < 64) {
    s_eden[t] = has_eden ? s_q[t] * mix_sign(a.eden_seed, (uint64_t)t) : 0.0f;
    float u = zero_acc();
    if (dims > (uint32_t)kTailStart) {
      int nb = (int)(dims - kTailStart) / 64;
      if (nb > kTailFoldBlocks) nb = kTailFoldBlocks;
      for (int b = 0; b < nb; ++b) u += mix_sign((uint64_t)b, (uint64_t)t) * s_q[kTailStart + 64 * b + t];
    }
    s_tail[t] = u;
  }
  __syncthreads();
  for (int h = 1; h < 128; h *= 2) {
    if (t < 64) fwht_stage(s_mid, 128, h, t);
    else fwht_stage(s_emid, 128, h, t - 64);
    if (h < 64) {
      if (t < 32) fwht_stage(s_eden, 64, h, t);
      else if (t < 64) fwht_stage(s_tail, 64, h, t - 32);
    }
    __syncthreads();
  }
  s_mid[t] *= a.c.inv_sqrt128;
  s_emid[t] *= a.c.inv_sqrt128;
  if (t < 64) {
    s_eden[t] *= a.c.inv_sqrt64;
    s_tail[t] *= a.c.inv_sqrt64;
  }
  __syncthreads();

  const bool has_tail = dims > (uint32_t)kTailStart;
  const float rs = a.c.rabitq_scale;
  const float ts = a.c.tail_fold_scale;

  // elementwise fields
  if (t < 64) {
    float v = s_q[t];
    p->prefix[t] = v;
    p->bit_weights[t][0] = v * 1.0f;
    p->bit_weights[t][1] = v * 2.0f;
    p->bit_weights[t][2] = v * 4.0f;
    p->bit_weights[t][3] = v * 8.0f;
    p->eden_q_rot[t] = s_eden[t];
    float tq = has_tail ? s_tail[t] : 0.0f;
    p->tail_fold_q[t] = tq;
    p->tail_fold_weights2[t] = has_tail ? 2.0f * (tq * ts) : 0.0f;
    // scan.rs:457-461
    p->prefix_weight[t] = eden_codec ? s_eden[t] * a.c.inv_sqrt64 : v;
  }
  {
    float rq = s_mid[t];
    p->rabitq_q[t] = rq;
    p->rabitq_weights2[t] = 2.0f * (rq * rs);
    p->eden_mid_q_rot[t] = s_emid[t];
    // scan.rs:528-532 (deltas) with eden_mid_inv_sqrt_d = 1/sqrt(128)
    float c0 = has_mid ? a.c.eden_mid_codebook[0] : 0.0f;
    float c1 = has_mid ? a.c.eden_mid_codebook[1] : 0.0f;
    float qq = s_emid[t] * a.c.inv_sqrt128;
    p->eden_mid_deltas[t] = (c1 - c0) * qq;
  }
  // rabitq_lut (scan.rs:188-201): 512 entries, 4 per thread
  for (int e = t; e < 512; e += 128) {
    int g = e >> 4, mask = e & 15;
    float p0 = s_mid[4 * g] * rs, p1 = s_mid[4 * g + 1] * rs;
    float p2 = s_mid[4 * g + 2] * rs, p3 = s_mid[4 * g + 3] * rs;
    float v0 = (mask & 1) ? p0 : -p0;
    float v1 = (mask & 2) ? p1 : -p1;
    float v2 = (mask & 4) ? p2 : -p2;
    float v3 = (mask & 8) ? p3 : -p3;
    p->rabitq_lut[g][mask] = v0 + v1 + v2 + v3;
  }
  if (t < 16) p->eden_codebook[t] = has_eden ? a.c.eden_codebook[t] : 0.0f;
  if (t < 27) p->pad[t] = 0.0f;

  // sequential reductions, one chain per thread, in the reference's order
  if (t == 0) {  // prefix_l1, prefix_sum (132-140)
    float l1 = zero_acc(), sum = zero_acc();
    for (int d = 0; d < 64; ++d) {
      float v = s_q[d];
      l1 += fabsf(v);
      sum += v;
    }
    p->prefix_l1 = l1;
    p->prefix_sum = sum;
  } else if (t == 1) {  // eden_mean_ip (149-151)
    float s = zero_acc();
    if (has_eden)
      for (int d = 0; d < 64; ++d) s += s_q[d] * a.eden_mean[d];
    p->eden_mean_ip = s;
    p->eden_inv_sqrt_d = a.c.inv_sqrt64;
  } else if (t == 2) {  // eden_mid_mean_ip (167-169)
    float s = zero_acc();
    if (has_mid)
      for (int d = 0; d < 128; ++d) s += s_q[64 + d] * a.mid_mean[d];
    p->eden_mid_mean_ip = s;
    p->eden_mid_inv_sqrt_d = a.c.inv_sqrt128;
    p->eden_mid_codebook[0] = has_mid ? a.c.eden_mid_codebook[0] : 0.0f;
    p->eden_mid_codebook[1] = has_mid ? a.c.eden_mid_codebook[1] : 0.0f;
  } else if (t == 3) {  // q_tail_sq (203-206)
    float s = zero_acc();
    for (uint32_t i = kTailStart; i < dims; ++i) s += s_q[i] * s_q[i];
    s_sums[0] = s;
  } else if (t == 4) {  // q_mid_sq (209-212)
    float s = zero_acc();
    for (int i = 0; i < 128; ++i) {
      float v = s_q[64 + i];
      s += v * v;
    }
    s_sums[1] = s;
  } else if (t == 5) {  // rabitq_base (182-186)
    float base = zero_acc();
    for (int d = 0; d < 128; ++d) base -= s_mid[d] * rs;
    p->rabitq_base = base;
    p->rabitq_scale = rs;
  } else if (t == 6) {  // tail_fold_base, s4_abs_budget (226-233)
    float base = zero_acc(), budget = zero_acc();
    if (has_tail) {
      for (int d = 0; d < 64; ++d) {
        float pos = s_tail[d] * ts;
        base -= pos;
        budget += fabsf(pos);
      }
    }
    p->tail_fold_base = base;
    p->s4_abs_budget = budget;
  } else if (t == 7) {  // EdenB1 base (scan.rs:528-531)
    float base = zero_acc();
    float c0 = has_mid ? a.c.eden_mid_codebook[0] : 0.0f;
    for (int d = 0; d < 128; ++d) base += c0 * (s_emid[d] * a.c.inv_sqrt128);
    p->eden_mid_base = base;
  } else if (t == 8) {
    p->dims = dims;
    p->prefix_codec = a.prefix_codec;
    p->mid_codec = a.mid_codec;
    p->has_tail_fold = has_tail ? 1u : 0u;
  }
  __syncthreads();
  if (t == 0) {
    float tail_sq = s_sums[0], mid_sq = s_sums[1];
    float qt = sqrtf(tail_sq);
    p->q_tail_norm = qt;
    p->q_mid_norm = sqrtf(mid_sq);
    p->q_after_prefix = sqrtf(mid_sq + tail_sq);
    p->q_after_s1 = qt;
  }
}

// ---------------------------------------------------------------------------
// strata scan
// ---------------------------------------------------------------------------

struct LaneBlock {
  float scale, offset, tail, mid_n, high_n;
  uint32_t nib[8];
};

// One (block, query) evaluation: the stage functions of src/scan.rs:453-634
// composed as run_default_scan_kernel (654-691) / the L0Only branch (753-790).
// Returns the pushed-survivor mask; score/prefix_ip are this lane's values.
__device__ __forceinline__ uint64_t eval_block(const uint8_t* __restrict__ blk, uint64_t active,
                                              const LaneBlock& m, const float* __restrict__ lut,
                                              const mrl_query_plan* __restrict__ p, const ScanParams& sp,
                                              float tau, float& prefix_ip_out, float& score_out,
                                              uint64_t* masks) {
  const float alpha = sp.alpha;
  if (sp.strata == MRL_STRATA_L0_ONLY) {
    // sign plane = bit 3 of every level; accum_plane skips weight == 0, and
    // adding a zero weight never changes a sum that started at +0.
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
    float ub = prefix_ip + alpha * p->q_after_prefix * x_rest;
    uint64_t surv = ballot(ub >= tau) & active;
    masks[1] = masks[2] = masks[3] = masks[4] = surv;
    prefix_ip_out = prefix_ip;
    score_out = prefix_ip;
    return surv;
  }

  // Stage: 4-bit prefix IP (scan.rs:453-517).  lut[d*16 + level] holds the
  // reference's product codebook[level] * weight (or level * weight), so the
  // per-vector sum over d is the same sequence of f32 additions.
  float acc = zero_acc();
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t w = m.nib[j];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = acc + lut[(8 * j + i) * 16 + ((w >> (4 * i)) & 15u)];
  }
  const bool eden = p->prefix_codec == MRL_PREFIX_EDEN_PROD;
  float prefix_ip = eden ? p->eden_mean_ip + m.scale * acc : acc * m.scale + m.offset * p->prefix_sum;
  float score = prefix_ip;
  float ub = prefix_ip + alpha * (p->q_mid_norm * m.mid_n + p->q_tail_norm * m.high_n);
  uint64_t surv = ballot(ub >= tau) & active;
  masks[1] = masks[2] = masks[3] = surv;
  prefix_ip_out = prefix_ip;

  const bool rabitq = sp.strata == MRL_STRATA_L1_RABITQ || sp.strata == MRL_STRATA_FULL64B;
  const bool full = sp.strata == MRL_STRATA_FULL64B;
  if (surv != 0 && rabitq) {
    // Stage: mid-band 1-bit IP (scan.rs:520-569), set bits added in d order.
    const uint64_t* __restrict__ s1p = reinterpret_cast<const uint64_t*>(blk + kDevS1);
    const bool b1 = p->mid_codec == MRL_MID_EDEN_B1;
    const float* __restrict__ w2 = b1 ? p->eden_mid_deltas : p->rabitq_weights2;
    float s1 = b1 ? p->eden_mid_base : p->rabitq_base;
#pragma unroll 16
    for (int d = 0; d < 128; ++d) {
      if (lane_in(s1p[d] & surv)) s1 = s1 + w2[d];
    }
    score = b1 ? score + (p->eden_mid_mean_ip + m.offset * s1) : score + s1 * m.mid_n;
    // Stage: post-S1 CS (scan.rs:572-584)
    float ub2 = score + alpha * p->q_after_s1 * m.high_n;
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
      const uint64_t* __restrict__ s4p = reinterpret_cast<const uint64_t*>(blk + kDevS4);
      float s4 = p->tail_fold_base;
#pragma unroll 16
      for (int d = 0; d < 64; ++d) {
        if (lane_in(s4p[d] & surv)) s4 = s4 + p->tail_fold_weights2[d];
      }
      score = score + s4 * hn * w_s4;
    }
  }
  masks[4] = surv;
  score_out = score;
  return surv;
}

template <int QT, bool DIAG>
__global__ __launch_bounds__(256) void k_scan(ScanArgs a) {
  __shared__ float s_lut[QT * 1024];
  __shared__ float s_rho[256];
  __shared__ float s_midf[256];

  const int tid = threadIdx.x;
  const uint32_t q0 = blockIdx.y * QT;
  const int nq = (int)min((uint32_t)QT, a.n_q - q0);

  for (int e = tid; e < QT * 1024; e += 256) {
    int qi = e >> 10;
    if (qi < nq) {
      const mrl_query_plan* p = a.plans + q0 + qi;
      int d = (e >> 4) & 63, l = e & 15;
      float cb = p->prefix_codec == MRL_PREFIX_EDEN_PROD ? p->eden_codebook[l] : (float)l;
      s_lut[e] = cb * p->prefix_weight[d];
    }
  }
  s_rho[tid] = a.flag_tabs[tid];
  s_midf[tid] = a.flag_tabs[256 + tid];
  __syncthreads();

  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lane = lane_id();
  const ScanParams sp = a.sp;
  uint64_t st_blocks = 0, st_active = 0, st_prefix = 0, st_s1 = 0, st_s4 = 0, st_pushed = 0;

  for (uint32_t pos = blockIdx.x * 4 + wave; pos < a.n_order; pos += gridDim.x * 4) {
    const uint32_t b = a.order ? a.order[pos] : pos;
    const uint8_t* __restrict__ blk = a.idx + (uint64_t)b * kBlockBytes;
    const uint32_t min_ts = *reinterpret_cast<const uint32_t*>(blk + kOrigMinTs);
    const uint32_t max_ts = *reinterpret_cast<const uint32_t*>(blk + kOrigMaxTs);
    const uint64_t tomb = *reinterpret_cast<const uint64_t*>(blk + kOrigTombstone);
    bool skip = false;
    if (sp.temporal) {  // scan.rs:719-730
      if (sp.has_lo && max_ts < sp.lo) skip = true;
      if (sp.has_hi && min_ts > sp.hi) skip = true;
    }
    const uint64_t active = ~tomb;
    if (skip || active == 0) {
      if (DIAG) {
        for (int qi = 0; qi < nq; ++qi) {
          uint64_t o = ((uint64_t)(q0 + qi) * a.n_blocks + b);
          if (lane < 5) a.d_masks[o * 5 + lane] = 0;
          a.d_prefix[o * 64 + lane] = 0.0f;
          a.d_score[o * 64 + lane] = 0.0f;
        }
      }
      continue;
    }
    // per-lane meta decode (block.rs:61-99)
    LaneBlock m;
    m.scale = h2f(reinterpret_cast<const uint16_t*>(blk + kDevScale)[lane]);
    m.offset = h2f(reinterpret_cast<const uint16_t*>(blk + kDevOffset)[lane]);
    m.tail = h2f(reinterpret_cast<const uint16_t*>(blk + kDevTail)[lane]);
    const uint32_t fl = blk[kDevFlags + lane];
    const float t = fmaxf(m.tail, 0.0f);
    m.mid_n = fmaxf(s_midf[fl] * t, 1e-6f);
    m.high_n = fmaxf(s_rho[fl] * t, 0.0f);
    const uint32_t* nibp = reinterpret_cast<const uint32_t*>(blk + kDevNibbles);
#pragma unroll
    for (int j = 0; j < 8; ++j) m.nib[j] = nibp[64 * j + lane];

    const uint32_t n_active = (uint32_t)__popcll(active);
    for (int qi = 0; qi < nq; ++qi) {
      const uint32_t q = q0 + qi;
      const mrl_query_plan* __restrict__ p = a.plans + q;
      const float tq = a.tau[q];
      const float tau = sp.exhaustive ? -INFINITY : tq;
      uint64_t masks[5];
      masks[0] = active;
      float prefix_ip, score;
      uint64_t surv = eval_block(blk, active, m, s_lut + qi * 1024, p, sp, tau, prefix_ip, score, masks);
      if (DIAG) {
        uint64_t o = ((uint64_t)q * a.n_blocks + b);
        if (lane < 5) {
          uint64_t mv = lane == 0 ? masks[0] : lane == 1 ? masks[1] : lane == 2 ? masks[2] : lane == 3 ? masks[3] : masks[4];
          a.d_masks[o * 5 + lane] = mv;
        }
        a.d_prefix[o * 64 + lane] = prefix_ip;
        a.d_score[o * 64 + lane] = score;
      } else {
        st_blocks += 1;
        st_active += n_active;
        st_prefix += (uint64_t)__popcll(masks[1]);
        st_s1 += (uint64_t)__popcll(masks[2]);
        st_s4 += (uint64_t)__popcll(masks[3]);
        st_pushed += (uint64_t)__popcll(surv);
        const bool mine = (surv >> lane) & 1ull;
        if (ballot(mine && score != score) != 0 && lane == 0) atomicOr(a.err, 1u);
        const uint64_t pm = ballot(mine && score >= tq);
        if (pm != 0) {
          const uint32_t first = (uint32_t)__ffsll((long long)pm) - 1;
          uint32_t base = 0;
          if (lane == first) base = atomicAdd(a.cand_count + q, (uint32_t)__popcll(pm));
          base = __shfl(base, (int)first);
          if ((pm >> lane) & 1ull) {
            uint32_t slot = base + lanes_below(pm);
            if (slot < a.cand_cap) {
              a.cand_score[(uint64_t)q * a.cand_cap + slot] = score;
              a.cand_row[(uint64_t)q * a.cand_cap + slot] = b * 64u + lane;
            }
          }
        }
      }
    }
  }
  if (!DIAG && lane == 0 && a.stats) {
    atomicAdd(a.stats + kStatBlocks, (unsigned long long)st_blocks);
    atomicAdd(a.stats + kStatActive, (unsigned long long)st_active);
    atomicAdd(a.stats + kStatPrefix, (unsigned long long)st_prefix);
    atomicAdd(a.stats + kStatS1, (unsigned long long)st_s1);
    atomicAdd(a.stats + kStatS4Budget, (unsigned long long)st_s4);
    atomicAdd(a.stats + kStatPushed, (unsigned long long)st_pushed);
  }
}

// ---------------------------------------------------------------------------
// top-K selection over per-query candidate lists
// Order: score descending, then row ascending (a total order, so keeping the
// best K after every pass yields the global best K).
// ---------------------------------------------------------------------------
constexpr int kSortCap = 8192;
constexpr int kSelThreads = 1024;


__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t row) {
  return ((uint64_t)key << 32) | (uint64_t)(~row);
}

// Descending bitonic sort of s[0..n2) (n2 a power of two).
__device__ void bitonic_desc(uint64_t* s, int n2) {
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

// Wave 0 finds the histogram bin holding the need-th entry, counting from
// the top bin down (desc) or from bin 0 up (asc).  Writes bin / count beyond.
__device__ void find_boundary(const uint32_t* hist, uint32_t nb, uint32_t need, bool desc,
                              uint32_t* out_bin, uint32_t* out_before) {
  if (threadIdx.x >= 64) return;
  const uint32_t lane = threadIdx.x;
  const uint32_t per = nb / 64;  // nb is 1024 or 2048
  uint32_t part = 0;
  for (uint32_t i = 0; i < per; ++i) {
    uint32_t bin = desc ? (nb - 1 - (lane * per + i)) : (lane * per + i);
    part += hist[bin];
  }
  // inclusive prefix over lanes
  uint32_t incl = part;
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t o = __shfl_up(incl, off);
    if ((int)lane >= off) incl += o;
  }
  const uint32_t excl = incl - part;
  const bool hit = excl < need && incl >= need;
  const uint64_t hm = __ballot(hit);
  const uint32_t src = (uint32_t)__ffsll((long long)hm) - 1;
  if (lane == src) {
    uint32_t before = excl;
    for (uint32_t i = 0; i < per; ++i) {
      uint32_t bin = desc ? (nb - 1 - (lane * per + i)) : (lane * per + i);
      uint32_t c = hist[bin];
      if (before + c >= need) {
        *out_bin = bin;
        *out_before = before;
        break;
      }
      before += c;
    }
  }
}

__global__ __launch_bounds__(kSelThreads) void k_select(SelectArgs a) {
  __shared__ uint64_t s_buf[kSortCap];
  __shared__ uint32_t s_hist[2048];
  __shared__ uint32_t s_misc[4];

  const uint32_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const uint32_t raw = a.cand_count[q];
  const uint32_t n = raw < a.cand_cap ? raw : a.cand_cap;
  const float* sc = a.cand_score + (uint64_t)q * a.cand_cap;
  const uint32_t* rw = a.cand_row + (uint64_t)q * a.cand_cap;
  const uint32_t K = a.k;
  if (tid == 0 && raw > a.cand_cap) a.overflow[q] = 1u;

  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};

  // gather mode: 0 all entries; 1 (key >> sel_shift) >= sel_prefix;
  // 2 key > tie_key, plus the tie_need smallest rows among key == tie_key.
  int mode = 0;
  uint32_t sel_shift = 0, sel_prefix = 0, tie_key = 0, tie_need = 0;
  if (n > (uint32_t)kSortCap) {
    // MSB-first radix select on the score key, stopping once everything at or
    // above the boundary prefix fits in the sort buffer.
    uint32_t prefix = 0, need = K;
    mode = 2;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass], wd = widths[pass];
      const uint32_t nb = 1u << wd;
      for (int i = tid; i < 2048; i += kSelThreads) s_hist[i] = 0;
      __syncthreads();
      for (uint32_t i = tid; i < n; i += kSelThreads) {
        uint32_t key = score_key(sc[i]);
        if (pass == 0 || (key >> (sh + wd)) == prefix) atomicAdd(&s_hist[(key >> sh) & (nb - 1)], 1u);
      }
      __syncthreads();
      find_boundary(s_hist, nb, need, true, &s_misc[0], &s_misc[1]);
      __syncthreads();
      const uint32_t bsel = s_misc[0], above = s_misc[1], inbin = s_hist[bsel];
      __syncthreads();
      const uint32_t definite = (K - need) + above;
      need -= above;
      prefix = (prefix << wd) | bsel;
      if (definite + inbin <= (uint32_t)kSortCap) {
        mode = 1;
        sel_shift = (uint32_t)sh;
        sel_prefix = prefix;
        break;
      }
    }
    if (mode == 2) {
      tie_key = prefix;  // exact K-th key; more exact ties than the buffer holds
      tie_need = need;
    }
  }

  if (tid == 0) s_misc[2] = 0;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kSelThreads) {
    uint32_t key = score_key(sc[i]);
    bool take = mode == 0 ? true : mode == 1 ? ((key >> sel_shift) >= sel_prefix) : (key > tie_key);
    if (take) {
      uint32_t slot = atomicAdd(&s_misc[2], 1u);
      if (slot < (uint32_t)kSortCap) s_buf[slot] = composite(key, rw[i]);
    }
  }
  __syncthreads();
  if (mode == 2) {
    // Keep the tie_need smallest rows among entries whose key equals tie_key
    // (radix select over the 32 row bits, ascending).  Rows are unique.
    uint32_t prefix = 0, need = tie_need;
    for (int pass = 0; pass < 3; ++pass) {
      const int sh = shifts[pass], wd = widths[pass];
      const uint32_t nb = 1u << wd;
      for (int i = tid; i < 2048; i += kSelThreads) s_hist[i] = 0;
      __syncthreads();
      for (uint32_t i = tid; i < n; i += kSelThreads) {
        if (score_key(sc[i]) != tie_key) continue;
        uint32_t r = rw[i];
        if (pass == 0 || (r >> (sh + wd)) == prefix) atomicAdd(&s_hist[(r >> sh) & (nb - 1)], 1u);
      }
      __syncthreads();
      find_boundary(s_hist, nb, need, false, &s_misc[0], &s_misc[1]);
      __syncthreads();
      need -= s_misc[1];
      prefix = (prefix << wd) | s_misc[0];
      __syncthreads();
    }
    const uint32_t row_max = prefix;
    for (uint32_t i = tid; i < n; i += kSelThreads) {
      uint32_t key = score_key(sc[i]);
      if (key == tie_key && rw[i] <= row_max) {
        uint32_t slot = atomicAdd(&s_misc[2], 1u);
        if (slot < (uint32_t)kSortCap) s_buf[slot] = composite(key, rw[i]);
      }
    }
    __syncthreads();
  }
  uint32_t m = s_misc[2];
  if (m > (uint32_t)kSortCap) m = kSortCap;  // cannot happen: the boundary search bounds m
  int n2 = 1;
  while ((uint32_t)n2 < m) n2 <<= 1;
  for (int i = (int)m + tid; i < n2; i += kSelThreads) s_buf[i] = 0ull;
  __syncthreads();
  bitonic_desc(s_buf, n2);

  const uint32_t keep = m < K ? m : K;
  if (a.final_pass) {
    for (uint32_t i = tid; i < keep; i += kSelThreads) {
      uint64_t c = s_buf[i];
      uint32_t row = ~(uint32_t)c;
      a.out_ids[(uint64_t)q * K + i] = ((uint64_t)(row >> 6) << 16) | (uint64_t)(row & 63u);
      a.out_scores[(uint64_t)q * K + i] = key_score((uint32_t)(c >> 32));
    }
    if (tid == 0) a.out_counts[q] = keep;
  } else {
    float* wsc = a.cand_score + (uint64_t)q * a.cand_cap;
    uint32_t* wrw = a.cand_row + (uint64_t)q * a.cand_cap;
    for (uint32_t i = tid; i < keep; i += kSelThreads) {
      uint64_t c = s_buf[i];
      wsc[i] = key_score((uint32_t)(c >> 32));
      wrw[i] = ~(uint32_t)c;
    }
    if (tid == 0) {
      a.cand_count[q] = keep;
      a.tau[q] = keep >= K ? key_score((uint32_t)(s_buf[K - 1] >> 32)) : -INFINITY;
    }
  }
}

// Resets per-query pass state without hipMemsetAsync (safe under graph capture).
__global__ void k_reset(uint32_t n_q, uint32_t* cand_count, float* tau, uint32_t* overflow,
                        unsigned long long* stats, uint32_t* err) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_q) {
    cand_count[i] = 0;
    tau[i] = -INFINITY;
    overflow[i] = 0;
  }
  if (stats && i < kStatCount) stats[i] = 0;
  if (i == 0) *err = 0;
}

__global__ void k_fill_f32(float* p, uint64_t n, float v) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
hipError_t launch_relayout(const uint8_t* src, uint8_t* dst, uint64_t n_blocks, bool to_device,
                           hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  uint32_t grid = (uint32_t)(n_blocks < 65536 ? n_blocks : 65536);
  if (to_device) hipLaunchKernelGGL(k_relayout_to_device, dim3(grid), dim3(64), 0, s, src, dst, n_blocks);
  else hipLaunchKernelGGL(k_relayout_to_host, dim3(grid), dim3(64), 0, s, src, dst, n_blocks);
  return hipGetLastError();
}

hipError_t launch_plan(const PlanArgs& a, hipStream_t s) {
  if (a.n_q == 0) return hipSuccess;
  hipLaunchKernelGGL(k_plan, dim3(a.n_q), dim3(128), 0, s, a);
  return hipGetLastError();
}

int scan_query_tile(uint32_t n_q) { return n_q >= 8 ? 8 : 1; }

hipError_t launch_scan(const ScanArgs& a, bool diag, hipStream_t s) {
  if (a.n_order == 0 || a.n_q == 0) return hipSuccess;
  const int qt = scan_query_tile(a.n_q);
  const uint32_t tiles = (a.n_q + qt - 1) / qt;
  uint32_t waves_needed = a.n_order;
  uint32_t grid = (waves_needed + 3) / 4;
  const uint32_t max_grid = tiles >= 64 ? 256 : (tiles >= 8 ? 1024 : 2048);
  if (grid > max_grid) grid = max_grid;
  dim3 g(grid, tiles);
  if (qt == 8) {
    if (diag) hipLaunchKernelGGL((k_scan<8, true>), g, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_scan<8, false>), g, dim3(256), 0, s, a);
  } else {
    if (diag) hipLaunchKernelGGL((k_scan<1, true>), g, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_scan<1, false>), g, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_select(const SelectArgs& a, uint32_t n_q, hipStream_t s) {
  if (n_q == 0) return hipSuccess;
  hipLaunchKernelGGL(k_select, dim3(n_q), dim3(kSelThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_reset(uint32_t n_q, uint32_t* cand_count, float* tau, uint32_t* overflow,
                        unsigned long long* stats, uint32_t* err, hipStream_t s) {
  uint32_t n = n_q > (uint32_t)kStatCount ? n_q : (uint32_t)kStatCount;
  hipLaunchKernelGGL(k_reset, dim3((n + 255) / 256), dim3(256), 0, s, n_q, cand_count, tau, overflow, stats,
                     err);
  return hipGetLastError();
}

hipError_t launch_fill(float* p, uint64_t n, float v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_f32, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace mrl
