// mrl_encode.hip -- gfx950 encoder: f32 rows -> PaxBlock64 records, byte-identical to
// encode_block_with_fits (src/quantize.rs:36-96) as driven by encode_f32_corpus_par
// (src/encoder.rs:195-219): timestamp = row index, one source id for every row.
//
// One wave per block.  The f32 arithmetic keeps the reference's operations and order
// (-ffp-contract=off, correctly rounded division/sqrt, IEEE denormals):
//  - running sums (norms, EDEN inner products) run with lane = vector, each lane
//    adding its own vector's terms in index order;
//  - FWHT butterflies run with lane = dim: stage h combines elements j and j + h
//    with one add or subtract, as the reference's in-place loops do, so the stage
//    results are the same values in any lane order;
//  - the bitplanes are wave ballots (bit v of plane word d = slot v);
//  - CRC-32 of the 4096 bytes: lane k folds bytes 64k..64k+63 into a register from
//    zero, the registers are moved to the end of the block with precomputed
//    zero-extension maps and xor-ed (CRC is linear over GF(2)), then the
//    all-ones initial register and final xor are applied.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mrl_half.h"
#include "mrl_internal.h"

namespace mrl {

namespace {

__device__ __forceinline__ float zero_acc() {
  float z = 0.0f;
  asm volatile("" : "+v"(z));
  return z;
}

// tail_rademacher / rademacher_diag sign (rotate.rs:53-67, eden.rs:75-88)
__device__ __forceinline__ float mix_sign(uint64_t a, uint64_t i) {
  uint64_t x = (a * 0x9E3779B97F4A7C15ull + i) * 0xBF58476D1CE4E5B9ull;
  x ^= x >> 30;
  x = x * 0x94D049BB133111EBull;
  x ^= x >> 27;
  return (x & 1ull) == 0 ? 1.0f : -1.0f;
}

// nearest_centroid (eden.rs:58-71): first index with cb[i] >= z, ties to the lower level
__device__ __forceinline__ int nearest_centroid(const float* cb, int n, float z) {
  int below = 0;
  while (below < n && cb[below] < z) ++below;
  if (below < n && cb[below] == z) return below;
  if (below == 0) return 0;
  if (below >= n) return n - 1;
  return fabsf(z - cb[below - 1]) <= fabsf(cb[below] - z) ? below - 1 : below;
}

__device__ __forceinline__ float rclamp(float x, float lo, float hi) {
  if (x < lo) x = lo;
  if (x > hi) x = hi;
  return x;
}

// Rust `f32 as u8`: saturating, NaN -> 0
__device__ __forceinline__ uint32_t as_u8(float x) {
  if (!(x == x) || x <= 0.0f) return 0u;
  if (x >= 255.0f) return 255u;
  return (uint32_t)x;
}

// In-place FWHT stages over a 64-point vector held one element per lane.
__device__ __forceinline__ float fwht64_lane(float y, uint32_t lane) {
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
    const float o = __shfl_xor(y, h);
    y = (lane & (uint32_t)h) ? (o - y) : (y + o);
  }
  return y;
}

// 128-point: elements lane and lane + 64.
__device__ __forceinline__ void fwht128_lane(float& y0, float& y1, uint32_t lane) {
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
    const float o0 = __shfl_xor(y0, h);
    const float o1 = __shfl_xor(y1, h);
    y0 = (lane & (uint32_t)h) ? (o0 - y0) : (y0 + o0);
    y1 = (lane & (uint32_t)h) ? (o1 - y1) : (y1 + o1);
  }
  const float x = y0, y = y1;
  y0 = x + y;
  y1 = x - y;
}

}  // namespace

__global__ __launch_bounds__(64) void k_encode(EncodeArgs a) {
  __shared__ __align__(16) uint8_t img[kBlockBytes];
  __shared__ float S[64][129];  // per-vector values (padded rows)
  __shared__ uint8_t lev[64][65];
  __shared__ uint8_t rq[64][129];
  __shared__ uint8_t fold[64][65];
  __shared__ uint32_t T[256];
  __shared__ float cb4[16];
  __shared__ float cb1[2];

  const uint32_t lane = threadIdx.x;
  for (int i = lane; i < 256; i += 64) T[i] = a.crc_tab[i];
  if (lane < 16) cb4[lane] = a.c.eden_codebook[lane];
  if (lane < 2) cb1[lane] = a.c.eden_mid_codebook[lane];
  __syncthreads();

  const uint32_t dims = a.dims;
  const float inv64 = a.c.inv_sqrt64, inv128 = a.c.inv_sqrt128;
  const float sqrt64 = a.sqrt64, sqrt128 = a.sqrt128;
  const int nb_tail = dims > (uint32_t)kTailStart
                          ? ((int)(dims - kTailStart) / 64 < kTailFoldBlocks ? (int)(dims - kTailStart) / 64
                                                                                : kTailFoldBlocks)
                          : 0;

  for (uint64_t b = blockIdx.x; b < a.n_blocks; b += gridDim.x) {
    const uint64_t row0 = b * 64;
    const uint32_t rows = (uint32_t)((a.n - row0) < 64 ? (a.n - row0) : 64);
    const uint32_t v = lane;
    const bool valid = v < rows;
    const float* xv = a.x + (row0 + (valid ? v : 0)) * dims;
    for (int i = 0; i < 16; ++i) reinterpret_cast<uint32_t*>(img)[lane * 16 + i] = 0u;

    float scale, offset;
    // ---- prefix: EDEN-prod (quantize.rs:265-295, eden.rs:225-269) or MinMax4 (220-246)
    if (a.eden_mean) {
      float nsq = zero_acc();
      for (int i = 0; i < 64; ++i) {
        const float c = xv[i] - a.eden_mean[i];
        nsq += c * c;
        S[v][i] = c;
      }
      const float cn = fmaxf(sqrtf(nsq), 1e-12f);
      const float inv = 1.0f / cn;
      for (int i = 0; i < 64; ++i) S[v][i] = (S[v][i] * inv) * mix_sign(a.eden_seed, (uint64_t)i);
      __syncthreads();
      for (int u = 0; u < 64; ++u) S[u][lane] = fwht64_lane(S[u][lane], lane) * inv64;
      __syncthreads();
      float ip = zero_acc();
      for (int i = 0; i < 64; ++i) {
        const float z = S[v][i];
        const int l = nearest_centroid(cb4, 16, z * sqrt64);
        lev[v][i] = (uint8_t)l;
        const float cw = cb4[l] * inv64;
        ip += z * cw;
      }
      const float s = fabsf(ip) > 1e-12f ? 1.0f / ip : 0.0f;
      scale = cn * s;
      offset = 0.0f;
    } else {
      float mn = INFINITY, mx = -INFINITY;
      for (int i = 0; i < 64; ++i) mn = fminf(mn, xv[i]);
      for (int i = 0; i < 64; ++i) mx = fmaxf(mx, xv[i]);
      const float range = fmaxf(mx - mn, 1e-8f);
      scale = range / 15.0f;
      offset = mn;
      for (int i = 0; i < 64; ++i) lev[v][i] = (uint8_t)as_u8(rclamp(roundf((xv[i] - offset) / scale), 0.0f, 15.0f));
    }

    // ---- mid band: EdenB1 (eden.rs:225-269 with d = 128, b = 1) or RaBitQ signs (quantize.rs:199-206)
    if (a.eden_mean && a.mid_mean) {
      float nsq = zero_acc();
      for (int i = 0; i < 128; ++i) {
        const float c = xv[kPrefixDims + i] - a.mid_mean[i];
        nsq += c * c;
        S[v][i] = c;
      }
      const float cn = fmaxf(sqrtf(nsq), 1e-12f);
      const float inv = 1.0f / cn;
      for (int i = 0; i < 128; ++i) S[v][i] = (S[v][i] * inv) * mix_sign(a.mid_seed, (uint64_t)i);
      __syncthreads();
      for (int u = 0; u < 64; ++u) {
        float y0 = S[u][lane], y1 = S[u][lane + 64];
        fwht128_lane(y0, y1, lane);
        S[u][lane] = y0 * inv128;
        S[u][lane + 64] = y1 * inv128;
      }
      __syncthreads();
      float ip = zero_acc();
      for (int i = 0; i < 128; ++i) {
        const float z = S[v][i];
        const int l = nearest_centroid(cb1, 2, z * sqrt128);
        rq[v][i] = (uint8_t)l;
        const float cw = cb1[l] * inv128;
        ip += z * cw;
      }
      const float s = fabsf(ip) > 1e-12f ? 1.0f / ip : 0.0f;
      offset = cn * s;
    } else {
      for (int u = 0; u < 64; ++u) {
        const float* xu = a.x + (row0 + (u < (int)rows ? u : 0)) * dims + kPrefixDims;
        float y0 = xu[lane], y1 = xu[lane + 64];
        fwht128_lane(y0, y1, lane);
        rq[u][lane] = (y0 * inv128) >= 0.0f;
        rq[u][lane + 64] = (y1 * inv128) >= 0.0f;
      }
    }

    // ---- folded tail signs (rotate.rs:73-100, quantize.rs:207-213)
    for (int u = 0; u < 64; ++u) {
      const float* xu = a.x + (row0 + (u < (int)rows ? u : 0)) * dims + kTailStart;
      float t = zero_acc();
      for (int bb = 0; bb < nb_tail; ++bb) t += mix_sign((uint64_t)bb, (uint64_t)lane) * xu[64 * bb + lane];
      t = fwht64_lane(t, lane) * inv64;
      fold[u][lane] = t >= 0.0f;
    }

    // ---- residual norms and rho flags (quantize.rs:180-197, block.rs:102-108)
    float msq = zero_acc();
    for (int i = 0; i < 128; ++i) {
      const float x = xv[kPrefixDims + i];
      msq += x * x;
    }
    float hsq = zero_acc();
    for (uint32_t d = kTailStart; d < dims; ++d) hsq += xv[d] * xv[d];
    const float rest = sqrtf(msq + hsq);
    const float high = sqrtf(hsq);
    uint32_t flags = 0;
    if (!(rest <= 1e-12f)) flags = as_u8(rclamp(roundf(rclamp(high / rest, 0.0f, 1.0f) * 255.0f), 0.0f, 255.0f));
    __syncthreads();
    if (valid) {
      uint8_t* m = img + kOrigMeta + 7 * v;
      const uint32_t hs = f32_to_f16(scale), ho = f32_to_f16(offset), hr = f32_to_f16(rest);
      m[0] = (uint8_t)hs;
      m[1] = (uint8_t)(hs >> 8);
      m[2] = (uint8_t)ho;
      m[3] = (uint8_t)(ho >> 8);
      m[4] = (uint8_t)hr;
      m[5] = (uint8_t)(hr >> 8);
      m[6] = (uint8_t)flags;
    }

    // ---- bitplanes (write_4bit_planes, quantize.rs:297-315): word d, bit v = slot v
    uint64_t w3 = 0, w2 = 0, w1 = 0, w0 = 0, wf = 0, wr0 = 0, wr1 = 0;
    for (int d = 0; d < 64; ++d) {
      const uint32_t l = valid ? lev[v][d] : 0u;
      const uint64_t b3 = __ballot(l & 8u), b2 = __ballot(l & 4u), b1 = __ballot(l & 2u), b0 = __ballot(l & 1u);
      const uint64_t bf = __ballot(valid && fold[v][d]);
      const uint64_t br0 = __ballot(valid && rq[v][d]);
      const uint64_t br1 = __ballot(valid && rq[v][d + 64]);
      if (lane == (uint32_t)d) {
        w3 = b3;
        w2 = b2;
        w1 = b1;
        w0 = b0;
        wf = bf;
        wr0 = br0;
        wr1 = br1;
      }
    }
    reinterpret_cast<uint64_t*>(img + kOrigS0)[lane] = w3;
    reinterpret_cast<uint64_t*>(img + kOrigS2)[lane] = w2;
    reinterpret_cast<uint64_t*>(img + kOrigS3)[lane] = w1;
    reinterpret_cast<uint64_t*>(img + kOrigS5)[lane] = w0;
    reinterpret_cast<uint64_t*>(img + kOrigS4)[lane] = wf;
    reinterpret_cast<uint64_t*>(img + kOrigS1)[lane] = wr0;
    reinterpret_cast<uint64_t*>(img + kOrigS1)[lane + 64] = wr1;
    if (lane == 0) {
      uint32_t* h = reinterpret_cast<uint32_t*>(img);
      h[0] = (uint32_t)row0;              // min_timestamp
      h[1] = (uint32_t)(row0 + rows - 1);  // max_timestamp
      h[2] = a.source;                     // source_mask
      const uint64_t tomb = rows < 64 ? (~0ull << rows) : 0ull;
      h[4] = (uint32_t)tomb;
      h[5] = (uint32_t)(tomb >> 32);
    }
    if (a.cluster) {
      // cluster-grouped convention: coarse_cluster_id and block_flags (block.rs:38-39) when every row of the
      // block is in one cluster below 65536
      const uint32_t c = lane < rows ? a.cluster[row0 + lane] : 0u;
      const uint32_t c0 = __shfl(c, 0);
      const bool one = __ballot(lane < rows && c != c0) == 0 && c0 < 65536u;
      if (lane == 0 && one) reinterpret_cast<uint32_t*>(img)[3] = c0 | (kBlockFlagOneCluster << 16);
    }
    __syncthreads();

    // ---- CRC-32 (recompute_crc, block.rs:186-190) over the block with crc = 0
    uint32_t c = 0;
    const uint8_t* chunk = img + 64 * lane;
    for (int j = 0; j < 64; ++j) c = T[(c ^ chunk[j]) & 0xffu] ^ (c >> 8);
    uint32_t z = 0;
    const uint32_t* zt = a.crc_zt + 32 * lane;
    for (int i = 0; i < 32; ++i) z ^= ((c >> i) & 1u) ? zt[i] : 0u;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) z ^= (uint32_t)__shfl_xor((int)z, off);
    if (lane == 0) reinterpret_cast<uint32_t*>(img)[kOrigCrc / 4] = z ^ a.crc_const;
    __syncthreads();
    const uint4* src = reinterpret_cast<const uint4*>(img) + 4 * lane;
    uint4* dst = reinterpret_cast<uint4*>(a.out + b * kBlockBytes) + 4 * lane;
    for (int i = 0; i < 4; ++i) dst[i] = src[i];
    __syncthreads();
  }
}

hipError_t launch_encode(const EncodeArgs& a, hipStream_t s) {
  if (a.n_blocks == 0) return hipSuccess;
  const uint32_t grid = (uint32_t)(a.n_blocks < 16384 ? a.n_blocks : 16384);
  hipLaunchKernelGGL(k_encode, dim3(grid), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace mrl
