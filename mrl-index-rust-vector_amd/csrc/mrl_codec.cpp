// mrl_codec.cpp -- ingest-side host code: f16, CRC-32, EDEN fit, PaxBlock64
// encoder (src/quantize.rs, src/eden.rs, src/rotate.rs) and the seeded
// synthetic corpora used by the benchmark.  Multi-threaded with std::thread.
//
// The encoder is byte-identical to the reference: f32 operations in the
// reference order, Rust f32::round == roundf (half away from zero), f16
// conversion with round-to-nearest-even (half 2.7.1).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "mrl_codec.h"
#include "mrl_internal.h"

namespace mrl {

// ---------------------------------------------------------------------------
// IEEE binary16
// ---------------------------------------------------------------------------
static inline uint32_t fbits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bitsf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if ((h & 0x7fffu) == 0) return bitsf(sign);
  if (e == 0x1f) return bitsf(sign | 0x7f800000u | (man ? (0x400000u | (man << 13)) : 0u));
  if (e == 0) {
    int shift = 0;
    while (!(man & 0x400u)) {
      man <<= 1;
      ++shift;
    }
    return bitsf(sign | ((uint32_t)(113 - shift) << 23) | ((man & 0x3ffu) << 13));
  }
  return bitsf(sign | ((e + 112u) << 23) | (man << 13));
}

uint16_t f32_to_f16(float f) {
  const uint32_t x = fbits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const int32_t e32 = (int32_t)((x >> 23) & 0xffu);
  const uint32_t man = x & 0x7fffffu;
  if (e32 == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  const int32_t e = e32 - 112;  // half exponent field
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  uint32_t sig, shift;
  uint16_t base;
  if (e > 0) {
    sig = man;
    shift = 13;
    base = (uint16_t)(sign | (uint16_t)(e << 10));
  } else {
    if (e < -10) return sign;
    sig = man | 0x800000u;
    shift = (uint32_t)(14 - e);
    base = sign;
  }
  uint32_t kept = sig >> shift;
  uint32_t rem = sig & ((1u << shift) - 1u);
  uint32_t halfway = 1u << (shift - 1);
  uint32_t out = base + kept;  // carry from the significand propagates into the exponent
  if (rem > halfway || (rem == halfway && (kept & 1u))) out += 1;
  return (uint16_t)out;
}

// ---------------------------------------------------------------------------
// CRC-32 (crc32fast 1.5.3 / ISO-HDLC), slicing by 8
// ---------------------------------------------------------------------------
static uint32_t g_crc[8][256];
static std::atomic<int> g_crc_ready{0};
static void crc_init() {
  if (g_crc_ready.load(std::memory_order_acquire)) return;
  static std::atomic<int> building{0};
  if (building.exchange(1)) {
    while (!g_crc_ready.load(std::memory_order_acquire)) std::this_thread::yield();
    return;
  }
  for (uint32_t i = 0; i < 256; ++i) {
    uint32_t c = i;
    for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
    g_crc[0][i] = c;
  }
  for (uint32_t i = 0; i < 256; ++i)
    for (int t = 1; t < 8; ++t) g_crc[t][i] = (g_crc[t - 1][i] >> 8) ^ g_crc[0][g_crc[t - 1][i] & 0xffu];
  g_crc_ready.store(1, std::memory_order_release);
}

uint32_t crc32(const uint8_t* p, size_t n) {
  crc_init();
  uint32_t c = 0xffffffffu;
  while (n >= 8) {
    uint32_t lo, hi;
    memcpy(&lo, p, 4);
    memcpy(&hi, p + 4, 4);
    lo ^= c;
    c = g_crc[7][lo & 0xff] ^ g_crc[6][(lo >> 8) & 0xff] ^ g_crc[5][(lo >> 16) & 0xff] ^ g_crc[4][lo >> 24] ^
        g_crc[3][hi & 0xff] ^ g_crc[2][(hi >> 8) & 0xff] ^ g_crc[1][(hi >> 16) & 0xff] ^ g_crc[0][hi >> 24];
    p += 8;
    n -= 8;
  }
  while (n--) c = g_crc[0][(c ^ *p++) & 0xffu] ^ (c >> 8);
  return c ^ 0xffffffffu;
}

// PaxBlock64::verify_crc (src/block.rs:192-197): CRC of the block with the
// crc field zeroed.
bool block_crc_ok(const uint8_t* block) {
  uint8_t copy[kBlockBytes];
  memcpy(copy, block, kBlockBytes);
  uint32_t expected;
  memcpy(&expected, copy + kOrigCrc, 4);
  memset(copy + kOrigCrc, 0, 4);
  return crc32(copy, kBlockBytes) == expected;
}

// ---------------------------------------------------------------------------
// rotations and EDEN (src/rotate.rs, src/eden.rs)
// ---------------------------------------------------------------------------
static void fwht(float* a, int n) {  // rotate.rs:13-33
  for (int h = 1; h < n; h *= 2)
    for (int i = 0; i < n; i += 2 * h)
      for (int j = i; j < i + h; ++j) {
        float x = a[j], y = a[j + h];
        a[j] = x + y;
        a[j + h] = x - y;
      }
  const float scale = 1.0f / sqrtf((float)n);
  for (int i = 0; i < n; ++i) a[i] *= scale;
}

static inline float mix_sign(uint64_t a, uint64_t i) {  // rotate.rs:53-67, eden.rs:75-88
  uint64_t x = (a * 0x9E3779B97F4A7C15ull + i) * 0xBF58476D1CE4E5B9ull;
  x ^= x >> 30;
  x *= 0x94D049BB133111EBull;
  x ^= x >> 27;
  return (x & 1ull) ? -1.0f : 1.0f;
}

static void rotate_tail_fold(const float* v, int len, float* u) {  // rotate.rs:73-100
  for (int d = 0; d < 64; ++d) u[d] = 0.0f;
  if (len > kTailStart) {
    int nb = std::min((len - kTailStart) / 64, kTailFoldBlocks);
    for (int b = 0; b < nb; ++b)
      for (int d = 0; d < 64; ++d) u[d] += mix_sign((uint64_t)b, (uint64_t)d) * v[kTailStart + 64 * b + d];
  }
  fwht(u, 64);
}

static const float kB1[2] = {-0.79788456f, 0.79788456f};
static const float kB4[16] = {-2.73258958f, -2.06901724f, -1.61804640f, -1.25623121f, -0.94234046f, -0.65675912f,
                              -0.38804830f, -0.12839503f, 0.12839503f,  0.38804830f,  0.65675912f,  0.94234046f,
                              1.25623121f,  1.61804640f,  2.06901724f,  2.73258958f};

const float* lloyd_max(int bits, int* n) {  // eden.rs:15-55 (b = 1 and 4 are the PaxBlock codecs)
  if (bits == 1) {
    *n = 2;
    return kB1;
  }
  if (bits == 4) {
    *n = 16;
    return kB4;
  }
  *n = 0;
  return nullptr;
}

static int nearest_centroid(const float* cb, int n, float z) {  // eden.rs:58-71
  int below = 0;
  while (below < n && cb[below] < z) ++below;
  if (below < n && cb[below] == z) return below;
  if (below == 0) return 0;
  if (below >= n) return n - 1;
  return fabsf(z - cb[below - 1]) <= fabsf(cb[below] - z) ? below - 1 : below;
}

// eden.rs:225-269; returns alpha = centered_norm * scale_s.
static float eden_encode(const float* mean, int d, int bits, uint64_t seed, const float* x, uint8_t* levels) {
  int ncb;
  const float* cb = lloyd_max(bits, &ncb);
  const float sqrt_d = sqrtf((float)d);
  const float inv_sqrt_d = 1.0f / sqrt_d;
  float c[128];
  float norm_sq = 0.0f;
  for (int i = 0; i < d; ++i) {
    float v = x[i] - mean[i];
    c[i] = v;
    norm_sq += v * v;
  }
  const float cn = fmaxf(sqrtf(norm_sq), 1e-12f);  // f32::max: a NaN norm yields 1e-12
  const float inv = 1.0f / cn;
  for (int i = 0; i < d; ++i) c[i] *= inv;
  for (int i = 0; i < d; ++i) c[i] *= mix_sign(seed, (uint64_t)i);
  fwht(c, d);
  float ip = 0.0f;
  for (int i = 0; i < d; ++i) {
    int l = nearest_centroid(cb, ncb, c[i] * sqrt_d);
    levels[i] = (uint8_t)l;
    float cw = cb[l] * inv_sqrt_d;
    ip += c[i] * cw;
  }
  const float s = fabsf(ip) > 1e-12f ? 1.0f / ip : 0.0f;
  return cn * s;
}

static inline float rclamp(float x, float lo, float hi) {
  if (x < lo) x = lo;
  if (x > hi) x = hi;
  return x;
}
static inline uint8_t as_u8(float x) {  // Rust `as u8`: saturating, NaN -> 0
  if (!(x == x) || x <= 0.0f) return 0;
  if (x >= 255.0f) return 255;
  return (uint8_t)x;
}

// ---------------------------------------------------------------------------
// encode_block_with_fits (src/quantize.rs:36-96)
// ---------------------------------------------------------------------------
static inline void put16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}
static inline void or_bit(uint8_t* block, int off, int d, int slot) { block[off + 8 * d + (slot >> 3)] |= (uint8_t)(1u << (slot & 7)); }

int encode_block(const float* vecs, uint32_t n, uint32_t dims, const uint32_t* ts, const uint32_t* src,
                 const EdenFitView* eden, const EdenFitView* eden_mid, uint8_t* block, uint32_t cluster) {
  if (n == 0 || n > 64 || dims < (uint32_t)(kPrefixDims + kRabitqDims)) return MRL_ERR_INVALID_ARG;
  if (eden && (eden->dim != 64 || eden->bits != 4)) return MRL_ERR_INVALID_ARG;
  if (eden_mid && (!eden || eden_mid->dim != 128 || eden_mid->bits != 1)) return MRL_ERR_INVALID_ARG;
  memset(block, 0, kBlockBytes);
  uint32_t min_ts = 0xffffffffu, max_ts = 0, smask = 0;
  for (uint32_t i = 0; i < n; ++i) {
    const float* v = vecs + (size_t)i * dims;
    min_ts = std::min(min_ts, ts[i]);
    max_ts = std::max(max_ts, ts[i]);
    smask |= src[i];
    uint8_t bits4[64], rq[128], fold[64];
    float scale, offset;
    // mid-band signs and folded-tail signs (quantize.rs:199-213)
    float rot[128];
    memcpy(rot, v + kPrefixDims, sizeof(rot));
    fwht(rot, 128);
    float tf[64];
    rotate_tail_fold(v, (int)dims, tf);
    for (int d = 0; d < 64; ++d) fold[d] = tf[d] >= 0.0f;
    if (eden) {  // quantize_vector_eden_dual (265-295)
      scale = eden_encode(eden->mean, 64, 4, eden->seed, v, bits4);
      if (eden_mid) {
        offset = eden_encode(eden_mid->mean, 128, 1, eden_mid->seed, v + kPrefixDims, rq);
      } else {
        offset = 0.0f;
        for (int d = 0; d < 128; ++d) rq[d] = rot[d] >= 0.0f;
      }
    } else {  // quantize_vector (220-246)
      float mn = INFINITY, mx = -INFINITY;
      for (int d = 0; d < 64; ++d) mn = fminf(mn, v[d]);
      for (int d = 0; d < 64; ++d) mx = fmaxf(mx, v[d]);
      const float range = fmaxf(mx - mn, 1e-8f);
      scale = range / 15.0f;
      offset = mn;
      for (int d = 0; d < 64; ++d) bits4[d] = as_u8(rclamp(roundf((v[d] - offset) / scale), 0.0f, 15.0f));
      for (int d = 0; d < 128; ++d) rq[d] = rot[d] >= 0.0f;
    }
    // residual_norms (180-197) and VectorMeta::pack_rho_flags (block.rs:102-108)
    float mid_sq = 0.0f;
    for (int d = 0; d < 128; ++d) {
      float x = v[kPrefixDims + d];
      mid_sq += x * x;
    }
    float high_sq = 0.0f;
    for (uint32_t d = kTailStart; d < dims; ++d) high_sq += v[d] * v[d];
    const float rest = sqrtf(mid_sq + high_sq);
    const float high = sqrtf(high_sq);
    uint8_t flags = 0;
    if (!(rest <= 1e-12f)) flags = as_u8(rclamp(roundf(rclamp(high / rest, 0.0f, 1.0f) * 255.0f), 0.0f, 255.0f));
    uint8_t* m = block + kOrigMeta + 7 * i;
    put16(m, f32_to_f16(scale));
    put16(m + 2, f32_to_f16(offset));
    put16(m + 4, f32_to_f16(rest));
    m[6] = flags;
    for (int d = 0; d < 64; ++d) {  // write_4bit_planes (297-315)
      if (bits4[d] & 8) or_bit(block, kOrigS0, d, (int)i);
      if (bits4[d] & 4) or_bit(block, kOrigS2, d, (int)i);
      if (bits4[d] & 2) or_bit(block, kOrigS3, d, (int)i);
      if (bits4[d] & 1) or_bit(block, kOrigS5, d, (int)i);
    }
    for (int d = 0; d < 128; ++d)
      if (rq[d]) or_bit(block, kOrigS1, d, (int)i);
    for (int d = 0; d < 64; ++d)
      if (fold[d]) or_bit(block, kOrigS4, d, (int)i);
  }
  uint64_t tomb = 0;
  for (uint32_t i = n; i < 64; ++i) tomb |= 1ull << i;  // unused slots: zero meta, tombstoned
  memcpy(block + kOrigMinTs, &min_ts, 4);
  memcpy(block + kOrigMaxTs, &max_ts, 4);
  memcpy(block + 8, &smask, 4);
  memcpy(block + kOrigTombstone, &tomb, 8);
  if (cluster < 65536u) {  // coarse_cluster_id, block_flags (block.rs:38-39)
    put16(block + 12, (uint16_t)cluster);
    put16(block + 14, (uint16_t)kBlockFlagOneCluster);
  }
  uint32_t crc = crc32(block, kBlockBytes);  // recompute_crc (block.rs:186-190)
  memcpy(block + kOrigCrc, &crc, 4);
  return MRL_OK;
}

int parallel_for(uint64_t n, int n_threads, const std::function<void(uint64_t, uint64_t)>& fn) {
  if (n_threads <= 0) n_threads = (int)std::max(1u, std::thread::hardware_concurrency());
  if ((uint64_t)n_threads > n) n_threads = (int)std::max<uint64_t>(1, n);
  if (n_threads <= 1) {
    fn(0, n);
    return 0;
  }
  std::vector<std::thread> th;
  std::atomic<uint64_t> next{0};
  const uint64_t chunk = std::max<uint64_t>(1, std::min<uint64_t>(256, n / ((uint64_t)n_threads * 8) + 1));
  for (int t = 0; t < n_threads; ++t)
    th.emplace_back([&]() {
      for (;;) {
        uint64_t s = next.fetch_add(chunk);
        if (s >= n) break;
        fn(s, std::min(n, s + chunk));
      }
    });
  for (auto& t : th) t.join();
  return 0;
}

uint32_t block_cluster(const uint32_t* c, uint64_t n) {
  if (n == 0 || c[0] >= 65536u) return kNoCluster;
  for (uint64_t i = 1; i < n; ++i)
    if (c[i] != c[0]) return kNoCluster;
  return c[0];
}

int encode_corpus(const float* matrix, uint64_t n, uint32_t dims, uint32_t default_source,
                  const EdenFitView* eden, const EdenFitView* eden_mid, int n_threads, uint8_t* out,
                  const uint32_t* cluster) {
  const uint64_t n_blocks = (n + 63) / 64;
  std::atomic<int> status{MRL_OK};
  parallel_for(n_blocks, n_threads, [&](uint64_t b0, uint64_t b1) {
    uint32_t ts[64], src[64];
    for (uint64_t b = b0; b < b1; ++b) {
      const uint64_t start = b * 64, end = std::min(n, start + 64);
      for (uint64_t j = start; j < end; ++j) {
        ts[j - start] = (uint32_t)j;  // encoder.rs:184-189
        src[j - start] = default_source;
      }
      const uint32_t cl = cluster ? block_cluster(cluster + start, end - start) : kNoCluster;
      int rc = encode_block(matrix + start * dims, (uint32_t)(end - start), dims, ts, src, eden, eden_mid,
                            out + b * kBlockBytes, cl);
      if (rc != MRL_OK) status.store(rc);
    }
  });
  return status.load();
}

int eden_fit_band(const float* rows, uint64_t n_rows, uint32_t stride, uint32_t start, uint32_t dim, float* mean) {
  if (n_rows == 0 || dim == 0) return MRL_ERR_INVALID_ARG;  // eden.rs:152
  for (uint32_t d = 0; d < dim; ++d) mean[d] = 0.0f;
  for (uint64_t r = 0; r < n_rows; ++r) {
    const float* x = rows + r * stride;
    for (uint32_t d = 0; d < dim; ++d) mean[d] += x[start + d];
  }
  const float inv = 1.0f / (float)n_rows;
  for (uint32_t d = 0; d < dim; ++d) mean[d] *= inv;
  return MRL_OK;
}

// ---------------------------------------------------------------------------
// seeded synthetic corpora (benchmark inputs; not part of the reference)
// counter-based: row r of a corpus depends only on (seed, r)
// ---------------------------------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Standard normal draws for (seed, stream, row): Box-Muller on 53-bit uniforms.
void gaussian_row(uint64_t seed, uint64_t stream, uint64_t row, uint32_t n, float* out) {
  uint64_t key = mix64(seed * 0x9E3779B97F4A7C15ull ^ mix64(stream + 0x632BE59BD9B4E019ull) ^ mix64(row));
  for (uint32_t i = 0; i < n; i += 2) {
    uint64_t h1 = mix64(key + 2ull * i + 1);
    uint64_t h2 = mix64(key + 2ull * i + 2);
    double u1 = ((double)(h1 >> 11) + 1.0) * (1.0 / 9007199254740993.0);  // (0, 1]
    double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);          // [0, 1)
    double rad = sqrt(-2.0 * log(u1));
    double ang = 6.283185307179586 * u2;
    out[i] = (float)(rad * cos(ang));
    if (i + 1 < n) out[i + 1] = (float)(rad * sin(ang));
  }
}

static void l2_normalize(float* v, uint32_t n) {
  float s = 0.0f;
  for (uint32_t i = 0; i < n; ++i) s += v[i] * v[i];
  float nrm = fmaxf(sqrtf(s), 1e-12f);
  for (uint32_t i = 0; i < n; ++i) v[i] /= nrm;
}

// x_d = (1+d)^-1/2 z_d + offset, L2-normalised
static void base_vector(uint64_t seed, uint64_t stream, uint64_t row, uint32_t dims, float offset, float* out) {
  gaussian_row(seed, stream, row, dims, out);
  for (uint32_t d = 0; d < dims; ++d) out[d] = out[d] * (1.0f / sqrtf((float)(d + 1))) + offset;
  l2_normalize(out, dims);
}

uint32_t synth_cluster(const SynthSpec& s, uint64_t row) {
  return s.n_centroids ? (uint32_t)(mix64(mix64(s.seed_assign) ^ (row * 0xD1B54A32D192ED03ull)) % s.n_centroids) : 0u;
}

void synth_doc(const SynthSpec& s, uint64_t row, float* out) {
  if (s.n_centroids == 0) {
    base_vector(s.seed, 1, row, s.dims, s.mean_offset, out);
    return;
  }
  const uint64_t c = synth_cluster(s, row);
  base_vector(s.seed_centroids, 2, c, s.dims, s.mean_offset, out);
  std::vector<float> noise(s.dims);
  gaussian_row(s.seed, 3, row, s.dims, noise.data());
  const float sig = s.noise_sigma / sqrtf((float)s.dims);
  for (uint32_t d = 0; d < s.dims; ++d) out[d] += sig * noise[d];
  l2_normalize(out, s.dims);
}

void synth_query(const SynthSpec& s, uint64_t seed_q, float noise_sigma, int fresh, uint64_t qi, float* out,
                 uint64_t* src_row) {
  if (fresh) {
    base_vector(seed_q, 4, qi, s.dims, s.mean_offset, out);
    if (src_row) *src_row = ~0ull;
    return;
  }
  const uint64_t row = mix64(mix64(seed_q) + qi * 0x9E3779B97F4A7C15ull) % s.n_docs;
  synth_doc(s, row, out);
  std::vector<float> noise(s.dims);
  gaussian_row(seed_q, 5, qi, s.dims, noise.data());
  const float sig = noise_sigma / sqrtf((float)s.dims);
  for (uint32_t d = 0; d < s.dims; ++d) out[d] += sig * noise[d];
  l2_normalize(out, s.dims);
  if (src_row) *src_row = row;
}

}  // namespace mrl
