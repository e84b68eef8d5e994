/*
 * mrl_oracle.c -- CPU restatement of the reference PaxBlock64 scan path.
 *
 * TEST INFRASTRUCTURE ONLY (see mrl_oracle.h).  Each function names the
 * reference lines it follows.  Floating-point expressions keep the
 * reference's operand order; the build uses -ffp-contract=off so no
 * multiply-add is fused, exactly as rustc emits separate fmul/fadd.
 */
#define _GNU_SOURCE
#include "mrl_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

_Static_assert(sizeof(ora_plan) == 1664 * 4, "ora_plan layout");

size_t ora_plan_size(void) { return sizeof(ora_plan); }

/* ------------------------------------------------------------------ */
/* little-endian field access                                          */
/* ------------------------------------------------------------------ */
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }
static void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static void wr32(uint8_t *p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
static void wr64(uint8_t *p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
static uint64_t plane_word(const uint8_t *block, int off, int d) { return rd64(block + off + 8 * d); }

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Rust f32::max / f32::min ignore a NaN operand, like C fmaxf / fminf. */
static float rmax(float a, float b) { return fmaxf(a, b); }
/* Rust f32::clamp (core::f32::clamp): NaN passes through. */
static float rclamp(float x, float lo, float hi) {
  if (x < lo) x = lo;
  if (x > hi) x = hi;
  return x;
}
/* Rust `f as u8`: saturating, NaN -> 0. */
static uint8_t f32_as_u8(float x) {
  if (!(x == x)) return 0;
  if (x <= 0.0f) return 0;
  if (x >= 255.0f) return 255;
  return (uint8_t)x;
}

/* ------------------------------------------------------------------ */
/* IEEE binary16 (half 2.7.1 f16::to_f32 / f16::from_f32, used by      */
/* src/block.rs:61-70,92-98)                                           */
/* ------------------------------------------------------------------ */
float ora_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if ((h & 0x7fffu) == 0) return bits_f32(sign);
  if (exp == 0x1f) {
    if (man == 0) return bits_f32(sign | 0x7f800000u);
    return bits_f32(sign | 0x7fc00000u | (man << 13)); /* NaN: quiet bit set */
  }
  if (exp == 0) { /* subnormal half -> normal float */
    int e = 0;
    while ((man & 0x400u) == 0) { man <<= 1; ++e; }
    man &= 0x3ffu;
    uint32_t fexp = (uint32_t)(127 - 15 + 1 - e);
    return bits_f32(sign | (fexp << 23) | (man << 13));
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t ora_f32_to_f16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13)); /* NaN stays NaN */
  }
  int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
  if (e <= 0) {
    /* subnormal half (or zero) */
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t hm = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (hm & 1u))) hm += 1;
    return (uint16_t)(sign | hm);
  }
  uint32_t hm = man >> 13;
  uint32_t rem = man & 0x1fffu;
  uint16_t out = (uint16_t)(sign | ((uint32_t)e << 10) | hm);
  if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) out += 1; /* carries into exp */
  return out;
}

void ora_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = ora_f16_to_f32(in[i]);
}
void ora_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = ora_f32_to_f16(in[i]);
}

/* src/block.rs:61-99 (VectorMeta accessors). */
static float meta_scale(const uint8_t *b, int v) { return ora_f16_to_f32(rd16(b + ORA_OFF_META + 7 * v)); }
static float meta_offset(const uint8_t *b, int v) { return ora_f16_to_f32(rd16(b + ORA_OFF_META + 7 * v + 2)); }
static float meta_tail(const uint8_t *b, int v) { return ora_f16_to_f32(rd16(b + ORA_OFF_META + 7 * v + 4)); }
static uint8_t meta_flags(const uint8_t *b, int v) { return b[ORA_OFF_META + 7 * v + 6]; }
static float meta_rho(const uint8_t *b, int v) { return (float)meta_flags(b, v) / 255.0f; }
static float meta_mid_norm(const uint8_t *b, int v) {
  float t = rmax(meta_tail(b, v), 0.0f);
  float r = rclamp(meta_rho(b, v), 0.0f, 1.0f);
  return sqrtf(rmax(1.0f - r * r, 0.0f)) * t;
}
static float meta_high_norm(const uint8_t *b, int v) { return meta_rho(b, v) * rmax(meta_tail(b, v), 0.0f); }

void ora_meta_decode(const uint8_t *block, int slot, float out[6]) {
  out[0] = meta_scale(block, slot);
  out[1] = meta_offset(block, slot);
  out[2] = meta_tail(block, slot);
  out[3] = meta_rho(block, slot);
  out[4] = meta_mid_norm(block, slot);
  out[5] = meta_high_norm(block, slot);
}

/* src/block.rs:102-108 */
uint8_t ora_pack_rho_flags(float high_tail_norm, float rest_norm) {
  if (rest_norm <= 1e-12f) return 0;
  float r = rclamp(high_tail_norm / rest_norm, 0.0f, 1.0f);
  return f32_as_u8(rclamp(roundf(r * 255.0f), 0.0f, 255.0f));
}

/* crc32fast 1.5.3: CRC-32/ISO-HDLC (reflected 0xEDB88320). */
uint32_t ora_crc32(const uint8_t *data, size_t n) {
  static uint32_t table[256];
  static int init = 0;
  if (!init) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      table[i] = c;
    }
    init = 1;
  }
  uint32_t crc = 0xffffffffu;
  for (size_t i = 0; i < n; ++i) crc = table[(crc ^ data[i]) & 0xffu] ^ (crc >> 8);
  return crc ^ 0xffffffffu;
}

/* src/block.rs:186-197 */
static void recompute_crc(uint8_t *block) {
  wr32(block + ORA_OFF_CRC, 0);
  wr32(block + ORA_OFF_CRC, ora_crc32(block, ORA_BLOCK_BYTES));
}
int ora_verify_crc(const uint8_t *block) {
  uint8_t copy[ORA_BLOCK_BYTES];
  memcpy(copy, block, ORA_BLOCK_BYTES);
  uint32_t expected = rd32(copy + ORA_OFF_CRC);
  wr32(copy + ORA_OFF_CRC, 0);
  return ora_crc32(copy, ORA_BLOCK_BYTES) == expected;
}

/* ------------------------------------------------------------------ */
/* src/rotate.rs                                                       */
/* ------------------------------------------------------------------ */
/* rotate.rs:13-33 */
void ora_fwht_inplace(float *a, int n) {
  int h = 1;
  while (h < n) {
    int step = h * 2;
    for (int i = 0; i < n; i += step) {
      for (int j = i; j < i + h; ++j) {
        float x = a[j];
        float y = a[j + h];
        a[j] = x + y;
        a[j + h] = x - y;
      }
    }
    h = step;
  }
  float scale = 1.0f / sqrtf((float)n);
  for (int i = 0; i < n; ++i) a[i] *= scale;
}

/* rotate.rs:36-42 */
void ora_rotate_mid_band(const float *mid128, float *out128) {
  memcpy(out128, mid128, 128 * sizeof(float));
  ora_fwht_inplace(out128, 128);
}

/* rotate.rs:46-49; std::f32::consts::PI rounds to the same float as (float)M_PI. */
float ora_rabitq_bit_scale(void) { return sqrtf(2.0f / (float)M_PI) / sqrtf((float)ORA_RABITQ_DIMS); }

/* rotate.rs:53-67 and eden.rs:75-88 share this SplitMix-style mix. */
static float splitmix_sign(uint64_t a, uint64_t i) {
  uint64_t x = (a * 0x9E3779B97F4A7C15ull + i) * 0xBF58476D1CE4E5B9ull;
  x ^= x >> 30;
  x = x * 0x94D049BB133111EBull;
  x ^= x >> 27;
  return (x & 1ull) == 0 ? 1.0f : -1.0f;
}
float ora_tail_rademacher(uint64_t block, uint64_t dim) { return splitmix_sign(block, dim); }

/* rotate.rs:73-93 */
void ora_fold_tail(const float *vec, int len, float *u) {
  for (int d = 0; d < 64; ++d) u[d] = 0.0f;
  if (len <= ORA_TAIL_START) return;
  int available = len - ORA_TAIL_START;
  int n_blocks = available / ORA_PREFIX_DIMS;
  if (n_blocks > ORA_TAIL_FOLD_BLOCKS) n_blocks = ORA_TAIL_FOLD_BLOCKS;
  if (n_blocks == 0) return;
  for (int b = 0; b < n_blocks; ++b) {
    int base = ORA_TAIL_START + b * ORA_PREFIX_DIMS;
    for (int d = 0; d < ORA_TAIL_FOLD_DIMS; ++d)
      u[d] += ora_tail_rademacher((uint64_t)b, (uint64_t)d) * vec[base + d];
  }
}

/* rotate.rs:96-100 */
void ora_rotate_tail_fold(const float *vec, int len, float *out64) {
  ora_fold_tail(vec, len, out64);
  ora_fwht_inplace(out64, 64);
}

/* rotate.rs:124-126 */
float ora_tail_fold_bit_scale(void) { return sqrtf(2.0f / (float)M_PI) / sqrtf((float)ORA_TAIL_FOLD_DIMS); }

/* ------------------------------------------------------------------ */
/* src/eden.rs                                                         */
/* ------------------------------------------------------------------ */
/* eden.rs:15-44 */
static const float EDEN_B1[2] = {-0.79788456f, 0.79788456f};
static const float EDEN_B2[4] = {-1.51041761f, -0.45278003f, 0.45278003f, 1.51041761f};
static const float EDEN_B3[8] = {-2.15194570f, -1.34390928f, -0.75600528f, -0.24509418f,
                                 0.24509418f,  0.75600528f,  1.34390928f,  2.15194570f};
static const float EDEN_B4[16] = {-2.73258958f, -2.06901724f, -1.61804640f, -1.25623121f,
                                  -0.94234046f, -0.65675912f, -0.38804830f, -0.12839503f,
                                  0.12839503f,  0.38804830f,  0.65675912f,  0.94234046f,
                                  1.25623121f,  1.61804640f,  2.06901724f,  2.73258958f};

/* eden.rs:47-55 */
int ora_lloyd_max_normal(int bits, const float **out) {
  switch (bits) {
    case 1: *out = EDEN_B1; return 2;
    case 2: *out = EDEN_B2; return 4;
    case 3: *out = EDEN_B3; return 8;
    case 4: *out = EDEN_B4; return 16;
    default: *out = NULL; return 0;
  }
}

/* eden.rs:58-71: slice::binary_search_by on a strictly increasing codebook
 * returns Ok(i) on an exact match, else Err(number of entries < z). */
int ora_nearest_centroid(const float *cb, int n, float z) {
  int cnt = 0;
  while (cnt < n && cb[cnt] < z) ++cnt;
  if (cnt < n && cb[cnt] == z) return cnt;
  if (cnt == 0) return 0;
  if (cnt >= n) return n - 1;
  if (fabsf(z - cb[cnt - 1]) <= fabsf(cb[cnt] - z)) return cnt - 1;
  return cnt;
}

/* eden.rs:75-88 */
float ora_rademacher_diag(uint64_t seed, uint64_t i) { return splitmix_sign(seed, i); }

/* eden.rs:91-98 */
void ora_structured_hadamard_inplace(float *v, int d, uint64_t seed) {
  for (int i = 0; i < d; ++i) v[i] *= ora_rademacher_diag(seed, (uint64_t)i);
  ora_fwht_inplace(v, d);
}

/* eden.rs:130-159 (fit_band): sequential sum over rows, then *= 1/n. */
int ora_eden_fit_band(const float *rows, uint64_t n_rows, uint64_t row_stride, uint32_t start,
                      uint32_t dim, float *mean) {
  if (n_rows == 0) return ORA_ERR_ARG;
  for (uint32_t d = 0; d < dim; ++d) mean[d] = 0.0f;
  for (uint64_t r = 0; r < n_rows; ++r) {
    const float *x = rows + r * row_stride;
    for (uint32_t d = 0; d < dim; ++d) mean[d] += x[start + d];
  }
  float inv = 1.0f / (float)n_rows;
  for (uint32_t d = 0; d < dim; ++d) mean[d] *= inv;
  return ORA_OK;
}

/* eden.rs:182-191 (observe_prefix). */
void ora_eden_observe(float *mean, uint32_t dim, uint64_t *n_observed, const float *x) {
  uint64_t n = *n_observed + 1;
  float inv = 1.0f / (float)n;
  for (uint32_t d = 0; d < dim; ++d) mean[d] += (x[d] - mean[d]) * inv;
  *n_observed = n;
}

/* eden.rs:225-269 */
int ora_eden_encode_slice(const ora_eden_fit *fit, const float *x, uint8_t *levels,
                          float *out_centered_norm, float *out_scale_s) {
  int d = (int)fit->dim;
  const float *cb;
  int ncb = ora_lloyd_max_normal((int)fit->bits, &cb);
  if (ncb == 0 || d <= 0 || d > 1024) return ORA_ERR_ARG;
  float sqrt_d = sqrtf((float)d);
  float inv_sqrt_d = 1.0f / sqrt_d;
  float centered[1024];
  float norm_sq = 0.0f;
  for (int i = 0; i < d; ++i) {
    float v = x[i] - fit->mean[i];
    centered[i] = v;
    norm_sq += v * v;
  }
  float centered_norm = rmax(sqrtf(norm_sq), 1e-12f);
  float inv_norm = 1.0f / centered_norm;
  for (int i = 0; i < d; ++i) centered[i] *= inv_norm;
  ora_structured_hadamard_inplace(centered, d, fit->seed);
  float ip = 0.0f;
  for (int i = 0; i < d; ++i) {
    int level = ora_nearest_centroid(cb, ncb, centered[i] * sqrt_d);
    levels[i] = (uint8_t)level;
    float cw = cb[level] * inv_sqrt_d;
    ip += centered[i] * cw;
  }
  float scale_s = fabsf(ip) > 1e-12f ? 1.0f / ip : 0.0f;
  *out_centered_norm = centered_norm;
  *out_scale_s = scale_s;
  return ORA_OK;
}

/* eden.rs:275-281 */
void ora_eden_rotate_query(const ora_eden_fit *fit, const float *q, float *out) {
  memcpy(out, q, fit->dim * sizeof(float));
  ora_structured_hadamard_inplace(out, (int)fit->dim, fit->seed);
}

/* eden.rs:289-302 */
float ora_eden_score_ip(const ora_eden_fit *fit, const float *q, const float *q_rot,
                        const uint8_t *levels, float alpha) {
  int d = (int)fit->dim;
  const float *cb;
  ora_lloyd_max_normal((int)fit->bits, &cb);
  float inv_sqrt_d = 1.0f / sqrtf((float)d);
  float dot_cw = 0.0f;
  for (int i = 0; i < d; ++i) dot_cw += q_rot[i] * cb[levels[i]] * inv_sqrt_d;
  float mean_ip = 0.0f;
  for (int i = 0; i < d; ++i) mean_ip += q[i] * fit->mean[i];
  return mean_ip + alpha * dot_cw;
}

/* ------------------------------------------------------------------ */
/* src/quantize.rs (encoder; the scan tests need blocks)               */
/* ------------------------------------------------------------------ */
/* quantize.rs:180-197 */
static void residual_norms(const float *vec, int dims, float *rest, uint8_t *flags) {
  float mid_sq = 0.0f;
  for (int i = 0; i < ORA_RABITQ_DIMS; ++i) {
    float x = vec[ORA_PREFIX_DIMS + i];
    mid_sq += x * x;
  }
  float high_sq = 0.0f;
  for (int i = ORA_TAIL_START; i < dims; ++i) high_sq += vec[i] * vec[i];
  float rest_norm = sqrtf(mid_sq + high_sq);
  float high_norm = sqrtf(high_sq);
  *rest = rest_norm;
  *flags = ora_pack_rho_flags(high_norm, rest_norm);
}

/* quantize.rs:199-213 */
static void mid_and_fold_bits(const float *vec, int dims, uint8_t *rabitq, uint8_t *fold) {
  float rotated[128];
  ora_rotate_mid_band(vec + ORA_PREFIX_DIMS, rotated);
  for (int i = 0; i < 128; ++i) rabitq[i] = rotated[i] >= 0.0f ? 1 : 0;
  float folded[64];
  ora_rotate_tail_fold(vec, dims, folded);
  for (int i = 0; i < 64; ++i) fold[i] = folded[i] >= 0.0f ? 1 : 0;
}

static void write_meta(uint8_t *block, int slot, float scale, float offset, float tail, uint8_t flags) {
  uint8_t *m = block + ORA_OFF_META + 7 * slot;
  wr16(m, ora_f32_to_f16(scale));
  wr16(m + 2, ora_f32_to_f16(offset));
  wr16(m + 4, ora_f32_to_f16(tail));
  m[6] = flags;
}

static void set_bit(uint8_t *block, int off, int d, int slot) {
  uint64_t w = plane_word(block, off, d) | (1ull << slot);
  wr64(block + off + 8 * d, w);
}

/* quantize.rs:297-333 */
static void write_planes(uint8_t *block, int slot, const uint8_t *bits4, const uint8_t *rabitq,
                         const uint8_t *fold) {
  for (int d = 0; d < 64; ++d) {
    uint8_t q = bits4[d];
    if (q & 8) set_bit(block, ORA_OFF_S0, d, slot);
    if (q & 4) set_bit(block, ORA_OFF_S2, d, slot);
    if (q & 2) set_bit(block, ORA_OFF_S3, d, slot);
    if (q & 1) set_bit(block, ORA_OFF_S5, d, slot);
  }
  for (int d = 0; d < 128; ++d)
    if (rabitq[d]) set_bit(block, ORA_OFF_S1, d, slot);
  for (int d = 0; d < 64; ++d)
    if (fold[d]) set_bit(block, ORA_OFF_S4, d, slot);
}

/* quantize.rs:36-96 with quantize_vector (220-246) and
 * quantize_vector_eden_dual (265-295). */
int ora_encode_block(const float *vecs, int n, int dims, const uint32_t *ts, const uint32_t *src,
                     const ora_eden_fit *eden, const ora_eden_fit *eden_mid, uint8_t *block) {
  if (n <= 0 || n > 64 || dims < ORA_PREFIX_DIMS + ORA_RABITQ_DIMS) return ORA_ERR_ARG;
  if (eden && (eden->dim != 64 || eden->bits != 4)) return ORA_ERR_ARG;
  if (eden_mid && (!eden || eden_mid->dim != 128 || eden_mid->bits != 1)) return ORA_ERR_ARG;
  memset(block, 0, ORA_BLOCK_BYTES);
  uint32_t min_ts = 0xffffffffu, max_ts = 0, source_mask = 0;
  for (int i = 0; i < n; ++i) {
    const float *vec = vecs + (size_t)i * dims;
    if (ts[i] < min_ts) min_ts = ts[i];
    if (ts[i] > max_ts) max_ts = ts[i];
    source_mask |= src[i];
    uint8_t bits4[64], rabitq[128], fold[64];
    float scale, offset;
    if (eden) {
      float cn, ss;
      ora_eden_encode_slice(eden, vec, bits4, &cn, &ss);
      scale = cn * ss;
      float mid_alpha = 0.0f;
      if (eden_mid) {
        float mcn, mss;
        ora_eden_encode_slice(eden_mid, vec + ORA_PREFIX_DIMS, rabitq, &mcn, &mss);
        mid_alpha = mcn * mss;
      } else {
        uint8_t tmpfold[64];
        mid_and_fold_bits(vec, dims, rabitq, tmpfold);
      }
      uint8_t tmprq[128];
      mid_and_fold_bits(vec, dims, tmprq, fold);
      offset = mid_alpha;
    } else {
      float min_v = INFINITY, max_v = -INFINITY;
      for (int d = 0; d < 64; ++d) min_v = fminf(min_v, vec[d]);
      for (int d = 0; d < 64; ++d) max_v = fmaxf(max_v, vec[d]);
      float range = rmax(max_v - min_v, 1e-8f);
      scale = range / 15.0f;
      offset = min_v;
      for (int d = 0; d < 64; ++d)
        bits4[d] = f32_as_u8(rclamp(roundf((vec[d] - offset) / scale), 0.0f, 15.0f));
      mid_and_fold_bits(vec, dims, rabitq, fold);
    }
    float rest;
    uint8_t flags;
    residual_norms(vec, dims, &rest, &flags);
    write_meta(block, i, scale, offset, rest, flags);
    write_planes(block, i, bits4, rabitq, fold);
  }
  uint64_t tomb = 0;
  for (int i = n; i < 64; ++i) {
    tomb |= 1ull << i;
    write_meta(block, i, 0.0f, 0.0f, 0.0f, 0);
  }
  wr32(block + ORA_OFF_MIN_TS, min_ts);
  wr32(block + ORA_OFF_MAX_TS, max_ts);
  wr32(block + ORA_OFF_SOURCE_MASK, source_mask);
  wr64(block + ORA_OFF_TOMBSTONE, tomb);
  recompute_crc(block);
  return ORA_OK;
}

/* quantize.rs:347-367 */
void ora_extract_bits4(const uint8_t *block, int slot, uint8_t *out) {
  uint64_t m = 1ull << slot;
  for (int d = 0; d < 64; ++d) {
    uint8_t q = 0;
    if (plane_word(block, ORA_OFF_S0, d) & m) q |= 8;
    if (plane_word(block, ORA_OFF_S2, d) & m) q |= 4;
    if (plane_word(block, ORA_OFF_S3, d) & m) q |= 2;
    if (plane_word(block, ORA_OFF_S5, d) & m) q |= 1;
    out[d] = q;
  }
}

/* ------------------------------------------------------------------ */
/* QueryPlan::from_query_codec (src/scan.rs:105-266)                   */
/* ------------------------------------------------------------------ */
int ora_plan_build(const float *query, int dims, int prefix_codec, int mid_codec,
                   const ora_eden_fit *eden, const ora_eden_fit *eden_mid, ora_plan *p) {
  if (dims < ORA_PREFIX_DIMS + ORA_RABITQ_DIMS) return ORA_ERR_ARG; /* scan.rs:114 */
  if (prefix_codec == ORA_PREFIX_EDEN_PROD) {                       /* scan.rs:115-119 */
    if (!eden || eden->dim != 64 || eden->bits != 4) return ORA_ERR_ARG;
  }
  if (mid_codec == ORA_MID_EDEN_B1) {                               /* scan.rs:120-124 */
    if (!eden_mid || eden_mid->dim != 128 || eden_mid->bits != 1) return ORA_ERR_ARG;
  }
  memset(p, 0, sizeof(*p));
  p->dims = (uint32_t)dims;
  p->prefix_codec = prefix_codec;
  p->mid_codec = mid_codec;

  /* 126-140 */
  memcpy(p->prefix, query, 64 * sizeof(float));
  float prefix_l1 = 0.0f, prefix_sum = 0.0f;
  for (int d = 0; d < 64; ++d) {
    float q = p->prefix[d];
    prefix_l1 += fabsf(q);
    prefix_sum += q;
    p->bit_weights[d][0] = q * 1.0f;
    p->bit_weights[d][1] = q * 2.0f;
    p->bit_weights[d][2] = q * 4.0f;
    p->bit_weights[d][3] = q * 8.0f;
  }

  /* 142-157 */
  float eden_mean_ip = 0.0f;
  float eden_inv_sqrt_d = 1.0f / sqrtf(64.0f);
  if (eden) {
    ora_eden_rotate_query(eden, query, p->eden_q_rot);
    for (int d = 0; d < 64; ++d) eden_mean_ip += query[d] * eden->mean[d];
    eden_inv_sqrt_d = 1.0f / sqrtf((float)eden->dim);
    const float *cb;
    int n = ora_lloyd_max_normal((int)eden->bits, &cb);
    for (int i = 0; i < n; ++i) p->eden_codebook[i] = cb[i];
  }
  p->eden_mean_ip = eden_mean_ip;
  p->eden_inv_sqrt_d = eden_inv_sqrt_d;

  /* 159-174 */
  float eden_mid_mean_ip = 0.0f;
  float eden_mid_inv_sqrt_d = 1.0f / sqrtf(128.0f);
  if (eden_mid) {
    const float *mid_raw = query + 64;
    ora_eden_rotate_query(eden_mid, mid_raw, p->eden_mid_q_rot);
    for (int d = 0; d < 128; ++d) eden_mid_mean_ip += mid_raw[d] * eden_mid->mean[d];
    eden_mid_inv_sqrt_d = 1.0f / sqrtf((float)eden_mid->dim);
    p->eden_mid_codebook[0] = EDEN_B1[0];
    p->eden_mid_codebook[1] = EDEN_B1[1];
  }
  p->eden_mid_mean_ip = eden_mid_mean_ip;
  p->eden_mid_inv_sqrt_d = eden_mid_inv_sqrt_d;

  /* 176-186 */
  ora_rotate_mid_band(query + 64, p->rabitq_q);
  float rabitq_scale = ora_rabitq_bit_scale();
  p->rabitq_scale = rabitq_scale;
  float rabitq_base = 0.0f;
  for (int d = 0; d < 128; ++d) {
    float pos = p->rabitq_q[d] * rabitq_scale;
    rabitq_base -= pos;
    p->rabitq_weights2[d] = 2.0f * pos;
  }
  p->rabitq_base = rabitq_base;

  /* 188-201 */
  for (int g = 0; g < 32; ++g) {
    float p0 = p->rabitq_q[4 * g] * rabitq_scale;
    float p1 = p->rabitq_q[4 * g + 1] * rabitq_scale;
    float p2 = p->rabitq_q[4 * g + 2] * rabitq_scale;
    float p3 = p->rabitq_q[4 * g + 3] * rabitq_scale;
    for (int mask = 0; mask < 16; ++mask) {
      float s0 = (mask & 1) ? p0 : -p0;
      float s1 = (mask & 2) ? p1 : -p1;
      float s2 = (mask & 4) ? p2 : -p2;
      float s3 = (mask & 8) ? p3 : -p3;
      p->rabitq_lut[g][mask] = s0 + s1 + s2 + s3;
    }
  }

  /* 203-214 */
  float q_tail_sq = 0.0f;
  for (int i = ORA_TAIL_START; i < dims; ++i) q_tail_sq += query[i] * query[i];
  float q_tail_norm = sqrtf(q_tail_sq);
  float q_mid_sq = 0.0f;
  for (int i = 0; i < 128; ++i) {
    float x = query[64 + i];
    q_mid_sq += x * x; /* powi(2) lowers to x*x */
  }
  float q_mid_norm = sqrtf(q_mid_sq);
  float q_after_prefix = sqrtf(q_mid_sq + q_tail_sq);

  /* 216-233 */
  int has_tail_fold = dims > ORA_TAIL_START;
  if (has_tail_fold) ora_rotate_tail_fold(query, dims, p->tail_fold_q);
  float tail_fold_scale = ora_tail_fold_bit_scale();
  float tail_fold_base = 0.0f, s4_abs_budget = 0.0f;
  if (has_tail_fold) {
    for (int d = 0; d < 64; ++d) {
      float pos = p->tail_fold_q[d] * tail_fold_scale;
      tail_fold_base -= pos;
      p->tail_fold_weights2[d] = 2.0f * pos;
      s4_abs_budget += fabsf(pos);
    }
  }

  p->has_tail_fold = (uint32_t)has_tail_fold;
  p->tail_fold_base = tail_fold_base;
  p->q_tail_norm = q_tail_norm;
  p->q_mid_norm = q_mid_norm;
  p->q_after_prefix = q_after_prefix;
  p->q_after_s1 = q_tail_norm;
  p->s4_abs_budget = s4_abs_budget;
  p->prefix_l1 = prefix_l1;
  p->prefix_sum = prefix_sum;

  /* Values the stages recompute from the plan on every block. */
  for (int d = 0; d < 64; ++d) /* scan.rs:457-461 */
    p->prefix_weight[d] = prefix_codec == ORA_PREFIX_EDEN_PROD
                              ? p->eden_q_rot[d] * p->eden_inv_sqrt_d
                              : p->prefix[d];
  { /* scan.rs:523-532 */
    float base = 0.0f;
    float c0 = p->eden_mid_codebook[0], c1 = p->eden_mid_codebook[1];
    float inv = p->eden_mid_inv_sqrt_d;
    for (int d = 0; d < 128; ++d) {
      float q = p->eden_mid_q_rot[d] * inv;
      base += c0 * q;
      p->eden_mid_deltas[d] = (c1 - c0) * q;
    }
    p->eden_mid_base = base;
  }
  return ORA_OK;
}

/* ------------------------------------------------------------------ */
/* Shortlist (src/scan.rs:304-399)                                     */
/* ------------------------------------------------------------------ */
typedef struct hit {
  uint64_t id; /* VectorId::as_u64: block << 16 | slot (block.rs:213-215) */
  float score;
} hit;

typedef struct shortlist {
  uint32_t capacity;
  uint32_t len;
  hit *heap;
  uint32_t min_idx;
  float min_score;
  float floor_tau;
} shortlist;

static void sl_init(shortlist *s, uint32_t capacity, float floor_tau) {
  s->capacity = capacity < 1 ? 1 : capacity;
  s->len = 0;
  s->heap = (hit *)malloc(sizeof(hit) * s->capacity);
  s->min_idx = 0;
  s->min_score = INFINITY;
  s->floor_tau = floor_tau;
}
static void sl_free(shortlist *s) { free(s->heap); s->heap = NULL; }

/* scan.rs:342-348 */
static float sl_threshold(const shortlist *s) {
  if (s->len < s->capacity) return s->floor_tau;
  return rmax(s->min_score, s->floor_tau);
}

/* scan.rs:371-382 */
static void sl_recompute_min(shortlist *s) {
  uint32_t min_idx = 0;
  float min_score = INFINITY;
  for (uint32_t i = 0; i < s->len; ++i) {
    if (s->heap[i].score < min_score) {
      min_score = s->heap[i].score;
      min_idx = i;
    }
  }
  s->min_idx = min_idx;
  s->min_score = min_score;
}

/* scan.rs:351-368 */
static void sl_push(shortlist *s, hit h) {
  if (h.score < s->floor_tau) return;
  if (s->len < s->capacity) {
    uint32_t idx = s->len;
    if (h.score < s->min_score) {
      s->min_score = h.score;
      s->min_idx = idx;
    }
    s->heap[s->len++] = h;
    return;
  }
  if (h.score > s->min_score) {
    s->heap[s->min_idx] = h;
    sl_recompute_min(s);
  }
}

/* scan.rs:384-388 */
static void sl_merge(shortlist *dst, const shortlist *src) {
  for (uint32_t i = 0; i < src->len; ++i) sl_push(dst, src->heap[i]);
}

/* scan.rs:390-394: stable sort, descending; a NaN makes partial_cmp panic. */
static int sl_into_sorted(shortlist *s, uint64_t *ids, float *scores) {
  for (uint32_t i = 0; i < s->len; ++i)
    if (s->heap[i].score != s->heap[i].score) return -ORA_ERR_NAN;
  /* stable insertion-merge sort */
  uint32_t n = s->len;
  hit *tmp = (hit *)malloc(sizeof(hit) * (n ? n : 1));
  for (uint32_t width = 1; width < n; width *= 2) {
    for (uint32_t lo = 0; lo < n; lo += 2 * width) {
      uint32_t mid = lo + width < n ? lo + width : n;
      uint32_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      uint32_t i = lo, j = mid, k = lo;
      while (i < mid && j < hi) {
        /* take from the right run only when strictly greater (keeps order of equals) */
        if (s->heap[j].score > s->heap[i].score) tmp[k++] = s->heap[j++];
        else tmp[k++] = s->heap[i++];
      }
      while (i < mid) tmp[k++] = s->heap[i++];
      while (j < hi) tmp[k++] = s->heap[j++];
    }
    memcpy(s->heap, tmp, sizeof(hit) * n);
  }
  free(tmp);
  for (uint32_t i = 0; i < n; ++i) {
    ids[i] = s->heap[i].id;
    scores[i] = s->heap[i].score;
  }
  return (int)n;
}

/* ------------------------------------------------------------------ */
/* Stages (src/scan.rs:418-691)                                        */
/* ------------------------------------------------------------------ */
typedef struct block_state {
  float scores[64];
  uint64_t survivors;
  float mid_n[64];
  float high_n[64];
  uint64_t active;
} block_state;

typedef struct scan_ctx {
  const uint8_t *block;
  const ora_plan *plan;
  const ora_scan_config *cfg;
  float tau;
  float alpha;
} scan_ctx;

static int includes_prefix_4bit(int depth) { return depth != ORA_STRATA_L0_ONLY; }
static int includes_rabitq(int depth) { return depth == ORA_STRATA_L1_RABITQ || depth == ORA_STRATA_FULL64B; }
static int includes_tail_fold(int depth) { return depth == ORA_STRATA_FULL64B; }

static int ctz64(uint64_t x) { return __builtin_ctzll(x); }
static int popc64(uint64_t x) { return __builtin_popcountll(x); }

/* scan.rs:453-517.  The SWAR byte lanes only regroup vectors; each vector's
 * code_dot is still summed over d = 0..63 in order, skipping weight == 0. */
static void stage_prefix_ip_and_cs_split(const scan_ctx *c, block_state *st) {
  const ora_plan *p = c->plan;
  int use_eden = p->prefix_codec == ORA_PREFIX_EDEN_PROD;
  float acc[64];
  for (int v = 0; v < 64; ++v) acc[v] = 0.0f;
  for (int d = 0; d < 64; ++d) {
    float weight = use_eden ? p->eden_q_rot[d] * p->eden_inv_sqrt_d : p->prefix[d];
    if (weight == 0.0f) continue;
    uint64_t b0 = plane_word(c->block, ORA_OFF_S5, d);
    uint64_t b1 = plane_word(c->block, ORA_OFF_S3, d);
    uint64_t b2 = plane_word(c->block, ORA_OFF_S2, d);
    uint64_t b3 = plane_word(c->block, ORA_OFF_S0, d);
    for (int v = 0; v < 64; ++v) {
      unsigned level = (unsigned)(((b0 >> v) & 1) | (((b1 >> v) & 1) << 1) | (((b2 >> v) & 1) << 2) |
                                  (((b3 >> v) & 1) << 3));
      if (use_eden) acc[v] += p->eden_codebook[level] * weight;
      else acc[v] += (float)level * weight;
    }
  }
  uint64_t survivors = 0;
  for (int v = 0; v < 64; ++v) {
    uint64_t bit = 1ull << v;
    if ((st->active & bit) == 0) continue;
    st->mid_n[v] = rmax(meta_mid_norm(c->block, v), 1e-6f);
    st->high_n[v] = rmax(meta_high_norm(c->block, v), 0.0f);
    float scale = meta_scale(c->block, v);
    float code_dot_v = acc[v];
    float prefix_ip;
    if (use_eden) {
      prefix_ip = p->eden_mean_ip + scale * code_dot_v;
    } else {
      float offset = meta_offset(c->block, v);
      prefix_ip = code_dot_v * scale + offset * p->prefix_sum;
    }
    st->scores[v] = prefix_ip;
    float ub = prefix_ip + c->alpha * (p->q_mid_norm * st->mid_n[v] + p->q_tail_norm * st->high_n[v]);
    if (ub >= c->tau) survivors |= bit;
  }
  st->survivors = survivors;
}

/* scan.rs:520-569 */
static void stage_rabitq_ip(const scan_ctx *c, block_state *st) {
  const ora_plan *p = c->plan;
  if (p->mid_codec == ORA_MID_EDEN_B1) {
    float base = 0.0f;
    float deltas[128];
    float c0 = p->eden_mid_codebook[0], c1 = p->eden_mid_codebook[1];
    float inv = p->eden_mid_inv_sqrt_d;
    for (int d = 0; d < 128; ++d) {
      float q = p->eden_mid_q_rot[d] * inv;
      base += c0 * q;
      deltas[d] = (c1 - c0) * q;
    }
    float cw_dot[64];
    for (int v = 0; v < 64; ++v) cw_dot[v] = base;
    for (int d = 0; d < 128; ++d) {
      uint64_t bits = plane_word(c->block, ORA_OFF_S1, d) & st->survivors;
      while (bits) {
        int v = ctz64(bits);
        cw_dot[v] += deltas[d];
        bits &= bits - 1;
      }
    }
    uint64_t s_bits = st->survivors;
    while (s_bits) {
      int v = ctz64(s_bits);
      float mid_alpha = meta_offset(c->block, v);
      st->scores[v] += p->eden_mid_mean_ip + mid_alpha * cw_dot[v];
      s_bits &= s_bits - 1;
    }
    return;
  }
  float s1_dot[64];
  for (int v = 0; v < 64; ++v) s1_dot[v] = p->rabitq_base;
  for (int d = 0; d < 128; ++d) {
    uint64_t bits = plane_word(c->block, ORA_OFF_S1, d) & st->survivors;
    float w = p->rabitq_weights2[d];
    while (bits) {
      int v = ctz64(bits);
      s1_dot[v] += w;
      bits &= bits - 1;
    }
  }
  uint64_t s_bits = st->survivors;
  while (s_bits) {
    int v = ctz64(s_bits);
    st->scores[v] += s1_dot[v] * st->mid_n[v];
    s_bits &= s_bits - 1;
  }
}

/* scan.rs:572-584 */
static void stage_cs_tail(const scan_ctx *c, block_state *st) {
  uint64_t survivors2 = 0, check = st->survivors;
  while (check) {
    int v = ctz64(check);
    float ub = st->scores[v] + c->alpha * c->plan->q_after_s1 * st->high_n[v];
    if (ub >= c->tau) survivors2 |= 1ull << v;
    check &= check - 1;
  }
  st->survivors = survivors2;
}

/* scan.rs:587-607 */
static void stage_s4_abs_budget(const scan_ctx *c, block_state *st) {
  if (!includes_tail_fold(c->cfg->strata_depth)) return;
  if (!(c->plan->has_tail_fold && c->plan->s4_abs_budget > 0.0f)) return;
  float w_s4 = c->cfg->stratum4_weight;
  uint64_t survivors3 = 0, bits = st->survivors;
  while (bits) {
    int v = ctz64(bits);
    float ub = st->scores[v] + c->alpha * rmax(st->high_n[v], 1e-6f) * w_s4 * c->plan->s4_abs_budget;
    if (ub >= c->tau) survivors3 |= 1ull << v;
    bits &= bits - 1;
  }
  st->survivors = survivors3;
}

/* scan.rs:610-634 */
static void stage_tail_fold_ip(const scan_ctx *c, block_state *st) {
  if (!includes_tail_fold(c->cfg->strata_depth)) return;
  if (!c->plan->has_tail_fold) return;
  float w_s4 = c->cfg->stratum4_weight;
  float s4_dot[64];
  for (int v = 0; v < 64; ++v) s4_dot[v] = c->plan->tail_fold_base;
  for (int d = 0; d < 64; ++d) {
    uint64_t bits = plane_word(c->block, ORA_OFF_S4, d) & st->survivors;
    float w = c->plan->tail_fold_weights2[d];
    while (bits) {
      int v = ctz64(bits);
      s4_dot[v] += w;
      bits &= bits - 1;
    }
  }
  uint64_t s_bits = st->survivors;
  while (s_bits) {
    int v = ctz64(s_bits);
    st->scores[v] += s4_dot[v] * rmax(st->high_n[v], 1e-6f) * w_s4;
    s_bits &= s_bits - 1;
  }
}

/* scan.rs:654-691; masks[1..3] record survivors after each gate. */
static void run_default_scan_kernel(const scan_ctx *c, block_state *st, ora_scan_stats *stats,
                                    uint64_t *masks) {
  int depth = c->cfg->strata_depth;
  stage_prefix_ip_and_cs_split(c, st);
  if (masks) masks[1] = masks[2] = masks[3] = st->survivors;
  if (stats) stats->after_prefix += (uint64_t)popc64(st->survivors);
  if (st->survivors == 0) return;
  if (includes_rabitq(depth)) {
    stage_rabitq_ip(c, st);
    stage_cs_tail(c, st);
  }
  if (masks) masks[2] = masks[3] = st->survivors;
  if (stats) stats->after_s1 += (uint64_t)popc64(st->survivors);
  if (st->survivors == 0) return;
  if (includes_tail_fold(depth)) {
    stage_s4_abs_budget(c, st);
    if (masks) masks[3] = st->survivors;
    if (stats) stats->after_s4_budget += (uint64_t)popc64(st->survivors);
    if (st->survivors == 0) return;
    stage_tail_fold_ip(c, st);
  } else if (stats) {
    stats->after_s4_budget += (uint64_t)popc64(st->survivors);
  }
}

/* scan.rs:709-799 with an explicit tau instead of shortlist.threshold().
 * Returns the pushed survivor mask; *skipped set when the block is not scored. */
static uint64_t scan_block_core(const uint8_t *block, const ora_plan *plan, const ora_scan_config *cfg,
                                float tau, int has_lo, uint32_t lo, int has_hi, uint32_t hi,
                                ora_scan_stats *stats, block_state *st, uint64_t *masks, int *skipped) {
  *skipped = 1;
  if (cfg->temporal_filter_enable) {
    if (has_lo && rd32(block + ORA_OFF_MAX_TS) < lo) return 0;
    if (has_hi && rd32(block + ORA_OFF_MIN_TS) > hi) return 0;
  }
  float alpha = cfg->cs_tolerance;
  uint64_t active = ~rd64(block + ORA_OFF_TOMBSTONE);
  if (active == 0) return 0;
  *skipped = 0;
  if (stats) {
    stats->blocks += 1;
    stats->active_vecs += (uint64_t)popc64(active);
  }
  memset(st, 0, sizeof(*st));
  st->active = active;
  if (masks) masks[0] = active;
  scan_ctx c = {block, plan, cfg, tau, alpha};

  if (!includes_prefix_4bit(cfg->strata_depth)) { /* 753-790 */
    float code_dot[64];
    for (int v = 0; v < 64; ++v) code_dot[v] = 0.0f;
    for (int d = 0; d < 64; ++d) { /* accum_plane, 402-413 */
      float weight = plan->bit_weights[d][3];
      if (weight == 0.0f) continue;
      uint64_t bits = plane_word(block, ORA_OFF_S0, d) & active;
      while (bits) {
        int v = ctz64(bits);
        code_dot[v] += weight;
        bits &= bits - 1;
      }
    }
    uint64_t survivors = 0;
    for (int v = 0; v < 64; ++v) {
      uint64_t bit = 1ull << v;
      if ((active & bit) == 0) continue;
      float scale = meta_scale(block, v);
      float offset = meta_offset(block, v);
      float prefix_ip = code_dot[v] * scale + offset * plan->prefix_sum;
      st->scores[v] = prefix_ip;
      float x_rest = rmax(meta_tail(block, v), 0.0f);
      float ub = prefix_ip + alpha * plan->q_after_prefix * x_rest;
      if (ub >= tau) survivors |= bit;
    }
    if (masks) masks[1] = masks[2] = masks[3] = masks[4] = survivors;
    if (survivors && stats) {
      uint64_t n = (uint64_t)popc64(survivors);
      stats->after_prefix += n;
      stats->after_s1 += n;
      stats->after_s4_budget += n;
      stats->pushed += n;
    }
    return survivors;
  }
  run_default_scan_kernel(&c, st, stats, masks);
  if (masks) masks[4] = st->survivors;
  if (st->survivors && stats) stats->pushed += (uint64_t)popc64(st->survivors);
  return st->survivors;
}

int ora_block_stages(const uint8_t *block, const ora_plan *plan, const ora_scan_config *cfg, float tau,
                     int has_lo, uint32_t lo, int has_hi, uint32_t hi, uint64_t masks[5],
                     float prefix_ip[64], float score[64]) {
  block_state st;
  int skipped;
  masks[0] = masks[1] = masks[2] = masks[3] = masks[4] = 0;
  memset(&st, 0, sizeof(st));
  /* stage 1 alone gives prefix_ip for every active slot */
  scan_block_core(block, plan, cfg, -INFINITY, has_lo, lo, has_hi, hi, NULL, &st, NULL, &skipped);
  if (skipped) {
    for (int v = 0; v < 64; ++v) prefix_ip[v] = score[v] = 0.0f;
    return 0;
  }
  if (includes_prefix_4bit(cfg->strata_depth)) {
    scan_ctx c = {block, plan, cfg, -INFINITY, cfg->cs_tolerance};
    block_state s1;
    memset(&s1, 0, sizeof(s1));
    s1.active = st.active;
    stage_prefix_ip_and_cs_split(&c, &s1);
    for (int v = 0; v < 64; ++v) prefix_ip[v] = s1.scores[v];
  } else {
    for (int v = 0; v < 64; ++v) prefix_ip[v] = st.scores[v];
  }
  scan_block_core(block, plan, cfg, tau, has_lo, lo, has_hi, hi, NULL, &st, masks, &skipped);
  for (int v = 0; v < 64; ++v) score[v] = st.scores[v];
  return 1;
}

/* scan.rs:694-706 + 636-651: scan one block into a shortlist. */
static void scan_block_into(const uint8_t *block, uint32_t block_idx, const ora_plan *plan,
                            const ora_scan_config *cfg, shortlist *sl, int has_lo, uint32_t lo,
                            int has_hi, uint32_t hi, ora_scan_stats *stats) {
  block_state st;
  int skipped;
  uint64_t surv = scan_block_core(block, plan, cfg, sl_threshold(sl), has_lo, lo, has_hi, hi, stats,
                                  &st, NULL, &skipped);
  while (surv) { /* finish_push */
    int v = ctz64(surv);
    hit h = {((uint64_t)block_idx << 16) | (uint64_t)v, st.scores[v]};
    sl_push(sl, h);
    surv &= surv - 1;
  }
}

typedef struct shard_job {
  const uint8_t *blocks;
  uint64_t first;
  uint64_t count;
  const ora_plan *plan;
  const ora_scan_config *cfg;
  int has_lo, has_hi;
  uint32_t lo, hi;
  float floor_tau;
  shortlist local;
} shard_job;

typedef struct shard_pool {
  shard_job *jobs;
  uint64_t n_jobs;
  uint64_t next;
  pthread_mutex_t mu;
} shard_pool;

static void *shard_worker(void *arg) {
  shard_pool *pool = (shard_pool *)arg;
  for (;;) {
    pthread_mutex_lock(&pool->mu);
    uint64_t j = pool->next++;
    pthread_mutex_unlock(&pool->mu);
    if (j >= pool->n_jobs) break;
    shard_job *job = &pool->jobs[j];
    for (uint64_t k = 0; k < job->count; ++k) {
      uint64_t bi = job->first + k;
      scan_block_into(job->blocks + bi * ORA_BLOCK_BYTES, (uint32_t)bi, job->plan, job->cfg, &job->local,
                      job->has_lo, job->lo, job->has_hi, job->hi, NULL);
    }
  }
  return NULL;
}

/* scan.rs:813-886 */
int64_t ora_scan_blocks(const uint8_t *blocks, uint64_t n_blocks, const ora_plan *plan,
                        const ora_scan_config *cfg, int has_lo, uint32_t lo, int has_hi, uint32_t hi,
                        uint64_t *out_ids, float *out_scores, ora_scan_stats *stats) {
  if (stats) memset(stats, 0, sizeof(*stats));
  if (n_blocks == 0) return 0;
  shortlist sl;
  sl_init(&sl, cfg->shortlist_cand, -INFINITY);
  const uint64_t PAR_THRESHOLD = 64;
  int threads = cfg->n_threads > 0 ? cfg->n_threads : 1;
  if (cfg->numa_sharding && n_blocks >= PAR_THRESHOLD && stats == NULL) {
    uint64_t warmup = (uint64_t)cfg->shortlist_cand / 64 + 1;
    if (warmup > 32) warmup = 32;
    if (warmup > n_blocks) warmup = n_blocks;
    for (uint64_t i = 0; i < warmup; ++i)
      scan_block_into(blocks + i * ORA_BLOCK_BYTES, (uint32_t)i, plan, cfg, &sl, has_lo, lo, has_hi, hi, NULL);
    uint64_t rest = n_blocks - warmup;
    uint64_t shards = (uint64_t)threads * 2;
    if (shards < 8) shards = 8;
    uint64_t chunk = (rest + shards - 1) / shards;
    if (chunk < 16) chunk = 16;
    float floor_tau = sl_threshold(&sl);
    uint64_t n_jobs = (rest + chunk - 1) / chunk;
    shard_job *jobs = (shard_job *)calloc(n_jobs ? n_jobs : 1, sizeof(shard_job));
    for (uint64_t ci = 0; ci < n_jobs; ++ci) {
      shard_job *j = &jobs[ci];
      j->blocks = blocks;
      j->first = warmup + ci * chunk;
      j->count = (ci + 1) * chunk <= rest ? chunk : rest - ci * chunk;
      j->plan = plan;
      j->cfg = cfg;
      j->has_lo = has_lo; j->lo = lo;
      j->has_hi = has_hi; j->hi = hi;
      j->floor_tau = floor_tau;
      sl_init(&j->local, cfg->shortlist_cand, floor_tau);
    }
    shard_pool pool = {jobs, n_jobs, 0, PTHREAD_MUTEX_INITIALIZER};
    int nt = threads;
    if ((uint64_t)nt > n_jobs) nt = (int)n_jobs;
    if (nt <= 1) {
      shard_worker(&pool);
    } else {
      pthread_t *tids = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nt);
      for (int t = 0; t < nt; ++t) pthread_create(&tids[t], NULL, shard_worker, &pool);
      for (int t = 0; t < nt; ++t) pthread_join(tids[t], NULL);
      free(tids);
    }
    for (uint64_t ci = 0; ci < n_jobs; ++ci) {
      sl_merge(&sl, &jobs[ci].local);
      sl_free(&jobs[ci].local);
    }
    free(jobs);
    int r = sl_into_sorted(&sl, out_ids, out_scores);
    sl_free(&sl);
    return r;
  }
  for (uint64_t i = 0; i < n_blocks; ++i)
    scan_block_into(blocks + i * ORA_BLOCK_BYTES, (uint32_t)i, plan, cfg, &sl, has_lo, lo, has_hi, hi, stats);
  int r = sl_into_sorted(&sl, out_ids, out_scores);
  sl_free(&sl);
  return r;
}

void ora_exhaustive_scores(const uint8_t *blocks, uint64_t n_blocks, const ora_plan *plan,
                           const ora_scan_config *cfg, int has_lo, uint32_t lo, int has_hi, uint32_t hi,
                           float *out_scores, uint8_t *out_valid) {
  for (uint64_t b = 0; b < n_blocks; ++b) {
    block_state st;
    int skipped;
    uint64_t surv = scan_block_core(blocks + b * ORA_BLOCK_BYTES, plan, cfg, -INFINITY, has_lo, lo, has_hi,
                                    hi, NULL, &st, NULL, &skipped);
    for (int v = 0; v < 64; ++v) {
      int ok = !skipped && ((surv >> v) & 1ull);
      out_valid[b * 64 + v] = (uint8_t)ok;
      out_scores[b * 64 + v] = ok ? st.scores[v] : NAN;
    }
  }
}


/* ========================================================================== */
/* post-scan rerank                                                            */
/* ========================================================================== */

/* embed.rs:115-152 */
float ora_dot(const float *a, const float *b, uint32_t n) {
  if (n == 768) {
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t i = 0; i < 768; i += 8)
      for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
    return acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
  }
  float s = -0.0f;
  for (uint32_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}

/* embed.rs:158-180, lowprec.rs:49-61 */
float ora_dot_fp16_768(const float *q, const float *v) {
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t i = 0; i < 768; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += q[i + j] * ora_f16_to_f32(ora_f32_to_f16(v[i + j]));
  return acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
}

/* lowprec.rs:72-94 */
void ora_int8_quantize_768(const float *v, int8_t *codes, uint16_t *scale_f16) {
  float max_abs = 0.0f;
  for (int i = 0; i < 768; ++i) max_abs = rmax(max_abs, fabsf(v[i]));
  const float scale = max_abs < 1e-12f ? 0.0f : max_abs / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  for (int i = 0; i < 768; ++i) {
    float q = roundf(v[i] * inv);
    if (q < -127.0f) q = -127.0f; /* f32::clamp; NaN stays NaN */
    if (q > 127.0f) q = 127.0f;
    int32_t iq = (q == q) ? (int32_t)q : 0; /* `as i32`: NaN -> 0 */
    codes[i] = (int8_t)iq;
  }
  *scale_f16 = ora_f32_to_f16(scale);
}

/* embed.rs:184-206 */
float ora_dot_int8_768(const float *q, const int8_t *codes, uint16_t scale_f16) {
  float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t i = 0; i < 768; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += q[i + j] * (float)codes[i + j];
  return (acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7]) * ora_f16_to_f32(scale_f16);
}

/* lowprec.rs:103-121 */
float ora_rerank_dot(int precision, const float *q, const float *row, uint32_t n) {
  if (precision == ORA_RERANK_FP16) return ora_dot_fp16_768(q, row);
  if (precision == ORA_RERANK_INT8) {
    int8_t codes[768];
    uint16_t sc;
    ora_int8_quantize_768(row, codes, &sc);
    return ora_dot_int8_768(q, codes, sc);
  }
  return ora_dot(q, row, n);
}

/* pipeline.rs:157-169: map then stable sort_by(b.1.partial_cmp(&a.1).unwrap()) */
int ora_rerank(int precision, const float *q, const float *rows, uint32_t n, const uint64_t *cand_rows,
               uint32_t n_cand, uint64_t *out_rows, float *out_scores) {
  for (uint32_t i = 0; i < n_cand; ++i) {
    out_rows[i] = cand_rows[i];
    out_scores[i] = ora_rerank_dot(precision, q, rows + cand_rows[i] * (uint64_t)n, n);
    if (out_scores[i] != out_scores[i]) return -ORA_ERR_NAN;
  }
  /* stable insertion sort, descending */
  for (uint32_t i = 1; i < n_cand; ++i) {
    const float s = out_scores[i];
    const uint64_t r = out_rows[i];
    uint32_t j = i;
    while (j > 0 && out_scores[j - 1] < s) {
      out_scores[j] = out_scores[j - 1];
      out_rows[j] = out_rows[j - 1];
      --j;
    }
    out_scores[j] = s;
    out_rows[j] = r;
  }
  return 0;
}


/* ring.rs:109-119 */
int ora_ring_search_exact(const float *pending, uint32_t n_pending, uint32_t dims, const float *q,
                          uint32_t top_k, uint64_t *out_local, float *out_scores) {
  uint64_t *cand = (uint64_t *)calloc(n_pending ? n_pending : 1, sizeof(uint64_t));
  uint64_t *rows = (uint64_t *)malloc(sizeof(uint64_t) * (n_pending ? n_pending : 1));
  float *sc = (float *)malloc(sizeof(float) * (n_pending ? n_pending : 1));
  for (uint32_t i = 0; i < n_pending; ++i) cand[i] = i;
  int rc = ora_rerank(ORA_RERANK_FP32, q, pending, dims, cand, n_pending, rows, sc);
  uint32_t keep = top_k < n_pending ? top_k : n_pending;
  if (rc == 0)
    for (uint32_t i = 0; i < keep; ++i) {
      out_local[i] = rows[i];
      out_scores[i] = sc[i];
    }
  free(cand);
  free(rows);
  free(sc);
  return rc ? rc : (int)keep;
}

/* scan.rs:311-399 driven as engine.rs:584-594 drives it */
int ora_shortlist_push_sorted(uint32_t capacity, const uint64_t *ids, const float *scores, uint32_t n,
                              const uint64_t *push_ids, const float *push_scores, uint32_t n_push,
                              uint64_t *out_ids, float *out_scores) {
  shortlist s;
  sl_init(&s, capacity, -INFINITY);
  for (uint32_t i = 0; i < n; ++i) {
    hit h = {ids[i], scores[i]};
    sl_push(&s, h);
  }
  for (uint32_t i = 0; i < n_push; ++i) {
    hit h = {push_ids[i], push_scores[i]};
    sl_push(&s, h);
  }
  int rc = sl_into_sorted(&s, out_ids, out_scores);
  sl_free(&s);
  return rc;
}
