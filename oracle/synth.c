/*
 * synth.c -- scalar formats and the deterministic input generator (CPU side).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  The GPU twin of the generator is
 * the package's csrc/synth.hip; tests check the two agree byte for byte.
 *
 * Generator definition (the configs of the benchmark are stated in terms of it):
 *   h      = splitmix64 output at position idx of the stream keyed by
 *            mix64((seed << 8) ^ stream)
 *   normal = Irwin-Hall(4) over the four 16-bit fields of h, centred and
 *            scaled to unit variance: (sum - 131070) * (1/37837.227...)
 *            -- an approximately normal variate bounded at +-3.46 sigma that
 *            every platform computes identically (integer sum, one fp32 mul).
 *   values = normal * sigma (one fp32 mul), then block quantisation:
 *            scale = absmax / 448 (fp32 div), q = e4m3_rne_satfinite(x / scale).
 * The layouts follow the definition (moe.py:29-40): hidden scales are
 * transposed [56, T]; weight scales are per 128x128 block.
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

/* ---------------------------------------------------------------------- */
/* scalar formats                                                          */
/* ---------------------------------------------------------------------- */
static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* OCP e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa; no infinities;
 * 0x7F/0xFF are NaN; max finite 448; subnormal step 2^-9. */
float orc_e4m3_to_f32(uint8_t v) {
  const uint32_t sign = (uint32_t)(v >> 7) << 31;
  const uint32_t e = (v >> 3) & 0xF, m = v & 7;
  if (e == 0xF && m == 7) return u2f(sign | 0x7FC00000u);
  if (e == 0) {
    /* subnormal: m * 2^-9 (exact in fp32) */
    float mag = (float)m * 0x1p-9f;
    return sign ? -mag : mag;
  }
  return u2f(sign | ((e + 120u) << 23) | (m << 20));
}

uint8_t orc_f32_to_e4m3(float x) {
  const uint32_t u = f2u(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(sign | 0x7F); /* NaN */
  const float af = u2f(a);
  if (af >= 448.0f) return (uint8_t)(sign | 0x7E);    /* satfinite (incl. inf) */
  if (af < 0x1p-6f) {
    /* subnormal range: round(af * 2^9) to nearest even; 8 -> min normal */
    float q = nearbyintf(af * 512.0f);
    return (uint8_t)(sign | (uint8_t)q);
  }
  int e = (int)(a >> 23) - 127;         /* -6 .. 8 */
  uint32_t keep = (a >> 20) & 7;         /* top 3 mantissa bits */
  const uint32_t rem = a & 0xFFFFFu;     /* discarded 20 bits   */
  if (rem > 0x80000u || (rem == 0x80000u && (keep & 1))) {
    keep++;
    if (keep == 8) {
      keep = 0;
      e++;
    }
  }
  /* e <= 8 here; e == 8 with keep == 7 would be 480 -> excluded above */
  if (e > 8 || (e == 8 && keep == 7)) return (uint8_t)(sign | 0x7E);
  return (uint8_t)(sign | (uint8_t)((e + 7) << 3) | (uint8_t)keep);
}

float orc_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

uint16_t orc_f32_to_bf16(float x) {
  const uint32_t u = f2u(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  const uint32_t r = u + 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

/* exp evaluated in double and rounded once to fp32: correctly rounded except
 * in astronomically rare double-rounding cases. */
float orc_exp_f32(float x) { return (float)exp((double)x); }

/* ---------------------------------------------------------------------- */
/* generator                                                               */
/* ---------------------------------------------------------------------- */
#define SM_GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
  z += SM_GAMMA;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t synth_hash(uint64_t seed, uint32_t stream, uint64_t idx) {
  const uint64_t key = mix64((seed << 8) ^ (uint64_t)stream);
  return mix64(key + idx * SM_GAMMA);
}

static const float IH4_INV_STD = 0x1.bb67aep-16f; /* 1/sqrt((65536^2-1)/3) */
static const float SIGMA_W13 = 0x1.83091ep-7f;    /* 1/sqrt(7168) */
static const float SIGMA_W2 = 0x1.6a09e6p-6f;     /* 1/sqrt(2048) */
static const float SIGMA_BIAS = 0x1.99999ap-4f;   /* 0.1 */

static inline float normal_from_hash(uint64_t h) {
  const int32_t s = (int32_t)((h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) +
                              (h >> 48));
  return (float)(s - 131070) * IH4_INV_STD;
}

float synth_normal(uint64_t seed, uint32_t stream, uint64_t idx) {
  return normal_from_hash(synth_hash(seed, stream, idx));
}

void synth_logits(uint64_t seed, int64_t T, float* out) {
  const uint64_t key = mix64((seed << 8) ^ SYN_LOGITS);
  const int64_t n = T * ORC_E_GLOBAL;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = normal_from_hash(mix64(key + (uint64_t)i * SM_GAMMA));
}

void synth_bias(uint64_t seed, const int32_t* hot_ids, int n_hot, float hot_add,
                uint16_t* out) {
  const uint64_t key = mix64((seed << 8) ^ SYN_BIAS);
  for (int e = 0; e < ORC_E_GLOBAL; ++e) {
    float b = normal_from_hash(mix64(key + (uint64_t)e * SM_GAMMA)) * SIGMA_BIAS;
    for (int j = 0; j < n_hot; ++j)
      if (hot_ids[j] == e) b = b + hot_add;
    out[e] = orc_f32_to_bf16(b);
  }
}

/* quantise n values given their absmax; returns the scale */
static inline float block_scale(float amax) { return amax > 0.0f ? amax / 448.0f : 1.0f; }

void synth_hidden(uint64_t seed, int64_t T, uint8_t* q, float* scale) {
  const uint64_t key = mix64((seed << 8) ^ SYN_HIDDEN);
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    for (int b = 0; b < ORC_NH_BLK; ++b) {
      float v[ORC_BLOCK];
      float amax = 0.0f;
      for (int j = 0; j < ORC_BLOCK; ++j) {
        const uint64_t idx = (uint64_t)t * ORC_H + (uint64_t)b * ORC_BLOCK + (uint64_t)j;
        v[j] = normal_from_hash(mix64(key + idx * SM_GAMMA));
        const float a = fabsf(v[j]);
        if (a > amax) amax = a;
      }
      const float s = block_scale(amax);
      scale[(int64_t)b * T + t] = s;
      uint8_t* dst = q + t * ORC_H + b * ORC_BLOCK;
      for (int j = 0; j < ORC_BLOCK; ++j) dst[j] = orc_f32_to_e4m3(v[j] / s);
    }
  }
}

void orc_quantize_hidden(const uint16_t* x, int64_t T, uint8_t* q, float* scale) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    for (int b = 0; b < ORC_NH_BLK; ++b) {
      const uint16_t* src = x + t * ORC_H + b * ORC_BLOCK;
      float amax = 0.0f;
      for (int j = 0; j < ORC_BLOCK; ++j) {
        const float a = fabsf(orc_bf16_to_f32(src[j]));
        if (a > amax) amax = a; /* NaN never compares greater */
      }
      const float s = block_scale(amax);
      scale[(int64_t)b * T + t] = s;
      uint8_t* dst = q + t * ORC_H + b * ORC_BLOCK;
      for (int j = 0; j < ORC_BLOCK; ++j) dst[j] = orc_f32_to_e4m3(orc_bf16_to_f32(src[j]) / s);
    }
  }
}

/* Generic [E, R, C] weight with 128x128 block scales [E, R/128, C/128]. */
static void synth_weight(uint64_t seed, uint32_t stream, float sigma, int rows, int cols, int e0,
                         int e1, uint8_t* q, float* scale) {
  const uint64_t key = mix64((seed << 8) ^ stream);
  const int rb_n = rows / ORC_BLOCK, cb_n = cols / ORC_BLOCK;
  const int64_t nblk = (int64_t)(e1 - e0) * rb_n * cb_n;
#pragma omp parallel for schedule(static)
  for (int64_t bi = 0; bi < nblk; ++bi) {
    const int e = e0 + (int)(bi / (rb_n * cb_n));
    const int rb = (int)((bi / cb_n) % rb_n);
    const int cb = (int)(bi % cb_n);
    static __thread float v[ORC_BLOCK * ORC_BLOCK];
    float amax = 0.0f;
    for (int r = 0; r < ORC_BLOCK; ++r) {
      const uint64_t row = (uint64_t)e * rows + (uint64_t)rb * ORC_BLOCK + (uint64_t)r;
      for (int c = 0; c < ORC_BLOCK; ++c) {
        const uint64_t idx = row * (uint64_t)cols + (uint64_t)cb * ORC_BLOCK + (uint64_t)c;
        const float x = normal_from_hash(mix64(key + idx * SM_GAMMA)) * sigma;
        v[r * ORC_BLOCK + c] = x;
        const float a = fabsf(x);
        if (a > amax) amax = a;
      }
    }
    const float s = block_scale(amax);
    scale[((int64_t)e * rb_n + rb) * cb_n + cb] = s;
    for (int r = 0; r < ORC_BLOCK; ++r) {
      uint8_t* dst = q + ((int64_t)e * rows + (int64_t)rb * ORC_BLOCK + r) * cols + cb * ORC_BLOCK;
      for (int c = 0; c < ORC_BLOCK; ++c) dst[c] = orc_f32_to_e4m3(v[r * ORC_BLOCK + c] / s);
    }
  }
}

void synth_w13(uint64_t seed, int e0, int e1, uint8_t* q, float* scale) {
  synth_weight(seed, SYN_W13, SIGMA_W13, ORC_2I, ORC_H, e0, e1, q, scale);
}

void synth_w2(uint64_t seed, int e0, int e1, uint8_t* q, float* scale) {
  synth_weight(seed, SYN_W2, SIGMA_W2, ORC_H, ORC_I, e0, e1, q, scale);
}
