/*
 * ishz_oracle.c — CPU restatement of the reference's quantized-weight path.
 * TEST INFRASTRUCTURE ONLY (see ishz_oracle.h for what pins each function).
 *
 * Dequantizers follow Sources/IshizukiKit/Core/GGMLDequant.swift (scalar walk of each block,
 * itself a port of ggml's dequantize_row_*). Arithmetic mirrors the reference's fp32 order:
 * every scale product is formed first and the weight is one multiply (and, for the min formats,
 * one subtraction), so results are bit-identical to the reference's.
 */
#include "ishz_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "../ishizuki_amd/csrc/ggml_grids.inc"

/* ---------------------------------------------------------------- geometry */

/* GGMLType.blockSize / typeSize, Sources/IshizukiKit/Config/GGUFFile.swift:45-80. */
int ishzo_block_size(uint32_t t) {
  switch (t) {
  case ISHZO_F32: case ISHZO_F16: case ISHZO_BF16: return 1;
  case ISHZO_Q4_0: return 32;
  case ISHZO_Q2_K: case ISHZO_Q4_K: case ISHZO_Q6_K: case ISHZO_IQ2_XXS: case ISHZO_IQ2_XS:
  case ISHZO_IQ3_XXS: case ISHZO_IQ1_S: case ISHZO_IQ3_S: case ISHZO_IQ2_S: case ISHZO_IQ4_XS:
  case ISHZO_IQ1_M: return 256;
  default: return 0;
  }
}

int ishzo_type_size(uint32_t t) {
  switch (t) {
  case ISHZO_F32: return 4;
  case ISHZO_F16: case ISHZO_BF16: return 2;
  case ISHZO_Q4_0: return 18;
  case ISHZO_Q2_K: return 84;
  case ISHZO_Q4_K: return 144;
  case ISHZO_Q6_K: return 210;
  case ISHZO_IQ2_XXS: return 66;
  case ISHZO_IQ2_XS: return 74;
  case ISHZO_IQ3_XXS: return 98;
  case ISHZO_IQ1_S: return 50;
  case ISHZO_IQ3_S: return 110;
  case ISHZO_IQ2_S: return 82;
  case ISHZO_IQ4_XS: return 136;
  case ISHZO_IQ1_M: return 56;
  default: return 0;
  }
}

/* ---------------------------------------------------------------- fp16 */

float ishzo_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float v = (float)man * 5.9604644775390625e-8f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t ishzo_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00 : 0x7c00);
  if (ax >= 0x477ff000u) return sign | 0x7c00; /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) {                      /* below 2^-14: subnormal or zero */
    /* value / 2^-24, rounded to nearest even, as an integer mantissa */
    float a;
    memcpy(&a, &ax, 4);
    float m = a * 16777216.0f; /* exact: scaling by a power of two */
    float r = nearbyintf(m);   /* default rounding mode: nearest even */
    return sign | (uint16_t)r;
  }
  uint32_t e = (ax >> 23) - 112, man = ax & 0x7fffff;
  uint32_t h = (e << 10) | (man >> 13), rest = man & 0x1fff;
  if (rest > 0x1000 || (rest == 0x1000 && (h & 1))) h++;
  return sign | (uint16_t)h;
}

static inline float round16(float f) { return ishzo_half_to_float(ishzo_float_to_half(f)); }

/* ---------------------------------------------------------------- block readers */

static inline float rd_half(const uint8_t *p) { return ishzo_half_to_float((uint16_t)(p[0] | p[1] << 8)); }
static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | p[1] << 8); }
static inline uint32_t rd_u32(const uint8_t *p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static inline int grid_byte(uint64_t e, int j) { return (int)((e >> (8 * j)) & 0xff); }
static inline float sign_of(uint8_t signs, int j) { return (signs >> j) & 1 ? -1.0f : 1.0f; }
/* ksigns_iq2xs[i]: the 7 stored sign bits plus an eighth making the count even. */
static inline uint8_t ksigns(int i) { return (uint8_t)(i | (__builtin_popcount(i) & 1) << 7); }

/* Q4_0 (ggml block_q4_0: fp16 d, 16 B of nibbles). The reference has no decoder: GGMLType
   .q40 exists (GGUFFile.swift:16,58) but GGMLDequant.supported omits it (GGMLDequant.swift:19).
   Element j is (lo(qs[j]) - 8) * d and element j + 16 is (hi(qs[j]) - 8) * d. */
static void deq_q4_0(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int j = 0; j < 16; j++) {
    y[j] = (float)((p[2 + j] & 0xf) - 8) * d;
    y[j + 16] = (float)((p[2 + j] >> 4) - 8) * d;
  }
}

/* GGMLDequant.q2K, Core/GGMLDequant.swift:125-152. */
static void deq_q2_k(const uint8_t *p, float *y) {
  float d = rd_half(p + 80), dmin = rd_half(p + 82);
  int out = 0, scale = 0;
  for (int n = 0; n < 256; n += 128) {
    int quants = 16 + n / 4;
    for (int shift = 0; shift < 8; shift += 2) {
      for (int lane = 0; lane < 2; lane++) {
        uint8_t sc = p[scale++];
        float dl = d * (float)(sc & 0xf), ml = dmin * (float)(sc >> 4);
        for (int l = 0; l < 16; l++) y[out++] = dl * (float)((p[quants + 16 * lane + l] >> shift) & 3) - ml;
      }
    }
  }
}

/* GGMLDequant.q6K, Core/GGMLDequant.swift:154-185. */
static void deq_q6_k(const uint8_t *p, float *y) {
  float d = rd_half(p + 208);
  int low = 0, high = 128, scale = 192;
  for (int out = 0; out < 256; out += 128) {
    for (int l = 0; l < 32; l++) {
      uint8_t bits = p[high + l];
      int q1 = (p[low + l] & 0xf) | ((bits >> 0) & 3) << 4;
      int q2 = (p[low + 32 + l] & 0xf) | ((bits >> 2) & 3) << 4;
      int q3 = (p[low + l] >> 4) | ((bits >> 4) & 3) << 4;
      int q4 = (p[low + 32 + l] >> 4) | ((bits >> 6) & 3) << 4;
      int g = l / 16;
      y[out + l] = d * (float)(int8_t)p[scale + g + 0] * (float)(q1 - 32);
      y[out + 32 + l] = d * (float)(int8_t)p[scale + g + 2] * (float)(q2 - 32);
      y[out + 64 + l] = d * (float)(int8_t)p[scale + g + 4] * (float)(q3 - 32);
      y[out + 96 + l] = d * (float)(int8_t)p[scale + g + 6] * (float)(q4 - 32);
    }
    low += 64;
    high += 32;
    scale += 8;
  }
}

/* 6-bit scale/min pair j of a Q4_K block (GGMLDequant.q4K.scaleMin, :193-205). */
static void q4k_scale_min(const uint8_t *p, int j, uint8_t *sc, uint8_t *m) {
  const uint8_t *q = p + 4;
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* GGMLDequant.q4K, Core/GGMLDequant.swift:187-220. */
static void deq_q4_k(const uint8_t *p, float *y) {
  float d = rd_half(p), dmin = rd_half(p + 2);
  for (int j = 0, pair = 0; j < 256; j += 64, pair += 2) {
    uint8_t s1, m1, s2, m2;
    q4k_scale_min(p, pair, &s1, &m1);
    q4k_scale_min(p, pair + 1, &s2, &m2);
    float d1 = d * (float)s1, dm1 = dmin * (float)m1;
    float d2 = d * (float)s2, dm2 = dmin * (float)m2;
    const uint8_t *qs = p + 16 + j / 2;
    for (int l = 0; l < 32; l++) {
      y[j + l] = d1 * (float)(qs[l] & 0xf) - dm1;
      y[j + 32 + l] = d2 * (float)(qs[l] >> 4) - dm2;
    }
  }
}

/* GGMLDequant.iq4XS, :222-241. */
static void deq_iq4_xs(const uint8_t *p, float *y) {
  float d = rd_half(p);
  uint16_t sh = rd_u16(p + 2);
  for (int ib = 0; ib < 8; ib++) {
    int lo = (p[4 + ib / 2] >> (4 * (ib % 2))) & 0xf;
    int hi = ((sh >> (2 * ib)) & 3) << 4;
    float dl = d * (float)((lo | hi) - 32);
    const uint8_t *qs = p + 8 + 16 * ib;
    for (int j = 0; j < 16; j++) {
      y[32 * ib + j] = dl * (float)ishz_kvalues_iq4nl[qs[j] & 0xf];
      y[32 * ib + 16 + j] = dl * (float)ishz_kvalues_iq4nl[qs[j] >> 4];
    }
  }
}

/* GGMLDequant.iq2XXS, :243-262. */
static void deq_iq2_xxs(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int ib = 0; ib < 8; ib++) {
    uint32_t a1 = rd_u32(p + 2 + 8 * ib), a2 = rd_u32(p + 2 + 8 * ib + 4);
    float db = d * (0.5f + (float)(a2 >> 28)) * 0.25f;
    for (int l = 0; l < 4; l++) {
      uint64_t e = ishz_iq2xxs_grid[(a1 >> (8 * l)) & 0xff];
      uint8_t s = ksigns((a2 >> (7 * l)) & 127);
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = db * (float)grid_byte(e, j) * sign_of(s, j);
    }
  }
}

/* GGMLDequant.iq2XS, :264-285. Element 8l+j of group ib32 is
   d*(0.5+nibble)*0.25 * grid[q & 511][j] * (sign bit j of ksigns[q >> 9] ? -1 : 1). */
static void deq_iq2_xs(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int ib = 0; ib < 8; ib++) {
    uint8_t sc = p[66 + ib];
    float db[2] = {d * (0.5f + (float)(sc & 0xf)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
    for (int l = 0; l < 4; l++) {
      uint16_t q = rd_u16(p + 2 + 2 * (4 * ib + l));
      uint64_t e = ishz_iq2xs_grid[q & 511];
      uint8_t s = ksigns(q >> 9);
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = db[l / 2] * (float)grid_byte(e, j) * sign_of(s, j);
    }
  }
}

/* GGMLDequant.iq2S, :287-309. */
static void deq_iq2_s(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int ib = 0; ib < 8; ib++) {
    uint8_t sc = p[74 + ib];
    float db[2] = {d * (0.5f + (float)(sc & 0xf)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
    int qh = p[66 + ib];
    for (int l = 0; l < 4; l++) {
      int idx = p[2 + 4 * ib + l] | ((qh << (8 - 2 * l)) & 0x300);
      uint64_t e = ishz_iq2s_grid[idx];
      uint8_t s = p[34 + 4 * ib + l];
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = db[l / 2] * (float)grid_byte(e, j) * sign_of(s, j);
    }
  }
}

/* GGMLDequant.iq3XXS, :311-330. */
static void deq_iq3_xxs(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int ib = 0; ib < 8; ib++) {
    uint32_t aux = rd_u32(p + 2 + 64 + 4 * ib);
    float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    for (int l = 0; l < 4; l++) {
      uint8_t s = ksigns((aux >> (7 * l)) & 127);
      uint32_t g1 = ishz_iq3xxs_grid[p[2 + 8 * ib + 2 * l]];
      uint32_t g2 = ishz_iq3xxs_grid[p[2 + 8 * ib + 2 * l + 1]];
      for (int j = 0; j < 4; j++) {
        y[32 * ib + 8 * l + j] = db * (float)grid_byte(g1, j) * sign_of(s, j);
        y[32 * ib + 8 * l + 4 + j] = db * (float)grid_byte(g2, j) * sign_of(s, j + 4);
      }
    }
  }
}

/* GGMLDequant.iq3S, :332-364. */
static void deq_iq3_s(const uint8_t *p, float *y) {
  float d = rd_half(p);
  int out = 0;
  for (int pair = 0; pair < 8; pair += 2) {
    uint8_t sc = p[2 + 64 + 8 + 32 + pair / 2];
    float db[2] = {d * (float)(1 + 2 * (sc & 0xf)), d * (float)(1 + 2 * (sc >> 4))};
    for (int g = 0; g < 2; g++) {
      int qh = p[66 + pair + g];
      const uint8_t *qs = p + 2 + 8 * (pair + g);
      const uint8_t *sg = p + 74 + 4 * (pair + g);
      for (int l = 0; l < 4; l++) {
        uint32_t g1 = ishz_iq3s_grid[qs[2 * l] | ((qh << (8 - 2 * l)) & 256)];
        uint32_t g2 = ishz_iq3s_grid[qs[2 * l + 1] | ((qh << (7 - 2 * l)) & 256)];
        for (int j = 0; j < 4; j++) {
          y[out + j] = db[g] * (float)grid_byte(g1, j) * sign_of(sg[l], j);
          y[out + 4 + j] = db[g] * (float)grid_byte(g2, j) * sign_of(sg[l], j + 4);
        }
        out += 8;
      }
    }
  }
}

/* GGMLDequant.iq1S, :366-385 (grid bytes read signed, delta +-1/8). */
static void deq_iq1_s(const uint8_t *p, float *y) {
  float d = rd_half(p);
  for (int ib = 0; ib < 8; ib++) {
    uint16_t qh = rd_u16(p + 34 + 2 * ib);
    float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
    float delta = (qh & 0x8000) ? -0.125f : 0.125f;
    for (int l = 0; l < 4; l++) {
      int idx = p[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8);
      uint64_t e = ishz_iq1s_grid[idx];
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = dl * ((float)(int8_t)grid_byte(e, j) + delta);
    }
  }
}

/* GGMLDequant.iq1M, :387-428. */
static void deq_iq1_m(const uint8_t *p, float *y) {
  uint16_t sc[4];
  for (int i = 0; i < 4; i++) sc[i] = rd_u16(p + 48 + 2 * i);
  uint16_t packed = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000));
  float d = ishzo_half_to_float(packed);
  for (int ib = 0; ib < 8; ib++) {
    uint16_t w = sc[ib / 2];
    int shift = 6 * (ib % 2);
    float dl1 = d * (float)(2 * ((w >> shift) & 7) + 1);
    float dl2 = d * (float)(2 * ((w >> (shift + 3)) & 7) + 1);
    int qh0 = p[32 + 2 * ib], qh1 = p[32 + 2 * ib + 1];
    int idx[4] = {p[4 * ib] | ((qh0 << 8) & 0x700), p[4 * ib + 1] | ((qh0 << 4) & 0x700),
                  p[4 * ib + 2] | ((qh1 << 8) & 0x700), p[4 * ib + 3] | ((qh1 << 4) & 0x700)};
    float delta[4] = {(qh0 & 0x08) ? -0.125f : 0.125f, (qh0 & 0x80) ? -0.125f : 0.125f,
                      (qh1 & 0x08) ? -0.125f : 0.125f, (qh1 & 0x80) ? -0.125f : 0.125f};
    for (int l = 0; l < 4; l++) {
      float dl = l < 2 ? dl1 : dl2;
      uint64_t e = ishz_iq1s_grid[idx[l]];
      for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = dl * ((float)(int8_t)grid_byte(e, j) + delta[l]);
    }
  }
}

/* GGMLDequant.dequantize, :25-62: refuse unknown types, ragged counts and short buffers. */
int ishzo_dequant(uint32_t type, const uint8_t *b, size_t nbytes, size_t count, float *y) {
  int bs = ishzo_block_size(type), ts = ishzo_type_size(type);
  if (!bs) return -1;
  if (count % (size_t)bs) return -2;
  size_t blocks = count / (size_t)bs;
  if (nbytes < blocks * (size_t)ts) return -3;
  void (*body)(const uint8_t *, float *) = NULL;
  switch (type) {
  case ISHZO_F32: for (size_t i = 0; i < blocks; i++) memcpy(y + i, b + 4 * i, 4); return 0;
  case ISHZO_F16: for (size_t i = 0; i < blocks; i++) y[i] = rd_half(b + 2 * i); return 0;
  case ISHZO_BF16:
    for (size_t i = 0; i < blocks; i++) {
      uint32_t bits = (uint32_t)rd_u16(b + 2 * i) << 16;
      memcpy(y + i, &bits, 4);
    }
    return 0;
  case ISHZO_Q4_0: body = deq_q4_0; break;
  case ISHZO_Q2_K: body = deq_q2_k; break;
  case ISHZO_Q4_K: body = deq_q4_k; break;
  case ISHZO_Q6_K: body = deq_q6_k; break;
  case ISHZO_IQ2_XXS: body = deq_iq2_xxs; break;
  case ISHZO_IQ2_XS: body = deq_iq2_xs; break;
  case ISHZO_IQ2_S: body = deq_iq2_s; break;
  case ISHZO_IQ3_XXS: body = deq_iq3_xxs; break;
  case ISHZO_IQ3_S: body = deq_iq3_s; break;
  case ISHZO_IQ1_S: body = deq_iq1_s; break;
  case ISHZO_IQ1_M: body = deq_iq1_m; break;
  case ISHZO_IQ4_XS: body = deq_iq4_xs; break;
  default: return -1;
  }
  for (size_t i = 0; i < blocks; i++) body(b + i * (size_t)ts, y + i * (size_t)bs);
  return 0;
}

/* ---------------------------------------------------------------- matmul */

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
}

static float dot_f32(const float *a, const float *b, int K) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int k = 0;
  for (; k + 8 <= K; k += 8)
    for (int u = 0; u < 8; u++) acc[u] += a[k + u] * b[k + u];
  for (; k < K; k++) acc[0] += a[k] * b[k];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

/* Rows of a [N][K] GGML matrix dequantized in parallel (ishzo_dequant per row). */
int ishzo_dequant_rows(uint32_t type, const uint8_t *blocks, int N, int K, float *out, int threads) {
  int bs = ishzo_block_size(type), ts = ishzo_type_size(type);
  if (!bs) return -1;
  if (K % bs) return -2;
  size_t rb = (size_t)(K / bs) * (size_t)ts;
  set_threads(threads);
  int rc = 0;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    int r = ishzo_dequant(type, blocks + (size_t)n * rb, rb, (size_t)K, out + (size_t)n * K);
    if (r) rc = r;
  }
  return rc;
}

/* Dequantize-then-dot, the reference's CPU definition (GGMLKernelTests.swift:111-140 checks
   the matvec against the expanded weight exactly this way). */
int ishzo_ggml_matmul(uint32_t type, const float *x, int M, int K, const uint8_t *blocks, int N,
                      float *y, int threads) {
  int bs = ishzo_block_size(type), ts = ishzo_type_size(type);
  if (!bs) return -1;
  if (K % bs) return -2;
  size_t rb = (size_t)(K / bs) * (size_t)ts;
  float *w = (float *)malloc((size_t)N * (size_t)K * sizeof(float));
  if (!w) return -4;
  set_threads(threads);
  int rc = 0;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    int r = ishzo_dequant(type, blocks + (size_t)n * rb, rb, (size_t)K, w + (size_t)n * K);
    if (r) rc = r;
  }
  if (!rc) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
      for (int m = 0; m < M; m++) y[(size_t)m * N + n] = dot_f32(x + (size_t)m * K, w + (size_t)n * K, K);
  }
  free(w);
  return rc;
}

/* Fused variant: one row is decoded into a thread-local buffer and dotted immediately. */
int ishzo_ggml_matmul_fused(uint32_t type, const float *x, int M, int K, const uint8_t *blocks,
                            int N, float *y, int threads) {
  int bs = ishzo_block_size(type), ts = ishzo_type_size(type);
  if (!bs) return -1;
  if (K % bs) return -2;
  size_t rb = (size_t)(K / bs) * (size_t)ts;
  set_threads(threads);
  int rc = 0;
#pragma omp parallel
  {
    float *w = (float *)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
    for (int n = 0; n < N; n++) {
      int r = ishzo_dequant(type, blocks + (size_t)n * rb, rb, (size_t)K, w);
      if (r) rc = r;
      for (int m = 0; m < M; m++) y[(size_t)m * N + n] = dot_f32(x + (size_t)m * K, w, K);
    }
    free(w);
  }
  return rc;
}

/* ---------------------------------------------------------------- affine */

/* MLX affine pack: w[n][k] = s[n][k/gs] * q + b[n][k/gs], q = bits-wide field k of the row's
   little-endian u32 stream (Quantize/WeightedAffineQuantizer.swift:142-153; read back the same
   way in Core/VerifyMatmul.swift:173-188). */
int ishzo_affine_dequant(const uint32_t *codes, const uint16_t *scales, const uint16_t *biases,
                         int N, int K, int bits, int group, float *out) {
  if (bits < 1 || bits > 8 || group <= 0 || K % group || ((size_t)K * bits) % 32) return -1;
  size_t wpr = (size_t)K * bits / 32;
  int gpr = K / group;
  uint32_t mask = (1u << bits) - 1;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    const uint32_t *row = codes + (size_t)n * wpr;
    for (int g = 0; g < gpr; g++) {
      float s = ishzo_half_to_float(scales[(size_t)n * gpr + g]);
      float b = ishzo_half_to_float(biases[(size_t)n * gpr + g]);
      for (int k = g * group; k < (g + 1) * group; k++) {
        size_t bit = (size_t)k * bits;
        uint64_t pair = row[bit / 32];
        if (bit / 32 + 1 < wpr) pair |= (uint64_t)row[bit / 32 + 1] << 32;
        uint32_t q = (uint32_t)(pair >> (bit % 32)) & mask;
        out[(size_t)n * K + k] = s * (float)q + b;
      }
    }
  }
  return 0;
}

int ishzo_affine_matmul(const float *x, int M, int K, const uint32_t *codes,
                        const uint16_t *scales, const uint16_t *biases, int N, int bits,
                        int group, float *y, int threads) {
  float *w = (float *)malloc((size_t)N * (size_t)K * sizeof(float));
  if (!w) return -4;
  int rc = ishzo_affine_dequant(codes, scales, biases, N, K, bits, group, w);
  set_threads(threads);
  if (!rc) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
      for (int m = 0; m < M; m++) y[(size_t)m * N + n] = dot_f32(x + (size_t)m * K, w + (size_t)n * K, K);
  }
  free(w);
  return rc;
}

/* ---------------------------------------------------------------- CPU baseline (bench.py only) */

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

static int cmp_double(const void *a, const void *b) {
  double x = *(const double *)a, y = *(const double *)b;
  return (x > y) - (x < y);
}

/* One rotated 2-bit affine GEMV (PackedLinear's rotated path, Core/Hadamard.swift:180-231) on the
   CPU: x (fp16) is rotated by hadamardRotate and rounded to fp16, then y = x.W^T with
     variant 0: W dequantized in full into a dense fp32 [N][K] (the reference's CPU definition of
                a quantized matmul: dequantize, then an fp32 dot per output),
     variant 1: each word's 16 codes decoded inside the dot, per group
                s * sum(q x) + b * sum(x), no dense W.
   OpenMP over output rows. Each of `reps` calls is timed separately; returns the median seconds.
   y gets the last call's output (fp32). */
double ishzo_bench_affine_linear(const uint16_t *xh, int K, const float *signs, int block,
                                 const uint32_t *codes, const uint16_t *scales, const uint16_t *biases,
                                 int N, int group, int variant, int reps, int threads, float *y) {
  if (K % group || K % 16 || reps < 1 || reps > 64) return -1.0;
  set_threads(threads);
  const int wpr = K / 16, gpr = K / group;
  float *xr = (float *)malloc((size_t)K * sizeof(float));
  float *xs = (float *)malloc((size_t)gpr * sizeof(float));
  float *w = variant == 0 ? (float *)malloc((size_t)N * (size_t)K * sizeof(float)) : NULL;
  if (!xr || !xs || (variant == 0 && !w)) {
    free(xr);
    free(xs);
    free(w);
    return -1.0;
  }
  double t[64];
  for (int r = 0; r < reps; r++) {
    double t0 = now_s();
    for (int k = 0; k < K; k++) xr[k] = ishzo_half_to_float(xh[k]);
    if (block > 1) ishzo_hadamard(xr, 1, K, block, signs, 0, xr);
    for (int k = 0; k < K; k++) xr[k] = ishzo_half_to_float(ishzo_float_to_half(xr[k]));
    if (variant == 0) {
      ishzo_affine_dequant(codes, scales, biases, N, K, 2, group, w);
#pragma omp parallel for schedule(static)
      for (int n = 0; n < N; n++) y[n] = dot_f32(xr, w + (size_t)n * K, K);
    } else {
      for (int g = 0; g < gpr; g++) {
        float a = 0.0f;
        for (int k = g * group; k < (g + 1) * group; k++) a += xr[k];
        xs[g] = a;
      }
#pragma omp parallel for schedule(static)
      for (int n = 0; n < N; n++) {
        const uint32_t *row = codes + (size_t)n * wpr;
        float acc = 0.0f;
        for (int g = 0; g < gpr; g++) {
          float qx = 0.0f;
          for (int c = g * group / 16; c < (g + 1) * group / 16; c++) {
            const uint32_t word = row[c];
            const float *xv = xr + 16 * c;
            float part = 0.0f;
            for (int j = 0; j < 16; j++) part += (float)((word >> (2 * j)) & 3u) * xv[j];
            qx += part;
          }
          acc += ishzo_half_to_float(scales[(size_t)n * gpr + g]) * qx +
                 ishzo_half_to_float(biases[(size_t)n * gpr + g]) * xs[g];
        }
        y[n] = acc;
      }
    }
    t[r] = now_s() - t0;
  }
  free(xr);
  free(xs);
  free(w);
  qsort(t, (size_t)reps, sizeof(double), cmp_double);
  return reps % 2 ? t[reps / 2] : 0.5 * (t[reps / 2 - 1] + t[reps / 2]);
}

/* ---------------------------------------------------------------- Hadamard */

/* hadamardRotate, Core/Hadamard.swift:8-23: fp32, signs before the transform (or after when
   inverse), orthonormal scale 1/sqrt(b), natural (Sylvester) order: H[i][j] = (-1)^popc(i&j). */
void ishzo_hadamard(const float *x, int rows, int width, int block, const float *signs,
                    int inverse, float *y) {
  float scale = 1.0f / sqrtf((float)block);
  float *v = (float *)malloc((size_t)block * sizeof(float));
  for (int r = 0; r < rows; r++) {
    for (int b0 = 0; b0 < width; b0 += block) {
      const float *xi = x + (size_t)r * width + b0;
      for (int i = 0; i < block; i++) v[i] = xi[i] * ((!inverse && signs) ? signs[b0 + i] : 1.0f);
      for (int h = 1; h < block; h <<= 1)
        for (int i = 0; i < block; i += 2 * h)
          for (int j = i; j < i + h; j++) {
            float a = v[j], c = v[j + h];
            v[j] = a + c;
            v[j + h] = a - c;
          }
      float *yo = y + (size_t)r * width + b0;
      for (int i = 0; i < block; i++) yo[i] = v[i] * scale * ((inverse && signs) ? signs[b0 + i] : 1.0f);
    }
  }
  free(v);
}

/* ---------------------------------------------------------------- EXL3 */

/* Single-rounding fp16 helpers: the sum/fma is exact in double, then rounded once. */
static inline uint16_t f16_add(uint16_t a, uint16_t b) {
  double s = (double)ishzo_half_to_float(a) + (double)ishzo_half_to_float(b);
  return ishzo_float_to_half((float)s); /* s exact in double; one float rounding is exact too */
}

/* exl3_decode, Core/EXL3.swift:136-147 (codebooks of exllamav3): a 16-bit trellis state to
   an fp16 weight. 3INST/MCG: scramble, mask to two fp16 values, add them (fp16 rounding).
   MUL1: byte-sum of s*0x83DCD12D into an fp16 of 1024+sum, then fp16 fma(h, c1, c0). */
float ishzo_exl3_decode(uint32_t s, int cb) {
  if (cb == 2) {
    uint32_t x = s * 0x83DCD12Du;
    uint32_t p = (x & 0x00ff00ffu) + ((x >> 8) & 0x00ff00ffu);
    uint16_t h = (uint16_t)((p & 0xffffu) + (p >> 16) + 0x6400u);
    double v = (double)ishzo_half_to_float(h) * (double)ishzo_half_to_float(0x1eee) +
               (double)ishzo_half_to_float(0xc931);
    /* v is exact in double (22-bit product plus an 11-bit addend a few exponents away) */
    return ishzo_half_to_float(ishzo_float_to_half((float)v));
  }
  uint32_t x = cb == 1 ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
  x = (x & 0x8fff8fffu) ^ 0x3b603b60u;
  return ishzo_half_to_float(f16_add((uint16_t)(x & 0xffff), (uint16_t)(x >> 16)));
}

/* Bit position (exclusive end) of weight p's 16-bit state in the tile's ring
   (exl3_end, Core/EXL3.swift:149-151). */
static inline uint32_t exl3_end(uint32_t p, uint32_t ka, int half) {
  return half ? (p >> 1) * (2 * ka + 1) + ka + (p & 1) * (ka + 1) : (p + 1) * ka;
}

/* EXL3Kernels.dequantize + exl3_decode8 (Core/EXL3.swift:168-206, scatter :272-282), restated
   bit by bit: a tile's int16 words pair little-endian into u32 words read as one MSB-first
   ring; weight p (0..255) takes the 16 bits ending at end(p) (wrapping); p = 8*lane + i
   lands at row (lane%4)*2 + {0,1,8,9}[i%4], column lane/4 + 8*(i/4) of the 16x16 tile. */
int ishzo_exl3_dequant(const int16_t *trellis, int K, int N, int bits2, int cb, float *out) {
  if (bits2 < 2 || bits2 > 16 || cb < 0 || cb > 2) return -1;
  int half = bits2 & 1;
  if (half && cb != 2) return -1;
  uint32_t ka = (uint32_t)(bits2 / 2);
  uint32_t ring = half ? 128 * (2 * ka + 1) : 256 * ka;
  int words16 = 8 * bits2; /* 16*bits int16 per tile */
  int tk_n = K / 16, tn_n = N / 16;
  static const int rmap[4] = {0, 1, 8, 9};
#pragma omp parallel for schedule(static)
  for (int tk = 0; tk < tk_n; tk++)
    for (int tn = 0; tn < tn_n; tn++) {
      const uint16_t *t16 = (const uint16_t *)trellis + ((size_t)tk * tn_n + tn) * words16;
      for (uint32_t p = 0; p < 256; p++) {
        uint32_t end = exl3_end(p, ka, half);
        uint32_t st = 0;
        for (int b = 0; b < 16; b++) {
          uint32_t pos = (end + ring - 16 + (uint32_t)b) % ring;
          uint32_t word = (uint32_t)t16[2 * (pos / 32)] | (uint32_t)t16[2 * (pos / 32) + 1] << 16;
          st = (st << 1) | ((word >> (31 - pos % 32)) & 1);
        }
        int lane = (int)p / 8, i = (int)p % 8;
        int row = (lane % 4) * 2 + rmap[i % 4], col = lane / 4 + 8 * (i / 4);
        out[(size_t)(tk * 16 + row) * N + tn * 16 + col] = ishzo_exl3_decode(st, cb);
      }
    }
  return 0;
}

/* EXL3Kernels.apply, Core/EXL3.swift:82-124 (fp16 activations; every cast to x.dtype is an
   fp16 rounding here). */
int ishzo_exl3_apply(const float *x, int M, int K, const int16_t *trellis, const float *suh,
                     const float *svh, int N, int bits2, int cb, float *y, int threads) {
  float *w = (float *)malloc((size_t)K * N * sizeof(float));
  float *xh = (float *)malloc((size_t)M * K * sizeof(float));
  float *yh = (float *)malloc((size_t)M * N * sizeof(float));
  int rc = ishzo_exl3_dequant(trellis, K, N, bits2, cb, w);
  if (!rc) {
    ishzo_hadamard(x, M, K, 128, suh, 0, xh);
    for (size_t i = 0; i < (size_t)M * K; i++) xh[i] = round16(xh[i]);
    set_threads(threads);
#pragma omp parallel
    {
      float *col = (float *)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
      for (int n = 0; n < N; n++) {
        for (int k = 0; k < K; k++) col[k] = w[(size_t)k * N + n];
        for (int m = 0; m < M; m++) {
          float acc = 0.0f;
          for (int k = 0; k < K; k++) acc += xh[(size_t)m * K + k] * col[k];
          yh[(size_t)m * N + n] = acc;
        }
      }
      free(col);
    }
    ishzo_hadamard(yh, M, N, 128, svh, 1, y);
    for (size_t i = 0; i < (size_t)M * N; i++) y[i] = round16(y[i]);
  }
  free(w);
  free(xh);
  free(yh);
  return rc;
}

/* ---------------------------------------------------------------- MoE */

/* MoEBlock.callAsFunction routing, Text/MoEBlock.swift:124-134. */
void ishzo_moe_route(const float *logits, int T, int E, int topk, int normalize, int32_t *ids,
                     float *weights) {
  float *g = (float *)malloc((size_t)E * sizeof(float));
  for (int t = 0; t < T; t++) {
    const float *l = logits + (size_t)t * E;
    float mx = l[0];
    for (int e = 1; e < E; e++) mx = l[e] > mx ? l[e] : mx;
    float sum = 0.0f;
    for (int e = 0; e < E; e++) {
      g[e] = expf(l[e] - mx);
      sum += g[e];
    }
    for (int e = 0; e < E; e++) g[e] /= sum;
    float tot = 0.0f;
    for (int s = 0; s < topk; s++) {
      int best = -1;
      for (int e = 0; e < E; e++) {
        int used = 0;
        for (int q = 0; q < s; q++) used |= ids[(size_t)t * topk + q] == e;
        /* softmax is strictly increasing in the logit, so ranking logits picks the same top-k
           as argPartition over the probabilities, without rounding ties */
        if (!used && (best < 0 || l[e] > l[best])) best = e;
      }
      ids[(size_t)t * topk + s] = best;
      weights[(size_t)t * topk + s] = g[best];
      tot += g[best];
    }
    if (normalize)
      for (int s = 0; s < topk; s++) weights[(size_t)t * topk + s] /= tot;
  }
  free(g);
}

/* ResidentExperts.swiglu + the weighted sum (Text/MoEBlock.swift:147-149,168-171) with fp16
   activations: each projection's output is fp16, silu(g) = g*sigmoid(g) and the product with
   up are fp16 elementwise ops, the weighted sum over slots is fp32 and narrows once. */
int ishzo_moe_swiglu(uint32_t type, const float *x, int T, int H, const int32_t *ids,
                     const float *weights, int topk, const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, int E, int I, const float *shared, const float *shared_gate,
                     float *y, int threads) {
  int bs = ishzo_block_size(type), ts = ishzo_type_size(type);
  if (!bs || H % bs || I % bs) return -1;
  size_t gate_bytes = (size_t)I * (H / bs) * ts, down_bytes = (size_t)H * (I / bs) * ts;
  int P = T * topk;
  float *h = (float *)malloc((size_t)P * I * sizeof(float));
  float *o = (float *)malloc((size_t)P * H * sizeof(float));
  int rc = 0;
  set_threads(threads);
#pragma omp parallel
  {
    float *w = (float *)malloc((size_t)(H > I ? H : I) * sizeof(float));
#pragma omp for schedule(dynamic)
    for (int pi = 0; pi < P; pi++) {
      int t = pi / topk, e = ids[pi];
      if (e < 0 || e >= E) { rc = -2; continue; }
      const float *xt = x + (size_t)t * H;
      size_t rb = (size_t)(H / bs) * ts;
      for (int i = 0; i < I; i++) {
        ishzo_dequant(type, gate + e * gate_bytes + i * rb, rb, (size_t)H, w);
        float g = round16(dot_f32(xt, w, H));
        ishzo_dequant(type, up + e * gate_bytes + i * rb, rb, (size_t)H, w);
        float u = round16(dot_f32(xt, w, H));
        float sg = round16(1.0f / (1.0f + expf(-g)));
        h[(size_t)pi * I + i] = round16(round16(g * sg) * u);
      }
      size_t rd = (size_t)(I / bs) * ts;
      for (int j = 0; j < H; j++) {
        ishzo_dequant(type, down + e * down_bytes + j * rd, rd, (size_t)I, w);
        o[(size_t)pi * H + j] = round16(dot_f32(h + (size_t)pi * I, w, I));
      }
    }
    free(w);
  }
  for (int t = 0; t < T; t++)
    for (int j = 0; j < H; j++) {
      float acc = 0.0f;
      for (int s = 0; s < topk; s++) acc += o[((size_t)t * topk + s) * H + j] * weights[(size_t)t * topk + s];
      /* shared expert (Text/MoEBlock.swift:158-160): sigmoid(sharedGate(x)) in x.dtype, times
         shared(x) in x.dtype, widened and added in fp32 before the one narrowing */
      if (shared && shared_gate)
        acc += round16(round16(1.0f / (1.0f + expf(-shared_gate[t]))) * shared[(size_t)t * H + j]);
      y[(size_t)t * H + j] = round16(acc);
    }
  free(h);
  free(o);
  return rc;
}
