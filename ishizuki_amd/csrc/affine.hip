// MLX affine (2-bit) quantized matmul with the blockwise Walsh-Hadamard rotation, on gfx950.
//
// Replaces the rotated PackedLinear path (Sources/IshizukiKit/Core/Hadamard.swift:180-231):
// hadamardRotate (:8-23), MLX quantizedMM for one row, VerifyMatmul.applyAny for 2..8 rows
// (Core/VerifyMatmul.swift:73-120). Pack format (Quantize/WeightedAffineQuantizer.swift:142-153):
// codes u32 [N][K/16], code k at bits 2*(k%16) of word k/16; scales and biases [N][K/GS];
// w = s*q + b.
//
// Code extraction: masking field i (bits 2i..2i+1, i <= 4) of a word in place, with 0x6400
// above it, gives the fp16 value 1024 + 4^i * c for codes i and i+8 of the word at once; fields
// 5..7 do the same after one shift by 10. The x slot that meets that pair is pre-divided by 4^i
// when x is staged (a power of two, exact), so every product is c * x + 1024 * x' and a single
// accumulator works; the 1024 * sum(x') per group is a constant of x, subtracted once.
#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace ishz {

// Power-of-4 divisor of pair p (0..7) of a word: fields 0..4 in place, 5..7 after >> 10.
DEV float pair_div(int p) { return p < 5 ? (float)(1 << (2 * p)) : (float)(1 << (2 * (p - 5))); }
DEV uint32_t pair_mask(int p) { return 0x00030003u << (2 * (p < 5 ? p : p - 5)); }

DEV float ld_scale(const uint16_t *p, bool bf16) {
  const uint32_t v = *p;
  return bf16 ? __builtin_bit_cast(float, v << 16) : h2f(v);
}

// ------------------------------------------------------------------- Walsh-Hadamard in LDS
// In-place normalised WHT (natural/Sylvester order) of `width` floats in LDS, blocks of `block`
// (power of two), signs applied before (or after, inverse). All threads of the block take part.
DEV void lds_wht(float *v, int width, int block, const float *signs, bool inverse) {
  if (signs && !inverse)
    for (int i = threadIdx.x; i < width; i += blockDim.x) v[i] *= signs[i];
  __syncthreads();
  for (int h = 1; h < block; h <<= 1) {
    for (int p = threadIdx.x; p < width / 2; p += blockDim.x) {
      const int i = ((p & ~(h - 1)) << 1) | (p & (h - 1));  // butterfly (i, i + h), h a power of 2
      const float a = v[i], c = v[i + h];
      v[i] = a + c;
      v[i + h] = a - c;
    }
    __syncthreads();
  }
  const float scale = 1.0f / __builtin_sqrtf((float)block);
  for (int i = threadIdx.x; i < width; i += blockDim.x)
    v[i] = v[i] * scale * ((signs && inverse) ? signs[i] : 1.0f);
  __syncthreads();
}

DEV float load_act(const void *x, size_t i, int dt) {
  if (dt == ISHZ_DT_F32) return ((const float *)x)[i];
  const uint16_t b = ((const uint16_t *)x)[i];
  return dt == ISHZ_DT_F16 ? h2f(b) : __builtin_bit_cast(float, (uint32_t)b << 16);
}
DEV void store_act(void *y, size_t i, int dt, float v) {
  if (dt == ISHZ_DT_F32) {
    ((float *)y)[i] = v;
  } else if (dt == ISHZ_DT_F16) {
    ((uint16_t *)y)[i] = f2h(v);
  } else {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = ((u & 0x7fffffffu) > 0x7f800000u) ? (u | 0x400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    ((uint16_t *)y)[i] = (uint16_t)(u >> 16);
  }
}

// hadamardRotate as a kernel. Blocks up to 128: one wave per 128 contiguous values, two per
// lane, butterflies across lanes by shuffles (stages above the block size skipped). Larger
// blocks: one workgroup per block, in LDS. fp32 math, output in `out_dt`.
__global__ __launch_bounds__(256) void hadamard_wave_kernel(const void *__restrict__ x, int in_dt,
                                                            size_t chunks, int width, int block,
                                                            const float *__restrict__ signs,
                                                            int inverse, void *__restrict__ y,
                                                            int out_dt) {
  const size_t c = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= chunks) return;
  const int lane = threadIdx.x & 63;
  const size_t base = c * 128 + 2 * lane;
  const int col = (int)(base % width);
  float v0 = load_act(x, base, in_dt), v1 = load_act(x, base + 1, in_dt);
  if (signs && !inverse) {
    v0 *= signs[col];
    v1 *= signs[col + 1];
  }
  if (block >= 2) {
    const float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
  }
  for (int m = 1; 2 * m < block; m <<= 1) {
    const float p0 = __shfl_xor(v0, m, 64), p1 = __shfl_xor(v1, m, 64);
    const bool hi = (lane & m) != 0;
    v0 = hi ? p0 - v0 : v0 + p0;
    v1 = hi ? p1 - v1 : v1 + p1;
  }
  const float scale = 1.0f / __builtin_sqrtf((float)block);
  v0 *= scale;
  v1 *= scale;
  if (signs && inverse) {
    v0 *= signs[col];
    v1 *= signs[col + 1];
  }
  store_act(y, base, out_dt, v0);
  store_act(y, base + 1, out_dt, v1);
}

__global__ __launch_bounds__(256) void hadamard_kernel(const void *__restrict__ x, int in_dt,
                                                       int width, int block,
                                                       const float *__restrict__ signs,
                                                       int inverse, void *__restrict__ y,
                                                       int out_dt) {
  extern __shared__ float hv[];
  const size_t base = (size_t)blockIdx.x * block;
  const int col = (int)(base % width);
  for (int i = threadIdx.x; i < block; i += blockDim.x) hv[i] = load_act(x, base + i, in_dt);
  lds_wht(hv, block, block, signs ? signs + col : nullptr, inverse != 0);
  for (int i = threadIdx.x; i < block; i += blockDim.x) store_act(y, base + i, out_dt, hv[i]);
}

// ------------------------------------------------------------------- GEMV (M = 1)
// Unit = 64 weights = 16 bytes of codes (4 words) of one row; LPR lanes per row, 64/LPR rows per
// wave, waves take equal shares of row groups and ping-pong two register batches of units (the
// same streaming scheme as the GGML GEMV). With ROT, x is rotated in LDS before staging.
constexpr int AFF_B = 4;  // units per batch

struct AffRaw {
  u4 q;
  uint32_t s, b;
};

template <int GS, int LPR, bool ROT>
__global__ __launch_bounds__(256) void affine_gemv(const uint16_t *__restrict__ x,
                                                   const float *__restrict__ signs, int block,
                                                   const uint32_t *__restrict__ codes,
                                                   const uint16_t *__restrict__ scales,
                                                   const uint16_t *__restrict__ biases, int bf16s,
                                                   int K, int N, uint16_t *__restrict__ y,
                                                   int groups_per_wave) {
  extern __shared__ __align__(16) uint32_t smem[];
  const int units = K / 64;
  const int ug = (units + 15) / 16;
  u4 *slots = (u4 *)smem;                      // ug*16*8 slots (R = 8)
  float *sums = (float *)(slots + ug * 16 * 8);  // ug*16*2 (C offset, X plain)
  float *xr = sums + ug * 16 * 2;              // K floats (rotated x), ROT only

  constexpr int RPW = 64 / LPR, B = AFF_B;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPR, rg = lane / LPR;
  const int nb = (units + B * LPR - 1) / (B * LPR);
  const int gpr = K / GS;
  const int gw = blockIdx.x * (blockDim.x >> 6) + wave;
  const int g_end = min((gw + 1) * groups_per_wave, (N + RPW - 1) / RPW);
  const int g_last = max(g_end - 1, 0);

  auto load_batch = [&](int g, int bi, AffRaw *r) {
    const int row = min(min(g, g_last) * RPW + rg, N - 1);
    const uint32_t *cr = codes + (size_t)row * (K / 16);
    const uint16_t *sr = scales + (size_t)row * gpr, *br = biases + (size_t)row * gpr;
#pragma unroll
    for (int i = 0; i < B; i++) {
      const int u = min(sub + (bi * B + i) * LPR, units - 1);
      r[i].q = *(const u4 *)(cr + 4 * u);
      r[i].s = sr[(64 * u) / GS];
      r[i].b = br[(64 * u) / GS];
    }
  };
  int g = gw * groups_per_wave, bi = 0;
  AffRaw cur[B], alt[B];
  load_batch(g, 0, cur);

  // ---- stage x (rotated first when ROT): slots of x / 4^i, per-unit offset and plain sums
  if constexpr (ROT) {
    for (int i = threadIdx.x; i < K; i += blockDim.x) xr[i] = h2f(x[i]);
    lds_wht(xr, K, block, signs, false);
    for (int i = threadIdx.x; i < K; i += blockDim.x) xr[i] = (float)(_Float16)xr[i];  // x.dtype
    __syncthreads();
  }
  auto xv = [&](int k) -> float { return ROT ? xr[k] : h2f(x[k]); };
  for (int i = threadIdx.x; i < ug * 16 * 8; i += blockDim.x) {
    const int u = (i / 128) * 16 + (i & 15), r = (i >> 4) & 7;  // slot r = word t = r/2, half
    if (u < units) {
      const int t = r >> 1, p0 = (r & 1) * 4, kw = 64 * u + 16 * t;
      uint32_t d[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int e = -2 * ((p0 + j) < 5 ? (p0 + j) : (p0 + j) - 5);  // x / 4^i, exact
        d[j] = (uint32_t)f2h(__builtin_ldexpf(xv(kw + p0 + j), e)) |
               (uint32_t)f2h(__builtin_ldexpf(xv(kw + p0 + j + 8), e)) << 16;
      }
      slots[i] = u4{d[0], d[1], d[2], d[3]};
    }
  }
  __syncthreads();
  // Per unit: C = 1024 * sum of its 64 staged x' (the code offset) and X = sum of x (for the
  // bias), read back from the slots in a fixed order.
  for (int i = threadIdx.x; i < ug * 16; i += blockDim.x) {
    const int u = (i / 16) * 16 + (i & 15);
    if (u < units) {
      const u4 *sl = slots + (u >> 4) * 128 + (u & 15);
      float c = 0.0f, xs = 0.0f;
#pragma unroll
      for (int r = 0; r < 8; r++) {
        const u4 v = sl[r * 16];
#pragma unroll
        for (int d = 0; d < 4; d++) {
          const int p = (r & 1) * 4 + d;
          const h2 hv = as_h2(v[d]);
          const float pr = (float)hv.x + (float)hv.y;
          c += pr;
          xs += __builtin_ldexpf(pr, 2 * (p < 5 ? p : p - 5));
        }
      }
      float *sm = sums + (u >> 4) * 32 + (u & 15);
      sm[0] = 1024.0f * c;
      sm[16] = xs;
    }
  }
  __syncthreads();
  const uint32_t mg = vconst(0x64006400u);

  float acc = 0.0f;
  auto advance = [&](int &gg, int &bb) {
    if (++bb == nb) {
      bb = 0;
      gg++;
    }
  };
  auto consume = [&](int gg, int bb, const AffRaw *r) {
#pragma unroll
    for (int i = 0; i < B; i++) {
      const int u0 = sub + (bb * B + i) * LPR, u = min(u0, units - 1);
      const u4 *sl = slots + (u >> 4) * 128 + (u & 15);
      float S = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t w = r[i].q[t], w10 = w >> 10;
        const u4 a = sl[(2 * t) * 16], c = sl[(2 * t + 1) * 16];
        S = dot2(and_or(w, 0x00030003u, mg), a.x, S);
        S = dot2(and_or(w, 0x000C000Cu, mg), a.y, S);
        S = dot2(and_or(w, 0x00300030u, mg), a.z, S);
        S = dot2(and_or(w, 0x00C000C0u, mg), a.w, S);
        S = dot2(and_or(w, 0x03000300u, mg), c.x, S);
        S = dot2(and_or(w10, 0x00030003u, mg), c.y, S);
        S = dot2(and_or(w10, 0x000C000Cu, mg), c.z, S);
        S = dot2(and_or(w10, 0x00300030u, mg), c.w, S);
      }
      const float *sm = sums + (u >> 4) * 32 + (u & 15);
      const float v = ld_scale((const uint16_t *)&r[i].s, bf16s) * (S - sm[0]) +
                      ld_scale((const uint16_t *)&r[i].b, bf16s) * sm[16];
      acc += u0 < units ? v : 0.0f;
    }
    if (bb == nb - 1) {
      acc = group_sum<LPR>(acc);
      const int row = gg * RPW + rg;
      if (sub == 0 && row < N) y[row] = f2h(acc);
      acc = 0.0f;
    }
  };
  while (g < g_end) {
    int g1 = g, b1 = bi;
    advance(g1, b1);
    load_batch(g1, b1, alt);
    consume(g, bi, cur);
    if (g1 >= g_end) break;
    int g2 = g1, b2 = b1;
    advance(g2, b2);
    load_batch(g2, b2, cur);
    consume(g1, b1, alt);
    g = g2;
    bi = b2;
  }
}

// ------------------------------------------------------------------- verify (MFMA, M <= 16)
// Tokens are the A operand, decoded codes the B operand (see the GGML verify kernel). One group
// of 64 = two MFMA 16x16x32 steps; in step s lane group g takes pairs 4s..4s+3 of word g. B is
// the raw masked pairs (1024 + 4^i c); A is x divided to match. Per group and token, C - 1024 *
// sum(A) is sum(c x), and sum(x) (for the bias) comes from an MFMA against ones.
template <int GS, int T>
__global__ __launch_bounds__(1024) void affine_verify(const uint16_t *__restrict__ x, int M, int K,
                                                      const uint32_t *__restrict__ codes,
                                                      const uint16_t *__restrict__ scales,
                                                      const uint16_t *__restrict__ biases,
                                                      int bf16s, int N, uint16_t *__restrict__ y) {
  extern __shared__ __align__(16) float red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int groups = K / 64, gpr = K / GS;
  const int n0 = blockIdx.x * 16 * T;
  const bool tok = j < M;
  const uint16_t *xr = x + (size_t)(tok ? j : 0) * K;
  const uint32_t mg = vconst(0x64006400u);
  const h8 ones = as_h8(u4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});

  f4 acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = f4{0, 0, 0, 0};
  for (int G = wave; G < groups; G += KS) {
    // A operands for the group's two steps: x[16g + 4s + i] and x[16g + 4s + 8 + i], i < 4
    h8 Ap[2], Ax[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int kb = 64 * G + 16 * g + 4 * s;
      const u2 lo = tok ? *(const u2 *)(xr + kb) : u2{0, 0};
      const u2 hi = tok ? *(const u2 *)(xr + kb + 8) : u2{0, 0};
      const uint16_t l4[4] = {(uint16_t)lo.x, (uint16_t)(lo.x >> 16), (uint16_t)lo.y, (uint16_t)(lo.y >> 16)};
      const uint16_t h4v[4] = {(uint16_t)hi.x, (uint16_t)(hi.x >> 16), (uint16_t)hi.y, (uint16_t)(hi.y >> 16)};
      u4 ap, ax;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int p = 4 * s + i;
        const _Float16 inv = (_Float16)(1.0f / pair_div(p));
        const _Float16 a = __builtin_bit_cast(_Float16, l4[i]), b = __builtin_bit_cast(_Float16, h4v[i]);
        ap[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(a * inv)) |
                (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(b * inv)) << 16;
        ax[i] = (uint32_t)l4[i] | (uint32_t)h4v[i] << 16;
      }
      Ap[s] = as_h8(ap);
      Ax[s] = as_h8(ax);
    }
    f4 off = mfma32(Ap[0], ones, f4{0, 0, 0, 0});
    off = mfma32(Ap[1], ones, off);
    f4 xs = mfma32(Ax[0], ones, f4{0, 0, 0, 0});
    xs = mfma32(Ax[1], ones, xs);
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int row = min(n0 + 16 * t + j, N - 1);
      const uint32_t w = codes[(size_t)row * (K / 16) + 4 * G + g], w10 = w >> 10;
      const u4 b0 = {and_or(w, 0x00030003u, mg), and_or(w, 0x000C000Cu, mg),
                     and_or(w, 0x00300030u, mg), and_or(w, 0x00C000C0u, mg)};
      const u4 b1 = {and_or(w, 0x03000300u, mg), and_or(w10, 0x00030003u, mg),
                     and_or(w10, 0x000C000Cu, mg), and_or(w10, 0x00300030u, mg)};
      f4 c = mfma32(Ap[0], as_h8(b0), f4{0, 0, 0, 0});
      c = mfma32(Ap[1], as_h8(b1), c);
      const size_t gi = (size_t)row * gpr + (64 * G) / GS;
      const float sc = ld_scale(scales + gi, bf16s != 0), bi = ld_scale(biases + gi, bf16s != 0);
      acc[t] += sc * (c - 1024.0f * off) + bi * xs;
    }
  }
#pragma unroll
  for (int t = 0; t < T; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) red[((wave * T + t) * 4 + r) * 64 + lane] = acc[t][r];
  __syncthreads();
  for (int o = threadIdx.x; o < T * 256; o += blockDim.x) {
    const int t = o >> 8, r = (o >> 6) & 3, l = o & 63;
    float s = 0.0f;
    for (int v = 0; v < KS; v++) s += red[((v * T + t) * 4 + r) * 64 + l];
    const int tk = 4 * (l >> 4) + r, n = n0 + 16 * t + (l & 15);
    if (tk < M && n < N) y[(size_t)tk * N + n] = f2h(s);
  }
}

// ------------------------------------------------------------------- host
static int num_cu_aff() {
  static int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      return v;
    return 256;
  }();
  return n;
}

static bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

template <int GS, int LPR, bool ROT>
static int launch_affine_gemv(const void *x, const float *signs, int block, const uint32_t *codes,
                              const void *scales, const void *biases, int bf16s, int K, int N,
                              void *y, hipStream_t st) {
  constexpr int RPW = 64 / LPR;
  const int groups = (N + RPW - 1) / RPW;
  const int capacity = num_cu_aff() * 4 * 4;
  const int per_wave = (groups + capacity - 1) / capacity;
  const int waves = (groups + per_wave - 1) / per_wave;
  const size_t ug = (size_t)(K / 64 + 15) / 16;
  const size_t lds = ug * 16 * 8 * 16 + ug * 16 * 2 * 4 + (ROT ? (size_t)K * 4 : 0);
  if (lds > 160 * 1024) return decline("K too large for the affine GEMV's LDS");
  hipLaunchKernelGGL((affine_gemv<GS, LPR, ROT>), dim3((waves + 3) / 4), dim3(256), lds, st,
                     (const uint16_t *)x, signs, block, codes, (const uint16_t *)scales,
                     (const uint16_t *)biases, bf16s, K, N, (uint16_t *)y, per_wave);
  ISHZ_LAUNCH_CHECK("affine gemv launch");
  return ISHZ_OK;
}

template <int GS, bool ROT>
static int affine_gemv_lpr(const void *x, const float *signs, int block, const uint32_t *codes,
                           const void *scales, const void *biases, int bf16s, int K, int N,
                           void *y, hipStream_t st) {
  const int units = K / 64;
  if (units <= 32)
    return launch_affine_gemv<GS, 8, ROT>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
  if (units <= 128)
    return launch_affine_gemv<GS, 16, ROT>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
  return launch_affine_gemv<GS, 32, ROT>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
}

template <int GS>
static int affine_verify_launch(const void *x, int M, int K, const uint32_t *codes,
                                const void *scales, const void *biases, int bf16s, int N, void *y,
                                hipStream_t st) {
  constexpr int T = 2;
  const int wgs = (N + 16 * T - 1) / (16 * T);
  const int groups = K / 64;
  int ks = 1;
  while (ks < 16 && ks < groups && wgs * ks < num_cu_aff() * 16) ks *= 2;
  hipLaunchKernelGGL((affine_verify<GS, T>), dim3(wgs), dim3(64 * ks), (size_t)ks * T * 256 * 4, st,
                     (const uint16_t *)x, M, K, codes, (const uint16_t *)scales,
                     (const uint16_t *)biases, bf16s, N, (uint16_t *)y);
  ISHZ_LAUNCH_CHECK("affine verify launch");
  return ISHZ_OK;
}

static int check_affine(const void *x, int x_dtype, int M, int K, const void *codes,
                        const void *scales, const void *biases, int scale_dtype, int N, int bits,
                        int group, const void *y) {
  if (x_dtype != ISHZ_DT_F16) return decline("activations must be fp16");
  if (bits != 2) return decline("only 2-bit packs are decoded in-kernel");
  if (group != 64 && group != 128) return decline("group size must be 64 or 128");
  if (scale_dtype != ISHZ_DT_F16 && scale_dtype != ISHZ_DT_BF16) return decline("scales must be fp16 or bf16");
  if (M < 1 || M > 16) return decline("row count outside 1..16");
  if (K <= 0 || K % 128 || N <= 0) return decline("K must be a positive multiple of 128");
  if (!x || !codes || !scales || !biases || !y) return einval("null pointer");
  return ISHZ_OK;
}

static int affine_dispatch(const void *x, int M, int K, const float *signs, int block,
                           const uint32_t *codes, const void *scales, const void *biases,
                           int bf16s, int N, int group, void *y, hipStream_t st) {
  const bool rot = block > 0;
  if (M == 1) {
    if (group == 64)
      return rot ? affine_gemv_lpr<64, true>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st)
                 : affine_gemv_lpr<64, false>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
    return rot ? affine_gemv_lpr<128, true>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st)
               : affine_gemv_lpr<128, false>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
  }
  return group == 64 ? affine_verify_launch<64>(x, M, K, codes, scales, biases, bf16s, N, y, st)
                     : affine_verify_launch<128>(x, M, K, codes, scales, biases, bf16s, N, y, st);
}

}  // namespace ishz

using namespace ishz;

extern "C" int ishz_hadamard(const void *x, int dtype, int rows, int width, int block,
                             const float *signs, int inverse, void *y, ishz_stream_t stream) {
  if (dtype < ISHZ_DT_F32 || dtype > ISHZ_DT_BF16) return decline("unsupported dtype");
  if (!pow2(block) || block > 4096) return decline("block must be a power of two <= 4096");
  if (rows <= 0 || width <= 0 || width % block) return einval("block does not divide the width");
  if (!x || !y) return einval("null pointer");
  if (block <= 128) {
    if (width % 128) return decline("width must be a multiple of 128 for blocks up to 128");
    const size_t chunks = (size_t)rows * width / 128;
    hipLaunchKernelGGL(hadamard_wave_kernel, dim3((unsigned)((chunks + 3) / 4)), dim3(256), 0, S(stream), x,
                       dtype, chunks, width, block, signs, inverse, y, dtype);
  } else {
    hipLaunchKernelGGL(hadamard_kernel, dim3((unsigned)((size_t)rows * width / block)), dim3(256),
                       (size_t)block * 4, S(stream), x, dtype, width, block, signs, inverse, y, dtype);
  }
  ISHZ_LAUNCH_CHECK("hadamard launch");
  return ISHZ_OK;
}

extern "C" int ishz_affine_matmul(const void *x, int x_dtype, int M, int K, const uint32_t *codes,
                                  const void *scales, const void *biases, int scale_dtype, int N,
                                  int bits, int group, void *y, ishz_stream_t stream) {
  int rc = check_affine(x, x_dtype, M, K, codes, scales, biases, scale_dtype, N, bits, group, y);
  if (rc) return rc;
  return affine_dispatch(x, M, K, nullptr, 0, codes, scales, biases, scale_dtype == ISHZ_DT_BF16, N,
                         group, y, S(stream));
}

extern "C" size_t ishz_affine_workspace_size(int M, int K) {
  return M > 1 ? (size_t)M * K * 2 : 0;
}

extern "C" int ishz_affine_linear(const void *x, int x_dtype, int M, int K, const float *signs,
                                  int block, const uint32_t *codes, const void *scales,
                                  const void *biases, int scale_dtype, int N, int bits, int group,
                                  void *y, void *workspace, size_t workspace_bytes,
                                  ishz_stream_t stream) {
  int rc = check_affine(x, x_dtype, M, K, codes, scales, biases, scale_dtype, N, bits, group, y);
  if (rc) return rc;
  if (block > 0 && (!pow2(block) || block > 4096 || K % block)) return decline("bad Hadamard block");
  const int bf16s = scale_dtype == ISHZ_DT_BF16;
  hipStream_t st = S(stream);
  if (block == 0 || M == 1)
    return affine_dispatch(x, M, K, signs, block, codes, scales, biases, bf16s, N, group, y, st);
  if (!workspace || workspace_bytes < ishz_affine_workspace_size(M, K))
    return einval("workspace too small (ishz_affine_workspace_size)");
  rc = ishz_hadamard(x, ISHZ_DT_F16, M, K, block, signs, 0, workspace, stream);
  if (rc) return rc;
  return affine_dispatch(workspace, M, K, nullptr, 0, codes, scales, biases, bf16s, N, group, y, st);
}
