// GGML quantized matmul on gfx950: streaming GEMV (M = 1), MFMA verify (M = 2..16), dequant and
// gather writers. Replaces GGMLKernels (Sources/IshizukiKit/Core/GGMLKernels.swift).
#include "ggml_formats.h"
#include "vgemm.h"
#include "precise.h"

#include <cstdlib>

#define ISHZ_TABLE_QUAL static __device__
#include "ggml_grids.inc"
#include "ggml_iq.h"

namespace ishz {

// ----------------------------------------------------------------------------- tables in LDS
// IQ2_XS grid entries as fp16 (values 8, 25, 43), either in the permuted pair order of the GEMV
// (x0,x2,x1,x3,...) or in natural order for the MFMA B operand; with `sgn`, also the 128 sign
// patterns of ksigns (index | parity << 7) as natural-order fp16 sign-bit masks (the GEMV computes
// its masks in registers).
template <bool PERM>
DEV void build_iq2xs_tables(u4 *grid, u4 *sgn) {
  for (int e = threadIdx.x; e < 512 + (sgn ? 128 : 0); e += blockDim.x) {
    if (e < 512) {
      const uint64_t v = ishz_iq2xs_grid[e];
      uint32_t hv[8];
#pragma unroll
      for (int j = 0; j < 8; j++) hv[j] = f2h((float)((v >> (8 * j)) & 0xff));
      grid[e] = PERM ? u4{hv[0] | hv[2] << 16, hv[1] | hv[3] << 16, hv[4] | hv[6] << 16,
                          hv[5] | hv[7] << 16}
                     : u4{hv[0] | hv[1] << 16, hv[2] | hv[3] << 16, hv[4] | hv[5] << 16,
                          hv[6] | hv[7] << 16};
    } else {
      const int i = e - 512;
      const uint32_t s = (uint32_t)i | (uint32_t)(__builtin_popcount(i) & 1) << 7;
      auto bit = [&](int j) { return ((s >> j) & 1u) << 15; };
      sgn[i] = u4{bit(0) | bit(1) << 16, bit(2) | bit(3) << 16, bit(4) | bit(5) << 16, bit(6) | bit(7) << 16};
    }
  }
}

DEV void build_iq2xs_tables_perm(u4 *grid, u4 *sgn) { build_iq2xs_tables<true>(grid, sgn); }
DEV void build_iq2xs_tables_nat(u4 *grid, u4 *sgn) { build_iq2xs_tables<false>(grid, sgn); }

// ----------------------------------------------------------------------------- verify (MFMA)
// A workgroup owns T tiles of 16 weight rows; its KS waves split the row's blocks round-robin
// and their partial 16x16 C tiles are summed through LDS at the end.
template <class F, int T>
__global__ __launch_bounds__(1024) void verify_kernel(const uint16_t *__restrict__ x, int M, int K,
                                                      const uint8_t *__restrict__ w, int N, Out y) {
  extern __shared__ __align__(16) uint32_t vsm[];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  u4 *grid = (u4 *)vsm, *sgn = grid + 512;
  float *red = (float *)(vsm + (F::GRID ? (512 + 128) * 4 : 0));
  if constexpr (F::GRID) {
    build_iq2xs_tables<false>(grid, sgn);
    __syncthreads();
  }

  const int nblk = K / F::BS;
  const size_t rb = (size_t)nblk * F::TS;
  const int n0 = blockIdx.x * 16 * T;
  const uint8_t *rows[T];
#pragma unroll
  for (int t = 0; t < T; t++) rows[t] = w + (size_t)min(n0 + 16 * t + j, N - 1) * rb;
  const bool tok = j < M;
  const uint16_t *xr = x + (size_t)(tok ? j : 0) * K;

  f4 acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = f4{0, 0, 0, 0};
  for (int b = wave; b < nblk; b += KS) {
    if constexpr (F::GRID)
      F::template vblock_lds<T>(rows, b, g, xr, tok, acc, (const u2 *)grid, (const u2 *)sgn);
    else
      F::template vblock<T>(rows, b, g, xr, tok, acc);
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
    if (tk < M && n < N) y.put((size_t)tk * N + n, tk, s);
  }
}

// ----------------------------------------------------------------------------- dequant/gather
// Scalar restatement of the CPU decoder per 8-element slice (the same fp32 operations in the
// same order, so the values written are the reference's own), used by the expand and gather
// writers. Slice e of a block covers elements 8e .. 8e+7.
#pragma clang fp contract(off)
template <uint32_t TYPE>
DEV void decode8(const uint8_t *p, int e, float *v) {
  if constexpr (TYPE == ISHZ_GGML_Q4_0) {
    const float d = h2f(ld2(p));
    const int j0 = (e & 1) * 8, hi = e >> 1;
    for (int i = 0; i < 8; i++) {
      const int q = hi ? p[2 + j0 + i] >> 4 : p[2 + j0 + i] & 15;
      v[i] = (float)(q - 8) * d;
    }
  } else if constexpr (TYPE == ISHZ_GGML_Q4_K) {
    const float d = h2f(ld2(p)), dmin = h2f(ld2(p + 2));
    const int k = 8 * e, jj = k / 64, hi = (k / 32) & 1, l0 = k & 31;
    const uint32_t s0 = ld4<4>(p + 4), s1 = ld4<4>(p + 8), s2 = ld4<4>(p + 12);
    int sc, m;
    q4k_scale_min(s0, s1, s2, 2 * jj + hi, sc, m);
    const float dl = d * (float)sc, ml = dmin * (float)m;
    for (int i = 0; i < 8; i++) {
      const uint8_t q = p[16 + 32 * jj + l0 + i];
      v[i] = dl * (float)(hi ? q >> 4 : q & 15) - ml;
    }
  } else if constexpr (TYPE == ISHZ_GGML_Q6_K) {
    const float d = h2f(ld2(p + 208));
    const int k = 8 * e, n = k / 128, qq = (k / 32) & 3, l0 = k & 31;
    const float scl = (float)(int8_t)p[192 + 8 * n + l0 / 16 + 2 * qq];
    for (int i = 0; i < 8; i++) {
      const int l = l0 + i;
      const uint8_t ql = p[64 * n + 32 * (qq & 1) + l], qh = p[128 + 32 * n + l];
      const int q = ((qq >> 1) ? ql >> 4 : ql & 15) | ((qh >> (2 * qq)) & 3) << 4;
      v[i] = d * scl * (float)(q - 32);
    }
  } else if constexpr (TYPE == ISHZ_GGML_IQ2_XS) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint8_t sc = p[66 + ib];
    const float db = d * (0.5f + (float)((l < 2) ? (sc & 15) : (sc >> 4))) * 0.25f;
    const uint32_t q = ld2(p + 2 + 2 * (4 * ib + l));
    const uint64_t ent = ishz_iq2xs_grid[q & 511];
    const uint32_t s = (q >> 9) | (__builtin_popcount(q >> 9) & 1) << 7;
    for (int i = 0; i < 8; i++)
      v[i] = db * (float)((ent >> (8 * i)) & 0xff) * (((s >> i) & 1) ? -1.0f : 1.0f);
  } else if constexpr (TYPE == ISHZ_GGML_Q2_K) {
    // weights 128n + 32s + 16 lane + l: bits 2s of qs[32n + 16 lane + l], scale byte 8n + 2s + lane
    const float d = h2f(ld2(p + 80)), dmin = h2f(ld2(p + 82));
    const int k = 8 * e, n = k / 128, s = (k / 32) & 3, ln = (k / 16) & 1, l0 = k & 15;
    const uint8_t sc = p[8 * n + 2 * s + ln];
    const float dl = d * (float)(sc & 0xf), ml = dmin * (float)(sc >> 4);
    for (int i = 0; i < 8; i++) v[i] = dl * (float)((p[16 + 32 * n + 16 * ln + l0 + i] >> (2 * s)) & 3) - ml;
  } else if constexpr (TYPE == ISHZ_GGML_IQ4_XS) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, j0 = (e & 1) * 8, hi = (e >> 1) & 1;
    const int lo = (p[4 + ib / 2] >> (4 * (ib % 2))) & 0xf, hb = ((ld2(p + 2) >> (2 * ib)) & 3) << 4;
    const float dl = d * (float)((lo | hb) - 32);
    for (int i = 0; i < 8; i++) {
      const uint8_t q = p[8 + 16 * ib + j0 + i];
      v[i] = dl * (float)ishz_kvalues_iq4nl[hi ? q >> 4 : q & 0xf];
    }
  } else if constexpr (TYPE == ISHZ_GGML_IQ2_XXS) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint32_t a1 = ld2(p + 2 + 8 * ib) | ld2(p + 4 + 8 * ib) << 16;
    const uint32_t a2 = ld2(p + 6 + 8 * ib) | ld2(p + 8 + 8 * ib) << 16;
    const float db = d * (0.5f + (float)(a2 >> 28)) * 0.25f;
    const uint64_t ent = ishz_iq2xxs_grid[(a1 >> (8 * l)) & 0xff];
    const uint32_t q7 = (a2 >> (7 * l)) & 127, s = q7 | (__builtin_popcount(q7) & 1) << 7;
    for (int i = 0; i < 8; i++)
      v[i] = db * (float)((ent >> (8 * i)) & 0xff) * (((s >> i) & 1) ? -1.0f : 1.0f);
  } else if constexpr (TYPE == ISHZ_GGML_IQ2_S) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint8_t sc = p[74 + ib];
    const float db = d * (0.5f + (float)(l < 2 ? (sc & 0xf) : (sc >> 4))) * 0.25f;
    const int idx = p[2 + 4 * ib + l] | ((p[66 + ib] << (8 - 2 * l)) & 0x300);
    const uint64_t ent = ishz_iq2s_grid[idx];
    const uint8_t s = p[34 + 4 * ib + l];
    for (int i = 0; i < 8; i++)
      v[i] = db * (float)((ent >> (8 * i)) & 0xff) * (((s >> i) & 1) ? -1.0f : 1.0f);
  } else if constexpr (TYPE == ISHZ_GGML_IQ3_XXS) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint32_t aux = ld2(p + 66 + 4 * ib) | ld2(p + 68 + 4 * ib) << 16;
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    const uint32_t q7 = (aux >> (7 * l)) & 127, s = q7 | (__builtin_popcount(q7) & 1) << 7;
    const uint32_t g1 = ishz_iq3xxs_grid[p[2 + 8 * ib + 2 * l]], g2 = ishz_iq3xxs_grid[p[3 + 8 * ib + 2 * l]];
    for (int i = 0; i < 8; i++) {
      const uint32_t gv = i < 4 ? (g1 >> (8 * i)) & 0xff : (g2 >> (8 * (i - 4))) & 0xff;
      v[i] = db * (float)gv * (((s >> i) & 1) ? -1.0f : 1.0f);
    }
  } else if constexpr (TYPE == ISHZ_GGML_IQ3_S) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint8_t sc = p[106 + ib / 2];
    const float db = d * (float)(1 + 2 * ((ib & 1) ? (sc >> 4) : (sc & 0xf)));
    const int qh = p[66 + ib];
    const uint8_t *qs = p + 2 + 8 * ib;
    const uint32_t g1 = ishz_iq3s_grid[qs[2 * l] | ((qh << (8 - 2 * l)) & 256)];
    const uint32_t g2 = ishz_iq3s_grid[qs[2 * l + 1] | ((qh << (7 - 2 * l)) & 256)];
    const uint8_t s = p[74 + 4 * ib + l];
    for (int i = 0; i < 8; i++) {
      const uint32_t gv = i < 4 ? (g1 >> (8 * i)) & 0xff : (g2 >> (8 * (i - 4))) & 0xff;
      v[i] = db * (float)gv * (((s >> i) & 1) ? -1.0f : 1.0f);
    }
  } else if constexpr (TYPE == ISHZ_GGML_IQ1_S) {
    const float d = h2f(ld2(p));
    const int ib = e / 4, l = e & 3;
    const uint32_t qh = ld2(p + 34 + 2 * ib);
    const float dl = d * (float)(2 * ((qh >> 12) & 7) + 1);
    const float delta = (qh & 0x8000) ? -0.125f : 0.125f;
    const uint64_t ent = ishz_iq1s_grid[p[2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)];
    for (int i = 0; i < 8; i++) v[i] = dl * ((float)(int8_t)((ent >> (8 * i)) & 0xff) + delta);
  } else if constexpr (TYPE == ISHZ_GGML_IQ1_M) {
    const uint32_t s0 = ld2(p + 48), s1 = ld2(p + 50), s2 = ld2(p + 52), s3 = ld2(p + 54);
    const float d = h2f((s0 >> 12) | ((s1 >> 8) & 0x00f0) | ((s2 >> 4) & 0x0f00) | (s3 & 0xf000));
    const int ib = e / 4, l = e & 3;
    const uint32_t w = ld2(p + 48 + 2 * (ib / 2));
    const int shift = 6 * (ib % 2) + (l < 2 ? 0 : 3);
    const float dl = d * (float)(2 * ((w >> shift) & 7) + 1);
    const int qb = p[32 + 2 * ib + (l >> 1)];
    const int idx = p[4 * ib + l] | (((l & 1) ? (qb >> 4) : qb) & 7) << 8;
    const float delta = (qb & ((l & 1) ? 0x80 : 0x08)) ? -0.125f : 0.125f;
    const uint64_t ent = ishz_iq1s_grid[idx];
    for (int i = 0; i < 8; i++) v[i] = dl * ((float)(int8_t)((ent >> (8 * i)) & 0xff) + delta);
  }
}
#pragma clang fp contract(on)

DEV uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

DEV void store8(void *out, size_t idx, int dt, const float *v) {
  if (dt == ISHZ_DT_F32) {
    f4 *o = (f4 *)((float *)out + idx);
    o[0] = f4{v[0], v[1], v[2], v[3]};
    o[1] = f4{v[4], v[5], v[6], v[7]};
  } else {
    uint32_t h[4];
    for (int i = 0; i < 4; i++)
      h[i] = dt == ISHZ_DT_F16 ? (uint32_t)f2h(v[2 * i]) | (uint32_t)f2h(v[2 * i + 1]) << 16
                               : (uint32_t)f2bf(v[2 * i]) | (uint32_t)f2bf(v[2 * i + 1]) << 16;
    *(u4 *)((uint16_t *)out + idx) = u4{h[0], h[1], h[2], h[3]};
  }
}

template <uint32_t TYPE, int BS, int TS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w, size_t nslices,
                                                      void *out, int dt) {
  for (size_t s = blockIdx.x * (size_t)blockDim.x + threadIdx.x; s < nslices;
       s += (size_t)gridDim.x * blockDim.x) {
    const size_t blk = s / (BS / 8);
    const int e = (int)(s % (BS / 8));
    float v[8];
    decode8<TYPE>(w + blk * TS, e, v);
    store8(out, s * 8, dt, v);
  }
}

template <uint32_t TYPE, int BS, int TS>
__global__ __launch_bounds__(256) void gather_kernel(const int32_t *__restrict__ ids, int n_ids,
                                                     const uint8_t *__restrict__ w, int n_rows,
                                                     int K, void *out, int dt) {
  const size_t per_row = (size_t)K / 8, total = per_row * n_ids;
  const size_t rb = (size_t)(K / BS) * TS;
  for (size_t s = blockIdx.x * (size_t)blockDim.x + threadIdx.x; s < total;
       s += (size_t)gridDim.x * blockDim.x) {
    const int slot = (int)(s / per_row);
    const int k8 = (int)(s % per_row);
    const int id = ids[slot];
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (id >= 0 && id < n_rows) decode8<TYPE>(w + (size_t)id * rb + (size_t)(k8 * 8 / BS) * TS, k8 % (BS / 8), v);
    store8(out, s * 8, dt, v);
  }
}

// fp32 activations (precise.h): a row's slices decoded by decode8, the CPU decoder's values.
template <uint32_t TYPE, int BS, int TS>
struct GgmlDec {
  struct Args {
    const uint8_t *w;
    size_t rb;  // bytes per row
  };
  static DEV void decode(const Args &a, int row, int s, float *v) {
    decode8<TYPE>(a.w + (size_t)row * a.rb + (size_t)(s * 8 / BS) * TS, s % (BS / 8), v);
  }
};

// ----------------------------------------------------------------------------- host
// The types with a GPU decoder (GGMLDequant.supported, Core/GGMLDequant.swift:19-24, plus Q4_0).
#define ISHZ_GGML_FORMATS(X)                                                                     \
  X(ISHZ_GGML_Q4_0, FQ4_0) X(ISHZ_GGML_Q4_K, FQ4_K) X(ISHZ_GGML_Q6_K, FQ6_K) X(ISHZ_GGML_IQ2_XS, FIQ2_XS) \
  ISHZ_GGML_QUARTER_FORMATS(X)
#define ISHZ_GGML_QUARTER_FORMATS(X)                                                             \
  X(ISHZ_GGML_Q2_K, FQ2_K) X(ISHZ_GGML_IQ4_XS, FIQ4_XS) X(ISHZ_GGML_IQ2_XXS, FIQ2_XXS)           \
  X(ISHZ_GGML_IQ2_S, FIQ2_S) X(ISHZ_GGML_IQ3_XXS, FIQ3_XXS) X(ISHZ_GGML_IQ3_S, FIQ3_S)          \
  X(ISHZ_GGML_IQ1_S, FIQ1_S) X(ISHZ_GGML_IQ1_M, FIQ1_M)

static int block_size(uint32_t t) {
  switch (t) {
#define X(T, F) case T: return F::BS;
    ISHZ_GGML_FORMATS(X)
#undef X
  default: return 0;
  }
}
static int type_size(uint32_t t) {
  switch (t) {
#define X(T, F) case T: return F::TS;
    ISHZ_GGML_FORMATS(X)
#undef X
  default: return 0;
  }
}

static int g_num_cu = 0;
static int num_cu() {
  if (!g_num_cu) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_num_cu = n;
    else
      g_num_cu = 256;
  }
  return g_num_cu;
}

int gemv_num_cu() { return num_cu(); }

template <class F>
static int verify(const void *x, int M, int K, const void *w, int N, const Out &y, hipStream_t st, void *ws = nullptr,
                  size_t ws_bytes = 0);

template <class F>
static int gemv(const void *x, int K, const void *w, int N, const Out &y, hipStream_t st) {
  if (K % F::GEMV_K_MULT) return verify<F>(x, 1, K, w, N, y, st);
  const typename F::Args a{(const uint8_t *)w, (size_t)(K / F::BS) * F::TS, K, N};
  return launch_gemv<F>(a, x, y.y, st, y.dt, y.rs);
}

template <class F, int T>
static int launch_verify(const void *x, int M, int K, const void *w, int N, const Out &y, hipStream_t st) {
  const int wgs = (N + 16 * T - 1) / (16 * T);
  const int nblk = K / F::BS;
  int ks = 1;
  while (ks < 16 && ks < nblk && wgs * ks < num_cu() * 16) ks *= 2;
  const size_t lds = (F::GRID ? (512 + 128) * 16 : 0) + (size_t)ks * T * 256 * 4;
  hipLaunchKernelGGL((verify_kernel<F, T>), dim3(wgs), dim3(64 * ks), lds, st, (const uint16_t *)x,
                     M, K, (const uint8_t *)w, N, y);
  ISHZ_LAUNCH_CHECK("verify launch");
  return ISHZ_OK;
}

template <class F>
static int verify(const void *x, int M, int K, const void *w, int N, const Out &y, hipStream_t st, void *ws,
                  size_t ws_bytes) {
  if (M >= 2 && K % 256 == 0) return vgemm<F>(x, M, K, w, N, y, st, ws, ws_bytes);
  if (N >= 4096) return launch_verify<F, 2>(x, M, K, w, N, y, st);
  return launch_verify<F, 1>(x, M, K, w, N, y, st);
}

// The quarter-block formats: K is always a multiple of 256 (their block), so M = 1 is the
// streaming GEMV and M >= 2 the streaming MFMA kernel.
template <class F>
static int quarter(const void *x, int M, int K, const void *w, int N, const Out &y, hipStream_t st, void *ws = nullptr,
                   size_t ws_bytes = 0) {
  if (M == 1) {
    const typename F::Args a{(const uint8_t *)w, (size_t)(K / F::BS) * F::TS, K, N};
    return launch_gemv<F>(a, x, y.y, st, y.dt, y.rs);
  }
  return vgemm<F>(x, M, K, w, N, y, st, ws, ws_bytes);
}

__global__ __launch_bounds__(256) void vgemm_sum_kernel(const float *__restrict__ part, int S, size_t n, int N, Out y) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int k = 0; k < S; k++) s += part[(size_t)k * n + i];
    y.put(i, (int)(i / N), s);
  }
}

static int check_matmul(uint32_t type, int x_dtype, int M, int lo, int hi, int K,
                        size_t blocks_bytes, int N, const void *x, const void *w, const void *y) {
  const int bs = block_size(type);
  if (!bs) return decline("unsupported GGML type " + std::to_string(type));
  if (x_dtype != ISHZ_DT_F16 && x_dtype != ISHZ_DT_BF16 && x_dtype != ISHZ_DT_F32)
    return decline("activations must be fp16, bf16 or fp32");
  if (M < lo || M > hi) return decline("row count outside the kernel's range");
  if (K <= 0 || K % bs) return decline("K is not a whole number of blocks");
  if (N <= 0) return decline("N must be positive");
  if (blocks_bytes < (size_t)N * (K / bs) * type_size(type)) return decline("blocks buffer too short");
  if (!x || !w || !y) return einval("null pointer");
  return ISHZ_OK;
}

}  // namespace ishz

using namespace ishz;

extern "C" int ishz_ggml_block_size(uint32_t type) { return block_size(type); }
extern "C" int ishz_ggml_type_size(uint32_t type) { return type_size(type); }

// Workspace: the activation image (bf16 / fp32 x), then the K split's fp32 parts.
extern "C" size_t ishz_ggml_workspace_size(uint32_t type, int M, int K, int N) {
  if (!block_size(type) || M < 1 || M > 16 || K <= 0 || N <= 0) return 0;
  return act_image_bytes(M, K) + (K % 256 ? 0 : vgemm_workspace(M, K, N, num_cu()));
}

// x (any activation dtype) -> fp16 image; then the product with outputs in x's dtype.
static int ggml_call(uint32_t type, const void *x, int x_dtype, int M, int K, const void *blocks, int N, void *y,
                     void *workspace, size_t workspace_bytes, hipStream_t st, bool few) {
  if (x_dtype == ISHZ_DT_F32) {  // fp32 x at fp32 precision: exact fp32 weights, fp32 FMAs
    switch (type) {
#define X(T, F)                                                                                              \
  case T:                                                                                                    \
    return launch_precise<GgmlDec<T, F::BS, F::TS>>({(const uint8_t *)blocks, (size_t)(K / F::BS) * F::TS},   \
                                                    x, ISHZ_DT_F32, M, K, N, y, st);
      ISHZ_GGML_FORMATS(X)
#undef X
    }
    return decline("unsupported GGML type");
  }
  StreamTemp tmp(st);
  void *img = workspace;
  size_t left = workspace_bytes;
  const size_t ib = act_image_bytes(M, K);
  if (x_dtype != ISHZ_DT_F16) {
    if (!workspace || workspace_bytes < ib) {  // no room for the image: a temporary of its own
      int rc = tmp.get(ib);
      if (rc) return rc;
      img = tmp.p;
    } else {
      workspace = (char *)workspace + ib;
      left -= ib;
    }
  } else if (workspace && workspace_bytes >= ib) {
    workspace = (char *)workspace + ib;
    left -= ib;
  }
  const uint16_t *xh;
  const float *rs;
  int rc = act_prepare(x, x_dtype, M, K, img, st, &xh, &rs);
  if (rc) return rc;
  const Out o{y, x_dtype, rs};
  void *ws = workspace;
  const size_t wb = ws ? left : 0;
  if (M == 1 && !few) {
    switch (type) {
    case ISHZ_GGML_Q4_0: return gemv<FQ4_0>(xh, K, blocks, N, o, st);
    case ISHZ_GGML_Q4_K: return gemv<FQ4_K>(xh, K, blocks, N, o, st);
    case ISHZ_GGML_Q6_K: return gemv<FQ6_K>(xh, K, blocks, N, o, st);
    case ISHZ_GGML_IQ2_XS: return gemv<FIQ2_XS>(xh, K, blocks, N, o, st);
    }
  }
  switch (type) {
  case ISHZ_GGML_Q4_0: return verify<FQ4_0>(xh, M, K, blocks, N, o, st, ws, wb);
  case ISHZ_GGML_Q4_K: return verify<FQ4_K>(xh, M, K, blocks, N, o, st, ws, wb);
  case ISHZ_GGML_Q6_K: return verify<FQ6_K>(xh, M, K, blocks, N, o, st, ws, wb);
  case ISHZ_GGML_IQ2_XS: return verify<FIQ2_XS>(xh, M, K, blocks, N, o, st, ws, wb);
#define X(T, F) case T: return quarter<F>(xh, M, K, blocks, N, o, st, ws, wb);
    ISHZ_GGML_QUARTER_FORMATS(X)
#undef X
  }
  return decline("unsupported GGML type");
}

extern "C" int ishz_ggml_matvec_ws(uint32_t type, const void *x, int x_dtype, int M, int K, const void *blocks,
                                   size_t blocks_bytes, int N, void *y, void *workspace, size_t workspace_bytes,
                                   ishz_stream_t stream) {
  int rc = check_matmul(type, x_dtype, M, 1, 16, K, blocks_bytes, N, x, blocks, y);
  if (rc) return rc;
  return ggml_call(type, x, x_dtype, M, K, blocks, N, y, workspace, workspace_bytes, S(stream), false);
}

extern "C" int ishz_ggml_matvec(uint32_t type, const void *x, int x_dtype, int M, int K,
                                const void *blocks, size_t blocks_bytes, int N, void *y,
                                ishz_stream_t stream) {
  return ishz_ggml_matvec_ws(type, x, x_dtype, M, K, blocks, blocks_bytes, N, y, nullptr, 0, stream);
}

extern "C" int ishz_ggml_matmul_few(uint32_t type, const void *x, int x_dtype, int M, int K,
                                    const void *blocks, size_t blocks_bytes, int N, int row_blocks,
                                    void *y, ishz_stream_t stream) {
  (void)row_blocks;
  if (block_size(type) != 256) return decline("matmulFew takes 256-element block types only");
  int rc = check_matmul(type, x_dtype, M, 2, 8, K, blocks_bytes, N, x, blocks, y);
  if (rc) return rc;
  return ggml_call(type, x, x_dtype, M, K, blocks, N, y, nullptr, 0, S(stream), true);
}

template <uint32_t TYPE, int BS, int TS>
static int dequant_t(const void *w, size_t count, void *out, int dt, hipStream_t st) {
  const size_t slices = count / 8;
  const int blocks = (int)std::min<size_t>((slices + 255) / 256, (size_t)num_cu() * 32);
  hipLaunchKernelGGL((dequant_kernel<TYPE, BS, TS>), dim3(blocks), dim3(256), 0, st,
                     (const uint8_t *)w, slices, out, dt);
  ISHZ_LAUNCH_CHECK("dequant launch");
  return ISHZ_OK;
}

extern "C" int ishz_ggml_dequant(uint32_t type, const void *blocks, size_t blocks_bytes,
                                 size_t count, void *out, int out_dtype, ishz_stream_t stream) {
  const int bs = block_size(type);
  if (!bs) return decline("unsupported GGML type " + std::to_string(type));
  if (out_dtype < ISHZ_DT_F32 || out_dtype > ISHZ_DT_BF16) return decline("unsupported output dtype");
  if (count == 0 || count % bs) return decline("count is not a whole number of blocks");
  if (blocks_bytes < count / bs * type_size(type)) return decline("blocks buffer too short");
  if (!blocks || !out) return einval("null pointer");
  hipStream_t st = S(stream);
  switch (type) {
#define X(T, F) case T: return dequant_t<T, F::BS, F::TS>(blocks, count, out, out_dtype, st);
    ISHZ_GGML_FORMATS(X)
#undef X
  }
  return decline("unsupported GGML type");
}

template <uint32_t TYPE, int BS, int TS>
static int gather_t(const int32_t *ids, int n_ids, const void *w, int n_rows, int K, void *out,
                    int dt, hipStream_t st) {
  const size_t slices = (size_t)n_ids * K / 8;
  const int blocks = (int)std::min<size_t>((slices + 255) / 256, (size_t)num_cu() * 32);
  hipLaunchKernelGGL((gather_kernel<TYPE, BS, TS>), dim3(blocks), dim3(256), 0, st, ids, n_ids,
                     (const uint8_t *)w, n_rows, K, out, dt);
  ISHZ_LAUNCH_CHECK("gather launch");
  return ISHZ_OK;
}

extern "C" int ishz_ggml_gather(uint32_t type, const int32_t *ids, int n_ids, const void *blocks,
                                size_t blocks_bytes, int n_rows, int K, void *out, int out_dtype,
                                ishz_stream_t stream) {
  const int bs = block_size(type);
  if (!bs) return decline("unsupported GGML type " + std::to_string(type));
  if (out_dtype < ISHZ_DT_F32 || out_dtype > ISHZ_DT_BF16) return decline("unsupported output dtype");
  if (K <= 0 || K % bs) return decline("K is not a whole number of blocks");
  if (n_ids <= 0) return decline("no ids");
  if (n_rows <= 0 || blocks_bytes < (size_t)n_rows * (K / bs) * type_size(type))
    return decline("blocks buffer too short");
  if (!ids || !blocks || !out) return einval("null pointer");
  hipStream_t st = S(stream);
  switch (type) {
#define X(T, F) case T: return gather_t<T, F::BS, F::TS>(ids, n_ids, blocks, n_rows, K, out, out_dtype, st);
    ISHZ_GGML_FORMATS(X)
#undef X
  }
  return decline("unsupported GGML type");
}
