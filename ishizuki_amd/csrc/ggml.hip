// GGML quantized matmul on gfx950: streaming GEMV (M = 1), MFMA verify (M = 2..16), dequant and
// gather writers. Replaces GGMLKernels (Sources/IshizukiKit/Core/GGMLKernels.swift).
#include "ggml_formats.h"
#include "vgemm.h"

#include <cstdlib>

#define ISHZ_TABLE_QUAL static __device__
#include "ggml_grids.inc"

namespace ishz {

// ----------------------------------------------------------------------------- tables in LDS
// IQ2_XS grid entries as fp16 (values 8, 25, 43) and the 128 sign patterns of ksigns
// (index | parity << 7) as fp16 sign-bit masks, either in the permuted pair order of the GEMV
// (x0,x2,x1,x3,...) or in natural order for the MFMA B operand.
template <bool PERM>
DEV void build_iq2xs_tables(u4 *grid, u4 *sgn) {
  for (int e = threadIdx.x; e < 512 + 128; e += blockDim.x) {
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
      sgn[i] = PERM ? u4{bit(0) | bit(2) << 16, bit(1) | bit(3) << 16, bit(4) | bit(6) << 16,
                         bit(5) | bit(7) << 16}
                    : u4{bit(0) | bit(1) << 16, bit(2) | bit(3) << 16, bit(4) | bit(5) << 16,
                         bit(6) | bit(7) << 16};
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
                                                      const uint8_t *__restrict__ w, int N,
                                                      uint16_t *__restrict__ y) {
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
    if (tk < M && n < N) y[(size_t)tk * N + n] = f2h(s);
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

// ----------------------------------------------------------------------------- host
static int block_size(uint32_t t) {
  switch (t) {
  case ISHZ_GGML_Q4_0: return FQ4_0::BS;
  case ISHZ_GGML_Q4_K: return FQ4_K::BS;
  case ISHZ_GGML_Q6_K: return FQ6_K::BS;
  case ISHZ_GGML_IQ2_XS: return FIQ2_XS::BS;
  default: return 0;
  }
}
static int type_size(uint32_t t) {
  switch (t) {
  case ISHZ_GGML_Q4_0: return FQ4_0::TS;
  case ISHZ_GGML_Q4_K: return FQ4_K::TS;
  case ISHZ_GGML_Q6_K: return FQ6_K::TS;
  case ISHZ_GGML_IQ2_XS: return FIQ2_XS::TS;
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
static int env_int(const char *name) {
  const char *e = getenv(name);
  return e ? atoi(e) : 0;
}
int gemv_batch_override() {
  static const int v = env_int("ISHZ_GEMV_B");
  return v;
}
int gemv_depth_override() {
  static const int v = env_int("ISHZ_GEMV_D");
  return v;
}
int gemv_occ_override() {
  static const int v = env_int("ISHZ_GEMV_OCC");
  return v;
}

template <class F>
static int verify(const void *x, int M, int K, const void *w, int N, void *y, hipStream_t st);

template <class F>
static int gemv(const void *x, int K, const void *w, int N, void *y, hipStream_t st) {
  if (K % F::GEMV_K_MULT) return verify<F>(x, 1, K, w, N, y, st);
  const typename F::Args a{(const uint8_t *)w, (size_t)(K / F::BS) * F::TS, K, N};
  return launch_gemv<F>(a, x, y, st);
}

template <class F, int T>
static int launch_verify(const void *x, int M, int K, const void *w, int N, void *y, hipStream_t st) {
  const int wgs = (N + 16 * T - 1) / (16 * T);
  const int nblk = K / F::BS;
  int ks = 1;
  while (ks < 16 && ks < nblk && wgs * ks < num_cu() * 16) ks *= 2;
  const size_t lds = (F::GRID ? (512 + 128) * 16 : 0) + (size_t)ks * T * 256 * 4;
  hipLaunchKernelGGL((verify_kernel<F, T>), dim3(wgs), dim3(64 * ks), lds, st, (const uint16_t *)x,
                     M, K, (const uint8_t *)w, N, (uint16_t *)y);
  ISHZ_LAUNCH_CHECK("verify launch");
  return ISHZ_OK;
}

template <class F>
static int verify(const void *x, int M, int K, const void *w, int N, void *y, hipStream_t st) {
  static const bool old = getenv("ISHZ_OLD_VERIFY") != nullptr;
  if (M >= 2 && K % 256 == 0 && !old) return vgemm<F>(x, M, K, w, N, y, st);
  if (N >= 4096) return launch_verify<F, 2>(x, M, K, w, N, y, st);
  return launch_verify<F, 1>(x, M, K, w, N, y, st);
}

static int check_matmul(uint32_t type, int x_dtype, int M, int lo, int hi, int K,
                        size_t blocks_bytes, int N, const void *x, const void *w, const void *y) {
  const int bs = block_size(type);
  if (!bs) return decline("unsupported GGML type " + std::to_string(type));
  if (x_dtype != ISHZ_DT_F16) return decline("activations must be fp16");
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

extern "C" int ishz_ggml_matvec(uint32_t type, const void *x, int x_dtype, int M, int K,
                                const void *blocks, size_t blocks_bytes, int N, void *y,
                                ishz_stream_t stream) {
  int rc = check_matmul(type, x_dtype, M, 1, 16, K, blocks_bytes, N, x, blocks, y);
  if (rc) return rc;
  hipStream_t st = S(stream);
  if (M == 1) {
    switch (type) {
    case ISHZ_GGML_Q4_0: return gemv<FQ4_0>(x, K, blocks, N, y, st);
    case ISHZ_GGML_Q4_K: return gemv<FQ4_K>(x, K, blocks, N, y, st);
    case ISHZ_GGML_Q6_K: return gemv<FQ6_K>(x, K, blocks, N, y, st);
    case ISHZ_GGML_IQ2_XS: return gemv<FIQ2_XS>(x, K, blocks, N, y, st);
    }
  }
  switch (type) {
  case ISHZ_GGML_Q4_0: return verify<FQ4_0>(x, M, K, blocks, N, y, st);
  case ISHZ_GGML_Q4_K: return verify<FQ4_K>(x, M, K, blocks, N, y, st);
  case ISHZ_GGML_Q6_K: return verify<FQ6_K>(x, M, K, blocks, N, y, st);
  case ISHZ_GGML_IQ2_XS: return verify<FIQ2_XS>(x, M, K, blocks, N, y, st);
  }
  return decline("unsupported GGML type");
}

extern "C" int ishz_ggml_matmul_few(uint32_t type, const void *x, int x_dtype, int M, int K,
                                    const void *blocks, size_t blocks_bytes, int N, int row_blocks,
                                    void *y, ishz_stream_t stream) {
  (void)row_blocks;
  if (block_size(type) != 256) return decline("matmulFew takes 256-element block types only");
  int rc = check_matmul(type, x_dtype, M, 2, 8, K, blocks_bytes, N, x, blocks, y);
  if (rc) return rc;
  hipStream_t st = S(stream);
  switch (type) {
  case ISHZ_GGML_Q4_K: return verify<FQ4_K>(x, M, K, blocks, N, y, st);
  case ISHZ_GGML_Q6_K: return verify<FQ6_K>(x, M, K, blocks, N, y, st);
  case ISHZ_GGML_IQ2_XS: return verify<FIQ2_XS>(x, M, K, blocks, N, y, st);
  }
  return decline("unsupported GGML type");
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
  case ISHZ_GGML_Q4_0: return dequant_t<ISHZ_GGML_Q4_0, 32, 18>(blocks, count, out, out_dtype, st);
  case ISHZ_GGML_Q4_K: return dequant_t<ISHZ_GGML_Q4_K, 256, 144>(blocks, count, out, out_dtype, st);
  case ISHZ_GGML_Q6_K: return dequant_t<ISHZ_GGML_Q6_K, 256, 210>(blocks, count, out, out_dtype, st);
  case ISHZ_GGML_IQ2_XS: return dequant_t<ISHZ_GGML_IQ2_XS, 256, 74>(blocks, count, out, out_dtype, st);
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
  case ISHZ_GGML_Q4_0: return gather_t<ISHZ_GGML_Q4_0, 32, 18>(ids, n_ids, blocks, n_rows, K, out, out_dtype, st);
  case ISHZ_GGML_Q4_K: return gather_t<ISHZ_GGML_Q4_K, 256, 144>(ids, n_ids, blocks, n_rows, K, out, out_dtype, st);
  case ISHZ_GGML_Q6_K: return gather_t<ISHZ_GGML_Q6_K, 256, 210>(ids, n_ids, blocks, n_rows, K, out, out_dtype, st);
  case ISHZ_GGML_IQ2_XS: return gather_t<ISHZ_GGML_IQ2_XS, 256, 74>(ids, n_ids, blocks, n_rows, K, out, out_dtype, st);
  }
  return decline("unsupported GGML type");
}
