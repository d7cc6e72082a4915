// Streaming MFMA GEMM for 2..16 drafted rows over block-quantized weights (GGML formats): each
// weight is decoded once into an MFMA B operand and multiplied against every token.
//
// Step = 256 weights of each of a tile's 16 rows; lane (n, g) = (lane % 16, lane / 16) owns the
// step's quarter g of row n (64 weights, one or two 128-bit loads) and decodes it into the B
// operands of 8 MFMAs 16x16x32. The quarter splits into NS scale groups ("sub-units", 8 / NS
// MFMAs each, one accumulator each). A is "diagonal": A row m = 4 gg + tt holds token tt's staged
// x for k-slot gg only, so C row 4 gg + tt collects token tt's dot with lane group gg's sub-unit,
// and lane (n, G) ends each step holding its own quarter's partials for four tokens in its four
// C registers: it applies its own scales, with no exchange between lanes. Four tokens per MFMA;
// NQ token quads reuse the same decoded B. The lane-group partials of a row are summed by
// shuffles once per tile.
//
// A workgroup (NW waves) owns a run of tiles; its waves split each tile's steps (step j goes to
// wave j % NW) and sum their partials in LDS. x is staged in LDS per K chunk, in A-operand order:
// token image [step][g][mfma] of 16-byte words, plus per (step, g, sub-unit) the sums the
// epilogue needs for every token (1024 * sum of the staged A values, the magic-number offset;
// and the plain sum of x).
//
// A format F provides:
//   VNS                              sub-units per quarter
//   VRaw vload(row, j, g)            the quarter's codes and the row's step header
//   void vdecode(r, B[8], tabs)      B operands (MFMA b of sub-unit b / (8 / VNS))
//   void vstage(xrow, j, g, s, A, off1, X)   A words of sub-unit s (8 / VNS of them) and sums
//   void vscale(r, g, s, sc, mn)     value of sub-unit s = sc * (C - off1) + mn * X
//   VGRID                            LDS tables (IQ2_XS grid and signs, natural order)
#pragma once
#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace ishz {

DEV void build_iq2xs_tables_nat(u4 *grid, u4 *sgn);

template <class F, int NQ, int D, int NW>
__global__ __launch_bounds__(64 * NW) void vgemm_kernel(const uint16_t *__restrict__ x, int M, int K,
                                                       const uint8_t *__restrict__ w, size_t rb, int N,
                                                       uint16_t *__restrict__ y, int Kc, int tiles_per_wg) {
  constexpr int NS = F::VNS, MPS = 8 / NS;  // MFMAs per sub-unit
  constexpr int MT = 4 * NQ;                // tokens padded to whole quads
  extern __shared__ __align__(16) u4 vgsm[];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, G = lane >> 4;
  const int ntiles = (N + 15) / 16;
  const int tb = blockIdx.x * tiles_per_wg, te = min(tb + tiles_per_wg, ntiles);
  const int cs = Kc / 256;                   // steps per chunk
  const int IW = cs * 32 + 1;                // token image stride (16-byte words, padded)
  u4 *zero = vgsm + M * IW;                   // 8 words of zeros (non-diagonal A)
  float *sums = (float *)(zero + 8);         // [cs][4][NS][2][MT]
  float *accb = sums + cs * 4 * NS * 2 * MT;  // [wave][tile][quad][4][16]
  u4 *tabs = (u4 *)(accb + NW * tiles_per_wg * NQ * 64);
  const uint32_t mg = vconst(0x64006400u);

  for (int i = threadIdx.x; i < 8; i += blockDim.x) zero[i] = u4{0, 0, 0, 0};
  for (int i = threadIdx.x; i < NW * tiles_per_wg * NQ * 64; i += blockDim.x) accb[i] = 0.0f;
  if constexpr (F::VGRID) build_iq2xs_tables_nat(tabs, tabs + 512);
  // A row of this lane: gg = n / 4 (lane group whose k-slot it fills), token tt = n % 4.
  const int gg = n >> 2, tt = n & 3;

  for (int kc0 = 0; kc0 < K; kc0 += Kc) {
    const int steps = min(Kc, K - kc0) / 256;
    // ---- stage every token's x for this chunk
    for (int it = threadIdx.x; it < MT * steps * 4 * NS; it += blockDim.x) {
      const int s = it % NS, g = (it / NS) % 4, j = (it / (NS * 4)) % steps, tk = it / (NS * 4 * steps);
      float off1 = 0.0f, X = 0.0f;
      if (tk < M) {
        u4 A[MPS];
        F::vstage(x + (size_t)tk * K + kc0, j, g, s, A, off1, X);
        u4 *dst = vgsm + tk * IW + (j * 4 + g) * 8 + s * MPS;
#pragma unroll
        for (int b = 0; b < MPS; b++) dst[b] = A[b];
      }
      float *sp = sums + (((j * 4 + g) * NS + s) * 2) * MT;
      sp[tk] = off1;
      sp[MT + tk] = X;
    }
    __syncthreads();

    // ---- stream this wave's (tile, step) sequence: steps wave, wave + NW, ... of each tile
    typedef typename F::VRaw Raw;
    const bool active = wave < steps && tb < te;
    const int j_last = wave + (steps - 1 - wave) / NW * NW;
    const uint8_t *wc = w + (size_t)(kc0 / 256) * F::VSTEP_BYTES;
    auto load = [&](int tile, int j, Raw &r) {
      const int row = min(min(tile, te - 1) * 16 + n, N - 1);
      r = F::vload(wc + (size_t)row * rb, min(j, j_last), G);
    };
    auto advance = [&](int &tile, int &j) {
      j += NW;
      if (j > j_last) {
        j = wave;
        tile++;
      }
    };
    Raw ring[D];
    int lt = tb, lj = wave;
    if (active) {
#pragma unroll
      for (int d = 0; d < D - 1; d++) {
        load(lt, lj, ring[d]);
        advance(lt, lj);
      }
    }
    f4 acc[NQ];
    int ct = tb, cj = wave;
    while (active && ct < te) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        load(lt, lj, ring[(d + D - 1) % D]);
        advance(lt, lj);
        if (ct >= te) break;
        const int tl = ct - tb, j = cj;
        if (j == wave) {
#pragma unroll
          for (int q = 0; q < NQ; q++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[q][r] = 0.0f;
        }
        const Raw &r = ring[d];
        u4 B[8];
        F::vdecode(r, B, mg, tabs, tabs + 512);
        float sc[NS], mn[NS];
#pragma unroll
        for (int s = 0; s < NS; s++) F::vscale(r, G, s, sc[s], mn[s]);
#pragma unroll
        for (int q = 0; q < NQ; q++) {
          const int tka = 4 * q + tt;
          const u4 *ab = (gg == G && tka < M) ? vgsm + tka * IW + (j * 4 + G) * 8 : zero;
#pragma unroll
          for (int s = 0; s < NS; s++) {
            f4 C = f4{0, 0, 0, 0};
#pragma unroll
            for (int b = 0; b < MPS; b++) C = mfma32(as_h8(ab[s * MPS + b]), as_h8(B[s * MPS + b]), C);
            const float *sp = sums + (((j * 4 + G) * NS + s) * 2) * MT + 4 * q;
            const f4 off = *(const f4 *)sp, X = *(const f4 *)(sp + MT);
#pragma unroll
            for (int e = 0; e < 4; e++) acc[q][e] += sc[s] * (C[e] - off[e]) + mn[s] * X[e];
          }
        }
        if (j == j_last) {
          // sum the four lane groups' quarters of each row, then park the wave's partial
#pragma unroll
          for (int q = 0; q < NQ; q++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
              float a = acc[q][e];
              a += __shfl_xor(a, 16, 64);
              a += __shfl_xor(a, 32, 64);
              if (G == 0) accb[(((wave * tiles_per_wg + tl) * NQ + q) * 4 + e) * 16 + n] += a;
            }
        }
        advance(ct, cj);
      }
    }
    __syncthreads();  // partials parked; the x image is free for the next chunk
  }
  // ---- sum the waves' partials and write y
  for (int o = threadIdx.x; o < (te - tb) * NQ * 64; o += blockDim.x) {
    const int tl = o / (NQ * 64), q = (o / 64) % NQ, e = (o / 16) % 4, nn = o % 16;
    float s = 0.0f;
    for (int v = 0; v < NW; v++) s += accb[(((v * tiles_per_wg + tl) * NQ + q) * 4 + e) * 16 + nn];
    const int tk = 4 * q + e, row = (tb + tl) * 16 + nn;
    if (tk < M && row < N) y[(size_t)tk * N + row] = f2h(s);
  }
}

int gemv_num_cu();

template <class F, int NQ>
static int launch_vgemm(const void *x, int M, int K, const void *w, int N, void *y, hipStream_t st) {
  constexpr int D = 4, NW = 8;
  constexpr int NS = F::VNS, MT = 4 * NQ;
  const int ntiles = (N + 15) / 16;
  const int T = (ntiles + gemv_num_cu() - 1) / gemv_num_cu();  // tiles per workgroup: one round of CUs
  const int wgs = (ntiles + T - 1) / T;
  auto need = [&](int kc) {
    const int cs = kc / 256;
    return (size_t)M * (cs * 32 + 1) * 16 + 8 * 16 + (size_t)cs * 4 * NS * 2 * MT * 4 +
           (size_t)NW * T * NQ * 64 * 4 + (F::VGRID ? (512 + 128) * 16 : 0);
  };
  const size_t budget = 150 * 1024;
  int Kc = K;
  while (Kc > 256 && need(Kc) > budget) Kc -= 256;
  if (need(Kc) > budget) return decline("verify x does not fit in LDS");
  const size_t rb = (size_t)(K / F::BS) * F::TS;
  hipLaunchKernelGGL((vgemm_kernel<F, NQ, D, NW>), dim3(wgs), dim3(64 * NW), need(Kc), st, (const uint16_t *)x, M, K,
                     (const uint8_t *)w, rb, N, (uint16_t *)y, Kc, T);
  ISHZ_LAUNCH_CHECK("vgemm launch");
  return ISHZ_OK;
}

template <class F>
static int vgemm(const void *x, int M, int K, const void *w, int N, void *y, hipStream_t st) {
  switch ((M + 3) / 4) {
    case 1: return launch_vgemm<F, 1>(x, M, K, w, N, y, st);
    case 2: return launch_vgemm<F, 2>(x, M, K, w, N, y, st);
    case 3: return launch_vgemm<F, 3>(x, M, K, w, N, y, st);
    default: return launch_vgemm<F, 4>(x, M, K, w, N, y, st);
  }
}

}  // namespace ishz
