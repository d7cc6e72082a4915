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

#include "affine_fmt.h"
#include "affine_nbit.h"
#include "common.h"
#include "gemv.h"
#include "precise.h"

namespace ishz {
// hadamardRotate as a kernel. Blocks up to 128: one wave per 128 contiguous values, two per
// lane, butterflies across lanes by DPP and row swaps (stages above the block size skipped). Larger
// blocks: one workgroup per block, in LDS. fp32 math, output in `out_dt`.
__global__ __launch_bounds__(256) void hadamard_wave_kernel(const void *__restrict__ x, int in_dt,
                                                            size_t chunks, int width, int block,
                                                            const float *__restrict__ signs,
                                                            int inverse, void *__restrict__ y,
                                                            int out_dt) {
  const size_t c = (size_t)blockIdx.x * 4 + wave_id();
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
  // partner lane ^ m by DPP inside 16-lane rows, by the row swaps across them; the lower lane keeps
  // v + p, the upper p - v, as fma(v, +-1, p) (exact, the same rounding)
  auto stage = [&](float p0, float p1, int m) {
    const float s = (lane & m) ? -1.0f : 1.0f;
    v0 = __builtin_fmaf(v0, s, p0);
    v1 = __builtin_fmaf(v1, s, p1);
  };
  if (block > 2) stage(ISHZ_DPP(v0, 0xB1), ISHZ_DPP(v1, 0xB1), 1);
  if (block > 4) stage(ISHZ_DPP(v0, 0x4E), ISHZ_DPP(v1, 0x4E), 2);
  if (block > 8) stage(ISHZ_DPP(ISHZ_DPP(v0, 0x141), 0x1B), ISHZ_DPP(ISHZ_DPP(v1, 0x141), 0x1B), 4);
  if (block > 16) stage(ISHZ_DPP(ISHZ_DPP(v0, 0x141), 0x140), ISHZ_DPP(ISHZ_DPP(v1, 0x141), 0x140), 8);
  if (block > 32) stage(lane_xor16(v0), lane_xor16(v1), 16);
  if (block > 64) stage(lane_xor32(v0), lane_xor32(v1), 32);
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
                                                      int bf16s, int N, Out y) {
  extern __shared__ __align__(16) float red[];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
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
    if (tk < M && n < N) y.put((size_t)tk * N + n, tk, s);
  }
}

// ------------------------------------------------------------------- verify v2 (MFMA, M <= 16)
// Streaming MFMA GEMM for 2..16 drafted rows: each weight is decoded once into an MFMA B operand
// and multiplied against every token. A workgroup (8 waves) owns a run of 16-row tiles; its waves
// split each tile's K steps (step j of a tile goes to wave j % 8) and sum their partials in LDS.
//
// Step = 4 units (256 weights) of the tile's 16 rows: lane (n, g) = (lane % 16, lane / 16) loads
// the 16 code bytes of unit 4j + g of row n, i.e. one 128-bit load per lane, and decodes slot r
// (r < 8) of it into the B operand of MFMA r. A is "diagonal": A row m = 4 tt + gg holds token
// tt's staged x (the GEMV's slot image) for k-slot gg only, so C row 4 tt + gg collects token
// tt's dot with unit 4j + gg alone, and lane (n, G) ends each step with token G's four unit
// partials of row n in its four C registers, ready for the units' scale and bias. Four tokens
// per MFMA; NQ token quads reuse the same decoded B.
template <int GS, bool BF16S, int NQ, int D>
__global__ __launch_bounds__(512) void affine_vgemm(const uint16_t *__restrict__ x, int M, int K,
                                                    const uint32_t *__restrict__ codes,
                                                    const uint16_t *__restrict__ scales,
                                                    const uint16_t *__restrict__ biases, int N,
                                                    Out y, int Kc, int tiles_per_wg,
                                                    const float *__restrict__ signs, int block,
                                                    const u4 *__restrict__ img) {
  using F = FAffine<GS, BF16S>;
  constexpr int R = F::R;
  extern __shared__ __align__(16) u4 vlds[];
  const int lane = threadIdx.x & 63, wave = wave_id(), nw = blockDim.x >> 6;
  const int n = lane & 15, G = lane >> 4;
  const int units = K / 64, gpr = K / GS;
  const int ntiles = (N + 15) / 16;
  const int tb = blockIdx.x * tiles_per_wg, te = min(tb + tiles_per_wg, ntiles);
  // token images IW + 1 words apart: consecutive tokens start 16 bytes apart in the LDS banks
  const int IW = F::img_words(Kc) + 1, ugc = (Kc / 64 + 15) / 16;
  u4 *zero = vlds + M * IW;                            // 8 slots x 16 lanes of zeros
  float *accb = (float *)(zero + 128);                 // [wave][tile][quad][lane] partials
  const uint32_t mg = vconst(0x64006400u);

#ifdef ISHZ_TIMING
  uint64_t ts[5];
  ts[0] = __builtin_amdgcn_s_memrealtime();
#endif
  for (int i = threadIdx.x; i < 128; i += blockDim.x) zero[i] = u4{0, 0, 0, 0};
  for (int i = threadIdx.x; i < nw * tiles_per_wg * NQ * 64; i += blockDim.x) accb[i] = 0.0f;
  // A row of this lane: token tt = n / 4 of each quad, unit group gg = n % 4; only gg == G holds x.
  const int tt = n >> 2, gg = n & 3;

  for (int kc0 = 0; kc0 < K; kc0 += Kc) {
    const int klen = min(Kc, K - kc0), ucs = klen / 64, steps = ucs / 4;
    // ---- stream: this wave's (tile, step) sequence, steps wave, wave + nw, ... of each tile.
    // Load and consume cursors (tile, step) advance in step; loads past the end re-read the
    // wave's last step (always in range) and are dropped. Ring of D steps: the main loop consumes
    // D steps per pass and loads as many, with no exit in between, so the waits are for the step
    // being consumed; the last (total % D) steps are already in the ring.
    struct Raw {
      u4 q;
      uint32_t s[2], b[2];
    };
    const bool active = wave < steps && tb < te;
    const int j_last = wave + (steps - 1 - wave) / nw * nw;  // this wave's last step of a tile
    auto load = [&](int tile, int j, Raw &r) {
      const int row = min(min(tile, te - 1) * 16 + n, N - 1);
      const int u = kc0 / 64 + 4 * min(j, j_last);  // first unit of the step
      r.q = *(const u4 *)(codes + (size_t)row * (K / 16) + 4 * (u + G));
      if constexpr (GS == 64) {
        const u2 sv = *(const u2 *)(scales + (size_t)row * gpr + u), bv = *(const u2 *)(biases + (size_t)row * gpr + u);
        r.s[0] = sv.x, r.s[1] = sv.y, r.b[0] = bv.x, r.b[1] = bv.y;
      } else {
        r.s[0] = scales[(size_t)row * gpr + u / 2] | (uint32_t)scales[(size_t)row * gpr + u / 2 + 1] << 16;
        r.b[0] = biases[(size_t)row * gpr + u / 2] | (uint32_t)biases[(size_t)row * gpr + u / 2 + 1] << 16;
        r.s[1] = r.s[0], r.b[1] = r.b[0];
      }
    };
    auto advance = [&](int &tile, int &j) {
      j += nw;
      if (j > j_last) {
        j = wave;
        tile++;
      }
    };
    Raw ring[D];
    int lt = tb, lj = wave;
    const int total = active ? (te - tb) * ((j_last - wave) / nw + 1) : 0;
    // the first weight steps go out before the staging when x comes from the prestaged image (its
    // copy then overlaps their latency: M = 8 at 17408 x 5120, 13.5 -> 12.9 us), after it when the
    // workgroup rotates x itself (the rotation's loads would queue behind them: M = 2, 12.5 -> 12.1)
    if (active && img) {
#pragma unroll
      for (int d = 0; d < D - 1; d++) {
        load(lt, lj, ring[d]);
        advance(lt, lj);
      }
    }
    // ---- stage x[tk][kc0 .. kc0 + klen) of every token: copied from the prestaged images (Kc a
    // multiple of 1024, so a chunk's slots and sums are two runs of each image), or computed
    // (rotated first when block > 0), 8 values per lane per item
    if (img) {
      const int IWf = F::img_words(K), ugf = (K / 64 + 15) / 16, g0 = kc0 / 1024;
      const int ugt = (ucs + 15) / 16;  // groups in this chunk (the last may be short)
      const int ns = ugt * 16 * R, nq = ugt * 16 * F::Q / 4;
      // straight into LDS (global_load_lds_dwordx4), one token image per wave, all its runs of 64
      // words in flight at once: a loop of load-then-store copies waits out one memory latency per
      // word a thread copies. The loop is kept to a few scalar instructions per load: a wave issues
      // about one instruction per 1.7 ns, so per-chunk index arithmetic (a division by the chunk
      // count, 64-bit offsets) cost more than the loads' latency.
      for (int tk = wave; tk < M; tk += nw) {
        const u4 *src = img + (size_t)tk * IWf + g0 * 16 * R + lane;
        u4 *dst = vlds + tk * IW;
        for (int o = 0; o < ns; o += 64, src += 64, dst += 64)
          if (o + lane < ns) __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
        src = img + (size_t)tk * IWf + ugf * 16 * R + g0 * 16 * F::Q / 4 + lane;
        dst = vlds + tk * IW + ugc * 16 * R;
        for (int o = 0; o < nq; o += 64, src += 64, dst += 64)
          if (o + lane < nq) __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
      }
      __syncthreads();  // (waits for the wave's loads, then the barrier)
    } else {
      const int per_tok = (klen + 511) / 512, items = M * per_tok;
      const float scale = block > 1 ? 1.0f / __builtin_sqrtf((float)block) : 1.0f;
      constexpr int PF = 4;
      for (int i0 = wave; i0 < items; i0 += PF * nw) {
        u4 xv[PF];
        f4 sg[PF][2];
#pragma unroll
        for (int j = 0; j < PF; j++) {
          const int it = min(i0 + j * nw, items - 1), tk = it / per_tok, ps = it % per_tok;
          const int k = min(ps * 512 + 8 * lane, klen - 8);
          xv[j] = *(const u4 *)(x + (size_t)tk * K + kc0 + k);
          if (signs) {
            sg[j][0] = *(const f4 *)(signs + kc0 + k);
            sg[j][1] = *(const f4 *)(signs + kc0 + k + 4);
          }
        }
#pragma unroll
        for (int j = 0; j < PF; j++) {
          const int it = i0 + j * nw;
          if (it >= items) break;
          const int tk = it / per_tok, ps = it % per_tok, k = ps * 512 + 8 * lane;
          float v[8];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const h2 hv = as_h2(xv[j][e]);
            v[2 * e] = (float)hv.x;
            v[2 * e + 1] = (float)hv.y;
          }
          if (block > 0) F::rot8(v, signs ? sg[j] : nullptr, block, scale, lane);
          u4 *img = vlds + tk * IW;
          F::put8(img, (float *)(img + ugc * 16 * R), k, v, k < klen);
        }
      }
      __syncthreads();
    }

#ifdef ISHZ_TIMING
    ts[1] = ts[2] = __builtin_amdgcn_s_memrealtime();
#endif
    if (active && !img) {
#pragma unroll
      for (int d = 0; d < D - 1; d++) {
        load(lt, lj, ring[d]);
        advance(lt, lj);
      }
    }
    float acc[NQ];
    int ct = tb, cj = wave;
    auto consume = [&](const Raw &r) {
      const int tl = ct - tb, j = cj;
      if (j == wave) {
#pragma unroll
        for (int q = 0; q < NQ; q++) acc[q] = accb[((wave * tiles_per_wg + tl) * NQ + q) * 64 + lane];
      }
      // B operands: slot r2 of the unit (word r2 / 2, pairs 4 (r2 % 2) .. + 3)
      u4 B[8];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t w = r.q[t], w10 = w >> 10;
        B[2 * t] = u4{and_or(w, 0x00030003u, mg), and_or(w, 0x000C000Cu, mg), and_or(w, 0x00300030u, mg),
                      and_or(w, 0x00C000C0u, mg)};
        B[2 * t + 1] = u4{and_or(w, 0x03000300u, mg), and_or(w10, 0x00030003u, mg),
                          and_or(w10, 0x000C000Cu, mg), and_or(w10, 0x00300030u, mg)};
      }
      const int ua = 4 * j + gg;  // chunk-relative unit of this lane's A row
      float sc[4], bi[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t sv = GS == 64 ? (r.s[e >> 1] >> (16 * (e & 1))) : (r.s[0] >> (16 * (e >> 1)));
        const uint32_t bv = GS == 64 ? (r.b[e >> 1] >> (16 * (e & 1))) : (r.b[0] >> (16 * (e >> 1)));
        sc[e] = F::ld_s(sv & 0xffffu);
        bi[e] = F::ld_s(bv & 0xffffu);
      }
#pragma unroll
      for (int q = 0; q < NQ; q++) {
        const int tka = 4 * q + tt;  // token of this lane's A row
        const u4 *ab = (gg == G && tka < M) ? vlds + tka * IW + (ua >> 4) * 16 * R + (ua & 15) : zero;
        f4 C = f4{0, 0, 0, 0};
#pragma unroll
        for (int r2 = 0; r2 < 8; r2++) C = mfma32(as_h8(ab[16 * r2]), as_h8(B[r2]), C);
        // lane (n, G): token 4q + G, units 4j .. 4j + 3 of row n
        const int tkc = min(4 * q + G, M - 1);
        const float *sm = (const float *)(vlds + tkc * IW + ugc * 16 * R) + ((4 * j) >> 4) * 32 + ((4 * j) & 15);
        const f4 off = *(const f4 *)sm, X = *(const f4 *)(sm + 16);
        float a = acc[q];
#pragma unroll
        for (int e = 0; e < 4; e++) a += sc[e] * (C[e] - off[e]) + bi[e] * X[e];
        acc[q] = a;
      }
      if (j == j_last) {
#pragma unroll
        for (int q = 0; q < NQ; q++) accb[((wave * tiles_per_wg + tl) * NQ + q) * 64 + lane] = acc[q];
      }
      advance(ct, cj);
    };
    int c = 0;
    for (; c + D <= total; c += D) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        load(lt, lj, ring[(d + D - 1) % D]);
        advance(lt, lj);
        consume(ring[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < D - 1; d++)
      if (c + d < total) consume(ring[d]);
#ifdef ISHZ_TIMING
    ts[3] = __builtin_amdgcn_s_memrealtime();
#endif
    __syncthreads();  // partials written; x image free for the next chunk
  }
#ifdef ISHZ_TIMING
  ts[4] = __builtin_amdgcn_s_memrealtime();
  if (lane == 0)
    for (int i = 0; i < 5; i++) ishz_timing[(blockIdx.x * 8 + wave) * 5 + i] = ts[i];
#endif
  // ---- sum the waves' partials and write y
  for (int o = threadIdx.x; o < (te - tb) * NQ * 64; o += blockDim.x) {
    const int tl = o / (NQ * 64), q = (o / 64) % NQ, l = o % 64;
    float s = 0.0f;
    for (int w = 0; w < nw; w++) s += accb[((w * tiles_per_wg + tl) * NQ + q) * 64 + l];
    const int tk = 4 * q + (l >> 4), row = (tb + tl) * 16 + (l & 15);
    if (tk < M && row < N) y.put((size_t)tk * N + row, tk, s);
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

// x staged once for every workgroup of the GEMV or verify kernel: one wave per 512-value pass
// (blockIdx.y = token) writes the slots and sums, laid out exactly as those kernels' LDS
// (block <= 128; one image of img_words(K) 16-byte words per token).
__global__ __launch_bounds__(64) void affine_prestage_kernel(FAffine<64, false>::Args a, const uint16_t *__restrict__ x,
                                                             u4 *__restrict__ img) {
  using F = FAffine<64, false>;
  const int ug = (F::units(a.K) + 15) / 16;
  const int c0 = blockIdx.x, nw = gridDim.x;
  x += (size_t)blockIdx.y * a.K;  // token
  img += (size_t)blockIdx.y * F::img_words(a.K);
  F::stage_group(a, img, (float *)(img + ug * 16 * F::R), c0, nw, F::load_group(a, x, c0, nw));
}

template <int GS>
static int affine_gemv(const void *x, const float *signs, int block, const uint32_t *codes,
                       const void *scales, const void *biases, int bf16s, int K, int N, const Out &y,
                       hipStream_t st) {
  if (bf16s) {
    const typename FAffine<GS, true>::Args a{codes, (const uint16_t *)scales, (const uint16_t *)biases, signs, block, K, N};
    return launch_gemv<FAffine<GS, true>>(a, x, y.y, st, y.dt, y.rs);
  }
  const typename FAffine<GS, false>::Args a{codes, (const uint16_t *)scales, (const uint16_t *)biases, signs, block, K, N};
  return launch_gemv<FAffine<GS, false>>(a, x, y.y, st, y.dt, y.rs);
}

template <int GS, bool BF16S, int NQ>
static int affine_vgemm_launch(const void *x, int M, int K, const uint32_t *codes, const void *scales,
                               const void *biases, int N, const Out &y, hipStream_t st, const float *signs,
                               int block, const u4 *img) {
  using F = FAffine<GS, BF16S>;
  constexpr int D = NQ == 1 ? 6 : 4;  // ring depth, measured best per token-quad count on MI355X
  const int ntiles = (N + 15) / 16;
  // tiles per workgroup: one round of CUs, at most 16 / NQ (the waves' per-tile partials live in
  // LDS: a very wide output, such as a vocabulary head, takes several rounds instead)
  const int T = std::min((ntiles + num_cu_aff() - 1) / num_cu_aff(), std::max(1, 16 / NQ));
  const int wgs = (ntiles + T - 1) / T;
  constexpr int NW = 8;  // waves per workgroup: two per SIMD, so one issues while the other waits
  const size_t fixed = 128 * 16 + (size_t)NW * T * NQ * 64 * 4;
  const size_t budget = 150 * 1024;
  int Kc = K;
  auto need = [&](int kc) { return fixed + (size_t)M * (F::img_words(kc) + 1) * 16; };
  const int kstep = img ? 1024 : 256;  // image chunks must start on a 16-unit group
  while (Kc > kstep && need(Kc) > budget) Kc = (Kc - 1) / kstep * kstep;
  if (need(Kc) > budget) return decline("verify workspace does not fit in LDS");
  const size_t lds = need(Kc);
  hipLaunchKernelGGL((affine_vgemm<GS, BF16S, NQ, D>), dim3(wgs), dim3(64 * NW), lds, st, (const uint16_t *)x, M, K,
                     codes, (const uint16_t *)scales, (const uint16_t *)biases, N, y, Kc, T, signs,
                     block, img);
  ISHZ_LAUNCH_CHECK("affine verify launch");
  return ISHZ_OK;
}

template <int GS, bool BF16S>
static int affine_vgemm_nq(const void *x, int M, int K, const uint32_t *codes, const void *scales,
                           const void *biases, int N, const Out &y, hipStream_t st, const float *signs = nullptr,
                           int block = 0, const u4 *img = nullptr) {
  switch ((M + 3) / 4) {
    case 1: return affine_vgemm_launch<GS, BF16S, 1>(x, M, K, codes, scales, biases, N, y, st, signs, block, img);
    case 2: return affine_vgemm_launch<GS, BF16S, 2>(x, M, K, codes, scales, biases, N, y, st, signs, block, img);
    case 3: return affine_vgemm_launch<GS, BF16S, 3>(x, M, K, codes, scales, biases, N, y, st, signs, block, img);
    default: return affine_vgemm_launch<GS, BF16S, 4>(x, M, K, codes, scales, biases, N, y, st, signs, block, img);
  }
}

template <int GS>
static int affine_verify_launch(const void *x, int M, int K, const uint32_t *codes,
                                const void *scales, const void *biases, int bf16s, int N, const Out &y,
                                hipStream_t st) {
  if (K % 256 == 0)
    return bf16s ? affine_vgemm_nq<GS, true>(x, M, K, codes, scales, biases, N, y, st)
                 : affine_vgemm_nq<GS, false>(x, M, K, codes, scales, biases, N, y, st);
  constexpr int T = 2;
  const int wgs = (N + 16 * T - 1) / (16 * T);
  const int groups = K / 64;
  int ks = 1;
  while (ks < 16 && ks < groups && wgs * ks < num_cu_aff() * 16) ks *= 2;
  hipLaunchKernelGGL((affine_verify<GS, T>), dim3(wgs), dim3(64 * ks), (size_t)ks * T * 256 * 4, st,
                     (const uint16_t *)x, M, K, codes, (const uint16_t *)scales,
                     (const uint16_t *)biases, bf16s, N, y);
  ISHZ_LAUNCH_CHECK("affine verify launch");
  return ISHZ_OK;
}

// fp32 activations (precise.h): w = s * q + b in fp32 (mul, then add: the oracle's and MLX's
// dequantize), q the bits-wide field k of the row's little-endian u32 stream.
struct AffDec {
  struct Args {
    const uint32_t *codes;
    const uint16_t *scales, *biases;
    int K, bits, group;
    bool bf16s;
  };
  static DEV void decode(const Args &a, int row, int s, float *v) {
    const size_t wpr = (size_t)a.K * a.bits / 32;
    const uint32_t *rw = a.codes + (size_t)row * wpr;
    const size_t g = (size_t)row * (a.K / a.group) + (size_t)(8 * s) / a.group;
    const float sc = ld_scale(a.scales + g, a.bf16s), bi = ld_scale(a.biases + g, a.bf16s);
    const uint32_t mask = (1u << a.bits) - 1;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const size_t bit = (size_t)(8 * s + i) * a.bits;
      const size_t w = bit / 32;
      const int off = (int)(bit % 32);
      uint32_t q = rw[w] >> off;
      if (off + a.bits > 32) q |= rw[w + 1] << (32 - off);
      v[i] = __fadd_rn(__fmul_rn(sc, (float)(q & mask)), bi);
    }
  }
};

// Exact weights, fp32 sums: fp32 x (its precision), and fp16 / bf16 x with groups other than 64 /
// 128 (the fp16 kernels' layouts). y in x's dtype.
static int affine_precise(const void *x, int xdt, int M, int K, const uint32_t *codes, const void *scales,
                          const void *biases, int bf16s, int N, int bits, int group, void *y, hipStream_t st) {
  const AffDec::Args a{codes, (const uint16_t *)scales, (const uint16_t *)biases, K, bits, group, bf16s != 0};
  return launch_precise<AffDec>(a, x, xdt, M, K, N, y, st);
}

static int check_affine(const void *x, int x_dtype, int M, int K, const void *codes,
                        const void *scales, const void *biases, int scale_dtype, int N, int bits,
                        int group, const void *y) {
  if (x_dtype != ISHZ_DT_F16 && x_dtype != ISHZ_DT_BF16 && x_dtype != ISHZ_DT_F32)
    return decline("activations must be fp16, bf16 or fp32");
  if (bits < 2 || bits > 8) return decline("packs of 2 to 8 bits are decoded in-kernel");
  if (group < 32 || group % 32 || K % group) return decline("group size must be a multiple of 32 dividing K");
  if (scale_dtype != ISHZ_DT_F16 && scale_dtype != ISHZ_DT_BF16) return decline("scales must be fp16 or bf16");
  if (M < 1 || M > 16) return decline("row count outside 1..16");
  if (K <= 0 || K % 128 || N <= 0) return decline("K must be a positive multiple of 128");
  if (!x || !codes || !scales || !biases || !y) return einval("null pointer");
  return ISHZ_OK;
}

// Packs of 3 to 8 bits (x already rotated when the layer rotates).
static int affine_nbit_dispatch(const void *x, int M, int K, const uint32_t *codes, const void *scales,
                                const void *biases, int bf16s, int N, int bits, int group, const Out &y,
                                hipStream_t st) {
#define ISHZ_NB(B)                                                                                      \
  case B:                                                                                              \
    if (group == 64)                                                                                   \
      return bf16s ? affine_nbit<B, 64, true>(x, M, K, codes, scales, biases, N, y, st)                \
                   : affine_nbit<B, 64, false>(x, M, K, codes, scales, biases, N, y, st);              \
    return bf16s ? affine_nbit<B, 128, true>(x, M, K, codes, scales, biases, N, y, st)                 \
                 : affine_nbit<B, 128, false>(x, M, K, codes, scales, biases, N, y, st);
  switch (bits) {
    ISHZ_NB(3)
    ISHZ_NB(4)
    ISHZ_NB(5)
    ISHZ_NB(6)
    ISHZ_NB(7)
    ISHZ_NB(8)
  }
#undef ISHZ_NB
  return decline("packs of 2 to 8 bits are decoded in-kernel");
}

static int affine_dispatch(const void *x, int M, int K, const float *signs, int block,
                           const uint32_t *codes, const void *scales, const void *biases,
                           int bf16s, int N, int group, const Out &y, hipStream_t st) {
  if (M == 1) {
    return group == 64 ? affine_gemv<64>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st)
                       : affine_gemv<128>(x, signs, block, codes, scales, biases, bf16s, K, N, y, st);
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
  hipStream_t st = S(stream);
  if (x_dtype == ISHZ_DT_F32 || (group != 64 && group != 128))
    return affine_precise(x, x_dtype, M, K, codes, scales, biases, scale_dtype == ISHZ_DT_BF16, N, bits, group, y, st);
  StreamTemp tmp(st);  // bf16 activations: their fp16 image
  if (x_dtype != ISHZ_DT_F16 && (rc = tmp.get(act_image_bytes(M, K)))) return rc;
  const uint16_t *xh;
  const float *rs;
  if ((rc = act_prepare(x, x_dtype, M, K, tmp.p, st, &xh, &rs))) return rc;
  const Out o{y, x_dtype, rs};
  if (bits != 2)
    return affine_nbit_dispatch(xh, M, K, codes, scales, biases, scale_dtype == ISHZ_DT_BF16, N, bits, group, o, st);
  return affine_dispatch(xh, M, K, nullptr, 0, codes, scales, biases, scale_dtype == ISHZ_DT_BF16, N, group, o, st);
}

// Room for the rotated activations (fp16, general path) or every row's staged x image (what the
// verify workgroups copy; a null or smaller workspace stages x in every workgroup); bf16 / fp32
// activations: x rotated in its own dtype (up to 4 bytes a value), then its fp16 image. One fp16
// row needs none: the GEMV rotates and stages x in each workgroup.
extern "C" size_t ishz_affine_workspace_size(int M, int K) {
  if (K <= 0 || M <= 0) return 0;
  const size_t f16 = std::max((size_t)M * K * 2, (size_t)M * FAffine<64, false>::img_words(K) * 16);
  return std::max(f16, (size_t)M * K * 4 + act_image_bytes(M, K));
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
  if (x_dtype != ISHZ_DT_F16) {
    // hadamardRotate in x's own dtype (Core/Hadamard.swift:8-23, the rotated activation the
    // reference multiplies), then its fp16 image and the unrotated product
    if (!workspace || workspace_bytes < ishz_affine_workspace_size(M, K))
      return einval("workspace too small (ishz_affine_workspace_size)");
    const void *xr = x;
    void *img = workspace;
    if (block > 0) {
      if ((rc = ishz_hadamard(x, x_dtype, M, K, block, signs, 0, workspace, stream))) return rc;
      xr = workspace;
      img = (char *)workspace + (size_t)M * K * 4;
    }
    if (x_dtype == ISHZ_DT_F32 || (group != 64 && group != 128))
      return affine_precise(xr, x_dtype, M, K, codes, scales, biases, bf16s, N, bits, group, y, st);
    const uint16_t *xh;
    const float *rs;
    if ((rc = act_prepare(xr, x_dtype, M, K, img, st, &xh, &rs))) return rc;
    const Out o{y, x_dtype, rs};
    if (bits != 2) return affine_nbit_dispatch(xh, M, K, codes, scales, biases, bf16s, N, bits, group, o, st);
    return affine_dispatch(xh, M, K, nullptr, 0, codes, scales, biases, bf16s, N, group, o, st);
  }
  const Out o{y, ISHZ_DT_F16, nullptr};
  if (group != 64 && group != 128) {  // other groups: x rotated once into the workspace, exact weights
    if (block == 0) return affine_precise(x, ISHZ_DT_F16, M, K, codes, scales, biases, bf16s, N, bits, group, y, st);
    if (!workspace || workspace_bytes < ishz_affine_workspace_size(M, K))
      return einval("workspace too small (ishz_affine_workspace_size)");
    if ((rc = ishz_hadamard(x, ISHZ_DT_F16, M, K, block, signs, 0, workspace, stream))) return rc;
    return affine_precise(workspace, ISHZ_DT_F16, M, K, codes, scales, biases, bf16s, N, bits, group, y, st);
  }
  if (bits != 2) {  // 3- to 8-bit packs: rotate x once into the workspace, then the matmul
    if (block == 0) return affine_nbit_dispatch(x, M, K, codes, scales, biases, bf16s, N, bits, group, o, st);
    if (!workspace || workspace_bytes < ishz_affine_workspace_size(M, K))
      return einval("workspace too small (ishz_affine_workspace_size)");
    rc = ishz_hadamard(x, ISHZ_DT_F16, M, K, block, signs, 0, workspace, stream);
    if (rc) return rc;
    return affine_nbit_dispatch(workspace, M, K, codes, scales, biases, bf16s, N, bits, group, o, st);
  }
  if (block == 0 || M == 1)
    return affine_dispatch(x, M, K, signs, block, codes, scales, biases, bf16s, N, group, o, st);
  if (block <= 128 && K % 256 == 0) {
    // x rotated and staged once into the workspace (every token's image), else the rotation is
    // fused into each workgroup's staging; two tokens rotate faster in the workgroups than the
    // extra launch costs (measured on MI355X at 17408x5120: 14.3 vs 15.3 us; from four tokens up
    // the prestaged image wins)
    const u4 *img = nullptr;
    if (M > 2 && workspace && workspace_bytes >= ishz_affine_workspace_size(M, K)) {
      const FAffine<64, false>::Args a{codes, nullptr, nullptr, signs, block, K, N};
      hipLaunchKernelGGL(affine_prestage_kernel, dim3((K + 511) / 512, M), dim3(64), 0, st, a, (const uint16_t *)x,
                         (u4 *)workspace);
      ISHZ_LAUNCH_CHECK("affine prestage launch");
      img = (const u4 *)workspace;
    }
    if (group == 64)
      return bf16s ? affine_vgemm_nq<64, true>(x, M, K, codes, scales, biases, N, o, st, signs, block, img)
                   : affine_vgemm_nq<64, false>(x, M, K, codes, scales, biases, N, o, st, signs, block, img);
    return bf16s ? affine_vgemm_nq<128, true>(x, M, K, codes, scales, biases, N, o, st, signs, block, img)
                 : affine_vgemm_nq<128, false>(x, M, K, codes, scales, biases, N, o, st, signs, block, img);
  }
  if (!workspace || workspace_bytes < ishz_affine_workspace_size(M, K))
    return einval("workspace too small (ishz_affine_workspace_size)");
  rc = ishz_hadamard(x, ISHZ_DT_F16, M, K, block, signs, 0, workspace, stream);
  if (rc) return rc;
  return affine_dispatch(workspace, M, K, nullptr, 0, codes, scales, biases, bf16s, N, group, o, st);
}
