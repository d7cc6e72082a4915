// MLX affine 2-bit packs as the GEMV skeleton reads them (FAffine), with the Walsh-Hadamard
// rotation of x fused into the staging, and the LDS transform for blocks above 128.
// Pack format (Quantize/WeightedAffineQuantizer.swift:142-153): codes u32 [N][K/16], code k at
// bits 2*(k%16) of word k/16; scales and biases [N][K/GS]; w = s*q + b.
#pragma once
#include "common.h"
#include "gemv.h"

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

// ------------------------------------------------------------------- GEMV (M = 1)
// Format for the shared streaming GEMV skeleton. Unit = 64 weights = 16 bytes of codes (4 words)
// of one row, with its group's scale and bias. Slot r of a unit is word t = r / 2, pairs
// p = 4 (r % 2) .. +3: the x at offsets p and p + 8 of the word's 16, divided by 4^i of the pair.
// Sums: 0 = 1024 * the unit's staged x' (the code offset), 1 = the unit's plain x (the bias).
template <int GS, bool BF16S>
struct FAffine {
  struct Args {
    const uint32_t *codes;
    const uint16_t *scales, *biases;
    const float *signs;
    int block;  // Hadamard block (0: x is not rotated)
    int K, N;
  };
  struct Raw {
    u4 q;
    uint32_t s, b;
  };
  struct LaneC {};
  // ring depth 3: measured best on MI355X at 17408x5120 with and without the rotation (9.5 vs
  // 10.4 us at 5 rotated)
  static constexpr int R = 8, Q = 2, RING = 3, GRID_ENTRIES = 0;
  // 512 threads: eight waves share one staged (and rotated) x, so at most two 512-element
  // rotation passes per wave at K = 5120.
  static constexpr int WG = 512;
  static __host__ __device__ int units(int K) { return K / 64; }
  // 16-byte words of the staged x: slots, then the two sums per unit.
  static __host__ __device__ int img_words(int K) { return (units(K) + 15) / 16 * (16 * R + 4 * Q); }
  // Resident waves per SIMD the grid is sized for: with a plain x copy, many short waves balance
  // the SIMDs best; rotating x while staging favours fewer, longer waves.
  static int occ(const Args &a) { return a.block > 0 ? 2 : 4; }
  // Blocks above 128 are rotated in an LDS copy of x (one fp32 per element).
  static size_t extra_lds_bytes(const Args &a) { return a.block > 128 ? (size_t)a.K * 4 : 0; }
  static DEV LaneC lane(int) { return {}; }
  static DEV Raw load(const Args &a, int row, int u) {
    const size_t g = (size_t)row * (a.K / GS) + (64 * u) / GS;
    return {*(const u4 *)(a.codes + (size_t)row * (a.K / 16) + 4 * u), a.scales[g], a.biases[g]};
  }

  // Writes x[k], x[k + 1] (k even, already rotated and rounded to fp16) to their slots and
  // returns their contributions to the unit's sums.
  static DEV void put2(uint16_t *xh, int k, float v0, float v1, float &c, float &xsum) {
    c = 0.0f;
    xsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const float v = e ? v1 : v0;
      const int kk = k + e, u = kk >> 6, w = kk & 63, q = w & 15, p = q & 7;
      const int r = 2 * (w >> 4) + (p >> 2);
      const uint16_t h = f2h(__builtin_ldexpf(v, -2 * (p < 5 ? p : p - 5)));  // x / 4^i, exact
      xh[((u >> 4) * 16 * R + r * 16 + (u & 15)) * 8 + (p & 3) * 2 + (q >> 3)] = h;
      c += h2f(h);
      xsum += v;
    }
  }
  static DEV void put_sums(float *xsum, int k, float c, float xs) {
    c = group_sum<32>(c);
    xs = group_sum<32>(xs);
    if ((threadIdx.x & 31) == 0) {
      const int u = k >> 6;
      float *sm = xsum + (u >> 4) * 16 * Q + (u & 15);
      sm[0] = 1024.0f * c;
      sm[16] = xs;
    }
  }

  // x[k .. k + 7] (k % 8 == 0, rotated and rounded to fp16) of lane l and x[k ^ 8 ...] of lane
  // l ^ 1 fill two slots of one code word: the lanes swap the halves the other writes (one DPP
  // per dword pair), so each writes one whole 16-byte slot. Unit sums over 8 lanes by DPP.
  static DEV void put8(u4 *xs, float *xsum, int k, const float *v, bool valid) {
    const int t = (k >> 4) & 3, hf = (k >> 3) & 1, u = k >> 6;
    uint32_t h[8];
    float c = 0.0f, xsm = 0.0f;
#pragma unroll
    for (int p = 0; p < 8; p++) {
      h[p] = f2h(__builtin_ldexpf(v[p], -2 * (p < 5 ? p : p - 5)));  // x / 4^i, exact
      xsm += v[p];
    }
#pragma unroll
    for (int p = 0; p < 8; p += 2) c = dot2(h[p] | h[p + 1] << 16, 0x3C003C00u, c);  // + h_p + h_p+1
    // Selects by mask (a select between two elements of h would become a dynamic index, i.e.
    // scratch memory).
    const uint32_t hm = 0u - (uint32_t)hf;
    uint32_t keep[4], send[2];
#pragma unroll
    for (int j = 0; j < 4; j++) keep[j] = (h[4 + j] & hm) | (h[j] & ~hm);
#pragma unroll
    for (int j = 0; j < 2; j++)
      send[j] = ((h[2 * j] | h[2 * j + 1] << 16) & hm) | ((h[4 + 2 * j] | h[5 + 2 * j] << 16) & ~hm);
    uint32_t rv[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
      rv[j] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)send[j], 0xB1, 0xf, 0xf, true);  // lane ^ 1
    u4 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t r = (rv[j >> 1] >> (16 * (j & 1))) & 0xffffu;
      o[j] = hf ? (r | keep[j] << 16) : (keep[j] | r << 16);
    }
    if (valid) xs[(u >> 4) * 16 * R + (2 * t + hf) * 16 + (u & 15)] = o;
    c = group_sum<8>(c);
    xsm = group_sum<8>(xsm);
    if (valid && (threadIdx.x & 7) == 0) {
      float *sm = xsum + (u >> 4) * 16 * Q + (u & 15);
      sm[0] = 1024.0f * c;
      sm[16] = xsm;
    }
  }

  // Butterfly inside a lane: pairs (i, i + H) of its eight values.
  template <int H>
  static DEV void lbfly(float *v) {
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (!(i & H)) {
        const float p = v[i], q = v[i + H];
        v[i] = p + q;
        v[i + H] = p - q;
      }
  }

  // Butterfly across lanes: partner = lane ^ m (m = 1, 2, 4, 8 within a 16-lane row, from DPP
  // quad permutes and row mirrors); the lower lane keeps a + b, the upper b's partner - b, both as
  // fma(v, +-1, partner) (exact products, so one rounding, as the add or subtract): one DPP move
  // and one FMA per value instead of an add, a subtract and a select. sgn = -1 on the upper lanes.
  template <int M>
  static DEV float xbfly(float v, float sgn) {
    float t;
    if constexpr (M == 1) t = ISHZ_DPP(v, 0xB1);
    else if constexpr (M == 2) t = ISHZ_DPP(v, 0x4E);
    else if constexpr (M == 4) t = ISHZ_DPP(ISHZ_DPP(v, 0x141), 0x1B);  // half mirror, quad reverse
    else t = ISHZ_DPP(ISHZ_DPP(v, 0x141), 0x140);                      // half mirror, mirror
    return __builtin_fmaf(v, sgn, t);
  }

  // hadamardRotate on a lane's eight consecutive values: sign flip, butterflies (h = 1, 2, 4
  // in-lane, 8 .. 64 across lanes) and 1/sqrt(block), rounded to fp16 (block <= 128).
  static DEV void rot8(float *v, const f4 *sg, int bl, float scale, int lane) {
    if (sg)
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] *= sg[e >> 2][e & 3];
    const float sg1 = lane & 1 ? -1.0f : 1.0f, sg2 = lane & 2 ? -1.0f : 1.0f;
    const float sg4 = lane & 4 ? -1.0f : 1.0f, sg8 = lane & 8 ? -1.0f : 1.0f;
    if (bl > 1) lbfly<1>(v);
    if (bl > 2) lbfly<2>(v);
    if (bl > 4) lbfly<4>(v);
    if (bl > 8)
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = xbfly<1>(v[e], sg1);
    if (bl > 16)
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = xbfly<2>(v[e], sg2);
    if (bl > 32)
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = xbfly<4>(v[e], sg4);
    if (bl > 64)
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = xbfly<8>(v[e], sg8);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (float)(_Float16)(v[e] * scale);
  }

  // Eight consecutive x per lane, 512 per wave pass: hadamardRotate's sign flip, butterflies
  // (h = 1, 2, 4 in-lane, 8 .. 64 across lanes) and 1/sqrt(block), rounded to fp16 as the
  // reference's rotated activation is, then written to the slots. Loads for PF passes are issued
  // before any is used. One barrier.
  static constexpr int PF = 4;
  struct XPre {
    u4 xv[PF];
    f4 sg[PF][2];
  };
  static DEV XPre load_group(const Args &a, const uint16_t *x, int c0, int nw) {
    const int lane = threadIdx.x & 63;
    const int npass = (a.K + 511) / 512;
    XPre p;
#pragma unroll
    for (int j = 0; j < PF; j++) {
      const int k = min(min(c0 + j * nw, npass - 1) * 512 + 8 * lane, a.K - 8);
      p.xv[j] = *(const u4 *)(x + k);
      if (a.signs) {
        p.sg[j][0] = *(const f4 *)(a.signs + k);
        p.sg[j][1] = *(const f4 *)(a.signs + k + 4);
      }
    }
    return p;
  }
  // Rotates and stages passes c0, c0 + nw, ... (PF of them) of this wave from their loads, into
  // LDS or (prestage) into the global image.
  static DEV void stage_group(const Args &a, u4 *xs, float *xsum, int c0, int nw, const XPre &cur) {
    const int lane = threadIdx.x & 63;
    const int bl = a.block;
    const float scale = bl > 1 ? 1.0f / __builtin_sqrtf((float)bl) : 1.0f;
    const int npass = (a.K + 511) / 512;
#pragma unroll
    for (int j = 0; j < PF; j++) {
      if (c0 + j * nw >= npass) break;
      const int k = (c0 + j * nw) * 512 + 8 * lane;
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const h2 hv = as_h2(cur.xv[j][e]);
        v[2 * e] = (float)hv.x;
        v[2 * e + 1] = (float)hv.y;
      }
      if (bl > 0) rot8(v, a.signs ? cur.sg[j] : nullptr, bl, scale, lane);
      put8(xs, xsum, k, v, k < a.K);
    }
  }

  static DEV XPre stage_load(const Args &a, const uint16_t *x, int) {
    XPre p{};
    if (a.block > 128) return p;
    return load_group(a, x, threadIdx.x >> 6, blockDim.x >> 6);
  }
  static DEV void stage(const Args &a, const uint16_t *x, u4 *xs, float *xsum, u4 *extra, int, const XPre &pre) {
    const int lane = threadIdx.x & 63, wave = wave_id(), nw = blockDim.x >> 6;
    if (a.block > 128) {
      uint16_t *xh = (uint16_t *)xs;
      float *xr = (float *)extra;
      for (int i = threadIdx.x; i < a.K; i += blockDim.x) xr[i] = h2f(x[i]);
      lds_wht(xr, a.K, a.block, a.signs, false);  // ends with a barrier
      for (int c0 = wave * 128; c0 < a.K; c0 += nw * 128) {
        const int k = c0 + 2 * lane;
        float c, s;
        put2(xh, k, (float)(_Float16)xr[k], (float)(_Float16)xr[k + 1], c, s);
        put_sums(xsum, k, c, s);
      }
      __syncthreads();
      return;
    }
    const int npass = (a.K + 511) / 512;
    stage_group(a, xs, xsum, wave, nw, pre);  // first group: loads issued by stage_load
    for (int c0 = wave + PF * nw; c0 < npass; c0 += PF * nw)
      stage_group(a, xs, xsum, c0, nw, load_group(a, x, c0, nw));
    __syncthreads();
  }

  static DEV float ld_s(uint32_t v) { return BF16S ? __builtin_bit_cast(float, v << 16) : h2f(v); }
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &) {
    float S = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t w = r.q[t], w10 = w >> 10;
      const u4 a = s.slot(2 * t), c = s.slot(2 * t + 1);
      S = dot2(and_or(w, 0x00030003u, s.mg), a.x, S);
      S = dot2(and_or(w, 0x000C000Cu, s.mg), a.y, S);
      S = dot2(and_or(w, 0x00300030u, s.mg), a.z, S);
      S = dot2(and_or(w, 0x00C000C0u, s.mg), a.w, S);
      S = dot2(and_or(w, 0x03000300u, s.mg), c.x, S);
      S = dot2(and_or(w10, 0x00030003u, s.mg), c.y, S);
      S = dot2(and_or(w10, 0x000C000Cu, s.mg), c.z, S);
      S = dot2(and_or(w10, 0x00300030u, s.mg), c.w, S);
    }
    return ld_s(r.s) * (S - s.sum(0)) + ld_s(r.b) * s.sum(1);
  }
};

}  // namespace ishz
