// GGML block formats as the gfx950 kernels read them: one struct per format.
//
// Block layouts follow the CPU definition in Sources/IshizukiKit/Core/GGMLDequant.swift (cited per
// format); Q4_0 follows ggml's block_q4_0 (the reference has no decoder for it).
//
// Two readers per format:
//  * GEMV (M = 1). A "unit" is a fixed slice of a row's block bytes (16 B of codes: 32 or 64
//    weights). Lanes stream units of one row with 128-bit loads; a unit's dot product with x is
//    formed from exact fp16 codes (v_dot2_f32_f16) and scaled once per scale group in fp32. x
//    sits in LDS as fp16 with every aligned group of four reordered (x0, x2, x1, x3), so the
//    two halves a nibble/byte mask pulls out of one code word meet their activations in one
//    dword.
//  * Verify (M = 2..16 on MFMA). Tokens are the A operand (16 rows, M used), decoded weights the
//    B operand (16 weight rows = 16 columns), so the lane that decoded weight row j also holds
//    C column j and applies that row's scale itself. A step is one scale group (32 or 16
//    weights); B holds exact integer codes and the scale multiplies the fp32 C tile.
#pragma once
#include "common.h"
#include <algorithm>

namespace ishz {

// LDS working set of the GEMV kernel. x is stored in the order lanes consume it: a unit reads R
// 16-byte slots (8 fp16 x each, pair-permuted) and Q sums of 16 x. Slot r of unit u lives at
// (u / 16) * 16R + r * 16 + u % 16, so the 16 lanes that read slot r of 16 consecutive units in
// one instruction touch 256 contiguous bytes: every LDS bank once, no conflicts.
struct GemvShared {
  uint32_t mg;           // 0x64006400 held in a VGPR (magic exponent for code -> fp16)
  const u4 *x;
  const float *xsum;
  const u4 *grid;        // i-quant grid as fp16, permuted like x (IQ2_XS only)
  const u4 *sgn;         // i-quant sign masks for the same order (IQ2_XS only)
  template <int R>
  DEV u4 slot(int u, int r) const { return x[(u >> 4) * 16 * R + r * 16 + (u & 15)]; }
  template <int Q>
  DEV float sum(int u, int q) const { return xsum[(u >> 4) * 16 * Q + q * 16 + (u & 15)]; }
};

DEV void unpack(u4 a, u4 b, uint32_t *d) {
  d[0] = a.x, d[1] = a.y, d[2] = a.z, d[3] = a.w, d[4] = b.x, d[5] = b.y, d[6] = b.z, d[7] = b.w;
}

// x0..x7 (natural) -> (x0,x2,x1,x3, x4,x6,x5,x7): the order of the nibble/byte pairs below.
DEV u4 perm0213(u4 a) {
  u4 r;
  r.x = (a.x & 0xffffu) | (a.y << 16);
  r.y = (a.x >> 16) | (a.y & 0xffff0000u);
  r.z = (a.z & 0xffffu) | (a.w << 16);
  r.w = (a.z >> 16) | (a.w & 0xffff0000u);
  return r;
}
DEV u2 perm0213(u2 a) {
  u2 r;
  r.x = (a.x & 0xffffu) | (a.y << 16);
  r.y = (a.x >> 16) | (a.y & 0xffff0000u);
  return r;
}

// Sum over the 8 fp16 x pairs of a lane's operand (as dwords) times codes.
DEV float dot8(const uint32_t *c, const uint32_t *x, float acc) {
#pragma unroll
  for (int i = 0; i < 8; i++) acc = dot2(c[i], x[i], acc);
  return acc;
}

// 6-bit scale and min of sub-block j of a Q4_K block; s0..s2 are header bytes 4..15
// (GGMLDequant.q4K.scaleMin, Core/GGMLDequant.swift:193-205).
DEV void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &m) {
  const int sh = 8 * (j & 3);
  const uint32_t a = s0 >> sh, b = s1 >> sh, c = s2 >> sh;
  if (j < 4) {
    sc = a & 63;
    m = b & 63;
  } else {
    sc = (c & 15) | ((a >> 6) & 3) << 4;
    m = ((c >> 4) & 15) | ((b >> 6) & 3) << 4;
  }
}

// ------------------------------------------------------------------------------------- Q4_0
// ggml block_q4_0: fp16 d at 0, qs[16] at 2; element j = (lo(qs[j]) - 8) d, j + 16 = hi.
struct FQ4_0 {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q4_0;
  static constexpr int BS = 32, TS = 18, UPB = 1;  // unit: the whole block, 32 weights
  static constexpr int BATCH = 4;  // units per lane per batch (two batches in flight)
  static constexpr bool XSUM = true, GRID = false;
  static constexpr int R = 4, Q = 2;  // x slots: lo run k0, k0+8, hi run k0+16, k0+24
  static DEV int slot_k(int u, int r) { return 32 * u + 8 * r; }
  static DEV int sum_k(int u, int q) { return 32 * u + 16 * q; }
  static constexpr int SUM_LEN = 16;
  struct Raw {
    u4 q;
    uint32_t d;
  };
  static DEV Raw load(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)u * TS;
    return {ld16<2>(p + 2), ld2(p)};
  }
  // Low nibbles become 1024 + q and high nibbles 1024 + 16q (masked in place, no shift); the
  // offsets come back out through the per-16 sums of x.
  static DEV float dot(const Raw &r, int u, const GemvShared &s) {
    uint32_t xl[8], xh[8], lo[8], hi[8];
    unpack(s.slot<R>(u, 0), s.slot<R>(u, 1), xl);
    unpack(s.slot<R>(u, 2), s.slot<R>(u, 3), xh);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t q = r.q[t], q8 = q >> 8;
      lo[2 * t] = and_or(q, 0x000F000Fu, s.mg);
      lo[2 * t + 1] = and_or(q8, 0x000F000Fu, s.mg);
      hi[2 * t] = and_or(q, 0x00F000F0u, s.mg);
      hi[2 * t + 1] = and_or(q8, 0x00F000F0u, s.mg);
    }
    const float sl = dot8(lo, xl, 0.0f), sh = dot8(hi, xh, 0.0f);
    const float xs_l = s.sum<Q>(u, 0), xs_h = s.sum<Q>(u, 1);
    return h2f(r.d) * ((sl - 1032.0f * xs_l) + (0.0625f * sh - 72.0f * xs_h));
  }

  // Verify: one MFMA 16x16x32 per block. Lane group g takes k = 8g..8g+7: lo nibbles of bytes
  // 0..7 (g=0), 8..15 (g=1), hi nibbles of the same (g=2,3).
  static constexpr int VSTEP = 32;
  template <int T>
  static DEV void vblock(const uint8_t *const *rows, int b, int g, const uint16_t *xr, bool tok,
                         f4 *acc) {
    u4 a = tok ? ld16<16>((const uint8_t *)(xr + b * 32 + 8 * g)) : u4{0, 0, 0, 0};
    const h8 A = as_h8(perm0213(a));
    const int sh = (g >> 1) * 4;
#pragma unroll
    for (int t = 0; t < T; t++) {
      const uint8_t *p = rows[t] + (size_t)b * TS;
      const u2 q = ld8<2>(p + 2 + 8 * (g & 1));
      const float d = h2f(ld2(p));
      u4 B;
      B.x = unmagic((q.x >> sh) & 0x000F000Fu, 1032);
      B.y = unmagic((q.x >> (sh + 8)) & 0x000F000Fu, 1032);
      B.z = unmagic((q.y >> sh) & 0x000F000Fu, 1032);
      B.w = unmagic((q.y >> (sh + 8)) & 0x000F000Fu, 1032);
      const f4 c = mfma32(A, as_h8(B), f4{0, 0, 0, 0});
      acc[t] += d * c;
    }
  }
};

// ------------------------------------------------------------------------------------- Q4_K
// GGMLDequant.q4K (Core/GGMLDequant.swift:187-220): d, dmin fp16 at 0, 2; 12 B of 6-bit
// scales/mins at 4; qs[128] at 16. 64-weight chunk jj: low nibbles of qs[32jj+l] are weights
// 64jj+l (sub-block 2jj), high nibbles 64jj+32+l (sub-block 2jj+1); w = d*sc*q - dmin*m.
struct FQ4_K {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q4_K;
  static constexpr int BS = 256, TS = 144, UPB = 4;  // unit: 32 B of qs (chunk jj), 64 weights
  static constexpr int BATCH = 2;
  static constexpr bool XSUM = true, GRID = false;
  static constexpr int R = 8, Q = 2;  // slots: lo run k0 + 8i (i < 4), hi run k0 + 32 + 8i
  static DEV int k0_of(int u) { return (u >> 2) * 256 + (u & 3) * 64; }
  static DEV int slot_k(int u, int r) { return k0_of(u) + 8 * r; }
  static DEV int sum_k(int u, int q) { return k0_of(u) + 32 * q; }
  static constexpr int SUM_LEN = 32;
  // The four lanes of a block (a quad: units are consecutive per lane) each load one dword of
  // its 16-byte header and share them by quad broadcast, so the header is read once.
  struct Raw {
    u4 q0, q1;
    uint32_t h;
  };
  static DEV Raw load(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)(u >> 2) * TS;
    const uint8_t *qs = p + 16 + 32 * (u & 3);
    return {ld16<16>(qs), ld16<16>(qs + 16), ld4<4>(p + 4 * (u & 3))};
  }
  // Chunk jj: low nibbles of its 32 bytes are sub-block 2jj (weights k0..k0+31), high nibbles
  // sub-block 2jj+1 (k0+32..k0+63). Low nibbles become 1024 + q, high ones 1024 + 16q, and
  // with S = sum code * x and X = sum x over the sub-block: sum q x = S - 1024 X, or S/16 - 64 X.
  static DEV float dot(const Raw &r, int u, const GemvShared &s) {
    const int jj = u & 3;
    uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int hb = 0; hb < 2; hb++) {
      uint32_t xl[8], xh[8];
      unpack(s.slot<R>(u, 2 * hb), s.slot<R>(u, 2 * hb + 1), xl);
      unpack(s.slot<R>(u, 4 + 2 * hb), s.slot<R>(u, 5 + 2 * hb), xh);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t q = qw[4 * hb + t], q8 = q >> 8;
        sl = dot2(and_or(q, 0x000F000Fu, s.mg), xl[2 * t], sl);
        sl = dot2(and_or(q8, 0x000F000Fu, s.mg), xl[2 * t + 1], sl);
        sh = dot2(and_or(q, 0x00F000F0u, s.mg), xh[2 * t], sh);
        sh = dot2(and_or(q8, 0x00F000F0u, s.mg), xh[2 * t + 1], sh);
      }
    }
    // scales/mins of sub-blocks 2jj, 2jj+1 (GGMLDequant.q4K.scaleMin), branch-free
    const uint32_t h0 = quad_bcast<0>(r.h), s0 = quad_bcast<1>(r.h), s1 = quad_bcast<2>(r.h),
                   s2 = quad_bcast<3>(r.h);
    const bool lo4 = jj < 2;
    const uint32_t sh0 = 16 * (jj & 1);  // byte 2jj & 3 of the scale words
    const uint32_t a0 = s0 >> sh0, b0 = s1 >> sh0, c0 = s2 >> sh0;
    const uint32_t a1 = a0 >> 8, b1 = b0 >> 8, c1 = c0 >> 8;
    const uint32_t sc0 = lo4 ? (a0 & 63) : ((c0 & 15) | ((a0 >> 2) & 48));
    const uint32_t m0 = lo4 ? (b0 & 63) : (((c0 >> 4) & 15) | ((b0 >> 2) & 48));
    const uint32_t sc1 = lo4 ? (a1 & 63) : ((c1 & 15) | ((a1 >> 2) & 48));
    const uint32_t m1 = lo4 ? (b1 & 63) : (((c1 >> 4) & 15) | ((b1 >> 2) & 48));
    const float d = h2f(h0 & 0xffff), dmin = h2f(h0 >> 16);
    const float xs_l = s.sum<Q>(u, 0), xs_h = s.sum<Q>(u, 1);
    const float dl0 = d * (float)sc0, dl1 = d * (float)sc1;
    return dl0 * (sl - 1024.0f * xs_l) - (dmin * (float)m0) * xs_l +
           dl1 * (0.0625f * sh - 64.0f * xs_h) - (dmin * (float)m1) * xs_h;
  }

  // Verify: one MFMA 16x16x32 per sub-block; lane group g takes l = 8g..8g+7 of it, i.e. the
  // low or high nibbles of qs[32jj + 8g .. +7]. The min term needs sum_k x over the sub-block
  // per token: one extra MFMA against a B of ones, shared by every tile.
  static constexpr int VSTEP = 32;
  template <int T>
  static DEV void vblock(const uint8_t *const *rows, int b, int g, const uint16_t *xr, bool tok,
                         f4 *acc) {
    const uint16_t *xb = xr + b * 256 + 8 * g;
    h8 A[8];
    f4 X[8];
    const h8 ones = as_h8(u4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u});
#pragma unroll
    for (int s = 0; s < 8; s++) {
      u4 a = tok ? ld16<16>((const uint8_t *)(xb + 32 * s)) : u4{0, 0, 0, 0};
      A[s] = as_h8(perm0213(a));
      X[s] = mfma32(A[s], ones, f4{0, 0, 0, 0});
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
      const uint8_t *p = rows[t] + (size_t)b * TS;
      const u4 h = ld16<16>(p);
      u2 q[4];
#pragma unroll
      for (int jj = 0; jj < 4; jj++) q[jj] = ld8<8>(p + 16 + 32 * jj + 8 * g);
      const float d = h2f(h.x & 0xffff), dmin = h2f(h.x >> 16);
#pragma unroll
      for (int jj = 0; jj < 4; jj++) {
        u4 bl, bh;
        bl.x = unmagic(q[jj].x & 0x000F000Fu, 1024);
        bl.y = unmagic((q[jj].x >> 8) & 0x000F000Fu, 1024);
        bl.z = unmagic(q[jj].y & 0x000F000Fu, 1024);
        bl.w = unmagic((q[jj].y >> 8) & 0x000F000Fu, 1024);
        bh.x = unmagic((q[jj].x >> 4) & 0x000F000Fu, 1024);
        bh.y = unmagic((q[jj].x >> 12) & 0x000F000Fu, 1024);
        bh.z = unmagic((q[jj].y >> 4) & 0x000F000Fu, 1024);
        bh.w = unmagic((q[jj].y >> 12) & 0x000F000Fu, 1024);
        int sc0, m0, sc1, m1;
        q4k_scale_min(h.y, h.z, h.w, 2 * jj, sc0, m0);
        q4k_scale_min(h.y, h.z, h.w, 2 * jj + 1, sc1, m1);
        const f4 c0 = mfma32(A[2 * jj], as_h8(bl), f4{0, 0, 0, 0});
        const f4 c1 = mfma32(A[2 * jj + 1], as_h8(bh), f4{0, 0, 0, 0});
        acc[t] += (d * (float)sc0) * c0 - (dmin * (float)m0) * X[2 * jj] +
                  (d * (float)sc1) * c1 - (dmin * (float)m1) * X[2 * jj + 1];
      }
    }
  }
};

// ------------------------------------------------------------------------------------- Q6_K
// GGMLDequant.q6K (Core/GGMLDequant.swift:154-185): ql[128] at 0, qh[64] at 128, int8 sc[16]
// at 192, fp16 d at 208. Half n (128 weights), l in 0..31: weights 128n + l + 32qq take the low
// (qq 0,1) or high (qq 2,3) nibble of ql[64n + 32(qq&1) + l] and bits 2qq..2qq+1 of
// qh[32n + l]; w = d * sc[8n + l/16 + 2qq] * (q - 32).
struct FQ6_K {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q6_K;
  static constexpr int BS = 256, TS = 210, UPB = 4;  // unit: (n, l-half), 64 weights
  static constexpr int BATCH = 2;
  static constexpr bool XSUM = true, GRID = false;
  static constexpr int R = 8, Q = 4;  // slot 2qq + i: k0 + 32qq + 8i; sum qq: k0 + 32qq
  static DEV int k0_of(int u) { return (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16; }
  static DEV int slot_k(int u, int r) { return k0_of(u) + 32 * (r >> 1) + 8 * (r & 1); }
  static DEV int sum_k(int u, int q) { return k0_of(u) + 32 * q; }
  static constexpr int SUM_LEN = 16;
  struct Raw {
    u4 qa, qb, qh;
    u2 sc;
    uint32_t d;
  };
  static DEV Raw load(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)(u >> 2) * TS;
    const int n = (u >> 1) & 1, lh = u & 1;
    Raw r;
    r.qa = ld16<2>(p + 64 * n + 16 * lh);
    r.qb = ld16<2>(p + 64 * n + 32 + 16 * lh);
    r.qh = ld16<2>(p + 128 + 32 * n + 16 * lh);
    r.sc = ld8<2>(p + 192 + 8 * n);
    r.d = ld2(p + 208);
    return r;
  }
  // Each 6-bit code becomes 1024 + q; sum (q - 32) x = S - 1056 X over a 16-weight group.
  static DEV float dot(const Raw &r, int u, const GemvShared &s) {
    const int lh = u & 1;
    float S[4] = {0, 0, 0, 0};
    uint32_t xv[4][8];
#pragma unroll
    for (int qq = 0; qq < 4; qq++) unpack(s.slot<R>(u, 2 * qq), s.slot<R>(u, 2 * qq + 1), xv[qq]);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t a = r.qa[t], bq = r.qb[t], h = r.qh[t];
      const uint32_t v[4] = {(a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u),
                             (bq & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u),
                             ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u),
                             ((bq >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u)};
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        S[qq] = dot2(and_or(v[qq], 0x003F003Fu, s.mg), xv[qq][2 * t], S[qq]);
        S[qq] = dot2(and_or(v[qq] >> 8, 0x003F003Fu, s.mg), xv[qq][2 * t + 1], S[qq]);
      }
    }
    // sc[8n + lh + 2qq]: bytes lh, lh+2 of the low word, lh, lh+2 of the high word.
    const float d = h2f(r.d);
    const int sh = 8 * lh;
    const float s0 = (float)(int8_t)(r.sc.x >> sh), s1 = (float)(int8_t)(r.sc.x >> (sh + 16));
    const float s2 = (float)(int8_t)(r.sc.y >> sh), s3 = (float)(int8_t)(r.sc.y >> (sh + 16));
    return (d * s0) * (S[0] - 1056.0f * s.sum<Q>(u, 0)) + (d * s1) * (S[1] - 1056.0f * s.sum<Q>(u, 1)) +
           (d * s2) * (S[2] - 1056.0f * s.sum<Q>(u, 2)) + (d * s3) * (S[3] - 1056.0f * s.sum<Q>(u, 3));
  }

  // Verify: MFMA 16x16x16, one per 16-weight scale group (n, qq, lh); lane group g takes
  // l = 16lh + 4g .. +3.
  static constexpr int VSTEP = 16;
  template <int T>
  static DEV void vblock(const uint8_t *const *rows, int b, int g, const uint16_t *xr, bool tok,
                         f4 *acc) {
    const uint16_t *xb = xr + b * 256 + 4 * g;
    h4 A[16];  // index (n*2 + lh)*4 + qq
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
      for (int lh = 0; lh < 2; lh++)
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
          u2 a = tok ? ld8<8>((const uint8_t *)(xb + 128 * n + 32 * qq + 16 * lh)) : u2{0, 0};
          A[(n * 2 + lh) * 4 + qq] = as_h4(perm0213(a));
        }
#pragma unroll
    for (int t = 0; t < T; t++) {
      const uint8_t *p = rows[t] + (size_t)b * TS;
      const u4 sc = ld16<2>(p + 192);
      const float d = h2f(ld2(p + 208));
#pragma unroll
      for (int n = 0; n < 2; n++)
#pragma unroll
        for (int lh = 0; lh < 2; lh++) {
          const int l0 = 16 * lh + 4 * g;
          const uint32_t a = ld4<2>(p + 64 * n + l0), bq = ld4<2>(p + 64 * n + 32 + l0);
          const uint32_t h = ld4<2>(p + 128 + 32 * n + l0);
          const uint32_t v[4] = {(a & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u),
                                 (bq & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u),
                                 ((a >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u),
                                 ((bq >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u)};
#pragma unroll
          for (int qq = 0; qq < 4; qq++) {
            u2 B;
            B.x = unmagic(v[qq] & 0x003F003Fu, 1056);
            B.y = unmagic((v[qq] >> 8) & 0x003F003Fu, 1056);
            const int si = 8 * n + lh + 2 * qq;  // scale byte index
            const float scl = (float)(int8_t)(sc[si >> 2] >> (8 * (si & 3)));
            const f4 c = mfma16(A[(n * 2 + lh) * 4 + qq], as_h4(B), f4{0, 0, 0, 0});
            acc[t] += (d * scl) * c;
          }
        }
    }
  }
};

// ----------------------------------------------------------------------------------- IQ2_XS
// GGMLDequant.iq2XS (Core/GGMLDequant.swift:264-285): fp16 d at 0, qs u16[32] at 2 (9-bit grid
// index, 7-bit sign index), scales u8[8] at 66. Entry l of group ib (weights 32ib + 8l + j) is
// d*(0.5+nibble)*0.25 * grid[q&511][j] * sign(ksigns[q>>9], j), nibble = scales[ib] lo for
// l < 2, hi otherwise.
struct FIQ2_XS {
  static constexpr uint32_t TYPE = ISHZ_GGML_IQ2_XS;
  static constexpr int BS = 256, TS = 74, UPB = 4;  // unit: two groups, 16 B of qs, 64 weights
  static constexpr int BATCH = 2;
  static constexpr bool XSUM = false, GRID = true;
  static constexpr int R = 8, Q = 1;  // slot l: k0 + 8l
  static DEV int slot_k(int u, int r) { return (u >> 2) * 256 + (u & 3) * 64 + 8 * r; }
  static DEV int sum_k(int u, int q) { return 0; }
  static constexpr int SUM_LEN = 16;
  struct Raw {
    u4 q;
    uint32_t sc, d;
  };
  static DEV Raw load(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)(u >> 2) * TS;
    const int pp = u & 3;
    return {ld16<2>(p + 2 + 16 * pp), ld2(p + 66 + 2 * pp), ld2(p)};
  }
  static DEV float dot(const Raw &r, int u, const GemvShared &s) {
    const float d = h2f(r.d);
    float acc = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) {
      const uint32_t q = (r.q[l >> 1] >> (16 * (l & 1))) & 0xffffu;
      const u4 G = s.grid[q & 511], M = s.sgn[q >> 9];
      const u4 X = s.slot<R>(u, l);
      float e = dot2(G.x ^ M.x, X.x, 0.0f);
      e = dot2(G.y ^ M.y, X.y, e);
      e = dot2(G.z ^ M.z, X.z, e);
      e = dot2(G.w ^ M.w, X.w, e);
      const uint32_t nib = (r.sc >> (8 * (l >> 2) + 4 * ((l >> 1) & 1))) & 15;
      acc += (d * (0.5f + (float)nib) * 0.25f) * e;
    }
    return acc;
  }

  // Verify: MFMA 16x16x16 per 16-weight half-group (one scale nibble, entries 2h, 2h+1);
  // lane group g takes entry 2h + g/2, weights 4(g&1)..+3, from the natural-order LDS grid.
  static constexpr int VSTEP = 16;
  template <int T>
  static DEV void vblock_lds(const uint8_t *const *rows, int b, int g, const uint16_t *xr,
                             bool tok, f4 *acc, const u2 *grid_nat, const u2 *sgn_nat) {
    const uint16_t *xb = xr + b * 256 + 4 * g;
    h4 A[16];
#pragma unroll
    for (int st = 0; st < 16; st++)
      A[st] = as_h4(tok ? ld8<8>((const uint8_t *)(xb + 16 * st)) : u2{0, 0});
#pragma unroll
    for (int t = 0; t < T; t++) {
      const uint8_t *p = rows[t] + (size_t)b * TS;
      const float d = h2f(ld2(p));
      const u4 scales = ld16<2>(p + 66 - 8);  // bytes 58..73: scales are the top 8
#pragma unroll
      for (int ib = 0; ib < 8; ib++) {
        const u2 qs = ld8<2>(p + 2 + 8 * ib);  // entries 0..3 of the group
        const uint32_t sb = (ib < 4 ? scales.z : scales.w) >> (8 * (ib & 3));
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const uint32_t q = (h == 0 ? qs.x : qs.y) >> (16 * (g >> 1)) & 0xffffu;
          const u2 G = grid_nat[(q & 511) * 2 + (g & 1)];
          const u2 Sg = sgn_nat[(q >> 9) * 2 + (g & 1)];
          const u2 B = {G.x ^ Sg.x, G.y ^ Sg.y};
          const float nib = (float)((sb >> (4 * h)) & 15);
          const f4 c = mfma16(A[2 * ib + h], as_h4(B), f4{0, 0, 0, 0});
          acc[t] += (d * (0.5f + nib) * 0.25f) * c;
        }
      }
    }
  }
};

}  // namespace ishz
