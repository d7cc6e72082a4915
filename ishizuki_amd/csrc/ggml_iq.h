// The GGML formats beyond the four headline ones: Q2_K, IQ4_XS, IQ2_XXS, IQ2_S, IQ3_XXS, IQ3_S,
// IQ1_S, IQ1_M (GGMLDequant, Core/GGMLDequant.swift:125-428; block layouts per format below).
//
// All are 256-weight super-blocks, so one reader serves both kernels: a "quarter" is 64
// weights of one block (two 32-weight sub-blocks, or for Q2_K one 16-byte run of codes), the
// GEMV's unit and the MFMA verify's per-lane step share alike. A format supplies
//   VRaw vload(row, j, g)        quarter g of block j: its codes and the header fields it needs
//   void vdecode(r, B[8], mg, tabs, -)   eight 16-byte words of exact fp16 codes, 8 weights each
//   void vscale(r, g, s, sc, mn) sub-unit s of the quarter is worth sc * (codes . x - OFF * X) + mn * X
//   int xk(g, r)                 the first of the 8 weights word r covers (within the block)
//   tab_bytes(), build_tab(t)    its LDS tables (codebooks as fp16, sign masks)
// and the base turns that into the GEMV dot and the verify staging. Codebook entries become fp16
// once per workgroup in LDS, so decoding 8 weights is one ds_read_b128 (plus one for the signs).
// Sign masks are XORed onto the fp16 sign bits; every code is an exact small integer in fp16.
#pragma once
#include "ggml_formats.h"

// The codebooks (ishz_iq*_grid, ishz_kvalues_iq4nl) come from ggml_grids.inc, included first.

namespace ishz {

DEV uint32_t byte_of(uint32_t w, int i) { return __builtin_amdgcn_ubfe(w, 8 * i, 8); }

// ------------------------------------------------------------------------- table builders
// Grid entries of 8 bytes -> 8 fp16 (natural order), unsigned or as int8.
template <bool SIGNED>
DEV void tab_grid8(const uint64_t *g, int n, u4 *dst) {
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const uint64_t v = g[e];
    uint32_t h[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t b = (uint32_t)(v >> (8 * j)) & 0xff;
      h[j] = f2h(SIGNED ? (float)(int8_t)b : (float)b);
    }
    dst[e] = u4{h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
  }
}
// Grid entries of 4 bytes -> 4 fp16.
DEV void tab_grid4(const uint32_t *g, int n, u2 *dst) {
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const uint32_t v = g[e];
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; j++) h[j] = f2h((float)((v >> (8 * j)) & 0xff));
    dst[e] = u2{h[0] | h[1] << 16, h[2] | h[3] << 16};
  }
}

// ------------------------------------------------------------------------- shared base
template <class D>
struct GgmlQuarter : GgmlGemv<D> {
  static constexpr int BS = 256, UPB = 4, UNIT_BLOCKS = 1, GEMV_K_MULT = 256;
  static constexpr bool GRID = false, VGRID = false;
  // GEMV: 512-thread workgroups at four waves per SIMD, so each workgroup's codebook build and x
  // staging serve eight waves (measured 8-15 % faster at 17408x5120 on MI355X than 256 threads at
  // two waves per SIMD for every codebook format)
  static constexpr int WG = 512;
  static int occ(const typename GgmlGemv<D>::Args &) { return 4; }
  static constexpr int R = 8;
  static DEV int slot_k(int u, int r) { return (u >> 2) * 256 + D::xk(u & 3, r); }
  static DEV int sum_k(int u, int q) { return (u >> 2) * 256 + D::xk(u & 3, q * (8 / D::VNS)); }
  static DEV auto load_row(const uint8_t *row, int u) { return D::vload(row, u >> 2, u & 3); }
  struct LaneC {
    int g;
  };
  // A lane's units are sub, sub + LPR, ... with LPR a multiple of 16: always quarter sub % 4.
  static DEV LaneC lane(int sub) { return {sub & 3}; }
  template <class Raw>
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &c) {
    constexpr int NS = D::VNS, MPS = 8 / NS;
    u4 B[8];
    D::vdecode(r, B, s.mg, s.grid, s.grid);
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NS; q++) {
      float S = 0.0f;
#pragma unroll
      for (int b = 0; b < MPS; b++) {
        const u4 X = s.slot(q * MPS + b), W = B[q * MPS + b];
        S = dot2(W.x, X.x, S);
        S = dot2(W.y, X.y, S);
        S = dot2(W.z, X.z, S);
        S = dot2(W.w, X.w, S);
      }
      float sc, mn;
      D::vscale(r, c.g, q, sc, mn);
      if constexpr (D::XSUM) {
        const float X = s.sum(q);
        acc += sc * (S - D::OFF * X) + mn * X;
      } else {
        acc += sc * S;
      }
    }
    return acc;
  }
  static constexpr size_t tab_bytes() { return D::TAB_BYTES; }
  static DEV void gemv_tables(u4 *t) { D::build_tab(t); }
  static DEV void vtables(u4 *t) { D::build_tab(t); }
  static DEV void vstage(const uint16_t *x, int j, int g, int s, u4 *A, float &off1, float &X) {
    constexpr int MPS = 8 / D::VNS;
    X = 0.0f;
#pragma unroll
    for (int b = 0; b < MPS; b++) {
      const uint16_t *p = x + 256 * j + D::xk(g, s * MPS + b);
      A[b] = D::XPERM ? vx8p(p, X) : vx8s(p, X);
    }
    off1 = D::OFF * X;
  }
  static constexpr float voff() { return D::OFF; }  // off1 of vstage, per unit of X
  // Natural order, with the sum of the 8 values.
  static DEV u4 vx8s(const uint16_t *p, float &X) {
    const u4 v = *(const u4 *)p;
#pragma unroll
    for (int e = 0; e < 4; e++) X = dot2(v[e], 0x3C003C00u, X);
    return v;
  }
};

#define ISHZ_QUARTER_COMMON(NAME, T, SIZE)                  \
  static constexpr uint32_t TYPE = T;                       \
  static constexpr int TS = SIZE, VSTEP_BYTES = SIZE;       \
  typedef VRaw Raw;                                         \
  using GgmlQuarter<NAME>::load_row;                        \
  using GgmlQuarter<NAME>::dot;

// ------------------------------------------------------------------------- Q2_K
// GGMLDequant.q2K (:125-152): scales[16] at 0 (low nibble scale, high nibble min, one per 16
// weights), qs[64] at 16, d at 80, dmin at 82. Half n (128 weights) uses qs[32n .. 32n + 31];
// byte 16 lane + l holds weights 128n + 32s + 16 lane + l in bits 2s..2s+1 (s = 0..3), scale byte
// 8n + 2s + lane. Quarter g = (n, lane) = (g / 2, g % 2): 16 bytes of codes, sub-unit s = shift.
// Codes are masked in place (1024 + 4^s q, exact) against pair-permuted x.
struct FQ2_K : GgmlQuarter<FQ2_K> {
  struct VRaw {
    u4 q;
    u2 sc;
    uint32_t dd;
  };
  ISHZ_QUARTER_COMMON(FQ2_K, ISHZ_GGML_Q2_K, 84)
  static constexpr int VNS = 4, Q = 4, SUM_LEN = 16;
  static constexpr bool XSUM = true, XPERM = true;
  static constexpr float OFF = 1024.0f;
  static constexpr size_t TAB_BYTES = 0;
  static DEV void build_tab(u4 *) {}
  static DEV int xk(int g, int r) { return (g >> 1) * 128 + (r >> 1) * 32 + (g & 1) * 16 + 8 * (r & 1); }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<4>(p + 16 + 16 * g), ld8<4>(p + 8 * (g >> 1)), ld4<4>(p + 80)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t mg, const u4 *, const u4 *) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const uint32_t m = 0x00030003u << (2 * s);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint32_t a = r.q[2 * h], b = r.q[2 * h + 1];
        B[2 * s + h] = u4{and_or(a, m, mg), and_or(a >> 8, m, mg), and_or(b, m, mg), and_or(b >> 8, m, mg)};
      }
    }
  }
  static DEV void vscale(const VRaw &r, int g, int s, float &sc, float &mn) {
    const int i = (g & 1) + 2 * s;  // byte of the 8 loaded
    const uint32_t b = byte_of(i < 4 ? r.sc.x : r.sc.y, i & 3);
    sc = h2f(r.dd & 0xffff) * (float)(b & 15) * (1.0f / (float)(1 << (2 * s)));
    mn = -(h2f(r.dd >> 16) * (float)(b >> 4));
  }
};

// ------------------------------------------------------------------------- IQ4_XS
// GGMLDequant.iq4XS (:222-241): d at 0, scales_h (u16) at 2, scales_l[4] at 4, qs[128] at 8;
// sub-block ib: scale (nibble ib of scales_l | 2 bits ib of scales_h << 4) - 32, 16 bytes of qs:
// low nibble of byte j is weight j, high nibble weight j + 16, values kvalues_iq4nl[nibble].
// LDS table: for a byte b = lo | hi << 4 the fp16 pair (kvalues[lo], kvalues[hi]); the index
// for weights (j, j + 1) is built from the nibbles of two neighbouring bytes.
struct FIQ4_XS : GgmlQuarter<FIQ4_XS> {
  struct VRaw {
    u4 q0, q1;
    uint32_t hd, sl;
  };
  ISHZ_QUARTER_COMMON(FIQ4_XS, ISHZ_GGML_IQ4_XS, 136)
  static constexpr int VNS = 2, Q = 1, SUM_LEN = 32;
  static constexpr bool XSUM = false, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr bool VPLAIN = true;  // no offset, no min: value = sc * C
  static constexpr size_t TAB_BYTES = 256 * 4;
  static DEV void build_tab(u4 *t) {
    uint32_t *p = (uint32_t *)t;
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
      p[i] = (uint32_t)f2h((float)ishz_kvalues_iq4nl[i & 15]) | (uint32_t)f2h((float)ishz_kvalues_iq4nl[i >> 4]) << 16;
  }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<8>(p + 8 + 32 * g), ld16<8>(p + 24 + 32 * g), ld4<4>(p), ld4<4>(p + 4)};
  }
  // Two pair-table words from one dword of codes (nibbles already isolated per byte).
  static DEV u2 pairs(uint32_t t, const uint32_t *tab) {
    const uint32_t u = t | (t >> 4);
    return u2{tab[u & 0xff], tab[(u >> 16) & 0xff]};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *tabs, const u4 *) {
    const uint32_t *tab = (const uint32_t *)tabs;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const u4 q = h ? r.q1 : r.q0;
#pragma unroll
      for (int hi = 0; hi < 2; hi++)
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const uint32_t a = q[2 * half], b = q[2 * half + 1];
          const uint32_t ta = (hi ? a >> 4 : a) & 0x0F0F0F0Fu, tb = (hi ? b >> 4 : b) & 0x0F0F0F0Fu;
          const u2 pa = pairs(ta, tab), pb = pairs(tb, tab);
          B[4 * h + 2 * hi + half] = u4{pa.x, pa.y, pb.x, pb.y};
        }
    }
  }
  static DEV void vscale(const VRaw &r, int g, int s, float &sc, float &mn) {
    const int ib = 2 * g + s;
    const uint32_t lo = (r.sl >> (4 * ib)) & 15, hi = ((r.hd >> (16 + 2 * ib)) & 3) << 4;
    sc = h2f(r.hd & 0xffff) * (float)((int)(lo | hi) - 32);
    mn = 0.0f;
  }
};

// ------------------------------------------------------------------------- IQ2_XXS
// GGMLDequant.iq2XXS (:243-262): d at 0, then per sub-block 8 bytes: four grid indices (a1) and
// a word a2 holding four 7-bit ksigns indices and the 4-bit scale (a2 >> 28):
// w = d (0.5 + scale) / 4 * grid[idx][j] * sign.
struct FIQ2_XXS : GgmlQuarter<FIQ2_XXS> {
  struct VRaw {
    u4 q;
    uint32_t d;
  };
  ISHZ_QUARTER_COMMON(FIQ2_XXS, ISHZ_GGML_IQ2_XXS, 66)
  static constexpr int VNS = 2, Q = 1, SUM_LEN = 32;
  static constexpr bool XSUM = false, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr bool VPLAIN = true;  // no offset, no min: value = sc * C
  static constexpr size_t TAB_BYTES = 256 * 16;
  static DEV void build_tab(u4 *t) { tab_grid8<false>(ishz_iq2xxs_grid, 256, t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<2>(p + 2 + 16 * g), ld2(p)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int l = 0; l < 4; l++)
        B[4 * h + l] = t[byte_of(r.q[2 * h], l)] ^ sign_words(ksigns_pattern(__builtin_amdgcn_ubfe(r.q[2 * h + 1], 7 * l, 7)));
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    sc = h2f(r.d) * (0.5f + (float)(r.q[2 * s + 1] >> 28)) * 0.25f;
    mn = 0.0f;
  }
};

// ------------------------------------------------------------------------- IQ2_S
// GGMLDequant.iq2S (:287-309): d at 0, qs[32] at 2 (grid index low bytes, 4 per sub-block),
// signs[32] at 34 (one byte per 8 weights), qh[8] at 66 (2 high bits per index), scales[8] at 74
// (a nibble per 16 weights): w = d (0.5 + nibble) / 4 * grid[idx][j] * sign.
struct FIQ2_S : GgmlQuarter<FIQ2_S> {
  struct VRaw {
    u2 qs, sg;
    uint32_t qh, sc, d;
  };
  ISHZ_QUARTER_COMMON(FIQ2_S, ISHZ_GGML_IQ2_S, 82)
  static constexpr int VNS = 4, Q = 1, SUM_LEN = 16;
  static constexpr bool XSUM = false, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr bool VPLAIN = true;  // no offset, no min: value = sc * C
  static constexpr size_t TAB_BYTES = 1024 * 16;
  static DEV void build_tab(u4 *t) { tab_grid8<false>(ishz_iq2s_grid, 1024, t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    // qh, sc: the dwords ending with the quarter's two bytes (bits 16..31); d: bits 0..15 of the
    // block's first dword (dword loads: see FIQ2_XS::Raw)
    return {ld8<2>(p + 2 + 8 * g), ld8<2>(p + 34 + 8 * g), ld4<2>(p + 64 + 2 * g), ld4<2>(p + 72 + 2 * g), ld4<2>(p)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t qh = byte_of(r.qh, 2 + h);
#pragma unroll
      for (int l = 0; l < 4; l++) {
        const uint32_t idx = byte_of(r.qs[h], l) | ((qh << (8 - 2 * l)) & 0x300u);
        B[4 * h + l] = t[idx] ^ sign_words(byte_of(r.sg[h], l));
      }
    }
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    const uint32_t nib = (r.sc >> (16 + 4 * s)) & 15;  // s = 2 h + (l >= 2): byte h, nibble s & 1
    sc = h2f(r.d & 0xffffu) * (0.5f + (float)nib) * 0.25f;
    mn = 0.0f;
  }
};

// ------------------------------------------------------------------------- IQ3_XXS
// GGMLDequant.iq3XXS (:311-330): d at 0, qs[64] at 2 (two 4-value grid indices per 8 weights),
// then per sub-block a word aux at 66 + 4 ib: four 7-bit ksigns indices and the scale (aux >> 28):
// w = d (0.5 + scale) / 2 * grid[idx][j] * sign.
struct FIQ3_XXS : GgmlQuarter<FIQ3_XXS> {
  struct VRaw {
    u4 q;
    u2 aux;
    uint32_t d;
  };
  ISHZ_QUARTER_COMMON(FIQ3_XXS, ISHZ_GGML_IQ3_XXS, 98)
  static constexpr int VNS = 2, Q = 1, SUM_LEN = 32;
  static constexpr bool XSUM = false, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr bool VPLAIN = true;  // no offset, no min: value = sc * C
  static constexpr size_t TAB_BYTES = 256 * 8;
  static DEV void build_tab(u4 *t) { tab_grid4(ishz_iq3xxs_grid, 256, (u2 *)t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<2>(p + 2 + 16 * g), ld8<2>(p + 66 + 8 * g), ld2(p)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
    const u2 *grid = (const u2 *)t;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int l = 0; l < 4; l++) {
        const uint32_t w = r.q[2 * h + (l >> 1)];
        const u2 g1 = grid[byte_of(w, 2 * (l & 1))], g2 = grid[byte_of(w, 2 * (l & 1) + 1)];
        B[4 * h + l] = u4{g1.x, g1.y, g2.x, g2.y} ^ sign_words(ksigns_pattern(__builtin_amdgcn_ubfe(r.aux[h], 7 * l, 7)));
      }
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    sc = h2f(r.d) * (0.5f + (float)(r.aux[s] >> 28)) * 0.5f;
    mn = 0.0f;
  }
};

// ------------------------------------------------------------------------- IQ3_S
// GGMLDequant.iq3S (:332-364): d at 0, qs[64] at 2 (grid index low bytes, two per 8 weights),
// qh[8] at 66 (the indices' 9th bits, one byte per sub-block), signs[32] at 74 (a byte per 8
// weights), scales[4] at 106 (a nibble per sub-block): w = d (1 + 2 nibble) * grid[idx][j] * sign.
struct FIQ3_S : GgmlQuarter<FIQ3_S> {
  struct VRaw {
    u4 q;
    u2 sg;
    uint32_t qh, sc, d;
  };
  ISHZ_QUARTER_COMMON(FIQ3_S, ISHZ_GGML_IQ3_S, 110)
  static constexpr int VNS = 2, Q = 1, SUM_LEN = 32;
  static constexpr bool XSUM = false, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr bool VPLAIN = true;  // no offset, no min: value = sc * C
  static constexpr size_t TAB_BYTES = 512 * 8;
  static DEV void build_tab(u4 *t) { tab_grid4(ishz_iq3s_grid, 512, (u2 *)t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    // qh: the dword ending with the quarter's two bytes (bits 16..31); sc: the dword ending with its
    // scale byte (bits 24..31); d: bits 0..15 of the block's first dword (see FIQ2_XS::Raw)
    return {ld16<2>(p + 2 + 16 * g), ld8<2>(p + 74 + 8 * g), ld4<2>(p + 64 + 2 * g), ld4<1>(p + 103 + g), ld4<2>(p)};
  }
  // Index 2l of sub-block ib takes its 9th bit from bit 2l of qh[ib], index 2l + 1 from bit 2l + 1.
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
    const u2 *grid = (const u2 *)t;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t qh = byte_of(r.qh, 2 + h);
#pragma unroll
      for (int l = 0; l < 4; l++) {
        const uint32_t w = r.q[2 * h + (l >> 1)];
        const uint32_t i1 = byte_of(w, 2 * (l & 1)) | ((qh << (8 - 2 * l)) & 256u);
        const uint32_t i2 = byte_of(w, 2 * (l & 1) + 1) | ((qh << (7 - 2 * l)) & 256u);
        const u2 g1 = grid[i1], g2 = grid[i2];
        B[4 * h + l] = u4{g1.x, g1.y, g2.x, g2.y} ^ sign_words(byte_of(r.sg[h], l));
      }
    }
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    sc = h2f(r.d & 0xffffu) * (float)(1 + 2 * (int)((r.sc >> (24 + 4 * s)) & 15));
    mn = 0.0f;
  }
};

// ------------------------------------------------------------------------- IQ1_S
// GGMLDequant.iq1S (:366-385): d at 0, qs[32] at 2 (index low bytes), qh[8] (u16) at 34: bits
// 3l..3l+2 the index's high bits, bits 12..14 the scale, bit 15 the delta's sign:
// w = d (2 scale + 1) (grid[idx][j] + delta), grid values -1, 0, 1, delta = +-1/8. The delta
// term comes back through the per-sub-block sum of x.
struct FIQ1_S : GgmlQuarter<FIQ1_S> {
  struct VRaw {
    u2 qs;
    uint32_t qh, d;
  };
  ISHZ_QUARTER_COMMON(FIQ1_S, ISHZ_GGML_IQ1_S, 50)
  static constexpr int VNS = 2, Q = 2, SUM_LEN = 32;
  static constexpr bool XSUM = true, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr size_t TAB_BYTES = 2048 * 16;
  static DEV void build_tab(u4 *t) { tab_grid8<true>(ishz_iq1s_grid, 2048, t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld8<2>(p + 2 + 8 * g), ld4<2>(p + 34 + 4 * g), ld2(p)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int l = 0; l < 4; l++)
        B[4 * h + l] = t[byte_of(r.qs[h], l) | __builtin_amdgcn_ubfe(r.qh, 16 * h + 3 * l, 3) << 8];
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    const uint32_t qh = r.qh >> (16 * s);
    sc = h2f(r.d) * (float)(2 * (int)((qh >> 12) & 7) + 1);
    mn = sc * ((qh & 0x8000u) ? -0.125f : 0.125f);
  }
};

// ------------------------------------------------------------------------- IQ1_M
// GGMLDequant.iq1M (:387-428): qs[32] at 0, qh[16] at 32 (per index pair: high bits 0..2 /
// 4..6 and the delta signs in bits 3 / 7), scales[8] at 48 as four u16: 3-bit scales for each
// 16 weights, and the fp16 d spread over their top nibbles. Sub-unit = 8 weights (own delta).
struct FIQ1_M : GgmlQuarter<FIQ1_M> {
  struct VRaw {
    u2 qs;
    uint32_t qh;
    u2 sc;
  };
  ISHZ_QUARTER_COMMON(FIQ1_M, ISHZ_GGML_IQ1_M, 56)
  static constexpr int VNS = 8, Q = 8, SUM_LEN = 8;
  static constexpr bool XSUM = true, XPERM = false;
  static constexpr float OFF = 0.0f;
  static constexpr size_t TAB_BYTES = 2048 * 16;
  static DEV void build_tab(u4 *t) { tab_grid8<true>(ishz_iq1s_grid, 2048, t); }
  static DEV int xk(int g, int r) { return 64 * g + 8 * r; }
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld8<2>(p + 8 * g), ld4<2>(p + 32 + 4 * g), ld8<2>(p + 48)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *t, const u4 *) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int l = 0; l < 4; l++) {
        const uint32_t qb = byte_of(r.qh, 2 * h + (l >> 1));
        const uint32_t hi = (l & 1) ? (qb >> 4) & 7 : qb & 7;
        B[4 * h + l] = t[byte_of(r.qs[h], l) | hi << 8];
      }
  }
  static DEV void vscale(const VRaw &r, int g, int s, float &sc, float &mn) {
    const uint32_t s0 = r.sc.x & 0xffff, s1 = r.sc.x >> 16, s2 = r.sc.y & 0xffff, s3 = r.sc.y >> 16;
    const uint32_t dbits = (s0 >> 12) | ((s1 >> 8) & 0x00f0) | ((s2 >> 4) & 0x0f00) | (s3 & 0xf000);
    const uint32_t w = (g & 2 ? r.sc.y : r.sc.x) >> (16 * (g & 1));  // scales word of sub-blocks 2g, 2g + 1
    const int h = s >> 2, l = s & 3;
    const uint32_t sh = 6 * h + (l >= 2 ? 3 : 0);
    sc = h2f(dbits) * (float)(2 * (int)((w >> sh) & 7) + 1);
    const uint32_t qb = byte_of(r.qh, 2 * h + (l >> 1));
    mn = sc * ((qb & ((l & 1) ? 0x80u : 0x08u)) ? -0.125f : 0.125f);
  }
};

#undef ISHZ_QUARTER_COMMON

}  // namespace ishz
