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
#include <algorithm>

#include "common.h"
#include "gemv.h"

namespace ishz {

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

// What the GEMV skeleton needs from a GGML format: row pointers, unit count and the x staging
// (x slots in consumption order, per-group sums, i-quant tables).
DEV void build_iq2xs_tables_perm(u4 *grid, u4 *sgn);
DEV void build_iq2xs_tables_nat(u4 *grid, u4 *sgn);

template <class D>
struct GgmlGemv {
  struct Args {
    const uint8_t *w;
    size_t rb;  // bytes per row
    int K, N;
  };
  static constexpr int GRID_ENTRIES = 512;
  // GEMV ring depth (batches per lane in flight = RING - 1): measured on MI355X at 17408x5120, two
  // beats three to five for every GGUF format by 6-11 % (a deeper ring unrolls more copies of the
  // decode loop body and issues more of a short wave's work before its first consume)
  static constexpr int RING = 2;
  // Streaming-verify ring depth: two, measured best for every GGUF format at 17408x5120, M = 8
  // (4-10 % faster than three to six)
  static constexpr int VDEPTH = 2;
  // Resident waves per SIMD the grid is sized for: two measured best on MI355X at 17408x5120
  // (fewer, longer waves amortise the x staging every workgroup repeats).
  static int occ(const Args &) { return 2; }
  static __host__ __device__ int units(int K) { return K / D::BS * D::UPB / D::UNIT_BLOCKS; }
  static size_t extra_lds_bytes(const Args &) { return D::gemv_tab_bytes(); }
  // LDS tables (codebooks, sign masks) the decoders index: bytes, and the builder every
  // workgroup runs once (GEMV: pair-permuted like x; verify: natural order). IQ2_XS's here;
  // formats with other tables replace all three.
  static constexpr size_t tab_bytes() { return D::GRID ? (512 + 128) * 16 : 0; }
  // the GEMV reads IQ2_XS's codebook only (its sign masks are computed in registers)
  static constexpr size_t gemv_tab_bytes() { return D::GRID ? 512 * 16 : D::tab_bytes(); }
  static DEV void gemv_tables(u4 *t) {
    if constexpr (D::GRID) build_iq2xs_tables_perm(t, nullptr);
  }
  static DEV void vtables(u4 *t) {
    if constexpr (D::VGRID) build_iq2xs_tables_nat(t, t + 512);
  }
  static constexpr bool XPERM = true;  // x slots staged pair-permuted (perm0213) or natural
  static DEV u4 xperm(u4 v) { return D::XPERM ? perm0213(v) : v; }  // a format may replace it
  static DEV auto load(const Args &a, int row, int u) { return D::load_row(a.w + (size_t)row * a.rb, u); }
  // Loads for U slots (US sums) per thread are issued together before any is stored, so
  // staging costs a memory latency per U items rather than one each; the first round's loads
  // are issued by stage_load, ahead of the weight batches.
  static constexpr int U = 4, US = 2, SLMAX = 4;  // SUM_LEN <= 32
  struct XPre {
    u4 v[U];
    u4 sv[US][SLMAX];
  };
  static DEV void load_slots(const uint16_t *x, int units, int i0, u4 *v) {
    const int ns = (units + 15) / 16 * 16 * D::R;
#pragma unroll
    for (int j = 0; j < U; j++) {
      const int i = min(i0 + j * (int)blockDim.x, ns - 1);
      const int u = min((i / (16 * D::R)) * 16 + (i & 15), units - 1), r = (i >> 4) % D::R;
      v[j] = *(const u4 *)(x + D::slot_k(u, r));
    }
  }
  static DEV void load_sums(const uint16_t *x, int units, int i0, u4 (*v)[SLMAX]) {
    constexpr int SL = D::SUM_LEN / 8;
    if constexpr (D::XSUM) {
      const int nq = (units + 15) / 16 * 16 * D::Q;
#pragma unroll
      for (int j = 0; j < US; j++) {
        const int i = min(i0 + j * (int)blockDim.x, nq - 1);
        const int u = min((i / (16 * D::Q)) * 16 + (i & 15), units - 1), q = (i >> 4) % D::Q;
        const u4 *p = (const u4 *)(x + D::sum_k(u, q));
#pragma unroll
        for (int h = 0; h < SL; h++) v[j][h] = p[h];
      }
    }
  }
  static DEV XPre stage_load(const Args &, const uint16_t *x, int units) {
    XPre p;
    load_slots(x, units, threadIdx.x, p.v);
    load_sums(x, units, threadIdx.x, p.sv);
    return p;
  }
  static DEV void store_slots(u4 *xs, int units, int i0, const u4 *v) {
    const int ns = (units + 15) / 16 * 16 * D::R;
#pragma unroll
    for (int j = 0; j < U; j++) {
      const int i = i0 + j * (int)blockDim.x;
      if (i < ns && (i / (16 * D::R)) * 16 + (i & 15) < units) xs[i] = D::xperm(v[j]);
    }
  }
  static DEV void store_sums(float *xsum, int units, int i0, const u4 (*v)[SLMAX]) {
    constexpr int SL = D::SUM_LEN / 8;
    const int nq = (units + 15) / 16 * 16 * D::Q;
#pragma unroll
    for (int j = 0; j < US; j++) {
      const int i = i0 + j * (int)blockDim.x;
      if (i < nq && (i / (16 * D::Q)) * 16 + (i & 15) < units) {
        float sm = 0.0f;
#pragma unroll
        for (int h = 0; h < SL; h++)
#pragma unroll
          for (int e = 0; e < 4; e++) sm = dot2(v[j][h][e], 0x3C003C00u, sm);  // + both halves
        xsum[i] = sm;
      }
    }
  }
  // Every slot and sum of nimg x images (image i at x + i * xstride, staged at xs + i ns and
  // xsum + i nq): one index space over all images, so each round's slot and sum loads for every
  // image go out together and the staging costs a memory latency per round, not per image.
  // Threads tid0 .. tid0 + nthr - 1 take part (all of them by default).
  static DEV void stage_images(const uint16_t *x, size_t xstride, int nimg, u4 *xs, float *xsum, int units,
                               int tid0 = 0, int nthr = 0) {
    const int ug = (units + 15) / 16, bd = nthr ? nthr : (int)blockDim.x, tid = (int)threadIdx.x - tid0;
    const int ns = ug * 16 * D::R, nq = D::XSUM ? ug * 16 * D::Q : 0;
    const int rs = (nimg * ns + U * bd - 1) / (U * bd), rq = (nimg * nq + US * bd - 1) / (US * bd);
    for (int round = 0; round < max(rs, rq); round++) {
      u4 v[U];
      u4 sv[US][SLMAX];
      const int i0 = round * U * bd + tid, q0 = round * US * bd + tid;
#pragma unroll
      for (int j = 0; j < U; j++) {
        const int i = min(i0 + j * bd, nimg * ns - 1), im = i / ns, ii = i % ns;
        const int u = min((ii / (16 * D::R)) * 16 + (ii & 15), units - 1), r = (ii >> 4) % D::R;
        v[j] = *(const u4 *)(x + im * xstride + D::slot_k(u, r));
      }
      if constexpr (D::XSUM) {
        constexpr int SL = D::SUM_LEN / 8;
#pragma unroll
        for (int j = 0; j < US; j++) {
          const int i = min(q0 + j * bd, nimg * nq - 1), im = i / nq, ii = i % nq;
          const int u = min((ii / (16 * D::Q)) * 16 + (ii & 15), units - 1), q = (ii >> 4) % D::Q;
          const u4 *p = (const u4 *)(x + im * xstride + D::sum_k(u, q));
#pragma unroll
          for (int h = 0; h < SL; h++) sv[j][h] = p[h];
        }
      }
#pragma unroll
      for (int j = 0; j < U; j++) {
        const int i = i0 + j * bd, ii = i % ns;
        if (i < nimg * ns && (ii / (16 * D::R)) * 16 + (ii & 15) < units) xs[i] = D::xperm(v[j]);
      }
      if constexpr (D::XSUM) {
        constexpr int SL = D::SUM_LEN / 8;
#pragma unroll
        for (int j = 0; j < US; j++) {
          const int i = q0 + j * bd, ii = i % nq;
          if (i < nimg * nq && (ii / (16 * D::Q)) * 16 + (ii & 15) < units) {
            float sm = 0.0f;
#pragma unroll
            for (int h = 0; h < SL; h++)
#pragma unroll
              for (int e = 0; e < 4; e++) sm = dot2(sv[j][h][e], 0x3C003C00u, sm);  // + both halves
            xsum[i] = sm;
          }
        }
      }
    }
  }
  static DEV void stage(const Args &, const uint16_t *x, u4 *xs, float *xsum, u4 *extra, int units,
                        const XPre &pre) {
    stage_body(x, xs, xsum, extra, units, pre);
  }
  // The staging itself (formats with their own Args call it from their stage).
  static DEV void stage_body(const uint16_t *x, u4 *xs, float *xsum, u4 *extra, int units, const XPre &pre) {
    const int ug = (units + 15) / 16, bd = blockDim.x;
    const int ns = ug * 16 * D::R;
    store_slots(xs, units, threadIdx.x, pre.v);  // first round: loads issued by stage_load
    for (int i0 = threadIdx.x + U * bd; i0 < ns; i0 += U * bd) {
      u4 v[U];
      load_slots(x, units, i0, v);
      store_slots(xs, units, i0, v);
    }
    if constexpr (D::XSUM) {
      const int nq = ug * 16 * D::Q;
      store_sums(xsum, units, threadIdx.x, pre.sv);
      for (int i0 = threadIdx.x + US * bd; i0 < nq; i0 += US * bd) {
        u4 v[US][SLMAX];
        load_sums(x, units, i0, v);
        store_sums(xsum, units, i0, v);
      }
    }
    D::gemv_tables(extra);
    __syncthreads();
  }
};

// Verify staging: perm0213 of 8 consecutive x (the pair order of nibble codes), natural order.
DEV u4 vx8p(const uint16_t *x, float &X) {
  const u4 v = *(const u4 *)x;
#pragma unroll
  for (int e = 0; e < 4; e++) X = dot2(v[e], 0x3C003C00u, X);
  return perm0213(v);
}
DEV u4 vx8n(const uint16_t *x) { return *(const u4 *)x; }

// ------------------------------------------------------------------------------------- Q4_0
// ggml block_q4_0: fp16 d at 0, qs[16] at 2; element j = (lo(qs[j]) - 8) d, j + 16 = hi.
struct FQ4_0 : GgmlGemv<FQ4_0> {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q4_0;
  static constexpr int BS = 32, TS = 18;
  // GEMV unit: two blocks (36 bytes, dword aligned when rows hold an even number of blocks),
  // 64 weights; so the GEMV needs K % 64 == 0 (the verify kernel takes any K % 32 == 0).
  static constexpr int UPB = 1, UNIT_BLOCKS = 2, GEMV_K_MULT = 64;
  static constexpr bool XSUM = true, GRID = false;
  static constexpr int R = 8, Q = 4;  // slots k0 + 8r; sums of 16 at k0 + 16q
  static DEV int slot_k(int u, int r) { return 64 * u + 8 * r; }
  static DEV int sum_k(int u, int q) { return 64 * u + 16 * q; }
  static constexpr int SUM_LEN = 16;
  struct Raw {
    u4 a, b;
    uint32_t c;
  };
  static DEV Raw load_row(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)u * 2 * TS;
    return {ld16<4>(p), ld16<4>(p + 16), ld4<4>(p + 32)};
  }
  struct LaneC {};
  static DEV LaneC lane(int sub) { return {}; }
  // Block A: d = bytes 0-1, qs = bytes 2..17 (realigned by two bytes); block B: d = bytes
  // 18-19, qs = bytes 20..35 (dword aligned). Low nibbles become 1024 + q, high ones 1024 + 16q;
  // the offsets come back out through the per-16 sums of x.
  static DEV float half_dot(const uint32_t *qs, const UnitX &s, int r0, int q0) {
    uint32_t xl[8], xh[8];
    unpack(s.slot(r0), s.slot(r0 + 1), xl);
    unpack(s.slot(r0 + 2), s.slot(r0 + 3), xh);
    float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint32_t q = qs[t], q8 = q >> 8;
      a0 = dot2(and_or(q, 0x000F000Fu, s.mg), xl[2 * t], a0);
      a1 = dot2(and_or(q8, 0x000F000Fu, s.mg), xl[2 * t + 1], a1);
      b0 = dot2(and_or(q, 0x00F000F0u, s.mg), xh[2 * t], b0);
      b1 = dot2(and_or(q8, 0x00F000F0u, s.mg), xh[2 * t + 1], b1);
    }
    return ((a0 + a1) - 1032.0f * s.sum(q0)) + (0.0625f * (b0 + b1) - 72.0f * s.sum(q0 + 1));
  }
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &) {
    const uint32_t qa[4] = {__builtin_amdgcn_alignbyte(r.a.y, r.a.x, 2), __builtin_amdgcn_alignbyte(r.a.z, r.a.y, 2),
                            __builtin_amdgcn_alignbyte(r.a.w, r.a.z, 2), __builtin_amdgcn_alignbyte(r.b.x, r.a.w, 2)};
    const uint32_t qb[4] = {r.b.y, r.b.z, r.b.w, r.c};
    return h2f(r.a.x & 0xffff) * half_dot(qa, s, 0, 0) + h2f(r.b.x >> 16) * half_dot(qb, s, 4, 2);
  }

  // Streaming verify: a lane's quarter of a 256-weight step is its GEMV unit (blocks 8j + 2g,
  // 8j + 2g + 1); sub-units (block, low / high nibbles), two MFMAs each. High nibbles decode to
  // 1024 + 16q, so their scale carries the 1/16.
  static constexpr int VNS = 4, VSTEP_BYTES = 8 * TS;
  static constexpr bool VGRID = false;
  typedef Raw VRaw;
  static DEV VRaw vload(const uint8_t *row, int j, int g) { return load_row(row + (size_t)j * VSTEP_BYTES, g); }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t mg, const u4 *, const u4 *) {
    const uint32_t q[8] = {__builtin_amdgcn_alignbyte(r.a.y, r.a.x, 2), __builtin_amdgcn_alignbyte(r.a.z, r.a.y, 2),
                           __builtin_amdgcn_alignbyte(r.a.w, r.a.z, 2), __builtin_amdgcn_alignbyte(r.b.x, r.a.w, 2),
                           r.b.y, r.b.z, r.b.w, r.c};
#pragma unroll
    for (int blk = 0; blk < 2; blk++)
#pragma unroll
      for (int hi = 0; hi < 2; hi++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const uint32_t m = hi ? 0x00F000F0u : 0x000F000Fu;
          const uint32_t q0 = q[4 * blk + 2 * b], q1 = q[4 * blk + 2 * b + 1];
          B[(2 * blk + hi) * 2 + b] = u4{and_or(q0, m, mg), and_or(q0 >> 8, m, mg), and_or(q1, m, mg), and_or(q1 >> 8, m, mg)};
        }
  }
  static DEV void vstage(const uint16_t *x, int j, int g, int s, u4 *A, float &off1, float &X) {
    const uint16_t *p = x + 256 * j + 64 * g + 32 * (s >> 1) + 16 * (s & 1);
    X = 0.0f;
    A[0] = vx8p(p, X);
    A[1] = vx8p(p + 8, X);
    off1 = 1024.0f * X;
  }
  static constexpr float voff() { return 1024.0f; }  // off1 of vstage, per unit of X
  static constexpr float vkappa(int s) { return (s & 1) ? -128.0f : -8.0f; }  // mn = vkappa sc
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    const float d = h2f(s >> 1 ? r.b.x >> 16 : r.a.x & 0xffff);
    sc = (s & 1) ? 0.0625f * d : d;
    mn = -8.0f * d;
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
struct FQ4_K : GgmlGemv<FQ4_K> {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q4_K;
  static constexpr int BS = 256, TS = 144, UPB = 4;  // unit: 32 B of qs (chunk jj), 64 weights
  static constexpr int UNIT_BLOCKS = 1, GEMV_K_MULT = 256;
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
  static DEV Raw load_row(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)(u >> 2) * TS;
    const uint8_t *qs = p + 16 + 32 * (u & 3);
    return {ld16<16>(qs), ld16<16>(qs + 16), ld4<4>(p + 4 * (u & 3))};
  }
  // Lane constants: a lane always decodes the same chunk jj = sub % 4 of a block, so the
  // placement of its two sub-blocks' 6-bit scale/min fields (GGMLDequant.q4K.scaleMin,
  // Core/GGMLDequant.swift:193-205) is fixed per lane: sub-block j < 4 reads bits [8j, 8j+6) of
  // words 1/2 of the header; j >= 4 reads 4 bits of word 3 and the top 2 bits of words 1/2.
  struct LaneC {
    bool lo;             // jj < 2
    uint32_t sh, wa, wh;  // bit offset of sub-block 2jj, low-field width (6 or 4), high width (0 or 2)
  };
  static DEV LaneC lane(int sub) {
    const int jj = sub & 3;
    return {jj < 2, (uint32_t)(16 * (jj & 1)), jj < 2 ? 6u : 4u, jj < 2 ? 0u : 2u};
  }
  // Chunk jj: low nibbles of its 32 bytes are sub-block 2jj (weights k0..k0+31), high nibbles
  // sub-block 2jj+1 (k0+32..k0+63). Low nibbles become 1024 + q, high ones 1024 + 16q, and
  // with S = sum code * x and X = sum x over the sub-block: sum q x = S - 1024 X, or S/16 - 64 X.
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &c) {
    const uint32_t qw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
    for (int hb = 0; hb < 2; hb++) {
      uint32_t xl[8], xh[8];
      unpack(s.slot(2 * hb), s.slot(2 * hb + 1), xl);
      unpack(s.slot(4 + 2 * hb), s.slot(5 + 2 * hb), xh);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const uint32_t q = qw[4 * hb + t], q8 = q >> 8;
        a0 = dot2(and_or(q, 0x000F000Fu, s.mg), xl[2 * t], a0);
        a1 = dot2(and_or(q8, 0x000F000Fu, s.mg), xl[2 * t + 1], a1);
        b0 = dot2(and_or(q, 0x00F000F0u, s.mg), xh[2 * t], b0);
        b1 = dot2(and_or(q8, 0x00F000F0u, s.mg), xh[2 * t + 1], b1);
      }
    }
    const uint32_t h0 = quad_bcast<0>(r.h), s0 = quad_bcast<1>(r.h), s1 = quad_bcast<2>(r.h),
                   s2 = quad_bcast<3>(r.h);
    const uint32_t A = c.lo ? s0 : s2, B = c.lo ? s1 : s2;
    const uint32_t mo = c.lo ? 0u : 4u;  // the min's low field sits 4 bits up in word 3
    auto field = [&](uint32_t w, uint32_t off, uint32_t wd, uint32_t top, uint32_t sh) {
      return __builtin_amdgcn_ubfe(w, off, wd) | (__builtin_amdgcn_ubfe(top, sh + 6, c.wh) << 4);
    };
    const uint32_t sc0 = field(A, c.sh, c.wa, s0, c.sh), m0 = field(B, c.sh + mo, c.wa, s1, c.sh);
    const uint32_t sc1 = field(A, c.sh + 8, c.wa, s0, c.sh + 8), m1 = field(B, c.sh + 8 + mo, c.wa, s1, c.sh + 8);
    const float d = h2f(h0 & 0xffff), dmin = h2f(h0 >> 16);
    const float dl0 = d * (float)sc0, dl1 = d * (float)sc1;
    const float xs_l = s.sum(0), xs_h = s.sum(1);
    return dl0 * ((a0 + a1) - 1024.0f * xs_l) - (dmin * (float)m0) * xs_l +
           dl1 * (0.0625f * (b0 + b1) - 64.0f * xs_h) - (dmin * (float)m1) * xs_h;
  }

  // Streaming verify: step = one super-block; a lane's quarter is chunk g (32 bytes of qs):
  // sub-unit 0 = sub-block 2g (low nibbles), 1 = sub-block 2g + 1 (high, 1024 + 16q).
  static constexpr int VNS = 2, VSTEP_BYTES = TS;
  static constexpr bool VGRID = false;
  struct VRaw {
    u4 h, q0, q1;
  };
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<16>(p), ld16<16>(p + 16 + 32 * g), ld16<16>(p + 32 + 32 * g)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t mg, const u4 *, const u4 *) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int hi = 0; hi < 2; hi++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const uint32_t m = hi ? 0x00F000F0u : 0x000F000Fu;
        const uint32_t q0 = q[2 * b], q1 = q[2 * b + 1];
        B[hi * 4 + b] = u4{and_or(q0, m, mg), and_or(q0 >> 8, m, mg), and_or(q1, m, mg), and_or(q1 >> 8, m, mg)};
      }
  }
  static DEV void vstage(const uint16_t *x, int j, int g, int s, u4 *A, float &off1, float &X) {
    const uint16_t *p = x + 256 * j + 64 * g + 32 * s;
    X = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = vx8p(p + 8 * b, X);
    off1 = 1024.0f * X;
  }
  static constexpr float voff() { return 1024.0f; }  // off1 of vstage, per unit of X
  static DEV void vscale(const VRaw &r, int g, int s, float &sc, float &mn) {
    int scv, m;
    q4k_scale_min(r.h.y, r.h.z, r.h.w, 2 * g + s, scv, m);
    const float d = h2f(r.h.x & 0xffff), dmin = h2f(r.h.x >> 16);
    sc = d * (float)scv * (s ? 0.0625f : 1.0f);
    mn = -(dmin * (float)m);
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
struct FQ6_K : GgmlGemv<FQ6_K> {
  static constexpr uint32_t TYPE = ISHZ_GGML_Q6_K;
  static constexpr int BS = 256, TS = 210, UPB = 4;  // unit: (n, l-half), 64 weights
  static constexpr int UNIT_BLOCKS = 1, GEMV_K_MULT = 256;
  static constexpr bool XSUM = true, GRID = false;
  static constexpr int R = 8, Q = 4;  // slot 2qq + i: k0 + 32qq + 8i; sum qq: k0 + 32qq
  static DEV int k0_of(int u) { return (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16; }
  static DEV int slot_k(int u, int r) { return k0_of(u) + 32 * (r >> 1) + 8 * (r & 1); }
  static DEV int sum_k(int u, int q) { return k0_of(u) + 32 * q; }
  static constexpr int SUM_LEN = 16;
  // Odd blocks sit two bytes off dword alignment (unaligned 16-byte loads; re-aligning in
  // registers was measured slower here, the kernel being VALU-bound).
  struct Raw {
    u4 qa, qb, qh;
    u2 sc;
    uint32_t d;
  };
  static DEV Raw load_row(const uint8_t *row, int u) {
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
  struct LaneC {
    uint32_t sh;  // 8 * lh: byte of the scale words this lane's l-half reads
  };
  static DEV LaneC lane(int sub) { return {(uint32_t)(8 * (sub & 1))}; }
  // Codes are assembled in place as fp16 halves: q1, q2 (low nibbles + qh bits) become 1024 + q,
  // q3, q4 (high nibbles + qh bits) 1024 + 16q with no shift of the nibble; sum (q - 32) x over a
  // 16-weight group is S - 1056 X, or S/16 - 96 X.
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &c) {
    float S[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};
    const u4 QA = r.qa, QB = r.qb, QH = r.qh;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const u4 x0 = s.slot(t >> 1), x1 = s.slot(2 + (t >> 1)), x2 = s.slot(4 + (t >> 1)),
               x3 = s.slot(6 + (t >> 1));
      const int o = 2 * (t & 1);
      const uint32_t a = QA[t], b = QB[t], h4 = QH[t] << 4, h2 = QH[t] << 2;
      const uint32_t a8 = a >> 8, b8 = b >> 8, h48 = QH[t] >> 4, h28 = QH[t] >> 6;
      S[0][0] = dot2(and_or(a, 0x000F000Fu, and_or(h4, 0x00300030u, s.mg)), x0[o], S[0][0]);
      S[0][1] = dot2(and_or(a8, 0x000F000Fu, and_or(h48, 0x00300030u, s.mg)), x0[o + 1], S[0][1]);
      S[1][0] = dot2(and_or(b, 0x000F000Fu, and_or(h2, 0x00300030u, s.mg)), x1[o], S[1][0]);
      S[1][1] = dot2(and_or(b8, 0x000F000Fu, and_or(h28, 0x00300030u, s.mg)), x1[o + 1], S[1][1]);
      S[2][0] = dot2(and_or(a, 0x00F000F0u, and_or(h4, 0x03000300u, s.mg)), x2[o], S[2][0]);
      S[2][1] = dot2(and_or(a8, 0x00F000F0u, and_or(h48, 0x03000300u, s.mg)), x2[o + 1], S[2][1]);
      S[3][0] = dot2(and_or(b, 0x00F000F0u, and_or(h2, 0x03000300u, s.mg)), x3[o], S[3][0]);
      S[3][1] = dot2(and_or(b8, 0x00F000F0u, and_or(h28, 0x03000300u, s.mg)), x3[o + 1], S[3][1]);
    }
    // sc[8n + lh + 2qq]: bytes lh, lh+2 of the low word, lh, lh+2 of the high word.
    const float d = h2f(r.d);
    const float s0 = (float)(int8_t)(r.sc.x >> c.sh), s1 = (float)(int8_t)(r.sc.x >> (c.sh + 16));
    const float s2 = (float)(int8_t)(r.sc.y >> c.sh), s3 = (float)(int8_t)(r.sc.y >> (c.sh + 16));
    return (d * s0) * ((S[0][0] + S[0][1]) - 1056.0f * s.sum(0)) +
           (d * s1) * ((S[1][0] + S[1][1]) - 1056.0f * s.sum(1)) +
           (d * s2) * (0.0625f * (S[2][0] + S[2][1]) - 96.0f * s.sum(2)) +
           (d * s3) * (0.0625f * (S[3][0] + S[3][1]) - 96.0f * s.sum(3));
  }

  // Streaming verify: step = one super-block; lane group g takes half n = g / 2, l in
  // 16 (g % 2) .. + 15: sub-unit qq (scale sc[8n + g % 2 + 2qq]) = weights 128n + 32qq + l, two
  // MFMAs (l halves). Codes decode to 1024 + q (q = 0..63) from a nibble of ql and two bits of qh.
  static constexpr int VNS = 4, VSTEP_BYTES = TS;
  static constexpr bool VGRID = false;
  struct VRaw {
    u4 ql0, ql1, qh, sc;
    uint32_t d;
  };
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    const int n = g >> 1, lh = g & 1;
    return {ld16<2>(p + 64 * n + 16 * lh), ld16<2>(p + 64 * n + 32 + 16 * lh), ld16<2>(p + 128 + 32 * n + 16 * lh),
            ld16<2>(p + 192), ld2(p + 208)};
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t mg, const u4 *, const u4 *) {
#pragma unroll
    for (int qq = 0; qq < 4; qq++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        uint32_t o[4];
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
          const int t = 2 * h + t2;
          const uint32_t a = ((qq & 1) ? r.ql1[t] : r.ql0[t]) >> (qq >= 2 ? 4 : 0);
          const uint32_t hq = r.qh[t];
          const uint32_t hs = qq == 0 ? hq << 4 : qq == 1 ? hq << 2 : qq == 2 ? hq : hq >> 2;
          o[2 * t2] = and_or(a, 0x000F000Fu, and_or(hs, 0x00300030u, mg));
          o[2 * t2 + 1] = and_or(a >> 8, 0x000F000Fu, and_or(hs >> 8, 0x00300030u, mg));
        }
        B[qq * 2 + h] = u4{o[0], o[1], o[2], o[3]};
      }
  }
  static DEV void vstage(const uint16_t *x, int j, int g, int s, u4 *A, float &off1, float &X) {
    const uint16_t *p = x + 256 * j + 128 * (g >> 1) + 16 * (g & 1) + 32 * s;
    X = 0.0f;
    A[0] = vx8p(p, X);
    A[1] = vx8p(p + 8, X);
    off1 = 1024.0f * X;
  }
  static constexpr float voff() { return 1024.0f; }  // off1 of vstage, per unit of X
  static constexpr float vkappa(int) { return -32.0f; }  // mn = -32 sc
  static DEV void vscale(const VRaw &r, int g, int s, float &sc, float &mn) {
    const int bi = 8 * (g >> 1) + (g & 1) + 2 * s;  // scale byte
    const float d = h2f(r.d) * (float)(int8_t)(r.sc[bi >> 2] >> (8 * (bi & 3)));
    sc = d;
    mn = -32.0f * d;
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

// Sign masks, computed in registers: bit j of the 8-bit pattern s flips the fp16 sign of weight j
// (natural pair order). With t = s << 7 (bits 7..14), word w is t * (2^(8-2w) + 2^(23-2w)): both
// multiplier and t fit 24 bits, so this is one full-rate v_mul_u32_u24 (a 32-bit v_mul_lo_u32 is
// quarter rate), and the two shifted copies of the pattern occupy disjoint bits, so bits 15 and 31
// hold signs 2w and 2w + 1; everything else is masked off.
DEV u4 sign_words(uint32_t s) {
  constexpr uint32_t SB = 0x80008000u;
  const uint32_t t = s << 7;
  return u4{mul24(t, 0x800100u) & SB, mul24(t, 0x200040u) & SB, mul24(t, 0x080010u) & SB,
            mul24(t, 0x020004u) & SB};
}
DEV uint32_t ksigns_pattern(uint32_t idx) { return idx | (__builtin_popcount(idx) & 1u) << 7; }

// ----------------------------------------------------------------------------------- IQ2_XS
// GGMLDequant.iq2XS (Core/GGMLDequant.swift:264-285): fp16 d at 0, qs u16[32] at 2 (9-bit grid
// index, 7-bit sign index), scales u8[8] at 66. Entry l of group ib (weights 32ib + 8l + j) is
// d*(0.5+nibble)*0.25 * grid[q&511][j] * sign(ksigns[q>>9], j), nibble = scales[ib] lo for
// l < 2, hi otherwise.
// IQ2_XS sign masks of one ksigns index (7 bits; the eighth sign is their parity) in the GEMV's
// pair order (x0,x2 | x1,x3 | x4,x6 | x5,x7), sign bits at 15 and 31 of each word, computed in
// registers instead of read from an LDS table. With t = s << 7, word w is t * (2^a + 2^b), a
// 24-bit by 24-bit product (full-rate v_mul_u32_u24): the two shifted copies of the pattern occupy
// disjoint bits, so the product is their OR, and bits 15 and 31 are signs (0, 2), (1, 3), (4, 6),
// (5, 7); the caller keeps only those bits (mask 0x80008000).
DEV u4 iq2xs_sign_words(uint32_t idx) {
  const uint32_t t = (idx | (__builtin_popcount(idx) & 1u) << 7) << 7;
  return u4{mul24(t, 0x400100u), mul24(t, 0x200080u), mul24(t, 0x040010u), mul24(t, 0x020008u)};
}

struct FIQ2_XS : GgmlGemv<FIQ2_XS> {
  static constexpr uint32_t TYPE = ISHZ_GGML_IQ2_XS;
  static constexpr int BS = 256, TS = 74, UPB = 4;  // unit: two groups, 16 B of qs, 64 weights
  static constexpr int UNIT_BLOCKS = 1, GEMV_K_MULT = 256;
  static constexpr bool XSUM = false, GRID = true;
  static constexpr int R = 8, Q = 1;  // slot l: k0 + 8l
  static constexpr int WG = 512;  // as the other codebook formats (GgmlQuarter): 13.0 vs 13.9 us
  static int occ(const Args &) { return 4; }
  static DEV int slot_k(int u, int r) { return (u >> 2) * 256 + (u & 3) * 64 + 8 * r; }
  static DEV int sum_k(int u, int q) { return 0; }
  static constexpr int SUM_LEN = 16;
  // sc: the dword ending with the unit's two scale bytes (bits 16..31); d: the dword starting with
  // the block's fp16 d (bits 0..15). Whole-dword loads: a 2-byte load's zero extension, kept as a
  // mask on the ring's registers, made the compiler wait for every load in flight at the loop's
  // back edge.
  struct Raw {
    u4 q;
    uint32_t sc, d;
  };
  static DEV Raw load_row(const uint8_t *row, int u) {
    const uint8_t *p = row + (size_t)(u >> 2) * TS;
    const int pp = u & 3;
    return {ld16<2>(p + 2 + 16 * pp), ld4<2>(p + 64 + 2 * pp), ld4<2>(p)};
  }
  struct LaneC {};
  static DEV LaneC lane(int sub) { return {}; }
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &) {
    // entries 2j, 2j + 1 (16 weights) share nibble j of the unit's scale bytes:
    // d * (0.5 + nib) * 0.25 = (d / 4) * nib + d / 8, exact scalings of d
    const float d = h2f(r.d & 0xffffu), dq = 0.25f * d, dh = 0.125f * d;
    const u4 QS = r.q;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float e = 0.0f;
#pragma unroll
      for (int l = 2 * j; l < 2 * j + 2; l++) {
        const uint32_t q = (QS[j] >> (16 * (l & 1))) & 0xffffu;
        const u4 G = s.grid[q & 511], M = iq2xs_sign_words(q >> 9);
        const u4 X = s.slot(l);
        constexpr uint32_t SB = 0x80008000u;
        e = dot2(G.x ^ (M.x & SB), X.x, e);
        e = dot2(G.y ^ (M.y & SB), X.y, e);
        e = dot2(G.z ^ (M.z & SB), X.z, e);
        e = dot2(G.w ^ (M.w & SB), X.w, e);
      }
      const float nib = (float)__builtin_amdgcn_ubfe(r.sc, 16 + 4 * j, 4);
      acc = fmaf(fmaf(dq, nib, dh), e, acc);
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

  // Streaming verify: step = one super-block; lane group g takes groups 2g, 2g + 1 (entries
  // e = 0..7, 8 weights each, one MFMA each); sub-unit e / 2 shares one 4-bit scale. B is the
  // grid entry with its signs (exact small integers in fp16); A is x in natural order.
  static constexpr int VNS = 4, VSTEP_BYTES = TS;
  static constexpr bool VGRID = true;
  static constexpr bool VPLAIN = true;  // signed grid entries times the scale: value = sc * C
  struct VRaw {
    u4 q;
    uint32_t sc, d;
  };
  static DEV VRaw vload(const uint8_t *row, int j, int g) {
    const uint8_t *p = row + (size_t)j * TS;
    return {ld16<2>(p + 2 + 16 * g), ld2(p + 66 + 2 * g), ld2(p)};
  }
  // signs from registers (sign_words) rather than the LDS table: one random LDS read fewer per
  // eight weights, 2-3 % faster at 17408x5120, M = 8
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t, const u4 *grid, const u4 *) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t q = (r.q[e >> 1] >> (16 * (e & 1))) & 0xffffu;
      B[e] = grid[q & 511] ^ sign_words(ksigns_pattern(q >> 9));
    }
  }
  static DEV void vstage(const uint16_t *x, int j, int g, int s, u4 *A, float &off1, float &X) {
    const uint16_t *p = x + 256 * j + 64 * g + 16 * s;
    A[0] = vx8n(p);
    A[1] = vx8n(p + 8);
    off1 = 0.0f;
    X = 0.0f;
  }
  static DEV void vscale(const VRaw &r, int, int s, float &sc, float &mn) {
    const uint32_t nib = (r.sc >> (8 * (s >> 1) + 4 * (s & 1))) & 15;
    sc = h2f(r.d) * (0.5f + (float)nib) * 0.25f;
    mn = 0.0f;
  }
};

}  // namespace ishz
