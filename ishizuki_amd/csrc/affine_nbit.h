// MLX affine packs of 3 to 8 bits per weight (2 bits too, for the MoE experts; the 2-bit matmul
// has its own format, FAffine) (VerifyMatmul.applyAny: the 4- and 8-bit fast paths
// and the generic one for 3, 5, 6 and 7 bits, Core/VerifyMatmul.swift:83-89,
// 273-290; pack layout Quantize/WeightedAffineQuantizer.swift:142-153): w[n][k] = s[n][k/gs] * q +
// b[n][k/gs], q the bits-wide field k of the row's little-endian u32 stream, so a word holds 8
// (4-bit) or 4 (8-bit) consecutive codes and 64 codes of any width fill 2 * bits whole words.
//
// One format serves both skeletons: a "unit" / verify quarter is 64 weights of one group (group
// size 64 or 128), 32 or 64 bytes of codes plus the group's scale and bias. Codes are masked in
// place with the fp16 exponent of 1024 (`v_and_or_b32`), so a word yields exact fp16 1024 + q in
// pairs; the offset and the bias come back through the sum of x over the unit:
//   sum_k w_k x_k = s * (sum (1024 + q_k) x_k - 1024 X) + b * X.
// Pair orders: 4-bit word >> 4j masked with 0x000F000F gives codes (j, j + 4); 8-bit word (>> 8)
// masked with 0x00FF00FF gives (0, 2) and (1, 3). x is staged in the same pair order. 3, 5, 6
// and 7 bits: codes (2j, 2j + 1) are the low 2 * bits of one funnel shift of the unit's words (a
// compile-time offset into the stream), masked and shifted into a pair; x in natural order.
#pragma once
#include "ggml_formats.h"
#include "vgemm.h"

namespace ishz {

// (x0, x4, x1, x5, x2, x6, x3, x7): the pair order of 4-bit codes masked from one word.
DEV u4 perm04(u4 a) {
  return u4{(a.x & 0xffffu) | (a.z << 16), (a.x >> 16) | (a.z & 0xffff0000u), (a.y & 0xffffu) | (a.w << 16),
            (a.y >> 16) | (a.w & 0xffff0000u)};
}

// One weight row of an affine pack: its code words and its groups' scales and biases.
struct AffRow {
  const uint32_t *codes;
  const uint16_t *scales, *biases;
};

// The problem the streaming MFMA kernel runs for these packs (one group: the whole matrix).
struct VAffineN {
  const uint16_t *x;
  const uint32_t *codes;
  const uint16_t *scales, *biases;
  int M, K, N;
  Out y;
  int wpr, gpr;  // code words and scale groups per row
  DEV AffRow arow(int row) const {
    return {codes + (size_t)row * wpr, scales + (size_t)row * gpr, biases + (size_t)row * gpr};
  }
  struct Group {};
  DEV bool group(int, Group &) const { return true; }
  DEV int count(const Group &) const { return M; }
  DEV int rows(const Group &) const { return N; }
  DEV const uint16_t *xrow(const Group &, int tk) const { return x + (size_t)tk * K; }
  DEV const uint8_t *wrow(const Group &, int) const { return nullptr; }  // the format reads through vload_p
  DEV void finish(const Group &, int c0, int m, int tb, int te, const float *out) const {
    for (int o = threadIdx.x; o < (te - tb) * 256; o += blockDim.x) {
      const int tk = (o >> 4) & 15, row = (tb + (o >> 8)) * 16 + (o & 15);
      if (tk < m && row < N) y.put((size_t)(c0 + tk) * N + row, c0 + tk, out[o]);
    }
  }
};

template <int BITS, int GS, bool BF16S>
struct FAffineN : GgmlGemv<FAffineN<BITS, GS, BF16S>> {
  static_assert(BITS >= 2 && BITS <= 8, "2- to 8-bit packs");
  using Base = GgmlGemv<FAffineN<BITS, GS, BF16S>>;
  struct Args {
    const uint32_t *codes;
    const uint16_t *scales, *biases;
    int K, N;
  };
  static constexpr int WPU = 64 * BITS / 32;  // code words per 64-weight unit
  static constexpr int BS = 64, UPB = 1, UNIT_BLOCKS = 1;
  static constexpr int RING = 3;  // as FAffine::RING
  static constexpr int R = 8, Q = 2, SUM_LEN = 32;
  static constexpr bool XSUM = true, GRID = false, VGRID = false, XPERM = BITS == 8;
  static constexpr bool MASKED = BITS == 4 || BITS == 8;  // whole codes per word: masked in place
  static DEV u4 xperm(u4 v) {
    if constexpr (BITS == 4) return perm04(v);
    else if constexpr (BITS == 8) return perm0213(v);
    else return v;
  }
  static __host__ __device__ int units(int K) { return K / 64; }
  static int occ(const Args &) { return 2; }
  static size_t extra_lds_bytes(const Args &) { return 0; }
  static DEV int slot_k(int u, int r) { return 64 * u + 8 * r; }
  static DEV int sum_k(int u, int q) { return 64 * u + 32 * q; }
  struct Raw {
    u2 q[WPU / 2];
    uint32_t s, b;
  };
  static DEV uint32_t word(const Raw &r, int i) { return r.q[i >> 1][i & 1]; }
  static DEV float ld_s(uint32_t v) { return BF16S ? __builtin_bit_cast(float, v << 16) : h2f(v); }
  // Unit u of a row: its codes and its group's scale and bias.
  static DEV Raw load_unit(const AffRow &w, int u) {
    Raw r;
    const u2 *c = (const u2 *)(w.codes + (size_t)u * WPU);  // 8-byte aligned: rows are K * BITS / 8 bytes
#pragma unroll
    for (int i = 0; i < WPU / 2; i++) r.q[i] = c[i];
    r.s = w.scales[u * 64 / GS];
    r.b = w.biases[u * 64 / GS];
    return r;
  }
  static DEV Raw load(const Args &a, int row, int u) {
    const size_t gpr = a.K / GS;
    return load_unit({a.codes + (size_t)row * (a.K * BITS / 32), a.scales + row * gpr, a.biases + row * gpr}, u);
  }
  struct LaneC {};
  static DEV LaneC lane(int) { return {}; }
  // Eight B-operand / dot words of 8 codes each, in the x pair order.
  static DEV void decode(const Raw &r, u4 *B, uint32_t mg) {
#pragma unroll
    for (int t = 0; t < 8; t++) {
      if constexpr (BITS == 4) {
        const uint32_t w = word(r, t);
        B[t] = u4{and_or(w, 0x000F000Fu, mg), and_or(w >> 4, 0x000F000Fu, mg), and_or(w >> 8, 0x000F000Fu, mg),
                  and_or(w >> 12, 0x000F000Fu, mg)};
      } else if constexpr (BITS == 8) {
        const uint32_t w0 = word(r, 2 * t), w1 = word(r, 2 * t + 1);
        B[t] = u4{and_or(w0, 0x00FF00FFu, mg), and_or(w0 >> 8, 0x00FF00FFu, mg), and_or(w1, 0x00FF00FFu, mg),
                  and_or(w1 >> 8, 0x00FF00FFu, mg)};
      } else {
        constexpr uint32_t MASK = (1u << BITS) - 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int p = (8 * t + 2 * i) * BITS, wi = p >> 5, o = p & 31;  // codes 8t + 2i, + 1
          const uint32_t lo = word(r, wi);
          const uint32_t win = o + 2 * BITS <= 32 ? lo >> o : __builtin_amdgcn_alignbit(word(r, wi + 1), lo, o);
          B[t][i] = (((win >> BITS) & MASK) << 16) | and_or(win, MASK, mg);
        }
      }
    }
  }
  static DEV float dot(const Raw &r, const UnitX &s, const LaneC &) {
    u4 B[8];
    decode(r, B, s.mg);
    float S = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const u4 X = s.slot(t);
      S = dot2(B[t].x, X.x, S);
      S = dot2(B[t].y, X.y, S);
      S = dot2(B[t].z, X.z, S);
      S = dot2(B[t].w, X.w, S);
    }
    const float X = s.sum(0) + s.sum(1);
    return ld_s(r.s) * (S - 1024.0f * X) + ld_s(r.b) * X;
  }
  typedef typename Base::XPre XPre;
  static DEV XPre stage_load(const Args &, const uint16_t *x, int units) {
    XPre p;
    Base::load_slots(x, units, threadIdx.x, p.v);
    Base::load_sums(x, units, threadIdx.x, p.sv);
    return p;
  }
  static DEV void stage(const Args &, const uint16_t *x, u4 *xs, float *xsum, u4 *extra, int units, const XPre &pre) {
    Base::stage_body(x, xs, xsum, extra, units, pre);
  }

  // Streaming MFMA verify: quarter g of step j is unit 4j + g of the chunk; one scale group per
  // quarter (VNS = 1, eight MFMAs).
  static constexpr int VNS = 1, VSTEP_BYTES = 0, VDEPTH = 2;
  typedef Raw VRaw;
  // Any problem whose rows are affine rows: P::arow(group, row) or, with one group, P::arow(row).
  template <class P>
  static DEV VRaw vload_p(const P &p, const typename P::Group &gp, int row, int kc0, int j, int g) {
    if constexpr (requires { p.arow(gp, row); })
      return load_unit(p.arow(gp, row), kc0 / 64 + 4 * j + g);
    else
      return load_unit(p.arow(row), kc0 / 64 + 4 * j + g);
  }
  static DEV void vdecode(const VRaw &r, u4 *B, uint32_t mg, const u4 *, const u4 *) { decode(r, B, mg); }
  static DEV void vstage(const uint16_t *x, int j, int g, int, u4 *A, float &off1, float &X) {
    const uint16_t *p = x + 256 * j + 64 * g;
    X = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const u4 v = *(const u4 *)(p + 8 * b);
#pragma unroll
      for (int e = 0; e < 4; e++) X = dot2(v[e], 0x3C003C00u, X);
      A[b] = xperm(v);
    }
    off1 = 1024.0f * X;
  }
  static constexpr float voff() { return 1024.0f; }  // off1 of vstage, per unit of X
  static DEV void vscale(const VRaw &r, int, int, float &sc, float &mn) {
    sc = ld_s(r.s);
    mn = ld_s(r.b);
  }
};

// y[M][N] = x . W^T for a 3- to 8-bit pack: the streaming GEMV at M = 1, the streaming MFMA
// kernel for M = 2..16 (K a multiple of 256 there; declined otherwise).
template <int BITS, int GS, bool BF16S>
static int affine_nbit(const void *x, int M, int K, const uint32_t *codes, const void *scales, const void *biases,
                       int N, const Out &y, hipStream_t st) {
  using F = FAffineN<BITS, GS, BF16S>;
  if (K % 64) return decline("K must be a multiple of 64");
  if (M == 1) {
    const typename F::Args a{codes, (const uint16_t *)scales, (const uint16_t *)biases, K, N};
    return launch_gemv<F>(a, x, y.y, st, y.dt, y.rs);
  }
  if (K % 256) return decline("verify rows need K a multiple of 256 for packs other than 2-bit");
  const VAffineN p{(const uint16_t *)x, codes, (const uint16_t *)scales, (const uint16_t *)biases, M, K, N,
                   y, K * BITS / 32, K / GS};
  const int ntiles = (N + 15) / 16;
  const int T = (ntiles + gemv_num_cu() - 1) / gemv_num_cu();
  switch ((M + 3) / 4) {
    case 1: return launch_vgemm_p<F, VAffineN, 1>(p, K, N, 1, T, st);
    case 2: return launch_vgemm_p<F, VAffineN, 2>(p, K, N, 1, T, st);
    case 3: return launch_vgemm_p<F, VAffineN, 3>(p, K, N, 1, T, st);
    default: return launch_vgemm_p<F, VAffineN, 4>(p, K, N, 1, T, st);
  }
}

}  // namespace ishz
