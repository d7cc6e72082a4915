// EXL3 trellis-coded projections on gfx950, decoded inside the matmul.
//
// Replaces EXL3Kernels (Sources/IshizukiKit/Core/EXL3.swift:79-332): apply (:82-100) = rotate in,
// matvec (1..16 rows), rotate out; dequantize (:133-147); rotate (:102-124).
//
// Format (EXL3Tensor, :9-77): trellis int16 [K/16][N/16][16*bits], one 16x16 tile per
// (tk, tn). A tile's int16s pair little-endian into u32 words read as one MSB-first ring of
// RING bits; weight p (0..255) is the codebook image of the 16 bits ending at end(p) (wrapping);
// p = 8*lane + i sits at row (lane%4)*2 + {0,1,8,9}[i%4], column lane/4 + 8*(i/4).
//
// Work split: lane (j = l%16, g = l/16) decodes positions 8*(4*(j%8) + g) + 4*(j/8) + {0..3},
// which are rows 2g + {0,1,8,9} of column j: every weight of a tile is decoded exactly once per
// wave, already in MFMA B-operand order (k rows by lane group, column j by lane).
#include <algorithm>
#include <type_traits>
#include <cstdlib>

#include <mutex>
#include <string>

#include "common.h"


namespace ishz {

// exl3_decode (EXL3.swift:136-147): 3INST / MCG / MUL1 codebooks, fp16 single rounding.
DEV _Float16 exl3_decode(uint32_t s, int cb) {
  if (cb == 2) {
    const uint32_t x = s * 0x83DCD12Du;
    const uint32_t p = (x & 0x00ff00ffu) + ((x >> 8) & 0x00ff00ffu);
    const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)((p & 0xffffu) + (p >> 16) + 0x6400u));
    return __builtin_fmaf16(h, __builtin_bit_cast(_Float16, (uint16_t)0x1eee),
                            __builtin_bit_cast(_Float16, (uint16_t)0xc931));
  }
  uint32_t x = cb == 1 ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
  x = (x & 0x8fff8fffu) ^ 0x3b603b60u;
  return __builtin_bit_cast(_Float16, (uint16_t)x) + __builtin_bit_cast(_Float16, (uint16_t)(x >> 16));
}

// Where the states lie in a tile's bit ring. At an integer rate of KA bits per weight, position p
// consumes KA bits and its state ends at ring bit KA (p + 1). At a half rate (KA + 1/2 bits) an
// even/odd pair consumes 2 KA + 1 bits, the even position KA of them and the odd one KA + 1. A
// state is the 16 ring bits ending there, read MSB first (bit 0 is the top bit of word 0), so it
// reaches back into the bits of earlier positions and wraps around the ring.
template <int KA, bool HALF>
struct Trellis {
  static constexpr int RING = HALF ? 128 * (2 * KA + 1) : 256 * KA;  // bits per 16x16 tile
  static constexpr int WORDS = RING / 32;
  static __host__ __device__ constexpr int bit_end(int p) {
    return HALF ? (p / 2) * (2 * KA + 1) + KA + (p % 2) * (KA + 1) : (p + 1) * KA;
  }
  // First ring bit of position p's state.
  static DEV int first_bit(int p) { return (bit_end(p) + RING - 16) % RING; }
  // Start of the state of position p0 + i relative to that of p0 (p0 even).
  static constexpr int offset(int i) { return bit_end(i) - bit_end(0); }
  // The 16-bit state starting at ring bit b: the 32 bits from b are one funnel shift of the word
  // holding b and the next word (b on a word boundary: that word alone); the state is the top half.
  static DEV uint32_t state(const uint32_t *tile, int b) {
    const int w = b >> 5, o = b & 31;
    const uint32_t hi = tile[w];
    const uint32_t bits32 = o ? __builtin_amdgcn_alignbit(hi, tile[(w + 1) % WORDS], 32 - o) : hi;
    return bits32 >> 16;
  }
  // The four weights at positions p0 .. p0 + 3, as two packed fp16 pairs.
  static DEV u2 decode4(const uint32_t *tile, int p0, int cb) {
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
      h[i] = __builtin_bit_cast(uint16_t, exl3_decode(state(tile, (first_bit(p0) + offset(i)) % RING), cb));
    return u2{h[0] | h[1] << 16, h[2] | h[3] << 16};
  }
};

// ------------------------------------------------------------------- matvec / verify
// A workgroup owns one column tile tn (16 outputs); its KS waves take tiles tk = wave, wave+KS,
// ... and partial results are summed through LDS. MF: one MFMA 16x16x16 per tile (tokens in A,
// up to 16). Otherwise (M = 1) each lane dots its four weights with x in fp32 (v_dot2) and the
// four k-groups of a column are summed by cross-lane shuffles.
template <int KA, bool HALF, bool MF>
__global__ __launch_bounds__(1024) void exl3_mm(const uint16_t *__restrict__ xh, int M, int K,
                                                const uint32_t *__restrict__ trellis, int N, int cb,
                                                float *__restrict__ yh) {
  using TR = Trellis<KA, HALF>;
  extern __shared__ __align__(16) float red[];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int tn = blockIdx.x, tiles_n = N / 16, tiles_k = K / 16;
  const int p0 = 8 * (4 * (j & 7) + g) + 4 * (j >> 3);
  const uint32_t *col = trellis + (size_t)tn * TR::WORDS;
  const size_t tstride = (size_t)tiles_n * TR::WORDS;

  if constexpr (MF) {
    const bool tok = j < M;
    const uint16_t *xr = xh + (size_t)(tok ? j : 0) * K + 2 * g;
    f4 acc = {0, 0, 0, 0};
    for (int tk = wave; tk < tiles_k; tk += KS) {
      const u2 B = TR::decode4(col + tk * tstride, p0, cb);
      const u2 A = tok ? u2{*(const uint32_t *)(xr + 16 * tk), *(const uint32_t *)(xr + 16 * tk + 8)}
                       : u2{0, 0};
      acc = mfma16(as_h4(A), as_h4(B), acc);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) red[(wave * 4 + r) * 64 + lane] = acc[r];
    __syncthreads();
    for (int o = threadIdx.x; o < 256; o += blockDim.x) {
      const int r = o >> 6, l = o & 63;
      float s = 0.0f;
      for (int v = 0; v < KS; v++) s += red[(v * 4 + r) * 64 + l];
      const int t = 4 * (l >> 4) + r;
      if (t < M) yh[(size_t)t * N + tn * 16 + (l & 15)] = s;
    }
  } else {
    const uint16_t *xr = xh + 2 * g;
    float acc = 0.0f;
    for (int tk = wave; tk < tiles_k; tk += KS) {
      const u2 B = TR::decode4(col + tk * tstride, p0, cb);
      acc = dot2(B.x, *(const uint32_t *)(xr + 16 * tk), acc);
      acc = dot2(B.y, *(const uint32_t *)(xr + 16 * tk + 8), acc);
    }
    acc += lane_xor16(acc);
    acc += lane_xor32(acc);
    if (g == 0) red[wave * 16 + j] = acc;
    __syncthreads();
    if (threadIdx.x < 16) {
      float s = 0.0f;
      for (int v = 0; v < KS; v++) s += red[v * 16 + threadIdx.x];
      yh[tn * 16 + threadIdx.x] = s;
    }
  }
}

// fp32 activations at fp32 precision (EXL3Kernels.matvec templated on the activation type,
// Core/EXL3.swift:286-330): each weight's exact fp16 decode, widened, times fp32 x in fp32 FMAs,
// for up to 16 token rows. The work split of exl3_mm: a workgroup per column tile, its waves
// taking K tiles round-robin; lane (j, g) holds rows 2g + {0, 1, 8, 9} of column j.
template <int KA, bool HALF>
__global__ __launch_bounds__(256) void exl3_mm_f32(const float *__restrict__ x, int M, int K,
                                                   const uint32_t *__restrict__ trellis, int N, int cb,
                                                   float *__restrict__ yh) {
  using TR = Trellis<KA, HALF>;
  __shared__ float red[4][16][16];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int tn = blockIdx.x, tiles_n = N / 16, tiles_k = K / 16;
  const int p0 = 8 * (4 * (j & 7) + g) + 4 * (j >> 3);
  const uint32_t *col = trellis + (size_t)tn * TR::WORDS;
  const size_t tstride = (size_t)tiles_n * TR::WORDS;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; m++) acc[m] = 0.0f;
  for (int tk = wave; tk < tiles_k; tk += KS) {
    const u2 B = TR::decode4(col + tk * tstride, p0, cb);
    const float w0 = h2f(B.x & 0xffffu), w1 = h2f(B.x >> 16), w2 = h2f(B.y & 0xffffu), w3 = h2f(B.y >> 16);
    const float *xr = x + 16 * tk + 2 * g;
#pragma unroll
    for (int m = 0; m < 16; m++) {
      if (m >= M) continue;
      const float2 a = *(const float2 *)(xr + (size_t)m * K), b = *(const float2 *)(xr + (size_t)m * K + 8);
      float t = acc[m];
      t = __builtin_fmaf(w0, a.x, t);
      t = __builtin_fmaf(w1, a.y, t);
      t = __builtin_fmaf(w2, b.x, t);
      t = __builtin_fmaf(w3, b.y, t);
      acc[m] = t;
    }
  }
#pragma unroll
  for (int m = 0; m < 16; m++) {
    if (m >= M) continue;
    float v = acc[m];
    v += lane_xor16(v);
    v += lane_xor32(v);
    if (g == 0) red[wave][m][j] = v;
  }
  __syncthreads();
  for (int o = threadIdx.x; o < M * 16; o += blockDim.x) {
    const int m = o >> 4, jj = o & 15;
    float v = 0.0f;
    for (int w = 0; w < KS; w++) v += red[w][m][jj];
    yh[(size_t)m * N + tn * 16 + jj] = v;
  }
}

// ------------------------------------------------------------------- streaming matvec / verify
// For rates whose four lane states span at most 32 bits: a lane's window is one v_alignbit of
// two tile words, each state one bit-field extract, and two weights are decoded per packed fp16
// operation. A workgroup owns TN column tiles and its waves split the K tiles (tk = wave, wave +
// KS, ...), keeping D steps of tile words and x in flight; partials meet in LDS at the end.
template <int KA, bool HALF>
struct Trellis32 {
  using TR = Trellis<KA, HALF>;
  static constexpr bool FITS = TR::offset(3) <= 16;  // the four states within 32 bits
  // The lane's 32-bit window (from the first bit of p0's state): words ja, jb funnel-shifted by amt.
  struct Win {
    int ja, jb, amt;
  };
  static DEV Win window(int p0) {
    const int b = TR::first_bit(p0), w = b >> 5, o = b & 31;
    return o ? Win{w, (w + 1) % TR::WORDS, 32 - o} : Win{w, w, 0};
  }
  // Bit-field offset of state i inside the window.
  static constexpr int field(int i) { return 16 - TR::offset(i); }
};

// Codebook images of two states, packed as fp16 (a in the low half): exl3_decode, pairwise.
template <int CB>
DEV uint32_t exl3_decode2(uint32_t sa, uint32_t sb) {
  if constexpr (CB == 2) {
    auto p = [](uint32_t s) {
      const uint32_t x = s * 0x83DCD12Du;
      const uint32_t q = (x & 0x00ff00ffu) + ((x >> 8) & 0x00ff00ffu);
      return ((q & 0xffffu) + (q >> 16) + 0x6400u) & 0xffffu;
    };
    const h2 h = as_h2(p(sa) | p(sb) << 16);
    const h2 m = as_h2(0x1eee1eeeu), c = as_h2(0xc931c931u);
    return __builtin_bit_cast(uint32_t, (h2)__builtin_elementwise_fma(h, m, c));
  } else {
    auto x = [](uint32_t s) {
      const uint32_t v = CB == 1 ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
      return (v & 0x8fff8fffu) ^ 0x3b603b60u;
    };
    const uint32_t xa = x(sa), xb = x(sb);
    const uint32_t lo = __builtin_amdgcn_perm(xb, xa, 0x05040100u), hi = __builtin_amdgcn_perm(xb, xa, 0x07060302u);
    return __builtin_bit_cast(uint32_t, as_h2(lo) + as_h2(hi));
  }
}

// 3INST / MCG image of one state as the two fp16 halves whose sum is the weight (exl3_decode
// before its final add). The M = 1 matvec multiplies them by (x, x) as two MFMA k-entries: the
// halves meet x in fp32, so the weight's fp16 rounding of their sum is skipped (a difference of
// at most half an fp16 ulp per weight, inside the matmul tolerance; dequantization keeps the
// exact decode).
template <int CB>
DEV uint32_t exl3_halves(uint32_t s) {
  static_assert(CB != 2, "MUL1 decodes to one fp16 directly");
  const uint32_t v = CB == 1 ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
  return (v & 0x8fff8fffu) ^ 0x3b603b60u;
}
DEV uint32_t dup_lo(uint32_t p) { return __builtin_amdgcn_perm(p, p, 0x01000100u); }
DEV uint32_t dup_hi(uint32_t p) { return __builtin_amdgcn_perm(p, p, 0x03020302u); }

template <int KA, bool HALF, int CB, bool MF, int TN, int D>
__global__ __launch_bounds__(1024) void exl3_mm2(const uint16_t *__restrict__ xh, int M, int K,
                                                const uint32_t *__restrict__ trellis, int N,
                                                float *__restrict__ yh) {
  using TR = Trellis<KA, HALF>;
  using T32 = Trellis32<KA, HALF>;
  extern __shared__ __align__(16) float red2[];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int tn0 = blockIdx.x * TN, tiles_n = N / 16, tiles_k = K / 16;
  const typename T32::Win wn = T32::window(8 * (4 * (j & 7) + g) + 4 * (j >> 3));
  const int tok = MF ? (j < M ? j : 0) : 0;
  const uint16_t *xr = xh + (size_t)tok * K + 2 * g;
  const size_t tstride = (size_t)tiles_n * TR::WORDS;
  const uint32_t *base = trellis + (size_t)tn0 * TR::WORDS;

  struct Raw {
    uint32_t w[TN][2];
    uint32_t xa, xb;
  };
  const int nsteps = tiles_k > wave ? (tiles_k - wave + KS - 1) / KS : 0;
  auto load = [&](int i, Raw &r) {
    const int tk = wave + KS * min(i, nsteps - 1);
    const uint32_t *tp = base + tk * tstride;
#pragma unroll
    for (int t = 0; t < TN; t++) {
      r.w[t][0] = tp[t * TR::WORDS + wn.ja];
      r.w[t][1] = tp[t * TR::WORDS + wn.jb];
    }
    r.xa = *(const uint32_t *)(xr + 16 * tk);
    r.xb = *(const uint32_t *)(xr + 16 * tk + 8);
  };
  using Acc = typename std::conditional<MF, f4, float>::type;
  Acc acc[TN];
#pragma unroll
  for (int t = 0; t < TN; t++) acc[t] = Acc{};
  Raw ring[D];
  if (nsteps > 0) {
#pragma unroll
    for (int d = 0; d < D - 1; d++) load(d, ring[d]);
  }
  const bool live = MF ? j < M : true;
  for (int i0 = 0; i0 < nsteps; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const int i = i0 + d;
      if (i >= nsteps) break;
      load(i + D - 1, ring[(d + D - 1) % D]);
      const Raw &r = ring[d];
#pragma unroll
      for (int t = 0; t < TN; t++) {
        const uint32_t win = __builtin_amdgcn_alignbit(r.w[t][0], r.w[t][1], wn.amt);
        const uint32_t s0 = __builtin_amdgcn_ubfe(win, T32::field(0), 16);
        const uint32_t s1 = __builtin_amdgcn_ubfe(win, T32::field(1), 16);
        const uint32_t s2 = __builtin_amdgcn_ubfe(win, T32::field(2), 16);
        const uint32_t s3 = __builtin_amdgcn_ubfe(win, T32::field(3), 16);
        const uint32_t b01 = exl3_decode2<CB>(s0, s1), b23 = exl3_decode2<CB>(s2, s3);
        if constexpr (MF) {
          const u2 A = live ? u2{r.xa, r.xb} : u2{0, 0};
          acc[t] = mfma16(as_h4(A), as_h4(u2{b01, b23}), acc[t]);
        } else {
          acc[t] = dot2(b23, r.xb, dot2(b01, r.xa, acc[t]));
        }
      }
    }
  }
  if constexpr (MF) {
#pragma unroll
    for (int t = 0; t < TN; t++)
#pragma unroll
      for (int q = 0; q < 4; q++) red2[((wave * TN + t) * 4 + q) * 64 + lane] = acc[t][q];
    __syncthreads();
    for (int o = threadIdx.x; o < TN * 256; o += blockDim.x) {
      const int t = o >> 8, q = (o >> 6) & 3, l = o & 63;
      float sum = 0.0f;
      for (int v = 0; v < KS; v++) sum += red2[((v * TN + t) * 4 + q) * 64 + l];
      const int tk = 4 * (l >> 4) + q;
      if (tk < M) yh[(size_t)tk * N + (tn0 + t) * 16 + (l & 15)] = sum;
    }
  } else {
#pragma unroll
    for (int t = 0; t < TN; t++) {
      float a = acc[t];
      a += lane_xor16(a);
      a += lane_xor32(a);
      if (g == 0) red2[(wave * TN + t) * 16 + j] = a;
    }
    __syncthreads();
    for (int o = threadIdx.x; o < TN * 16; o += blockDim.x) {
      float sum = 0.0f;
      for (int v = 0; v < KS; v++) sum += red2[(v * TN + (o >> 4)) * 16 + (o & 15)];
      yh[(tn0 + (o >> 4)) * 16 + (o & 15)] = sum;
    }
  }
}

// The 128-point Walsh-Hadamard transform of one block held as two values per lane (lane l holds
// entries 2l, 2l + 1), in Sylvester order, scaled by 1 / sqrt(128): the in-lane pair first, then
// one cross-lane exchange per bit of the lane index. The rotation kernel and the matvec's fused
// input rotation both use it, so their results are bit-identical.
DEV void wht128_pair(float &v0, float &v1, int lane) {
  float a = v0 + v1, b = v0 - v1;
  v0 = a;
  v1 = b;
  // partner lane ^ m: m = 1, 2, 4, 8 by DPP inside 16-lane rows, 16 and 32 by the row swaps
  // (v_permlane16_swap / v_permlane32_swap) instead of LDS-pipe shuffles; the lower lane keeps
  // v + p, the upper p - v, as fma(v, +-1, p) (exact, the same rounding)
  auto stage = [&](float p0, float p1, int m) {
    const float s = (lane & m) ? -1.0f : 1.0f;
    v0 = __builtin_fmaf(v0, s, p0);
    v1 = __builtin_fmaf(v1, s, p1);
  };
  stage(ISHZ_DPP(v0, 0xB1), ISHZ_DPP(v1, 0xB1), 1);                                    // quad_perm [1,0,3,2]
  stage(ISHZ_DPP(v0, 0x4E), ISHZ_DPP(v1, 0x4E), 2);                                    // quad_perm [2,3,0,1]
  stage(ISHZ_DPP(ISHZ_DPP(v0, 0x141), 0x1B), ISHZ_DPP(ISHZ_DPP(v1, 0x141), 0x1B), 4);    // half mirror, quad reverse
  stage(ISHZ_DPP(ISHZ_DPP(v0, 0x141), 0x140), ISHZ_DPP(ISHZ_DPP(v1, 0x141), 0x140), 8);  // half mirror, mirror
  auto swap = [&](float v, int m) {  // the value of lane ^ m, m = 16 or 32
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = m == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (lane & m) ? r[0] : r[1]);
  };
  stage(swap(v0, 16), swap(v1, 16), 16);
  stage(swap(v0, 32), swap(v1, 32), 32);
  const float r = 0.08838834764831845f;  // 1 / sqrt(128)
  v0 *= r;
  v1 *= r;
}

// Wide-step matvec / verify for the integer rates of 1, 2 and 4 bits: a wave's step is TN = 32/KA
// adjacent column tiles of one K tile (1 KB contiguous), fetched with one 128-bit load per lane
// and spread through LDS, so each wave keeps kilobytes in flight instead of the few hundred
// bytes that per-lane word loads give. Lanes decode as in exl3_mm2 (32-bit windows, pairwise
// codebook). The K tiles split over workgroups (blockIdx.y) and over a workgroup's waves; each K
// split stores its partial outputs into its own [M][N] slice of yh (summed later in split order).
//
// ROT: xh is the unrotated x and suh its input scales; each workgroup rotates the 128-point blocks
// that cover its K tiles, for every row, into LDS (after its first weight loads are issued) and
// reads x there, in place of a separate rotation launch.
template <int KA, int CB, bool MF, int D, bool ROT = false, int NTG = 1>
__global__ __launch_bounds__(256) void exl3_mm3(const uint16_t *__restrict__ xh, int M, int K,
                                               const uint32_t *__restrict__ trellis, int N,
                                               float *__restrict__ yh, int tk_per_wg,
                                               const uint16_t *__restrict__ suh = nullptr) {
  using TR = Trellis<KA, false>;
  using T32 = Trellis32<KA, false>;
  constexpr int TN = 32 / KA, W = TR::WORDS;  // TN tiles of W words = 256 words per step
  extern __shared__ __align__(16) float sm3[];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int tn0 = blockIdx.x * TN, tiles_n = N / 16, tiles_k = K / 16;
  const int tk0 = blockIdx.y * tk_per_wg, tk1 = min(tk0 + tk_per_wg, tiles_k);
  const typename T32::Win wn = T32::window(8 * (4 * (j & 7) + g) + 4 * (j >> 3));
  // HM (3INST / MCG, M <= 8): the dots on MFMA 16x16x32 with the weights' fp16 halves as k
  // entries. In MFMA i of tile quad q, lane group g decodes tile 4q + (g + i) % 4; A row 4 m + e
  // holds token m's x (each value twice, against a weight's two halves) when e = (g + i) % 4 and
  // is zero otherwise, so C row 4 m + e collects token m's dot with tile 4q + e alone: lane group
  // m ends with token m's sums for the quad's four tiles in its four C registers. Four tokens per
  // MFMA set, NTG sets for up to 4 NTG tokens, every set on the same decoded weights.
  constexpr bool HM = !MF && CB != 2;
  constexpr int NX = HM ? NTG : 1;  // x words per lane and step: one per token group
  int tok[NX];
#pragma unroll
  for (int t = 0; t < NX; t++) tok[t] = HM ? min((j >> 2) + 4 * t, M - 1) : MF ? (j < M ? j : 0) : 0;
  const bool live = MF ? j < M : true;
  const size_t tstride = (size_t)tiles_n * W;  // words between K tiles
  const uint32_t *base = trellis + (size_t)tn0 * W + 4 * lane;
  uint32_t *stage = (uint32_t *)sm3 + wave * 256;  // this wave's step
  float *red = sm3 + KS * 256;

  struct Raw {
    u4 w;
    uint32_t xa[NX], xb[NX];
  };
  const int nsteps = tk1 - tk0 > wave ? (tk1 - tk0 - wave + KS - 1) / KS : 0;
  auto load = [&](int i, Raw &r) {
    const int tk = tk0 + wave + KS * min(i, nsteps - 1);
    r.w = *(const u4 *)(base + tk * tstride);
    if constexpr (!ROT)
#pragma unroll
      for (int t = 0; t < NX; t++) {
        const uint16_t *xr = xh + (size_t)tok[t] * K + 2 * g + 16 * tk;
        r.xa[t] = *(const uint32_t *)xr;
        r.xb[t] = *(const uint32_t *)(xr + 8);
      }
  };
  using Acc = typename std::conditional<MF || HM, f4, float>::type;
  constexpr int NACC = HM ? NTG * TN / 4 : TN;  // HM: [token group][tile quad]
  Acc acc[NACC];
#pragma unroll
  for (int t = 0; t < NACC; t++) acc[t] = Acc{};
  Raw ring[D];
  if (nsteps > 0) {
#pragma unroll
    for (int d = 0; d < D - 1; d++) load(d, ring[d]);
  }
  // ROT: x of this workgroup's K range, rotated, at xl[k - kb0] (fp16, as the rotation kernel
  // rounds it); every wave takes whole 128-blocks
  // (row m at xl[m * XS + k - kb0], XS = tk_per_wg * 16 + 256 halves: the K range rounded out to
  // whole blocks); every wave takes whole (row, block) pairs
  const int kb0 = (tk0 * 16) & ~127, XS = tk_per_wg * 16 + 256;
  const uint16_t *xl = (const uint16_t *)(red + (MF ? TN * 256 : KS * TN * 16 * M));
  if constexpr (ROT) {
    uint16_t *xw = (uint16_t *)(red + (MF ? TN * 256 : KS * TN * 16 * M));
    const int nblk = (min((tk1 * 16 + 127) & ~127, K) - kb0) / 128;
    for (int q = wave; q < M * nblk; q += KS) {
      const int m = q / nblk, b = kb0 + 128 * (q % nblk);
      const int c = b + 2 * lane;
      const uint16_t *xm = xh + (size_t)m * K;
      float v0 = h2f(xm[c]) * h2f(suh[c]), v1 = h2f(xm[c + 1]) * h2f(suh[c + 1]);
      wht128_pair(v0, v1, lane);
      xw[m * XS + c - kb0] = f2h(v0);
      xw[m * XS + c - kb0 + 1] = f2h(v1);
    }
    __syncthreads();
  }
  for (int i0 = 0; i0 < nsteps; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const int i = i0 + d;
      if (i >= nsteps) break;
      load(i + D - 1, ring[(d + D - 1) % D]);
      Raw &r = ring[d];
      if constexpr (ROT)
#pragma unroll
        for (int t = 0; t < NX; t++) {
          const int xo = tok[t] * XS + 16 * (tk0 + wave + KS * i) - kb0 + 2 * g;
          r.xa[t] = *(const uint32_t *)(xl + xo);
          r.xb[t] = *(const uint32_t *)(xl + xo + 8);
        }
      *(u4 *)(stage + 4 * lane) = r.w;  // the wave's own buffer: its LDS operations stay in order
      if constexpr (HM) {
        // A of MFMA i, token group tg: the lane's token's x (rows of lane group g), each value
        // twice, on the lanes of rows 4 m + (g + i) % 4 of the group's live tokens m
        u4 A[NTG][4];
#pragma unroll
        for (int tg = 0; tg < NTG; tg++) {
          const u4 X = {dup_lo(r.xa[tg]), dup_hi(r.xa[tg]), dup_lo(r.xb[tg]), dup_hi(r.xb[tg])};
          const bool on_tok = (j >> 2) + 4 * tg < M;
#pragma unroll
          for (int i = 0; i < 4; i++) A[tg][i] = on_tok && (((j & 3) - g) & 3) == i ? X : u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int q = 0; q < TN / 4; q++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int t = 4 * q + ((g + i) & 3);
            const uint32_t win = __builtin_amdgcn_alignbit(stage[t * W + wn.ja], stage[t * W + wn.jb], wn.amt);
            const u4 B = {exl3_halves<CB>(__builtin_amdgcn_ubfe(win, T32::field(0), 16)),
                          exl3_halves<CB>(__builtin_amdgcn_ubfe(win, T32::field(1), 16)),
                          exl3_halves<CB>(__builtin_amdgcn_ubfe(win, T32::field(2), 16)),
                          exl3_halves<CB>(__builtin_amdgcn_ubfe(win, T32::field(3), 16))};
#pragma unroll
            for (int tg = 0; tg < NTG; tg++)
              acc[tg * (TN / 4) + q] = mfma32(as_h8(A[tg][i]), as_h8(B), acc[tg * (TN / 4) + q]);
          }
      } else {
#pragma unroll
        for (int t = 0; t < TN; t++) {
          const uint32_t win = __builtin_amdgcn_alignbit(stage[t * W + wn.ja], stage[t * W + wn.jb], wn.amt);
          const uint32_t s0 = __builtin_amdgcn_ubfe(win, T32::field(0), 16);
          const uint32_t s1 = __builtin_amdgcn_ubfe(win, T32::field(1), 16);
          const uint32_t s2 = __builtin_amdgcn_ubfe(win, T32::field(2), 16);
          const uint32_t s3 = __builtin_amdgcn_ubfe(win, T32::field(3), 16);
          const uint32_t b01 = exl3_decode2<CB>(s0, s1), b23 = exl3_decode2<CB>(s2, s3);
          if constexpr (MF) {
            const u2 A = live ? u2{r.xa[0], r.xb[0]} : u2{0, 0};
            acc[t] = mfma16(as_h4(A), as_h4(u2{b01, b23}), acc[t]);
          } else {
            acc[t] = dot2(b23, r.xb[0], dot2(b01, r.xa[0], acc[t]));
          }
        }
      }
    }
  }
  // partials: sum over the wave's lane groups (M = 1) and over the workgroup's waves in LDS, then
  // a store into this split's own [M][N] slice
  if constexpr (MF) {
    // the waves add their tiles into LDS one after another (fixed order, no atomics)
    for (int v = 0; v < KS; v++) {
      if (wave == v) {
#pragma unroll
        for (int t = 0; t < TN; t++)
#pragma unroll
          for (int q = 0; q < 4; q++) {
            float &r = red[(t * 4 + q) * 64 + lane];
            r = v == 0 ? acc[t][q] : r + acc[t][q];
          }
      }
      __syncthreads();
    }
    for (int o = threadIdx.x; o < TN * 256; o += blockDim.x) {
      const int t = o >> 8, q = (o >> 6) & 3, l = o & 63;
      const int tk = 4 * (l >> 4) + q;
      if (tk < M) {
        yh[(size_t)blockIdx.y * M * N + (size_t)tk * N + (tn0 + t) * 16 + (l & 15)] = red[o];
      }
    }
  } else {
    // red[wave][token][tile][column]
    if constexpr (HM) {
#pragma unroll
      for (int tg = 0; tg < NTG; tg++)
        if (g + 4 * tg < M)
#pragma unroll
          for (int q = 0; q < TN / 4; q++)
#pragma unroll
            for (int e = 0; e < 4; e++)
              red[((wave * M + g + 4 * tg) * TN + 4 * q + e) * 16 + j] = acc[tg * (TN / 4) + q][e];
    } else {  // M = 1
#pragma unroll
      for (int t = 0; t < NACC; t++) {
        float a = acc[t];
        a += lane_xor16(a);
        a += lane_xor32(a);
        if (g == 0) red[(wave * TN + t) * 16 + j] = a;
      }
    }
    __syncthreads();
    for (int o = threadIdx.x; o < M * TN * 16; o += blockDim.x) {
      const int m = o / (TN * 16), t = (o >> 4) % TN;
      float sum = 0.0f;
      for (int v = 0; v < KS; v++) sum += red[((v * M + m) * TN + t) * 16 + (o & 15)];
      yh[(size_t)blockIdx.y * M * N + (size_t)m * N + (tn0 + t) * 16 + (o & 15)] = sum;
    }
  }
}


// ------------------------------------------------------------------- dequantize
template <int KA, bool HALF>
__global__ __launch_bounds__(256) void exl3_dequant_kernel(const uint32_t *__restrict__ trellis,
                                                           int K, int N, int cb, void *out,
                                                           int dt) {
  using TR = Trellis<KA, HALF>;
  const size_t tile = blockIdx.x * 4 + wave_id();
  const int tiles_n = N / 16;
  if (tile >= (size_t)(K / 16) * tiles_n) return;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const u2 v = TR::decode4(trellis + tile * TR::WORDS, 8 * (4 * (j & 7) + g) + 4 * (j >> 3), cb);
  const size_t tk = tile / tiles_n, tn = tile % tiles_n;
  const uint16_t h[4] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y, (uint16_t)(v.y >> 16)};
  const int rows[4] = {2 * g, 2 * g + 1, 2 * g + 8, 2 * g + 9};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const size_t o = (tk * 16 + rows[i]) * (size_t)N + tn * 16 + j;
    const float f = h2f(h[i]);
    if (dt == ISHZ_DT_F32) ((float *)out)[o] = f;
    else if (dt == ISHZ_DT_F16) ((uint16_t *)out)[o] = h[i];
    else ((uint16_t *)out)[o] = (uint16_t)((__builtin_bit_cast(uint32_t, f) + 0x7fffu +
                                            ((__builtin_bit_cast(uint32_t, f) >> 16) & 1u)) >> 16);
  }
}

// ------------------------------------------------------------------- 128-point rotation
// EXL3Kernels.rotate (EXL3.swift:102-124): per 128 block, (x * s if before) -> WHT / sqrt(128)
// -> (* s if after), fp32, cast to the output dtype. One wave per block, two values per lane. An
// fp32 input may be nsum back-to-back slices summed first (the matvec's K-split partials).
__global__ __launch_bounds__(256) void exl3_rotate_kernel(const void *__restrict__ x, int in_dt,
                                                          size_t blocks, int width,
                                                          const uint16_t *__restrict__ scales,
                                                          int before, void *__restrict__ y,
                                                          int out_dt, int nsum, const float *__restrict__ rs) {
  const size_t blk = (size_t)blockIdx.x * 4 + wave_id();
  if (blk >= blocks) return;
  const int lane = threadIdx.x & 63;
  const size_t base = blk * 128 + 2 * lane;
  const int col = (int)((blk * 128) % width) + 2 * lane;
  const float s0 = h2f(scales[col]), s1 = h2f(scales[col + 1]);  // issued first: independent
  float v0, v1;
  if (in_dt == ISHZ_DT_F32) {  // fp32 input: the sum of nsum slices (K-split partials), in order
    const size_t slice = blocks * 128;
    const float *xf = (const float *)x + base;
    v0 = 0.0f;
    v1 = 0.0f;
    for (int q0 = 0; q0 < nsum; q0 += 16) {  // sixteen slices' loads in flight, summed in order
      float2 p[16];
#pragma unroll
      for (int i = 0; i < 16; i++) p[i] = q0 + i < nsum ? *(const float2 *)(xf + (q0 + i) * slice) : float2{0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 16; i++) {
        v0 += p[i].x;
        v1 += p[i].y;
      }
    }
  } else {
    v0 = load_act(x, base, in_dt);
    v1 = load_act(x, base + 1, in_dt);
  }
  if (before) {
    v0 *= s0;
    v1 *= s1;
  }
  wht128_pair(v0, v1, lane);
  if (!before) {
    v0 *= s0;
    v1 *= s1;
  }
  if (rs) {  // outputs of a rescaled activation image: its row's factor back
    const float f = rs[(blk * 128) / width];
    v0 *= f;
    v1 *= f;
  }
  store_act(y, base, out_dt, v0);
  store_act(y, base + 1, out_dt, v1);
}

// y[m][n] = the S K-split parts summed in split order, times rs[m] when the activations were
// rescaled into their fp16 image (rs null: not).
__global__ __launch_bounds__(256) void exl3_sum_parts_kernel(const float *__restrict__ part, int S, size_t n, int N,
                                                             const float *__restrict__ rs, float *__restrict__ y) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int k = 0; k < S; k++) s += part[(size_t)k * n + i];
    y[i] = rs ? s * rs[i / N] : s;
  }
}

// ------------------------------------------------------------------- host
static int num_cu_e() {
  static int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      return v;
    return 256;
  }();
  return n;
}

// Calls F.template operator()<KA, HALF>() for a rate given as bits2 = 2 * bits.
template <class F>
static int by_rate(int bits2, F &&f) {
  switch (bits2) {
  case 2: return f.template operator()<1, false>();
  case 3: return f.template operator()<1, true>();
  case 4: return f.template operator()<2, false>();
  case 5: return f.template operator()<2, true>();
  case 6: return f.template operator()<3, false>();
  case 7: return f.template operator()<3, true>();
  case 8: return f.template operator()<4, false>();
  case 10: return f.template operator()<5, false>();
  case 12: return f.template operator()<6, false>();
  case 14: return f.template operator()<7, false>();
  case 16: return f.template operator()<8, false>();
  }
  return decline("EXL3 rate is not one of 1, 1.5, 2, 2.5, 3, 3.5, 4..8 bits");
}

// EXL3Tensor.init validation (EXL3.swift:29-55).
static int check_exl3(int K, int N, int bits2, int cb) {
  if (cb < 0 || cb > 2) return decline("unknown EXL3 codebook");
  if ((bits2 & 1) && cb != 2) return decline("half-integer EXL3 rates need the mul1 codebook");
  if (K <= 0 || N <= 0 || K % 128 || N % 128) return decline("EXL3 K and N must be multiples of 128");
  return ISHZ_OK;
}

}  // namespace ishz

using namespace ishz;

extern "C" int ishz_exl3_dequant(const int16_t *trellis, int K, int N, int bits2, int codebook,
                                 void *out, int out_dtype, ishz_stream_t stream) {
  if (codebook < 0 || codebook > 2 || ((bits2 & 1) && codebook != 2)) return decline("bad codebook/rate");
  if (K <= 0 || N <= 0 || K % 16 || N % 16) return decline("EXL3 K and N must be multiples of 16");
  if (out_dtype < ISHZ_DT_F32 || out_dtype > ISHZ_DT_BF16) return decline("unsupported output dtype");
  if (!trellis || !out) return einval("null pointer");
  const size_t tiles = (size_t)(K / 16) * (N / 16);
  return by_rate(bits2, [&]<int KA, bool HALF>() -> int {
    hipLaunchKernelGGL((exl3_dequant_kernel<KA, HALF>), dim3((unsigned)((tiles + 3) / 4)), dim3(256), 0,
                       S(stream), (const uint32_t *)trellis, K, N, codebook, out, out_dtype);
    ISHZ_LAUNCH_CHECK("exl3 dequant launch");
    return ISHZ_OK;
  });
}

extern "C" int ishz_exl3_rotate(const void *x, int in_dtype, int rows, int width,
                                const uint16_t *scales, int before, void *y, int out_dtype,
                                ishz_stream_t stream) {
  if (in_dtype < ISHZ_DT_F32 || in_dtype > ISHZ_DT_BF16 || out_dtype < ISHZ_DT_F32 || out_dtype > ISHZ_DT_BF16)
    return decline("rotation takes fp32, fp16 or bf16");
  if (rows <= 0 || width <= 0 || width % 128) return einval("width must be a multiple of 128");
  if (!x || !y || !scales) return einval("null pointer");
  const size_t blocks = (size_t)rows * (width / 128);
  hipLaunchKernelGGL(exl3_rotate_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, S(stream), x,
                     in_dtype, blocks, width, scales, before, y, out_dtype, 1, nullptr);
  ISHZ_LAUNCH_CHECK("exl3 rotate launch");
  return ISHZ_OK;
}

// K splits of the wide-step kernel: about four workgroups per CU up to eight rows (the
// halves-on-MFMA kernel; at 17408 x 5120, 2 bpw, M = 2: 25.1 -> 23.9 us against two), two for the
// decoded-weight MFMA kernel (tn_blocks workgroups per split), at most 64.
static int exl3_splits(int M, int K, int tn_blocks);
// Floats the matvec's K-split parts take at most: the split count of the fewest column blocks (32
// tiles per step at 1 bit) times M N.
static size_t exl3_part_floats(int M, int K, int N) {
  return (size_t)std::max(1, exl3_splits(M, K, std::max(1, N / 16 / 32))) * M * N;
}
static int exl3_splits(int M, int K, int tn_blocks) {
  const int tiles_k = K / 16;
  return std::max(1, std::min({tiles_k / 4, (M <= 8 ? 4 : 2) * num_cu_e() / tn_blocks, 64}));
}

// The matvec into `part` (exl3_part_floats(M, K, N) floats): the wide-step kernel writes each K
// split's partial product to its own [M][N] slice and *nparts says how many; the other kernels
// write the whole product to the first slice and *nparts = 1.
// With `suh` (exl3_fused_rotation(..) true) xh is the unrotated x and the wide-step kernel
// rotates it itself.
static int exl3_matvec_core(const void *xh, int M, int K, const int16_t *trellis, int N, int bits2, int codebook,
                            float *part, int *nparts, hipStream_t st, const uint16_t *suh = nullptr) {
  *nparts = 1;
  const int wgs = N / 16, tiles_k = K / 16;
  int ks = 1;
  while (ks < 16 && ks < tiles_k && wgs * ks < num_cu_e() * 16) ks *= 2;
  return by_rate(bits2, [&]<int KA, bool HALF>() -> int {
    if constexpr (!HALF && (KA == 1 || KA == 2 || KA == 4)) {
      constexpr int TN = 32 / KA, KS3 = 4, D = 4;  // a step covers TN column tiles: N must tile by them
      constexpr int D1 = 3;  // ring depth at M = 1 (MFMA dots): 23.7 -> 23.1 us at 5120 -> 17408, 2 bpw
      if ((N / 16) % TN == 0) {
        const int tn_blocks = N / 16 / TN;
        const int per = (tiles_k + exl3_splits(M, K, tn_blocks) - 1) / exl3_splits(M, K, tn_blocks);
        const int nsplit = (tiles_k + per - 1) / per;
        float *out = part;
        *nparts = nsplit;
        auto go = [&]<int CB>() -> int {
          // the halves-on-MFMA kernel for the 3INST / MCG codebooks up to 8 rows, the dot2 kernel
          // for MUL1 at M = 1, the decoded-weight MFMA kernel otherwise
          const bool hm = (CB != 2 && M <= 8) || M == 1;
          const size_t lds = (size_t)KS3 * 256 * 4 + (hm ? (size_t)KS3 * TN * 16 * 4 * M : (size_t)TN * 256 * 4) +
                             (suh ? (size_t)M * (per * 16 + 256) * 2 : 0);  // ROT: the rotated K range of x
          if (hm && M > 4 && suh)
            hipLaunchKernelGGL((exl3_mm3<KA, CB, false, D1, true, 2>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per, suh);
          else if (hm && M > 4)
            hipLaunchKernelGGL((exl3_mm3<KA, CB, false, D1, false, 2>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per);
          else if (hm && suh)
            hipLaunchKernelGGL((exl3_mm3<KA, CB, false, D1, true>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per, suh);
          else if (hm)
            hipLaunchKernelGGL((exl3_mm3<KA, CB, false, D1>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per);
          else if (suh)
            hipLaunchKernelGGL((exl3_mm3<KA, CB, true, D, true>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per, suh);
          else
            hipLaunchKernelGGL((exl3_mm3<KA, CB, true, D>), dim3(tn_blocks, nsplit), dim3(64 * KS3), lds, st,
                               (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, out, per);
          ISHZ_LAUNCH_CHECK("exl3 matvec launch");
          return ISHZ_OK;
        };
        return codebook == 0 ? go.template operator()<0>()
                             : codebook == 1 ? go.template operator()<1>() : go.template operator()<2>();
      }
    }
    if (suh) return einval("the fused input rotation needs the wide-step kernel");
    if constexpr (Trellis32<KA, HALF>::FITS) {
      {
        // TN = 4 column tiles per workgroup (N % 128 == 0 makes N / 16 a multiple of 8); 4 waves
        // split the K tiles, each with a 4-deep prefetch ring.
        constexpr int TN = 4, KS2 = 4;
        const size_t lds = M == 1 ? (size_t)KS2 * TN * 16 * 4 : (size_t)KS2 * TN * 256 * 4;
        auto go = [&]<int CB>() -> int {
          auto launch = [&]<int D>() {
            if (M == 1)
              hipLaunchKernelGGL((exl3_mm2<KA, HALF, CB, false, TN, D>), dim3(N / 16 / TN), dim3(64 * KS2), lds,
                                 st, (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, part);
            else
              hipLaunchKernelGGL((exl3_mm2<KA, HALF, CB, true, TN, D>), dim3(N / 16 / TN), dim3(64 * KS2), lds,
                                 st, (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, part);
          };
          launch.template operator()<4>();
          ISHZ_LAUNCH_CHECK("exl3 matvec launch");
          return ISHZ_OK;
        };
        return codebook == 0 ? go.template operator()<0>()
                             : codebook == 1 ? go.template operator()<1>() : go.template operator()<2>();
      }
    }
    if (M == 1)
      hipLaunchKernelGGL((exl3_mm<KA, HALF, false>), dim3(wgs), dim3(64 * ks), (size_t)ks * 16 * 4,
                         st, (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, codebook, part);
    else
      hipLaunchKernelGGL((exl3_mm<KA, HALF, true>), dim3(wgs), dim3(64 * ks), (size_t)ks * 256 * 4,
                         st, (const uint16_t *)xh, M, K, (const uint32_t *)trellis, N, codebook, part);
    ISHZ_LAUNCH_CHECK("exl3 matvec launch");
    return ISHZ_OK;
  });
}

// y [M][N] fp32 from fp32 x (one slice, no K split).
static int exl3_matvec_f32(const float *x, int M, int K, const int16_t *trellis, int N, int bits2, int cb,
                           float *yh, hipStream_t st) {
  return by_rate(bits2, [&]<int KA, bool HALF>() -> int {
    hipLaunchKernelGGL((exl3_mm_f32<KA, HALF>), dim3(N / 16), dim3(256), 0, st, x, M, K, (const uint32_t *)trellis,
                       N, cb, yh);
    ISHZ_LAUNCH_CHECK("exl3 fp32 matvec launch");
    return ISHZ_OK;
  });
}

// The matvec's device temporaries: the fp16 image of bf16 activations, then the K splits'
// fp32 partial products.
extern "C" size_t ishz_exl3_matvec_workspace_size(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  return act_image_bytes(M, K) + exl3_part_floats(M, K, N) * 4;
}

extern "C" int ishz_exl3_matvec_ws(const void *xh, int x_dtype, int M, int K, const int16_t *trellis, int N,
                                   int bits2, int codebook, float *yh, void *workspace, size_t workspace_bytes,
                                   ishz_stream_t stream) {
  int rc = check_exl3(K, N, bits2, codebook);
  if (rc) return rc;
  if (x_dtype < ISHZ_DT_F32 || x_dtype > ISHZ_DT_BF16) return decline("activations must be fp16, bf16 or fp32");
  if (M < 1 || M > 16) return decline("row count outside 1..16");
  if (!xh || !trellis || !yh) return einval("null pointer");
  hipStream_t st = S(stream);
  if (x_dtype == ISHZ_DT_F32) return exl3_matvec_f32((const float *)xh, M, K, trellis, N, bits2, codebook, yh, st);
  // with a workspace of ishz_exl3_matvec_workspace_size bytes nothing is allocated; without one
  // (ishz_exl3_matvec) the image and the parts are stream-ordered temporaries
  const bool own = workspace && workspace_bytes >= ishz_exl3_matvec_workspace_size(M, K, N);
  if (workspace && !own) return einval("workspace too small (ishz_exl3_matvec_workspace_size)");
  StreamTemp tmp(st), parts(st);
  void *img = own ? workspace : nullptr;
  float *pp = own ? (float *)((char *)workspace + act_image_bytes(M, K)) : nullptr;
  if (!own) {
    if (x_dtype != ISHZ_DT_F16 && (rc = tmp.get(act_image_bytes(M, K)))) return rc;
    if ((rc = parts.get(exl3_part_floats(M, K, N) * 4))) return rc;
    img = tmp.p;
    pp = (float *)parts.p;
  }
  const uint16_t *x16;
  const float *rs;
  if ((rc = act_prepare(xh, x_dtype, M, K, img, st, &x16, &rs))) return rc;
  // the K splits' partial products, then their sum in split order: the same bits on every call
  int np;
  if ((rc = exl3_matvec_core(x16, M, K, trellis, N, bits2, codebook, pp, &np, st))) return rc;
  const size_t n = (size_t)M * N;
  hipLaunchKernelGGL(exl3_sum_parts_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)), dim3(256), 0, st,
                     pp, np, n, N, rs, yh);
  ISHZ_LAUNCH_CHECK("exl3 sum launch");
  return ISHZ_OK;
}

extern "C" int ishz_exl3_matvec(const void *xh, int x_dtype, int M, int K, const int16_t *trellis,
                                int N, int bits2, int codebook, float *yh, ishz_stream_t stream) {
  return ishz_exl3_matvec_ws(xh, x_dtype, M, K, trellis, N, bits2, codebook, yh, nullptr, 0, stream);
}

// Whether exl3_matvec_core takes the wide-step kernel, which can rotate x itself, and the
// workgroup's rotated slice of x fits beside the kernel's own LDS. One row only: with 8 rows each
// workgroup rotates ~8x the blocks before its first MFMA, which measured slower (17408x5120 at
// 2 bpw: 37.8 us against 34.7 us for the separate rotation launch).
static bool exl3_fused_rotation(int M, int K, int N, int bits2) {
  const int KA = bits2 / 2;
  // up to two rows: every workgroup rotates its K range of every row, which measured faster than
  // the separate rotation launch at M = 1 and 2 (17408x5120: 32.7 vs 33.7 us at M = 2), even at 4
  // and slower at 8 (38.0 vs 35.3); with the halves-on-MFMA kernel, even at 4 (27.5-27.7 vs
  // 27.8) and slower at 8 (34.6-34.8 vs 33.5-33.7)
  if (M > 2 || !(bits2 == 2 || bits2 == 4 || bits2 == 8) || (N / 16) % (32 / KA)) return false;
  const int TN = 32 / KA, tiles_k = K / 16, splits = exl3_splits(M, K, N / 16 / TN);
  const size_t per = (tiles_k + splits - 1) / splits;
  const size_t own = 4 * 256 * 4 + std::max((size_t)4 * TN * 16 * 4 * M, (size_t)TN * 256 * 4);
  return own + (size_t)M * (per * 16 + 256) * 2 <= 120 * 1024;
}

// x rotated (in x's dtype, up to 4 bytes a value), the fp16 image of bf16 / fp32 rotated
// activations, then the matvec's K-split partials (fp32 [splits][M][N], splits bounded by the
// widest column step of any rate, 32 tiles).
static size_t exl3_rot_bytes(int M, int K) { return ((size_t)M * K * 4 + 255) / 256 * 256; }
extern "C" size_t ishz_exl3_workspace_size(int M, int K, int N) {
  return exl3_rot_bytes(M, K) + act_image_bytes(M, K) + exl3_part_floats(M, K, N) * 4;
}

// Device scratch of ishz_exl3_apply_static: every GPU the library runs on holds its own copy
// until the process ends. Host code never passes `scratch` itself (its host-side name is not a
// device address): the per-device address from hipGetSymbolAddress is used instead.
static __device__ __align__(256) uint8_t scratch[ISHZ_EXL3_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag scratch_once[kMaxDevices];
void *scratch_ptr[kMaxDevices];
hipError_t scratch_err[kMaxDevices];
}  // namespace

// This device's scratch address, looked up once per device with that device current.
static int exl3_scratch(hipStream_t st, void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail("hipGetDevice", e);
  if (st) {
    int sdev = -1;
    if ((e = hipStreamGetDevice(st, &sdev)) != hipSuccess) return fail("hipStreamGetDevice", e);
    if (sdev != dev) return einval("the stream belongs to another device than the current one");
  }
  if (dev < 0 || dev >= kMaxDevices) return einval("device index beyond the scratch table");
  std::call_once(scratch_once[dev], [dev] {
    scratch_err[dev] = hipGetSymbolAddress(&scratch_ptr[dev], HIP_SYMBOL(scratch));
  });
  if (scratch_err[dev] != hipSuccess) return fail("hipGetSymbolAddress(scratch)", scratch_err[dev]);
  *out = scratch_ptr[dev];
  return ISHZ_OK;
}

extern "C" int ishz_exl3_apply(const void *x, int x_dtype, int M, int K, const int16_t *trellis,
                               const uint16_t *suh, const uint16_t *svh, int N, int bits2,
                               int codebook, void *y, void *workspace, size_t workspace_bytes,
                               ishz_stream_t stream) {
  int rc = check_exl3(K, N, bits2, codebook);
  if (rc) return rc;
  if (x_dtype < ISHZ_DT_F32 || x_dtype > ISHZ_DT_BF16) return decline("activations must be fp16, bf16 or fp32");
  if (M < 1 || M > 16) return decline("row count outside 1..16");
  if (!x || !trellis || !suh || !svh || !y) return einval("null pointer");
  if (!workspace || workspace_bytes < ishz_exl3_workspace_size(M, K, N))
    return einval("workspace too small (ishz_exl3_workspace_size)");
  hipStream_t st = S(stream);
  uint8_t *xr = (uint8_t *)workspace, *img = xr + exl3_rot_bytes(M, K);
  float *yh = (float *)(img + act_image_bytes(M, K));
  int np = 1;
  const float *rs = nullptr;
  if (x_dtype == ISHZ_DT_F16 && exl3_fused_rotation(M, K, N, bits2)) {  // the matvec rotates its own K range of x
    if ((rc = exl3_matvec_core(x, M, K, trellis, N, bits2, codebook, yh, &np, st, suh))) return rc;
  } else {
    // rotated into x's dtype (EXL3Kernels.apply rotates `to: x.dtype`, Core/EXL3.swift:85), then
    // (bf16 / fp32) its fp16 image
    if ((rc = ishz_exl3_rotate(x, x_dtype, M, K, suh, 1, xr, x_dtype, stream))) return rc;
    if (x_dtype == ISHZ_DT_F32) {  // fp32 precision: exact weights, fp32 FMAs
      if ((rc = exl3_matvec_f32((const float *)xr, M, K, trellis, N, bits2, codebook, yh, st))) return rc;
    } else {
      const uint16_t *x16;
      if ((rc = act_prepare(xr, x_dtype, M, K, img, st, &x16, &rs))) return rc;
      if ((rc = exl3_matvec_core(x16, M, K, trellis, N, bits2, codebook, yh, &np, st))) return rc;
    }
  }
  const size_t blocks = (size_t)M * (N / 128);  // output rotation, summing the K-split partials
  hipLaunchKernelGGL(exl3_rotate_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, st, yh,
                     ISHZ_DT_F32, blocks, N, svh, 0, y, x_dtype, np, rs);
  ISHZ_LAUNCH_CHECK("exl3 rotate launch");
  return ISHZ_OK;
}

// ishz_exl3_apply with the library's own device scratch in place of a caller workspace: no
// allocation of any kind. Calls that overlap on one GPU share the scratch and race.
extern "C" int ishz_exl3_apply_static(const void *x, int x_dtype, int M, int K, const int16_t *trellis,
                                      const uint16_t *suh, const uint16_t *svh, int N, int bits2, int codebook,
                                      void *y, ishz_stream_t stream) {
  int rc = check_exl3(K, N, bits2, codebook);
  if (rc) return rc;
  if (x_dtype < ISHZ_DT_F32 || x_dtype > ISHZ_DT_BF16) return decline("activations must be fp16, bf16 or fp32");
  if (M < 1 || M > 16) return decline("row count outside 1..16");
  const size_t need = ishz_exl3_workspace_size(M, K, N);
  if (need > ISHZ_EXL3_STATIC_SCRATCH_BYTES)
    return einval("M x K x N needs " + std::to_string(need) + " bytes of scratch, above the static " +
                  std::to_string((size_t)ISHZ_EXL3_STATIC_SCRATCH_BYTES) + " (use ishz_exl3_apply)");
  void *ws = nullptr;
  if ((rc = exl3_scratch(S(stream), &ws))) return rc;
  return ishz_exl3_apply(x, x_dtype, M, K, trellis, suh, svh, N, bits2, codebook, y, ws, need, stream);
}
