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
// A workgroup (NW waves) owns a run of tiles; its waves share the tiles' steps and sum their
// partials in LDS. x is staged in LDS per K chunk, in A-operand order:
// token image [step][g][mfma] of 16-byte words, plus per (step, g, sub-unit) the sums the
// epilogue needs for every token (1024 * sum of the staged A values, the magic-number offset;
// and the plain sum of x).
//
// A format F provides:
//   VNS                              sub-units per quarter
//   VRaw vload(row, j, g)            the quarter's codes and the row's step header (or
//   VRaw vload_p(p, group, row, kc0, j, g)   for packs held in several arrays)
//   void vdecode(r, B[8], tabs)      B operands (MFMA b of sub-unit b / (8 / VNS))
//   void vstage(xrow, j, g, s, A, off1, X)   A words of sub-unit s (8 / VNS of them) and sums
//   void vscale(r, g, s, sc, mn)     value of sub-unit s = sc * (C - off1) + mn * X
//   vtables(tabs), tab_bytes()       LDS tables the decoder reads (codebooks, sign masks)
//   VDEPTH                           steps kept in flight (register ring)
//   VPLAIN (optional, true)          off1 and mn are always zero: value = sc * C, so the epilogue
//                                    reads no sums
//   voff() (optional)                off1 is always voff() * X: the epilogue reads X only
//   vkappa(s) (optional, with voff)  mn is always vkappa(s) * sc: staging stores the sub-unit's
//                                    (vkappa - voff) X as the MFMA chain's initial C, and the
//                                    epilogue is sc * C alone
#pragma once
#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace ishz {

template <class F>
__host__ __device__ constexpr bool vgemm_plain() {
  if constexpr (requires { F::VPLAIN; }) return F::VPLAIN;
  else return false;
}
template <class F>
__host__ __device__ constexpr bool vgemm_kappa() {
  return requires { F::vkappa(0); };
}

// What is multiplied: a "problem" P supplies, per workgroup row blockIdx.y (a group: the whole
// matrix, or one routed expert), the token rows of x, the weight rows, and the output writer.
//   bool group(gy, Group &)      false: nothing to do (an expert slot past the active count)
//   int count(g), rows(g)         tokens (any number; 16 per pass) and weight rows of the group
//   const uint16_t *xrow(g, tk)   token tk's activations (K of them)
//   const uint8_t *wrow(g, row)   weight row (row < rows(g))
//   void finish(g, c0, M, tb, te, out)   write tokens c0 .. c0 + M - 1 of tiles tb .. te - 1;
//                                 out[(tile - tb) * 256 + tk * 16 + n] is row 16 tile + n
//   PAIRS                         tiles_per_wg must be even and start even (SwiGLU pairs)
//   optional: void prologue() run by every thread of every workgroup before group() (ends with a
//   barrier), with static size_t extra_lds(p) bytes of its own LDS at byte offset p.lds_off
// Work split: a workgroup owns tiles tb .. te - 1 of its group and, with S > 1 (K split: the
// problem's finish then writes fp32 partials), the S-th part blockIdx.x % S of the K steps; the
// (tile, step) items go to its waves round-robin (item i to wave i % NW), so short K still uses
// every wave.
template <class F, class P, int NQ, int D, int NW>
__global__ __launch_bounds__(64 * NW) void vgemm_kernel(P p, int K, int Kc, int tiles_per_wg, int S) {
  constexpr int NS = F::VNS, MPS = 8 / NS;  // MFMAs per sub-unit
  constexpr int MT = 4 * NQ;                // tokens per pass, padded to whole quads
  typedef typename P::Group Group;
  Group gp;
  extern __shared__ __align__(16) u4 vgsm[];
  if constexpr (requires { p.prologue(); }) p.prologue();  // every thread; ends with a barrier
  if (!p.group(blockIdx.y, gp)) return;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int n = lane & 15, G = lane >> 4;
  const int N = p.rows(gp), ntiles = (N + 15) / 16;
  const int tb = (blockIdx.x / S) * tiles_per_wg, te = min(tb + tiles_per_wg, ntiles);
  if (tb >= te) return;
  const int split = blockIdx.x % S, ksteps = K / 256;
  const int kb = split * ksteps / S * 256, ke = (split + 1) * ksteps / S * 256;  // this part of K
  const int ntl = te - tb;
  const int cs = Kc / 256;                    // steps per chunk
  const int IW = cs * 32 + 1;                 // token image stride (16-byte words, padded)
  u4 *zero = vgsm + MT * IW;                  // 8 words of zeros (non-diagonal A)
  float *sums = (float *)(zero + 8);          // [cs][4][NS][2][MT]
  const bool whole = tiles_per_wg >= NW;      // waves take whole tiles (else they split steps)
  float *accb = sums + cs * 4 * NS * 2 * MT;  // [wave][tile][quad][4][16], split mode only
  float *outb = accb + (whole ? 0 : NW * tiles_per_wg * NQ * 64);  // [tile][16 tokens][16 rows]
  u4 *tabs = (u4 *)(outb + tiles_per_wg * 256);
  const uint32_t mg = vconst(0x64006400u);

  for (int i = threadIdx.x; i < 8; i += blockDim.x) zero[i] = u4{0, 0, 0, 0};
  F::vtables(tabs);
  // A row of this lane: gg = n / 4 (lane group whose k-slot it fills), token tt = n % 4.
  const int gg = n >> 2, tt = n & 3;
  const int count = p.count(gp);

  for (int c0 = 0; c0 < count; c0 += MT) {
    const int M = min(MT, count - c0);
    if (whole)
      for (int i = threadIdx.x; i < ntl * 256; i += blockDim.x) outb[i] = 0.0f;
    else
      for (int i = threadIdx.x; i < NW * tiles_per_wg * NQ * 64; i += blockDim.x) accb[i] = 0.0f;
    for (int kc0 = kb; kc0 < ke; kc0 += Kc) {
      const int steps = min(Kc, ke - kc0) / 256;
      // ---- stage every token's x for this chunk
      for (int it = threadIdx.x; it < MT * steps * 4 * NS; it += blockDim.x) {
        const int s = it % NS, g = (it / NS) % 4, j = (it / (NS * 4)) % steps, tk = it / (NS * 4 * steps);
        float off1 = 0.0f, X = 0.0f;
        if (tk < M) {
          u4 A[MPS];
          F::vstage(p.xrow(gp, c0 + tk) + kc0, j, g, s, A, off1, X);
          u4 *dst = vgsm + tk * IW + (j * 4 + g) * 8 + s * MPS;
#pragma unroll
          for (int b = 0; b < MPS; b++) dst[b] = A[b];
        }
        float *sp = sums + (((j * 4 + g) * NS + s) * 2) * MT;
        if constexpr (vgemm_kappa<F>()) sp[tk] = F::vkappa(s) * X - off1;  // the chain's initial C
        else sp[tk] = off1;
        sp[MT + tk] = X;
      }
      __syncthreads();

      // ---- stream this wave's items (tile, step). With at least NW tiles per workgroup each wave
      // takes whole tiles (tiles wave, wave + NW, ...; partials go straight to outb); with fewer,
      // the tiles' steps are dealt round-robin (item i to wave i % NW; partials meet in accb).
      typedef typename F::VRaw Raw;
      const int items = ntl * steps;
      const int cnt = whole ? (ntl > wave ? (ntl - wave + NW - 1) / NW : 0) * steps
                            : (items > wave ? (items - wave + NW - 1) / NW : 0);
      // Item cursors (tile tl, step j): item k is tile wave + NW (k / steps), step k % steps
      // (whole tiles), or item wave + NW k of the workgroup's (tile, step) sequence (dealt steps).
      // They advance without dividing: a division by the runtime step count for every load,
      // consume and park test was most of the loop's scalar instructions.
      struct Cur {
        int tl, j;
      };
      auto next = [&](Cur c) {
        if (whole) {
          if (++c.j == steps) {
            c.j = 0;
            c.tl += NW;
          }
        } else {
          c.j += NW;
          while (c.j >= steps) {
            c.j -= steps;
            c.tl++;
          }
        }
        return c;
      };
      const Cur c0 = whole ? Cur{wave, 0} : Cur{wave / steps, wave % steps};
      auto load = [&](const Cur &c, Raw &r) {
        const int row = min((tb + c.tl) * 16 + n, N - 1);
        if constexpr (requires { F::vload_p(p, gp, row, kc0, c.j, G); })
          r = F::vload_p(p, gp, row, kc0, c.j, G);  // formats whose rows are not one byte run
        else
          r = F::vload(p.wrow(gp, row) + (size_t)(kc0 / 256) * F::VSTEP_BYTES, c.j, G);
      };
      // the load cursor runs D - 1 items ahead and stops at the wave's last item (loads past the
      // end re-read it and are dropped)
      Cur lc = c0, cc = c0;
      int lk = 0;
      auto load_next = [&](Raw &r) {
        load(lc, r);
        if (lk < cnt - 1) {
          lc = next(lc);
          lk++;
        }
      };
      Raw ring[D];
      if (cnt > 0) {
#pragma unroll
        for (int d = 0; d < D - 1; d++) load_next(ring[d]);
      }
      f4 acc[NQ];
#pragma unroll
      for (int q = 0; q < NQ; q++) acc[q] = f4{0, 0, 0, 0};
      for (int k0 = 0; k0 < cnt; k0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
          const int k = k0 + d;
          if (k >= cnt) break;
          load_next(ring[(d + D - 1) % D]);
          const int tl = cc.tl, j = cc.j;
          const Raw &r = ring[d];
          u4 B[8];
          F::vdecode(r, B, mg, tabs, tabs + 512);
          float sc[NS], mn[NS];
#pragma unroll
          for (int s = 0; s < NS; s++) F::vscale(r, G, s, sc[s], mn[s]);
#pragma unroll
          for (int q = 0; q < NQ; q++) {
            if (4 * q >= M) break;
            const int tka = 4 * q + tt;
            const u4 *ab = (gg == G && tka < M) ? vgsm + tka * IW + (j * 4 + G) * 8 : zero;
#pragma unroll
            for (int s = 0; s < NS; s++) {
              f4 C = f4{0, 0, 0, 0};
              if constexpr (vgemm_kappa<F>())  // (vkappa - voff) X: sc C is then the sub-unit's value
                C = *(const f4 *)(sums + (((j * 4 + G) * NS + s) * 2) * MT + 4 * q);
#pragma unroll
              for (int b = 0; b < MPS; b++) C = mfma32(as_h8(ab[s * MPS + b]), as_h8(B[s * MPS + b]), C);
              if constexpr (vgemm_plain<F>() || vgemm_kappa<F>()) {
#pragma unroll
                for (int e = 0; e < 4; e++) acc[q][e] = fmaf(sc[s], C[e], acc[q][e]);
              } else if constexpr (requires { F::voff(); }) {
                // off1 = voff X: sc (C - voff X) + mn X = sc C + (mn - voff sc) X, one sum read
                const f4 X = *(const f4 *)(sums + (((j * 4 + G) * NS + s) * 2 + 1) * MT + 4 * q);
                const float cx = mn[s] - F::voff() * sc[s];
#pragma unroll
                for (int e = 0; e < 4; e++) acc[q][e] = fmaf(sc[s], C[e], fmaf(cx, X[e], acc[q][e]));
              } else {
                const float *sp = sums + (((j * 4 + G) * NS + s) * 2) * MT + 4 * q;
                const f4 off = *(const f4 *)sp, X = *(const f4 *)(sp + MT);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[q][e] += sc[s] * (C[e] - off[e]) + mn[s] * X[e];
              }
            }
          }
          // park at the wave's last item of a tile: sum the row's four lane-group quarters
          cc = next(cc);
          if (k + 1 == cnt || cc.tl != tl) {
#pragma unroll
            for (int q = 0; q < NQ; q++) {
              if (4 * q >= M) break;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                float a = acc[q][e];
                a += lane_xor16(a);
                a += lane_xor32(a);
                if (G == 0) {
                  if (whole) outb[tl * 256 + (4 * q + e) * 16 + n] += a;
                  else accb[(((wave * tiles_per_wg + tl) * NQ + q) * 4 + e) * 16 + n] += a;
                }
                acc[q][e] = 0.0f;
              }
            }
          }
        }
      }
      __syncthreads();  // partials parked; the x image is free for the next chunk
    }
    if (!whole) {  // sum the waves' partials
      for (int o = threadIdx.x; o < ntl * 256; o += blockDim.x) {
        const int tl = o >> 8, tk = (o >> 4) & 15, nn = o & 15;
        float sm = 0.0f;
        if (tk < MT)
          for (int v = 0; v < NW; v++) sm += accb[(((v * tiles_per_wg + tl) * NQ + (tk >> 2)) * 4 + (tk & 3)) * 16 + nn];
        outb[o] = sm;
      }
      __syncthreads();
    }
    p.finish(gp, c0, M, tb, te, outb);
    __syncthreads();
  }
}

int gemv_num_cu();

template <class F, int NQ, int NW>
static size_t vgemm_lds(int Kc, int T) {
  constexpr int MT = 4 * NQ;
  const int cs = Kc / 256;
  return (size_t)MT * (cs * 32 + 1) * 16 + 8 * 16 + (size_t)cs * 4 * F::VNS * 2 * MT * 4 +
         (T >= NW ? 0 : (size_t)NW * T * NQ * 64 * 4) + (size_t)T * 256 * 4 + F::tab_bytes();
}

// Launch over `groups` groups of (up to) `rows` weight rows each; T tiles per workgroup, K in S parts.
template <class F, class P, int NQ>
static int launch_vgemm_p(const P &p, int K, int rows, int groups, int T, hipStream_t st, int S = 1) {
  constexpr int NW = 8;
  constexpr int D = F::VDEPTH;  // ring depth: what fits the registers with the format's raw
  const int ntiles = (rows + 15) / 16;
  size_t extra = 0;  // the problem's own LDS (P::extra_lds), after the kernel's
  if constexpr (requires { P::extra_lds(p); }) extra = (P::extra_lds(p) + 15) / 16 * 16;
  const size_t budget = 150 * 1024 - extra;
  int Kc = (K / 256 + S - 1) / S * 256;  // one part of K
  while (Kc > 256 && vgemm_lds<F, NQ, NW>(Kc, T) > budget) Kc -= 256;
  if (vgemm_lds<F, NQ, NW>(Kc, T) > budget) return decline("verify x does not fit in LDS");
  size_t lds = vgemm_lds<F, NQ, NW>(Kc, T);
  P p2 = p;
  if constexpr (requires { P::extra_lds(p); }) {
    lds = (lds + 15) / 16 * 16;
    p2.lds_off = (uint32_t)lds;
    lds += extra;
  }
  hipLaunchKernelGGL((vgemm_kernel<F, P, NQ, D, NW>), dim3((ntiles + T - 1) / T * S, groups), dim3(64 * NW), lds, st,
                     p2, K, Kc, T, S);
  ISHZ_LAUNCH_CHECK("vgemm launch");
  return ISHZ_OK;
}

// The plain problem: y[M][N] = x[M][K] . W^T for 2..16 tokens; with a K split, part [S][M][N]
// fp32 receives each part's partial product instead (summed by vgemm_sum_kernel).
struct VPlain {
  const uint16_t *x;
  const uint8_t *w;
  size_t rb;
  int M, K, N;
  Out y;
  float *part;
  int S;
  struct Group {};
  DEV bool group(int, Group &) const { return true; }
  DEV int count(const Group &) const { return M; }
  DEV int rows(const Group &) const { return N; }
  DEV const uint16_t *xrow(const Group &, int tk) const { return x + (size_t)tk * K; }
  DEV const uint8_t *wrow(const Group &, int row) const { return w + (size_t)row * rb; }
  DEV void finish(const Group &, int c0, int m, int tb, int te, const float *out) const {
    float *pp = part ? part + (size_t)(blockIdx.x % S) * M * N : nullptr;
    for (int o = threadIdx.x; o < (te - tb) * 256; o += blockDim.x) {
      const int tk = (o >> 4) & 15, row = (tb + (o >> 8)) * 16 + (o & 15);
      if (tk < m && row < N) {
        if (pp) pp[(size_t)(c0 + tk) * N + row] = out[o];
        else y.put((size_t)(c0 + tk) * N + row, c0 + tk, out[o]);
      }
    }
  }
};

// y = the S parts' partial products summed in part order, narrowed once (rows of N outputs).
__global__ __launch_bounds__(256) void vgemm_sum_kernel(const float *__restrict__ part, int S, size_t n, int N, Out y);

// K split for long K (>= 32 steps of 256: x no longer fits one workgroup's LDS and is restaged in
// chunks) and outputs too narrow to give every CU two workgroups' tiles: up to 8 tiles per
// workgroup (x is staged once per workgroup, so more tiles per workgroup stage it fewer times in
// all) and enough parts of K for one round of workgroups, each part at least 4 steps. Measured at
// 5120x25600, M = 8: Q4_K 57 -> 34 us; at K = 4096 the extra sum launch costs more than it saves.
// 1: no split.
inline int vgemm_splits(int M, int K, int N, int cus, int &T) {
  const int ntiles = (N + 15) / 16, steps = K / 256;
  T = (ntiles + cus - 1) / cus;  // tiles per workgroup without a split: one round of CUs
  if (M < 2 || ntiles >= 2 * cus || steps < 32) return 1;
  const int t8 = std::min(8, ntiles), runs = (ntiles + t8 - 1) / t8;
  const int S = std::min(std::max(cus / runs, 1), steps / 4);
  if (S < 2) return 1;
  T = t8;
  return S;
}
inline size_t vgemm_workspace(int M, int K, int N, int cus) {
  int T;
  const int S = vgemm_splits(M, K, N, cus, T);
  return S > 1 ? (size_t)S * M * N * 4 : 0;
}

template <class F>
static int vgemm(const void *x, int M, int K, const void *w, int N, const Out &y, hipStream_t st, void *ws = nullptr,
                 size_t ws_bytes = 0) {
  int T;
  int S = vgemm_splits(M, K, N, gemv_num_cu(), T);
  if (S > 1 && (!ws || ws_bytes < (size_t)S * M * N * 4)) {  // no room for the parts: unsplit
    S = 1;
    T = ((N + 15) / 16 + gemv_num_cu() - 1) / gemv_num_cu();
  }
  const VPlain p{(const uint16_t *)x, (const uint8_t *)w, (size_t)(K / F::BS) * F::TS, M, K, N, y,
                 S > 1 ? (float *)ws : nullptr, S};
  int rc;
  switch ((M + 3) / 4) {
    case 1: rc = launch_vgemm_p<F, VPlain, 1>(p, K, N, 1, T, st, S); break;
    case 2: rc = launch_vgemm_p<F, VPlain, 2>(p, K, N, 1, T, st, S); break;
    case 3: rc = launch_vgemm_p<F, VPlain, 3>(p, K, N, 1, T, st, S); break;
    default: rc = launch_vgemm_p<F, VPlain, 4>(p, K, N, 1, T, st, S); break;
  }
  if (rc || S == 1) return rc;
  const size_t n = (size_t)M * N;
  hipLaunchKernelGGL(vgemm_sum_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 2048)), dim3(256), 0, st,
                     (const float *)ws, S, n, N, y);
  ISHZ_LAUNCH_CHECK("vgemm sum launch");
  return ISHZ_OK;
}

}  // namespace ishz
