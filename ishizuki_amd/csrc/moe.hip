// MoE expert-gathered quantized SwiGLU FFN on gfx950.
//
// Restates MoEBlock.callAsFunction + ResidentExperts.swiglu (Sources/IshizukiKit/Text/
// MoEBlock.swift:124-171) over GGML-block experts: softmax over all E experts in fp32, top-k
// (ties to the lower index), optional renormalisation, then per (token, expert)
// down(silu(gate(x)) * up(x)), the k outputs weighted and summed in fp32, narrowed once.
// Activations between stages are rounded to x's dtype (fp16 or bf16) as the reference's
// gatherQuantizedMM outputs x.dtype; bf16 x and h are staged from fp16 images with a power-of-two
// factor per row.
//
// Kernels:
//  * Route + place: one workgroup, a 16-lane row per token. Top-k by rounds of a row-wide argmax,
//    then the per-expert pair lists and the active-expert list.
//  * One or two tokens: gate+up and down as gathered GEMVs over every (token, slot) pair (the
//    streaming GEMV skeleton), routing inside the first of the two launches and the combine in the
//    second's store.
//  * More tokens: the streaming MFMA kernel over active experts x tiles. An expert's gate and up
//    rows are two tiles of the same workgroup, tokens are gathered through the pair list, and
//    SwiGLU runs in the epilogue. Down works the same way and writes its rows in slot order. With
//    up to 16 tokens every gate/up workgroup routes and places in its own LDS, so the route +
//    place launch is skipped.
//  * Combine: the weighted fp32 sum per token.
// Only routed experts' blocks are ever read.
#include <algorithm>
#include <cstdlib>

#include "affine_nbit.h"
#include "ggml_formats.h"
#include "vgemm.h"

namespace ishz {

struct MoeRoute {
  int32_t *ids;       // [T*k] expert of (t, s)
  float *w;           // [T*k] routing weight of (t, s)
  int32_t *count;     // [1] number of active experts
  int32_t *active;    // [E] active experts, ascending
  int32_t *offs;      // [E+1] pair range of expert e in the sorted list
  int32_t *pair_q;    // [T*k] slot index q = t k + s of sorted pair (its token is q / k)
  int32_t *ids_out;   // optional caller copies of ids / w (null: none)
  float *w_out;
};


// Order-preserving unsigned key of a float: larger value, larger key (0 = retired).
DEV uint32_t okey(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
DEV float from_okey(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
// One step of an argmax over a 16-lane row: the larger key, then the lower index.
template <int CTRL>
DEV void argmax_step(uint32_t &k, int &i) {
  const uint32_t k2 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)k, CTRL, 0xf, 0xf, true);
  const int i2 = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xf, 0xf, true);
  const bool take = k2 > k || (k2 == k && i2 < i);
  k = take ? k2 : k;
  i = take ? i2 : i;
}
template <int CTRL>
DEV float row_max_step(float v) {
  return fmaxf(v, ISHZ_DPP(v, CTRL));
}

// LDS a routing row uses: the token's E order keys, then k winners and k probabilities.
__host__ __device__ inline int route_row_words(int E, int k) { return E + 2 * k; }

// One token's routing by a 16-lane row (MoEBlock.callAsFunction, Text/MoEBlock.swift:124-134):
// softmax max and sum by row reductions; k rounds of a row-wide argmax (DPP only) over the
// logits' order keys (larger logit first, ties to the lower index: the order argPartition gives
// over the probabilities, softmax being strictly increasing), each round retiring its winner.
// Slot s is the round-s winner, worth exp(l - max) / sum; the renormalisation divides by the
// slots' sum taken in slot order. Lane r holds experts r, r + 16, ... : in registers when
// NPL > 0 (E <= 16 NPL; a round is then a register scan), else in `row`'s LDS keys.
// `row` holds route_row_words(E, k) words of LDS.
template <int NPL>
DEV void route_token(const float *__restrict__ l, int E, int k, int normalize, int t, uint32_t *row,
                     const MoeRoute &R, int32_t *ids_lds) {
  constexpr int NR = NPL > 0 ? NPL : 1;
  const int r = threadIdx.x & 15;
  uint32_t *key = row, *win = row + E;
  float *pr = (float *)(row + E + k);
  uint32_t kr[NR];
  float mx = -INFINITY;
  if constexpr (NPL > 0) {
#pragma unroll
    for (int j = 0; j < NPL; j++) {
      const int e = r + 16 * j;
      const float v = e < E ? l[e] : -INFINITY;
      kr[j] = e < E ? okey(v) : 0u;
      mx = fmaxf(mx, v);
    }
  } else {
    for (int e = r; e < E; e += 16) {
      const float v = l[e];
      key[e] = okey(v);
      mx = fmaxf(mx, v);
    }
  }
  mx = row_max_step<0xB1>(mx);   // quad_perm [1,0,3,2]
  mx = row_max_step<0x4E>(mx);   // quad_perm [2,3,0,1]
  mx = row_max_step<0x141>(mx);  // row_half_mirror
  mx = row_max_step<0x140>(mx);  // row_mirror
  float sum = 0.0f;
  if constexpr (NPL > 0) {
#pragma unroll
    for (int j = 0; j < NPL; j++)
      if (r + 16 * j < E) sum += expf(from_okey(kr[j]) - mx);
  } else {
    for (int e = r; e < E; e += 16) sum += expf(from_okey(key[e]) - mx);
  }
  sum = group_sum<16>(sum);
  for (int s = 0; s < k; s++) {
    uint32_t bk = 0;
    int be = 0x7fffffff;
    if constexpr (NPL > 0) {
#pragma unroll
      for (int j = 0; j < NPL; j++) {  // ascending e: a tie keeps the lower index
        const bool take = kr[j] > bk;
        bk = take ? kr[j] : bk;
        be = take ? r + 16 * j : be;
      }
    } else {
      for (int e = r; e < E; e += 16) {
        const uint32_t kv = key[e];
        if (kv > bk) {
          bk = kv;
          be = e;
        }
      }
    }
    argmax_step<0xB1>(bk, be);
    argmax_step<0x4E>(bk, be);
    argmax_step<0x141>(bk, be);
    argmax_step<0x140>(bk, be);
    if constexpr (NPL > 0) {
#pragma unroll
      for (int j = 0; j < NPL; j++) kr[j] = (r + 16 * j == be) ? 0u : kr[j];  // retired
    }
    if (r == (be & 15)) {
      win[s] = (uint32_t)be;
      pr[s] = __builtin_bit_cast(float, bk);  // the winner's key, for now
      if constexpr (NPL == 0) key[be] = 0u;   // retired (a lane only reads its own entries)
    }
  }
  // probabilities in parallel, then the slot-order sum every lane forms alike (winners were
  // written by other lanes of the row: order the wave's LDS accesses)
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  for (int s = r; s < k; s += 16) pr[s] = expf(from_okey(__builtin_bit_cast(uint32_t, pr[s])) - mx) / sum;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  float tot = 0.0f;
  for (int s = 0; s < k; s++) tot += pr[s];
  for (int s = r; s < k; s += 16) {
    const int id = (int)win[s];
    const float w = normalize ? pr[s] / tot : pr[s];
    R.ids[t * k + s] = id;
    R.w[t * k + s] = w;
    if (ids_lds) ids_lds[t * k + s] = id;
    if (R.ids_out) R.ids_out[t * k + s] = id;
    if (R.w_out) R.w_out[t * k + s] = w;
  }
}

// Keys per lane held in registers for E experts (0: keys stay in LDS); MAXE is the largest E
// kept in registers (the 1024-thread fused kernel keeps the register budget at 128).
#define ISHZ_ROUTE_NPL(E, MAXE, CALL)             \
  do {                                            \
    if ((E) <= 64) CALL(4);                       \
    else if ((E) <= 128) CALL(8);                 \
    else if ((E) <= 256) CALL(16);                \
    else if ((E) <= 512 && MAXE >= 512) CALL(32); \
    else if ((E) <= 1024 && MAXE >= 1024) CALL(64); \
    else CALL(0);                                 \
  } while (0)

// Routing alone: a 16-lane row per token, blockDim / 16 tokens per workgroup.
static __global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ logits, int T, int E,
                                                        int k, int normalize, MoeRoute R) {
  extern __shared__ uint32_t rrows[];
  const int rw = threadIdx.x >> 4, t = blockIdx.x * (blockDim.x >> 4) + rw;
  if (t >= T) return;
#define ISHZ_CALL(N) route_token<N>(logits + (size_t)t * E, E, k, normalize, t, rrows + rw * route_row_words(E, k), R, nullptr)
  ISHZ_ROUTE_NPL(E, 1024, ISHZ_CALL);
#undef ISHZ_CALL
}

// Pair lists (one workgroup): per-expert counts in LDS, an exclusive prefix over experts by wave
// 0, then each pair takes the next free position of its expert (the order inside an expert does
// not affect any result: every pair's rows are computed independently). ORDERED: positions in
// (token, slot) order inside each expert instead, the same in every workgroup that places the
// same ids (a pair's rank among the earlier pairs of its expert: P^2 / 2 compares, for few pairs).
template <bool ORDERED = false>
DEV void place_pairs(int T, int E, int k, const MoeRoute &R, const int32_t *ids, int32_t *cnt) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int P = T * k;
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int q = threadIdx.x; q < P; q += blockDim.x) atomicAdd(&cnt[ids[q]], 1);
  __syncthreads();
  if (wave == 0) {
    int carry = 0, nact = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int c = e < E ? cnt[e] : 0;
      int incl = c, act = c > 0;
      for (int m = 1; m < 64; m <<= 1) {
        const int v = __shfl_up(incl, m, 64), a2 = __shfl_up(act, m, 64);
        if (lane >= m) {
          incl += v;
          act += a2;
        }
      }
      if (e < E) {
        R.offs[e] = carry + incl - c;
        cnt[e] = carry + incl - c;  // fill cursor
        if (c) R.active[nact + act - 1] = e;
      }
      carry += __shfl(incl, 63, 64);
      nact += __shfl(act, 63, 64);
    }
    if (lane == 0) {
      R.offs[E] = carry;
      R.count[0] = nact;
    }
  }
  __syncthreads();
  for (int q = threadIdx.x; q < P; q += blockDim.x) {
    int pos;
    if constexpr (ORDERED) {
      const int e = ids[q];
      int r = 0;
      for (int q2 = 0; q2 < q; q2++) r += ids[q2] == e;
      pos = R.offs[e] + r;
    } else {
      pos = atomicAdd(&cnt[ids[q]], 1);
    }
    R.pair_q[pos] = q;
  }
}

static __global__ __launch_bounds__(1024) void moe_place_kernel(int T, int E, int k, MoeRoute R) {
  extern __shared__ int32_t cnt[];  // E counts, then fill cursors
  place_pairs(T, E, k, R, R.ids, cnt);
}

// Routing and placement in one workgroup (up to 64 tokens routed at once, a 16-lane row each):
// one launch instead of two when the rows, the counts and the ids fit in LDS.
static __global__ __launch_bounds__(1024) void moe_route_place_kernel(const float *__restrict__ logits, int T, int E,
                                                               int k, int normalize, MoeRoute R) {
  extern __shared__ uint32_t rrows[];  // [rows][route_row_words] , E counts, then the T k ids
  const int nr = blockDim.x >> 4, rw = threadIdx.x >> 4;
  int32_t *cnt = (int32_t *)(rrows + nr * route_row_words(E, k)), *ids = cnt + E;
  for (int t = rw; t < T; t += nr) {
#define ISHZ_CALL(N) route_token<N>(logits + (size_t)t * E, E, k, normalize, t, rrows + rw * route_row_words(E, k), R, ids)
    ISHZ_ROUTE_NPL(E, 256, ISHZ_CALL);
#undef ISHZ_CALL
  }
  __syncthreads();
  place_pairs(T, E, k, R, ids, cnt);
}

DEV float r16(float v) { return (float)(_Float16)v; }
// The model's 16-bit activation type (fp16, or bf16 with bf): a value rounded to it, its bits,
// and the value of its bits. Every activation the reference materialises between the MoE
// stages (projection outputs, the SwiGLU ops, the shared expert's terms) takes this rounding.
DEV float bf16_round(float v) {
  uint32_t u = __builtin_bit_cast(uint32_t, v);
  u = ((u & 0x7fffffffu) > 0x7f800000u) ? (u | 0x400000u) : u + 0x7fffu + ((u >> 16) & 1u);
  return __builtin_bit_cast(float, u & 0xffff0000u);
}
template <bool BF>
DEV float rnd(float v) { return BF ? bf16_round(v) : r16(v); }
template <bool BF>
DEV uint16_t bits16(float v) { return BF ? (uint16_t)(__builtin_bit_cast(uint32_t, bf16_round(v)) >> 16) : f2h(v); }
template <bool BF>
DEV float from16(uint32_t b) { return BF ? __builtin_bit_cast(float, b << 16) : h2f(b); }
// h = silu(g) * u with the reference's roundings (Text/MoEBlock.swift:168-171): g and u the
// projections' outputs, sigmoid, g * sigmoid and the product each rounded to the activation type.
template <bool BF>
DEV uint16_t swiglu16(float gs, float us) {
  const float g = rnd<BF>(gs), u = rnd<BF>(us);
  const float sg = rnd<BF>(1.0f / (1.0f + __expf(-g)));
  return bits16<BF>(rnd<BF>(g * sg) * u);
}
// fn<BF>() with the activation type fixed at compile time: the fp16 epilogues carry no trace of
// the bf16 path (no factor loads, no per-value dtype tests).
template <class Fn>
DEV void by_act(bool bf, Fn &&fn) {
  if (bf) fn.template operator()<true>();
  else fn.template operator()<false>();
}

// gate + up for one 16-row tile of I of one active expert, 16 routed tokens at a time.
template <class F>
__global__ __launch_bounds__(1024) void moe_gate_up_kernel(const uint16_t *__restrict__ x, int H,
                                                           const uint8_t *__restrict__ gate,
                                                           const uint8_t *__restrict__ up, int I, int k,
                                                           MoeRoute R, uint16_t *__restrict__ h,
                                                           const float *__restrict__ rs, bool bf) {
  extern __shared__ __align__(16) float red[];
  const int a = blockIdx.y;
  if (a >= R.count[0]) return;
  const int e = R.active[a], p0 = R.offs[e], p1 = R.offs[e + 1];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nblk = H / F::BS;
  const size_t rb = (size_t)nblk * F::TS;
  const int i0 = blockIdx.x * 16;
  const size_t erow = (size_t)e * I + min(i0 + j, I - 1);
  const uint8_t *rows[2] = {gate + erow * rb, up + erow * rb};
  for (int c0 = p0; c0 < p1; c0 += 16) {
    const bool tok = c0 + j < p1;
    const uint16_t *xr = x + (size_t)(tok ? R.pair_q[c0 + j] / k : 0) * H;
    f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
    for (int b = wave; b < nblk; b += KS) F::template vblock<2>(rows, b, g, xr, tok, acc);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[((wave * 2 + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    by_act(bf, [&]<bool BF>() {
      for (int o = threadIdx.x; o < 256; o += blockDim.x) {
        const int r = o >> 6, l = o & 63;
        float gs = 0.0f, us = 0.0f;
        for (int v = 0; v < KS; v++) {
          gs += red[((v * 2 + 0) * 4 + r) * 64 + l];
          us += red[((v * 2 + 1) * 4 + r) * 64 + l];
        }
        const int t = 4 * (l >> 4) + r, i = i0 + (l & 15);
        if (c0 + t < p1 && i < I) {
          const float f = BF ? rs[R.pair_q[c0 + t] / k] : 1.0f;  // x's row factor (bf16 x)
          h[(size_t)(c0 + t) * I + i] = swiglu16<BF>(gs * f, us * f);
        }
      }
    });
    __syncthreads();
  }
}

// down projection: o[pair][H] = h[pair] . down_e^T, fp16.
template <class F>
__global__ __launch_bounds__(1024) void moe_down_kernel(const uint16_t *__restrict__ h, int I,
                                                        const uint8_t *__restrict__ down, int H,
                                                        MoeRoute R, uint16_t *__restrict__ o,
                                                        const float *__restrict__ rs, bool bf) {
  extern __shared__ __align__(16) float red[];
  const int a = blockIdx.y;
  if (a >= R.count[0]) return;
  const int e = R.active[a], p0 = R.offs[e], p1 = R.offs[e + 1];
  const int lane = threadIdx.x & 63, wave = wave_id(), KS = blockDim.x >> 6;
  const int j = lane & 15, g = lane >> 4;
  const int nblk = I / F::BS;
  const size_t rb = (size_t)nblk * F::TS;
  const int n0 = blockIdx.x * 32;
  const uint8_t *rows[2] = {down + ((size_t)e * H + min(n0 + j, H - 1)) * rb,
                            down + ((size_t)e * H + min(n0 + 16 + j, H - 1)) * rb};
  for (int c0 = p0; c0 < p1; c0 += 16) {
    const bool tok = c0 + j < p1;
    const uint16_t *xr = h + (size_t)(tok ? c0 + j : 0) * I;
    f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
    for (int b = wave; b < nblk; b += KS) F::template vblock<2>(rows, b, g, xr, tok, acc);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[((wave * 2 + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    by_act(bf, [&]<bool BF>() {
      for (int q = threadIdx.x; q < 512; q += blockDim.x) {
        const int t2 = q >> 8, r = (q >> 6) & 3, l = q & 63;
        float s = 0.0f;
        for (int v = 0; v < KS; v++) s += red[((v * 2 + t2) * 4 + r) * 64 + l];
        const int t = 4 * (l >> 4) + r, n = n0 + 16 * t2 + (l & 15);
        if (c0 + t < p1 && n < H)  // slot order; h's row factor (bf16)
          o[(size_t)R.pair_q[c0 + t] * H + n] = bits16<BF>(BF ? s * rs[c0 + t] : s);
      }
    });
    __syncthreads();
  }
}

static __global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *__restrict__ o, int H,
                                                          int T, int k, MoeRoute R,
                                                          const uint16_t *__restrict__ shared,
                                                          const uint16_t *__restrict__ shared_gate,
                                                          uint16_t *__restrict__ y, bool bf) {
  const size_t total = (size_t)T * H;
  by_act(bf, [&]<bool BF>() {
    for (size_t q = blockIdx.x * (size_t)blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
      const int t = (int)(q / H), n = (int)(q % H);
      float acc = 0.0f;
      for (int s = 0; s < k; s++) {
        acc += from16<BF>(o[((size_t)t * k + s) * H + n]) * R.w[t * k + s];  // o rows in slot order
      }
      if (shared) {  // the shared expert, widened and added before the one narrowing
        const float sg = rnd<BF>(1.0f / (1.0f + __expf(-from16<BF>(shared_gate[t]))));
        acc += rnd<BF>(sg * from16<BF>(shared[q]));
      }
      y[q] = bits16<BF>(acc);
    }
  });
}

// ------------------------------------------------------------------- streaming (MFMA) FFN
// The same two projections as problems of the streaming verify kernel: one group per active
// expert (blockIdx.y), its routed tokens gathered through the pair list.
//
// gate + up: the expert's gate and up rows interleave by tile (tile 2i = gate rows 16i .., tile
// 2i + 1 = the same up rows), so a workgroup holds both halves of each SwiGLU pair.
struct VMoeGateUp {
  const uint16_t *x;
  const uint8_t *gate, *up;
  size_t rb;
  int H, I;
  MoeRoute R;
  uint16_t *h;
  int k;
  const float *rs;  // x's row factors (bf16 x, staged from its fp16 image), or null
  bool bf;          // bf16 activations
  struct Group {
    int e, p0, p1;
  };
  DEV bool group(int a, Group &g) const {
    if (a >= R.count[0]) return false;
    g.e = R.active[a];
    g.p0 = R.offs[g.e];
    g.p1 = R.offs[g.e + 1];
    return true;
  }
  DEV int count(const Group &g) const { return g.p1 - g.p0; }
  DEV int rows(const Group &) const { return 2 * ((I + 15) / 16) * 16; }
  DEV const uint16_t *xrow(const Group &g, int tk) const { return x + (size_t)(R.pair_q[g.p0 + tk] / k) * H; }
  DEV const uint8_t *wrow(const Group &g, int row) const {
    const int tile = row >> 4, i = min((tile >> 1) * 16 + (row & 15), I - 1);
    return ((tile & 1) ? up : gate) + ((size_t)g.e * I + i) * rb;
  }
  DEV void finish(const Group &g, int c0, int m, int tb, int te, const float *out) const {
    finish_pairs(g, c0, m, tb, te, out, R.pair_q);
  }
  // pq: the sorted pairs' slot indices as this launch knows them (global, or the workgroup's own
  // LDS copy when it routes itself)
  DEV void finish_pairs(const Group &g, int c0, int m, int tb, int te, const float *out, const int32_t *pq) const {
    by_act(bf, [&]<bool BF>() {
      for (int o = threadIdx.x; o < (te - tb) / 2 * 256; o += blockDim.x) {
        const int pr = o >> 8, tk = (o >> 4) & 15, nn = o & 15;
        const int i = ((tb >> 1) + pr) * 16 + nn;
        if (tk < m && i < I) {
          const float f = BF ? rs[pq[g.p0 + c0 + tk] / k] : 1.0f;
          h[(size_t)(g.p0 + c0 + tk) * I + i] =
              swiglu16<BF>(out[(2 * pr) * 256 + tk * 16 + nn] * f, out[(2 * pr + 1) * 256 + tk * 16 + nn] * f);
        }
      }
    });
  }
};

// gate + up with the routing done by every workgroup (a few tokens): the separate route + place
// launch is skipped. Each workgroup routes every token and places the pairs (ORDERED, so all of
// them agree) into its own LDS; workgroup (0, 0) publishes ids, weights and the pair lists for
// the down projection and the combine, which run after this launch.
struct VMoeGateUpR : VMoeGateUp {
  const float *logits;
  int T, E, normalize;
  uint32_t lds_off;  // byte offset of the routing scratch in the dynamic LDS (set at launch)
  // scratch (int32 words): routing rows, ids [P], w [P], counts [E], count, active [E],
  // offs [E + 1], pair_q [P]
  // routing rows in LDS: one per token, at most the 32 16-lane rows of a 512-thread workgroup
  __host__ __device__ static int rows_used(int T) { return T < 32 ? T : 32; }
  static size_t extra_lds(const VMoeGateUpR &p) {
    const size_t P = (size_t)p.T * p.k;
    return ((size_t)rows_used(p.T) * route_row_words(p.E, p.k) + 3 * P + 3 * (size_t)p.E + 2) * 4;
  }
  DEV int32_t *scratch() const {
    extern __shared__ __align__(16) u4 vgsm[];
    return (int32_t *)((char *)vgsm + lds_off);
  }
  DEV MoeRoute lds_route() const {
    const int P = T * k;
    int32_t *b = scratch() + rows_used(T) * route_row_words(E, k);
    int32_t *ids = b, *w = b + P, *cnt = w + P, *count = cnt + E, *active = count + 1, *offs = active + E;
    int32_t *pair_q = offs + E + 1;
    return MoeRoute{ids, (float *)w, count, active, offs, pair_q, nullptr, nullptr};
  }
  DEV void prologue() const {
    const MoeRoute L = lds_route();
    const int nr = min(rows_used(T), (int)(blockDim.x >> 4)), rw = route_row_words(E, k), row = threadIdx.x >> 4;
    if (row < nr)
      for (int t = row; t < T; t += nr) {
#define ISHZ_CALL(NPL) route_token<NPL>(logits + (size_t)t * E, E, k, normalize, t, (uint32_t *)scratch() + row * rw, L, nullptr)
        ISHZ_ROUTE_NPL(E, 256, ISHZ_CALL);
#undef ISHZ_CALL
        __builtin_amdgcn_wave_barrier();  // the row's LDS is reused by its next token
      }
    __syncthreads();
    place_pairs<true>(T, E, k, L, L.ids, L.ids + 2 * T * k);
    __syncthreads();
    if (blockIdx.x == 0 && blockIdx.y == 0) {  // publish
      const int P = T * k;
      for (int q = threadIdx.x; q < P; q += blockDim.x) {
        R.ids[q] = L.ids[q];
        R.w[q] = L.w[q];
        R.pair_q[q] = L.pair_q[q];
        if (R.ids_out) R.ids_out[q] = L.ids[q];
        if (R.w_out) R.w_out[q] = L.w[q];
      }
      for (int e = threadIdx.x; e <= E; e += blockDim.x) {
        R.offs[e] = L.offs[e];
        if (e < E) R.active[e] = L.active[e];
      }
      if (threadIdx.x == 0) R.count[0] = L.count[0];
    }
  }
  DEV bool group(int a, Group &g) const {
    const MoeRoute L = lds_route();
    if (a >= L.count[0]) return false;
    g.e = L.active[a];
    g.p0 = L.offs[g.e];
    g.p1 = L.offs[g.e + 1];
    return true;
  }
  DEV const uint16_t *xrow(const Group &g, int tk) const { return x + (size_t)(lds_route().pair_q[g.p0 + tk] / k) * H; }
  // the global pair list is written by workgroup (0, 0) during this launch: read the LDS copy
  DEV void finish(const Group &g, int c0, int m, int tb, int te, const float *out) const {
    finish_pairs(g, c0, m, tb, te, out, lds_route().pair_q);
  }
};

// down: o[pair][H] = h[pair] . down_e^T (fp16).
struct VMoeDown {
  const uint16_t *h;
  const uint8_t *down;
  size_t rb;
  int I, H;
  MoeRoute R;
  uint16_t *o;
  const float *rs;  // h's row factors (bf16 h, staged from its fp16 image), or null
  bool bf;
  struct Group {
    int e, p0, p1;
  };
  DEV bool group(int a, Group &g) const {
    if (a >= R.count[0]) return false;
    g.e = R.active[a];
    g.p0 = R.offs[g.e];
    g.p1 = R.offs[g.e + 1];
    return true;
  }
  DEV int count(const Group &g) const { return g.p1 - g.p0; }
  DEV int rows(const Group &) const { return H; }
  DEV const uint16_t *xrow(const Group &g, int tk) const { return h + (size_t)(g.p0 + tk) * I; }
  DEV const uint8_t *wrow(const Group &g, int row) const { return down + ((size_t)g.e * H + row) * rb; }
  DEV void finish(const Group &g, int c0, int m, int tb, int te, const float *out) const {
    by_act(bf, [&]<bool BF>() {
      for (int q = threadIdx.x; q < (te - tb) * 256; q += blockDim.x) {
        const int tk = (q >> 4) & 15, row = (tb + (q >> 8)) * 16 + (q & 15);
        if (tk < m && row < H)  // slot order
          o[(size_t)R.pair_q[g.p0 + c0 + tk] * H + row] = bits16<BF>(BF ? out[q] * rs[g.p0 + c0 + tk] : out[q]);
      }
    });
  }
};

// ------------------------------------------------------------------- gathered GEMV (few tokens)
// With one or two tokens every routed (token, slot) pair is a GEMV of its own; the streaming
// GEMV skeleton runs all of them in two launches and nothing else runs:
//  * gate + up + SwiGLU: pair p = t k + s (slot order) owns rows p 2I .. p 2I + 2I - 1, in blocks
//    of eight: four gate rows, then the same four up rows (row 8b + i of the pair: gate row 4b + i,
//    row 8b + 4 + i: up row 4b + i), and a workgroup owns whole blocks, so its final store forms
//    h = silu(gate) * up of each of its rows with the reference's fp16 roundings (Text/MoEBlock.swift
//    :168-171) and writes h [P][I]. Every workgroup routes the tokens itself before its first
//    weight load (a 16-lane row per token, ids kept in LDS); workgroup 0 publishes the ids and
//    weights for the down launch and the caller. A row group never straddles two pairs (2I is a
//    multiple of 256), so the expert id is wave-uniform.
//  * down + combine: rows run in blocks of four outputs of one pair, the token's k pairs' blocks
//    of the same four outputs in turn (row j: token j / (H k), slot (j / 4) % k, output
//    4 ((j / 4k) % (H / 4)) + j % 4), and a workgroup owns whole runs of k blocks; x is the pairs'
//    h. Its outputs are combined in the workgroup's final store: y = sum over slots of
//    w_s fp16(down_s), in fp32 in slot order, plus the shared expert's term, narrowed once
//    (Text/MoEBlock.swift:143-160).
typedef __attribute__((address_space(3))) const int32_t lds_i32;
typedef __attribute__((address_space(3))) const float lds_f32;

struct MoeTokens {
  const float *logits;
  int T, E, normalize;
  MoeRoute R;  // ids / weights (and the caller's copies) written by workgroup 0
};

// a, or b when c (wave-uniform): a plus an offset that is either zero or b - a. Written as a
// plain select of two argument fields, the compiler loads the field from the kernel arguments at a
// computed offset, a memory load every weight batch would then depend on; an offset kept opaque
// keeps both fields in registers, and a's address space (global loads, not flat).
template <class T>
DEV T *pick_ptr(bool c, T *a, T *b) {
  int64_t d = (const char *)b - (const char *)a;
  asm("" : "+s"(d));
  return (T *)((const char *)a + (c ? d : 0));
}

template <class F>
struct FMoeGateUp : F {
  struct Args {
    const uint8_t *gate, *up;
    size_t rb;
    int K, N;  // K = H, N = P 2I
    int I, k;
    MoeTokens rt;
    const uint16_t *x;  // [T][H] (bf16 x: its fp16 image)
    const float *rs;    // the image's row factors, or null
    bool bf;
  };
  struct XPre {};
  struct Prep {
    lds_i32 *ids;  // [T k] expert of (t, s), in LDS
  };
  // one workgroup per CU for both gathered GEMVs: measured at the Qwen shape, T = 1, Q4_K experts
  // 20.95 -> 20.4 us against two (down alone 21.0 -> 20.7; gate/up alone neutral; three and four
  // slower: 21.6, 22.8)
  static int occ(const Args &) { return 1; }
  // LDS after the format's tables: a routing row per token, the ids, scratch for the weights
  static size_t route_words(const Args &a) { return (size_t)a.rt.T * route_row_words(a.rt.E, a.k) + 2 * a.rt.T * a.k; }
  static size_t extra_lds_bytes(const Args &a) { return F::tab_bytes() + route_words(a) * 4; }
  static __host__ __device__ int nx(const Args &a) { return a.N / (2 * a.I * a.k); }  // tokens
  static DEV int xsel(const Args &a, int row) { return row / (2 * a.I * a.k); }
  static constexpr bool X_ALL = true;  // every token's x is staged (by prepare), image t at t
  static DEV Prep prepare(const Args &a, u4 *extra, void *lds_x) {
    uint32_t *rows = (uint32_t *)extra + F::tab_bytes() / 4;
    const int rw = route_row_words(a.rt.E, a.k);
    int32_t *ids = (int32_t *)(rows + a.rt.T * rw);
    if (threadIdx.x >= 64) {  // the other waves stage every token's x meanwhile
      u4 *xs = (u4 *)lds_x;
      const int ug = (F::units(a.K) + 15) / 16;
      F::stage_images(a.x, a.K, a.rt.T, xs, (float *)(xs + a.rt.T * ug * 16 * F::R), F::units(a.K), 64,
                      blockDim.x - 64);
    } else if ((int)threadIdx.x < 16 * a.rt.T) {  // wave 0: token t on lanes 16 t .. 16 t + 15
      const int t = threadIdx.x >> 4;
      MoeRoute R = a.rt.R;
      if (blockIdx.x) {  // only workgroup 0 publishes
        R.ids = ids + a.rt.T * a.k;
        R.w = (float *)(ids + a.rt.T * a.k);
        R.ids_out = nullptr;
        R.w_out = nullptr;
      }
      const float *l = a.rt.logits + (size_t)t * a.rt.E;
#define ISHZ_CALL(NPL) route_token<NPL>(l, a.rt.E, a.k, a.rt.normalize, t, rows + t * rw, R, ids)
      ISHZ_ROUTE_NPL(a.rt.E, 256, ISHZ_CALL);
#undef ISHZ_CALL
    }
    __syncthreads();
    return {(lds_i32 *)ids};
  }
  static __host__ __device__ int group_align(const Args &, int rpw) { return 8 / rpw; }
  // weight row of row j' (0 .. 2I) of a pair: gate or up, and its index i
  static DEV bool is_up(int j) { return (j >> 2) & 1; }
  static DEV int wrow(int j) { return ((j >> 3) << 2) | (j & 3); }
  static DEV const uint8_t *row_ptr(const Args &a, const Prep &pp, int row) {
    const int r0 = __builtin_amdgcn_readfirstlane(row);  // a batch's rows share pair and gate/up
    const int p = r0 / (2 * a.I);
    const int e = pp.ids[p], j = row - p * 2 * a.I;
    return pick_ptr(is_up(r0 - p * 2 * a.I), a.gate, a.up) + ((size_t)e * a.I + wrow(j)) * a.rb;
  }
  static DEV auto load(const Args &a, const Prep &pp, int row, int u) { return F::load_row(row_ptr(a, pp, row), u); }
  static DEV XPre stage_load(const Args &, const uint16_t *, int) { return {}; }
  static DEV void stage(const Args &, const uint16_t *, u4 *, float *, u4 *extra, int, const XPre &, int, int) {
    F::gemv_tables(extra);  // x was staged by prepare
    __syncthreads();
  }
  // rows row0 .. row0 + nrows: whole eight-row blocks; h [P][I] fp16
  static DEV void store(const Args &a, uint16_t *h, int row0, int nrows, const float *vals) {
    by_act(a.bf, [&]<bool BF>() {
      for (int q = threadIdx.x; q < nrows / 2; q += blockDim.x) {
        const int blk = q >> 2, i4 = q & 3, j = row0 + 8 * blk;
        const int p = j / (2 * a.I), i = wrow(j - p * 2 * a.I) + i4;
        const float f = BF ? a.rs[p / a.k] : 1.0f;
        h[(size_t)p * a.I + i] = swiglu16<BF>(vals[8 * blk + i4] * f, vals[8 * blk + 4 + i4] * f);
      }
    });
  }
};

template <class F>
struct FMoeDown : F {
  struct Args {
    const uint8_t *down;
    size_t rb;
    int K, N;  // K = I, N = P H
    int H, k;
    const int32_t *ids;  // [T k], from the gate/up launch
    const float *w;      // [T k] routing weights
    const uint16_t *shared, *shared_gate;  // optional: shared expert output [T][H] and gate logit [T]
    const uint16_t *h;   // [P][I] SwiGLU outputs of the gate/up launch: the x images
    const float *rs;     // h's row factors (bf16: h staged from its fp16 image), or null
    bool bf;
  };
  struct XPre {};
  struct Prep {
    lds_i32 *ids;  // [P] expert of each pair, in LDS before the first weight load
    lds_f32 *w;    // [P] routing weight of each pair
  };
  static int occ(const Args &) { return 1; }  // as FMoeGateUp
  static size_t extra_lds_bytes(const Args &a) { return F::tab_bytes() + ((size_t)nx(a) * 8 + 15) / 16 * 16; }
  static __host__ __device__ int nx(const Args &a) { return a.N / a.H; }  // pairs
  static constexpr bool X_ALL = true;  // every pair's h is staged (by prepare), image p at p
  // The loads of ids and weights go out first, then the staging of every pair's h (which waits
  // for its own loads); both arrive in the same memory round trip, before the first weight load
  // (whose rows the ids select) is issued.
  static DEV Prep prepare(const Args &a, u4 *extra, void *lds_x) {
    const int P = nx(a), tid = threadIdx.x;
    int32_t *ids = (int32_t *)((char *)extra + F::tab_bytes());
    float *w = (float *)(ids + P);
    int32_t id = 0;
    float wv = 0.0f;
    if (tid < P) {
      id = a.ids[tid];
      wv = a.w[tid];
    }
    u4 *xs = (u4 *)lds_x;
    const int units = F::units(a.K), ug = (units + 15) / 16;
    F::stage_images(a.h, a.K, P, xs, (float *)(xs + P * ug * 16 * F::R), units);
    if (tid < P) {
      ids[tid] = id;
      w[tid] = wv;
    }
    for (int i = tid + blockDim.x; i < P; i += blockDim.x) {
      ids[i] = a.ids[i];
      w[i] = a.w[i];
    }
    __syncthreads();
    return {(lds_i32 *)ids, (lds_f32 *)w};
  }
  static __host__ __device__ int group_align(const Args &a, int rpw) { return 4 * a.k / rpw; }
  static DEV int pair_of(const Args &a, int row) { return (row / (a.H * a.k)) * a.k + (row >> 2) % a.k; }
  static DEV int out_of(const Args &a, int row) { return ((row >> 2) / a.k % (a.H / 4)) * 4 + (row & 3); }
  static DEV int xsel(const Args &a, int row) { return pair_of(a, row); }
  static DEV const uint8_t *row_ptr(const Args &a, const Prep &pp, int row) {
    const int r0 = __builtin_amdgcn_readfirstlane(row) & ~3;  // the group's four-row block
    const int e = pp.ids[pair_of(a, r0)];
    return a.down + ((size_t)e * a.H + out_of(a, r0) + (row & 3)) * a.rb;
  }
  static DEV auto load(const Args &a, const Prep &pp, int row, int u) { return F::load_row(row_ptr(a, pp, row), u); }
  static DEV XPre stage_load(const Args &, const uint16_t *, int) { return {}; }
  static DEV void stage(const Args &, const uint16_t *, u4 *, float *, u4 *extra, int, const XPre &, int, int) {
    F::gemv_tables(extra);  // h was staged by prepare
    __syncthreads();
  }
  // rows row0 .. row0 + nrows (whole runs of k four-row blocks): one output per four-row block
  // position, its k slots' fp16 rows weighted in fp32 in slot order, then the shared term.
  static DEV void store(const Args &a, uint16_t *y, int row0, int nrows, const float *vals, const Prep &pp) {
    const int run = 4 * a.k;
    by_act(a.bf, [&]<bool BF>() {
      for (int q = threadIdx.x; q < nrows / a.k; q += blockDim.x) {
        const int blk = q >> 2, rr = q & 3, j0 = row0 + blk * run;
        const int t = j0 / (a.H * a.k), r = out_of(a, j0) + rr;
        float acc = 0.0f;
        for (int s = 0; s < a.k; s++) {
          const float v = vals[blk * run + 4 * s + rr];
          acc += rnd<BF>(BF ? v * a.rs[t * a.k + s] : v) * pp.w[t * a.k + s];
        }
        if (a.shared) {
          const float sg = rnd<BF>(1.0f / (1.0f + __expf(-from16<BF>(a.shared_gate[t]))));
          acc += rnd<BF>(sg * from16<BF>(a.shared[(size_t)t * a.H + r]));
        }
        y[(size_t)t * a.H + r] = bits16<BF>(acc);
      }
    });
  }
};

// Quads per pass sized for about twice an expert's expected load (T k / E tokens) plus two;
// an expert with more tokens takes further passes.
template <class F, class P>
static int moe_vgemm(const P &p, int T, int E, int k, int K, int rows, int groups, int tiles_per_wg, hipStream_t st) {
  const int want = (2 * T * k / std::max(E, 1) + 2 + 3) / 4;
  switch (std::max(1, std::min({4, (T + 3) / 4, want}))) {
    case 1: return launch_vgemm_p<F, P, 1>(p, K, rows, groups, tiles_per_wg, st);
    case 2: return launch_vgemm_p<F, P, 2>(p, K, rows, groups, tiles_per_wg, st);
    case 3: return launch_vgemm_p<F, P, 3>(p, K, rows, groups, tiles_per_wg, st);
    default: return launch_vgemm_p<F, P, 4>(p, K, rows, groups, tiles_per_wg, st);
  }
}

// ------------------------------------------------------------------- host
// Standalone routing launch: 16 rows per workgroup, or 4 when a row's LDS is large.
static int route_launch(const float *logits, int T, int E, int k, int normalize, const MoeRoute &R, hipStream_t st) {
  const size_t row = (size_t)route_row_words(E, k) * 4;
  const int rows = 16 * row <= 64 * 1024 ? 16 : 4;
  if (rows * row > 160 * 1024) return decline("too many experts for one routing workgroup");
  hipLaunchKernelGGL(moe_route_kernel, dim3((T + rows - 1) / rows), dim3(16 * rows), rows * row, st, logits, T, E, k,
                     normalize, R);
  ISHZ_LAUNCH_CHECK("moe route launch");
  return ISHZ_OK;
}

struct MoeLayout {
  size_t ids, w, count, active, offs, pair_q, h, gu, o, ximg, himg, total;
};
static MoeLayout moe_layout(int T, int H, int E, int I, int k) {
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  MoeLayout L;
  const size_t P = (size_t)T * k;
  size_t off = 0;
  L.ids = off; off += al(P * 4);
  L.w = off; off += al(P * 4);
  L.count = off; off += al(4);
  L.active = off; off += al((size_t)E * 4);
  L.offs = off; off += al((size_t)(E + 1) * 4);
  L.pair_q = off; off += al(P * 4);
  L.h = off; off += al(P * I * 2);
  L.gu = off; off += al(P * 2 * I * 2);
  L.o = off; off += al(P * H * 2);
  L.ximg = off; off += al(act_image_bytes(T, H));      // bf16 x: its fp16 image
  L.himg = off; off += al(act_image_bytes((int)P, I));  // bf16 h: its fp16 image
  L.total = off;
  return L;
}

static MoeRoute moe_route_ptrs(void *ws, const MoeLayout &L) {
  uint8_t *b = (uint8_t *)ws;
  return MoeRoute{(int32_t *)(b + L.ids), (float *)(b + L.w), (int32_t *)(b + L.count),
                  (int32_t *)(b + L.active), (int32_t *)(b + L.offs), (int32_t *)(b + L.pair_q), nullptr,
                  nullptr};
}

static int ks_for(int tiles, int nblk) {
  int ks = 1;
  while (ks < 16 && ks < nblk && tiles * ks < 256 * 16) ks *= 2;
  return ks;
}

// One or two tokens take the gathered GEMVs when down's LDS (every pair's staged h and x image,
// about 2 I + 2.9 I bytes per pair) fits; otherwise the per-block kernels.
static bool gathered_gemv(int T, int H, int I, int k) {
  const size_t per_pair = (size_t)2 * I + ((size_t)I / 64 + 15) / 16 * 16 * (8 * 16 + 4 * 4);
  return H % 256 == 0 && I % 256 == 0 && T <= 2 && (size_t)T * k * per_pair <= 144 * 1024;
}

// Three to sixteen tokens on the streaming kernels: gate/up routes inside every workgroup
// (VMoeGateUpR) in place of the route + place launch.
static bool route_in_gate_up(int T, int H, int E, int I, int k) {
  return !gathered_gemv(T, H, I, k) && H % 256 == 0 && I % 256 == 0 && T > 2 && T <= 16 && E <= 256 &&
         T * k <= 256;
}

// The activation type of an FFN call: fp16, or bf16 (bf). bf16 x and h are staged from fp16
// images with a power-of-two factor per row (act_prepare: exact for bf16 values down to 2^-17 of
// their row's largest), and the projections' sums are multiplied back before their roundings.
struct MoeAct {
  bool bf;
  const float *rsx;  // x's row factors (bf16), or null
  void *himg;        // workspace for h's image (bf16)
};
// h's fp16 image and row factors for the down projection (bf16), or h itself.
static int moe_h_image(const MoeAct &ma, const uint16_t *h, int P, int I, hipStream_t st, const uint16_t **h16,
                       const float **rsh) {
  if (!ma.bf) {
    *h16 = h;
    *rsh = nullptr;
    return ISHZ_OK;
  }
  return act_prepare(h, ISHZ_DT_BF16, P, I, ma.himg, st, h16, rsh);
}

template <class F>
static int moe_ffn(const void *x, int T, int H, int E, int I, int k, const void *gate,
                   const void *up, const void *down, const MoeTokens &rt, uint16_t *h, uint16_t *gu, uint16_t *o,
                   const uint16_t *shared, const uint16_t *shared_gate, void *y, hipStream_t st, const MoeAct &ma) {
  const MoeRoute &R = rt.R;
  const uint16_t *h16;
  const float *rsh;
  const int amax = std::min(E, T * k);
  const size_t total = (size_t)T * H;
  // one or two tokens: every (token, slot) pair is a GEMV; two launches of the streaming GEMV
  // (routing in the first, the combine in the second)
  if (gathered_gemv(T, H, I, k)) {
    const int P = T * k;
    const typename FMoeGateUp<F>::Args ga{(const uint8_t *)gate, (const uint8_t *)up, (size_t)(H / F::BS) * F::TS,
                                          H, P * 2 * I, I, k, rt, (const uint16_t *)x, ma.rsx, ma.bf};
    int rc = launch_gemv<FMoeGateUp<F>>(ga, x, gu, st);
    if (rc) return rc;
    if ((rc = moe_h_image(ma, gu, P, I, st, &h16, &rsh))) return rc;
    const typename FMoeDown<F>::Args da{(const uint8_t *)down, (size_t)(I / F::BS) * F::TS, I, P * H, H, k,
                                        R.ids, R.w, shared, shared_gate, h16, rsh, ma.bf};
    return launch_gemv<FMoeDown<F>>(da, h16, y, st);
  }
  // streaming MFMA kernels from 3 tokens up; one or two tokens (a GEMV per expert) run faster on
  // the per-block kernels below, which start streaming without staging x
  if (H % 256 == 0 && I % 256 == 0 && T > 2) {
    // tiles per workgroup: about two workgroups per CU over the routed experts, one when they hold
    // two tokens or fewer each (measured at the Qwen shape: T = 8, 1.2 tokens per expert, 65.6 ->
    // 60.7 us with one; T = 64, 4 per expert, 134 -> 153 us); gate/up: an even count, whole SwiGLU
    // pairs; with 8 or more a wave takes whole tiles
    const int tiles_gu = 2 * ((I + 15) / 16), tiles_dn = (H + 15) / 16;
    const int act = std::min(amax, 128);
    const int per_cu = T * k <= 2 * act ? 1 : 2;
    auto pick = [&](int tiles, int even) {
      int t = std::max(1, std::min(32, tiles * act / (gemv_num_cu() * per_cu)));
      if (even) t = std::max(2, t & ~1);
      return t;
    };
    const VMoeGateUp gu{(const uint16_t *)x, (const uint8_t *)gate, (const uint8_t *)up,
                        (size_t)(H / F::BS) * F::TS, H, I, R, h, k, ma.rsx, ma.bf};
    int rc;
    if (route_in_gate_up(T, H, E, I, k)) {
      VMoeGateUpR gr{};
      static_cast<VMoeGateUp &>(gr) = gu;
      gr.logits = rt.logits;
      gr.T = T;
      gr.E = E;
      gr.normalize = rt.normalize;
      rc = moe_vgemm<F>(gr, T, E, k, H, tiles_gu * 16, amax, pick(tiles_gu, 1), st);
    } else {
      rc = moe_vgemm<F>(gu, T, E, k, H, tiles_gu * 16, amax, pick(tiles_gu, 1), st);
    }
    if (rc) return rc;
    if ((rc = moe_h_image(ma, h, T * k, I, st, &h16, &rsh))) return rc;
    const VMoeDown dn{h16, (const uint8_t *)down, (size_t)(I / F::BS) * F::TS, I, H, R, o, rsh, ma.bf};
    rc = moe_vgemm<F>(dn, T, E, k, I, H, amax, pick(tiles_dn, 0), st);
    if (rc) return rc;
  } else {
    int ks = ks_for((I / 16) * amax, H / F::BS);
    hipLaunchKernelGGL((moe_gate_up_kernel<F>), dim3(I / 16, amax), dim3(64 * ks), (size_t)ks * 2 * 256 * 4, st,
                       (const uint16_t *)x, H, (const uint8_t *)gate, (const uint8_t *)up, I, k, R, h, ma.rsx, ma.bf);
    ISHZ_LAUNCH_CHECK("moe gate/up launch");
    int rc = moe_h_image(ma, h, T * k, I, st, &h16, &rsh);
    if (rc) return rc;
    ks = ks_for((H / 32) * amax, I / F::BS);
    hipLaunchKernelGGL((moe_down_kernel<F>), dim3((H + 31) / 32, amax), dim3(64 * ks), (size_t)ks * 2 * 256 * 4,
                       st, h16, I, (const uint8_t *)down, H, R, o, rsh, ma.bf);
    ISHZ_LAUNCH_CHECK("moe down launch");
  }
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)std::min<size_t>((total + 255) / 256, 4096)), dim3(256), 0,
                     st, o, H, T, k, R, shared, shared_gate, (uint16_t *)y, ma.bf);
  ISHZ_LAUNCH_CHECK("moe combine launch");
  return ISHZ_OK;
}

// Routing, and the pair lists when `place` (the streaming MFMA projections need them; the
// gathered GEMVs read the slot-order ids only): one launch when it fits one workgroup's LDS.
static int moe_route_all(const float *logits, int T, int E, int topk, int normalize, const MoeRoute &R, bool place,
                         hipStream_t st) {
  const int nr = std::min((T + 3) / 4 * 4, 64);  // routing rows: whole waves, at most 16
  const size_t fused_lds = ((size_t)nr * route_row_words(E, topk) + E + (size_t)T * topk) * 4;
  if (!place) return route_launch(logits, T, E, topk, normalize, R, st);
  if (fused_lds <= 64 * 1024) {
    hipLaunchKernelGGL(moe_route_place_kernel, dim3(1), dim3(16 * nr), fused_lds, st, logits, T, E, topk, normalize, R);
    ISHZ_LAUNCH_CHECK("moe route launch");
    return ISHZ_OK;
  }
  const int rc = route_launch(logits, T, E, topk, normalize, R, st);
  if (rc) return rc;
  hipLaunchKernelGGL(moe_place_kernel, dim3(1), dim3(1024), (size_t)E * 4, st, T, E, topk, R);
  ISHZ_LAUNCH_CHECK("moe place launch");
  return ISHZ_OK;
}

// ------------------------------------------------------------------- affine experts
// StackedExperts (Text/MoEBlock.swift:22-50): every expert's gate, up and down as one MLX affine
// pack each ([E][I][H], [E][I][H], [E][H][I] weights; scales and biases per group). The same
// projections as the GGUF problems above, their rows read as affine rows.
struct AffPack {
  const uint32_t *codes;
  const uint16_t *scales, *biases;
  int wpr, gpr;  // code words and groups per weight row
  DEV AffRow row(size_t r) const { return {codes + r * wpr, scales + r * gpr, biases + r * gpr}; }
};
struct VMoeGateUpA : VMoeGateUp {
  AffPack g, u;
  DEV AffRow arow(const Group &gp, int row) const {
    const int tile = row >> 4, i = min((tile >> 1) * 16 + (row & 15), I - 1);
    return ((tile & 1) ? u : g).row((size_t)gp.e * I + i);
  }
};
struct VMoeDownA : VMoeDown {
  AffPack d;
  DEV AffRow arow(const Group &gp, int row) const { return d.row((size_t)gp.e * H + row); }
};

// One or two tokens: the gathered GEMVs with affine rows.
template <class F>
struct FMoeGateUpA : FMoeGateUp<F> {
  struct Args : FMoeGateUp<F>::Args {
    AffPack g, u;
  };
  using Prep = typename FMoeGateUp<F>::Prep;
  static DEV auto load(const Args &a, const Prep &pp, int row, int u) {
    using B = FMoeGateUp<F>;
    const int r0 = __builtin_amdgcn_readfirstlane(row);
    const int p = r0 / (2 * a.I);
    const int e = pp.ids[p], j = row - p * 2 * a.I;
    const bool up = B::is_up(r0 - p * 2 * a.I);
    const AffPack pk{pick_ptr(up, a.g.codes, a.u.codes), pick_ptr(up, a.g.scales, a.u.scales),
                     pick_ptr(up, a.g.biases, a.u.biases), a.g.wpr, a.g.gpr};
    return F::load_unit(pk.row((size_t)e * a.I + B::wrow(j)), u);
  }
};
template <class F>
struct FMoeDownA : FMoeDown<F> {
  struct Args : FMoeDown<F>::Args {
    AffPack d;
  };
  using Prep = typename FMoeDown<F>::Prep;
  static DEV auto load(const Args &a, const Prep &pp, int row, int u) {
    const int r0 = __builtin_amdgcn_readfirstlane(row) & ~3;
    const int e = pp.ids[FMoeDown<F>::pair_of(a, r0)];
    return F::load_unit(a.d.row((size_t)e * a.H + FMoeDown<F>::out_of(a, r0) + (row & 3)), u);
  }
};

template <class F>
static int moe_ffn_affine(const void *x, int T, int H, int E, int I, int k, const AffPack &gate, const AffPack &up,
                          const AffPack &down, const MoeTokens &rt, uint16_t *h, uint16_t *gu, uint16_t *o,
                          const uint16_t *shared, const uint16_t *shared_gate, void *y, hipStream_t st,
                          const MoeAct &ma) {
  const MoeRoute &R = rt.R;
  const uint16_t *h16;
  const float *rsh;
  const int amax = std::min(E, T * k);
  const size_t total = (size_t)T * H;
  if (gathered_gemv(T, H, I, k)) {  // as moe_ffn: every (token, slot) pair a GEMV, two launches
    const int P = T * k;
    typename FMoeGateUpA<F>::Args ga{};
    static_cast<typename FMoeGateUp<F>::Args &>(ga) = typename FMoeGateUp<F>::Args{
        nullptr, nullptr, 0, H, P * 2 * I, I, k, rt, (const uint16_t *)x, ma.rsx, ma.bf};
    ga.g = gate;
    ga.u = up;
    int rc = launch_gemv<FMoeGateUpA<F>>(ga, x, gu, st);
    if (rc) return rc;
    if ((rc = moe_h_image(ma, gu, P, I, st, &h16, &rsh))) return rc;
    typename FMoeDownA<F>::Args da{};
    static_cast<typename FMoeDown<F>::Args &>(da) =
        typename FMoeDown<F>::Args{nullptr, 0, I, P * H, H, k, R.ids, R.w, shared, shared_gate, h16, rsh, ma.bf};
    da.d = down;
    return launch_gemv<FMoeDownA<F>>(da, h16, y, st);
  }
  const int tiles_gu = 2 * ((I + 15) / 16), tiles_dn = (H + 15) / 16;
  const int act = std::min(amax, 128);
  auto pick = [&](int tiles, int even) {  // two workgroups per CU (one measured slower here)
    int t = std::max(1, std::min(32, tiles * act / (gemv_num_cu() * 2)));
    if (even) t = std::max(2, t & ~1);
    return t;
  };
  VMoeGateUpA pgu{};
  static_cast<VMoeGateUp &>(pgu) = VMoeGateUp{(const uint16_t *)x, nullptr, nullptr, 0, H, I, R, h, k, ma.rsx, ma.bf};
  pgu.g = gate;
  pgu.u = up;
  int rc = moe_vgemm<F>(pgu, T, E, k, H, tiles_gu * 16, amax, pick(tiles_gu, 1), st);
  if (rc) return rc;
  if ((rc = moe_h_image(ma, h, T * k, I, st, &h16, &rsh))) return rc;
  VMoeDownA dn{};
  static_cast<VMoeDown &>(dn) = VMoeDown{h16, nullptr, 0, I, H, R, o, rsh, ma.bf};
  dn.d = down;
  rc = moe_vgemm<F>(dn, T, E, k, I, H, amax, pick(tiles_dn, 0), st);
  if (rc) return rc;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)std::min<size_t>((total + 255) / 256, 4096)), dim3(256), 0,
                     st, o, H, T, k, R, shared, shared_gate, (uint16_t *)y, ma.bf);
  ISHZ_LAUNCH_CHECK("moe combine launch");
  return ISHZ_OK;
}

// The affine experts of the widths other than 4 and 8 bits (2, 3 and 5 to 7): instantiated in
// moe_affine_w23.hip and moe_affine_w567.hip, which include this file's body, so that the three
// translation units compile in parallel.
#define ISHZ_MOE_AFFINE_ARGS                                                                                  \
  const void *x, int T, int H, int E, int I, int k, const AffPack &gate, const AffPack &up, const AffPack &down, \
      const MoeTokens &rt, uint16_t *h, uint16_t *gu, uint16_t *o, const uint16_t *shared,                     \
      const uint16_t *shared_gate, void *y, hipStream_t st, const MoeAct &ma
#define ISHZ_MOE_AFFINE_PASS x, T, H, E, I, k, gate, up, down, rt, h, gu, o, shared, shared_gate, y, st, ma
int moe_affine_w23(int bits, int group, bool bf16s, ISHZ_MOE_AFFINE_ARGS);
int moe_affine_w567(int bits, int group, bool bf16s, ISHZ_MOE_AFFINE_ARGS);

}  // namespace ishz

#ifndef ISHZ_MOE_BODY_ONLY
using namespace ishz;

extern "C" size_t ishz_moe_workspace_size(int T, int H, int E, int I, int topk) {
  return moe_layout(T, H, E, I, topk).total;
}

extern "C" int ishz_moe_route(const float *logits, int T, int E, int topk, int normalize,
                              int32_t *ids, float *weights, ishz_stream_t stream) {
  if (T <= 0 || E <= 0 || topk <= 0 || topk > E || topk > 64) return decline("bad routing shape");
  if ((size_t)4 * route_row_words(E, topk) * 4 > 160 * 1024) return decline("too many experts for one routing workgroup");
  if (!logits || !ids || !weights) return einval("null pointer");
  MoeRoute R{ids, weights, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  return route_launch(logits, T, E, topk, normalize, R, S(stream));
}

extern "C" int ishz_moe_swiglu(uint32_t type, const void *x, int x_dtype, int T, int H,
                               const float *logits, int E, int topk, int normalize,
                               const void *gate, const void *up, const void *down,
                               size_t expert_bytes, int I, const void *shared, const void *shared_gate,
                               void *y, int32_t *ids_out, float *weights_out, void *workspace,
                               size_t workspace_bytes, ishz_stream_t stream) {
  const int bs = ishz_ggml_block_size(type);
  if (type != ISHZ_GGML_Q4_K && type != ISHZ_GGML_Q6_K && type != ISHZ_GGML_Q4_0)
    return decline("MoE experts must be Q4_0, Q4_K or Q6_K");
  if (x_dtype != ISHZ_DT_F16 && x_dtype != ISHZ_DT_BF16) return decline("activations must be fp16 or bf16");
  if (T <= 0 || E <= 0 || topk <= 0 || topk > E || E > 4096) return decline("bad routing shape");
  if (topk > 64 || (size_t)4 * route_row_words(E, topk) * 4 > 160 * 1024)
    return decline("too many experts for one routing workgroup");
  if (H <= 0 || I <= 0 || H % bs || I % bs) return decline("H and I must be whole blocks");
  const size_t need = (size_t)I * (H / bs) * ishz_ggml_type_size(type);
  if (expert_bytes < need || (size_t)H * (I / bs) * ishz_ggml_type_size(type) > expert_bytes)
    return decline("expert buffers too short");
  if (!x || !logits || !gate || !up || !down || !y) return einval("null pointer");
  if (!shared != !shared_gate) return einval("the shared expert needs both its output and its gate");
  const MoeLayout L = moe_layout(T, H, E, I, topk);
  if (!workspace || workspace_bytes < L.total) return einval("workspace too small (ishz_moe_workspace_size)");
  MoeRoute R = moe_route_ptrs(workspace, L);
  R.ids_out = ids_out;
  R.w_out = weights_out;
  hipStream_t st = S(stream);
  const MoeTokens rt{logits, T, E, normalize, R};
  // (the gathered GEMVs, and gate/up for a few tokens, route inside their first launch)
  if (!gathered_gemv(T, H, I, topk) && !route_in_gate_up(T, H, E, I, topk)) {
    const int rc = moe_route_all(logits, T, E, topk, normalize, R, true, st);
    if (rc) return rc;
  }
  uint16_t *h = (uint16_t *)((uint8_t *)workspace + L.h), *o = (uint16_t *)((uint8_t *)workspace + L.o);
  uint16_t *gu = (uint16_t *)((uint8_t *)workspace + L.gu);
  const uint16_t *sh = (const uint16_t *)shared, *sg = (const uint16_t *)shared_gate;
  MoeAct ma{x_dtype == ISHZ_DT_BF16, nullptr, (uint8_t *)workspace + L.himg};
  if (ma.bf) {  // the model's activations in bf16 (MoEBlock runs in x.dtype): x's fp16 image
    const uint16_t *x16;
    const int rc = act_prepare(x, ISHZ_DT_BF16, T, H, (uint8_t *)workspace + L.ximg, st, &x16, &ma.rsx);
    if (rc) return rc;
    x = x16;
  }
  switch (type) {
  case ISHZ_GGML_Q4_K: return moe_ffn<FQ4_K>(x, T, H, E, I, topk, gate, up, down, rt, h, gu, o, sh, sg, y, st, ma);
  case ISHZ_GGML_Q6_K: return moe_ffn<FQ6_K>(x, T, H, E, I, topk, gate, up, down, rt, h, gu, o, sh, sg, y, st, ma);
  default: return moe_ffn<FQ4_0>(x, T, H, E, I, topk, gate, up, down, rt, h, gu, o, sh, sg, y, st, ma);
  }
}

extern "C" int ishz_moe_swiglu_affine(const void *x, int x_dtype, int T, int H, const float *logits, int E,
                                      int topk, int normalize, const uint32_t *gate_codes,
                                      const void *gate_scales, const void *gate_biases,
                                      const uint32_t *up_codes, const void *up_scales, const void *up_biases,
                                      const uint32_t *down_codes, const void *down_scales,
                                      const void *down_biases, int scale_dtype, int bits, int group, int I,
                                      const void *shared, const void *shared_gate, void *y, int32_t *ids_out,
                                      float *weights_out, void *workspace, size_t workspace_bytes,
                                      ishz_stream_t stream) {
  if (bits < 2 || bits > 8) return decline("affine experts of 2 to 8 bits are decoded in-kernel");
  if (group != 64 && group != 128) return decline("group size must be 64 or 128");
  if (scale_dtype != ISHZ_DT_F16 && scale_dtype != ISHZ_DT_BF16) return decline("scales must be fp16 or bf16");
  if (x_dtype != ISHZ_DT_F16 && x_dtype != ISHZ_DT_BF16) return decline("activations must be fp16 or bf16");
  if (T <= 0 || E <= 0 || topk <= 0 || topk > E || E > 4096) return decline("bad routing shape");
  if (topk > 64 || (size_t)4 * route_row_words(E, topk) * 4 > 160 * 1024)
    return decline("too many experts for one routing workgroup");
  if (H <= 0 || I <= 0 || H % 256 || I % 256) return decline("H and I must be multiples of 256");
  if (!x || !logits || !gate_codes || !gate_scales || !gate_biases || !up_codes || !up_scales || !up_biases ||
      !down_codes || !down_scales || !down_biases || !y)
    return einval("null pointer");
  if (!shared != !shared_gate) return einval("the shared expert needs both its output and its gate");
  const MoeLayout L = moe_layout(T, H, E, I, topk);
  if (!workspace || workspace_bytes < L.total) return einval("workspace too small (ishz_moe_workspace_size)");
  MoeRoute R = moe_route_ptrs(workspace, L);
  R.ids_out = ids_out;
  R.w_out = weights_out;
  hipStream_t st = S(stream);
  const MoeTokens rt{logits, T, E, normalize, R};
  if (!gathered_gemv(T, H, I, topk)) {
    const int rc = moe_route_all(logits, T, E, topk, normalize, R, true, st);
    if (rc) return rc;
  }
  const uint16_t *sh = (const uint16_t *)shared, *sg = (const uint16_t *)shared_gate;
  uint16_t *h = (uint16_t *)((uint8_t *)workspace + L.h), *o = (uint16_t *)((uint8_t *)workspace + L.o);
  uint16_t *gu = (uint16_t *)((uint8_t *)workspace + L.gu);
  const AffPack gp{gate_codes, (const uint16_t *)gate_scales, (const uint16_t *)gate_biases, H * bits / 32, H / group};
  const AffPack upk{up_codes, (const uint16_t *)up_scales, (const uint16_t *)up_biases, H * bits / 32, H / group};
  const AffPack dp{down_codes, (const uint16_t *)down_scales, (const uint16_t *)down_biases, I * bits / 32, I / group};
  const bool bf = scale_dtype == ISHZ_DT_BF16;
  MoeAct ma{x_dtype == ISHZ_DT_BF16, nullptr, (uint8_t *)workspace + L.himg};
  if (ma.bf) {  // bf16 activations: x's fp16 image
    const uint16_t *x16;
    const int rc = act_prepare(x, ISHZ_DT_BF16, T, H, (uint8_t *)workspace + L.ximg, st, &x16, &ma.rsx);
    if (rc) return rc;
    x = x16;
  }
#define ISHZ_MA(B, G)                                                                                          \
  return bf ? moe_ffn_affine<FAffineN<B, G, true>>(x, T, H, E, I, topk, gp, upk, dp, rt, h, gu, o, sh, sg, y, st, \
                                                   ma)                                                        \
            : moe_ffn_affine<FAffineN<B, G, false>>(x, T, H, E, I, topk, gp, upk, dp, rt, h, gu, o, sh, sg, y, st, ma)
  if (bits == 4) {
    if (group == 64) ISHZ_MA(4, 64);
    ISHZ_MA(4, 128);
  }
  if (bits == 8) {
    if (group == 64) ISHZ_MA(8, 64);
    ISHZ_MA(8, 128);
  }
#undef ISHZ_MA
  if (bits <= 3)
    return moe_affine_w23(bits, group, bf, x, T, H, E, I, topk, gp, upk, dp, rt, h, gu, o, sh, sg, y, st, ma);
  return moe_affine_w567(bits, group, bf, x, T, H, E, I, topk, gp, upk, dp, rt, h, gu, o, sh, sg, y, st, ma);
}
#endif  // ISHZ_MOE_BODY_ONLY
