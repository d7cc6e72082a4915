// MoE expert-gathered quantized SwiGLU FFN on gfx950.
//
// Restates MoEBlock.callAsFunction + ResidentExperts.swiglu (Sources/IshizukiKit/Text/
// MoEBlock.swift:124-171) over GGML-block experts: softmax over all E experts in fp32, top-k
// (ties to the lower index), optional renormalisation, then per (token, expert)
// down(silu(gate(x)) * up(x)), the k outputs weighted and summed in fp32, narrowed once.
// Activations between stages are fp16 as the reference's gatherQuantizedMM outputs x.dtype.
//
// Kernels: route (one workgroup: routing, per-expert pair lists, active-expert list); gate+up
// (grid over active experts x 16-row tiles of I; the expert's gate and up rows are two MFMA
// tiles of the same workgroup, tokens gathered through the pair list; SwiGLU in the epilogue);
// down (active experts x tiles of H); combine (weighted sum per token). Only routed experts'
// blocks are ever read.
#include <algorithm>
#include <cstdlib>

#include "ggml_formats.h"
#include "vgemm.h"

namespace ishz {

struct MoeRoute {
  int32_t *ids;       // [T*k] expert of (t, s)
  float *w;           // [T*k] routing weight of (t, s)
  int32_t *count;     // [1] number of active experts
  int32_t *active;    // [E] active experts, ascending
  int32_t *offs;      // [E+1] pair range of expert e in the sorted list
  int32_t *pair_tok;  // [T*k] token of sorted pair
  int32_t *inv;       // [T*k] sorted position of (t, s)
};

// Routing ranks each expert against the token's whole logit row (rank = experts with a larger
// logit, or an equal one at a lower index): the top-k are the experts of rank < k, already in the
// reference's order (logit descending, ties to the lower index). Softmax max and sum are wave
// reductions; the top-k probabilities are summed in rank order for the renormalisation.
DEV float wave_max(float v) {
  v = fmaxf(v, ISHZ_DPP(v, 0xB1));
  v = fmaxf(v, ISHZ_DPP(v, 0x4E));
  v = fmaxf(v, ISHZ_DPP(v, 0x141));
  v = fmaxf(v, ISHZ_DPP(v, 0x140));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

// Routing: one 64-lane workgroup per token, so tokens route in parallel.
__global__ __launch_bounds__(64) void moe_route_kernel(const float *__restrict__ logits, int T, int E,
                                                       int k, int normalize, MoeRoute R) {
  extern __shared__ __align__(16) float rowb[];  // the token's logits, padded to whole float4; then 64 probs
  const int lane = threadIdx.x, t = blockIdx.x;
  const int E4 = (E + 3) & ~3;
  float *pb = rowb + E4;
  const float *l = logits + (size_t)t * E;
  float mx = -INFINITY;
  for (int e = lane; e < E4; e += 64) {
    const float v = e < E ? l[e] : -INFINITY;  // -inf never ranks above a logit
    rowb[e] = v;
    mx = fmaxf(mx, v);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
  for (int e = lane; e < E; e += 64) sum += expf(rowb[e] - mx);
  sum = group_sum<64>(sum);
  __syncthreads();
  for (int e = lane; e < E; e += 64) {
    const float v = rowb[e];
    int rank = 0;
#pragma unroll 8
    for (int f = 0; f < E4; f += 4) {
      const f4 u = *(const f4 *)(rowb + f);
#pragma unroll
      for (int c = 0; c < 4; c++) rank += (u[c] > v) | ((u[c] == v) & (f + c < e));
    }
    if (rank < k) {
      R.ids[t * k + rank] = e;
      pb[rank] = expf(v - mx) / sum;
    }
  }
  __syncthreads();
  float tot = 0.0f;  // rank-order sum of the top-k probabilities
  for (int s = 0; s < k; s++) tot += pb[s];
  if (lane < k) {
    const float p = pb[lane];
    R.w[t * k + lane] = normalize ? p / tot : p;
  }
}

// Pair lists (one workgroup): per-expert counts in LDS, an exclusive prefix over experts by wave
// 0, then each pair takes the next free position of its expert (the order inside an expert does
// not affect any result: every pair's rows are computed independently).
__global__ __launch_bounds__(1024) void moe_place_kernel(int T, int E, int k, MoeRoute R) {
  extern __shared__ int32_t cnt[];  // E counts, then fill cursors
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int P = T * k;
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int q = threadIdx.x; q < P; q += blockDim.x) atomicAdd(&cnt[R.ids[q]], 1);
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
    const int pos = atomicAdd(&cnt[R.ids[q]], 1);
    R.pair_tok[pos] = q / k;
    R.inv[q] = pos;
  }
}

DEV float r16(float v) { return (float)(_Float16)v; }

// gate + up for one 16-row tile of I of one active expert, 16 routed tokens at a time.
template <class F>
__global__ __launch_bounds__(1024) void moe_gate_up_kernel(const uint16_t *__restrict__ x, int H,
                                                           const uint8_t *__restrict__ gate,
                                                           const uint8_t *__restrict__ up, int I,
                                                           MoeRoute R, uint16_t *__restrict__ h) {
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
    const uint16_t *xr = x + (size_t)(tok ? R.pair_tok[c0 + j] : 0) * H;
    f4 acc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
    for (int b = wave; b < nblk; b += KS) F::template vblock<2>(rows, b, g, xr, tok, acc);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[((wave * 2 + t) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    for (int o = threadIdx.x; o < 256; o += blockDim.x) {
      const int r = o >> 6, l = o & 63;
      float gs = 0.0f, us = 0.0f;
      for (int v = 0; v < KS; v++) {
        gs += red[((v * 2 + 0) * 4 + r) * 64 + l];
        us += red[((v * 2 + 1) * 4 + r) * 64 + l];
      }
      const int t = 4 * (l >> 4) + r, i = i0 + (l & 15);
      if (c0 + t < p1 && i < I) {
        const float g16 = r16(gs), u16 = r16(us);
        const float sg = r16(1.0f / (1.0f + __expf(-g16)));
        h[(size_t)(c0 + t) * I + i] = f2h(r16(g16 * sg) * u16);
      }
    }
    __syncthreads();
  }
}

// down projection: o[pair][H] = h[pair] . down_e^T, fp16.
template <class F>
__global__ __launch_bounds__(1024) void moe_down_kernel(const uint16_t *__restrict__ h, int I,
                                                        const uint8_t *__restrict__ down, int H,
                                                        MoeRoute R, uint16_t *__restrict__ o) {
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
    for (int q = threadIdx.x; q < 512; q += blockDim.x) {
      const int t2 = q >> 8, r = (q >> 6) & 3, l = q & 63;
      float s = 0.0f;
      for (int v = 0; v < KS; v++) s += red[((v * 2 + t2) * 4 + r) * 64 + l];
      const int t = 4 * (l >> 4) + r, n = n0 + 16 * t2 + (l & 15);
      if (c0 + t < p1 && n < H) o[(size_t)(c0 + t) * H + n] = f2h(s);
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t *__restrict__ o, int H,
                                                          int T, int k, MoeRoute R,
                                                          uint16_t *__restrict__ y) {
  const size_t total = (size_t)T * H;
  for (size_t q = blockIdx.x * (size_t)blockDim.x + threadIdx.x; q < total;
       q += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(q / H), n = (int)(q % H);
    float acc = 0.0f;
    for (int s = 0; s < k; s++) acc += h2f(o[(size_t)R.inv[t * k + s] * H + n]) * R.w[t * k + s];
    y[q] = f2h(acc);
  }
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
  DEV const uint16_t *xrow(const Group &g, int tk) const { return x + (size_t)R.pair_tok[g.p0 + tk] * H; }
  DEV const uint8_t *wrow(const Group &g, int row) const {
    const int tile = row >> 4, i = min((tile >> 1) * 16 + (row & 15), I - 1);
    return ((tile & 1) ? up : gate) + ((size_t)g.e * I + i) * rb;
  }
  DEV void finish(const Group &g, int c0, int m, int tb, int te, const float *out) const {
    for (int o = threadIdx.x; o < (te - tb) / 2 * 256; o += blockDim.x) {
      const int pr = o >> 8, tk = (o >> 4) & 15, nn = o & 15;
      const int i = ((tb >> 1) + pr) * 16 + nn;
      if (tk < m && i < I) {
        const float g16 = r16(out[(2 * pr) * 256 + tk * 16 + nn]), u16 = r16(out[(2 * pr + 1) * 256 + tk * 16 + nn]);
        const float sg = r16(1.0f / (1.0f + __expf(-g16)));
        h[(size_t)(g.p0 + c0 + tk) * I + i] = f2h(r16(g16 * sg) * u16);
      }
    }
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
    for (int q = threadIdx.x; q < (te - tb) * 256; q += blockDim.x) {
      const int tk = (q >> 4) & 15, row = (tb + (q >> 8)) * 16 + (q & 15);
      if (tk < m && row < H) o[(size_t)(g.p0 + c0 + tk) * H + row] = f2h(out[q]);
    }
  }
};

// Token quads per pass: an expert receives at most T tokens (one slot per token).
template <class F, class P>
static int moe_vgemm(const P &p, int T, int K, int rows, int groups, int tiles_per_wg, hipStream_t st) {
  switch (std::min(4, (T + 3) / 4)) {
    case 1: return launch_vgemm_p<F, P, 1>(p, K, rows, groups, tiles_per_wg, st);
    case 2: return launch_vgemm_p<F, P, 2>(p, K, rows, groups, tiles_per_wg, st);
    case 3: return launch_vgemm_p<F, P, 3>(p, K, rows, groups, tiles_per_wg, st);
    default: return launch_vgemm_p<F, P, 4>(p, K, rows, groups, tiles_per_wg, st);
  }
}

// ------------------------------------------------------------------- host
struct MoeLayout {
  size_t ids, w, count, active, offs, pair_tok, inv, h, o, total;
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
  L.pair_tok = off; off += al(P * 4);
  L.inv = off; off += al(P * 4);
  L.h = off; off += al(P * I * 2);
  L.o = off; off += al(P * H * 2);
  L.total = off;
  return L;
}

static MoeRoute moe_route_ptrs(void *ws, const MoeLayout &L) {
  uint8_t *b = (uint8_t *)ws;
  return MoeRoute{(int32_t *)(b + L.ids), (float *)(b + L.w), (int32_t *)(b + L.count),
                  (int32_t *)(b + L.active), (int32_t *)(b + L.offs), (int32_t *)(b + L.pair_tok),
                  (int32_t *)(b + L.inv)};
}

static int ks_for(int tiles, int nblk) {
  int ks = 1;
  while (ks < 16 && ks < nblk && tiles * ks < 256 * 16) ks *= 2;
  return ks;
}

template <class F>
static int moe_ffn(const void *x, int T, int H, int E, int I, int k, const void *gate,
                   const void *up, const void *down, MoeRoute R, uint16_t *h, uint16_t *o, void *y,
                   hipStream_t st) {
  const int amax = std::min(E, T * k);
  static const bool old = getenv("ISHZ_OLD_MOE") != nullptr;
  // streaming MFMA kernels from 3 tokens up; one or two tokens (a GEMV per expert) run faster on
  // the per-block kernels below, which start streaming without staging x
  if (H % 256 == 0 && I % 256 == 0 && T > 2 && !old) {
    // tiles per workgroup: about two workgroups per CU over the routed experts (gate/up: an even
    // count, whole SwiGLU pairs); with 8 or more a wave takes whole tiles
    const int tiles_gu = 2 * ((I + 15) / 16), tiles_dn = (H + 15) / 16;
    const int act = std::min(amax, 128);
    auto pick = [&](int tiles, int even) {
      int t = std::max(1, std::min(32, tiles * act / (gemv_num_cu() * 2)));
      if (even) t = std::max(2, t & ~1);
      return t;
    };
    const VMoeGateUp gu{(const uint16_t *)x, (const uint8_t *)gate, (const uint8_t *)up,
                        (size_t)(H / F::BS) * F::TS, H, I, R, h};
    int rc = moe_vgemm<F>(gu, T, H, tiles_gu * 16, amax, pick(tiles_gu, 1), st);
    if (rc) return rc;
    const VMoeDown dn{h, (const uint8_t *)down, (size_t)(I / F::BS) * F::TS, I, H, R, o};
    rc = moe_vgemm<F>(dn, T, I, H, amax, pick(tiles_dn, 0), st);
    if (rc) return rc;
  } else {
    int ks = ks_for((I / 16) * amax, H / F::BS);
    hipLaunchKernelGGL((moe_gate_up_kernel<F>), dim3(I / 16, amax), dim3(64 * ks), (size_t)ks * 2 * 256 * 4, st,
                       (const uint16_t *)x, H, (const uint8_t *)gate, (const uint8_t *)up, I, R, h);
    ISHZ_LAUNCH_CHECK("moe gate/up launch");
    ks = ks_for((H / 32) * amax, I / F::BS);
    hipLaunchKernelGGL((moe_down_kernel<F>), dim3((H + 31) / 32, amax), dim3(64 * ks), (size_t)ks * 2 * 256 * 4,
                       st, h, I, (const uint8_t *)down, H, R, o);
    ISHZ_LAUNCH_CHECK("moe down launch");
  }
  const size_t total = (size_t)T * H;
  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)std::min<size_t>((total + 255) / 256, 4096)), dim3(256), 0,
                     st, o, H, T, k, R, (uint16_t *)y);
  ISHZ_LAUNCH_CHECK("moe combine launch");
  return ISHZ_OK;
}

}  // namespace ishz

using namespace ishz;

extern "C" size_t ishz_moe_workspace_size(int T, int H, int E, int I, int topk) {
  return moe_layout(T, H, E, I, topk).total;
}

extern "C" int ishz_moe_route(const float *logits, int T, int E, int topk, int normalize,
                              int32_t *ids, float *weights, ishz_stream_t stream) {
  if (T <= 0 || E <= 0 || topk <= 0 || topk > E || topk > 64) return decline("bad routing shape");
  if ((size_t)(E + 3 + 64) * 4 > 64 * 1024) return decline("too many experts for one routing workgroup");
  if (!logits || !ids || !weights) return einval("null pointer");
  MoeRoute R{ids, weights, nullptr, nullptr, nullptr, nullptr, nullptr};
  hipLaunchKernelGGL(moe_route_kernel, dim3(T), dim3(64), (size_t)(E + 3 + 64) * 4, S(stream), logits, T, E, topk,
                     normalize, R);
  ISHZ_LAUNCH_CHECK("moe route launch");
  return ISHZ_OK;
}

extern "C" int ishz_moe_swiglu(uint32_t type, const void *x, int x_dtype, int T, int H,
                               const float *logits, int E, int topk, int normalize,
                               const void *gate, const void *up, const void *down,
                               size_t expert_bytes, int I, void *y, int32_t *ids_out,
                               float *weights_out, void *workspace, size_t workspace_bytes,
                               ishz_stream_t stream) {
  const int bs = ishz_ggml_block_size(type);
  if (type != ISHZ_GGML_Q4_K && type != ISHZ_GGML_Q6_K && type != ISHZ_GGML_Q4_0)
    return decline("MoE experts must be Q4_0, Q4_K or Q6_K");
  if (x_dtype != ISHZ_DT_F16) return decline("activations must be fp16");
  if (T <= 0 || E <= 0 || topk <= 0 || topk > E || E > 4096) return decline("bad routing shape");
  if (topk > 64 || (size_t)(E + 3 + 64) * 4 > 64 * 1024) return decline("too many experts for one routing workgroup");
  if (H <= 0 || I <= 0 || H % bs || I % bs) return decline("H and I must be whole blocks");
  const size_t need = (size_t)I * (H / bs) * ishz_ggml_type_size(type);
  if (expert_bytes < need || (size_t)H * (I / bs) * ishz_ggml_type_size(type) > expert_bytes)
    return decline("expert buffers too short");
  if (!x || !logits || !gate || !up || !down || !y) return einval("null pointer");
  const MoeLayout L = moe_layout(T, H, E, I, topk);
  if (!workspace || workspace_bytes < L.total) return einval("workspace too small (ishz_moe_workspace_size)");
  MoeRoute R = moe_route_ptrs(workspace, L);
  hipStream_t st = S(stream);
  hipLaunchKernelGGL(moe_route_kernel, dim3(T), dim3(64), (size_t)(E + 3 + 64) * 4, st, logits, T, E, topk,
                     normalize, R);
  ISHZ_LAUNCH_CHECK("moe route launch");
  hipLaunchKernelGGL(moe_place_kernel, dim3(1), dim3(1024), (size_t)E * 4, st, T, E, topk, R);
  ISHZ_LAUNCH_CHECK("moe place launch");
  uint16_t *h = (uint16_t *)((uint8_t *)workspace + L.h), *o = (uint16_t *)((uint8_t *)workspace + L.o);
  int rc;
  switch (type) {
  case ISHZ_GGML_Q4_K: rc = moe_ffn<FQ4_K>(x, T, H, E, I, topk, gate, up, down, R, h, o, y, st); break;
  case ISHZ_GGML_Q6_K: rc = moe_ffn<FQ6_K>(x, T, H, E, I, topk, gate, up, down, R, h, o, y, st); break;
  default: rc = moe_ffn<FQ4_0>(x, T, H, E, I, topk, gate, up, down, R, h, o, y, st); break;
  }
  if (rc) return rc;
  if (ids_out && hipMemcpyAsync(ids_out, R.ids, (size_t)T * topk * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
    return fail("moe ids copy", hipGetLastError());
  if (weights_out && hipMemcpyAsync(weights_out, R.w, (size_t)T * topk * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
    return fail("moe weights copy", hipGetLastError());
  return ISHZ_OK;
}
