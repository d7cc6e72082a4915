// The streaming M = 1 GEMV skeleton shared by every weight format (GGML blocks, MLX affine).
//
// A workgroup owns a contiguous, equal share of row groups (64/LPR rows each, LPR lanes per row);
// lane `sub` of a row takes units sub, sub + LPR, ... (its slots), so a group is upl unit batches
// (one unit per lane per batch). The workgroup's batches are dealt to its waves in equal contiguous
// ranges, so every wave streams the same number of units to within one; a row split between two
// waves leaves a partial dot from each in LDS, summed in wave order at the end. A wave keeps D - 1
// batches in flight in a register ring; loads are never predicated and every batch a loop
// iteration loads is consumed on every path, so the compiler's waits are for the batch being
// decoded only. The first batches are issued before x is staged into LDS.
//
// A format F provides: Args (pointers and sizes), Raw (one unit's registers), LaneC (per-lane
// constants), units(K), load(args, row, u), dot(raw, UnitX, LaneC), stage_load(...) (x loads
// issued first, kept in an XPre) and stage(...) (fills the LDS slots and sums of x, see UnitX),
// extra_lds_bytes(args), R / Q (slots and sums per unit), RING (the ring depth D) and occ(args)
// (resident waves per SIMD the grid is sized for). A format whose rows read different activation
// vectors (a batch of gathered experts) also provides nx(args), the number of x images (LDS is
// sized for all of them), xsel(args, row), the image a row reads (uniform over a row group), and
// a stage taking the first and last image the workgroup's rows read: only those are staged.
#pragma once
#include <algorithm>
#include <cstdlib>

#include "common.h"

namespace ishz {

// x as a GEMV lane sees it for one unit. The kernel stages x in LDS in the order lanes consume
// it: a unit reads R 16-byte slots (8 fp16 x each) and Q fp32 sums of x. Slot r of unit u lives
// at (u / 16) * 16R + r * 16 + u % 16, so the 16 lanes that read slot r of 16 consecutive units
// in one instruction touch 256 contiguous bytes (every LDS bank once), and a lane's successive
// units differ by a uniform offset (folded into the ds_read immediate).
struct UnitX {
  const u4 *xs;    // slot 0 of the unit; slot r at xs[16 r]
  const float *sm; // sum 0 of the unit; sum q at sm[16 q]
  uint32_t mg;     // 0x64006400 held in a VGPR (magic exponent for code -> fp16)
  const u4 *grid;  // i-quant grid as fp16, pair-permuted like x (IQ2_XS)
  const u4 *sgn;   // i-quant sign masks in the same order (IQ2_XS)
  DEV u4 slot(int r) const { return xs[16 * r]; }
  DEV float sum(int q) const { return sm[16 * q]; }
};

DEV void unpack(u4 a, u4 b, uint32_t *d) {
  d[0] = a.x, d[1] = a.y, d[2] = a.z, d[3] = a.w, d[4] = b.x, d[5] = b.y, d[6] = b.z, d[7] = b.w;
}

// x0..x7 (natural) -> (x0,x2,x1,x3, x4,x6,x5,x7): the order of the nibble/byte pairs a mask
// pulls out of one code word.
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

template <class F>
__host__ __device__ constexpr bool gemv_multi_x() {
  return requires(const typename F::Args &a) { F::nx(a); };
}
template <class F>
__host__ __device__ int gemv_nx(const typename F::Args &a) {
  if constexpr (gemv_multi_x<F>()) return F::nx(a);
  else return 1;
}

// Optional format hooks. prepare(args, lds, xs): runs first, before any weight load, and returns a
// value handed to every load(args, prep, row, u) (the gathered-expert formats route their tokens
// there, so the loads know which expert a row reads). group_align(args, RPW): workgroup row
// ranges start on multiples of this many row groups. store(args, y, row0, nrows, vals): writes
// the workgroup's outputs from their final dots in LDS (vals[i] is row row0 + i), with prepare's
// value as a sixth argument where the format takes one. X_ALL: every x
// image is staged (image i at slot i), not only those of the workgroup's rows.
template <class F>
__host__ __device__ constexpr bool gemv_has_prepare() {
  return requires { &F::prepare; };
}
template <class F>
__host__ __device__ constexpr bool gemv_has_align() {
  return requires(const typename F::Args &a) { F::group_align(a, 1); };
}
template <class F>
__host__ __device__ constexpr bool gemv_has_store() {
  return requires { &F::store; };
}
// Interleaved row groups (see gemv_kernel) for formats without hooks that need contiguous rows:
// 17408 x 5120 on MI355X, Q4_0 13.2 -> 12.3 us, Q4_K 13.7 -> 12.6, Q6_K 18.7 -> 18.0, IQ2_XS
// 14.2 -> 13.7 (the 2-bit affine pack unchanged).
template <class F>
__host__ __device__ constexpr bool gemv_interleaved() {
  return !gemv_has_prepare<F>() && !gemv_has_store<F>() && !gemv_multi_x<F>() && !gemv_has_align<F>();
}
template <class F>
__host__ __device__ int gemv_align(const typename F::Args &a, int rpw) {
  if constexpr (gemv_has_align<F>()) return F::group_align(a, rpw);
  else return 1;
}

// Threads per workgroup: F::WG where the format sets it (the workgroup shares one staged copy of
// x, so a larger one stages fewer copies, each with more waves), else 256; rows of more than 384
// units (BIG: K above 24576 for 64-weight units) take 1024, one workgroup per CU: x is then 50 KB
// and more, and staging it once per CU instead of two to four times measured 10-14 % faster at
// K = 25600 (Q4_K, Q6_K, IQ2_XS, N = 5120) on MI355X. 64 lanes per row also takes 1024.
template <class F, int LPR = 16, bool BIG = false>
__host__ __device__ constexpr int gemv_threads() {
  if constexpr (LPR >= 64 || BIG) return 1024;
  else if constexpr (requires { F::WG; }) return F::WG;
  else return 256;
}

template <class F, int LPR, int D, bool RAGGED, bool BIG = false>
__global__ __launch_bounds__((gemv_threads<F, LPR, BIG>())) void gemv_kernel(typename F::Args args, const uint16_t *__restrict__ x,
                                                   Out out, int nwg, int part_off) {
  static_assert(LPR % 16 == 0, "lanes per row must be a multiple of 16");
  extern __shared__ __align__(16) uint32_t smem[];
  const int K = args.K, N = args.N;
  const int units = F::units(K);
  const int ugroups = (units + 15) / 16;
  const int nx = gemv_nx<F>(args);
  u4 *xs = (u4 *)smem;
  float *xsum = (float *)(xs + nx * ugroups * 16 * F::R);
  u4 *extra = (u4 *)(xsum + nx * ugroups * 16 * F::Q);  // format tables / scratch
  float *part = (float *)((char *)smem + part_off);      // [wave][row of the workgroup] partial dots

  constexpr int RPW = 64 / LPR, WPG = gemv_threads<F, LPR, BIG>() / 64;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int sub = lane % LPR, rg = lane / LPR;
  const int upl = (units + LPR - 1) / LPR;  // units per lane per row
  // workgroup b of nwg owns row groups [b G / nwg, (b + 1) G / nwg) (in units of GA groups);
  // their upl unit batches per group are dealt to its waves in equal contiguous ranges [tb, te)
  const int G = (N + RPW - 1) / RPW, GA = gemv_align<F>(args, RPW), GU = (G + GA - 1) / GA;
  // IL: the workgroup's groups are b, b + nwg, b + 2 nwg, ... (indexed 0 .. ng - 1 here), so at any
  // moment the grid streams one compact window of the matrix rather than nwg separate ranges.
  constexpr bool IL = gemv_interleaved<F>();
  const int gf = IL ? 0 : min((int)((long long)blockIdx.x * GU / nwg) * GA, G);
  const int gend = IL ? (G - (int)blockIdx.x + nwg - 1) / nwg : min((int)((long long)(blockIdx.x + 1) * GU / nwg) * GA, G);
  auto phys = [&](int g) { return IL ? (int)blockIdx.x + g * nwg : g; };
  const int T = (gend - gf) * upl, nrows = (gend - gf) * RPW;
  const int tb = T * wave / WPG, te = T * (wave + 1) / WPG;
  const typename F::LaneC lc = F::lane(sub);

  // Unit of slot k of a lane's row; with RAGGED, a slot past the row's units reloads its last unit.
  auto unit = [&](int k) {
    if constexpr (RAGGED) return min(sub + k * LPR, units - 1);
    return sub + k * LPR;
  };
  // Batch t = (group g, slot k). A batch past the wave's last (the ring runs ahead of the consumer
  // by D - 1) loads row 0's first unit on every lane: one cache line, never consumed.
  const auto prep = [&] {
    if constexpr (gemv_has_prepare<F>()) return F::prepare(args, extra, xs);
    else return 0;
  }();
  auto load_b = [&](int t, int g, int k, typename F::Raw &r) {
    const bool live = t < te;
    const int row = live ? min(phys(g) * RPW + rg, N - 1) : 0, u = live ? unit(k) : 0;
    if constexpr (gemv_has_prepare<F>()) r = F::load(args, prep, row, u);
    else r = F::load(args, row, u);
  };
  auto advance = [&](int &g, int &k) {
    if (++k == upl) {
      k = 0;
      g++;
    }
  };

  // Ring of D register batches: batch t sits in buf[(t - tb) % D]; before batch t is consumed,
  // batch t + D - 1 is issued into the slot batch t - 1 freed. Every batch a loop iteration loads
  // is consumed on every path through the loop and results go to LDS, so the compiler's waits are
  // for the batch being consumed only (a load left pending across the back edge, or a global
  // store between loads, would make it wait for everything). x's first staging loads go out
  // before the weight batches: the memory counter is in order, so staging waits only for x.
#ifdef ISHZ_TIMING
  uint64_t ts[5];
  ts[0] = __builtin_amdgcn_s_memrealtime();
#endif
  const typename F::XPre pre = F::stage_load(args, x, units);
  typename F::Raw buf[D];
  int gl = gf + (T ? tb / upl : 0), kl = T ? tb % upl : 0;
  const int gc0 = gl, kc0 = kl;
#pragma unroll
  for (int d = 0; d < D - 1; d++) {
    load_b(tb + d, gl, kl, buf[d]);
    advance(gl, kl);
  }

  // after the first loads are out (visible after staging's barrier)
  for (int i = threadIdx.x; i < WPG * nrows; i += WPG * 64) part[i] = 0.0f;
  int im0 = 0;  // first x image of this workgroup's rows
  if constexpr (requires { F::X_ALL; }) {  // every image staged, image i at slot i
    F::stage(args, x, xs, xsum, extra, units, pre, 0, nx - 1);
  } else if constexpr (gemv_multi_x<F>()) {
    im0 = F::xsel(args, min(gf * RPW, N - 1));
    F::stage(args, x, xs, xsum, extra, units, pre, im0, F::xsel(args, min(max(gend * RPW - 1, gf * RPW), N - 1)));
  } else {
    F::stage(args, x, xs, xsum, extra, units, pre);  // ends with a barrier
  }
#ifdef ISHZ_TIMING
  ts[1] = ts[2] = ts[3] = __builtin_amdgcn_s_memrealtime();
#endif
  const uint32_t mg = vconst(0x64006400u);
  const u4 *grid = extra, *sgn = extra + F::GRID_ENTRIES;
  auto view = [&](int g, int k) {
    int xo = 0, so = 0;  // the group's x image
    if constexpr (gemv_multi_x<F>()) {
      const int im = F::xsel(args, g * RPW) - im0;
      xo = im * ugroups * 16 * F::R;
      so = im * ugroups * 16 * F::Q;
    }
    const int u = unit(k);
    return UnitX{xs + xo + (u >> 4) * 16 * F::R + (u & 15), xsum + so + (u >> 4) * 16 * F::Q + (u & 15), mg, grid, sgn};
  };

  // RAGGED slots past the row's units are decoded (from a real unit) and masked out, never
  // branched around: see the ring above. A row's partial goes to LDS at its last slot or at the
  // wave's last batch.
  float acc = 0.0f;
  auto consume = [&](int t, int g, int k, const typename F::Raw &r) {
    const float v = F::dot(r, view(g, k), lc);
    if constexpr (RAGGED) acc += sub + k * LPR < units ? v : 0.0f;
    else acc += v;
    if (k == upl - 1 || t == te - 1) {
      const float s = group_sum<LPR>(acc);
      if (sub == 0) part[wave * nrows + (g - gf) * RPW + rg] = s;
      acc = 0.0f;
    }
  };
  int gc = gc0, kc = kc0, t = tb;
  for (; t + D <= te; t += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      load_b(t + d + D - 1, gl, kl, buf[(d + D - 1) % D]);
      advance(gl, kl);
      consume(t + d, gc, kc, buf[d]);
      advance(gc, kc);
    }
  }
  // the last (te - tb) % D batches are already in buf[0 ..]
#pragma unroll
  for (int d = 0; d < D - 1; d++)
    if (t + d < te) {
      consume(t + d, gc, kc, buf[d]);
      advance(gc, kc);
    }

#ifdef ISHZ_TIMING
  ts[4] = __builtin_amdgcn_s_memrealtime();
  if (lane == 0)
    for (int i = 0; i < 5; i++) ishz_timing[(blockIdx.x * WPG + wave) * 5 + i] = ts[i];
#endif
  // Each output: the partials of the waves whose batch ranges meet its group, in wave order.
  __syncthreads();
  for (int i = threadIdx.x; i < nrows; i += WPG * 64) {
    const int b0 = (i / RPW) * upl, b1 = b0 + upl - 1;
    const int w0 = (WPG * (b0 + 1) - 1) / T, w1 = (WPG * (b1 + 1) - 1) / T;  // waves holding b0, b1
    float s = 0.0f;
    for (int w = w0; w <= w1; w++) s += part[w * nrows + i];
    if constexpr (gemv_has_store<F>()) part[i] = s;  // only this thread reads row i's partials
    else if (IL) {
      const int r = phys(i / RPW) * RPW + i % RPW;
      if (r < N) out.put(r, 0, s);
    } else if (gf * RPW + i < N) out.put(gf * RPW + i, 0, s);
  }
  if constexpr (gemv_has_store<F>()) {
    __syncthreads();
    if constexpr (requires { F::store(args, (uint16_t *)out.y, 0, 0, part, prep); })
      F::store(args, (uint16_t *)out.y, gf * RPW, min(nrows, N - gf * RPW), part, prep);
    else
      F::store(args, (uint16_t *)out.y, gf * RPW, min(nrows, N - gf * RPW), part);
  }
}

int gemv_num_cu();

// Grid: one resident round of workgroups (at most what the compiled kernel's registers and this
// launch's LDS allow), each an equal share of row groups. LDS: the staged x images and sums, the
// format's tables, then the waves' partial dots for the workgroup's rows.
template <class F, int LPR, bool RAGGED, bool BIG = false>
static int launch_gemv_k(const typename F::Args &a, const void *x, const Out &o, hipStream_t st) {
  constexpr int RPW = 64 / LPR;
  constexpr int NT = gemv_threads<F, LPR, BIG>(), WPG = NT / 64;
  const int units = F::units(a.K);
  const size_t ug = (size_t)(units + 15) / 16;
  const size_t xlds = gemv_nx<F>(a) * (ug * 16 * F::R * 16 + ug * 16 * F::Q * 4) + F::extra_lds_bytes(a);
  const size_t part_off = (xlds + 15) / 16 * 16;
  if (part_off > 160 * 1024) return decline("K too large for the GEMV's LDS copy of x");
  auto kern = gemv_kernel<F, LPR, F::RING, RAGGED, BIG>;
  const int GA = gemv_align<F>(a, RPW), groups = (a.N + RPW - 1) / RPW, units_g = (groups + GA - 1) / GA;
  const int wg_cap = std::max(F::occ(a) * 4 / WPG, 1);  // workgroups per CU the grid is sized for
  int nwg = 0;
  size_t lds = 0;
  // the rows per workgroup depend on the workgroup count, and the occupancy on the LDS: settle both
  for (int per_cu = wg_cap, it = 0; it < 3; it++) {
    nwg = std::min(gemv_num_cu() * std::min(per_cu, wg_cap), units_g);
    const size_t rows = (size_t)(units_g + nwg - 1) / nwg * GA * RPW;
    lds = part_off + WPG * rows * 4;
    if (lds > 160 * 1024) {  // very tall outputs: more workgroups, several rounds
      const size_t room = (160 * 1024 - part_off) / (WPG * 4 * RPW * (size_t)GA);
      if (room < 1) return decline("no LDS left for the GEMV's partial sums");
      nwg = std::min((int)((units_g + room - 1) / room), units_g);
      lds = part_off + WPG * ((size_t)(units_g + nwg - 1) / nwg * GA * RPW) * 4;
      break;
    }
    int pc = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&pc, kern, NT, lds) != hipSuccess || pc < 1) pc = 1;
    if (pc >= per_cu || pc >= wg_cap) break;
    per_cu = pc;
  }
  hipLaunchKernelGGL(kern, dim3(nwg), dim3(NT), lds, st, a, (const uint16_t *)x, o, nwg, (int)part_off);
  ISHZ_LAUNCH_CHECK("gemv launch");
  return ISHZ_OK;
}

// Lanes per row: 16 for rows of up to 160 units, 32 up to 384; longer rows take 16 again, in
// 1024-thread workgroups (at K = 25600, N = 5120 on MI355X: Q4_K 20.7 -> 19.8 us, Q6_K 28.0 ->
// 27.5, IQ2_XS 20.4 -> 18.8 against 64 lanes per row, whose last slot was 12 % padding). RAGGED:
// the row's units are not a whole number of every lane's slots. x is fp16 (or an activation image, with its row
// factor in rs); y in dtype odt.
template <class F>
static int launch_gemv(const typename F::Args &a, const void *x, void *y, hipStream_t st, int odt = ISHZ_DT_F16,
                       const float *rs = nullptr) {
  const int units = F::units(a.K);
  const Out o{y, odt, rs};
  if (units <= 160) return units % 16 ? launch_gemv_k<F, 16, true>(a, x, o, st) : launch_gemv_k<F, 16, false>(a, x, o, st);
  if (units <= 384) return units % 32 ? launch_gemv_k<F, 32, true>(a, x, o, st) : launch_gemv_k<F, 32, false>(a, x, o, st);
  return units % 16 ? launch_gemv_k<F, 16, true, true>(a, x, o, st) : launch_gemv_k<F, 16, false, true>(a, x, o, st);
}

}  // namespace ishz
