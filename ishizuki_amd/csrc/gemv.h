// The streaming M = 1 GEMV skeleton shared by every weight format (GGML blocks, MLX affine).
//
// A wave owns a contiguous, equal share of row groups (64/LPR rows each, LPR lanes per row) and
// streams their units as one sequence: lane `sub` takes units sub, sub + LPR, ... of each row, in
// batches of B units held in a ring of D register batches, so D - 1 batches' loads are in
// flight while one is decoded. Loads are never predicated: a batch slot is valid for all lanes or none
// (unless RAGGED), and an invalid slot reloads the lane's first unit, so the waitcnt pass only
// waits for the batch being decoded. The first batches are issued before x is staged into LDS.
//
// A format F provides: Args (pointers and sizes), Raw (one unit's registers), LaneC (per-lane
// constants), units(K), load(args, row, u), dot(raw, UnitX, LaneC), stage_load(...) (x loads
// issued first, kept in an XPre) and stage(...) (fills the LDS slots and sums of x, see UnitX),
// extra_lds_bytes(args), and R / Q (slots and sums per unit). A format whose rows read different
// activation vectors (a batch of gathered experts) also provides nx(args), the number of x
// images (LDS is sized for all of them), xsel(args, row), the image a row reads (uniform over a
// row group), and a stage taking the first and last image the workgroup's rows read: only those
// are staged.
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

// Threads per workgroup: F::WG where the format sets it (the workgroup shares one staged copy of
// x, so a larger one stages fewer copies, each with more waves), else 256.
template <class F>
__host__ __device__ constexpr int gemv_threads() {
  if constexpr (requires { F::WG; }) return F::WG;
  else return 256;
}

template <class F, int LPR, int B, int D, bool RAGGED>
__global__ __launch_bounds__(gemv_threads<F>()) void gemv_kernel(typename F::Args args, const uint16_t *__restrict__ x,
                                                   uint16_t *__restrict__ y, int nwaves) {
  static_assert(LPR % 16 == 0, "lanes per row must be a multiple of 16");
  extern __shared__ __align__(16) uint32_t smem[];
  const int K = args.K, N = args.N;
  const int units = F::units(K);
  const int ugroups = (units + 15) / 16;
  const int nx = gemv_nx<F>(args);
  u4 *xs = (u4 *)smem;
  float *xsum = (float *)(xs + nx * ugroups * 16 * F::R);
  u4 *extra = (u4 *)(xsum + nx * ugroups * 16 * F::Q);  // format tables / scratch

  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int sub = lane % LPR, rg = lane / LPR;
  const int nb = (units + B * LPR - 1) / (B * LPR);  // batches per row
  const int gw = blockIdx.x * (blockDim.x >> 6) + wave;
  // wave gw of nwaves owns row groups [gw G / nwaves, (gw + 1) G / nwaves): every wave, and so
  // every CU of a full round, gets the same share to within one group
  const int G = (N + RPW - 1) / RPW;
  auto gstart = [&](int w) { return (int)((long long)min(w, nwaves) * G / nwaves); };
  const int g_end = gstart(gw + 1);
  const int g_last = max(g_end - 1, 0);
  const typename F::LaneC lc = F::lane(sub);

  // Unit of batch slot i; an invalid slot (past the row's units) reloads the lane's first unit.
  auto unit = [&](int bb, int i) {
    const int k = bb * B + i;
    if constexpr (RAGGED) return min(sub + k * LPR, units - 1);
    return sub + (k * LPR < units ? k : 0) * LPR;
  };
  auto load_batch = [&](int g, int bb, typename F::Raw *r) {
    const int row = min(min(g, g_last) * RPW + rg, N - 1);
#pragma unroll
    for (int i = 0; i < B; i++) r[i] = F::load(args, row, unit(bb, i));
  };

  // Ring of D register batches: batch i sits in buf[i % D]; before batch i is decoded, batch
  // i + D - 1 is issued into the slot batch i - 1 freed. Load and consume cursors (group,
  // batch-in-row) advance in step. x's first staging loads go out before the weight batches:
  // the memory counter is in order, so staging then waits only for x.
  const int g0 = gstart(gw);
  auto advance = [&](int &gg, int &bb) {
    if (++bb == nb) {
      bb = 0;
      gg++;
    }
  };
  const typename F::XPre pre = F::stage_load(args, x, units);
  typename F::Raw buf[D][B];
  int gl = g0, bl = 0;
#pragma unroll
  for (int d = 0; d < D - 1; d++) {
    load_batch(gl, bl, buf[d]);
    advance(gl, bl);
  }

  int im0 = 0;  // first x image of this workgroup's rows
  if constexpr (gemv_multi_x<F>()) {
    const int gfirst = gstart(blockIdx.x * (blockDim.x >> 6));
    const int glast = max(gstart((blockIdx.x + 1) * (blockDim.x >> 6)) - 1, gfirst);
    im0 = F::xsel(args, gfirst * RPW);
    F::stage(args, x, xs, xsum, extra, units, pre, im0, F::xsel(args, min(glast * RPW + RPW - 1, N - 1)));
  } else {
    F::stage(args, x, xs, xsum, extra, units, pre);  // ends with a barrier
  }
  const uint32_t mg = vconst(0x64006400u);
  const u4 *grid = extra, *sgn = extra + F::GRID_ENTRIES;
  const int lane_slot = (sub >> 4) * 16 * F::R + (sub & 15);
  const int lane_sum = (sub >> 4) * 16 * F::Q + (sub & 15);
  auto view = [&](int gg, int bb, int i) {
    int xo = 0, so = 0;  // the group's x image
    if constexpr (gemv_multi_x<F>()) {
      const int im = F::xsel(args, gg * RPW) - im0;
      xo = im * ugroups * 16 * F::R;
      so = im * ugroups * 16 * F::Q;
    }
    if constexpr (RAGGED) {
      const int u = unit(bb, i);
      return UnitX{xs + xo + (u >> 4) * 16 * F::R + (u & 15), xsum + so + (u >> 4) * 16 * F::Q + (u & 15), mg, grid,
                   sgn};
    } else {
      const int k = bb * B + i;
      return UnitX{xs + xo + lane_slot + k * LPR * F::R, xsum + so + lane_sum + k * LPR * F::Q, mg, grid, sgn};
    }
  };

  float acc = 0.0f;
  auto consume = [&](int gg, int bb, const typename F::Raw *r) {
#pragma unroll
    for (int i = 0; i < B; i++) {
      if constexpr (RAGGED) {
        const float v = F::dot(r[i], view(gg, bb, i), lc);
        acc += sub + (bb * B + i) * LPR < units ? v : 0.0f;
      } else if ((bb * B + i) * LPR < units) {
        acc += F::dot(r[i], view(gg, bb, i), lc);
      }
    }
    if (bb == nb - 1) {
      acc = group_sum<LPR>(acc);
      const int row = gg * RPW + rg;
      if (sub == 0 && row < N) y[row] = f2h(acc);
      acc = 0.0f;
    }
  };
  int gc = g0, bc = 0;
  while (gc < g_end) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      load_batch(gl, bl, buf[(d + D - 1) % D]);
      advance(gl, bl);
      if (gc < g_end) consume(gc, bc, buf[d]);
      advance(gc, bc);
    }
  }
}

int gemv_num_cu();
int gemv_batch_override();  // ISHZ_GEMV_B (tuning)
int gemv_occ_override();    // ISHZ_GEMV_OCC: resident waves per SIMD the grid is sized for (tuning)

// Grid: one resident round of waves (at most what the compiled kernel's registers and this
// launch's LDS allow), each wave an equal share of row groups.
template <class F, int LPR, int B, int D, bool RAGGED>
static int launch_gemv_kd(const typename F::Args &a, const void *x, void *y, hipStream_t st) {
  constexpr int RPW = 64 / LPR;
  const int units = F::units(a.K);
  const size_t ug = (size_t)(units + 15) / 16;
  const size_t lds = gemv_nx<F>(a) * (ug * 16 * F::R * 16 + ug * 16 * F::Q * 4) + F::extra_lds_bytes(a);
  if (lds > 160 * 1024) return decline("K too large for the GEMV's LDS copy of x");
  auto kern = gemv_kernel<F, LPR, B, D, RAGGED>;
  constexpr int NT = gemv_threads<F>(), WPG = NT / 64;
  int per_cu = 0;  // workgroups per CU, so per_cu * WPG / 4 waves per SIMD
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NT, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int groups = (a.N + RPW - 1) / RPW;
  const int occ = gemv_occ_override() > 0 ? gemv_occ_override() : F::occ(a);
  const int capacity = gemv_num_cu() * 4 * std::min(occ, std::max(per_cu * WPG / 4, 1));
  const int waves = std::min(capacity, groups);  // one resident round, groups spread evenly
  hipLaunchKernelGGL(kern, dim3((waves + WPG - 1) / WPG), dim3(NT), lds, st, a, (const uint16_t *)x, (uint16_t *)y,
                     waves);
  ISHZ_LAUNCH_CHECK("gemv launch");
  return ISHZ_OK;
}

int gemv_depth_override();  // ISHZ_GEMV_D (tuning)

template <class F, int LPR, int B, bool RAGGED>
static int launch_gemv_k(const typename F::Args &a, const void *x, void *y, hipStream_t st) {
  switch (gemv_depth_override() ? gemv_depth_override() : F::DEPTH) {
    case 4: return launch_gemv_kd<F, LPR, B, 4, RAGGED>(a, x, y, st);
    case 3: return launch_gemv_kd<F, LPR, B, 3, RAGGED>(a, x, y, st);
    default: return launch_gemv_kd<F, LPR, B, 2, RAGGED>(a, x, y, st);
  }
}

template <class F, int LPR, int B>
static int launch_gemv_lb(const typename F::Args &a, const void *x, void *y, hipStream_t st) {
  if (F::units(a.K) % LPR) return launch_gemv_k<F, LPR, B, true>(a, x, y, st);
  return launch_gemv_k<F, LPR, B, false>(a, x, y, st);
}


// Units per batch: ISHZ_GEMV_B, else the largest of F::PREFB, F::PREFB - 1, ... 2 that divides
// the units each lane streams per row.
template <class F, int LPR>
static int launch_gemv_l(const typename F::Args &a, const void *x, void *y, hipStream_t st) {
  const int upl = (F::units(a.K) + LPR - 1) / LPR;  // units per lane per row
  int b = gemv_batch_override();
  if (b < 2 || b > F::MAXB) {
    b = 2;
    for (int c = F::PREFB; c > 2; c--)
      if (upl % c == 0) {
        b = c;
        break;
      }
  }
  switch (b) {
    case 5: if constexpr (F::MAXB >= 5) return launch_gemv_lb<F, LPR, 5>(a, x, y, st);
    [[fallthrough]];
    case 4: if constexpr (F::MAXB >= 4) return launch_gemv_lb<F, LPR, 4>(a, x, y, st);
    [[fallthrough]];
    case 3: if constexpr (F::MAXB >= 3) return launch_gemv_lb<F, LPR, 3>(a, x, y, st);
    [[fallthrough]];
    default: return launch_gemv_lb<F, LPR, 2>(a, x, y, st);
  }
}

int gemv_lpr_override();  // ISHZ_GEMV_LPR (tuning)

template <class F>
static int launch_gemv(const typename F::Args &a, const void *x, void *y, hipStream_t st) {
  const int units = F::units(a.K);
  switch (gemv_lpr_override()) {
    case 16: return launch_gemv_l<F, 16>(a, x, y, st);
    case 32: return launch_gemv_l<F, 32>(a, x, y, st);
    case 64: return launch_gemv_l<F, 64>(a, x, y, st);
  }
  if (units <= 160) return launch_gemv_l<F, 16>(a, x, y, st);
  if (units <= 384) return launch_gemv_l<F, 32>(a, x, y, st);
  return launch_gemv_l<F, 64>(a, x, y, st);
}

}  // namespace ishz
