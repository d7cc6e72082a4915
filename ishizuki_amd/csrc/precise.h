// fp32 activations at fp32 precision. The reference's kernels are templated on the activation type
// and accumulate fp32 x in fp32 (Core/GGMLKernels.swift:196-237, Core/VerifyMatmul.swift:95-116;
// checked at 1e-5 of sum |x||w|, Tests/IshizukiKitTests/GGMLKernelTests.swift:131-137). The fp16
// kernels cannot meet that: they stage x in fp16 and carry a 1024-times offset in their fp32 sums.
// So an fp32 call takes this path instead: every weight is decoded to its exact fp32 value (the CPU
// decoder's operations in its order) and dotted with the fp32 x by fp32 FMAs.
//
// One wave per output row (four per workgroup); lane l takes the row's 8-weight slices l, l + 64,
// ..., in order, and the 64 lane partials meet in a fixed DPP / shuffle tree. Up to 16 token rows
// share each decoded slice. x is read straight from memory (each slice's 32 bytes per token; the
// rows of a workgroup hit the same lines in L2). A format D provides Args and
// decode(args, row, slice, v[8]).
#pragma once
#include "common.h"

namespace ishz {

template <class D>
__global__ __launch_bounds__(256) void precise_kernel(typename D::Args a, const float *__restrict__ x, int M, int K,
                                                      int N, void *__restrict__ y, int dt) {
  const int row = blockIdx.x * 4 + wave_id();
  if (row >= N) return;
  const int lane = threadIdx.x & 63;
  float acc[16];
#pragma unroll
  for (int m = 0; m < 16; m++) acc[m] = 0.0f;
  for (int s = lane; s < K / 8; s += 64) {
    float v[8];
    D::decode(a, row, s, v);
#pragma unroll
    for (int m = 0; m < 16; m++) {
      if (m >= M) continue;  // uniform; a break would stop the unrolling (acc in scratch)
      const f4 x0 = *(const f4 *)(x + (size_t)m * K + 8 * s), x1 = *(const f4 *)(x + (size_t)m * K + 8 * s + 4);
      float t = acc[m];
      t = __builtin_fmaf(v[0], x0.x, t);
      t = __builtin_fmaf(v[1], x0.y, t);
      t = __builtin_fmaf(v[2], x0.z, t);
      t = __builtin_fmaf(v[3], x0.w, t);
      t = __builtin_fmaf(v[4], x1.x, t);
      t = __builtin_fmaf(v[5], x1.y, t);
      t = __builtin_fmaf(v[6], x1.z, t);
      t = __builtin_fmaf(v[7], x1.w, t);
      acc[m] = t;
    }
  }
#pragma unroll
  for (int m = 0; m < 16; m++) {
    if (m >= M) continue;
    const float r = group_sum<64>(acc[m]);
    if (lane == 0) store_act(y, (size_t)m * N + row, dt, r);
  }
}

// y [M][N] (dtype dt) = x [M][K] (fp32) times the decoded weights. K % 8 == 0, M <= 16.
template <class D>
static int launch_precise(const typename D::Args &a, const float *x, int M, int K, int N, void *y, int dt,
                          hipStream_t st) {
  if (M < 1 || M > 16 || K % 8) return decline("fp32 path: 1..16 rows and K a multiple of 8");
  hipLaunchKernelGGL(precise_kernel<D>, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, a, x, M, K, N, y, dt);
  ISHZ_LAUNCH_CHECK("fp32 matmul launch");
  return ISHZ_OK;
}

}  // namespace ishz
