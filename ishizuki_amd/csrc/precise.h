// fp32 activations at fp32 precision. The reference's kernels are templated on the activation type
// and accumulate fp32 x in fp32 (Core/GGMLKernels.swift:196-237, Core/VerifyMatmul.swift:95-116;
// checked at 1e-5 of sum |x||w|, Tests/IshizukiKitTests/GGMLKernelTests.swift:131-137). The fp16
// kernels cannot meet that: they stage x in fp16 and carry a 1024-times offset in their fp32 sums.
// So an fp32 call takes this path instead: every weight is decoded to its exact fp32 value (the CPU
// decoder's operations in its order) and dotted with the fp32 x by fp32 FMAs. The same kernel, with
// fp16 / bf16 x widened exactly, also serves layouts the fp16 kernels do not take (affine groups of
// 32 or other multiples of 32 than 64 and 128).
//
// One wave per output row (four per workgroup); lane l takes the row's 8-weight slices l, l + 64,
// ..., in order, and the 64 lane partials meet in a fixed DPP / shuffle tree. Up to 16 token rows
// share each decoded slice. x is read straight from memory (each slice's 32 bytes per token; the
// rows of a workgroup hit the same lines in L2). A format D provides Args and
// decode(args, row, slice, v[8]).
#pragma once
#include "common.h"

namespace ishz {

// Eight activations of token row m from slice s: fp32 as they are, fp16 / bf16 widened exactly.
template <int XDT>
DEV void x8(const void *x, size_t o, float *v) {
  if constexpr (XDT == ISHZ_DT_F32) {
    const f4 a = *(const f4 *)((const float *)x + o), b = *(const f4 *)((const float *)x + o + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  } else {
    const u4 h = *(const u4 *)((const uint16_t *)x + o);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t b = (h[i >> 1] >> (16 * (i & 1))) & 0xffffu;
      v[i] = XDT == ISHZ_DT_F16 ? h2f(b) : __builtin_bit_cast(float, b << 16);
    }
  }
}

template <class D, int XDT>
__global__ __launch_bounds__(256) void precise_kernel(typename D::Args a, const void *__restrict__ x, int M, int K,
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
      float xv[8];
      x8<XDT>(x, (size_t)m * K + 8 * s, xv);
      float t = acc[m];
#pragma unroll
      for (int i = 0; i < 8; i++) t = __builtin_fmaf(v[i], xv[i], t);
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

// y [M][N] (in x's dtype xdt) = x [M][K] times the decoded weights. K % 8 == 0, M <= 16.
template <class D>
static int launch_precise(const typename D::Args &a, const void *x, int xdt, int M, int K, int N, void *y,
                          hipStream_t st) {
  if (M < 1 || M > 16 || K % 8) return decline("exact-weight path: 1..16 rows and K a multiple of 8");
  const dim3 grid((unsigned)((N + 3) / 4));
  if (xdt == ISHZ_DT_F32)
    hipLaunchKernelGGL((precise_kernel<D, ISHZ_DT_F32>), grid, dim3(256), 0, st, a, x, M, K, N, y, xdt);
  else if (xdt == ISHZ_DT_F16)
    hipLaunchKernelGGL((precise_kernel<D, ISHZ_DT_F16>), grid, dim3(256), 0, st, a, x, M, K, N, y, xdt);
  else
    hipLaunchKernelGGL((precise_kernel<D, ISHZ_DT_BF16>), grid, dim3(256), 0, st, a, x, M, K, N, y, xdt);
  ISHZ_LAUNCH_CHECK("exact-weight matmul launch");
  return ISHZ_OK;
}

}  // namespace ishz
