// Status reporting of the C ABI: the reason for the calling thread's last non-OK status.
#include <cstdio>

#include "common.h"

namespace ishz {
static thread_local std::string t_last_error;

void set_error(const std::string &msg) { t_last_error = msg; }

int fail(const char *what, hipError_t e) {
  set_error(std::string(what) + ": " + hipGetErrorString(e));
  return ISHZ_EHIP;
}

int decline(const std::string &why) {
  set_error("declined: " + why);
  return ISHZ_DECLINED;
}

int einval(const std::string &why) {
  set_error("invalid argument: " + why);
  return ISHZ_EINVAL;
}

// One workgroup per row: the row's largest magnitude (a max over the block), then every value
// times 2^-e rounded to fp16.
__global__ __launch_bounds__(256) void act_half_kernel(const void *__restrict__ x, int dt, int K,
                                                       uint16_t *__restrict__ xh, float *__restrict__ rs) {
  __shared__ float wmax[4];
  const size_t row = (size_t)blockIdx.x * K;
  // eight loads in flight per thread and pass (one at a time waited out a memory latency each)
  constexpr int U = 8;
  float m = 0.0f;
  for (int k0 = threadIdx.x; k0 < K; k0 += U * blockDim.x) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = k0 + u * (int)blockDim.x;
      v[u] = k < K ? fabsf(load_act(x, row + k, dt)) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; u++) m = fmaxf(m, v[u]);
  }
  m = fmaxf(m, ISHZ_DPP(m, 0xB1));   // the wave's max: quad, half-row and row by DPP,
  m = fmaxf(m, ISHZ_DPP(m, 0x4E));
  m = fmaxf(m, ISHZ_DPP(m, 0x141));
  m = fmaxf(m, ISHZ_DPP(m, 0x140));
  m = fmaxf(m, lane_xor16(m));       // across rows by the row swaps
  m = fmaxf(m, lane_xor32(m));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  // m = f 2^e, f in [0.5, 1), for every finite non-zero m; e capped at 127 so that 2^e stays a
  // finite fp32 factor (a row whose largest value lies in (2^127, FLT_MAX] lands in [0.5, 2))
  int e = 0;
  if (m > 0.0f && __builtin_isfinite(m)) {
    (void)frexpf(m, &e);
    e = e > 127 ? 127 : e;
  }
  const float down = ldexpf(1.0f, -e);
  for (int k0 = threadIdx.x; k0 < K; k0 += U * blockDim.x) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = k0 + u * (int)blockDim.x;
      v[u] = k < K ? load_act(x, row + k, dt) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = k0 + u * (int)blockDim.x;
      if (k < K) xh[row + k] = f2h(v[u] * down);
    }
  }
  if (threadIdx.x == 0) rs[blockIdx.x] = ldexpf(1.0f, e);
}

size_t act_image_bytes(int M, int K) { return ((size_t)M * K * 2 + 255) / 256 * 256 + ((size_t)M * 4 + 255) / 256 * 256; }

int act_prepare(const void *x, int dt, int M, int K, void *image, hipStream_t st, const uint16_t **xh,
                const float **rs) {
  if (dt == ISHZ_DT_F16) {
    *xh = (const uint16_t *)x;
    *rs = nullptr;
    return ISHZ_OK;
  }
  if (dt != ISHZ_DT_BF16 && dt != ISHZ_DT_F32) return decline("activations must be fp16, bf16 or fp32");
  if (!image) return einval("bf16 / fp32 activations need a workspace");
  uint16_t *h = (uint16_t *)image;
  float *r = (float *)((char *)image + ((size_t)M * K * 2 + 255) / 256 * 256);
  hipLaunchKernelGGL(act_half_kernel, dim3(M), dim3(256), 0, st, x, dt, K, h, r);
  ISHZ_LAUNCH_CHECK("activation image launch");
  *xh = h;
  *rs = r;
  return ISHZ_OK;
}
}  // namespace ishz

extern "C" const char *ishz_last_error(void) { return ishz::t_last_error.c_str(); }
extern "C" int ishz_version(void) { return 100; }
