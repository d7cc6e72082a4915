// Shared device helpers for the gfx950 (CDNA4, wave64) kernels of libishizuki_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/ishizuki_hip.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

#define DEV __device__ __forceinline__

// ---------------------------------------------------------------- loads
// GGUF blocks are only 2-byte aligned (18, 74 and 210-byte blocks). On amdhsa targets the
// hardware runs in unaligned mode, so a memcpy from a pointer known to be 2-aligned lowers to
// one global_load_dwordx{1,2,4}.
template <int A>
DEV u4 ld16(const uint8_t *p) {
  u4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, A), 16);
  return v;
}
template <int A>
DEV u2 ld8(const uint8_t *p) {
  u2 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, A), 8);
  return v;
}
template <int A>
DEV uint32_t ld4(const uint8_t *p) {
  uint32_t v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, A), 4);
  return v;
}
DEV uint32_t ld2(const uint8_t *p) { return *(const uint16_t *)__builtin_assume_aligned(p, 2); }
// Low 32 bits of a 24-bit by 24-bit product (both operands below 2^24). Plain C: the compiler
// emits v_mul_lo_u32, which on gfx950 issues at the rate of v_mul_u32_u24 (a dependent-chain
// microbenchmark gives both the same time); the inline-assembly v_mul_u32_u24 this replaced
// measured the same or slower (IQ2_XS GEMV, 25600x5120: 20.3-20.5 us against 19.2-19.3).
DEV uint32_t mul24(uint32_t a, uint32_t b) {
  __builtin_assume(a < (1u << 24) && b < (1u << 24));
  return a * b;
}

// 16 bytes at a 2-byte-aligned address. A global load that is not dword aligned costs about a
// third more in the memory pipeline, so the dword-aligned 20-byte window around the bytes is
// loaded instead and shifted into place with v_alignbyte_b32 (one op per dword). Reads up to 3
// bytes past the 16: callers guarantee those bytes are inside the buffer.
struct W20 {
  u4 a;
  uint32_t b;
  uint32_t sh;  // byte offset of the data inside the window (0..3)
};
DEV W20 ldw20(const uint8_t *p) {
  const uintptr_t ip = (uintptr_t)p;
  const uint8_t *q = (const uint8_t *)(ip & ~(uintptr_t)3);
  return {ld16<4>(q), ld4<4>(q + 16), (uint32_t)(ip & 3)};
}
DEV u4 realign(const W20 &w) {
  return u4{__builtin_amdgcn_alignbyte(w.a.y, w.a.x, w.sh), __builtin_amdgcn_alignbyte(w.a.z, w.a.y, w.sh),
            __builtin_amdgcn_alignbyte(w.a.w, w.a.z, w.sh), __builtin_amdgcn_alignbyte(w.b, w.a.w, w.sh)};
}

// ---------------------------------------------------------------- fp16 bits
DEV float h2f(uint32_t bits16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16); }
DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
DEV h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
DEV uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// Two small unsigned integers held in the low bits of each 16-bit half become exact fp16
// values by setting the exponent of 1024 above them and subtracting 1024 + bias.
DEV uint32_t magic(uint32_t halves) { return halves | 0x64006400u; }
DEV uint32_t unmagic(uint32_t halves, _Float16 off) {
  return as_u32(as_h2(halves | 0x64006400u) - h2{off, off});
}

// (a & mask) | orv: one v_and_or_b32 (gfx9 VOP3 encodings take no literal and read one SGPR, so
// orv is kept in a VGPR, see vconst, and the mask goes to an SGPR). Written in C, not inline
// assembly: the hazard recognizer cannot see into an asm statement and padded every one that fed
// a VALU with an s_nop (79 per five units in the headline GEMV's loop, 23 without; 10.9 -> 10.6 us).
DEV uint32_t and_or(uint32_t a, uint32_t mask, uint32_t orv) { return (a & mask) | orv; }
// A constant materialised once into a VGPR the compiler cannot rematerialise per use.
DEV uint32_t vconst(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

// Wave index within the workgroup as a wave-uniform (scalar) value, so that everything derived
// from it is computed on the scalar unit.
DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// fp32 += a.lo*b.lo + a.hi*b.hi (v_dot2_f32_f16).
DEV float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// ---------------------------------------------------------------- cross-lane sums
#define ISHZ_DPP(v, ctrl)                                                                  \
  __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, \
                                                        0xf, 0xf, true))
// The value of lane ^ 16 / lane ^ 32: the row swaps v_permlane16_swap / v_permlane32_swap of a
// register with itself (one VALU op, no LDS-pipe shuffle); the wave must be whole.
DEV float lane_xor16(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
}
DEV float lane_xor32(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

// Sum over aligned groups of W lanes (W = 8, 16, 32, 64); every lane of a group gets the sum.
template <int W>
DEV float group_sum(float v) {
  v += ISHZ_DPP(v, 0xB1);   // quad_perm [1,0,3,2]
  v += ISHZ_DPP(v, 0x4E);   // quad_perm [2,3,0,1]
  v += ISHZ_DPP(v, 0x141);  // row_half_mirror: lane j <- 7-j within 8
  if (W >= 16) v += ISHZ_DPP(v, 0x140);  // row_mirror: lane j <- 15-j within 16
  if (W >= 32) v += lane_xor16(v);
  if (W >= 64) v += lane_xor32(v);
  return v;
}

// Value of lane K of each quad (DPP quad_perm [K,K,K,K]).
template <int K>
DEV uint32_t quad_bcast(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, K * 0x55, 0xf, 0xf, false);
}

// ---------------------------------------------------------------- activations and outputs
DEV float load_act(const void *x, size_t i, int dt) {
  if (dt == ISHZ_DT_F32) return ((const float *)x)[i];
  const uint16_t b = ((const uint16_t *)x)[i];
  return dt == ISHZ_DT_F16 ? h2f(b) : __builtin_bit_cast(float, (uint32_t)b << 16);
}
// v narrowed to dt (fp32 as is; fp16 and bf16 round to nearest even, NaN stays NaN).
DEV void store_act(void *y, size_t i, int dt, float v) {
  if (dt == ISHZ_DT_F32) {
    ((float *)y)[i] = v;
  } else if (dt == ISHZ_DT_F16) {
    ((uint16_t *)y)[i] = f2h(v);
  } else {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = ((u & 0x7fffffffu) > 0x7f800000u) ? (u | 0x400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    ((uint16_t *)y)[i] = (uint16_t)(u >> 16);
  }
}
// Where a kernel's outputs go: dtype, and the per-token-row factor 2^e of rescaled activations
// (null: none; see act_prepare). Output i of token row t is v * rs[t] narrowed to dt.
struct Out {
  void *y;
  int dt;
  const float *rs;
  DEV void put(size_t i, int t, float v) const {
    if (dt == ISHZ_DT_F16 && !rs) ((uint16_t *)y)[i] = f2h(v);
    else store_act(y, i, dt, rs ? v * rs[t] : v);
  }
};

#ifdef ISHZ_TIMING
// Measurement builds only (-DISHZ_TIMING, never in the library): per-wave s_memrealtime stamps
// (100 MHz) at a kernel's phase boundaries, for a timeline of its phases; read back from the host
// with hipMemcpyFromSymbol.
__device__ uint64_t ishz_timing[4096 * 5];
#endif

// ---------------------------------------------------------------- MFMA
// C[i][j] += sum_k A[i][k] B[k][j], 16x16 fp32 tile. Lane l holds A row l%16 and B column l%16
// (k slots chosen by l/16; any consistent k order works) and C rows 4*(l/16)+r, column l%16.
DEV f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
DEV f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
DEV h8 as_h8(u4 v) { return __builtin_bit_cast(h8, v); }
DEV h4 as_h4(u2 v) { return __builtin_bit_cast(h4, v); }

// ---------------------------------------------------------------- host side
namespace ishz {
void set_error(const std::string &msg);
int fail(const char *what, hipError_t e);
int decline(const std::string &why);
int einval(const std::string &why);
inline hipStream_t S(ishz_stream_t s) { return (hipStream_t)s; }

// Activations other than fp16 (bf16, fp32) are converted once per call into an fp16 image with a
// power-of-two factor per row, and every kernel stages that image as it stages fp16 x:
//   xh[m][k] = fp16(x[m][k] * 2^-e_m),  2^(e_m - 1) <= max_k |x[m][k]| < 2^e_m,
// outputs multiplied back by rs[m] = 2^e_m (exact) in fp32 before their one narrowing to x's
// dtype. bf16 values (8 significant bits) land exactly down to 2^-17 of their row's largest
// (fp16 subnormals below 2^-14 still hold 8 bits there); smaller ones within 2^-25 of it. fp32
// values round to fp16 (2^-11 relative). The image: act_image_bytes(M, K) bytes of a workspace.
size_t act_image_bytes(int M, int K);
int act_prepare(const void *x, int dt, int M, int K, void *image, hipStream_t st, const uint16_t **xh,
                const float **rs);
// A stream-ordered temporary (hipMallocAsync / hipFreeAsync) for calls without a workspace.
struct StreamTemp {
  void *p = nullptr;
  hipStream_t st;
  explicit StreamTemp(hipStream_t s) : st(s) {}
  int get(size_t bytes) {
    const hipError_t e = hipMallocAsync(&p, bytes, st);
    return e == hipSuccess ? ISHZ_OK : fail("temporary allocation", e);
  }
  ~StreamTemp() {
    if (p) (void)hipFreeAsync(p, st);
  }
};
}  // namespace ishz

#define ISHZ_LAUNCH_CHECK(what)                     \
  do {                                              \
    hipError_t _e = hipGetLastError();              \
    if (_e != hipSuccess) return ishz::fail(what, _e); \
  } while (0)
