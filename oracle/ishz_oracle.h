/*
 * ishz_oracle — CPU restatement of Ishizuki's quantized-weight matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP kernels are held to: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. The product path
 * (ishizuki_amd/libishizuki_hip.so) never links or calls it.
 *
 * Every function follows a reference function, cited as path:line under the reference tree
 * (Swift sources of struffl/ishizuki). Pinning, per function:
 *   ishzo_dequant Q4_K/Q6_K/IQ2_XS (+Q2_K, IQ*, F16, BF16, F32) -- the reference's golden vectors
 *       (Tests/IshizukiKitTests/Fixtures/ggml-reference.bin, llama.cpp's own to_float).
 *   ishzo_dequant Q4_0      -- parity unpinned by the reference (it has no Q4_0 decoder); pinned
 *       by the ggml block definition's closed form and hand-built blocks in the tests.
 *   ishzo_exl3_dequant      -- exllamav3 golden vectors (exl3-reference.safetensors, 11 cases).
 *   ishzo_hadamard          -- closed form: H.H = I, H of a basis vector, brute-force matrix.
 *   ishzo_affine_dequant    -- closed form s*q+b (MLX's own dequantize is not importable here).
 *   ishzo_matmul / moe      -- brute-force loops over the pinned dequantizers.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGMLType raw values (Sources/IshizukiKit/Config/GGUFFile.swift:13-43). */
enum {
  ISHZO_F32 = 0, ISHZO_F16 = 1, ISHZO_Q4_0 = 2, ISHZO_Q2_K = 10, ISHZO_Q4_K = 12,
  ISHZO_Q6_K = 14, ISHZO_IQ2_XXS = 16, ISHZO_IQ2_XS = 17, ISHZO_IQ3_XXS = 18, ISHZO_IQ1_S = 19,
  ISHZO_IQ3_S = 21, ISHZO_IQ2_S = 22, ISHZO_IQ4_XS = 23, ISHZO_IQ1_M = 29, ISHZO_BF16 = 30
};

int ishzo_block_size(uint32_t type);  /* elements per block, 0 if unknown */
int ishzo_type_size(uint32_t type);   /* bytes per block, 0 if unknown */

float ishzo_half_to_float(uint16_t h);
uint16_t ishzo_float_to_half(float f);  /* round to nearest even */

/* 0 ok, -1 unsupported type, -2 count not whole blocks, -3 short buffer. */
int ishzo_dequant(uint32_t type, const uint8_t *bytes, size_t nbytes, size_t count, float *out);

/* Rows of W [N][K] dequantized in parallel (same values as ishzo_dequant of the whole matrix). */
int ishzo_dequant_rows(uint32_t type, const uint8_t *blocks, int N, int K, float *out, int threads);

/* y[m][n] = sum_k x[m][k] * W[n][k], W = dequant(blocks) row-major [N][K]; fp32 accumulate.
   threads <= 0 means all cores. Returns ishzo_dequant's status. */
int ishzo_ggml_matmul(uint32_t type, const float *x, int M, int K, const uint8_t *blocks,
                      int N, float *y, int threads);

/* Fused decode-dot variant (no dense W): same result up to summation order. */
int ishzo_ggml_matmul_fused(uint32_t type, const float *x, int M, int K, const uint8_t *blocks,
                            int N, float *y, int threads);

/* MLX affine pack: codes u32 [N][K*bits/32] (low bits first), scales/biases fp16 [N][K/gs]. */
int ishzo_affine_dequant(const uint32_t *codes, const uint16_t *scales, const uint16_t *biases,
                         int N, int K, int bits, int group, float *out);
int ishzo_affine_matmul(const float *x, int M, int K, const uint32_t *codes,
                        const uint16_t *scales, const uint16_t *biases, int N, int bits,
                        int group, float *y, int threads);

/* CPU baseline of the rotated 2-bit affine GEMV (bench.py's cpu_baseline leg): rotate x, then
   variant 0 dequantize-then-dot or variant 1 fused decode-dot; OpenMP over rows; the median of
   `reps` (<= 64) timings in seconds (negative on bad arguments). y: fp32 [N]. */
double ishzo_bench_affine_linear(const uint16_t *xh, int K, const float *signs, int block,
                                 const uint32_t *codes, const uint16_t *scales, const uint16_t *biases,
                                 int N, int group, int variant, int reps, int threads, float *y);

/* Blockwise normalised Walsh-Hadamard (Sylvester order) in fp32: y = WHT_b(x*signs)/sqrt(b)
   (inverse: signs applied after). signs may be NULL (all +1). x and y may alias. */
void ishzo_hadamard(const float *x, int rows, int width, int block, const float *signs,
                    int inverse, float *y);

/* EXL3 trellis int16 [K/16][N/16][16*bits]; bits2 = 2*bits (2..16); codebook 0=3INST,
   1=MCG, 2=MUL1. out fp32 [K][N]. 0 ok, -1 bad rate/codebook. */
int ishzo_exl3_dequant(const int16_t *trellis, int K, int N, int bits2, int codebook, float *out);
float ishzo_exl3_decode(uint32_t state, int codebook);

/* EXL3Kernels.apply for fp16 activations: xh = fp16(H128(x*suh)/sqrt128); yh = xh.W (fp32);
   y = fp16(H128(yh)/sqrt128 * svh). x, suh, svh given as floats (already fp16 values). */
int ishzo_exl3_apply(const float *x, int M, int K, const int16_t *trellis, const float *suh,
                     const float *svh, int N, int bits2, int codebook, float *y, int threads);

/* MoE routing (Text/MoEBlock.swift:124-134): softmax over E in fp32, top-k (ties -> lower
   index), optional renormalisation. ids [T][k] in descending score order. */
void ishzo_moe_route(const float *logits, int T, int E, int topk, int normalize, int32_t *ids,
                     float *weights);

/* Expert SwiGLU over Q4_K (or any GGML type) experts, fp16 activations. gate/up blocks are
   [E][I][H], down [E][H][I]. Emulates the reference's fp16 intermediates
   (ResidentExperts.swiglu, Text/MoEBlock.swift:168-171; weighting :147-149). With shared
   ([T][H]) and shared_gate ([T]), both fp16 values as floats, the shared expert's
   sigmoid(gate) * shared term is added in fp32 before the cast (:158-160). y [T][H]. */
int ishzo_moe_swiglu(uint32_t type, const float *x, int T, int H, const int32_t *ids,
                     const float *weights, int topk, const uint8_t *gate, const uint8_t *up,
                     const uint8_t *down, int E, int I, const float *shared, const float *shared_gate,
                     float *y, int threads);

#ifdef __cplusplus
}
#endif
