/*
 * ishizuki_hip.h — C ABI of libishizuki_hip.so, the MI355X (gfx950) quantized-weight matmul
 * path of Ishizuki. Plain C: device pointers, sizes, a HIP stream, an int status.
 *
 * Each entry point replaces one operation of the reference's Swift kernel API (cited as
 * path:line under struffl/ishizuki). The reference returns nil to mean "declined, fall back";
 * here that is ISHZ_DECLINED, returned before anything is launched. Errors the reference would
 * throw at validation are ISHZ_EINVAL; a failed HIP call is ISHZ_EHIP. ishz_last_error() gives
 * the reason for the last non-OK status on the calling thread.
 *
 * All pointers are device pointers unless stated. Calls are asynchronous on `stream` (a
 * hipStream_t; NULL = the default stream), never synchronise, and are reentrant: kernels keep no
 * state between calls. Swift reaches this header through include/module.modulemap.
 */
#ifndef ISHIZUKI_HIP_H
#define ISHIZUKI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *ishz_stream_t; /* hipStream_t */

enum { ISHZ_OK = 0, ISHZ_DECLINED = 1, ISHZ_EINVAL = 2, ISHZ_EHIP = 3 };

/* Element types of activations and outputs. The matmuls take x in any of them and write y in
   x's dtype, as the reference's kernels templated on the activation type do.
   - fp16 x: the fp16 kernels (x staged in fp16, fp32 accumulation).
   - bf16 x: the same kernels on an fp16 image of x with a power-of-two factor per row (the
     row's largest value lands in [0.5, 1); outputs are multiplied back, exactly, before their
     one narrowing). bf16 values convert exactly down to 2^-17 of their row's largest. The image
     lives in the call's workspace where the entry point takes one, else in a stream-ordered
     temporary (hipMallocAsync).
   - fp32 x: fp32 precision. Every weight is decoded to its exact fp32 value and dotted with the
     fp32 x by fp32 FMAs (no image, no temporary), as the reference accumulates fp32 x in fp32.
   The MoE FFN takes fp16 or bf16 x (its intermediates are rounded to x's dtype). */
enum { ISHZ_DT_F32 = 0, ISHZ_DT_F16 = 1, ISHZ_DT_BF16 = 2 };

/* GGML storage types, numbered as GGMLType's raw values (Config/GGUFFile.swift:13-43). */
enum {
  ISHZ_GGML_Q4_0 = 2,
  ISHZ_GGML_Q2_K = 10,
  ISHZ_GGML_Q4_K = 12,
  ISHZ_GGML_Q6_K = 14,
  ISHZ_GGML_IQ2_XXS = 16,
  ISHZ_GGML_IQ2_XS = 17,
  ISHZ_GGML_IQ3_XXS = 18,
  ISHZ_GGML_IQ1_S = 19,
  ISHZ_GGML_IQ3_S = 21,
  ISHZ_GGML_IQ2_S = 22,
  ISHZ_GGML_IQ4_XS = 23,
  ISHZ_GGML_IQ1_M = 29
};

/* Reason for the calling thread's last non-OK status (static storage, never NULL). */
const char *ishz_last_error(void);
/* ABI version of this library (major * 100 + minor). */
int ishz_version(void);

/* Measurement utility, no counterpart in the reference: a plain streaming read of `bytes`
 * (a multiple of 16) on `stream`, for timing the practical read ceiling of a weight matrix's
 * size beside the quantized matmuls. `sink` is a 4-byte device buffer it practically never
 * writes. */
int ishz_stream_read(const void *p, size_t bytes, void *sink, ishz_stream_t stream);

/* GGMLType.blockSize / typeSize (Config/GGUFFile.swift:44-80) for the types this library
   decodes (GGMLDequant.supported, Core/GGMLDequant.swift:19-24, plus Q4_0); 0 for any other
   type (ishz_ggml_geometry covers every GGMLType). */
int ishz_ggml_block_size(uint32_t type);
int ishz_ggml_type_size(uint32_t type);

/* GGMLKernels.matvec (Core/GGMLKernels.swift:177-213): y[M][N] = x[M][K] . W[N][K]^T with W
   the GGML blocks of `type`, rows of W contiguous, never expanded. x fp16, bf16 or fp32, y in
   x's dtype; M in
   1..16 (matvecBatch, :146). M = 1 runs the streaming GEMV, M >= 2 the MFMA verify kernel.
   Declines (ISHZ_DECLINED) for an unsupported type or dtype, M outside 1..16, K not a whole
   number of blocks, N < 1, or blocks_bytes < N * rowBytes (:181-189). */
int ishz_ggml_matvec(uint32_t type, const void *x, int x_dtype, int M, int K, const void *blocks,
                     size_t blocks_bytes, int N, void *y, ishz_stream_t stream);

/* ishz_ggml_matvec with a caller workspace of ishz_ggml_workspace_size(type, M, K, N) bytes (0:
   none is used): for outputs too narrow to give every CU its own tiles, the M >= 2 product is
   split along K into parts written as fp32 partials [S][M][N] and summed in part order, narrowed
   once -- the reference's split-K verify (Core/VerifyMatmul.swift:91-107: outputs [split, m, n]
   in fp32, then sum(axis: 0) and the cast). With a NULL or short workspace it is
   ishz_ggml_matvec. */
size_t ishz_ggml_workspace_size(uint32_t type, int M, int K, int N);
int ishz_ggml_matvec_ws(uint32_t type, const void *x, int x_dtype, int M, int K, const void *blocks,
                        size_t blocks_bytes, int N, void *y, void *workspace, size_t workspace_bytes,
                        ishz_stream_t stream);

/* GGMLKernels.matmulFew (Core/GGMLKernels.swift:219-253): the same product for M in 2..8
   (matmulFewRows, :217), 256-element block types only, as the reference. Each weight is decoded
   once into MFMA operand registers and multiplied against every row. row_blocks is accepted for
   signature parity and ignored (the tile shape is chosen per shape). */
int ishz_ggml_matmul_few(uint32_t type, const void *x, int x_dtype, int M, int K,
                         const void *blocks, size_t blocks_bytes, int N, int row_blocks, void *y,
                         ishz_stream_t stream);

/* GGMLKernels.dequantize (Core/GGMLKernels.swift:60-97): expand `count` elements of blocks to
   out (fp32, fp16 or bf16), bit-exact with the CPU definition (Core/GGMLDequant.swift:25). */
int ishz_ggml_dequant(uint32_t type, const void *blocks, size_t blocks_bytes, size_t count,
                      void *out, int out_dtype, ishz_stream_t stream);

/* GGMLKernels.gather (Core/GGMLKernels.swift:102-138): rows ids[0..n_ids) of W [n_rows][K]
   decoded into out [n_ids][K]. An id outside [0, n_rows) yields a row of zeros instead of a
   read out of bounds. */
int ishz_ggml_gather(uint32_t type, const int32_t *ids, int n_ids, const void *blocks,
                     size_t blocks_bytes, int n_rows, int K, void *out, int out_dtype,
                     ishz_stream_t stream);

/* hadamardRotate (Core/Hadamard.swift:8-23): per contiguous `block` of each row,
   y = WHT_block(x * signs) / sqrt(block) in fp32 (signs applied after the transform when
   inverse), Sylvester (natural) order, output in the input dtype. signs: fp32 [width] or NULL
   (all +1). block a power of two <= 4096; width * 4 bytes <= 64 KiB. */
int ishz_hadamard(const void *x, int dtype, int rows, int width, int block, const float *signs,
                  int inverse, void *y, ishz_stream_t stream);

/* MLX affine quantized matmul: y[M][N] = x[M][K] . W^T, W[n][k] = s[n][k/group] * q + b[...].
   codes u32 [N][K*bits/32], bits 2..8 (code k at bit k*bits of the row's little-endian u32
   stream: MLX's pack, Quantize/WeightedAffineQuantizer.swift:142-153), scales/biases
   [N][K/group] in scale_dtype (fp16 or bf16). x fp16, bf16 or fp32, y in x's dtype. M = 1 is
   the streaming GEMV (MLX
   quantizedMM's qmv, called at Core/Hadamard.swift:228-230); M = 2..16 the MFMA verify kernel
   (VerifyMatmul.applyAny, Core/VerifyMatmul.swift:73-120: its fast path takes 2, 4 and 8 bits,
   :89, its generic path the other widths, :273-290). Groups of 64 and 128 take those kernels;
   any other multiple of 32 dividing K (applyAny's groupSize % 32, :84) takes the exact-weight
   kernel (w = s * q + b in fp32, fp32 sums; one wave per output row). Declines: groups that are
   not a multiple of 32, K % 128 (and K % 256 for verify rows of packs other than 2-bit), other
   dtypes. */
int ishz_affine_matmul(const void *x, int x_dtype, int M, int K, const uint32_t *codes,
                       const void *scales, const void *biases, int scale_dtype, int N, int bits,
                       int group, void *y, ishz_stream_t stream);

/* The rotated PackedLinear forward (Core/Hadamard.swift:180-231): hadamardRotate(x, block,
   signs) rounded to x's dtype, then ishz_affine_matmul. block = 0 means no rotation. For fp16
   x and M = 1 the rotation runs inside the GEMV (x is rotated while it is staged into LDS);
   otherwise it is a separate kernel into `workspace` (ishz_affine_workspace_size bytes, which
   bf16 / fp32 x always needs). */
size_t ishz_affine_workspace_size(int M, int K);
int ishz_affine_linear(const void *x, int x_dtype, int M, int K, const float *signs, int block,
                       const uint32_t *codes, const void *scales, const void *biases,
                       int scale_dtype, int N, int bits, int group, void *y, void *workspace,
                       size_t workspace_bytes, ishz_stream_t stream);

/* EXL3 codebooks (EXL3Tensor.Codebook, Core/EXL3.swift:10-14); rates are bits2 = 2 * bits in
   {2,3,4,5,6,7,8,10,12,14,16} (supportedBits, :27), half-integer rates only with MUL1. */
enum { ISHZ_EXL3_3INST = 0, ISHZ_EXL3_MCG = 1, ISHZ_EXL3_MUL1 = 2 };

/* EXL3Kernels.dequantize (Core/EXL3.swift:133-147): trellis int16 [K/16][N/16][8*bits2] to a
   dense W [K][N] (fp32 / fp16 / bf16), bit-exact with the trellis decoder. */
int ishz_exl3_dequant(const int16_t *trellis, int K, int N, int bits2, int codebook, void *out,
                      int out_dtype, ishz_stream_t stream);

/* EXL3Kernels.rotate (Core/EXL3.swift:102-124, kernel :219-265): per 128-block of each row,
   (x * scales if before) -> WHT / sqrt(128) -> (* scales if not before), fp32 math, output in
   out_dtype; in and out fp32, fp16 or bf16. scales fp16 [width] (the suh / svh vectors). */
int ishz_exl3_rotate(const void *x, int in_dtype, int rows, int width, const uint16_t *scales,
                     int before, void *y, int out_dtype, ishz_stream_t stream);

/* EXL3Kernels.matvec (Core/EXL3.swift:149-164, kernel :286-330): yh[M][N] (fp32) = xh[M][K]
   (fp16, bf16 or fp32) . W, W decoded in-kernel. M in 1..16 (the reference: 1..8, 9..16 as two
   launches). The K-split partial products are summed in split order: the same bits on every
   call. ishz_exl3_matvec_ws takes them (and bf16 x's fp16 image) in a caller workspace of
   ishz_exl3_matvec_workspace_size(M, K, N) bytes and allocates nothing; ishz_exl3_matvec is the
   same call with stream-ordered temporaries (hipMallocAsync) instead. fp32 x needs neither.
   fp16 / bf16 x with the 3INST and MCG codebooks, up to 8 rows: each weight's two fp16 halves
   (its codebook image before their final add) meet x in fp32, so the weight's own fp16 rounding
   is skipped (at most half an fp16 ulp per weight); MUL1 and more rows multiply the decoded fp16
   weight. fp32 x multiplies the exactly decoded weight. */
size_t ishz_exl3_matvec_workspace_size(int M, int K, int N);
int ishz_exl3_matvec_ws(const void *xh, int x_dtype, int M, int K, const int16_t *trellis, int N,
                        int bits2, int codebook, float *yh, void *workspace, size_t workspace_bytes,
                        ishz_stream_t stream);
int ishz_exl3_matvec(const void *xh, int x_dtype, int M, int K, const int16_t *trellis, int N,
                     int bits2, int codebook, float *yh, ishz_stream_t stream);

/* EXL3Kernels.apply (Core/EXL3.swift:82-100): y = dt(rotate_out(xh . W)) with
   xh = dt(rotate_in(x)), dt = x's dtype (fp16, bf16 or fp32). Needs
   ishz_exl3_workspace_size(M, K, N) bytes of device workspace. */
size_t ishz_exl3_workspace_size(int M, int K, int N);
int ishz_exl3_apply(const void *x, int x_dtype, int M, int K, const int16_t *trellis,
                    const uint16_t *suh, const uint16_t *svh, int N, int bits2, int codebook,
                    void *y, void *workspace, size_t workspace_bytes, ishz_stream_t stream);

/* No counterpart in the reference: ishz_exl3_apply for callers that cannot allocate (code under
   HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It allocates nothing:
   the workspace is a static device array of ISHZ_EXL3_STATIC_SCRATCH_BYTES that each GPU holds
   until the process ends. Shapes whose ishz_exl3_workspace_size exceeds it give ISHZ_EINVAL.
   `stream` must belong to the current device. Calls that overlap on one GPU share the scratch
   and race: serialise them (one stream, or events). Same results as ishz_exl3_apply. */
#ifndef ISHZ_EXL3_STATIC_SCRATCH_BYTES /* a build of the library may set it smaller (-D) */
#define ISHZ_EXL3_STATIC_SCRATCH_BYTES (32u << 20)
#endif
int ishz_exl3_apply_static(const void *x, int x_dtype, int M, int K, const int16_t *trellis,
                           const uint16_t *suh, const uint16_t *svh, int N, int bits2, int codebook,
                           void *y, ishz_stream_t stream);

/* MoEBlock routing (Text/MoEBlock.swift:124-134): softmax over E logits (fp32) per token, the
   topk largest (ties to the lower index), renormalised to sum 1 when `normalize`. ids [T][topk]
   in descending order, weights [T][topk]. */
int ishz_moe_route(const float *logits, int T, int E, int topk, int normalize, int32_t *ids,
                   float *weights, ishz_stream_t stream);

/* The MoE FFN (MoEBlock.callAsFunction + ResidentExperts.swiglu, Text/MoEBlock.swift:124-171)
   over GGML-block experts: route (as ishz_moe_route), then for each routed (token, expert)
   down(silu(gate(x)) * up(x)) with intermediates in x's dtype, weighted and summed in fp32 into
   y [T][H] (x's dtype). x fp16 or bf16 (MoEBlock runs in the model's dtype; bf16 x and h are
   staged from fp16 images with a power-of-two factor per row, exact for bf16 values down to
   2^-17 of their row's largest). gate/up hold E experts of [I][H] blocks back to back, down E experts of
   [H][I]; expert_bytes is the size of one expert's matrix. Only routed experts' blocks are
   read. type: Q4_K (also Q4_0, Q6_K). shared / shared_gate (optional, both or neither): the
   shared expert's output shared(x) [T][H] and gate logit sharedGate(x) [T], in x's dtype, computed by
   the caller's own projections; sigmoid(gate) * shared is added in fp32 before the one cast
   (:158-160). ids_out / weights_out (optional, [T][topk]) receive the routing. workspace:
   ishz_moe_workspace_size bytes. (The reference runs this through MLX's gatherQuantizedMM over
   affine experts; GGUF experts are a composition of its routing with the GGML kernels.) */
size_t ishz_moe_workspace_size(int T, int H, int E, int I, int topk);

/* The same FFN over MLX affine stacked experts, the reference's own expert format
   (StackedExperts, Text/MoEBlock.swift:22-50, multiplied through gatherQuantizedMM at :45-49):
   gate and up packs hold E experts of [I][H] weights, down E experts of [H][I]; codes u32
   [E][rows][K * bits / 32], scales / biases [E][rows][K / group] in scale_dtype. bits 2 to 8,
   group 64 or 128, H and I multiples of 256. Routing, workspace and outputs as ishz_moe_swiglu. */
int ishz_moe_swiglu_affine(const void *x, int x_dtype, int T, int H, const float *logits, int E,
                           int topk, int normalize, const uint32_t *gate_codes, const void *gate_scales,
                           const void *gate_biases, const uint32_t *up_codes, const void *up_scales,
                           const void *up_biases, const uint32_t *down_codes, const void *down_scales,
                           const void *down_biases, int scale_dtype, int bits, int group, int I,
                           const void *shared, const void *shared_gate, void *y, int32_t *ids_out,
                           float *weights_out, void *workspace, size_t workspace_bytes,
                           ishz_stream_t stream);
int ishz_moe_swiglu(uint32_t type, const void *x, int x_dtype, int T, int H, const float *logits,
                    int E, int topk, int normalize, const void *gate, const void *up,
                    const void *down, size_t expert_bytes, int I, const void *shared,
                    const void *shared_gate, void *y, int32_t *ids_out, float *weights_out,
                    void *workspace, size_t workspace_bytes, ishz_stream_t stream);

/* ---------------------------------------------------------------- GGUF container (host side)
 * GGUFFile (Config/GGUFFile.swift:179-397): header, metadata and tensor table of a .gguf file,
 * the tensor bytes left in a read-only memory mapping. Malformed or unsupported files give
 * ISHZ_EINVAL with the reference's reason (ishz_last_error). Shapes are row-major (GGUF's dims
 * reversed); tensor offsets are relative to the data section, as in TensorInfo. Pointers here
 * are host pointers; the handle is immutable after open and may be shared between threads. */
typedef struct ishz_gguf ishz_gguf;
typedef struct ishz_gguf_value ishz_gguf_value;

/* GGMLType raw value known (1) or not (0), and its blockSize / typeSize
 * (Config/GGUFFile.swift:39-88); ISHZ_DECLINED for an unknown value. */
int ishz_ggml_type_known(uint32_t type);
int ishz_ggml_geometry(uint32_t type, int *block_size, int *type_size);

int ishz_gguf_open(const char *path, ishz_gguf **out);   /* GGUFFile.init(url:) */
void ishz_gguf_close(ishz_gguf *f);
uint32_t ishz_gguf_version(const ishz_gguf *f);
uint64_t ishz_gguf_data_offset(const ishz_gguf *f);       /* GGUFFile.dataOffset */
int64_t ishz_gguf_tensor_count(const ishz_gguf *f);
int64_t ishz_gguf_find_tensor(const ishz_gguf *f, const char *name);  /* subscript(tensor:); -1 if absent */
/* TensorInfo: name (owned by the handle), rank, shape[4] (row-major, unused dims 0), type,
 * offset (from the data section), byte count. */
int ishz_gguf_tensor_info(const ishz_gguf *f, int64_t i, const char **name, int *rank, int64_t *shape,
                          uint32_t *type, uint64_t *offset, uint64_t *nbytes);
/* data(for:) (:289-301): the tensor's bytes inside the mapping, or NULL (ISHZ_EINVAL) when they
 * run past the end of the file. */
const void *ishz_gguf_tensor_data(const ishz_gguf *f, int64_t i);
/* GGUFWeights.load's packed path (Core/GGUFWeights.swift:47-85): copy a tensor's blocks as they
 * lie on disk into caller-owned device memory (dst_bytes >= its byte count); returns when done. */
int ishz_gguf_tensor_upload(const ishz_gguf *f, int64_t i, void *dst, size_t dst_bytes, ishz_stream_t stream);

/* Metadata: keys in file order (a repeated key keeps its last value), values as GGUFValue
 * (:125-168). Arrays nest; scalars read through the reference's accessors (intValue,
 * floatValue, boolValue, stringValue), ISHZ_DECLINED when a value has no such reading. */
int64_t ishz_gguf_kv_count(const ishz_gguf *f);
const char *ishz_gguf_kv_key(const ishz_gguf *f, int64_t i);
int64_t ishz_gguf_find_kv(const ishz_gguf *f, const char *key);  /* subscript(_:); -1 if absent */
const ishz_gguf_value *ishz_gguf_kv_value(const ishz_gguf *f, int64_t i);
int ishz_gguf_value_type(const ishz_gguf_value *v);              /* GGUF value type 0..12 (9 = array) */
int64_t ishz_gguf_value_len(const ishz_gguf_value *v);           /* array length, -1 otherwise */
const ishz_gguf_value *ishz_gguf_value_elem(const ishz_gguf_value *v, int64_t j);
int ishz_gguf_value_int(const ishz_gguf_value *v, int64_t *out);
int ishz_gguf_value_float(const ishz_gguf_value *v, double *out);
int ishz_gguf_value_bool(const ishz_gguf_value *v, int *out);
int ishz_gguf_value_string(const ishz_gguf_value *v, const char **s, size_t *len);
int ishz_gguf_value_raw(const ishz_gguf_value *v, uint64_t *u, int64_t *i, double *d);

#ifdef __cplusplus
}
#endif
#endif /* ISHIZUKI_HIP_H */
