/*
 * onnxl_amd.h - C ABI of the MI355X (gfx950) quantized-matmul kernels.
 *
 * Each entry point is the GPU replacement of one onnx-light reference kernel
 * overload that writes into a preallocated output (the `Tensor &output`
 * overloads).  A reference-side adapter (KernelBase subclass registered with
 * RegisterKernelFn) calls these functions from KernelBase::Run.  Reference
 * paths below are relative to the onnx-light tree:
 *   km/ = onnx_light/onnx_extensions/kernels/kernels/math/
 *   kq/ = onnx_light/onnx_extensions/kernels/kernels/quantization/
 *
 * Conventions
 * - Tensors are described by onnxl_amd_tensor: ONNX TensorProto.DataType code,
 *   row-major dims, payload pointer and byte count.  4-bit types pack two
 *   elements per byte, low nibble first (the ONNX / reference layout).
 * - `location` says where the payload lives.  Device payloads are used in
 *   place; host payloads are staged to the device (inputs) or copied back
 *   (outputs) inside the call, which then completes before returning.
 * - An absent optional input is a NULL pointer or a descriptor with rank -1
 *   (the reference's empty `Tensor{}`).
 * - Outputs are preallocated by the caller with the shape the reference
 *   computes; a mismatch is an INVALID_ARGUMENT, as in the reference.
 * - `stream` is a hipStream_t (NULL = default stream).  Device-only calls are
 *   asynchronous on `stream`.
 * - Every function returns an onnxl_amd_status; the message of the last
 *   failure on the calling thread is returned by onnxl_amd_last_error().  The
 *   validation failures the reference raises as std::invalid_argument map to
 *   ONNXL_AMD_INVALID_ARGUMENT with the reference's message text.
 * - Calls on one device share a library-owned workspace: calls on different
 *   streams of the same device must be ordered by the caller.
 */
#ifndef ONNXL_AMD_H_
#define ONNXL_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ONNXL_AMD_MAX_RANK 8

typedef enum onnxl_amd_status {
  ONNXL_AMD_OK = 0,
  ONNXL_AMD_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument */
  ONNXL_AMD_UNSUPPORTED = 2,      /* valid for the reference, not handled on the GPU path */
  ONNXL_AMD_DEVICE_ERROR = 3,     /* HIP runtime failure */
  ONNXL_AMD_NOT_INITIALIZED = 4   /* onnxl_amd_init was not called */
} onnxl_amd_status;

typedef enum onnxl_amd_location { ONNXL_AMD_DEVICE = 0, ONNXL_AMD_HOST = 1 } onnxl_amd_location;

/* Element order of a payload.  Every tensor uses ONNXL_AMD_LAYOUT_ONNX except
 * a weight prepared by onnxl_amd_prepare_weight, which only the x input of
 * onnxl_amd_dequantize_linear_matmul accepts. */
typedef enum onnxl_amd_layout {
  ONNXL_AMD_LAYOUT_ONNX = 0,       /* row-major; 4-bit values two per byte, low nibble first */
  ONNXL_AMD_LAYOUT_TILED_INT4 = 1  /* the tiled INT4 / UINT4 form of onnxl_amd_prepare_weight */
} onnxl_amd_layout;

/* Mirrors the fields of the reference core::runtime::Tensor that kernels read
 * (core/runtime/memory/simple_tensor.h:526): data_type, shape, bytes. */
typedef struct onnxl_amd_tensor {
  int32_t data_type;                /* ONNX TensorProto.DataType code */
  int32_t rank;                     /* number of dims; -1 = absent optional input */
  int64_t dims[ONNXL_AMD_MAX_RANK]; /* row-major shape */
  void *data;                       /* payload (see location) */
  int64_t size_bytes;               /* payload bytes */
  int32_t location;                 /* onnxl_amd_location */
  int32_t layout;                   /* onnxl_amd_layout (0 = ONNX) */
} onnxl_amd_tensor;

/* Library lifetime.  init selects the device for all later calls on this
 * process; shutdown releases the workspace. */
int onnxl_amd_init(int device_ordinal);
int onnxl_amd_shutdown(void);
const char *onnxl_amd_last_error(void);
const char *onnxl_amd_version(void);

/* MatMul output shape (km/matmul_shape_utils.h:85-106): 1-D promotion, batch
 * broadcasting, promoted dims dropped.  out_dims holds ONNXL_AMD_MAX_RANK. */
int onnxl_amd_matmul_shape(const int64_t *a_dims, int32_t a_rank, const int64_t *b_dims,
                           int32_t b_rank, int64_t *out_dims, int32_t *out_rank);

/* MatMulInteger: Y = (A - a_zp) @ (B - b_zp) with int32 output.
 * A, B: UINT8 or INT8 (independently); zero points absent, scalar, [1], or
 * 1-D of size M (a) / N (b) with their input's dtype; Y: INT32.
 * Replaces kernel::MatMulInteger::operator()(a, b, a_zero_point,
 * b_zero_point, Tensor &output), km/kernel_matmul_integer.cc:231-234
 * (validation :178-208, arithmetic :89-176). */
int onnxl_amd_matmul_integer(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b,
                             const onnxl_amd_tensor *a_zero_point,
                             const onnxl_amd_tensor *b_zero_point, onnxl_amd_tensor *y,
                             void *stream);

/* QLinearMatMul: y = saturate(rint((float)Σ(a-za)(b-zb) * (a_s*b_s/y_s)) + zy).
 * a, b: UINT8/INT8; scales: FLOAT or FLOAT16 scalars; zero points: scalars
 * with their input's dtype; y dtype = y_zero_point dtype.  The sum is exact
 * for every K, as the reference's int64 sum (past K * max|a-za| * max|b-zb|
 * = 2^31 an int64-accumulating kernel runs instead of the MFMA GEMM).
 * Replaces kernel::QLinearMatMul::operator()(..., Tensor &output),
 * kq/kernel_qlinearmatmul.cc:242-267 (arithmetic :115-217). */
int onnxl_amd_qlinear_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *a_scale,
                             const onnxl_amd_tensor *a_zero_point, const onnxl_amd_tensor *b,
                             const onnxl_amd_tensor *b_scale,
                             const onnxl_amd_tensor *b_zero_point,
                             const onnxl_amd_tensor *y_scale,
                             const onnxl_amd_tensor *y_zero_point, onnxl_amd_tensor *y,
                             void *stream);

/* DequantizeLinear (opset 21 semantics of the reference): per-tensor,
 * per-axis (1-D scale of size x.shape[axis]) or blocked (scale rank == x
 * rank, only `axis` coarser; the block size is derived from the shapes).
 * x: UINT8, INT8, UINT16, INT16, INT32, FLOAT8E4M3FN, UINT4, INT4;
 * x_scale: FLOAT or FLOAT16; y dtype = x_scale dtype.
 * Replaces kernel::DequantizeLinear::operator() with and without zero point,
 * kq/kernel_dequantizelinear.cc:349-410, :426-502, :522-651, :670-693. */
int onnxl_amd_dequantize_linear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                                const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                onnxl_amd_tensor *y, void *stream);

/* QuantizeLinear: y = saturate(nearbyint(x / y_scale) + y_zero_point), the
 * division in IEEE fp32, for the integer outputs; the float outputs take the
 * reference's saturating cast of x / y_scale + y_zero_point (fp8: round to
 * nearest even; FLOAT4E2M1 and FLOAT6: nearest code, ties to even; without a
 * zero point nothing is added, so -0 stays -0).  x and y_scale: FLOAT or
 * FLOAT16.  The output dtype follows the reference's node dispatch
 * (kq/kernel_quantizelinear.cc:917-941): y_zero_point's dtype when it is
 * given (per-tensor, per-axis or blocked; UINT8, INT8, UINT16, INT16, UINT4,
 * INT4, UINT2, INT2, FLOAT8E4M3FN, FLOAT8E4M3FNUZ, FLOAT8E5M2,
 * FLOAT8E5M2FNUZ, FLOAT4E2M1, FLOAT6E2M3, FLOAT6E3M2), else output_dtype when
 * non-zero (UINT8, INT8, UINT16, INT16; FLOAT4E2M1 and FLOAT6 with a scalar
 * y_scale), else UINT8 with a scalar y_scale.  y must already carry that
 * dtype; sub-byte outputs are packed little-endian bit streams (element i at
 * bits i * bits onwards).  axis may be negative.
 * Replaces kernel::QuantizeLinear::operator(), kq/kernel_quantizelinear.cc:
 * 485-532 (per tensor), :543-648 (per tensor with zero point), :664-822 (per
 * axis and blocked with zero point), :833-916 (output_dtype). */
int onnxl_amd_quantize_linear(const onnxl_amd_tensor *x, const onnxl_amd_tensor *y_scale,
                              const onnxl_amd_tensor *y_zero_point, int64_t axis, int32_t output_dtype,
                              onnxl_amd_tensor *y, void *stream);

/* DynamicQuantizeLinear: x FLOAT (non-empty) -> y UINT8 of x's shape, y_scale a
 * 0-D FLOAT, y_zero_point a 0-D UINT8.  The range [min(x, 0), max(x, 0)] is
 * reduced on the device; scale = range / 255 (1 for an empty range).  The
 * reference rejects non-finite input; here the outputs cannot be inspected
 * without a synchronisation, so such input is reported by y_scale = NaN (the
 * caller checks it when it reads y_scale back).
 * Replaces kernel::DynamicQuantizeLinear::operator(),
 * kq/kernel_dynamicquantizelinear.cc:57-121. */
int onnxl_amd_dynamic_quantize_linear(const onnxl_amd_tensor *x, onnxl_amd_tensor *y,
                                      onnxl_amd_tensor *y_scale, onnxl_amd_tensor *y_zero_point,
                                      void *stream);

/* DequantizePacked: decodes a 1-D UINT8 vector in one of the reference's
 * fixed GGUF wire formats (`format`, e.g. "gguf:q4_0") into y of the given
 * shape and output_dtype (FLOAT, FLOAT16, BFLOAT16 or DOUBLE); the last
 * dimension holds whole blocks.  The GPU decodes the 20 formats without
 * codebooks (gguf:q4_0, q4_1, q5_0, q5_1, q8_0, q8_1, iq4_nl, q2_k, q3_k,
 * q4_k, q5_k, q6_k, q8_k, iq4_xs, tq1_0, tq2_0, mxfp4, nvfp4, q1_0, q2_0); the
 * reference's 7 codebook formats (iq1_s, iq1_m, iq2_xxs, iq2_xs, iq2_s,
 * iq3_xxs, iq3_s) return ONNXL_AMD_UNSUPPORTED, an unknown format
 * INVALID_ARGUMENT.
 * Replaces DequantizePackedTensor (onnx_core/runtime/dequantize_packed.cc:
 * 334-372) behind kernel::DequantizePacked::operator()
 * (kq/kernel_dequantize_packed.cc:11-15). */
int onnxl_amd_dequantize_packed(const onnxl_amd_tensor *x, const char *format, const int64_t *shape,
                                int32_t rank, int64_t output_dtype, onnxl_amd_tensor *y, void *stream);

/* Fused y = a @ W^T with W = DequantizePacked(x, format, shape = [N, K],
 * FLOAT16): a FLOAT16 [M, K], y FLOAT16 [M, N] (fp32 accumulation).  The
 * weight is in the ggml layout, each output's blocks contiguous along K; the
 * dequantized weights are rounded to FLOAT16 exactly as the unfused chain
 * rounds them, so only the fp32 summation order differs.  Every one of the
 * 27 GGUF profiles and any M: fused decode GEMVs for gguf:q4_0 / gguf:q8_0
 * (K % 64 == 0) and gguf:q4_k / gguf:q6_k with M <= 8, otherwise the weight
 * decoded to FLOAT16 [N, K] in the workspace and multiplied by the MFMA GEMM
 * reading its rows (no transpose written).  No
 * single reference kernel: it computes the DequantizePacked -> Transpose ->
 * MatMul chain, onnx_core/runtime/dequantize_packed.cc:334-372 ->
 * km/kernel_matmul.cc:181-223. */
int onnxl_amd_dequantize_packed_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x, const char *format,
                                       const int64_t *shape, int32_t rank, onnxl_amd_tensor *y, void *stream);

/* Convolution attributes, as the reference's ConvInteger / QLinearConv
 * Attributes: n_* entries of each array are used, 0 means the attribute is
 * absent (kernel_shape from w, strides and dilations 1, pads 0).  pads holds
 * the begin values of every spatial dim, then the end values. */
#define ONNXL_AMD_MAX_CONV_SPATIAL 3
enum {
  ONNXL_AMD_AUTO_PAD_NOTSET = 0,
  ONNXL_AMD_AUTO_PAD_SAME_UPPER = 1,
  ONNXL_AMD_AUTO_PAD_SAME_LOWER = 2,
  ONNXL_AMD_AUTO_PAD_VALID = 3
};
typedef struct onnxl_amd_conv_attrs {
  int32_t n_kernel_shape, n_strides, n_pads, n_dilations;
  int64_t kernel_shape[ONNXL_AMD_MAX_CONV_SPATIAL];
  int64_t strides[ONNXL_AMD_MAX_CONV_SPATIAL];
  int64_t pads[2 * ONNXL_AMD_MAX_CONV_SPATIAL];
  int64_t dilations[ONNXL_AMD_MAX_CONV_SPATIAL];
  int64_t group;
  int32_t auto_pad; /* ONNXL_AMD_AUTO_PAD_* */
} onnxl_amd_conv_attrs;

/* Output dims [N, M, out spatial...] of a convolution, with the reference's
 * attribute resolution (nn/kernel_conv_integer.cc:24-54, :107-141;
 * kq/kernel_qlinearconv.cc:53-119), for callers that allocate the output. */
int onnxl_amd_conv_shape(const int64_t *x_dims, int32_t x_rank, const int64_t *w_dims, int32_t w_rank,
                         const onnxl_amd_conv_attrs *attrs, int64_t *y_dims, int32_t *y_rank);

/* ConvInteger: x [N, C, spatial...] and w [M, C/group, kernel...] of INT8 or
 * UINT8, optional scalar x_zero_point and scalar or per-output-channel
 * w_zero_point; y INT32 [N, M, out...], the int32 sums of
 * (x - x_zp)(w - w_zp) over the taps inside x (wrapping like the
 * reference's int32 accumulator).  1 to 3 spatial dims.
 * Replaces kernel::ConvInteger::operator(), nn/kernel_conv_integer.cc:178-304. */
int onnxl_amd_conv_integer(const onnxl_amd_tensor *x, const onnxl_amd_tensor *w,
                           const onnxl_amd_tensor *x_zero_point, const onnxl_amd_tensor *w_zero_point,
                           const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y, void *stream);

/* QLinearConv: as ConvInteger with int64 sums, plus the optional INT32 bias B
 * [M], then y = saturate(nearbyint((float)sum * (x_scale * w_scale[m] /
 * y_scale)) + y_zero_point); FLOAT scalar x_scale / y_scale, scalar or
 * per-output-channel w_scale and w_zero_point; y dtype = y_zero_point's.
 * Replaces kernel::QLinearConv::operator(), kq/kernel_qlinearconv.cc:178-340. */
int onnxl_amd_qlinear_conv(const onnxl_amd_tensor *x, const onnxl_amd_tensor *x_scale,
                           const onnxl_amd_tensor *x_zero_point, const onnxl_amd_tensor *w,
                           const onnxl_amd_tensor *w_scale, const onnxl_amd_tensor *w_zero_point,
                           const onnxl_amd_tensor *y_scale, const onnxl_amd_tensor *y_zero_point,
                           const onnxl_amd_tensor *B, const onnxl_amd_conv_attrs *attrs, onnxl_amd_tensor *y,
                           void *stream);

/* MatMul for FLOAT16 / BFLOAT16 operands (fp32 accumulation, output rounded
 * to the input dtype).  Replaces kernel::MatMul::operator()(a, b, Tensor &)
 * for those dtypes, km/kernel_matmul.cc:242-253 (compute :61-147, :206-218). */
int onnxl_amd_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *b, onnxl_amd_tensor *y,
                     void *stream);

/* GroupedMatMul (onnx-light opset 29, the MoE expert contraction):
 * y[m, s, :] = input[m, :] @ W[g] (+ bias[g, :]), g = group_indices[m, s],
 * W[g] = weights[g] ([G, K, N]) or its transpose when transB != 0 (weights
 * [G, N, K]).  input, weights, bias and y FLOAT16 or BFLOAT16 (fp32 sums over
 * exact products; with a bias the sum is rounded to the dtype, the bias
 * added, the result rounded again, as MatMul followed by Add); group_indices
 * INT32 or INT64 [M, S]; y [M, S, N].  FLOAT and DOUBLE inputs, which the
 * reference also takes, return ONNXL_AMD_UNSUPPORTED, as do more than 4096
 * groups.  A group index outside [0, G) is an INVALID_ARGUMENT when the
 * indices are host memory; with device-resident indices the call cannot see
 * them before the work runs, and such a pair's row of y is NaN instead.
 * Replaces kernel::GroupedMatMul::operator(),
 * math/kernel_grouped_matmul.cc:48-103. */
int onnxl_amd_grouped_matmul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *weights,
                             const onnxl_amd_tensor *group_indices, const onnxl_amd_tensor *bias, int64_t transB,
                             onnxl_amd_tensor *y, void *stream);

/* Fused quantized MoE experts: y = GroupedMatMul(input, [Cast(to=cast_to)]
 * (DequantizeLinear(x, x_scale, x_zero_point, axis)), group_indices, bias,
 * transB), with x the quantized experts [G, K, N] (or [G, N, K] with transB):
 * INT4, UINT4, INT8, UINT8 or FLOAT8E4M3FN; per-tensor, per-axis or blocked
 * scales (FLOAT or FLOAT16) as DequantizeLinear takes them.  cast_to = 0
 * means no Cast node (the DequantizeLinear output dtype must then be the
 * input's).  input, bias and y as onnxl_amd_grouped_matmul (FLOAT16 or
 * BFLOAT16).  The experts are dequantized with the chain's roundings and
 * multiplied as GroupedMatMul does, except FLOAT8E4M3FN experts with FLOAT
 * scales constant along K within an expert (per tensor, per expert [G], per
 * column [N] or [G, 1, N]), cast_to = BFLOAT16, no zero point and transB = 0:
 * those run on the matrix cores with the fp8 codes as the B operand and the
 * fp32 sums multiplied by the scale, skipping the rounding of each scaled
 * weight to bfloat16 (at most 2^-9 relative per weight), as the fp8 path of
 * onnxl_amd_dequantize_linear_matmul does.  No single reference kernel: it
 * computes the chain kq/kernel_dequantizelinear.cc:522-693 ->
 * kernel_cast.cc:360-370 -> math/kernel_grouped_matmul.cc:22-103 that a
 * DequantizeLinear->[Cast]->GroupedMatMul subgraph runs node by node. */
int onnxl_amd_dequantize_linear_grouped_matmul(const onnxl_amd_tensor *input, const onnxl_amd_tensor *x,
                                               const onnxl_amd_tensor *x_scale, const onnxl_amd_tensor *x_zero_point,
                                               int64_t axis, int32_t cast_to, const onnxl_amd_tensor *group_indices,
                                               const onnxl_amd_tensor *bias, int64_t transB, onnxl_amd_tensor *y,
                                               void *stream);

/* Cast FLOAT -> FLOAT16 / BFLOAT16 (round-to-nearest-even), the Cast step
 * between DequantizeLinear and a bf16 MatMul.
 * Replaces the FLOAT->BFLOAT16 / FLOAT16 branch of the reference Cast kernel,
 * ext/kernels/kernels/tensor/kernel_cast.cc:360-370. */
int onnxl_amd_cast(const onnxl_amd_tensor *x, int32_t to, onnxl_amd_tensor *y, void *stream);

/* Transpose(x, perm = [1, 0]) of a 2-D tensor whose elements take 1, 2, 4 or
 * 8 bytes, into the preallocated y [x.dims[1], x.dims[0]].  Replaces the 2-D
 * case of the reference Transpose kernel, tensor/kernel_transpose.cc:98-111
 * (its preallocated-output checks and messages); other ranks and sub-byte
 * types return ONNXL_AMD_UNSUPPORTED.  The adapter uses it to lay a weight
 * decoded on the GPU as [N, K] out as [K, N] without a host round trip. */
int onnxl_amd_transpose_2d(const onnxl_amd_tensor *x, onnxl_amd_tensor *y, void *stream);

/* Fused Y = MatMul(A, [Cast(to=cast_to)](DequantizeLinear(x, x_scale,
 * x_zero_point, axis))) for a 2-D quantized weight x [K, N].  A: FLOAT16 or
 * BFLOAT16 [..., M, K]; the dequantized weight is rounded exactly as the
 * unfused reference chain rounds it (to x_scale's dtype, then to cast_to), so
 * only the fp32 summation order differs from the chain of the three kernels
 * above.  One exception: FLOAT8E4M3FN weights with FLOAT scales and
 * cast_to = BFLOAT16 on the matrix-core path (per-tensor or per-column scale,
 * no zero point, K % 32 == 0, N % 16 == 0) multiply the fp32
 * sums by the scale instead of rounding each scaled weight to bfloat16 (at
 * most 2^-9 relative per weight; with an infinite scale a column the chain
 * turns to NaN through 0 * inf is +-inf here).  cast_to = 0 means no Cast node (the DequantizeLinear output dtype
 * must then equal A's dtype).  Y dtype = A dtype.  x: INT4, UINT4, INT8,
 * UINT8, FLOAT8E4M3FN; per-tensor, per-axis (axis 1) or blocked along K
 * (axis 0) scales.  No single reference kernel: it computes the chain
 * kq/kernel_dequantizelinear.cc:522-693 -> kernel_cast.cc:360-370 ->
 * km/kernel_matmul.cc:181-223 that a DequantizeLinear->[Cast]->MatMul
 * subgraph runs node by node.  x may be a weight prepared by
 * onnxl_amd_prepare_weight (layout ONNXL_AMD_LAYOUT_TILED_INT4). */
int onnxl_amd_dequantize_linear_matmul(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x,
                                       const onnxl_amd_tensor *x_scale,
                                       const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                       int32_t cast_to, onnxl_amd_tensor *y, void *stream);

/* onnxl_amd_dequantize_linear_matmul with no allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, validation and results as
 * onnxl_amd_dequantize_linear_matmul (same kernels), but:
 * - every payload (A, x, x_scale, x_zero_point, y) must be device memory
 *   (no host staging; a host payload is an INVALID_ARGUMENT);
 * - its scratch is a fixed array of 8 MiB per device, held until the process
 *   ends: 64 KiB of counters (16384, one per 256-column strip of the ONNX-
 *   layout int4 GEMV) and 8128 KiB for split-K partial sums or a dequantised
 *   weight.  A call that needs more returns ONNXL_AMD_UNSUPPORTED, naming the
 *   sizes (the allocating entry point then serves it);
 * - it calls no hipMalloc / hipFree.
 * All calls on one device share that array: calls that overlap on one device
 * (different streams, or different threads without ordering) race.  The
 * counters are cleared once per device by onnxl_amd_init and every completed
 * call leaves them at zero. */
int onnxl_amd_dequantize_linear_matmul_noalloc(const onnxl_amd_tensor *a, const onnxl_amd_tensor *x,
                                               const onnxl_amd_tensor *x_scale,
                                               const onnxl_amd_tensor *x_zero_point, int64_t axis,
                                               int32_t cast_to, onnxl_amd_tensor *y, void *stream);

/* Session-time preparation of a constant INT4 / UINT4 weight x [K, N] (ONNX
 * layout) for onnxl_amd_dequantize_linear_matmul: writes it into `prepared`
 * (device memory of onnxl_amd_prepare_weight_size bytes, 16-byte aligned,
 * allocated by the caller) in a tiled order in which each 16-column tile's
 * full K range is contiguous, and sets prepared's data_type, dims and layout
 * (ONNXL_AMD_LAYOUT_TILED_INT4).  The prepared descriptor then replaces x in
 * every later call; the values, scales, zero points and results are those of
 * the original x.  This is the counterpart of the reference's kernel
 * preparations (core/runtime/kernels/kernel_context.h:45-76), through which
 * its Gemm kernel packs a constant B once per session
 * (km/kernel_gemm.cc:378-405, representation "Gemm:B:column-major-k-v1"). */
int onnxl_amd_prepare_weight_size(const onnxl_amd_tensor *x, int64_t *bytes);
int onnxl_amd_prepare_weight(const onnxl_amd_tensor *x, onnxl_amd_tensor *prepared, void *stream);

/* Session-time preparation of an ORT MatMulNBits weight (the format of
 * onnx_core/runtime/quantization.cc:916-930, decoded at :1806-1880) for
 * onnxl_amd_dequantize_linear_matmul, so that MatMul(A, W) with W [K, N] =
 * (code - zero point) * scale runs on the fused kernels without a dense W.
 * B: UINT8 [N, groups, block_size * bits / 8] (column n, row g * block + j at
 * bit (j % (8 / bits)) * bits of byte j / (8 / bits)); scales: FLOAT16
 * [N, groups]; zero_points: absent (2^(bits-1)) or packed UINT8 codes
 * [N, ceil(groups * bits / 8)].  Writes into caller-allocated device buffers
 * of the sizes onnxl_amd_prepare_matmul_nbits_size returns (16-byte aligned):
 *   weight: bits 4 -> the tiled layout of onnxl_amd_prepare_weight, INT4 (no
 *           zero points: code - 8) or UINT4; bits 8 -> [K, N] INT8 (code -
 *           128) or UINT8;
 *   scale: FLOAT16 [groups, N]; zero_point: UINT4 / UINT8 [groups, N] (set
 *           absent, rank -1, without zero points),
 * and sets their dtypes, dims and layouts; then pass (A, weight, scale,
 * zero_point, axis = 0, cast_to = 0) to onnxl_amd_dequantize_linear_matmul.
 * The format's checks raise INVALID_ARGUMENT with the reference's messages
 * (dimensions, block size, nonfinite scales, nonzero zero-point padding).
 * 2-bit weights, K not a multiple of block_size, FLOAT / BFLOAT16 scales and
 * floating-point zero points return ONNXL_AMD_UNSUPPORTED.  No single
 * reference kernel: the reference materialises the dense weight. */
int onnxl_amd_prepare_matmul_nbits_size(int64_t K, int64_t N, int64_t bits, int64_t block_size, int has_zero_points,
                                        int64_t *weight_bytes, int64_t *scale_bytes, int64_t *zero_point_bytes);
int onnxl_amd_prepare_matmul_nbits(const onnxl_amd_tensor *B, const onnxl_amd_tensor *scales,
                                   const onnxl_amd_tensor *zero_points, int64_t K, int64_t N, int64_t bits,
                                   int64_t block_size, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                                   onnxl_amd_tensor *zero_point, void *stream);

/* AWQ checkpoint weights (onnx_core/runtime/awq.cc; the reference imports
 * them with ImportAwqWeights, quantization.h:724, and decodes them with
 * ReconstructAwqWeights, quantization.h:735, awq.cc:370-387, through
 * DequantizeTensor, quantization.cc:3121-3147).  variant "gemm" (bits 4 or
 * 8): qweight INT32 [K, N * bits / 32] (4 bits: column n at nibble
 * {0,4,1,5,2,6,3,7}[n % 8] of word n / 8), qzeros INT32 [groups, N * bits /
 * 32], scales FLOAT16 / BFLOAT16 [groups, N]; "gemv" (4 bits): qweight INT32
 * [N, K / 8], qzeros INT32 [N, padded / 8], scales FLOAT16 [N, padded];
 * "gemv_fast" / "llm-awq" (4 bits): qweight INT16 [N / 4, K], qzeros (the
 * float zero terms; "scaled_zeros" upstream for llm-awq) and scales FLOAT16
 * [padded, N] (padded = the group count rounded as awq.cc:97-100 does).
 * W [K, N] = (code - zero) * scale (gemv_fast / llm-awq: code * scale +
 * zero term).  The format's checks raise INVALID_ARGUMENT with the
 * reference's messages.
 *
 * onnxl_amd_prepare_awq writes the fused DequantizeLinear -> MatMul operands
 * into caller-allocated device buffers of the sizes onnxl_amd_prepare_awq_size
 * returns (16-byte aligned): weight UINT4 in the tiled layout of
 * onnxl_amd_prepare_weight (4 bits) or UINT8 [K, N] (8 bits), zero_point UINT4
 * / UINT8 [groups, N], scale FLOAT16 [groups, N] (FLOAT16 scales) or FLOAT
 * (BFLOAT16 scales, widened exactly: pass cast_to = BFLOAT16), and sets their
 * descriptors; then pass (A, weight, scale, zero_point, axis = 0, cast_to) to
 * onnxl_amd_dequantize_linear_matmul.  gemv_fast / llm-awq return
 * ONNXL_AMD_UNSUPPORTED there (float zero terms).
 *
 * onnxl_amd_dequantize_awq decodes every variant to y [N, K] (the reference's
 * logical [out_features, in_features]) of y's dtype: FLOAT, FLOAT16,
 * BFLOAT16 or DOUBLE, rounded to nearest even, raising the reference's
 * "Dequantization output dtype overflow." where a value does not fit. */
int onnxl_amd_prepare_awq_size(const char *variant, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                               int32_t scale_dtype, int64_t *weight_bytes, int64_t *scale_bytes,
                               int64_t *zero_point_bytes);
int onnxl_amd_prepare_awq(const char *variant, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                          const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                          onnxl_amd_tensor *weight, onnxl_amd_tensor *scale, onnxl_amd_tensor *zero_point,
                          void *stream);
int onnxl_amd_dequantize_awq(const char *variant, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                             const onnxl_amd_tensor *scales, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                             onnxl_amd_tensor *y, void *stream);

/* GPTQ checkpoint weights (onnx_core/runtime/gptq.cc; ImportGptqWeights,
 * quantization.h:629, ReconstructGptqWeights, quantization.h:644, gptq.cc:399-412).  format
 * "gptq" (stored zero + 1), "gptq_v2" or "gptq_p"; bits 2-8 (5-7 and gptq_p
 * at 3 bits in planar 32-code blocks); words INT8 / INT16 / INT32 / INT64
 * (qweight's dtype): qweight [ceil(K * bits / word bits), N] (column n's
 * codes as a little-endian bit stream down the rows), qzeros [groups,
 * ceil(N * bits / word bits)], scales FLOAT16 / BFLOAT16 / FLOAT [groups, N],
 * g_idx INT32 [K] (the group of each row).  W [K, N] = (code - zero) *
 * scale[g_idx[k]].  The format's checks raise INVALID_ARGUMENT with the
 * reference's messages.
 *
 * onnxl_amd_prepare_gptq writes the fused operands as onnxl_amd_prepare_awq
 * does: codes of at most 4 bits as tiled UINT4, 5-8 bits as UINT8 [K, N];
 * scale FLOAT16 or FLOAT (BFLOAT16 widened; FLOAT / BFLOAT16 scales then take
 * cast_to = A's dtype).  A group map other than g_idx[k] = k / group_size
 * (act-order) and K not a multiple of group_size return ONNXL_AMD_UNSUPPORTED
 * there.  onnxl_amd_dequantize_gptq decodes every format and group map to
 * y [N, K] as onnxl_amd_dequantize_awq does. */
int onnxl_amd_prepare_gptq_size(const char *format, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                                int32_t word_dtype, int32_t scale_dtype, int64_t *weight_bytes, int64_t *scale_bytes,
                                int64_t *zero_point_bytes);
int onnxl_amd_prepare_gptq(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                           const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N,
                           int64_t bits, int64_t group_size, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                           onnxl_amd_tensor *zero_point, void *stream);
int onnxl_amd_dequantize_gptq(const char *format, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *qzeros,
                              const onnxl_amd_tensor *scales, const onnxl_amd_tensor *g_idx, int64_t K, int64_t N,
                              int64_t bits, int64_t group_size, onnxl_amd_tensor *y, void *stream);

/* BitBLAS row-packed weights (the encoding "onnx_light.bitblas_weights.v1":
 * ImportBitblasWeights / ExportBitblasWeights, quantization.h:664-670,
 * decoded by ReconstructBitblasWeights, bitblas.cc:341-347, which goes through
 * the GPTQ affine reconstruction, gptq.cc:222-228).  method "gptq" or "awq"
 * (the originating quantizer), K = in_features (a multiple of 32), N =
 * out_features (a multiple of 32 for gptq, 16 for awq), bits 2-8 (gptq: 2, 4
 * or 8), group_size -1, K, 32, 64 or 128, symmetric (codes from symmetric
 * GPTQ are stored signed and have no qzeros).  qweight INT8 [N, K * bits / 8]
 * (row n: its K codes as a little-endian bit stream), scales FLOAT16
 * [N, groups], qzeros INT8 [groups, N * bits / 8] (row g: N zero fields) or
 * empty / null when symmetric GPTQ.  W[n, k] = (code - zero) * scale in fp32
 * (exact: a code difference of at most 8 bits times an fp16 scale), the
 * signed codes XOR the midpoint with the midpoint as zero.  The format's
 * checks (Geometry, CheckTensor, CheckScales, bitblas.cc:38-106, 228-237)
 * raise INVALID_ARGUMENT with the reference's messages.
 *
 * onnxl_amd_dequantize_bitblas decodes to y [N, K] as onnxl_amd_dequantize_awq
 * does.  onnxl_amd_prepare_bitblas writes the fused operands as
 * onnxl_amd_prepare_awq does (codes of at most 4 bits tiled UINT4, else UINT8
 * [K, N]; zero points UINT4 / UINT8 [groups, N]; scales FLOAT16 [groups, N]);
 * pass them to onnxl_amd_dequantize_linear_matmul with axis 0. */
int onnxl_amd_dequantize_bitblas(const char *method, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *scales,
                                 const onnxl_amd_tensor *qzeros, int64_t K, int64_t N, int64_t bits,
                                 int64_t group_size, int32_t symmetric, onnxl_amd_tensor *y, void *stream);
int onnxl_amd_prepare_bitblas_size(const char *method, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                                   int32_t symmetric, int64_t *weight_bytes, int64_t *scale_bytes,
                                   int64_t *zero_point_bytes);
int onnxl_amd_prepare_bitblas(const char *method, const onnxl_amd_tensor *qweight, const onnxl_amd_tensor *scales,
                              const onnxl_amd_tensor *qzeros, int64_t K, int64_t N, int64_t bits, int64_t group_size,
                              int32_t symmetric, onnxl_amd_tensor *weight, onnxl_amd_tensor *scale,
                              onnxl_amd_tensor *zero_point, void *stream);

/* bitsandbytes weights (onnx_core/runtime/bitsandbytes.cc; the encoding
 * "onnx_light.bitsandbytes_weights.v1", imported by ImportBitsAndBytesWeights
 * and decoded by ReconstructBitsAndBytesWeights, bitsandbytes.cc:502-539,
 * through DequantizeTensor).  The caller parses the weight's quant state
 * (the JSON of bitsandbytes.cc:59-199) and passes its numbers: format 0 nf4,
 * 1 fp4, 2 int8; the logical [rows, cols] = [out_features, in_features];
 * block_size (32 .. 4096, a power of two; 0 for int8); nested_block_size 0 or
 * 256 and its nested_offset.  4-bit: weight UINT8 with ceil(rows * cols / 2)
 * elements (the flattened weight's codes, the even element in the high
 * nibble), absmax FLOAT [blocks] or, nested, UINT8 [blocks] with
 * nested_absmax FLOAT [ceil(blocks / 256)] and nested_quant_map FLOAT [256],
 * quant_map FLOAT [16] (the format's own table); int8: weight INT8
 * [rows, cols], absmax the FLOAT row maxima weight_scb [rows], the rest
 * null.  The reference's checks (Geometry, CheckTensor, CheckParameters,
 * bitsandbytes.cc:222-258, 317-379) raise INVALID_ARGUMENT with its messages.
 *
 * onnxl_amd_dequantize_bitsandbytes decodes to y [rows, cols] of y's dtype
 * (FLOAT, FLOAT16 or BFLOAT16): value = fp32(table[code] * scale), scale the
 * block's absmax, or fp32(fp32(nested_quant_map[code] * nested_absmax) +
 * nested_offset), or the row's fp32(weight_scb / 127); rounded to nearest
 * even, a value that is not finite raising "bitsandbytes nonfinite
 * reconstruction.".
 *
 * onnxl_amd_prepare_bitsandbytes runs the same checks, reconstructs every
 * value in reconstruction_dtype (the activations' dtype of the MatMul it
 * feeds) to raise that error once, and writes the resolved FLOAT scale of
 * every block (int8: every row) into a caller-allocated device buffer of
 * onnxl_amd_prepare_bitsandbytes_size bytes.  onnxl_amd_bitsandbytes_matmul
 * then computes MatMul(a, Transpose(Dequantize(Q, dtype = a's dtype))) per
 * call from the unchanged weight and those scales: y [..., rows] of a's
 * dtype (FLOAT16 or BFLOAT16) for a [..., cols]; no counterpart in the
 * reference as one call (its chain is the Dequantize kernel,
 * kernels/kernel_dequantize.cc:10-16, then Transpose and MatMul,
 * km/kernel_matmul.cc:225-253). */
int onnxl_amd_dequantize_bitsandbytes(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                      int64_t nested_block_size, float nested_offset, const onnxl_amd_tensor *weight,
                                      const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
                                      const onnxl_amd_tensor *nested_absmax,
                                      const onnxl_amd_tensor *nested_quant_map, onnxl_amd_tensor *y, void *stream);
int onnxl_amd_prepare_bitsandbytes_size(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                        int64_t *scale_bytes);
int onnxl_amd_prepare_bitsandbytes(int32_t format, int64_t rows, int64_t cols, int64_t block_size,
                                   int64_t nested_block_size, float nested_offset, const onnxl_amd_tensor *weight,
                                   const onnxl_amd_tensor *absmax, const onnxl_amd_tensor *quant_map,
                                   const onnxl_amd_tensor *nested_absmax, const onnxl_amd_tensor *nested_quant_map,
                                   int32_t reconstruction_dtype, onnxl_amd_tensor *scales, void *stream);
int onnxl_amd_bitsandbytes_matmul(const onnxl_amd_tensor *a, int32_t format, int64_t rows, int64_t cols,
                                  int64_t block_size, const onnxl_amd_tensor *weight, const onnxl_amd_tensor *scales,
                                  onnxl_amd_tensor *y, void *stream);

/* VPTQ weights (the encoding "onnx_light.vptq_weights.v1" of ai.rt:Dequantize:
 * ImportVptqWeights / ExportVptqWeights, quantization.h:898-902, decoded by
 * ReconstructVptqWeights, vptq.cc:401-443, through DequantizeTensor).  The
 * constructor metadata the layout depends on (VptqWeights,
 * quantization.h:884-895; index 0 of the pairs is the outlier codebook's,
 * 1 the main one's): */
typedef struct onnxl_amd_vptq_config {
  int64_t in_features, out_features, bits;
  int64_t vector_lens[2], num_centroids[2], num_res_centroids[2];
  double npercent;
  int64_t group_size, group_num;
  int32_t enable_norm, norm_dim, enable_perm;
} onnxl_amd_vptq_config;
/* Tensors (the checkpoint's names): indices INT32 [groups, vectors, words],
 * centroids ("centroids.weight") of the codebook dtype (FLOAT, FLOAT16 or
 * BFLOAT16) [groups, num_centroids[1] * vector_lens[1]]; res_centroids when
 * num_res_centroids[1] > 1; outlier_centroids and outlier_indices when
 * npercent > 0; weight_scale and weight_bias with enable_norm; perm INT32 [k]
 * with enable_perm; absent ones null.  The layout (outlier columns, groups,
 * index widths: Layout, vptq.cc:52-129) and the tensor, index, outlier-index
 * and permutation checks (CheckData, :203-240) raise INVALID_ARGUMENT with
 * the reference's messages.  Decodes to y [out_features, in_features] of y's
 * dtype (FLOAT, FLOAT16, BFLOAT16 or DOUBLE): the codebook values with the
 * residual and norm steps rounded to the codebook dtype, then WriteFloat
 * (quantization.cc:184-201, its nonfinite and range errors). */
int onnxl_amd_dequantize_vptq(const onnxl_amd_vptq_config *config, const onnxl_amd_tensor *indices,
                              const onnxl_amd_tensor *centroids, const onnxl_amd_tensor *res_centroids,
                              const onnxl_amd_tensor *outlier_centroids, const onnxl_amd_tensor *outlier_indices,
                              const onnxl_amd_tensor *weight_scale, const onnxl_amd_tensor *weight_bias,
                              const onnxl_amd_tensor *perm, onnxl_amd_tensor *y, void *stream);

/* GPTQModel FP8 weights (the encoding "onnx_light.gptqmodel_fp8_weights.v1"
 * of ai.rt:Dequantize: ImportGptqModelFp8Weights / ExportGptqModelFp8Weights,
 * quantization.h:603-612, decoded by ReconstructGptqModelFp8Weights,
 * gptqmodel_fp8.cc:284-300, through DequantizeTensor).  weight [N, K] =
 * [out_features, in_features] of FP8 codes whose data_type names the format
 * (FLOAT8E4M3FN, FLOAT8E4M3FNUZ, FLOAT8E5M2, FLOAT8E5M2FNUZ or FLOAT8E8M0),
 * weight_scale_inv FLOAT: [] for weight_scale_method "tensor", [N] for
 * "row", [N / b0, K / b1] for "block" with weight_block_size {b0, b1}
 * (block_rank 2; 0 otherwise).  Decodes to y [N, K] of y's dtype (FLOAT,
 * FLOAT16, BFLOAT16 or DOUBLE): value = float(code) / inverse scale,
 * correctly rounded (gptqmodel_fp8.cc:160-162), then WriteFloat's rounding.
 * The reference's checks (Geometry, the import's tensor check, CheckData:
 * :58-101, 246-254, 164-173) and WriteFloat's range check raise
 * INVALID_ARGUMENT with its messages, in its order. */
int onnxl_amd_dequantize_gptqmodel_fp8(int64_t in_features, int64_t out_features, const char *weight_scale_method,
                                       const int64_t *weight_block_size, int32_t block_rank,
                                       const onnxl_amd_tensor *weight, const onnxl_amd_tensor *weight_scale_inv,
                                       onnxl_amd_tensor *y, void *stream);

/* MX and NVFP4 weights (the encodings "onnx_light.mxfp4_weights.v1",
 * "onnx_light.mxfp6_e2m3_weights.v1", "onnx_light.mxfp8_weights.v1" and
 * "onnx_light.nvfp4_weights.v1" of ai.rt:Dequantize: ImportMxfp4Weights /
 * ImportMxfp6E2m3Weights / ImportMxfp8Weights / ImportNvfp4Weights and their
 * exporters, quantization.h:943-1012, decoded through DequantizeTensor,
 * quantization.cc:2032-2085).  format "mxfp4": weight UINT8 [rows, cols / 2]
 * (E2M1 codes, low nibble first), weight_scale UINT8 [rows, cols / 32] (E8M0);
 * "mxfp6_e2m3": weight UINT8 [rows, cols / 4 * 3] (E2M3 codes, LSB first),
 * weight_scale UINT8 [rows, cols / 32]; "mxfp8": weight FLOAT8E4M3FN
 * [rows, cols], weight_scale UINT8 [rows, cols / 32]; "nvfp4": weight UINT8
 * [rows, cols / 2], weight_scale FLOAT8E4M3FN [rows, cols / 16] and
 * weight_global_scale (ignored by the other formats).  Decodes to y
 * [rows, cols] of y's dtype (FLOAT, FLOAT16, BFLOAT16 or DOUBLE): code value
 * x 2^(e - 127) (NVFP4: x (local / global), the quotient rounded once), one
 * fp32 rounding, then WriteFloat's rounding.  The import's checks and the
 * reconstruction walk raise INVALID_ARGUMENT with the reference's messages,
 * the first failing group and element in the reference's order. */
int onnxl_amd_dequantize_mx_weights(const char *format, const onnxl_amd_tensor *weight,
                                    const onnxl_amd_tensor *weight_scale, float weight_global_scale,
                                    onnxl_amd_tensor *y, void *stream);

/* EXL3 weights (the encoding "onnx_light.exl3_weights.v1" of ai.rt:Dequantize,
 * GPTQModel's EXL3 module: ImportExl3Weights / ExportExl3Weights,
 * quantization.h:847-852, decoded by ReconstructExl3Weights, exl3.cc:309-357,
 * through DequantizeTensor).  trellis INT16 [k / 16, n / 16, 16 * bits]
 * (bits 1..8), suh FLOAT16 [k], svh FLOAT16 [n], and at most one codebook
 * marker, an INT32 scalar: mcg (0xCBAC1FED) or mul1 (0x83DCD12D); neither
 * selects the 3INST codebook.  Decodes to y [k, n] of y's dtype (FLOAT,
 * FLOAT16, BFLOAT16 or DOUBLE): trellis states through the codebook (binary16),
 * normalised 128-point Hadamard butterflies down the columns, x suh, the same
 * along the rows, x svh, every step one fp32 rounding, then WriteFloat's
 * rounding.  Validate's checks (exl3.cc:136-165; the upstream revision is the
 * exporter's) raise INVALID_ARGUMENT with the reference's messages, in its
 * order. */
int onnxl_amd_dequantize_exl3(const onnxl_amd_tensor *trellis, const onnxl_amd_tensor *suh,
                              const onnxl_amd_tensor *svh, const onnxl_amd_tensor *mcg, const onnxl_amd_tensor *mul1,
                              onnxl_amd_tensor *y, void *stream);

/* QQQ weights (the encoding "onnx_light.qqq_weights.v1" of ai.rt:Dequantize:
 * ImportQqqWeights / ExportQqqWeights, quantization.h, decoded by
 * ReconstructQqqWeights, qqq.cc:346-358, through DequantizeTensor).  The
 * caller passes the exported numbers and tensors: in_features k and
 * out_features n (multiples of 64), group_size -1 or 128, bits 4; B INT32
 * [k / 16, 2n] (the packed, permuted four-bit codes), s_channel FLOAT [1, n],
 * s_group FLOAT16 [k / 128, n] when grouped (group 128 and k != 128), else
 * FLOAT16 [0] or null.  The reference's checks (Geometry, CheckTensor,
 * qqq.cc:38-56, 136-141, with DecodeValues' 1 << 30 byte limit) raise
 * INVALID_ARGUMENT with its messages.
 *
 * onnxl_amd_dequantize_qqq decodes to y [n, k] of y's dtype (FLOAT, FLOAT16,
 * BFLOAT16 or DOUBLE): value = fp32(integer * channel scale), integer =
 * clamp(round-half-even((code - 8) * group scale), -128, 127) when grouped,
 * else the signed code * 16 (qqq.cc:185-202), then WriteFloat's rounding
 * (quantization.cc:184-201); CheckData's errors (qqq.cc:204-218: a channel or
 * group scale not finite or negative, a value not finite) and WriteFloat's
 * "Dequantization output dtype overflow." in the reference's order.
 *
 * onnxl_amd_prepare_qqq runs the same checks in `dtype` (the activations'
 * dtype of the MatMul it feeds) and writes the operands of
 * onnxl_amd_dequantize_linear_matmul into caller-allocated, 16-byte aligned
 * device buffers of onnxl_amd_prepare_qqq_size bytes: weight INT4 [k, n] in
 * the tiled layout with scale FLOAT [n] = 16 * channel scale (per channel),
 * or INT8 [k, n] holding the integers with scale = the channel scales
 * (grouped); it sets both descriptors.  MatMul(A, Transpose(Dequantize(Q,
 * dtype = A's dtype))) is then onnxl_amd_dequantize_linear_matmul(A, weight,
 * scale, null, axis 1, cast_to = A's dtype), value for value (x * scale
 * rounds the same exact product once).  A per-channel weight whose 16 *
 * channel scale overflows FLOAT returns ONNXL_AMD_UNSUPPORTED there. */
int onnxl_amd_dequantize_qqq(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                             const onnxl_amd_tensor *B, const onnxl_amd_tensor *s_channel,
                             const onnxl_amd_tensor *s_group, onnxl_amd_tensor *y, void *stream);
int onnxl_amd_prepare_qqq_size(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                               int64_t *weight_bytes, int64_t *scale_bytes);
int onnxl_amd_prepare_qqq(int64_t in_features, int64_t out_features, int64_t group_size, int64_t bits,
                          const onnxl_amd_tensor *B, const onnxl_amd_tensor *s_channel,
                          const onnxl_amd_tensor *s_group, int32_t dtype, onnxl_amd_tensor *weight,
                          onnxl_amd_tensor *scale, void *stream);

/* Waits for all work queued by this library on `stream`. */
int onnxl_amd_synchronize(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ONNXL_AMD_H_ */
