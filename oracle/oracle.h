/*
 * CPU oracle for the quantized-matmul path: a plain-C restatement of the
 * onnx-light reference arithmetic, used ONLY as the parity checker (tests,
 * smoke) and as the reported CPU baseline (bench.py `cpu_baseline`).  Nothing
 * in the shipped library links or calls this code.
 *
 * Each function cites the reference file:line whose semantics it restates.
 * Paths are relative to the onnx-light source tree:
 *   km/ = onnx_light/onnx_extensions/kernels/kernels/math/
 *   kq/ = onnx_light/onnx_extensions/kernels/kernels/quantization/
 *   rk/ = onnx_light/onnx_core/runtime/kernels/
 *
 * Pinning (how each function is checked independently of this restatement;
 * the tests live in tests/test_oracle_*.py):
 *   codecs        - exhaustive over all 2^8 / 2^16 codes against closed forms
 *                   (numpy float16, bit arithmetic), plus the reference's
 *                   fp8 and fp16 known-answer bit patterns.
 *   SplitMix64    - published first outputs of canonical SplitMix64, seed 0.
 *   MatMulInteger - reference known-answer tests + brute force in numpy int64.
 *   QLinearMatMul - reference known-answer tests (2-D u8/s8, ties-to-even,
 *                   saturation) + numpy float32 closed form.
 *   DequantizeLinear - reference known-answer tests (per-tensor, per-axis,
 *                   blocked, fp16, fp8, int4/uint4) + numpy closed form.
 *   MatMul fp16/bf16 - reference known-answer test + float64 bound.
 *   QuantizeLinear - the reference's known answers (u8/i8/u16/i16 per-tensor,
 *                   per-axis u8 and u16, fp16 rounding, fp8 e4m3fn, int4/uint4
 *                   per-axis) + numpy float32 closed form (true division,
 *                   np.rint, clip) over random inputs.
 *   DynamicQuantizeLinear - the reference's known answers (scale, zero point
 *                   and the ONNX export cases' outputs, all-zero input,
 *                   non-finite rejection) + numpy float32 closed form.
 * No function is "parity unpinned".
 */
#ifndef ONNXL_AMD_ORACLE_H_
#define ONNXL_AMD_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ONNX TensorProto.DataType codes used on this path. */
enum {
  ORC_FLOAT = 1, ORC_UINT8 = 2, ORC_INT8 = 3, ORC_UINT16 = 4, ORC_INT16 = 5,
  ORC_INT32 = 6, ORC_FLOAT16 = 10, ORC_BFLOAT16 = 16, ORC_FLOAT8E4M3FN = 17,
  ORC_FLOAT8E4M3FNUZ = 18, ORC_FLOAT8E5M2 = 19, ORC_FLOAT8E5M2FNUZ = 20, ORC_UINT4 = 21, ORC_INT4 = 22,
  ORC_FLOAT4E2M1 = 23, ORC_UINT2 = 25, ORC_INT2 = 26, ORC_FLOAT6E2M3 = 27, ORC_FLOAT6E3M2 = 28
};

/* ---- scalar codecs ---- */
uint16_t orc_f32_to_f16(float f);       /* rk/cast_helper.cc:51-87  */
float orc_f16_to_f32(uint16_t h);       /* rk/cast_helper.cc:89-122 */
uint16_t orc_f32_to_bf16(float f);      /* rk/cast_helper.cc:124-134 */
float orc_bf16_to_f32(uint16_t b);      /* rk/cast_helper.cc:136-141 */
uint8_t orc_f32_to_f8e4m3fn(float v);   /* rk/cast_float8.cc:27-81  */
float orc_f8e4m3fn_to_f32(uint8_t v);   /* rk/cast_float8.cc:83-118 */
uint8_t orc_read_4bit(const uint8_t *data, int64_t i); /* rk/cast_sub_byte.h:57-60 */
/* The further DequantizeLinear input codecs (rk/cast_float8.cc:174-380,
 * rk/cast_helper.cc:161-256, rk/cast_sub_byte.h:71-75): element i of a packed
 * buffer decoded to float. */
float orc_f8e4m3fnuz_to_f32(uint8_t v);
float orc_f8e5m2_to_f32(uint8_t v);
float orc_f8e5m2fnuz_to_f32(uint8_t v);
float orc_f4e2m1_to_f32(uint8_t nibble);
float orc_f6_to_f32(uint8_t bits, int dtype);
uint8_t orc_read_2bit(const uint8_t *data, int64_t i);
uint8_t orc_read_6bit(const uint8_t *data, int64_t i);
/* the decoded value of element i of x in dtype (every DequantizeLinear input) */
float orc_dq_decode(const void *x, int dtype, int64_t i);
void orc_dq_decode_n(const void *x, int dtype, int64_t n, float *out);
/* the QuantizeLinear float encoders (rk/cast_float8.cc, rk/cast_helper.cc):
 * fp32 -> FLOAT8E4M3FN / FNUZ / E5M2 / E5M2FNUZ, FLOAT4E2M1, FLOAT6 code */
uint8_t orc_f32_to_float_code(float v, int dtype);
int8_t orc_int4_to_i8(uint8_t nibble);  /* rk/cast_sub_byte.cc:81-88 */

/* Bulk codec helpers (same semantics as the scalar ones). */
void orc_f32_to_f16_n(const float *src, int64_t n, uint16_t *dst);
void orc_f16_to_f32_n(const uint16_t *src, int64_t n, float *dst);
void orc_f32_to_bf16_n(const float *src, int64_t n, uint16_t *dst);
void orc_bf16_to_f32_n(const uint16_t *src, int64_t n, float *dst);
void orc_f32_to_f8e4m3fn_n(const float *src, int64_t n, uint8_t *dst);
void orc_f8e4m3fn_to_f32_n(const uint8_t *src, int64_t n, float *dst);

/* ---- SplitMix64 (rk/random.cc:32-106) ---- */
uint64_t orc_splitmix64_next(uint64_t *state);
void orc_rand_uniform(uint64_t seed, int64_t n, double *out);
int orc_rand_int(int64_t low, int64_t high, uint64_t seed, int64_t n, int64_t *out);
void orc_randn(uint64_t seed, int64_t n, double *out);

/* ---- MatMul shape rules (km/matmul_shape_utils.h:24-106) ----
 * Writes the broadcast output shape; returns 0, or a nonzero code for
 * rank-0 (1), inner-dimension mismatch (2) or batch broadcast failure (3). */
int orc_matmul_output_shape(const int64_t *a_shape, int a_rank, const int64_t *b_shape,
                            int b_rank, int64_t *out_shape, int *out_rank);

/* ---- MatMulInteger (km/kernel_matmul_integer.cc:89-176) ----
 * a/b are UINT8 or INT8 element arrays; a_zp has a_zp_count (1 or M) int32
 * values, b_zp has b_zp_count (1 or N) values.  int32 accumulation with
 * two's-complement wrap (the reference's int32 `acc`). */
int orc_matmul_integer(const void *a, int a_dtype, const int64_t *a_shape, int a_rank,
                       const void *b, int b_dtype, const int64_t *b_shape, int b_rank,
                       const int32_t *a_zp, int64_t a_zp_count, const int32_t *b_zp,
                       int64_t b_zp_count, int32_t *y);

/* ---- QLinearMatMul (kq/kernel_qlinearmatmul.cc:115-217) ----
 * Row range [row_begin, row_end) of every batch matrix is computed (the full
 * job is row_begin=0, row_end=-1); used to time a bounded CPU sample. */
int orc_qlinear_matmul(const void *a, int a_dtype, const int64_t *a_shape, int a_rank,
                       int32_t a_zp, float a_scale, const void *b, int b_dtype,
                       const int64_t *b_shape, int b_rank, int32_t b_zp, float b_scale,
                       float y_scale, int32_t y_zp, int y_dtype, void *y, int64_t row_begin,
                       int64_t row_end);

/* ---- DequantizeLinear (kq/kernel_dequantizelinear.cc:65-693) ----
 * scale is FLOAT or FLOAT16 (the output dtype follows it); zp may be NULL
 * (zero point 0).  scale_count==1 selects per-tensor, scale_rank==x_rank
 * blocked, otherwise per-axis.  Returns 0 on success. */
int orc_dequantize_linear(const void *x, int x_dtype, const int64_t *x_shape, int x_rank,
                          const void *scale, int scale_dtype, const int64_t *s_shape,
                          int s_rank, const void *zp, int64_t axis, void *y);

/* ---- MatMul FLOAT (km/kernel_matmul.cc:61-147): k-sequential, no FMA. ----
 * Row range as for orc_qlinear_matmul; nthreads>1 splits rows over threads
 * (the reference parallelises over output elements; per-element order is
 * unchanged, so the result does not depend on the split). */
int orc_matmul_f32(const float *a, const int64_t *a_shape, int a_rank, const float *b,
                   const int64_t *b_shape, int b_rank, float *y, int64_t row_begin,
                   int64_t row_end, int nthreads);

/* ---- MatMul FLOAT16/BFLOAT16 (km/kernel_matmul.cc:206-218):
 * PromoteToFloat32 -> MatMulCompute<float> -> DemoteFromFloat32 ---- */
int orc_ort_nbits_decode(const uint8_t *B, const double *scales, int zp_kind, const uint8_t *zp_codes,
                         const double *zp_values, int64_t K, int64_t N, int bits, int64_t block, double *out);
int orc_grouped_matmul(int dtype, const void *x, int64_t M, int64_t K, const void *w, int64_t G, int64_t N,
                       int transB, const int64_t *idx, int64_t S, const void *bias, void *y);
int orc_matmul_half(const uint16_t *a, const int64_t *a_shape, int a_rank, const uint16_t *b,
                    const int64_t *b_shape, int b_rank, int dtype, uint16_t *y,
                    int64_t row_begin, int64_t row_end, int nthreads);

/* ---- QuantizeLinear (kq/kernel_quantizelinear.cc) ----
 * y = saturate(nearbyint(x / scale) + zero_point) for integer outputs
 * (:67-84 per-tensor, :133-174 per-axis, :339-380 blocked, :176-200 and
 * :435-457 4-bit), y = fp8(x / scale + zero_point) for FLOAT8E4M3FN
 * (:257-270, :459-473).  x and scale are FLOAT or FLOAT16 (decoded to fp32,
 * :33-55); fp32 division; the scale index rules are DequantizeLinear's.
 * zp (same dtype as y) may be NULL (zero).  y_dtype: UINT8, INT8, UINT16,
 * INT16, UINT4, INT4 or FLOAT8E4M3FN.  A NaN before the integer cast gives 0
 * (the x86-64 conversion of the reference build).  Returns 0, or 1 for an
 * unsupported combination. */
int orc_quantize_linear(const void *x, int x_dtype, const int64_t *x_shape, int x_rank,
                        const void *scale, int scale_dtype, const int64_t *s_shape, int s_rank,
                        const void *zp, int y_dtype, int64_t axis, void *y);

/* ---- DynamicQuantizeLinear (kq/kernel_dynamicquantizelinear.cc:57-121) ----
 * Returns 0, or 1 for an empty or non-finite x (the reference throws). */
int orc_dynamic_quantize_linear(const float *x, int64_t n, uint8_t *y, float *y_scale,
                                uint8_t *y_zero_point);

/* ---- DequantizePacked, the GGUF profiles without codebooks
 * (onnx_core/runtime/dequantize_packed.cc:173-279) ----
 * ggml_type 2 q4_0, 3 q4_1, 6 q5_0, 7 q5_1, 8 q8_0, 9 q8_1, 20 iq4_nl,
 * 10 q2_k, 11 q3_k, 12 q4_k, 13 q5_k, 14 q6_k, 15 q8_k, 23 iq4_xs,
 * 34 tq1_0, 35 tq2_0, 39 mxfp4, 40 nvfp4, 41 q1_0, 42 q2_0: nblocks blocks of
 * orc_packed_block_bytes(type) bytes -> orc_packed_block_values(type) *
 * nblocks FLOAT values (each fp32 step rounded on its own).  Returns 0, or 1
 * for another type.  The FLOAT16 / BFLOAT16 / DOUBLE outputs are the FLOAT
 * values converted (:358-370). */
int orc_packed_block_bytes(int ggml_type);
int orc_packed_block_values(int ggml_type);
int orc_dequantize_packed(int ggml_type, const uint8_t *x, int64_t nblocks, float *out);

/* ---- ConvInteger (nn/kernel_conv_integer.cc:178-304) and QLinearConv
 * (kq/kernel_qlinearconv.cc:178-340) ----
 * x [N, C, spatial...] and w [M, C/group, kernel...] of INT8 or UINT8;
 * spatial rank 1..ORC_MAX_RANK-2.  kernel_shape / strides / pads /
 * dilations may be NULL (the reference's defaults); auto_pad is one of the
 * ORC_AUTO_PAD_* values.  Output [N, M, out spatial...] (sizes from
 * orc_conv_geometry).  ConvInteger: int32 accumulation that wraps; absent
 * zero points are 0; w_zp has w_zp_count values (1 or M).  QLinearConv:
 * int64 accumulation plus bias (may be NULL), then
 * saturate(nearbyint((float)acc * (x_scale * w_scale[m] / y_scale)) + y_zp).
 * Returns 0, or 1 for attributes or shapes the reference rejects. */
#define ORC_AUTO_PAD_NOTSET 0
#define ORC_AUTO_PAD_SAME_UPPER 1
#define ORC_AUTO_PAD_SAME_LOWER 2
#define ORC_AUTO_PAD_VALID 3
int orc_conv_geometry(const int64_t *x_shape, int x_rank, const int64_t *w_shape,
                      const int64_t *kernel_shape, const int64_t *strides, const int64_t *pads,
                      const int64_t *dilations, int auto_pad, int64_t *k_out, int64_t *s_out,
                      int64_t *d_out, int64_t *pads_out, int64_t *out_spatial);
int orc_conv_integer(const void *x, int x_dtype, const int64_t *x_shape, int x_rank, const void *w,
                     int w_dtype, const int64_t *w_shape, const void *x_zp, const void *w_zp,
                     int64_t w_zp_count, int64_t group, const int64_t *kernel_shape,
                     const int64_t *strides, const int64_t *pads, const int64_t *dilations, int auto_pad,
                     int32_t *y);
int orc_qlinear_conv(const void *x, int x_dtype, const int64_t *x_shape, int x_rank, float x_scale,
                     int32_t x_zp, const void *w, int w_dtype, const int64_t *w_shape, const float *w_scale,
                     int64_t w_scale_count, const void *w_zp, int64_t w_zp_count, float y_scale,
                     int32_t y_zp, int y_signed, const int32_t *bias, int64_t group,
                     const int64_t *kernel_shape, const int64_t *strides, const int64_t *pads,
                     const int64_t *dilations, int auto_pad, void *y);


/* AWQ weights, awq.cc:185-247: variant 0 "gemm" (4 or 8 bits), 1 "gemv",
 * 2 "gemv_fast" / "llm-awq"; codes [N, K], zeros [N, groups], FLOAT values
 * [N, K]; scales and zero_terms (variant 2) are decoded values. */
int orc_awq_decode(int variant, int bits, const void *qweight, const void *qzeros, const float *zero_terms,
                   const float *scales, int64_t K, int64_t N, int64_t group, int64_t padded, uint8_t *codes,
                   uint8_t *zeros, float *out);

/* GPTQ weights, gptq.cc:166-228: format 0 "gptq" (zero + 1), 1 "gptq_v2",
 * 2 "gptq_p"; words of `width` bytes; codes [N, K], zeros [N, groups] INT16,
 * FLOAT values [N, K]; scales decoded [groups, N]; g_idx [K]. */
int orc_gptq_decode(int format, int bits, int width, const void *qweight, const void *qzeros, const float *scales,
                    const int32_t *g_idx, int64_t K, int64_t N, int64_t group, uint8_t *codes, int16_t *zeros,
                    float *out);

/* bitsandbytes weights (nf4 / fp4 / int8): table entry, side-tensor checks, reconstruction */
float orc_bnb_table(int format, int code);
int orc_bnb_check(int format, int64_t rows, int64_t cols, int64_t block, int nested, float offset,
                  const void *absmax, const float *quant_map, const float *nested_absmax, const float *nested_map);
int orc_bnb_reconstruct(int format, int64_t rows, int64_t cols, int64_t block, int nested, float offset,
                        const uint8_t *codes, const void *absmax, const float *nested_absmax,
                        const float *nested_map, int out_dtype, void *out);

/* VPTQ weights: the constructor metadata of the layout and the
 * reconstruction into values [n, k]. */
typedef struct orc_vptq_config {
  int64_t k, n, bits;
  int64_t vector_lens[2], num_centroids[2], num_res_centroids[2];
  double npercent;
  int64_t group_size, group_num;
  int32_t enable_norm, norm_dim, enable_perm, dtype;
} orc_vptq_config;
int orc_vptq_reconstruct(const orc_vptq_config *c, const uint32_t *indices, const void *centroids,
                         const void *res_centroids, const void *outlier_centroids, const int32_t *outlier_indices,
                         const void *scale, const void *bias, const int32_t *perm, int out_dtype, void *out);

/* GPTQModel FP8 weights: code_type one of the five FP8 data types; method 0
 * tensor, 1 row, 2 block (b0 x b1); values [n, k]. */
float orc_f8e8m0_to_f32(uint8_t v);
int orc_gptq_fp8_reconstruct(int64_t n, int64_t k, int code_type, int method, int64_t b0, int64_t b1,
                             const uint8_t *codes, const float *scales, int out_dtype, void *out);

/* EXL3 weights: trellis [k / 16, n / 16, 16 * bits] words, book 0 3INST, 1
 * MCG, 2 MUL1; values [k, n]. */
int orc_exl3_reconstruct(int64_t k, int64_t n, int bits, int book, const uint16_t *trellis, const uint16_t *suh,
                         const uint16_t *svh, int out_dtype, void *out);

/* MX / NVFP4 weights: format 0 MXFP4, 1 MXFP6 E2M3, 2 MXFP8, 3 NVFP4; values
 * [count] and the first failure's group / element. */
int orc_mx_reconstruct(int format, int64_t count, const uint8_t *codes, const uint8_t *scales, float global,
                       int out_dtype, void *out, int64_t *fail_group, int64_t *fail_element);

/* BitBLAS row-packed weights: raw codes [n, k] and the GPTQ affine values. */
int orc_bitblas_reconstruct(int64_t k, int64_t n, int64_t group, int bits, int signed_codes, const uint8_t *qweight,
                            const uint16_t *scales, const uint8_t *qzeros, int out_dtype, void *out, uint8_t *codes);

/* QQQ weights (four-bit, group -1 / 128): nibble position of (n, k) in the
 * packed words, storage index of a channel / group scale, and the
 * reconstruction with the format's checks. */
int64_t orc_qqq_position(int64_t k, int64_t n, int64_t group, int64_t n_index, int64_t k_index);
int64_t orc_qqq_scale_position(int64_t index, int channel);
int orc_qqq_reconstruct(int64_t k, int64_t n, int64_t group, const uint8_t *words, const float *s_channel,
                        const uint16_t *s_group, int out_dtype, void *out, uint8_t *codes);

#ifdef __cplusplus
}
#endif

#endif /* ONNXL_AMD_ORACLE_H_ */
