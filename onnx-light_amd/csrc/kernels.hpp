// Launch parameters and launcher declarations of the gfx950 kernels.  Plain
// structs passed by value as kernel arguments.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace onnxl_amd {

constexpr int kMaxBatchRank = 6;

// Maps a flat output-batch index to element offsets of A and B under ONNX
// MatMul broadcasting (row-major over `dims`; stride 0 = broadcast dim).
struct BatchMap {
  int rank = 0;
  int64_t dims[kMaxBatchRank] = {};
  int64_t a_stride[kMaxBatchRank] = {};
  int64_t b_stride[kMaxBatchRank] = {};
};

__host__ __device__ inline void BatchOffsets(const BatchMap &m, int64_t batch, int64_t &a_off,
                                             int64_t &b_off) {
  int64_t ao = 0, bo = 0, rem = batch;
  for (int d = m.rank - 1; d >= 0; --d) {
    const int64_t c = rem % m.dims[d];
    rem /= m.dims[d];
    ao += c * m.a_stride[d];
    bo += c * m.b_stride[d];
  }
  a_off = ao;
  b_off = bo;
}

// ---------------------------------------------------------------------------
// int8 MFMA GEMM shared by MatMulInteger and QLinearMatMul.
//
// The MFMA runs on a' = a - ca and b' = b - cb as signed bytes (ca = 128 for
// UINT8 A, i.e. a ^ 0x80, else 0; cb likewise).  With alpha_i = ca - za_i and
// beta_j = cb - zb_j the exact result is
//   Y_ij = sum_k a'b' + beta_j*RA_i + alpha_i*CB_j + K*alpha_i*beta_j,
// RA_i = sum_k a'_ik, CB_j = sum_k b'_kj, evaluated modulo 2^32 (which is the
// int32 wrap of the reference's accumulator).

enum IGemmEpilogue : int { kEpiInt32 = 0, kEpiQuant8 = 1, kEpiQuant8Row = 2 };

// Scalar zero points and scales that stay in device memory and are read by
// the kernels themselves, so the call needs no host synchronisation (a call
// captured in a HIP graph).  A null pointer keeps the value given on the
// host in the launch parameters.
struct QDevScalars {
  const uint8_t *za, *zb, *zy;  // one byte in A's / B's / Y's dtype
  const void *as, *bs, *ys;     // FLOAT, or FLOAT16 where the *_f16 flag is set
  int as_f16, bs_f16, ys_f16;
  // scales: the quotient is formed on the device, with the host value below
  // for a scale whose pointer is null
  int scales;
  float as_h, bs_h, ys_h;
};

// The constants the GEMM epilogues use: alpha = ca - za, beta = cb - zb,
// cs = (a_scale * b_scale) / y_scale in fp32 in that order
// (kq/kernel_qlinearmatmul.cc:156) and zy as a float.
struct QResolved {
  int32_t alpha, beta;
  float cs, zy;
};

__device__ inline float DevScale(const void *p, int f16) {
  return f16 ? (float)*static_cast<const _Float16 *>(p) : *static_cast<const float *>(p);
}

// Host values (alpha, beta, cs, zy) overridden by the device-resident ones.
__device__ inline QResolved ResolveQ(const QDevScalars &d, int a_u8, int b_u8, int y_signed, int32_t alpha,
                                     int32_t beta, float cs, float zy) {
  QResolved r{alpha, beta, cs, zy};
  if (d.za) r.alpha = a_u8 ? 128 - (int32_t)d.za[0] : -(int32_t)(int8_t)d.za[0];
  if (d.zb) r.beta = b_u8 ? 128 - (int32_t)d.zb[0] : -(int32_t)(int8_t)d.zb[0];
  if (d.scales) {
    const float sa = d.as ? DevScale(d.as, d.as_f16) : d.as_h;
    const float sb = d.bs ? DevScale(d.bs, d.bs_f16) : d.bs_h;
    const float sy = d.ys ? DevScale(d.ys, d.ys_f16) : d.ys_h;
    const float ab = sa * sb;
    r.cs = ab / sy;
  }
  if (d.zy) r.zy = (float)(y_signed ? (int32_t)(int8_t)d.zy[0] : (int32_t)d.zy[0]);
  return r;
}

// Implicit convolution operand: B is not a [K, N] matrix but one image of the
// zero-point-padded input in NHWC order, [Hp, Wp, C] bytes, and K runs over
// (kernel tap, channel) with C % 128 == 0, so a K step of 128 bytes is 128
// channels of one tap.  Output position n = (oh, ow) = (n / wo, n % wo) reads
// B row pixel (oh * stride_h + i * dilation_h, ow * stride_w + j * dilation_w)
// for tap (i, j): byte n_off(n) + t_off(t) + 16 * chunk with
//   n_off = oh * pix_row + ow * pix_col,
//   t_off = i * tap_row + j * tap_col + 128 * (t % spt),  tap = t / spt.
struct ImplicitConv {
  int64_t pix_row, pix_col;  // stride_h * Wp * C, stride_w * C
  int64_t tap_row, tap_col;  // dilation_h * Wp * C, dilation_w * C
  int64_t image_bytes;       // Hp * Wp * C
  int wo;                    // output width
  int spt;                   // K steps per tap: C / 128
  int kw;                    // kernel width
  uint32_t spt_magic, kw_magic;  // ceil(2^32 / d) (0 for d = 1): q = mulhi(x, magic)
};

struct IGemmParams {
  const int8_t *A;  // [.., M, K] row-major
  const int8_t *B;  // [.., K, N] row-major
  void *Y;          // [batch, M, N]
  int64_t M, N, K;
  int64_t batch;
  BatchMap bm;
  int a_u8, b_u8;
  // Per-row / per-column zero points (M / N bytes in A's / B's dtype), or
  // nullptr when the zero point is a single value: alpha_scalar / beta_scalar
  // then hold ca - za / cb - zb.
  const uint8_t *a_zp;
  const uint8_t *b_zp;
  int32_t alpha_scalar, beta_scalar;
  int need_ra, need_cb;  // beta != 0 anywhere / alpha != 0 anywhere
  // kEpiQuant8: v = rint((float)acc * cs) + zy, clamped to [qmin, qmax]
  float cs, zy, qmin, qmax;
  int y_signed;
  int epilogue;
  // Device-resident scalars replacing alpha_scalar, beta_scalar, cs and zy
  // (kEpiInt32 / kEpiQuant8); need_cb / need_ra are set when za / zb is one.
  QDevScalars dev;
  // kEpiQuant8Row (pipelined kernel only): row r uses the scale
  // row_xs * row_wscale[r or 0] / row_ys and adds row_bias[r] (if not null)
  // to the int32 sum exactly before the conversion.
  const float *row_wscale;
  int row_wscale_per;
  float row_xs, row_ys;
  const int32_t *row_bias;
  // B is an implicit convolution operand (pipelined kernel only)
  int implicit_conv;
  ImplicitConv cv;
};

void LaunchIGemm(const IGemmParams &p, hipStream_t stream);
// QLinearMatMul where the int32 MFMA sums can overflow: int64 accumulation
// (kq/kernel_qlinearmatmul.cc:187-191) in a VALU kernel; uses p.A, p.B, p.Y,
// M, N, K, batch, bm, a_u8, b_u8, cs, zy, qmin, qmax, y_signed, dev and the
// zero points za, zb given here (replaced by dev.za / dev.zb when set).
void LaunchQlmExact(const IGemmParams &p, int32_t za, int32_t zb, hipStream_t stream);
// Whether LaunchIGemm takes the pipelined MFMA kernel for p (kEpiQuant8Row
// requires it).
bool IGemmFastEligible(const IGemmParams &p);

// ---------------------------------------------------------------------------
// DequantizePacked, 32-value GGUF formats (ggml type codes 2, 3, 6, 7, 8, 9,
// 20): nblocks blocks -> 32 * nblocks values of out_dtype (FLOAT, FLOAT16,
// BFLOAT16 or DOUBLE).
bool PackedFormatOnGpu(int ggml_type);
void LaunchDequantizePacked(int ggml_type, const uint8_t *x, int64_t nblocks, int out_dtype, void *y,
                            hipStream_t stream);
// y[M, N] (FLOAT16) = a[M, K] (FLOAT16) x W^T, W the FLOAT16 decode of a
// gguf:q4_0 [N, K] weight; M <= 8, K % 64 == 0, a and w dword aligned.
bool GemvQ40Eligible(int64_t M, int64_t K, const void *a, const void *w);
void LaunchGemvQ40(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                   hipStream_t stream);
// The same for gguf:q8_0 (same eligibility).
// Fused 256-value GEMVs: q2_k (ggml type 10), q3_k (11), q4_k (12), q5_k
// (13), q6_k (14) and iq4_xs (23); K % 256 == 0, M <= 8, a 16-byte aligned,
// w aligned to GemvKAlignment(type) bytes (0: no fused GEMV for the type).
void LaunchGemvK(int ggml_type, const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                 hipStream_t s);
int GemvKAlignment(int ggml_type);
void LaunchGemvQ80(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                   hipStream_t stream);

// ---------------------------------------------------------------------------
// bitsandbytes weights (bnb.hip), logical [rows, cols] row-major: format 0
// nf4 / 1 fp4 (4-bit codes, the even element in the high nibble, one scale
// per 2^block_shift elements) or 2 int8 (signed bytes, one scale per row).
// Flag bits the kernels OR into *flag:
constexpr unsigned kBnbBadAbsmax = 1;  // a FLOAT absmax not finite or negative
constexpr unsigned kBnbBadScale = 2;   // a resolved scale not finite
constexpr unsigned kBnbBadValue = 4;   // a value not finite in fp32 or in the output dtype
struct BnbParams {
  int format;
  int64_t rows, cols;
  int block_shift;
  int nested;                // absmax holds UINT8 codes of the nested statistics
  float offset;              // nested_offset
  int64_t blocks;            // scales: ceil(rows * cols / block), or rows for int8
  const uint8_t *codes;
  const void *absmax;        // FLOAT [blocks] (int8: the row maxima), or UINT8 [blocks] when nested
  const float *nested_absmax;  // [ceil(blocks / 256)]
  const float *nested_map;     // [256]
  float *scales;             // [blocks]: written by LaunchBnbScales (unless null), read by the others
  unsigned *flag;
};
void LaunchBnbScales(const BnbParams &p, hipStream_t s);

// VPTQ weights (vptq.hip): flag words and the decoded layout.  flag[0] bit
// kVptqBadIndex: an index past its codebook; flag[1] / flag[2]: the
// complement of the first output index whose value is not finite / past
// the output dtype's range (0: none).
constexpr unsigned kVptqBadIndex = 1;
struct VptqParams {
  int64_t k, n;                      // in_features, out_features
  int64_t outliers, columns, groups, vectors, words;
  int main_bits, residual_bits;
  int64_t len0, len1, nc1, nr1;      // vector lengths, codebook sizes
  int dtype;                         // codebook dtype: kFloat, kFloat16, kBfloat16
  int norm_dim;
  const uint32_t *indices;           // [groups, vectors, words]
  const void *centroids, *res_centroids, *outlier_centroids;
  const int32_t *outlier_indices;    // [1, ceil(n / len0), outliers]
  const void *scale, *bias;          // norm (null without)
  const int32_t *perm;               // null without
  unsigned *flag;                    // 3 words
};
void LaunchVptqIndexCheck(const VptqParams &p, hipStream_t s);
void LaunchVptqDecode(const VptqParams &p, int out_dtype, void *y, hipStream_t s);

// GPTQModel FP8 weights (gptqmodel_fp8.hip): flag bits in the reference's order.
constexpr unsigned kGptqFp8BadScale = 1;   // an inverse scale not finite or not positive
constexpr unsigned kGptqFp8BadValue = 2;   // a value not finite in fp32
constexpr unsigned kGptqFp8BadOutput = 4;  // a value past the output dtype's range
struct GptqFp8Params {
  int64_t n, k;              // out_features, in_features
  int method;                // 0 tensor, 1 row, 2 block
  int64_t b0, b1, scale_cols;  // block rows / columns, scale columns (block)
  const uint8_t *codes;      // [n, k]
  const float *scales;       // weight_scale_inv
  unsigned *flag;
};
// code_dtype: one of the five FP8 types; out_dtype kFloat, kFloat16,
// kBfloat16 or kDouble; y [n, k] or null (the checks alone)
void LaunchGptqFp8Decode(const GptqFp8Params &p, int code_dtype, int out_dtype, void *y, hipStream_t s);

// MX / NVFP4 weights (mx_weights.hip).  `first` (zeroed by the caller)
// receives the complement of the smallest failure key group * 128 + step
// (step 0 a group's scale, 1 / 2 NVFP4's quotient not finite / zero, 3 + 2e
// element e's NaN code, 4 + 2e its value not finite), 0 when none; `flag`
// the output range bit.
enum MxFormat { kMxFp4 = 0, kMxFp6E2M3 = 1, kMxFp8 = 2, kMxNvfp4 = 3 };
constexpr unsigned kMxBadOutput = 1;  // a value past the output dtype's range
struct MxParams {
  int64_t count;          // rows * cols, a multiple of the group size
  const uint8_t *codes;   // packed codes (MXFP4 / NVFP4 nibbles, MXFP6 6-bit, MXFP8 bytes)
  const uint8_t *scales;  // one byte per group
  float global;           // NVFP4's global scale
  int aligned;            // codes and y 16-byte aligned: vector loads and stores
  uint64_t *first;
  unsigned *flag;
};
// y [rows, cols] of out_dtype (kFloat, kFloat16, kBfloat16, kDouble) or null
void LaunchMxDecode(const MxParams &p, int format, int out_dtype, void *y, hipStream_t s);

// EXL3 weights (exl3.hip): flag bits after the host's checks.
constexpr unsigned kExl3BadValue = 1;   // a reconstructed value not finite
constexpr unsigned kExl3BadOutput = 2;  // a value past the output dtype's range
struct Exl3Params {
  int64_t k, n;             // rows, columns (multiples of 128)
  int bits, book;           // trellis rate 1..8; codebook 0 3INST, 1 MCG, 2 MUL1
  const uint16_t *trellis;  // [k / 16, n / 16, 16 * bits]
  const uint16_t *suh;      // binary16 [k]
  const uint16_t *svh;      // binary16 [n]
  unsigned *flag;
};
// y [k, n] of out_dtype (kFloat, kFloat16, kBfloat16, kDouble)
void LaunchExl3Decode(const Exl3Params &p, int out_dtype, void *y, hipStream_t s);

// QQQ weights (qqq.hip): flag bits of a decode / preparation, in the order
// the reference raises them.
constexpr unsigned kQqqBadChannel = 1;   // a channel scale not finite or negative
constexpr unsigned kQqqBadGroup = 2;     // a group scale not finite or negative
constexpr unsigned kQqqBadValue = 4;     // a value not finite in fp32
constexpr unsigned kQqqBadOutput = 8;    // a value past the output dtype's range
constexpr unsigned kQqqBadPrepared = 16; // 16 * a channel scale overflows fp32 (no INT4 operand)
struct QqqParams {
  int64_t k, n;              // in_features, out_features (multiples of 64)
  int grouped;               // group 128 with k != 128
  const uint8_t *codes;      // B [k / 16, 2n] int32 words, as bytes
  const float *channel;      // s_channel [n] (stored order)
  const uint16_t *group;     // s_group [k / 128, n] fp16 (stored order), grouped only
  unsigned *flag;
};
// out_dtype kFloat, kFloat16, kBfloat16 or kDouble; y [n, k] or null (checks alone)
void LaunchQqqDecode(const QqqParams &p, int out_dtype, void *y, hipStream_t s);
// weight: INT4 [k, n] ONNX packing (per channel) or INT8 [k, n] (grouped); scale FLOAT [n]
void LaunchQqqPack(const QqqParams &p, uint8_t *weight, float *scale, hipStream_t s);
// out_dtype kFloat, kFloat16, kBfloat16, or 0: the finiteness check alone
void LaunchBnbDecode(const BnbParams &p, int out_dtype, void *y, hipStream_t s);
// y[M, N] FLOAT16 = a[M, K] x W^T, W the FLOAT16 decode of nf4 / fp4 codes
// [N, K] with resolved scales: M <= 4, K % 32 == 0, K % block == 0,
// 16-byte aligned a and codes.
bool BnbGemvEligible(int format, int64_t M, int64_t N, int64_t K, int64_t block, const void *a, const void *codes);
void LaunchBnbGemv(int format, const uint16_t *a, const uint8_t *codes, const float *scales, int64_t M, int64_t N,
                   int64_t K, int64_t block, uint16_t *y, hipStream_t s);

// ---------------------------------------------------------------------------
// ConvInteger / QLinearConv.  Spatial dims are right-aligned into 3 slots
// (missing leading dims have size 1, kernel 1, stride 1, dilation 1, pad 0).
struct ConvGeom {
  int64_t N, C, G, cpg, M, Mg;
  int64_t in[3], out[3];
  int k[3];
  int64_t s[3], d[3], pb[3];  // stride, dilation, leading pad
  int64_t in_size, P, ks, Kc;  // input plane size, output positions, kernel taps, cpg * ks
};

// QLinearConv requantization: y = saturate(rint((float)(acc + bias[m]) *
// (x_scale * w_scale[m] / y_scale)) + zy).
struct ConvQuant {
  float x_scale, y_scale;
  const float *w_scale;  // device, 1 or M values
  int w_scale_per_channel;
  const int32_t *bias;  // device, M values, or nullptr
  float zy, qmin, qmax;
};

// A 1x1 kernel with stride 1 and no padding reads x itself as the columns
// ([N, C, P] is [N, G, Kc, P]); no im2col pass, ConvColBytes 0.
bool ConvColIsInput(const ConvGeom &g);
size_t ConvColBytes(const ConvGeom &g);
// Implicit GEMM (group 1, 2-D, C % 128 == 0, P % 16 == 0, C * W and Kc <= 64 KB):
// the padded NHWC input (ConvImplicitInputBytes) and the tap-major weight
// (M * Kc bytes) replace the im2col matrix; ConvImplicitDesc describes the B
// operand for IGemmParams::cv (one image per batch entry).
bool ConvImplicitEligible(const ConvGeom &g);
size_t ConvImplicitInputBytes(const ConvGeom &g);
ImplicitConv ConvImplicitDesc(const ConvGeom &g);
void LaunchConvImplicitOperands(const ConvGeom &g, const uint8_t *x, uint8_t x_zp, const uint8_t *w, uint8_t *xh,
                                uint8_t *wr, hipStream_t stream);
void LaunchImToCol(const ConvGeom &g, const uint8_t *x, uint8_t x_zp, uint8_t *col, hipStream_t stream);
// q == nullptr: ConvInteger (int32 output); else QLinearConv (8-bit output).
// w_zp_per_channel: M device bytes, or nullptr for the value w_zp_scalar.
void LaunchDirectConv(const ConvGeom &g, const uint8_t *x, int x_u8, uint8_t x_zp, const uint8_t *w, int w_u8,
                      const uint8_t *w_zp_per_channel, int32_t w_zp_scalar, const ConvQuant *q, void *y,
                      hipStream_t stream);
void LaunchConvRequant(const ConvGeom &g, const int32_t *acc, const ConvQuant &q, uint8_t *y, hipStream_t stream);

// ---------------------------------------------------------------------------
// DequantizeLinear (standalone, element-wise).

struct DequantParams {
  const void *x;
  const void *scale;  // FLOAT or FLOAT16 values
  const void *zp;     // same storage type as x, or nullptr
  void *y;            // FLOAT or FLOAT16 (= scale dtype)
  int64_t n;          // elements of x
  int x_dtype, scale_f16;
  // scale index of flat element i: ((i / inner) / block) % ... computed as
  //   outer = i / (axis_len * inner); a = (i / inner) % axis_len; in = i % inner
  //   si = (outer * s_axis + a / block) * inner + in      (blocked, s_axis = axis_len / block)
  //   si = a                                                (per-axis)
  //   si = 0                                                (per-tensor)
  int mode;           // 0 per-tensor, 1 per-axis, 2 blocked
  int64_t inner, axis_len, block, s_axis;
};

void LaunchDequantize(const DequantParams &p, hipStream_t stream);

// QuantizeLinear (kq/kernel_quantizelinear.cc): y = saturate(nearbyint(x /
// scale) + zp) for integer outputs, fp8(x / scale + zp) for FLOAT8E4M3FN;
// same scale-index modes as DequantParams.
struct QuantParams {
  const void *x;      // FLOAT or FLOAT16
  const void *scale;  // FLOAT or FLOAT16
  const void *zp;     // y's storage type (packed nibbles for 4-bit), or nullptr
  void *y;
  int64_t n;
  int x_f16, scale_f16, y_dtype;
  int vec;            // x and y allow whole 8-element vector accesses
  int mode;           // 0 per-tensor, 1 per-axis, 2 blocked
  int64_t inner, axis_len, block, s_axis;
};
void LaunchQuantize(const QuantParams &p, hipStream_t stream);

// DynamicQuantizeLinear (kq/kernel_dynamicquantizelinear.cc:57-121) of n > 0
// FLOAT values.  A non-finite x leaves y_scale = NaN, y_zero_point = 0, y = 0.
size_t DynQuantScratchBytes(int64_t n);
void LaunchDynamicQuantize(const float *x, int64_t n, uint8_t *y, float *y_scale, uint8_t *y_zero_point,
                           void *scratch, hipStream_t stream);

// Cast FLOAT -> FLOAT16 / BFLOAT16 (round to nearest even).
void LaunchCastF32(const float *x, void *y, int64_t n, int to_bf16, hipStream_t stream);
// y [C, R] = x [R, C]^T, elements of 1, 2, 4 or 8 bytes (elementwise.hip)
void LaunchTranspose2d(const void *x, void *y, int64_t R, int64_t C, int elem_bytes, hipStream_t s);

// ---------------------------------------------------------------------------
// Dequantize-fused MatMul: Y[M,N] = A[M,K] @ W[K,N], W = round(deq(x)).

struct DqMatMulParams {
  const void *A;     // FLOAT16 / BFLOAT16 activations [batch*M, K] (contiguous rows)
  const uint8_t *W;  // quantized weight [K, N] (4-bit: N/2 bytes per row)
  const void *scale; // FLOAT or FLOAT16
  const uint8_t *zp; // same storage as W (per scale entry) or nullptr
  void *Y;           // activations dtype [batch*M, N]
  int64_t M, N, K;
  int w_dtype;       // kInt4, kUint4, kInt8, kUint8, kFloat8E4M3FN
  int scale_f16;     // scale storage is FLOAT16 (else FLOAT)
  int a_bf16;        // activations/output are BFLOAT16 (else FLOAT16)
  int mode;          // 0 per-tensor, 1 per-column (axis 1), 2 blocked along K (axis 0)
  int64_t block;     // rows of K per scale row (mode 2)
  // Rounding of the dequantized weight, as the unfused chain does it:
  //   deq_round: 1 = to FLOAT16 (x_scale FLOAT16), 0 = stays FLOAT
  //   cast_round: 16 = to BFLOAT16, 10 = to FLOAT16, 0 = none
  int deq_round_f16;
  int cast_round;
  // W is in the tiled 4-bit layout written by LaunchTileInt4 (INT4 / UINT4
  // only) instead of the ONNX row-major packing.
  int w_tiled;
};

// ---------------------------------------------------------------------------
// Tiled 4-bit weight layout (a session-time preparation of a constant
// INT4 / UINT4 weight x [K, N]):
//   16-column tiles t (N padded to a multiple of 16), each holding K padded to
//   a multiple of 128 rows as 128-row groups of 1 KiB; in a group, 16-byte
//   lane l = 16 * g + i holds four dwords c = 0..3, dword c = column 16t + i,
//   rows 128q + 32c + 8g + (0..7).  Row r0 + j sits at bits 4 * (j / 2)
//   (j even) or 16 + 4 * (j / 2) (j odd); values are offset binary
//   (INT4 q -> q + 8, UINT4 unchanged); padding rows and columns hold the
//   offset-binary zero.
int64_t TiledInt4Bytes(int64_t K, int64_t N);
void LaunchTileInt4(const uint8_t *x, int64_t K, int64_t N, int is_signed, uint32_t *out,
                    hipStream_t stream);

// Returns false when the shape/dtype combination has no GPU kernel.
bool LaunchDqMatMul(const DqMatMulParams &p, void *scratch, size_t scratch_bytes,
                    unsigned *counters, size_t n_counters, hipStream_t stream);
size_t DqMatMulScratchBytes(const DqMatMulParams &p);
size_t DqMatMulCounters(const DqMatMulParams &p);

// Plain FLOAT16 / BFLOAT16 MatMul (fp32 accumulate).
struct HMatMulParams {
  const uint16_t *A;
  const uint16_t *B;
  uint16_t *Y;
  int64_t M, N, K;
  int64_t batch;
  BatchMap bm;
  int bf16;
};
void LaunchHMatMul(const HMatMulParams &p, hipStream_t stream);
// Y = A @ B^T with B given as [N, K] row-major (batch 1).
void LaunchHMatMulBT(const HMatMulParams &p, hipStream_t stream);

// ---------------------------------------------------------------------------
// GroupedMatMul (grouped.hip): Y[m, s, :] = A[m, :] @ W[idx[m, s]] (+ bias).
struct GroupedParams {
  const void *A;     // [M, K] FLOAT16 / BFLOAT16
  const void *W;     // [G, K, N], or [G, N, K] with transB
  const void *idx;   // [M, S] INT32 / INT64
  const void *bias;  // [G, N] or nullptr
  void *Y;           // [M, S, N]
  int64_t M, K, N, G, S;
  int idx64, transB, bf16;
  int64_t nbn;       // column tiles of the GEMM core: ceil(N / 128)
  // device workspace: G + 1, G + 1 and M * S int32
  int32_t *row_off, *tile_off, *rows;
};
int64_t GroupedMaxTiles(const GroupedParams &p);
void LaunchGroupedMatMul(const GroupedParams &p, hipStream_t stream);

// Fused DequantizeLinear -> [Cast] -> GroupedMatMul (quantized MoE experts):
// the GroupedMatMul of `g` over W = Cast(DequantizeLinear(X, scale, zp)).
struct DqGroupedParams {
  GroupedParams g;   // g.W is set by the launcher (general path: w16)
  const uint8_t *X;  // quantized weights [G, K, N] ([G, N, K] with transB), ONNX packing
  const void *scale; // FLOAT or FLOAT16
  const uint8_t *zp; // storage of X's dtype, one per scale entry, or nullptr
  int x_dtype, scale_f16;
  // scale entry of flat weight element i: per-tensor (kind 0) 0; per-axis (1)
  // (i / inner) % axis_dim; blocked along the axis (2)
  // ((i / (inner * axis_dim)) * (axis_dim / block) + ((i / inner) % axis_dim) / block) * inner + i % inner
  int scale_kind;
  int64_t inner, axis_dim, block;
  // the chain's roundings: to FLOAT16 when the DequantizeLinear output is
  // FLOAT16; else the Cast's (16: BFLOAT16, 10: FLOAT16)
  int deq_round_f16, cast_round;
  // fp8 weights on the grouped MFMA core, sums scaled per column in fp32:
  // group g's column n uses scale[g * scale_grp_stride + (scale_per_col ? n : 0)]
  int fused, scale_per_col;
  int64_t scale_grp_stride;
  uint16_t *w16;     // general path: the dequantized weights (G * K * N), device workspace
};
// Whether the fused fp8 path takes these operands (shape and alignment).
bool DqGroupedFusedEligible(const DqGroupedParams &p);
void LaunchDqGroupedMatMul(const DqGroupedParams &p, hipStream_t stream);

// ---------------------------------------------------------------------------
// ORT MatMulNBits weight preparation (nbits.hip).
struct NbitsPrepParams {
  const uint8_t *B;         // [N, groups, block * bits / 8]
  const uint16_t *scales;   // FLOAT16 [N, groups]
  const uint8_t *zp;        // packed codes [N, ceil(groups * bits / 8)] or nullptr
  int64_t K, N, block, bits;
  void *weight;             // bits 4: tiled INT4 / UINT4; bits 8: [K, N] INT8 / UINT8
  void *scale_out;          // FLOAT16 [groups, N]
  void *zp_out;             // UINT4 / UINT8 [groups, N] (with zp)
};
void LaunchPrepareNbits(const NbitsPrepParams &p, hipStream_t stream);

// ---------------------------------------------------------------------------
// AWQ / GPTQ checkpoint weights (checkpoints.hip; layouts in
// checkpoint_layout.hpp).
struct CkptLayout;
// weight: tiled UINT4 (bits <= 4) or UINT8 [K, N]; zp_out: UINT4 / UINT8
// [groups, N]; scale_out: [groups, N] FLOAT16 (scale_dtype FLOAT16) or FLOAT
void LaunchCkptPrepare(const CkptLayout &L, const void *scales, int scale_dtype, void *weight, void *scale_out,
                       void *zp_out, hipStream_t stream);
// y [N, K] of out_dtype (FLOAT, FLOAT16, BFLOAT16, DOUBLE); zero_terms: AWQ
// gemv_fast / llm-awq FLOAT16 [padded, N]; g_idx: GPTQ group map [K] or null
void LaunchCkptDecode(const CkptLayout &L, const void *scales, int scale_dtype, const uint16_t *zero_terms,
                      const int32_t *g_idx, int out_dtype, void *y, hipStream_t stream);

}  // namespace onnxl_amd
