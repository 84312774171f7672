// QQQ weights (the encoding "onnx_light.qqq_weights.v1" of ai.rt:Dequantize,
// onnx_core/runtime/qqq.cc) on the device.
//
// A weight of logical shape [n, k] (out_features, in_features; k and n
// multiples of 64), four-bit codes in the packed words B [k / 16, 2n]: the
// codes sit in 16x16 tiles, (k / 16, n / 16) in row-major tile order and each
// tile row-major, and every 1024-code block is permuted (qqq.cc:57-67,
// Position :80-85); nibble p of the array is at bits 4 (p % 2) of byte p / 2
// (Code, :166-169).  Within a block, code (row, col) of tile j (row = k % 16,
// col = n % 16, j = (n / 16) % 4) is at nibble
//   index = i * 32 + j * 8 + lane,  i = 4 (col % 8) + row / 4,
//   p = 4 (col / 8) + row % 4,  lane = the interleave's inverse at p
// (grouped: p / 2 for even p, 4 + p / 2 for odd p; per channel: 2p + 1 for
// p < 4, 2 (p - 4) otherwise), the inverse of the source permutation
// 256 j + 16 (4 (i % 4) + p % 4) + i / 4 + 8 (p / 4).
// Scales are stored permuted too (ScalePosition, :144-149).
//
// Value (Reconstructed, :185-202): grouped (group 128, k != 128),
// integer = clamp(rint((code - 8) * group scale), -128, 127) -- the product
// of a 4-bit integer and an fp16 scale is exact in fp32, and rint rounds half
// to even keeping the sign of a zero, as the reference's double steps do --;
// per channel, integer = signed nibble * 16; value = fp32(integer * channel
// scale), one IEEE rounding with gradual underflow (RoundFloat, :162-183).
//
// Kernels:
//  - QqqDecodeKernel: 8 consecutive k of one row n per thread into FLOAT,
//    FLOAT16, BFLOAT16 or DOUBLE (or into nothing: the checks alone), raising
//    flags for CheckData's failures (:204-218: a channel or group scale not
//    finite or negative, a value not finite in fp32) and for a value that
//    does not fit the output dtype (WriteFloat, quantization.cc:184-201);
//  - QqqPackKernel: the operands of the fused DequantizeLinear -> MatMul
//    path: per channel the codes as ONNX-packed INT4 [k, n] (the signed
//    nibble is the INT4 value) with FLOAT scales 16 * channel scale (flagged
//    when that product overflows); grouped the clamped integers as INT8
//    [k, n] with the channel scales.  Both reproduce every value exactly:
//    x * scale rounds the same exact product once.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

// one IEEE rounding per product, as the reference's double -> float steps
#pragma clang fp contract(off)

namespace onnxl_amd {
namespace {

__device__ __forceinline__ int64_t QqqChannelPos(int64_t n) {
  const int64_t local = n & 31;
  return (n & ~int64_t{31}) + ((local & 7) >> 1) * 8 + (local >> 3) * 2 + (local & 1);
}

__device__ __forceinline__ int64_t QqqGroupPos(int64_t i) {
  return (i & ~int64_t{63}) + (i & 7) * 8 + ((i & 63) >> 3);
}

// nibble index of code (n, k) in B
__device__ __forceinline__ int64_t QqqNibble(const QqqParams &p, int64_t n, int64_t k) {
  const int64_t base = (k >> 4) * p.n * 16 + (n >> 4 >> 2) * 1024;  // the 1024-code block
  const int j = (int)((n >> 4) & 3), row = (int)(k & 15), col = (int)(n & 15);
  const int i = 4 * (col & 7) + (row >> 2);
  const int q = 4 * (col >> 3) + (row & 3);
  const int lane = p.grouped ? ((q & 1) ? 4 + (q >> 1) : (q >> 1)) : (q < 4 ? 2 * q + 1 : 2 * (q - 4));
  return base + i * 32 + j * 8 + lane;
}

__device__ __forceinline__ int QqqCode(const QqqParams &p, int64_t n, int64_t k) {
  const int64_t pos = QqqNibble(p, n, k);
  return (p.codes[pos >> 1] >> ((pos & 1) * 4)) & 15;
}

__device__ __forceinline__ bool BadScale(float s) { return !(__builtin_isfinite(s) && s >= 0.f); }

// the integer of (n, k) before the channel scale; flags a bad group scale
__device__ __forceinline__ float QqqInteger(const QqqParams &p, int64_t n, int64_t k, int code, unsigned &flag) {
  if (!p.grouped) return (float)(((code ^ 8) - 8) * 16);
  const float gs = F16ToF32(p.group[QqqGroupPos((k >> 7) * p.n + n)]);
  if (BadScale(gs)) flag |= kQqqBadGroup;
  const float r = __builtin_rintf((float)(code - 8) * gs);
  return __builtin_fminf(__builtin_fmaxf(r, -128.f), 127.f);
}

template <int OUT>
__global__ __launch_bounds__(256) void QqqDecodeKernel(const QqqParams p, void *__restrict__ y) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = p.k >> 3;
  if (t >= p.n * per_row) return;
  const int64_t n = t / per_row, k0 = (t - n * per_row) * 8;
  unsigned flag = 0;
  const float c = p.channel[QqqChannelPos(n)];
  if (k0 == 0 && BadScale(c)) flag |= kQqqBadChannel;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t k = k0 + e;
    v[e] = QqqInteger(p, n, k, QqqCode(p, n, k), flag) * c;
    if (!__builtin_isfinite(v[e])) flag |= kQqqBadValue;
  }
  const int64_t o = n * p.k + k0;
  if (y != nullptr) {
    if constexpr (OUT == kFloat) {
      float *d = static_cast<float *>(y) + o;
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = v[e];
    } else if constexpr (OUT == kDouble) {
      double *d = static_cast<double *>(y) + o;
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = (double)v[e];
    } else {
      uint16_t *d = static_cast<uint16_t *>(y) + o;
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
    }
  }
  if constexpr (OUT == kFloat16 || OUT == kBfloat16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t h = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
      const bool inf = OUT == kFloat16 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
      if (inf && __builtin_isfinite(v[e])) flag |= kQqqBadOutput;
    }
  }
  if (flag) atomicOr(p.flag, flag);
}

// Prepared operands: per channel, byte (k, j) of the INT4 [k, n] weight holds
// the codes of columns 2j (low nibble) and 2j + 1; grouped, byte (k, n) is
// the clamped integer.  One thread per 8 columns of one row k; the threads of
// row 0 also write those columns' FLOAT scales.
__global__ __launch_bounds__(256) void QqqPackKernel(const QqqParams p, uint8_t *__restrict__ w,
                                                     float *__restrict__ scale) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = p.n >> 3;
  if (t >= p.k * per_row) return;
  const int64_t k = t / per_row, n0 = (t - k * per_row) * 8;
  unsigned flag = 0;
  if (p.grouped) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int v = (int)QqqInteger(p, n0 + e, k, QqqCode(p, n0 + e, k), flag);
      const uint32_t b = (uint32_t)(v & 0xff) << (8 * (e & 3));
      if (e < 4) lo |= b;
      else hi |= b;
    }
    uint32_t *d = reinterpret_cast<uint32_t *>(w + k * p.n + n0);
    d[0] = lo;
    d[1] = hi;
  } else {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) word |= (uint32_t)QqqCode(p, n0 + e, k) << (4 * e);
    *reinterpret_cast<uint32_t *>(w + (k * p.n + n0) / 2) = word;
  }
  if (k == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float c = p.channel[QqqChannelPos(n0 + e)];
      const float s = p.grouped ? c : c * 16.f;
      if (!__builtin_isfinite(s)) flag |= kQqqBadPrepared;
      scale[n0 + e] = s;
    }
  }
  if (flag) atomicOr(p.flag, flag);
}

unsigned Blocks(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace

void LaunchQqqDecode(const QqqParams &p, int out_dtype, void *y, hipStream_t s) {
  const int64_t threads = p.n * (p.k >> 3);
  if (threads == 0) return;
  const dim3 g(Blocks(threads)), b(256);
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL(QqqDecodeKernel<kFloat>, g, b, 0, s, p, y); break;
  case kDouble: hipLaunchKernelGGL(QqqDecodeKernel<kDouble>, g, b, 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL(QqqDecodeKernel<kFloat16>, g, b, 0, s, p, y); break;
  default: hipLaunchKernelGGL(QqqDecodeKernel<kBfloat16>, g, b, 0, s, p, y); break;
  }
}

void LaunchQqqPack(const QqqParams &p, uint8_t *weight, float *scale, hipStream_t s) {
  const int64_t threads = p.k * (p.n >> 3);
  if (threads == 0) return;
  hipLaunchKernelGGL(QqqPackKernel, dim3(Blocks(threads)), dim3(256), 0, s, p, weight, scale);
}

}  // namespace onnxl_amd
