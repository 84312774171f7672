// VPTQ weights (the encoding "onnx_light.vptq_weights.v1" of ai.rt:Dequantize,
// onnx_core/runtime/vptq.cc) on the device.
//
// A weight [n, k] (out_features, in_features) stored as vector-quantization
// indices: the first `outliers` input columns come from an outlier codebook
// (vectors of len0 rows), the rest are split into groups of `columns`
// columns, each with its own codebook of len1-row vectors and optionally a
// residual codebook.  For row r and input column c (Reconstruct, :401-443):
//  - outlier column: index = outlier_indices[(r / len0) * outliers + c],
//    value = outlier_centroids[index * len0 + r % len0];
//  - grouped column: g = (c - outliers) / columns, j = (c - outliers) %
//    columns, index = bits [j * w, j * w + w) of the INT32 words of
//    (g, r / len1) (w = main + residual bits, Index :194-202), value =
//    centroids[(g * nc1 + (index & main mask)) * len1 + r % len1], plus the
//    residual vector res_centroids[(g * nr1 + (index >> main)) * len1 +
//    r % len1] rounded to the codebook dtype;
//  - the value lands in column perm[c] (or c), then with norm it is scaled
//    and shifted by weight_scale / weight_bias of that column (norm_dim 0) or
//    of the row (norm_dim 1), each step rounded to the codebook dtype.
// Values are the codebook dtype's, lifted to FLOAT; the output then takes
// WriteFloat's rounding and checks (quantization.cc:184-201).
//
// Kernels: VptqIndexCheckKernel flags an index past its codebook
// (CheckData, :203-221: every column of every group, padding included);
// VptqDecodeKernel writes one output per thread and records the first output
// index (in output order) of a value that is not finite and of one that does
// not fit the output dtype.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

// one IEEE rounding per step, as the reference's volatile float steps
#pragma clang fp contract(off)

namespace onnxl_amd {
namespace {

__device__ __forceinline__ float LoadCode(const void *p, int dtype, int64_t i) {
  if (dtype == kFloat) return static_cast<const float *>(p)[i];
  const uint16_t h = static_cast<const uint16_t *>(p)[i];
  return dtype == kFloat16 ? F16ToF32(h) : __uint_as_float((uint32_t)h << 16);
}

// the value rounded to the codebook dtype (fp32 values stay)
__device__ __forceinline__ float RoundTo(float v, int dtype) {
  if (dtype == kFloat16) return F16ToF32(F32ToF16(v));
  if (dtype == kBfloat16) return __uint_as_float((uint32_t)F32ToBf16(v) << 16);
  return v;
}

__device__ __forceinline__ uint32_t VptqIndex(const VptqParams &p, int64_t g, int64_t v, int64_t j) {
  const int w = p.main_bits + p.residual_bits;
  const int64_t bit = j * w;
  const uint32_t *word = p.indices + (g * p.vectors + v) * p.words + (bit >> 5);
  uint64_t raw = word[0];
  if ((int)(bit & 31) + w > 32) raw |= (uint64_t)word[1] << 32;
  return (uint32_t)((raw >> (bit & 31)) & ((uint64_t{1} << w) - 1));
}

__global__ __launch_bounds__(256) void VptqIndexCheckKernel(const VptqParams p) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.groups * p.vectors * p.columns) return;
  const int64_t j = t % p.columns, gv = t / p.columns;
  const uint32_t index = VptqIndex(p, gv / p.vectors, gv % p.vectors, j);
  const uint32_t mask = (uint32_t)((uint64_t{1} << p.main_bits) - 1);
  bool bad = (int64_t)(index & mask) >= p.nc1;
  if (p.residual_bits) bad = bad || (int64_t)(index >> p.main_bits) >= p.nr1;
  if (bad) atomicOr(p.flag, kVptqBadIndex);
}

template <int OUT> __global__ __launch_bounds__(256) void VptqDecodeKernel(const VptqParams p, void *__restrict__ y) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.n * p.k) return;
  const int64_t r = t / p.k, c = t - r * p.k;
  float value;
  if (c < p.outliers) {
    const int64_t index = p.outlier_indices[(r / p.len0) * p.outliers + c];
    value = LoadCode(p.outlier_centroids, p.dtype, index * p.len0 + r % p.len0);
  } else {
    const int64_t g = (c - p.outliers) / p.columns, j = (c - p.outliers) % p.columns;
    const uint32_t index = VptqIndex(p, g, r / p.len1, j);
    const uint32_t mask = (uint32_t)((uint64_t{1} << p.main_bits) - 1);
    value = LoadCode(p.centroids, p.dtype, (g * p.nc1 + (index & mask)) * p.len1 + r % p.len1);
    if (p.residual_bits)
      value = RoundTo(value + LoadCode(p.res_centroids, p.dtype,
                                       (g * p.nr1 + (index >> p.main_bits)) * p.len1 + r % p.len1),
                      p.dtype);
  }
  const int64_t dest = p.perm ? (int64_t)p.perm[c] : c;
  if (p.scale) {
    const int64_t i = p.norm_dim == 0 ? dest : r;
    value = RoundTo(value * LoadCode(p.scale, p.dtype, i), p.dtype);
    value = RoundTo(value + LoadCode(p.bias, p.dtype, i), p.dtype);
  }
  // WriteFloat raises at the first failing value in output order: each kind
  // keeps its smallest output index, as the complement under atomicMax
  const int64_t o = r * p.k + dest;
  if (!__builtin_isfinite(value)) atomicMax(p.flag + 1, ~(unsigned)o);
  if constexpr (OUT == kFloat) {
    static_cast<float *>(y)[o] = value;
  } else if constexpr (OUT == kDouble) {
    static_cast<double *>(y)[o] = (double)value;
  } else {
    const uint16_t h = OUT == kFloat16 ? F32ToF16(value) : F32ToBf16(value);
    const bool inf = OUT == kFloat16 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
    if (inf && __builtin_isfinite(value)) atomicMax(p.flag + 2, ~(unsigned)o);
    static_cast<uint16_t *>(y)[o] = h;
  }
}

unsigned Blocks(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace

void LaunchVptqIndexCheck(const VptqParams &p, hipStream_t s) {
  const int64_t threads = p.groups * p.vectors * p.columns;
  if (threads > 0) hipLaunchKernelGGL(VptqIndexCheckKernel, dim3(Blocks(threads)), dim3(256), 0, s, p);
}

void LaunchVptqDecode(const VptqParams &p, int out_dtype, void *y, hipStream_t s) {
  const int64_t threads = p.n * p.k;
  if (threads == 0) return;
  const dim3 g(Blocks(threads)), b(256);
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL(VptqDecodeKernel<kFloat>, g, b, 0, s, p, y); break;
  case kDouble: hipLaunchKernelGGL(VptqDecodeKernel<kDouble>, g, b, 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL(VptqDecodeKernel<kFloat16>, g, b, 0, s, p, y); break;
  default: hipLaunchKernelGGL(VptqDecodeKernel<kBfloat16>, g, b, 0, s, p, y); break;
  }
}

}  // namespace onnxl_amd
