// GPTQModel FP8 weights (the encoding "onnx_light.gptqmodel_fp8_weights.v1"
// of ai.rt:Dequantize, onnx_core/runtime/gptqmodel_fp8.cc) on the device.
//
// A weight [N, K] of FP8 codes (FLOAT8E4M3FN, E4M3FNUZ, E5M2, E5M2FNUZ or
// E8M0), row-major with no packing, and FLOAT inverse scales: one for the
// tensor, one per row, or one per (b0 x b1) block.  Value (Reconstructed,
// :160-162) = float(code) / scale, one IEEE division (correctly rounded).
//
// GptqFp8DecodeKernel: 8 consecutive k of one row per thread, output in
// FLOAT, FLOAT16, BFLOAT16 or DOUBLE (or nothing: the checks alone); flag
// bits for CheckData's failures (:164-173: a scale not finite or not
// positive, a value not finite) and for a value past the output dtype
// (WriteFloat, quantization.cc:184-201).  Every scale belongs to some
// element (the blocks tile the matrix), so checking the scales the threads
// read checks them all.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

// E8M0 (cast_float8.cc:451-461): 2^(bits - 127); 0 is 2^-127 (an fp32
// subnormal), 0xFF the quiet NaN.
__device__ __forceinline__ float E8M0ToF32(uint8_t c) {
  if (c == 0) return __uint_as_float(0x00400000u);
  if (c == 0xFF) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((uint32_t)c << 23);
}

template <int FT> __device__ __forceinline__ float DecodeFp8(uint8_t c) {
  if constexpr (FT == kFloat8E4M3FN) return Fp8E4M3ToF32(c);
  else if constexpr (FT == kFloat8E4M3FNUZ) return Fp8FnuzToF32<3, 8>(c);
  else if constexpr (FT == kFloat8E5M2) return Fp8E5M2ToF32(c);
  else if constexpr (FT == kFloat8E5M2FNUZ) return Fp8FnuzToF32<2, 16>(c);
  else return E8M0ToF32(c);
}

template <int FT, int OUT>
__global__ __launch_bounds__(256) void GptqFp8DecodeKernel(const GptqFp8Params p, void *__restrict__ y) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = (p.k + 7) / 8;
  if (t >= p.n * per_row) return;
  const int64_t n = t / per_row, k0 = (t - n * per_row) * 8;
  const int kc = (int)(p.k - k0 < 8 ? p.k - k0 : 8);
  unsigned flag = 0;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (e >= kc) break;
    const int64_t k = k0 + e;
    const int64_t si = p.method == 0 ? 0 : (p.method == 1 ? n : (n / p.b0) * p.scale_cols + k / p.b1);
    const float s = p.scales[si];
    if (!(__builtin_isfinite(s) && s > 0.f)) flag |= kGptqFp8BadScale;
    v[e] = DecodeFp8<FT>(p.codes[n * p.k + k]) / s;
    if (!__builtin_isfinite(v[e])) flag |= kGptqFp8BadValue;
    if constexpr (OUT == kFloat16 || OUT == kBfloat16) {
      const uint16_t h = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
      const bool inf = OUT == kFloat16 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
      if (inf && __builtin_isfinite(v[e])) flag |= kGptqFp8BadOutput;
    }
  }
  if (y != nullptr) {
    const int64_t o = n * p.k + k0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e >= kc) break;
      if constexpr (OUT == kFloat) static_cast<float *>(y)[o + e] = v[e];
      else if constexpr (OUT == kDouble) static_cast<double *>(y)[o + e] = (double)v[e];
      else static_cast<uint16_t *>(y)[o + e] = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
    }
  }
  if (flag) atomicOr(p.flag, flag);
}

template <int FT> void Launch(const GptqFp8Params &p, int out_dtype, void *y, hipStream_t s) {
  const int64_t threads = p.n * ((p.k + 7) / 8);
  const dim3 g((unsigned)((threads + 255) / 256)), b(256);
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL((GptqFp8DecodeKernel<FT, kFloat>), g, b, 0, s, p, y); break;
  case kDouble: hipLaunchKernelGGL((GptqFp8DecodeKernel<FT, kDouble>), g, b, 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL((GptqFp8DecodeKernel<FT, kFloat16>), g, b, 0, s, p, y); break;
  default: hipLaunchKernelGGL((GptqFp8DecodeKernel<FT, kBfloat16>), g, b, 0, s, p, y); break;
  }
}

}  // namespace

void LaunchGptqFp8Decode(const GptqFp8Params &p, int code_dtype, int out_dtype, void *y, hipStream_t s) {
  if (p.n * p.k == 0) return;
  switch (code_dtype) {
  case kFloat8E4M3FN: Launch<kFloat8E4M3FN>(p, out_dtype, y, s); break;
  case kFloat8E4M3FNUZ: Launch<kFloat8E4M3FNUZ>(p, out_dtype, y, s); break;
  case kFloat8E5M2: Launch<kFloat8E5M2>(p, out_dtype, y, s); break;
  case kFloat8E5M2FNUZ: Launch<kFloat8E5M2FNUZ>(p, out_dtype, y, s); break;
  default: Launch<kFloat8E8M0>(p, out_dtype, y, s); break;
  }
}

}  // namespace onnxl_amd
