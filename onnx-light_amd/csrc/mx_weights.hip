// MX and NVFP4 weights (the ai.rt:Dequantize encodings
// "onnx_light.mxfp4_weights.v1", "onnx_light.mxfp6_e2m3_weights.v1",
// "onnx_light.mxfp8_weights.v1" and "onnx_light.nvfp4_weights.v1",
// onnx_core/runtime/quantization.cc:1253-1750) on the device.
//
// A [rows, cols] weight in row-major groups of G consecutive elements along
// a row (G = 32, or 16 for NVFP4), one scale byte per group:
//   MXFP4  (:1458-1470)  low nibble first, E2M1 level * 2^(e - 127);
//   MXFP6  (:1700-1707)  four E2M3 codes in three bytes, LSB first (the
//                        element's 6 bits at bit 6i of the group's 24 bytes),
//                        value * 2^(e - 127), one fp32 rounding;
//   MXFP8  (:1591-1600)  E4M3FN code * E8M0 scale (byte 0 is 2^-127);
//   NVFP4  (:1322-1342)  low nibble first, E2M1 level * (E4M3FN local scale /
//                        FLOAT global scale), the quotient rounded once.
// Every product rounds once in fp32, which is the reference's volatile
// float product.
//
// MxDecodeKernel: 8 consecutive elements of one group per thread.  The
// reference validates group by group and raises the first failure, so each
// thread folds its group's and its elements' failures into one ordered key,
// group * 128 + step (step 0..2 the group's scale checks, 3 + 2e and 4 + 2e
// element e's code and value checks), and the smallest key wins (atomicMax of
// its complement over a zeroed word).
// WriteFloat's range check (quantization.cc:184-201) comes after every
// validation and is one flag bit.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

// E8M0 exponent byte -> 2^(e - 127); byte 0 is 2^-127 (an fp32 subnormal).
// Byte 255 is rejected before use.
__device__ __forceinline__ float MxScale(uint32_t e) {
  return e == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(e << 23);
}

template <int FMT, int OUT>
__global__ __launch_bounds__(256) void MxDecodeKernel(const MxParams p, void *__restrict__ y) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.count / 8) return;
  constexpr int G = FMT == kMxNvfp4 ? 16 : 32;
  const int64_t i0 = t * 8, group = i0 / G;
  const int e0 = (int)(i0 - group * G);
  uint64_t key = ~0ull;
  auto fail = [&](int step) {
    const uint64_t k = (uint64_t)group * 128u + (uint64_t)step;
    key = k < key ? k : key;
  };
  const uint32_t sb = p.scales[group];
  float scale;
  if constexpr (FMT == kMxNvfp4) {
    const float local = Fp8E4M3ToF32((uint8_t)sb);
    if (!(__builtin_isfinite(p.global) && p.global > 0.f && __builtin_isfinite(local) && local > 0.f)) fail(0);
    scale = local / p.global;
    if (!__builtin_isfinite(scale)) fail(1);
    else if (!(scale > 0.f)) fail(2);
  } else {
    if (sb == 255u) fail(0);
    scale = MxScale(sb);
  }
  float v[8];
  uint32_t codes[8];
  // the 8 codes' bytes (4, 6 or 8 of them), aligned to their size when
  // p.aligned, else read byte by byte
  const int64_t off = FMT == kMxFp8 ? i0 : (FMT == kMxFp6E2M3 ? i0 / 8 * 6 : i0 / 2);
  constexpr int NB = FMT == kMxFp8 ? 8 : (FMT == kMxFp6E2M3 ? 6 : 4);
  uint64_t bits = 0;
  if (p.aligned) {
    if constexpr (NB == 8) {
      bits = *reinterpret_cast<const uint64_t *>(p.codes + off);
    } else if constexpr (NB == 6) {
      const uint16_t *h = reinterpret_cast<const uint16_t *>(p.codes + off);
      bits = (uint64_t)h[0] | ((uint64_t)h[1] << 16) | ((uint64_t)h[2] << 32);
    } else {
      bits = *reinterpret_cast<const uint32_t *>(p.codes + off);
    }
  } else {
#pragma unroll
    for (int b = 0; b < NB; ++b) bits |= (uint64_t)p.codes[off + b] << (8 * b);
  }
  constexpr int CB = FMT == kMxFp8 ? 8 : (FMT == kMxFp6E2M3 ? 6 : 4);
#pragma unroll
  for (int e = 0; e < 8; ++e) codes[e] = (uint32_t)(bits >> (CB * e)) & ((1u << CB) - 1u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float level;
    if constexpr (FMT == kMxFp8) {
      level = Fp8E4M3ToF32((uint8_t)codes[e]);
      if ((codes[e] & 0x7fu) == 0x7fu) fail(3 + 2 * (e0 + e));
    } else if constexpr (FMT == kMxFp6E2M3) {
      level = Fp6ToF32<3>(codes[e]);
    } else {
      level = Fp4E2M1ToF32(codes[e]);
    }
    v[e] = level * scale;
    if (!__builtin_isfinite(v[e])) fail(4 + 2 * (e0 + e));
  }
  unsigned flag = 0;
  if constexpr (OUT == kFloat16 || OUT == kBfloat16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t hb = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
      const bool inf = OUT == kFloat16 ? (hb & 0x7c00u) == 0x7c00u : (hb & 0x7f80u) == 0x7f80u;
      if (inf && __builtin_isfinite(v[e])) flag = kMxBadOutput;
    }
  }
  if (y != nullptr) {
    if constexpr (OUT == kFloat) {
      float *o = static_cast<float *>(y) + i0;
      if (p.aligned) {
        reinterpret_cast<float4 *>(o)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4 *>(o)[1] = make_float4(v[4], v[5], v[6], v[7]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) __builtin_memcpy(o + e, &v[e], 4);
      }
    } else if constexpr (OUT == kDouble) {
      double *o = static_cast<double *>(y) + i0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const double d = (double)v[e];
        if (p.aligned) o[e] = d;
        else __builtin_memcpy(o + e, &d, 8);
      }
    } else {
      uint32_t wds[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t lo = OUT == kFloat16 ? F32ToF16(v[2 * e]) : F32ToBf16(v[2 * e]);
        const uint16_t hi = OUT == kFloat16 ? F32ToF16(v[2 * e + 1]) : F32ToBf16(v[2 * e + 1]);
        wds[e] = (uint32_t)lo | ((uint32_t)hi << 16);
      }
      uint16_t *o = static_cast<uint16_t *>(y) + i0;
      if (p.aligned) *reinterpret_cast<uint4 *>(o) = make_uint4(wds[0], wds[1], wds[2], wds[3]);
      else __builtin_memcpy(o, wds, 16);
    }
  }
  if (key != ~0ull) atomicMax(reinterpret_cast<unsigned long long *>(p.first), (unsigned long long)~key);
  if (flag) atomicOr(p.flag, flag);
}

template <int FMT> void Launch(const MxParams &p, int out_dtype, void *y, hipStream_t s) {
  const int64_t threads = p.count / 8;
  const dim3 g((unsigned)((threads + 255) / 256)), b(256);
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL((MxDecodeKernel<FMT, kFloat>), g, b, 0, s, p, y); break;
  case kDouble: hipLaunchKernelGGL((MxDecodeKernel<FMT, kDouble>), g, b, 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL((MxDecodeKernel<FMT, kFloat16>), g, b, 0, s, p, y); break;
  default: hipLaunchKernelGGL((MxDecodeKernel<FMT, kBfloat16>), g, b, 0, s, p, y); break;
  }
}

}  // namespace

void LaunchMxDecode(const MxParams &p, int format, int out_dtype, void *y, hipStream_t s) {
  if (p.count == 0) return;
  switch (format) {
  case kMxFp4: Launch<kMxFp4>(p, out_dtype, y, s); break;
  case kMxFp6E2M3: Launch<kMxFp6E2M3>(p, out_dtype, y, s); break;
  case kMxFp8: Launch<kMxFp8>(p, out_dtype, y, s); break;
  default: Launch<kMxNvfp4>(p, out_dtype, y, s); break;
  }
}

}  // namespace onnxl_amd
