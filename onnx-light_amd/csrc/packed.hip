// DequantizePacked (onnx_core/runtime/dequantize_packed.cc) for the 32-value
// GGUF block formats: q4_0, q4_1, q5_0, q5_1, q8_0, q8_1 and iq4_nl.  A block
// is an fp16 scale d (plus an fp16 minimum m for q4_1 / q5_1, a 4-byte high
// bit plane for q5_*, an fp16 sum for q8_1) and 32 codes; the value is
// d * q (+ m), every fp32 step rounded on its own (no contraction), then
// converted to the output dtype with the Cast rounding rules.
//
// Four threads share a block, 8 consecutive values each, so a wave writes
// 64 x 8 consecutive outputs: an HBM stream whose output dominates (fp32 is
// 7.1x the q4_0 bytes).
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

// d * q + m is two roundings in the reference (each step forced through a
// volatile fp32): no multiply-add may be fused in this file.  The operators
// are written out here, under the pragma; __fmul_rn / __fadd_rn come from a
// header the pragma does not reach and still let the backend fuse them.
#pragma clang fp contract(off)

namespace onnxl_amd {
namespace {

constexpr int kPkThreads = 256;

template <int TYPE> struct PkLayout;
template <> struct PkLayout<2> { static constexpr int bytes = 18, codes = 2; };   // q4_0
template <> struct PkLayout<3> { static constexpr int bytes = 20, codes = 4; };   // q4_1
template <> struct PkLayout<6> { static constexpr int bytes = 22, codes = 6; };   // q5_0
template <> struct PkLayout<7> { static constexpr int bytes = 24, codes = 8; };   // q5_1
template <> struct PkLayout<8> { static constexpr int bytes = 34, codes = 2; };   // q8_0
template <> struct PkLayout<9> { static constexpr int bytes = 36, codes = 4; };   // q8_1
template <> struct PkLayout<20> { static constexpr int bytes = 18, codes = 2; };  // iq4_nl

__constant__ int kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

__device__ __forceinline__ float Half2(const uint8_t *p) { return F16ToF32((uint16_t)(p[0] | (p[1] << 8))); }

// The output is not read again: vector stores go through a buffer descriptor
// over the workgroup's share with the write-through policy (sc1), so no dirty
// lines are left in the L2 to flush at the end of the kernel.
constexpr int kWriteThrough = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ShareRsrc(void *y, int64_t at, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(static_cast<char *>(y) + at, (short)0, bytes, 0x00020000);
}

template <int OUT> __device__ __forceinline__ void StoreEight(void *y, int64_t i0, const float *v, bool vec) {
  constexpr int kBytes = OUT == kFloat ? 32 : 16;  // per thread on the vector paths
  if constexpr (OUT == kFloat) {
    float *dst = static_cast<float *>(y) + i0;
    if (vec) {
      typedef int v4i __attribute__((ext_vector_type(4)));
      const __amdgpu_buffer_rsrc_t rs =
          ShareRsrc(y, ((int64_t)blockIdx.x * kPkThreads) * kBytes, kPkThreads * kBytes);
      const unsigned off = threadIdx.x * kBytes;
      __builtin_amdgcn_raw_buffer_store_b128(
          v4i{__builtin_bit_cast(int, v[0]), __builtin_bit_cast(int, v[1]), __builtin_bit_cast(int, v[2]),
              __builtin_bit_cast(int, v[3])},
          rs, off, 0, kWriteThrough);
      __builtin_amdgcn_raw_buffer_store_b128(
          v4i{__builtin_bit_cast(int, v[4]), __builtin_bit_cast(int, v[5]), __builtin_bit_cast(int, v[6]),
              __builtin_bit_cast(int, v[7])},
          rs, off + 16, 0, kWriteThrough);
    } else {
      for (int e = 0; e < 8; ++e) dst[e] = v[e];
    }
  } else if constexpr (OUT == kDouble) {
    double *dst = static_cast<double *>(y) + i0;
    for (int e = 0; e < 8; ++e) dst[e] = (double)v[e];
  } else {
    uint16_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
    uint16_t *dst = static_cast<uint16_t *>(y) + i0;
    if (vec) {
      typedef int v4i __attribute__((ext_vector_type(4)));
      v4i w;
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = (int)((uint32_t)h[2 * k] | (uint32_t)h[2 * k + 1] << 16);
      __builtin_amdgcn_raw_buffer_store_b128(w, ShareRsrc(y, ((int64_t)blockIdx.x * kPkThreads) * kBytes,
                                                          kPkThreads * kBytes),
                                             threadIdx.x * kBytes, 0, kWriteThrough);
    } else {
      for (int e = 0; e < 8; ++e) dst[e] = h[e];
    }
  }
}

template <int TYPE, int OUT>
__global__ __launch_bounds__(kPkThreads) void DequantPackedKernel(const uint8_t *__restrict__ x, int64_t nblocks,
                                                                  void *__restrict__ y, int vec) {
  const int64_t t = (int64_t)blockIdx.x * kPkThreads + threadIdx.x;
  if (t >= nblocks * 4) return;
  const int64_t b = t >> 2;
  const int i0 = (int)(t & 3) * 8;  // first of this thread's 8 values in the block
  const uint8_t *p = x + b * PkLayout<TYPE>::bytes;
  const float d = Half2(p);
  float v[8];
  if constexpr (TYPE == 8 || TYPE == 9) {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = d * (float)(int8_t)p[PkLayout<TYPE>::codes + i0 + e];
  } else {
    constexpr bool kAffine = TYPE == 3 || TYPE == 7, kFive = TYPE == 6 || TYPE == 7;
    // element i: nibble (i % 16) of the code bytes, low half for i < 16
    const uint8_t *codes = p + PkLayout<TYPE>::codes;
    const int shift = i0 >= 16 ? 4 : 0;
    uint32_t qh = 0;
    if constexpr (kFive) {
      const uint8_t *h = p + (kAffine ? 4 : 2);
      qh = (uint32_t)h[0] | (uint32_t)h[1] << 8 | (uint32_t)h[2] << 16 | (uint32_t)h[3] << 24;
    }
    float m = 0.f;
    if constexpr (kAffine) m = Half2(p + 2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = i0 + e;
      int q = (codes[i & 15] >> shift) & 15;
      if constexpr (kFive) q |= (int)((qh >> i) & 1u) << 4;
      if constexpr (TYPE == 20) {
        v[e] = d * (float)kIq4Values[q];
      } else {
        if constexpr (!kAffine) q -= kFive ? 16 : 8;
        v[e] = d * (float)q;
        if constexpr (kAffine) v[e] = v[e] + m;
      }
    }
  }
  StoreEight<OUT>(y, b * 32 + i0, v, vec != 0);
}

template <int TYPE> void LaunchPkOut(const uint8_t *x, int64_t nblocks, int out, void *y, int vec, hipStream_t s) {
  const dim3 g((unsigned)((nblocks * 4 + kPkThreads - 1) / kPkThreads));
  switch (out) {
  case kFloat: hipLaunchKernelGGL((DequantPackedKernel<TYPE, kFloat>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kFloat16: hipLaunchKernelGGL((DequantPackedKernel<TYPE, kFloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kBfloat16: hipLaunchKernelGGL((DequantPackedKernel<TYPE, kBfloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  default: hipLaunchKernelGGL((DequantPackedKernel<TYPE, kDouble>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  }
}

}  // namespace

bool PackedFormatOnGpu(int ggml_type) {
  return ggml_type == 2 || ggml_type == 3 || ggml_type == 6 || ggml_type == 7 || ggml_type == 8 ||
         ggml_type == 9 || ggml_type == 20;
}

void LaunchDequantizePacked(int ggml_type, const uint8_t *x, int64_t nblocks, int out_dtype, void *y,
                            hipStream_t s) {
  if (nblocks == 0) return;
  const int vec = reinterpret_cast<uintptr_t>(y) % 16 == 0;
  switch (ggml_type) {
  case 2: LaunchPkOut<2>(x, nblocks, out_dtype, y, vec, s); break;
  case 3: LaunchPkOut<3>(x, nblocks, out_dtype, y, vec, s); break;
  case 6: LaunchPkOut<6>(x, nblocks, out_dtype, y, vec, s); break;
  case 7: LaunchPkOut<7>(x, nblocks, out_dtype, y, vec, s); break;
  case 8: LaunchPkOut<8>(x, nblocks, out_dtype, y, vec, s); break;
  case 9: LaunchPkOut<9>(x, nblocks, out_dtype, y, vec, s); break;
  case 20: LaunchPkOut<20>(x, nblocks, out_dtype, y, vec, s); break;
  default: throw Unsupported("DequantizePacked: no GPU kernel for this format");
  }
}

}  // namespace onnxl_amd
