// AWQ and GPTQ checkpoint weights on the GPU (onnx_core/runtime/awq.cc,
// onnx_core/runtime/gptq.cc; layouts in checkpoint_layout.hpp).
//
// Preparation for the fused DequantizeLinear -> MatMul kernels, once per
// weight, so that MatMul(A, W) with W [K, N] = (code - zero) * scale runs on
// the decode GEMV / GEMM paths without a dense W:
//  - codes of at most 4 bits: the tiled UINT4 layout of the 4-bit paths
//    (each 16-column tile's K range contiguous, rows past K zero);
//  - 5 to 8 bits: UINT8 [K, N];
//  - zero points UINT4 (two per byte, ONNX order) or UINT8 [groups, N];
//  - scales [groups, N]: FLOAT16 and FLOAT kept, BFLOAT16 widened to FLOAT
//    (DequantizeLinear takes FLOAT or FLOAT16 scales; a Cast to BFLOAT16
//    then gives the reference's rounding); AWQ gemv's [N, padded] read
//    transposed.
// Decode of the whole weight to [N, K] values in FLOAT, FLOAT16, BFLOAT16 or
// DOUBLE (the reference's Reconstruct*Weights, then its WriteFloat).
// Every kernel is one thread per output word or element; all reads go
// through CkptCode / CkptZero.
#include "checkpoint_layout.hpp"
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kGroupRows = 128;  // the tiled layout's row group (gemv_q4_tiled.hip)

// Tiled 4-bit word idx = ((t * ngroups + q) * 64 + l) * 4 + c: column
// 16 t + l % 16, rows 128 q + 32 c + 8 (l / 16) + (0..7), row 2i at bits 4i
// and row 2i + 1 at bits 16 + 4i.
__global__ void CkptTileUint4Kernel(CkptLayout L, int64_t ngroups, int64_t total, uint32_t *__restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx & 3);
  const int l = (int)((idx >> 2) & 63);
  const int64_t tq = idx >> 8;
  const int64_t t = tq / ngroups, q = tq % ngroups;
  const int64_t col = 16 * t + (l & 15);
  const int64_t row0 = kGroupRows * q + 32 * c + 8 * (l >> 4);
  uint32_t word = 0;
  if (col < L.N) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t row = row0 + j;
      const uint32_t u = row < L.K ? CkptCode(L, row, col) : 0u;
      word |= u << ((j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1));
    }
  }
  out[idx] = word;
}

// UINT8 codes [K, N]
__global__ void CkptBytesKernel(CkptLayout L, uint8_t *__restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= L.K * L.N) return;
  out[e] = (uint8_t)CkptCode(L, e / L.N, e % L.N);
}

// zero points [groups, N]: UINT4 two per byte (element g * N + n in the low
// nibble when even) or UINT8
__global__ void CkptZerosKernel(CkptLayout L, int four, int64_t out_bytes, uint8_t *__restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= out_bytes) return;
  if (!four) {
    out[b] = (uint8_t)CkptZero(L, b / L.N, b % L.N);
    return;
  }
  uint32_t v = 0;
  for (int h = 0; h < 2; ++h) {
    const int64_t e = 2 * b + h;
    if (e >= L.groups * L.N) break;
    v |= (CkptZero(L, e / L.N, e % L.N) & 15u) << (4 * h);
  }
  out[b] = (uint8_t)v;
}

// scales [groups, N] from the checkpoint's layout: FLOAT16 and FLOAT copied,
// BFLOAT16 widened to FLOAT (exact)
template <typename E, bool WIDEN>
__global__ void CkptScalesKernel(CkptLayout L, const E *__restrict__ s, void *__restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= L.groups * L.N) return;
  const E v = s[CkptScaleIndex(L, e / L.N, e % L.N)];
  if constexpr (WIDEN) static_cast<uint32_t *>(out)[e] = (uint32_t)v << 16;
  else static_cast<E *>(out)[e] = v;
}

__device__ __forceinline__ float ScaleValue(const void *s, int dtype, int64_t i) {
  if (dtype == kFloat) return static_cast<const float *>(s)[i];
  const uint16_t h = static_cast<const uint16_t *>(s)[i];
  return dtype == kFloat16 ? F16ToF32(h) : Bf16ToF32(h);
}

// Dense values y [N, K]: (code - zero) * scale in fp32, or for AWQ gemv_fast
// / llm-awq code * scale rounded to fp32 plus the zero term; group of row k
// from g_idx (GPTQ) or k / group.
template <int OUT>
__global__ void CkptDecodeKernel(CkptLayout L, const void *__restrict__ scales, int scale_dtype,
                                 const uint16_t *__restrict__ zero_terms, const int32_t *__restrict__ g_idx,
                                 void *__restrict__ y) {
#pragma clang fp contract(off)
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= L.N * L.K) return;
  const int64_t n = e / L.K, k = e % L.K;
  const int64_t g = g_idx ? (int64_t)g_idx[k] : k / L.group;
  const float code = (float)CkptCode(L, k, n);
  const int64_t si = CkptScaleIndex(L, g, n);
  const float scale = ScaleValue(scales, scale_dtype, si);
  float v;
  if (L.kind == kAwqFast) {
    const float product = code * scale;
    v = product + F16ToF32(zero_terms[si]);
  } else {
    v = (code - (float)CkptZero(L, g, n)) * scale;
  }
  if constexpr (OUT == kFloat) static_cast<float *>(y)[e] = v;
  else if constexpr (OUT == kDouble) static_cast<double *>(y)[e] = (double)v;
  else if constexpr (OUT == kFloat16) static_cast<uint16_t *>(y)[e] = F32ToF16(v);
  else static_cast<uint16_t *>(y)[e] = F32ToBf16(v);
}

unsigned Blocks(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void LaunchCkptPrepare(const CkptLayout &L, const void *scales, int scale_dtype, void *weight, void *scale_out,
                       void *zp_out, hipStream_t stream) {
  const bool four = L.bits <= 4;
  if (four) {
    const int64_t ngroups = (L.K + kGroupRows - 1) / kGroupRows;
    const int64_t total = TiledInt4Bytes(L.K, L.N) / 4;
    if (total > 0)
      hipLaunchKernelGGL(CkptTileUint4Kernel, dim3(Blocks(total)), dim3(256), 0, stream, L, ngroups, total,
                         static_cast<uint32_t *>(weight));
  } else if (L.K * L.N > 0) {
    hipLaunchKernelGGL(CkptBytesKernel, dim3(Blocks(L.K * L.N)), dim3(256), 0, stream, L,
                       static_cast<uint8_t *>(weight));
  }
  const int64_t zp_bytes = four ? (L.groups * L.N + 1) / 2 : L.groups * L.N;
  if (zp_bytes > 0)
    hipLaunchKernelGGL(CkptZerosKernel, dim3(Blocks(zp_bytes)), dim3(256), 0, stream, L, (int)four, zp_bytes,
                       static_cast<uint8_t *>(zp_out));
  const dim3 sg(Blocks(L.groups * L.N));
  if (L.groups * L.N > 0) {
    if (scale_dtype == kFloat)
      hipLaunchKernelGGL((CkptScalesKernel<uint32_t, false>), sg, dim3(256), 0, stream, L,
                         static_cast<const uint32_t *>(scales), scale_out);
    else if (scale_dtype == kBfloat16)
      hipLaunchKernelGGL((CkptScalesKernel<uint16_t, true>), sg, dim3(256), 0, stream, L,
                         static_cast<const uint16_t *>(scales), scale_out);
    else
      hipLaunchKernelGGL((CkptScalesKernel<uint16_t, false>), sg, dim3(256), 0, stream, L,
                         static_cast<const uint16_t *>(scales), scale_out);
  }
}

void LaunchCkptDecode(const CkptLayout &L, const void *scales, int scale_dtype, const uint16_t *zero_terms,
                      const int32_t *g_idx, int out_dtype, void *y, hipStream_t stream) {
  const int64_t count = L.N * L.K;
  if (count == 0) return;
  const dim3 g(Blocks(count)), b(256);
  switch (out_dtype) {
  case kFloat:
    hipLaunchKernelGGL(CkptDecodeKernel<kFloat>, g, b, 0, stream, L, scales, scale_dtype, zero_terms, g_idx, y);
    break;
  case kFloat16:
    hipLaunchKernelGGL(CkptDecodeKernel<kFloat16>, g, b, 0, stream, L, scales, scale_dtype, zero_terms, g_idx, y);
    break;
  case kBfloat16:
    hipLaunchKernelGGL(CkptDecodeKernel<kBfloat16>, g, b, 0, stream, L, scales, scale_dtype, zero_terms, g_idx, y);
    break;
  default:
    hipLaunchKernelGGL(CkptDecodeKernel<kDouble>, g, b, 0, stream, L, scales, scale_dtype, zero_terms, g_idx, y);
    break;
  }
}

}  // namespace onnxl_amd
