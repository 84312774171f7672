// Element-wise kernels: standalone DequantizeLinear (per-tensor, per-axis,
// blocked; kq/kernel_dequantizelinear.cc) and the FLOAT -> FLOAT16/BFLOAT16
// Cast (ext/kernels/kernels/tensor/kernel_cast.cc:360-370).  Both are
// HBM-bound streams: each thread handles 8 consecutive elements so 4-bit
// inputs are read a whole 32-bit word at a time.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kPerThread = 8;
constexpr int kBlock = 256;

template <int XT, int MODE, bool F16S>
__global__ __launch_bounds__(kBlock) void DequantKernel(const DequantParams p) {
  const int64_t first = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * kPerThread;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int64_t i = first + e;
    if (i >= p.n) return;
    int64_t si = 0;
    if (MODE == 1) {
      si = (i / p.inner) % p.axis_len;
    } else if (MODE == 2) {
      const int64_t outer = i / (p.axis_len * p.inner);
      const int64_t a = (i / p.inner) % p.axis_len;
      si = (outer * p.s_axis + a / p.block) * p.inner + i % p.inner;
    }
    const float s = F16S ? F16ToF32(static_cast<const uint16_t *>(p.scale)[si])
                         : static_cast<const float *>(p.scale)[si];
    const float z = p.zp ? DecodeElement<XT>(p.zp, si) : 0.0f;
    const float v = SseMul(SseSub(DecodeElement<XT>(p.x, i), z), s);  // NaNs as the reference's x86-64 build
    if (F16S) {
      static_cast<uint16_t *>(p.y)[i] = F32ToF16(v);
    } else {
      static_cast<float *>(p.y)[i] = v;
    }
  }
}

template <int XT, int MODE>
void LaunchMode(const DequantParams &p, dim3 g, hipStream_t s) {
  if (p.scale_f16) hipLaunchKernelGGL((DequantKernel<XT, MODE, true>), g, dim3(kBlock), 0, s, p);
  else hipLaunchKernelGGL((DequantKernel<XT, MODE, false>), g, dim3(kBlock), 0, s, p);
}

template <int XT>
void LaunchX(const DequantParams &p, dim3 g, hipStream_t s) {
  if (p.mode == 0) LaunchMode<XT, 0>(p, g, s);
  else if (p.mode == 1) LaunchMode<XT, 1>(p, g, s);
  else LaunchMode<XT, 2>(p, g, s);
}

__global__ __launch_bounds__(kBlock) void CastF32Kernel(const float *x, uint16_t *y, int64_t n,
                                                        int to_bf16) {
  const int64_t first = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * kPerThread;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const int64_t i = first + e;
    if (i >= n) return;
    y[i] = to_bf16 ? F32ToBf16(x[i]) : F32ToF16(x[i]);
  }
}

}  // namespace

void LaunchDequantize(const DequantParams &p, hipStream_t s) {
  if (p.n == 0) return;
  const dim3 g((unsigned)((p.n + (int64_t)kBlock * kPerThread - 1) / ((int64_t)kBlock * kPerThread)));
  switch (p.x_dtype) {
  case kUint8: LaunchX<kUint8>(p, g, s); break;
  case kInt8: LaunchX<kInt8>(p, g, s); break;
  case kUint16: LaunchX<kUint16>(p, g, s); break;
  case kInt16: LaunchX<kInt16>(p, g, s); break;
  case kInt32: LaunchX<kInt32>(p, g, s); break;
  case kFloat8E4M3FN: LaunchX<kFloat8E4M3FN>(p, g, s); break;
  case kInt4: LaunchX<kInt4>(p, g, s); break;
  case kUint4: LaunchX<kUint4>(p, g, s); break;
  case kFloat8E4M3FNUZ: LaunchX<kFloat8E4M3FNUZ>(p, g, s); break;
  case kFloat8E5M2: LaunchX<kFloat8E5M2>(p, g, s); break;
  case kFloat8E5M2FNUZ: LaunchX<kFloat8E5M2FNUZ>(p, g, s); break;
  case kFloat4E2M1: LaunchX<kFloat4E2M1>(p, g, s); break;
  case kUint2: LaunchX<kUint2>(p, g, s); break;
  case kInt2: LaunchX<kInt2>(p, g, s); break;
  case kFloat6E2M3: LaunchX<kFloat6E2M3>(p, g, s); break;
  case kFloat6E3M2: LaunchX<kFloat6E3M2>(p, g, s); break;
  default: throw Unsupported("DequantizeLinear: no GPU kernel for this dtype");
  }
}

// Transpose of a [R, C] matrix of T (1, 2, 4 or 8 bytes): one 64 x 64 tile
// per 256-thread workgroup, read row-wise (consecutive threads on
// consecutive columns), held in LDS with a padded pitch, written row-wise
// in the output's order.  Tiles are dealt in row-major order over
// (row blocks, column blocks) with the row block in blockIdx.y.
template <typename T>
__global__ __launch_bounds__(256) void Transpose2dKernel(const T *__restrict__ x, T *__restrict__ y, int64_t R,
                                                         int64_t C) {
  __shared__ T tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = ty + 4 * i;
    if (r0 + rr < R && c0 + tx < C) tile[rr][tx] = x[(r0 + rr) * C + c0 + tx];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int cc = ty + 4 * i;  // output row c0 + cc, output column r0 + tx
    if (c0 + cc < C && r0 + tx < R) y[(c0 + cc) * R + r0 + tx] = tile[tx][cc];
  }
}

void LaunchTranspose2d(const void *x, void *y, int64_t R, int64_t C, int elem_bytes, hipStream_t s) {
  if (R == 0 || C == 0) return;
  const dim3 g((unsigned)((C + 63) / 64), (unsigned)((R + 63) / 64)), b(256);
  switch (elem_bytes) {
  case 1:
    hipLaunchKernelGGL(Transpose2dKernel<uint8_t>, g, b, 0, s, static_cast<const uint8_t *>(x),
                       static_cast<uint8_t *>(y), R, C);
    break;
  case 2:
    hipLaunchKernelGGL(Transpose2dKernel<uint16_t>, g, b, 0, s, static_cast<const uint16_t *>(x),
                       static_cast<uint16_t *>(y), R, C);
    break;
  case 4:
    hipLaunchKernelGGL(Transpose2dKernel<uint32_t>, g, b, 0, s, static_cast<const uint32_t *>(x),
                       static_cast<uint32_t *>(y), R, C);
    break;
  default:
    hipLaunchKernelGGL(Transpose2dKernel<uint64_t>, g, b, 0, s, static_cast<const uint64_t *>(x),
                       static_cast<uint64_t *>(y), R, C);
    break;
  }
}

void LaunchCastF32(const float *x, void *y, int64_t n, int to_bf16, hipStream_t s) {
  if (n == 0) return;
  const dim3 g((unsigned)((n + (int64_t)kBlock * kPerThread - 1) / ((int64_t)kBlock * kPerThread)));
  hipLaunchKernelGGL(CastF32Kernel, g, dim3(kBlock), 0, s, x, static_cast<uint16_t *>(y), n, to_bf16);
}

}  // namespace onnxl_amd
