// ConvInteger (nn/kernel_conv_integer.cc) and QLinearConv
// (kq/kernel_qlinearconv.cc) on the int8 GEMM core.
//
// For output channel m of group g and batch n the convolution is the GEMM
//   Y[n, g*Mg + r, p] = sum_k W[g*Mg + r, k] * Col[n, g, k, p]
// over k = (input channel of the group, kernel tap), with W in its ONNX
// layout [M, C/group, kernel...] (already the row-major A operand) and Col
// built by ImToColKernel: Col[n, g, k, p] is the input byte the tap reads for
// output position p, or x's zero point where the tap falls into the padding
// (which then contributes (x_zp - x_zp) * (w - w_zp) = 0, exactly the
// reference's skipped tap).  The GEMM output [n, g, Mg, P] is the NCHW output.
//
// DirectConvKernel computes the same sums one output per thread: the path for
// grouped convolutions with per-channel weight zero points (whose zero point
// would change along the GEMM batch), and for QLinearConv sums that int32
// does not hold exactly.  ConvRequantKernel applies QLinearConv's bias and
// requantization to the GEMM's int32 sums.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kCBlock = 256;

// Input coordinates of output position p and kernel tap (kz, ky, kx) along
// the three right-aligned spatial dims; false when the tap is in the padding.
__device__ __forceinline__ bool TapOffset(const ConvGeom &g, int64_t oz, int64_t oy, int64_t ox, int kz, int ky,
                                          int kx, int64_t &off) {
  const int64_t iz = oz * g.s[0] - g.pb[0] + kz * g.d[0];
  const int64_t iy = oy * g.s[1] - g.pb[1] + ky * g.d[1];
  const int64_t ix = ox * g.s[2] - g.pb[2] + kx * g.d[2];
  if (iz < 0 || iz >= g.in[0] || iy < 0 || iy >= g.in[1] || ix < 0 || ix >= g.in[2]) return false;
  off = (iz * g.in[1] + iy) * g.in[2] + ix;
  return true;
}

// Col[n, g, k, p] for a row (n, g, k) and 4 consecutive positions per thread.
__global__ __launch_bounds__(kCBlock) void ImToColKernel(const ConvGeom g, const uint8_t *x, uint8_t x_zp,
                                                          uint8_t *col) {
  const int64_t quads = (g.P + 3) / 4;
  const int64_t t = (int64_t)blockIdx.x * kCBlock + threadIdx.x;
  const int64_t rows = g.N * g.G * g.Kc;
  if (t >= rows * quads) return;
  const int64_t row = t / quads;
  const int64_t p0 = (t - row * quads) * 4;
  const int64_t k = row % g.Kc;
  const int64_t ng = row / g.Kc;  // n * G + grp
  const int64_t c = k / g.ks, tap = k - c * g.ks;
  const int kx = (int)(tap % g.k[2]), ky = (int)((tap / g.k[2]) % g.k[1]), kz = (int)(tap / (g.k[2] * g.k[1]));
  const int64_t grp = ng % g.G, n = ng / g.G;
  const uint8_t *plane = x + ((n * g.C + grp * g.cpg + c) * g.in_size);
  int64_t ox = p0 % g.out[2], oy = (p0 / g.out[2]) % g.out[1], oz = p0 / (g.out[2] * g.out[1]);
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint8_t v = x_zp;
    int64_t off;
    if (p0 + e < g.P && TapOffset(g, oz, oy, ox, kz, ky, kx, off)) v = plane[off];
    word |= (uint32_t)v << (8 * e);
    if (++ox == g.out[2]) {
      ox = 0;
      if (++oy == g.out[1]) {
        oy = 0;
        ++oz;
      }
    }
  }
  uint8_t *dst = col + row * g.P + p0;
  if (p0 + 4 <= g.P && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
    *reinterpret_cast<uint32_t *>(dst) = word;
  } else {
    for (int e = 0; e < 4 && p0 + e < g.P; ++e) dst[e] = (uint8_t)(word >> (8 * e));
  }
}

__device__ __forceinline__ int32_t ByteValue(const uint8_t *p, int64_t i, int is_u8) {
  return is_u8 ? (int32_t)p[i] : (int32_t)(int8_t)p[i];
}

// The reference's saturating requantization (kernel_qlinearconv.cc:127-138,
// :332-339): ties-to-even, zero point, clamp; NaN lands as 0 as it does
// through the x86-64 conversion.
__device__ __forceinline__ uint8_t Requant(int64_t acc, float cs, const ConvQuant &q) {
  const float v = __builtin_rintf((float)acc * cs) + q.zy;
  if (v != v) return 0;
  return (uint8_t)(int32_t)__builtin_amdgcn_fmed3f(v, q.qmin, q.qmax);
}

__device__ __forceinline__ float CombinedScale(const ConvQuant &q, int64_t m) {
  const float ws = q.w_scale[q.w_scale_per_channel ? m : 0];
  return q.x_scale * ws / q.y_scale;  // left to right, as :289
}

// One output per thread: (n, m, p) over the group's input channels and taps.
// QUANT: int64 sum, bias, requantization (QLinearConv); otherwise the int32
// wrap of ConvInteger.
template <bool QUANT>
__global__ __launch_bounds__(kCBlock) void DirectConvKernel(const ConvGeom g, const uint8_t *x, int x_u8,
                                                             uint8_t x_zp, const uint8_t *w, int w_u8,
                                                             const uint8_t *w_zp, int32_t w_zp_scalar,
                                                             const ConvQuant q, void *y) {
  const int64_t t = (int64_t)blockIdx.x * kCBlock + threadIdx.x;
  const int64_t total = g.N * g.M * g.P;
  if (t >= total) return;
  const int64_t p = t % g.P, nm = t / g.P;
  const int64_t m = nm % g.M, n = nm / g.M;
  const int64_t grp = m / g.Mg;
  const int32_t xz = x_u8 ? (int32_t)x_zp : (int32_t)(int8_t)x_zp;
  const int32_t wz = w_zp ? ByteValue(w_zp, m, w_u8) : w_zp_scalar;  // per channel, or the scalar
  const int64_t ox = p % g.out[2], oy = (p / g.out[2]) % g.out[1], oz = p / (g.out[2] * g.out[1]);
  int64_t acc = 0;
  uint32_t acc32 = 0;
  for (int64_t c = 0; c < g.cpg; ++c) {
    const uint8_t *plane = x + (n * g.C + grp * g.cpg + c) * g.in_size;
    const uint8_t *wrow = w + (m * g.cpg + c) * g.ks;
    int64_t tap = 0;
    for (int kz = 0; kz < g.k[0]; ++kz)
      for (int ky = 0; ky < g.k[1]; ++ky)
        for (int kx = 0; kx < g.k[2]; ++kx, ++tap) {
          int64_t off;
          if (!TapOffset(g, oz, oy, ox, kz, ky, kx, off)) continue;
          const int32_t prod = (ByteValue(plane, off, x_u8) - xz) * (ByteValue(wrow, tap, w_u8) - wz);
          if constexpr (QUANT) acc += prod;
          else acc32 += (uint32_t)prod;
        }
  }
  if constexpr (QUANT) {
    if (q.bias) acc += q.bias[m];
    static_cast<uint8_t *>(y)[t] = Requant(acc, CombinedScale(q, m), q);
  } else {
    static_cast<int32_t *>(y)[t] = (int32_t)acc32;
  }
}

// QLinearConv's bias and requantization of the GEMM's int32 sums [N, M, P]:
// 4 positions per thread, one channel per thread.
__global__ __launch_bounds__(kCBlock) void ConvRequantKernel(const ConvGeom g, const int32_t *acc, const ConvQuant q,
                                                             uint8_t *y) {
  const int64_t quads = (g.P + 3) / 4;
  const int64_t t = (int64_t)blockIdx.x * kCBlock + threadIdx.x;
  if (t >= g.N * g.M * quads) return;
  const int64_t nm = t / quads;
  const int64_t p0 = (t - nm * quads) * 4;
  const int64_t m = nm % g.M;
  const float cs = CombinedScale(q, m);
  const int64_t bias = q.bias ? q.bias[m] : 0;
  const int64_t base = nm * g.P + p0;
  for (int e = 0; e < 4 && p0 + e < g.P; ++e) y[base + e] = Requant((int64_t)acc[base + e] + bias, cs, q);
}

unsigned Blocks(int64_t threads) { return (unsigned)((threads + kCBlock - 1) / kCBlock); }

}  // namespace

size_t ConvColBytes(const ConvGeom &g) { return (size_t)(g.N * g.G * g.Kc * g.P); }

void LaunchImToCol(const ConvGeom &g, const uint8_t *x, uint8_t x_zp, uint8_t *col, hipStream_t s) {
  const int64_t threads = g.N * g.G * g.Kc * ((g.P + 3) / 4);
  if (threads == 0) return;
  hipLaunchKernelGGL(ImToColKernel, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_zp, col);
}

void LaunchDirectConv(const ConvGeom &g, const uint8_t *x, int x_u8, uint8_t x_zp, const uint8_t *w, int w_u8,
                      const uint8_t *w_zp_per_channel, int32_t w_zp_scalar, const ConvQuant *q, void *y,
                      hipStream_t s) {
  const int64_t threads = g.N * g.M * g.P;
  if (threads == 0) return;
  if (q)
    hipLaunchKernelGGL(DirectConvKernel<true>, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_u8, x_zp, w,
                       w_u8, w_zp_per_channel, w_zp_scalar, *q, y);
  else
    hipLaunchKernelGGL(DirectConvKernel<false>, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_u8, x_zp, w,
                       w_u8, w_zp_per_channel, w_zp_scalar, ConvQuant{}, y);
}

void LaunchConvRequant(const ConvGeom &g, const int32_t *acc, const ConvQuant &q, uint8_t *y, hipStream_t s) {
  const int64_t threads = g.N * g.M * ((g.P + 3) / 4);
  if (threads == 0) return;
  hipLaunchKernelGGL(ConvRequantKernel, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, acc, q, y);
}

}  // namespace onnxl_amd
