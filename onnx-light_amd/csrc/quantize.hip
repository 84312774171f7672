// QuantizeLinear (kq/kernel_quantizelinear.cc) and DynamicQuantizeLinear
// (kq/kernel_dynamicquantizelinear.cc): the producers in front of
// MatMulInteger / QLinearMatMul.  Both are HBM streams with an fp32 IEEE
// division per element (x / scale, as the reference divides), so each thread
// takes 8 consecutive elements with whole-vector loads and stores, and the
// scale index is stepped along the 8 elements instead of divided out for
// each.
#include <cfloat>

#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kQBlock = 256;
constexpr int kQPer = 8;  // elements per thread

typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// x is read once: non-temporal loads keep it from displacing cache lines that
// are reused.  y is not read again either: its stores write through the L2
// (sc1), because dirty write-back lines left in the L2 at the end of a kernel
// hold its completion until they are flushed.
constexpr int kWriteThrough = 16;
constexpr int kRsrcWord3 = 0x00020000;

__device__ __forceinline__ v4f LoadNt(const float *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
}

// Buffer descriptor over `bytes` bytes of y starting at byte `at` (a
// workgroup's share; the stores then carry the cache policy above).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t ShareRsrc(void *y, int64_t at, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(static_cast<char *>(y) + at, (short)0, bytes, kRsrcWord3);
}

template <bool F16> __device__ __forceinline__ float LoadF(const void *p, int64_t i) {
  if constexpr (F16) return F16ToF32(static_cast<const uint16_t *>(p)[i]);
  return static_cast<const float *>(p)[i];
}

// Saturation bounds of the integer outputs (numeric_limits of the reference's
// ZP type; -8..7 / 0..15 for 4-bit, :181-183).
template <int YT> struct Bounds;
template <> struct Bounds<kUint8> { static constexpr float lo = 0.f, hi = 255.f; };
template <> struct Bounds<kInt8> { static constexpr float lo = -128.f, hi = 127.f; };
template <> struct Bounds<kUint16> { static constexpr float lo = 0.f, hi = 65535.f; };
template <> struct Bounds<kInt16> { static constexpr float lo = -32768.f, hi = 32767.f; };
template <> struct Bounds<kUint4> { static constexpr float lo = 0.f, hi = 15.f; };
template <> struct Bounds<kInt4> { static constexpr float lo = -8.f, hi = 7.f; };
template <> struct Bounds<kUint2> { static constexpr float lo = 0.f, hi = 3.f; };
template <> struct Bounds<kInt2> { static constexpr float lo = -2.f, hi = 1.f; };

// Float outputs: the four fp8 types, FLOAT4E2M1 and the two FLOAT6 types.
template <int YT>
constexpr bool kFloatCode = YT == kFloat8E4M3FN || YT == kFloat8E4M3FNUZ || YT == kFloat8E5M2 ||
                            YT == kFloat8E5M2FNUZ || YT == kFloat4E2M1 || YT == kFloat6E2M3 || YT == kFloat6E3M2;

// Bits per stored element.
template <int YT>
constexpr int kYBitsOf = YT == kUint4 || YT == kInt4 || YT == kFloat4E2M1 ? 4
                         : YT == kUint2 || YT == kInt2                    ? 2
                         : YT == kFloat6E2M3 || YT == kFloat6E3M2         ? 6
                         : YT == kUint16 || YT == kInt16                  ? 16
                                                                          : 8;

// Zero point of scale index si (y's storage type) as a float.
template <int YT> __device__ __forceinline__ float ZeroPoint(const void *zp, int64_t si) {
  return DecodeElement<YT>(zp, si);
}

// The stored code of one element: the saturated integer (two's complement,
// narrowed by the store) or the float code.  NaN lands as 0 for the integer
// types, which is what the x86-64 float-to-int conversion of the reference
// build leaves after its two comparisons let NaN through (:75-80, :216-222).
// Float codes take x / scale + zero point (:228-268); without a zero point
// the caller passes z = -0, which adds nothing (-0 stays -0, :508-511).
template <int YT> __device__ __forceinline__ uint32_t QuantOne(float x, float s, float z) {
  const float q = x / s;  // IEEE division, as the reference divides
  if constexpr (kFloatCode<YT>) {
    const float v = q + z;
    if ((YT == kFloat8E4M3FN || YT == kFloat8E5M2) && v != v) {
      // The fp8 NaN keeps the fp32 NaN's sign, which the GPU and an x86-64
      // build set differently.  SSE returns its destination operand when both
      // are NaN, else the NaN one, and a negative default NaN for 0/0 and
      // inf/inf.  For x / s the destination is x; for the commutative q + z it
      // is the compiler's choice, and gcc -O2 puts z there.
      const uint32_t bits = z != z   ? __builtin_bit_cast(uint32_t, z)
                            : x != x ? __builtin_bit_cast(uint32_t, x)
                            : s != s ? __builtin_bit_cast(uint32_t, s)
                                     : 0xffc00000u;
      return (bits >> 31 ? 0x80u : 0u) | (YT == kFloat8E4M3FN ? 0x7fu : 0x7eu);
    }
    if constexpr (YT == kFloat8E4M3FN) return F32ToFp8E4M3Sat(v);
    else if constexpr (YT == kFloat8E4M3FNUZ) return F32ToFp8Sat<3, 8, true>(v);
    else if constexpr (YT == kFloat8E5M2) return F32ToFp8Sat<2, 15, false>(v);
    else if constexpr (YT == kFloat8E5M2FNUZ) return F32ToFp8Sat<2, 16, true>(v);
    else if constexpr (YT == kFloat4E2M1) return F32ToFp4E2M1(v);
    else return F32ToFp6<YT == kFloat6E2M3 ? 3 : 2>(v);
  } else {
    const float r = __builtin_rintf(q) + z;
    if (r != r) return 0u;
    return (uint32_t)(int)__builtin_amdgcn_fmed3f(r, Bounds<YT>::lo, Bounds<YT>::hi);
  }
}

template <bool XF16, int MODE, int YT>
__global__ __launch_bounds__(kQBlock) void QuantKernel(const QuantParams p) {
  const int64_t i0 = ((int64_t)blockIdx.x * kQBlock + threadIdx.x) * kQPer;
  if (i0 >= p.n) return;
  const bool full = i0 + kQPer <= p.n;
  float xv[kQPer];
  if (full && p.vec) {
    if constexpr (XF16) {
      const v8h h = __builtin_nontemporal_load(reinterpret_cast<const v8h *>(static_cast<const uint16_t *>(p.x) + i0));
#pragma unroll
      for (int e = 0; e < kQPer; ++e) xv[e] = (float)h[e];
    } else {
      const v4f a = LoadNt(static_cast<const float *>(p.x) + i0);
      const v4f b = LoadNt(static_cast<const float *>(p.x) + i0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[e] = a[e];
        xv[4 + e] = b[e];
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < kQPer; ++e) xv[e] = i0 + e < p.n ? LoadF<XF16>(p.x, i0 + e) : 0.f;
  }

  uint32_t code[kQPer];
  if constexpr (MODE == 0) {
    const float s = p.scale_f16 ? LoadF<true>(p.scale, 0) : LoadF<false>(p.scale, 0);
    const float z = p.zp ? ZeroPoint<YT>(p.zp, 0) : -0.f;
#pragma unroll
    for (int e = 0; e < kQPer; ++e) code[e] = QuantOne<YT>(xv[e], s, z);
  } else {
    // element i = (outer * axis_len + a) * inner + r; the scale index is a
    // (per-axis) or (outer * s_axis + a / block) * inner + r (blocked)
    const int64_t q = i0 / p.inner;
    int64_t r = i0 - q * p.inner;
    int64_t a = q % p.axis_len;
    int64_t outer = q / p.axis_len;
    int64_t ab = MODE == 2 ? a / p.block : 0;
    int64_t am = MODE == 2 ? a - ab * p.block : 0;
#pragma unroll
    for (int e = 0; e < kQPer; ++e) {
      // past the end `outer` leaves the scale tensor: those lanes load nothing
      const int64_t si = MODE == 1 ? a : (outer * p.s_axis + ab) * p.inner + r;
      if (full || i0 + e < p.n) {
        const float s = p.scale_f16 ? LoadF<true>(p.scale, si) : LoadF<false>(p.scale, si);
        const float z = p.zp ? ZeroPoint<YT>(p.zp, si) : -0.f;
        code[e] = QuantOne<YT>(xv[e], s, z);
      } else {
        code[e] = 0;
      }
      if (++r == p.inner) {
        r = 0;
        ++a;
        if (MODE == 2 && ++am == p.block) {
          am = 0;
          ++ab;
        }
        if (a == p.axis_len) {
          a = 0;
          am = 0;
          ab = 0;
          ++outer;
        }
      }
    }
  }

  // full vector stores go through the workgroup's buffer descriptor
  constexpr int kYBits = kYBitsOf<YT>;
  constexpr int kShare = kQBlock * kQPer * kYBits / 8;
  const unsigned off = threadIdx.x * (kQPer * kYBits / 8);
  if constexpr (kYBits == 2 || kYBits == 6) {
    // element i at bits kYBits * i of a little-endian bit stream (2-bit: four
    // per byte from the low bits; rk/cast_sub_byte.h); a thread's 8 elements
    // fill 2 or 6 whole bytes, stored one by one
    uint64_t word = 0;
#pragma unroll
    for (int e = 0; e < kQPer; ++e)
      word |= (uint64_t)(i0 + e < p.n ? (code[e] & ((1u << kYBits) - 1u)) : 0u) << (kYBits * e);
    uint8_t *y = static_cast<uint8_t *>(p.y) + i0 * kYBits / 8;
    const int64_t bytes = ((full ? kQPer : p.n - i0) * kYBits + 7) / 8;
#pragma unroll
    for (int k = 0; k < kQPer * kYBits / 8; ++k)
      if (k < bytes) y[k] = (uint8_t)(word >> (8 * k));
  } else if constexpr (kYBits == 4) {
    // element 2k in the low nibble of byte k (rk/cast_sub_byte.h:50-60)
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < kQPer; ++e) word |= (i0 + e < p.n ? (code[e] & 0xfu) : 0u) << (4 * e);
    uint8_t *y = static_cast<uint8_t *>(p.y) + (i0 >> 1);
    if (full && p.vec) {
      __builtin_amdgcn_raw_buffer_store_b32((int)word, ShareRsrc(p.y, (int64_t)blockIdx.x * kShare, kShare), off, 0,
                                            kWriteThrough);
    } else {
      const int64_t bytes = (p.n - i0 + 1) >> 1;
#pragma unroll
      for (int k = 0; k < kQPer / 2; ++k)
        if (k < bytes) y[k] = (uint8_t)(word >> (8 * k));
    }
  } else if constexpr (YT == kUint16 || YT == kInt16) {
    uint16_t *y = static_cast<uint16_t *>(p.y) + i0;
    if (full && p.vec) {
      v4i w;
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = (int)((code[2 * k] & 0xffffu) | (code[2 * k + 1] << 16));
      __builtin_amdgcn_raw_buffer_store_b128(w, ShareRsrc(p.y, (int64_t)blockIdx.x * kShare, kShare), off, 0,
                                             kWriteThrough);
    } else {
#pragma unroll
      for (int e = 0; e < kQPer; ++e)
        if (i0 + e < p.n) y[e] = (uint16_t)code[e];
    }
  } else {
    uint8_t *y = static_cast<uint8_t *>(p.y) + i0;
    if (full && p.vec) {
      v2i w;
#pragma unroll
      for (int k = 0; k < 2; ++k)
        w[k] = (int)((code[4 * k] & 0xffu) | (code[4 * k + 1] & 0xffu) << 8 | (code[4 * k + 2] & 0xffu) << 16 |
                     (code[4 * k + 3] << 24));
      __builtin_amdgcn_raw_buffer_store_b64(w, ShareRsrc(p.y, (int64_t)blockIdx.x * kShare, kShare), off, 0,
                                            kWriteThrough);
    } else {
#pragma unroll
      for (int e = 0; e < kQPer; ++e)
        if (i0 + e < p.n) y[e] = (uint8_t)code[e];
    }
  }
}

template <bool XF16, int MODE>
void LaunchQY(const QuantParams &p, dim3 g, hipStream_t s) {
  switch (p.y_dtype) {
  case kUint8: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kUint8>), g, dim3(kQBlock), 0, s, p); break;
  case kInt8: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kInt8>), g, dim3(kQBlock), 0, s, p); break;
  case kUint16: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kUint16>), g, dim3(kQBlock), 0, s, p); break;
  case kInt16: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kInt16>), g, dim3(kQBlock), 0, s, p); break;
  case kUint4: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kUint4>), g, dim3(kQBlock), 0, s, p); break;
  case kInt4: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kInt4>), g, dim3(kQBlock), 0, s, p); break;
  case kFloat8E4M3FN:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat8E4M3FN>), g, dim3(kQBlock), 0, s, p);
    break;
  case kFloat8E4M3FNUZ:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat8E4M3FNUZ>), g, dim3(kQBlock), 0, s, p);
    break;
  case kFloat8E5M2:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat8E5M2>), g, dim3(kQBlock), 0, s, p);
    break;
  case kFloat8E5M2FNUZ:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat8E5M2FNUZ>), g, dim3(kQBlock), 0, s, p);
    break;
  case kFloat4E2M1:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat4E2M1>), g, dim3(kQBlock), 0, s, p);
    break;
  case kUint2: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kUint2>), g, dim3(kQBlock), 0, s, p); break;
  case kInt2: hipLaunchKernelGGL((QuantKernel<XF16, MODE, kInt2>), g, dim3(kQBlock), 0, s, p); break;
  case kFloat6E2M3:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat6E2M3>), g, dim3(kQBlock), 0, s, p);
    break;
  case kFloat6E3M2:
    hipLaunchKernelGGL((QuantKernel<XF16, MODE, kFloat6E3M2>), g, dim3(kQBlock), 0, s, p);
    break;
  default: throw Unsupported("QuantizeLinear: no GPU kernel for this output dtype");
  }
}

template <bool XF16> void LaunchQX(const QuantParams &p, dim3 g, hipStream_t s) {
  if (p.mode == 0) LaunchQY<XF16, 0>(p, g, s);
  else if (p.mode == 1) LaunchQY<XF16, 1>(p, g, s);
  else LaunchQY<XF16, 2>(p, g, s);
}

// ---------------------------------------------------------------------------
// DynamicQuantizeLinear, two launches.  The min / max pass has kDqParts
// workgroups (fewer for small x), each writing one (min, max, non-finite)
// triple into structure-of-arrays partials [mn[P], mx[P], bad[P]].  The
// quantize pass covers x with one 8-element chunk per thread like
// QuantizeLinear; every workgroup issues its x loads, reduces the P partials
// itself while they land (min and max are order-independent, so all
// workgroups agree), derives scale and zero point with the reference's fp32
// operations and quantizes.  No atomics and no counters, so the pair can be
// captured in a graph.

constexpr int kDqBlock = 256;
constexpr int kDqParts = 512;
constexpr int kDqUnroll = 4;  // float4 loads in flight per thread in the min / max pass

__device__ __forceinline__ void BlockMinMax(float &mn, float &mx, float &bad) {
  __shared__ float red[3][kDqBlock / 64];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o));
    mx = fmaxf(mx, __shfl_xor(mx, o));
    bad = fmaxf(bad, __shfl_xor(bad, o));
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = mn;
    red[1][w] = mx;
    red[2][w] = bad;
  }
  __syncthreads();
  mn = red[0][0];
  mx = red[1][0];
  bad = red[2][0];
#pragma unroll
  for (int k = 1; k < kDqBlock / 64; ++k) {
    mn = fminf(mn, red[0][k]);
    mx = fmaxf(mx, red[1][k]);
    bad = fmaxf(bad, red[2][k]);
  }
}

__global__ __launch_bounds__(kDqBlock) void MinMaxKernel(const float *x, int64_t n, int vec, float *part) {
  // the range always contains 0 (:80-94): start from it
  float mn = 0.f, mx = 0.f, bad = 0.f;
  auto take = [&](float v) {
    if (!(__builtin_fabsf(v) <= FLT_MAX)) bad = 1.f;  // NaN or +-inf
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  };
  const int64_t t = (int64_t)blockIdx.x * kDqBlock + threadIdx.x;
  int64_t done = 0;
  if (vec) {
    const int64_t n4 = n >> 2;
    const int64_t stride = (int64_t)gridDim.x * kDqBlock * kDqUnroll;
    for (int64_t i = (int64_t)blockIdx.x * kDqBlock * kDqUnroll + threadIdx.x; i < n4; i += stride) {
      v4f v[kDqUnroll];
#pragma unroll
      for (int u = 0; u < kDqUnroll; ++u)
        v[u] = i + u * kDqBlock < n4 ? reinterpret_cast<const v4f *>(x)[i + u * kDqBlock] : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < kDqUnroll; ++u) {
        take(v[u][0]);
        take(v[u][1]);
        take(v[u][2]);
        take(v[u][3]);
      }
    }
    done = n4 << 2;
  }
  for (int64_t i = done + t; i < n; i += (int64_t)gridDim.x * kDqBlock) take(x[i]);
  BlockMinMax(mn, mx, bad);
  if (threadIdx.x == 0) {
    part[blockIdx.x] = mn;
    part[gridDim.x + blockIdx.x] = mx;
    part[2 * gridDim.x + blockIdx.x] = bad;
  }
}

__global__ __launch_bounds__(kDqBlock) void DynQuantKernel(const float *x, int64_t n, int vec, const float *part,
                                                           int nparts, uint8_t *y, float *y_scale,
                                                           uint8_t *y_zp) {
  const int64_t i0 = ((int64_t)blockIdx.x * kDqBlock + threadIdx.x) * kQPer;
  // workgroup-uniform, so the two load paths are a scalar branch
  const bool full = vec && ((int64_t)blockIdx.x + 1) * kDqBlock * kQPer <= n;
  float xv[kQPer];
  if (full) {
    const v4f a = LoadNt(x + i0), b = LoadNt(x + i0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xv[e] = a[e];
      xv[4 + e] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < kQPer; ++e) xv[e] = x[std::min<int64_t>(i0 + e, n - 1)];  // clamped ones are not stored
  }
  // The partials are loaded after x, all at once: the load counter retires
  // loads in issue order, so one wait covers x and the partials, which are
  // in flight together (a partial read twice changes no minimum or maximum).
  static_assert(kDqParts <= 2 * kDqBlock, "two partials per thread");
  float pmn[2], pmx[2], pbad[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int i = min((int)threadIdx.x + k * kDqBlock, nparts - 1);
    pmn[k] = part[i];
    pmx[k] = part[nparts + i];
    pbad[k] = part[2 * nparts + i];
  }
  float mn = fminf(pmn[0], pmn[1]), mx = fmaxf(pmx[0], pmx[1]), bad = fmaxf(pbad[0], pbad[1]);
  BlockMinMax(mn, mx, bad);
  // :96-106: scale = range / 255 (1 for an empty range), zero point
  // saturate(nearbyint(-min / scale))
  const float range = mx - mn;
  float scale = range == 0.f ? 1.f : range / 255.f;
  float zpf = __builtin_amdgcn_fmed3f(__builtin_rintf(-mn / scale), 0.f, 255.f);
  if (bad != 0.f) {
    scale = __builtin_nanf("");
    zpf = 0.f;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *y_scale = scale;
    *y_zp = (uint8_t)zpf;
  }
  if (i0 >= n) return;
  // :113-120: y = saturate(nearbyint(x / scale) + zero point)
  uint32_t code[kQPer];
#pragma unroll
  for (int e = 0; e < kQPer; ++e) {
    const float r = __builtin_rintf(xv[e] / scale) + zpf;
    code[e] = r != r ? 0u : (uint32_t)__builtin_amdgcn_fmed3f(r, 0.f, 255.f);
  }
  if (full) {
    v2i w;
#pragma unroll
    for (int k = 0; k < 2; ++k)
      w[k] = (int)(code[4 * k] | code[4 * k + 1] << 8 | code[4 * k + 2] << 16 | code[4 * k + 3] << 24);
    constexpr int kShare = kDqBlock * kQPer;
    __builtin_amdgcn_raw_buffer_store_b64(w, ShareRsrc(y, (int64_t)blockIdx.x * kShare, kShare),
                                          threadIdx.x * kQPer, 0, kWriteThrough);
  } else {
#pragma unroll
    for (int e = 0; e < kQPer; ++e)
      if (i0 + e < n) y[i0 + e] = (uint8_t)code[e];
  }
}

int DynQuantParts(int64_t n) {
  const int64_t per_block = (int64_t)kDqBlock * kDqUnroll * 4;
  return (int)std::min<int64_t>(kDqParts, std::max<int64_t>(1, (n + per_block - 1) / per_block));
}

}  // namespace

void LaunchQuantize(const QuantParams &p, hipStream_t s) {
  if (p.n == 0) return;
  const dim3 g((unsigned)((p.n + (int64_t)kQBlock * kQPer - 1) / ((int64_t)kQBlock * kQPer)));
  if (p.x_f16) LaunchQX<true>(p, g, s);
  else LaunchQX<false>(p, g, s);
}

size_t DynQuantScratchBytes(int64_t n) { return (size_t)DynQuantParts(n) * 3 * sizeof(float); }

void LaunchDynamicQuantize(const float *x, int64_t n, uint8_t *y, float *y_scale, uint8_t *y_zero_point,
                           void *scratch, hipStream_t s) {
  const int parts = DynQuantParts(n);
  const int vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
  float *part = static_cast<float *>(scratch);
  const int64_t chunk = (int64_t)kDqBlock * kQPer;
  hipLaunchKernelGGL(MinMaxKernel, dim3(parts), dim3(kDqBlock), 0, s, x, n, vec, part);
  hipLaunchKernelGGL(DynQuantKernel, dim3((unsigned)((n + chunk - 1) / chunk)), dim3(kDqBlock), 0, s, x, n, vec,
                     part, parts, y, y_scale, y_zero_point);
}

}  // namespace onnxl_amd
