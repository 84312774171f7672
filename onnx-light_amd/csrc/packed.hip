// DequantizePacked (onnx_core/runtime/dequantize_packed.cc) for the 32-value
// GGUF block formats q4_0, q4_1, q5_0, q5_1, q8_0, q8_1 and iq4_nl, and the
// 256-value k-quants q4_k and q6_k (below).  A 32-value block
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
#include <type_traits>

// The lattice grids of the IQ profiles, in constant memory (33 KB).
#define GGUF_CODEBOOK_QUAL static __constant__ const
#include "gguf_codebooks.h"

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

// ---------------------------------------------------------------------------
// q4_k and q6_k, 256-value blocks (dequantize_packed.cc:240-252): 8
// consecutive values i0 .. i0 + 7 (i0 % 8 == 0) of block p, with the
// reference's fp32 steps.
//  q4_k (144 bytes): fp16 d, fp16 dmin, 12 bytes of 6-bit scales / minima of
//   the eight 32-value sub-blocks, 128 code bytes: value i is nibble
//   (i / 32) % 2 of byte (i / 64) * 32 + i % 32; value = (d * scale) * q -
//   dmin * minimum.
//  q6_k (210 bytes): low nibbles, byte (i / 128) * 64 + i % 64, nibble
//   (i / 64) % 2; high 2 bits from byte 128 + (i / 128) * 32 + i % 32, field
//   (i / 32) % 4; int8 scale per 16 values at byte 192 + i / 16; fp16 d at
//   byte 208; value = (d * scale) * (q - 32).
//
// The NaN a step produces follows the reference's x86-64 build (SseMul,
// SseSub of device_codecs.hpp).

__device__ __forceinline__ void DecodeQ4K8(const uint8_t *p, int i0, float v[8]) {
  const float d = Half2(p), dmin = Half2(p + 2);
  const uint8_t *sc = p + 4;
  const int g = i0 >> 5;
  const int scale = g < 4 ? sc[g] & 63 : (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4);
  const int minimum = g < 4 ? sc[g + 4] & 63 : (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
  const float ds = SseMul(d, (float)scale);
  const float dm = SseMul(dmin, (float)minimum);
  const uint8_t *q = p + 16 + (i0 >> 6) * 32 + (i0 & 31);
  const int sh = 4 * (g & 1);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = SseSub(SseMul(ds, (float)((q[e] >> sh) & 15)), dm);
}

__device__ __forceinline__ void DecodeQ6K8(const uint8_t *p, int i0, float v[8]) {
  const float d = Half2(p + 208);
  const float ds = SseMul(d, (float)(int8_t)p[192 + (i0 >> 4)]);
  const uint8_t *ql = p + (i0 >> 7) * 64 + (i0 & 63);
  const uint8_t *qh = p + 128 + (i0 >> 7) * 32 + (i0 & 31);
  const int shl = 4 * ((i0 >> 6) & 1), shh = 2 * ((i0 >> 5) & 3);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    v[e] = SseMul(ds, (float)((((ql[e] >> shl) & 15) | (((qh[e] >> shh) & 3) << 4)) - 32));
}

template <int TYPE> struct KLayout;
template <> struct KLayout<10> { static constexpr int bytes = 84; };   // q2_k
template <> struct KLayout<11> { static constexpr int bytes = 110; };  // q3_k
template <> struct KLayout<12> { static constexpr int bytes = 144; };  // q4_k
template <> struct KLayout<13> { static constexpr int bytes = 176; };  // q5_k
template <> struct KLayout<14> { static constexpr int bytes = 210; };  // q6_k
template <> struct KLayout<23> { static constexpr int bytes = 136; };  // iq4_xs

template <int TYPE> __device__ __forceinline__ void DecodeK8(const uint8_t *p, int i0, float v[8]) {
  if constexpr (TYPE == 12) DecodeQ4K8(p, i0, v);
  else DecodeQ6K8(p, i0, v);
}

// 32 threads per block, 8 consecutive values each: thread t writes values
// 8t .. 8t + 7 of the output, as the 32-value kernel does.
template <int TYPE, int OUT>
__global__ __launch_bounds__(kPkThreads) void DequantPackedKKernel(const uint8_t *__restrict__ x, int64_t nblocks,
                                                                   void *__restrict__ y, int vec) {
  const int64_t t = (int64_t)blockIdx.x * kPkThreads + threadIdx.x;
  if (t >= nblocks * 32) return;
  const int64_t b = t >> 5;
  const int i0 = (int)(t & 31) * 8;
  float v[8];
  DecodeK8<TYPE>(x + b * KLayout<TYPE>::bytes, i0, v);
  StoreEight<OUT>(y, b * 256 + i0, v, vec != 0);
}

// ---------------------------------------------------------------------------
// The other profiles without codebooks (dequantize_packed.cc:199-279):
// q2_k, q3_k, q5_k, q8_k, iq4_xs, tq1_0, tq2_0 (256 values), mxfp4 (32),
// nvfp4 and q2_0 (64), q1_0 (128).  A thread computes 8 consecutive values
// of one block, value by value with byte reads (the block stays in L1 for
// the threads that share it), each fp32 step rounded on its own with the
// x86-64 NaN results.  Layouts and formulas are those of the oracle's
// pk_decode_ext.
template <int TYPE> struct XLayout;
template <> struct XLayout<10> { static constexpr int bytes = 84, values = 256; };   // q2_k
template <> struct XLayout<11> { static constexpr int bytes = 110, values = 256; };  // q3_k
template <> struct XLayout<13> { static constexpr int bytes = 176, values = 256; };  // q5_k
template <> struct XLayout<15> { static constexpr int bytes = 292, values = 256; };  // q8_k
template <> struct XLayout<23> { static constexpr int bytes = 136, values = 256; };  // iq4_xs
template <> struct XLayout<34> { static constexpr int bytes = 54, values = 256; };   // tq1_0
template <> struct XLayout<35> { static constexpr int bytes = 66, values = 256; };   // tq2_0
template <> struct XLayout<39> { static constexpr int bytes = 17, values = 32; };    // mxfp4
template <> struct XLayout<40> { static constexpr int bytes = 36, values = 64; };    // nvfp4
template <> struct XLayout<41> { static constexpr int bytes = 18, values = 128; };   // q1_0
template <> struct XLayout<42> { static constexpr int bytes = 18, values = 64; };    // q2_0

__constant__ int kFp4Twice[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

// value i of grouped bit planes: 8 / BITS planes of GROUP bytes
template <int BITS, int GROUP> __device__ __forceinline__ int Planes(const uint8_t *p, int i) {
  constexpr int kPlanes = 8 / BITS;
  return (p[(i / (kPlanes * GROUP)) * GROUP + i % GROUP] >> (BITS * ((i / GROUP) % kPlanes))) & ((1 << BITS) - 1);
}

template <int TYPE> __device__ __forceinline__ float DecodeX(const uint8_t *p, int i) {
  if constexpr (TYPE == 10) {  // q2_k
    const int g = i / 16;
    const float dq = SseMul(SseMul(Half2(p + 80), (float)(p[g] & 15)), (float)Planes<2, 32>(p + 16, i));
    return SseSub(dq, SseMul(Half2(p + 82), (float)(p[g] >> 4)));
  } else if constexpr (TYPE == 11) {  // q3_k
    const int g = i / 16;
    const int scale = (Planes<4, 8>(p + 96, g) | (Planes<2, 4>(p + 104, g) << 4)) - 32;
    const int q = Planes<2, 32>(p + 32, i) - (1 - Planes<1, 32>(p, i)) * 4;
    return SseMul(SseMul(Half2(p + 108), (float)scale), (float)q);
  } else if constexpr (TYPE == 13) {  // q5_k
    const uint8_t *sc = p + 4;
    const int g = i / 32;
    const int scale = g < 4 ? sc[g] & 63 : (sc[g + 4] & 15) | ((sc[g - 4] >> 6) << 4);
    const int minimum = g < 4 ? sc[g + 4] & 63 : (sc[g + 4] >> 4) | ((sc[g] >> 6) << 4);
    const int q = Planes<4, 32>(p + 48, i) | (Planes<1, 32>(p + 16, i) << 4);
    return SseSub(SseMul(SseMul(Half2(p), (float)scale), (float)q), SseMul(Half2(p + 2), (float)minimum));
  } else if constexpr (TYPE == 15) {  // q8_k: fp32 d
    const uint32_t bits = (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
    return SseMul(__builtin_bit_cast(float, bits), (float)(int8_t)p[4 + i]);
  } else if constexpr (TYPE == 23) {  // iq4_xs
    const int g = i / 32;
    const uint32_t high = (uint32_t)p[2] | (uint32_t)p[3] << 8;
    const int scale = (((p[4 + g / 2] >> (4 * (g % 2))) & 15) | (int)(((high >> (2 * g)) & 3u) << 4)) - 32;
    return SseMul(SseMul(Half2(p), (float)scale), (float)kIq4Values[Planes<4, 16>(p + 8, i)]);
  } else if constexpr (TYPE == 34) {  // tq1_0: base-3 digits
    const int start = i < 160 ? 0 : (i < 240 ? 32 : 48);
    const int width = i < 160 ? 32 : (i < 240 ? 16 : 4);
    const int offset = i < 160 ? i : (i < 240 ? i - 160 : i - 240);
    const int digit = offset / width;
    const int power = digit == 0 ? 1 : digit == 1 ? 3 : digit == 2 ? 9 : digit == 3 ? 27 : 81;
    const int q = ((p[start + offset % width] * power) & 255) * 3 / 256 - 1;
    return SseMul(Half2(p + 52), (float)q);
  } else if constexpr (TYPE == 35) {  // tq2_0
    return SseMul(Half2(p + 64), (float)(Planes<2, 32>(p, i) - 1));
  } else if constexpr (TYPE == 39) {  // mxfp4: e8m0 scale byte
    const uint32_t e = p[0];
    const uint32_t bits = e <= 1 ? 0x00200000u << e : (e - 1) << 23;
    return SseMul(__builtin_bit_cast(float, bits), (float)kFp4Twice[Planes<4, 16>(p + 1, i)]);
  } else if constexpr (TYPE == 40) {  // nvfp4: ue4m3 scale per 16 values
    const int g = i / 16, e = p[g], exponent = (e >> 3) & 15, mantissa = e & 7;
    const float scale = e == 0 || e == 127 ? 0.f
                        : exponent == 0    ? ldexpf((float)mantissa, -10)
                                           : ldexpf(1.f + (float)mantissa / 8.f, exponent - 8);
    return SseMul(scale, (float)kFp4Twice[Planes<4, 8>(p + 4 + 8 * g, i % 16)]);
  } else if constexpr (TYPE == 41) {  // q1_0: a sign bit per value
    // no arithmetic touches d, so its fp32 bits are the reference's software
    // conversion bit for bit: a signaling NaN stays signaling (the hardware
    // conversion would quiet it), and -d flips the sign bit only
    const uint32_t h = (uint32_t)p[0] | (uint32_t)p[1] << 8;
    const uint32_t bits = (h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)
                              ? ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13)
                              : __builtin_bit_cast(uint32_t, Half2(p));
    return __builtin_bit_cast(float, (p[2 + i / 8] >> (i % 8)) & 1 ? bits : bits ^ 0x80000000u);
  } else {  // q2_0
    return SseMul(Half2(p), (float)(Planes<2, 1>(p + 2, i) - 1));
  }
}

template <int TYPE, int OUT>
__global__ __launch_bounds__(kPkThreads) void DequantPackedXKernel(const uint8_t *__restrict__ x, int64_t nblocks,
                                                                   void *__restrict__ y, int vec) {
  constexpr int kV = XLayout<TYPE>::values, kTpb = kV / 8;  // threads per block
  const int64_t t = (int64_t)blockIdx.x * kPkThreads + threadIdx.x;
  if (t >= nblocks * kTpb) return;
  const int64_t b = t / kTpb;
  const int i0 = (int)(t % kTpb) * 8;
  const uint8_t *p = x + b * XLayout<TYPE>::bytes;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = DecodeX<TYPE>(p, i0 + e);
  StoreEight<OUT>(y, b * kV + i0, v, vec != 0);  // thread t writes values 8t .. 8t + 7
}

// ---------------------------------------------------------------------------
// The codebook profiles (dequantize_packed.cc:84-170): iq2_xxs, iq2_xs,
// iq2_s, iq3_xxs, iq3_s, iq1_s, iq1_m.  A 256-value block is 32 octets; a
// thread decodes octet o = 4 g + l of one block (values 8 o .. 8 o + 7):
// grid row(s) from gguf_codebooks.h, one sign bit per value (7 bits completed
// to even parity for iq2_xxs / iq2_xs / iq3_xxs), a per-octet scale; every
// fp32 product and sum rounded on its own, with the x86-64 NaN results.
// Field positions are those of the oracle's pk_decode_iq.
template <int TYPE> struct IqLayout;
template <> struct IqLayout<16> { static constexpr int bytes = 66; };   // iq2_xxs
template <> struct IqLayout<17> { static constexpr int bytes = 74; };   // iq2_xs
template <> struct IqLayout<22> { static constexpr int bytes = 82; };   // iq2_s
template <> struct IqLayout<18> { static constexpr int bytes = 98; };   // iq3_xxs
template <> struct IqLayout<21> { static constexpr int bytes = 110; };  // iq3_s
template <> struct IqLayout<19> { static constexpr int bytes = 50; };   // iq1_s
template <> struct IqLayout<29> { static constexpr int bytes = 56; };   // iq1_m

__device__ __forceinline__ uint32_t U16At(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8; }
__device__ __forceinline__ uint32_t U32At(const uint8_t *p) { return U16At(p) | U16At(p + 2) << 16; }
// +-1 for sign bit j; `parity`: 7 stored bits, the eighth makes the count even
__device__ __forceinline__ float SignBit(uint32_t bits, int j, bool parity) {
  if (parity) bits |= (uint32_t)(__builtin_popcount(bits) & 1) << 7;
  return (bits >> j) & 1u ? -1.f : 1.f;
}
// lane j of a grid row (one signed byte per lane)
__device__ __forceinline__ float Lane(uint64_t row, int j) { return (float)(int8_t)(uint8_t)(row >> (8 * j)); }

template <int TYPE> __device__ __forceinline__ void DecodeIq8(const uint8_t *p, int o, float v[8]) {
  const int g = o >> 2, l = o & 3;
  if constexpr (TYPE == 16 || TYPE == 17 || TYPE == 22) {
    uint32_t index, signs;
    float s;
    if constexpr (TYPE == 16) {
      const uint32_t w = U32At(p + 6 + 8 * g);
      index = p[2 + 8 * g + l];
      signs = (w >> (7 * l)) & 127u;
      s = (float)(w >> 28);
    } else if constexpr (TYPE == 17) {
      const uint32_t w = U16At(p + 2 + 2 * o);
      index = w & 511u;
      signs = w >> 9;
      s = (float)((p[66 + g] >> (4 * (l >> 1))) & 15);
    } else {
      index = p[2 + o] | (((uint32_t)p[66 + g] >> (2 * l)) & 3u) << 8;
      signs = p[34 + o];
      s = (float)((p[74 + g] >> (4 * (l >> 1))) & 15);
    }
    const float scale = SseMul(SseMul(Half2(p), 0.5f + s), 0.25f);
    const uint64_t row = TYPE == 16 ? kGgufIq2xxs[index] : (TYPE == 17 ? kGgufIq2xs[index] : kGgufIq2s[index]);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = SseMul(SseMul(scale, Lane(row, j)), SignBit(signs, j, TYPE != 22));
  } else if constexpr (TYPE == 18 || TYPE == 21) {
    uint32_t signs;
    float scale;
    if constexpr (TYPE == 18) {
      const uint32_t w = U32At(p + 66 + 4 * g);
      signs = (w >> (7 * l)) & 127u;
      scale = SseMul(SseMul(Half2(p), 0.5f + (float)(w >> 28)), 0.5f);
    } else {
      signs = p[74 + o];
      scale = SseMul(Half2(p), (float)(1 + 2 * ((p[106 + (g >> 1)] >> (4 * (g & 1))) & 15)));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t index = p[2 + 2 * o + h];
      if constexpr (TYPE == 21) index |= (((uint32_t)p[66 + g] >> (2 * l + h)) & 1u) << 8;
      const uint64_t row = TYPE == 18 ? kGgufIq3xxs[index] : kGgufIq3s[index];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[4 * h + j] = SseMul(SseMul(scale, Lane(row, j)), SignBit(signs, 4 * h + j, TYPE == 18));
    }
  } else {  // iq1_s, iq1_m
    uint32_t index;
    int mult;
    float d, delta;
    if constexpr (TYPE == 19) {
      const uint32_t h = U16At(p + 34 + 2 * g);
      d = Half2(p);
      index = p[2 + o] | ((h >> (3 * l)) & 7u) << 8;
      mult = 2 * (int)((h >> 12) & 7u) + 1;
      delta = h & 0x8000u ? -0.125f : 0.125f;
    } else {
      const uint32_t w0 = U16At(p + 48), w1 = U16At(p + 50), w2 = U16At(p + 52), w3 = U16At(p + 54);
      d = F16ToF32((uint16_t)((w0 >> 12) | (w1 >> 12) << 4 | (w2 >> 12) << 8 | (w3 >> 12) << 12));
      const uint32_t nib = (p[32 + (o >> 1)] >> (4 * (o & 1))) & 15u;
      index = p[o] | (nib & 7u) << 8;
      const uint32_t ws = (g >> 1) == 0 ? w0 : (g >> 1) == 1 ? w1 : (g >> 1) == 2 ? w2 : w3;
      mult = 2 * (int)((ws >> (6 * (g & 1) + 3 * (l >> 1))) & 7u) + 1;
      delta = nib & 8u ? -0.125f : 0.125f;
    }
    const float scale = SseMul(d, (float)mult);
    const uint64_t row = kGgufIq1s[index];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = SseMul(scale, Lane(row, j) + delta);
  }
}

template <int TYPE, int OUT>
__global__ __launch_bounds__(kPkThreads) void DequantPackedIqKernel(const uint8_t *__restrict__ x, int64_t nblocks,
                                                                    void *__restrict__ y, int vec) {
  const int64_t t = (int64_t)blockIdx.x * kPkThreads + threadIdx.x;
  if (t >= nblocks * 32) return;
  const int64_t b = t >> 5;
  const int o = (int)(t & 31);
  float v[8];
  DecodeIq8<TYPE>(x + b * IqLayout<TYPE>::bytes, o, v);
  StoreEight<OUT>(y, b * 256 + 8 * o, v, vec != 0);  // thread t writes values 8t .. 8t + 7
}

template <int TYPE> void LaunchPkIqOut(const uint8_t *x, int64_t nblocks, int out, void *y, int vec, hipStream_t s) {
  const dim3 g((unsigned)((nblocks * 32 + kPkThreads - 1) / kPkThreads));
  switch (out) {
  case kFloat: hipLaunchKernelGGL((DequantPackedIqKernel<TYPE, kFloat>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kFloat16: hipLaunchKernelGGL((DequantPackedIqKernel<TYPE, kFloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kBfloat16: hipLaunchKernelGGL((DequantPackedIqKernel<TYPE, kBfloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  default: hipLaunchKernelGGL((DequantPackedIqKernel<TYPE, kDouble>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  }
}

template <int TYPE> void LaunchPkXOut(const uint8_t *x, int64_t nblocks, int out, void *y, int vec, hipStream_t s) {
  const int64_t threads = nblocks * (XLayout<TYPE>::values / 8);
  const dim3 g((unsigned)((threads + kPkThreads - 1) / kPkThreads));
  switch (out) {
  case kFloat: hipLaunchKernelGGL((DequantPackedXKernel<TYPE, kFloat>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kFloat16: hipLaunchKernelGGL((DequantPackedXKernel<TYPE, kFloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kBfloat16: hipLaunchKernelGGL((DequantPackedXKernel<TYPE, kBfloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  default: hipLaunchKernelGGL((DequantPackedXKernel<TYPE, kDouble>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  }
}

template <int TYPE> void LaunchPkKOut(const uint8_t *x, int64_t nblocks, int out, void *y, int vec, hipStream_t s) {
  const dim3 g((unsigned)((nblocks * 32 + kPkThreads - 1) / kPkThreads));
  switch (out) {
  case kFloat: hipLaunchKernelGGL((DequantPackedKKernel<TYPE, kFloat>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kFloat16: hipLaunchKernelGGL((DequantPackedKKernel<TYPE, kFloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  case kBfloat16: hipLaunchKernelGGL((DequantPackedKKernel<TYPE, kBfloat16>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  default: hipLaunchKernelGGL((DequantPackedKKernel<TYPE, kDouble>), g, dim3(kPkThreads), 0, s, x, nblocks, y, vec); break;
  }
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

// ---------------------------------------------------------------------------
// Fused q4_0 GEMV: y[m, n] = sum_k a[m, k] * W[n, k] with W = the FLOAT16
// DequantizePacked values of a gguf:q4_0 [N, K] weight (ggml layout: the
// blocks of output n run along k, contiguous).  One wave per output n; each
// lane takes pairs of blocks (36 bytes, dword aligned when K % 64 == 0).
// Code byte j holds elements j (low nibble) and j + 16 (high nibble) of its
// block, so the two form one fp16 pair: (0x6400 | nibble) is 1024 + q exactly,
// adding -1032 gives q - 8 exactly, and the packed fp16 multiply by d rounds
// d * (q - 8) to FLOAT16 exactly as the DequantizePacked -> FLOAT16 chain
// does.  v_dot2_f32_f16 then accumulates with the activation pair
// (a[k + j], a[k + 16 + j]) in fp32.
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t AsH2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }

// Each wave computes kGvCols consecutive outputs at once, so the activation
// pairs it loads for a block serve all of them (loading and pairing the
// activation per output cost as much as the weight stream).  The
// workgroup's 4 * kGvCols weight rows are contiguous; they are staged through
// LDS in chunks of kGvChunkK values per row with 16-byte loads of
// consecutive addresses, and each lane reads its block pairs from there (a
// 36-byte stride: no bank conflicts).
constexpr int kGvCols = 4;
constexpr int kGvRows = 4 * kGvCols;              // outputs per workgroup
constexpr int kGvChunkK = 4096;                   // values per row per chunk: 64 block pairs, one per lane
constexpr int kGvRowBytes = kGvChunkK / 32 * 18;  // 2304

// Stages `rows` rows of `bytes` bytes (row r at src + r * stride) into LDS at
// r * bytes, with up to eight loads in flight per thread before their LDS
// stores: 16-byte pieces when every row start is 16-byte aligned, else dwords.
__device__ __forceinline__ void StageRows(uint32_t *stage, const uint8_t *src, int64_t stride, int rows, int bytes) {
  typedef int v4i __attribute__((ext_vector_type(4)));
  if ((bytes & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (stride & 15) == 0) {
    const int per_row = bytes / 16, total = rows * per_row;
    for (int i0 = threadIdx.x; i0 < total; i0 += 8 * 256) {
      v4i v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 256 * k;
        if (i < total) {
          const int r = i / per_row;
          v[k] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(src + r * stride) + (i - r * per_row));
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 256 * k;
        if (i < total) {
          const int r = i / per_row;
          reinterpret_cast<v4i *>(stage)[(r * bytes) / 16 + (i - r * per_row)] = v[k];
        }
      }
    }
  } else {
    const int per_row = bytes / 4, total = rows * per_row;
    for (int i0 = threadIdx.x; i0 < total; i0 += 8 * 256) {
      uint32_t v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 256 * k;
        if (i < total) {
          const int r = i / per_row;
          v[k] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(src + r * stride) + (i - r * per_row));
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int i = i0 + 256 * k;
        if (i < total) {
          const int r = i / per_row;
          stage[(r * bytes) / 4 + (i - r * per_row)] = v[k];
        }
      }
    }
  }
}

template <int M>
__global__ __launch_bounds__(256) void GemvQ40Kernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ w,
                                                     int64_t N, int64_t K, uint16_t *__restrict__ y) {
  __shared__ __align__(16) uint32_t stage[kGvRows * kGvRowBytes / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kGvRows;
  const int rows = (int)std::min<int64_t>(kGvRows, N - n0);
  const int64_t row_bytes = K / 32 * 18;
  float acc[kGvCols][M];
#pragma unroll
  for (int c = 0; c < kGvCols; ++c)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[c][m] = 0.f;
  const h2_t kMinus1032 = AsH2(0xE408E408u);
  for (int64_t kc = 0; kc < K; kc += kGvChunkK) {
    const int64_t chunk_k = std::min<int64_t>(kGvChunkK, K - kc);
    const int chunk_bytes = (int)(chunk_k / 32 * 18);  // a multiple of 36
    // stage rows [n0, n0 + rows) of this chunk: row r at stage byte r * chunk_bytes
    const uint8_t *src = w + n0 * row_bytes + kc / 32 * 18;
    StageRows(stage, src, row_bytes, rows, chunk_bytes);
    __syncthreads();
    for (int64_t jj = lane; jj < chunk_k / 64; jj += 64) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        // weight pairs (element j, element j + 16) of this block for each column
        h2_t wp[kGvCols][16];
#pragma unroll
        for (int c = 0; c < kGvCols; ++c) {
          const int r = wave * kGvCols + c;
          const int rr = r < rows ? r : 0;  // rows past N decode row 0 and are not stored
          const uint32_t *sp = stage + (rr * chunk_bytes + jj * 36 + 18 * blk - 2 * blk) / 4;
          // the block starts 18 * blk bytes into the pair (2 bytes into a dword
          // for blk 1): the 5 dwords from the one at or before its start cover
          // it, and stay inside the 36-byte pair; q[5] only feeds an unused
          // high word
          uint32_t q[6];
#pragma unroll
          for (int i = 0; i < 5; ++i) q[i] = sp[i];
          q[5] = q[4];
          const int sh = blk ? 2 : 0;  // byte offset of the block in q[0]
          const uint32_t q0 = sh ? __builtin_amdgcn_alignbyte(q[1], q[0], 2) : q[0];
          const uint32_t dbits = q0 & 0xffffu;
          const h2_t dd = AsH2(dbits | dbits << 16);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int byte = sh + 2 + 4 * t;  // first code byte of this dword within q
            const uint32_t lo = q[byte >> 2], hi = q[(byte >> 2) + 1];
            const uint32_t cw = (byte & 3) ? __builtin_amdgcn_alignbyte(hi, lo, byte & 3) : lo;
            const uint32_t nl = cw & 0x0F0F0F0Fu, nh = (cw >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              // bytes: [lo_e, 0, hi_e, 0] | 0x64006400
              const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + e) << 16) | (uint32_t)e;
              const uint32_t bits = __builtin_amdgcn_perm(nh, nl, sel) | 0x64006400u;
              wp[c][4 * t + e] = (AsH2(bits) + kMinus1032) * dd;
            }
          }
        }
        const int64_t k0 = (2 * (kc / 64 + jj) + blk) * 32;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint32_t *ar = reinterpret_cast<const uint32_t *>(a + m * K + k0);
          uint32_t al[8], ah[8];  // a[k0 + 0..15] and a[k0 + 16..31] as half pairs
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            al[i] = ar[i];
            ah[i] = ar[8 + i];
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const h2_t p0 = AsH2(__builtin_amdgcn_perm(ah[i], al[i], 0x05040100u));  // (a[2i], a[16 + 2i])
            const h2_t p1 = AsH2(__builtin_amdgcn_perm(ah[i], al[i], 0x07060302u));  // (a[2i+1], a[17 + 2i])
#pragma unroll
            for (int c = 0; c < kGvCols; ++c) {
              acc[c][m] = __builtin_amdgcn_fdot2(p0, wp[c][2 * i], acc[c][m], false);
              acc[c][m] = __builtin_amdgcn_fdot2(p1, wp[c][2 * i + 1], acc[c][m], false);
            }
          }
        }
      }
    }
    __syncthreads();  // the stage is rewritten by the next chunk
  }
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) {
    const int64_t n = n0 + wave * kGvCols + c;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = acc[c][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0 && n < N) y[m * N + n] = F32ToF16(s);
    }
  }
}

// Fused q8_0 GEMV, as the q4_0 one: y[m, n] = sum_k a[m, k] * W[n, k] with W
// the FLOAT16 decode of a gguf:q8_0 [N, K] weight (34-byte blocks: fp16 d and
// 32 int8 codes).  Chunks of 2048 values give one block per lane (64 blocks
// per row); a lane reads its block as the 9 dwords from the one at or before
// its start (34-byte stride, 0 or 2 bytes into the dword).  Codes pair as
// consecutive elements: (b ^ 0x80) | 0x6400 is 1152 + q exactly, one XOR
// with 0x64806480 for two codes placed in bytes 0 and 2; adding -1152 gives q
// and the packed multiply by d rounds d * q to FLOAT16 as the chain does.
constexpr int kGv8ChunkK = 2048;
constexpr int kGv8RowBytes = kGv8ChunkK / 32 * 34;  // 2176

template <int M>
__global__ __launch_bounds__(256) void GemvQ80Kernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ w,
                                                     int64_t N, int64_t K, uint16_t *__restrict__ y) {
  __shared__ __align__(16) uint32_t stage[kGvRows * kGv8RowBytes / 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kGvRows;
  const int rows = (int)std::min<int64_t>(kGvRows, N - n0);
  const int64_t row_bytes = K / 32 * 34;
  float acc[kGvCols][M];
#pragma unroll
  for (int c = 0; c < kGvCols; ++c)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[c][m] = 0.f;
  const h2_t kMinus1152 = AsH2(0xE480E480u);
  for (int64_t kc = 0; kc < K; kc += kGv8ChunkK) {
    const int64_t chunk_k = std::min<int64_t>(kGv8ChunkK, K - kc);
    const int cb = (int)(chunk_k / 32 * 34);  // a multiple of 68
    const uint8_t *src = w + n0 * row_bytes + kc / 32 * 34;
    StageRows(stage, src, row_bytes, rows, cb);
    __syncthreads();
    const int64_t jb = lane;  // block of this lane within the chunk
    if (jb < chunk_k / 32) {
      h2_t wp[kGvCols][16];  // weight pairs (element 2i, element 2i + 1) per column
#pragma unroll
      for (int c = 0; c < kGvCols; ++c) {
        const int r = wave * kGvCols + c;
        const int rr = r < rows ? r : 0;  // rows past N decode row 0 and are not stored
        const int byte0 = rr * cb + (int)jb * 34;  // 2-byte aligned
        const uint32_t *sp = stage + (byte0 >> 2);
        const int sh = byte0 & 3;  // 0 or 2
        uint32_t q[10];
#pragma unroll
        for (int i = 0; i < 9; ++i) q[i] = sp[i];  // 36 bytes; the block ends at or before the last
        q[9] = q[8];
        const uint32_t dbits = __builtin_amdgcn_alignbyte(q[1], q[0], sh) & 0xffffu;
        const h2_t dd = AsH2(dbits | dbits << 16);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int at = sh + 2 + 4 * t;  // code bytes 4t .. 4t + 3, at bytes into q
          const uint32_t cw = __builtin_amdgcn_alignbyte(q[(at >> 2) + 1], q[at >> 2], at & 3);
          // [b0, 0, b1, 0] and [b2, 0, b3, 0], then the offset into 1152 + q
          const uint32_t lo = __builtin_amdgcn_perm(0u, cw, 0x0c010c00u) ^ 0x64806480u;
          const uint32_t hi = __builtin_amdgcn_perm(0u, cw, 0x0c030c02u) ^ 0x64806480u;
          wp[c][2 * t] = (AsH2(lo) + kMinus1152) * dd;
          wp[c][2 * t + 1] = (AsH2(hi) + kMinus1152) * dd;
        }
      }
      const int64_t k0 = kc + jb * 32;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint32_t *ar = reinterpret_cast<const uint32_t *>(a + m * K + k0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const h2_t ap = AsH2(ar[i]);  // (a[2i], a[2i + 1])
#pragma unroll
          for (int c = 0; c < kGvCols; ++c) acc[c][m] = __builtin_amdgcn_fdot2(ap, wp[c][i], acc[c][m], false);
        }
      }
    }
    __syncthreads();  // the stage is rewritten by the next chunk
  }
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) {
    const int64_t n = n0 + wave * kGvCols + c;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = acc[c][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0 && n < N) y[m * N + n] = F32ToF16(s);
    }
  }
}

// Streamed q4_0 / q8_0 GEMV for K % 256 == 0 (every row starts 16-byte
// aligned) and a weight below 2 GiB, the same sums as the two kernels above
// in another order.  A workgroup is one wave and computes 4 consecutive
// outputs.  It streams its 4 rows in chunks of 128 q4_0 / 64 q8_0 blocks
// (2304 / 2176 bytes of each row): a chunk is requested at once as nine
// 16-byte loads per lane (load j: lanes 16r .. 16r + 15 read bytes
// 256j .. 256j + 255 of row r's chunk) and decoded in 4 steps, each as soon
// as the loads that hold its blocks have landed.  A landed load is copied to
// the wave's LDS window and its register is reloaded with the same piece of
// the next chunk, so the next chunk streams while this one is decoded.  The
// activations of a step are requested right after the weight pieces the
// step needs: vector memory loads complete in order, so the wait for them
// never covers a later weight piece.  The wave owns its LDS window, so no
// workgroup barrier is needed (a wave's LDS operations execute in order).
//
// Per lane and output, a step decodes 8 code bytes of one block: q4_0 half a
// block (values 8h .. 8h + 7 from the low nibbles, 16 + 8h .. 23 + 8h from
// the high ones), q8_0 a quarter (values 8h .. 8h + 7), read as three
// aligned LDS dwords and funnel-shifted (a block starts 0 or 2 bytes into a
// dword).  q4_0: v_perm spreads two code bytes into the low bytes of a half
// pair, and one AND-OR per nibble pair forms 1024 + q (low nibbles, bits
// 0-3) or 64 + q (high nibbles, bits 4-7, where the unit step of that
// exponent is 1); subtracting 1032 or 72 gives q - 8 exactly.  q8_0: XOR
// 0x80 per byte gives q + 128, v_perm places two of them under a 0x64 high
// byte (1152 + q) and subtracting 1152 gives q.  The packed multiply by d
// then rounds d * (q - 8) or d * q to FLOAT16 as the DequantizePacked ->
// FLOAT16 chain does.  The pairs are consecutive values, as are the fp16
// pairs of the 16-byte activation loads, and v_dot2_f32_f16 accumulates them
// in fp32.
// (x & mask) | bits in one v_and_or_b32 (the compiler splits it otherwise)
__device__ __forceinline__ uint32_t AndOr(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(bits));
  return r;
}

// the dword at byte offset o (o % 4 == 0) of an LDS stage s
__device__ __forceinline__ uint32_t LdsDword(const uint8_t *s, int o) {
  return *reinterpret_cast<const uint32_t *>(s + o);
}

template <int TYPE> struct Q0Stream;
template <> struct Q0Stream<2> { static constexpr int block = 18, lanes_per_block = 2, chunk_blocks = 128; };
template <> struct Q0Stream<8> { static constexpr int block = 34, lanes_per_block = 4, chunk_blocks = 64; };

constexpr int kQsRows = 4;    // outputs per workgroup (one wave)
constexpr int kQsPieces = 9;  // 16-byte loads per lane per chunk: 256 bytes of each row per load
constexpr int kQsSteps = 4;   // decode steps per chunk

// the last weight piece (load index) holding bytes of decode step s
template <int TYPE> constexpr int QsLastPiece(int s) {
  return ((s + 1) * (64 / Q0Stream<TYPE>::lanes_per_block) * Q0Stream<TYPE>::block - 1) / 256;
}

template <int TYPE, int M>
__global__ __launch_bounds__(64) void GemvQ0StreamKernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ w,
                                                         int64_t N, int64_t K, uint16_t *__restrict__ y) {
  using L = Q0Stream<TYPE>;
  constexpr int kBB = L::block;
  constexpr int kChunk = L::chunk_blocks * kBB;         // bytes of a row per chunk
  constexpr int kStepBlocks = 64 / L::lanes_per_block;  // blocks of a row per step
  constexpr int kStepBytes = kStepBlocks * kBB;
  constexpr int kActLoads = TYPE == 2 ? 2 : 1;          // 16-byte activation loads per step and row of a
  static_assert(kStepBlocks * kQsSteps == L::chunk_blocks, "4 steps per chunk");
  static_assert(kChunk % 16 == 0 && kChunk <= kQsPieces * 256 && kChunk > (kQsPieces - 1) * 256, "9 loads per chunk");
  static_assert(kStepBlocks % 2 == 0, "a lane's blocks keep one alignment in every step");
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  // +16: the third code dword of the window's last block lies past it (read, never used)
  __shared__ __align__(16) uint8_t stage[kQsRows * kChunk + 16];
  const int lane = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * kQsRows;
  const int64_t nb = K / 32;
  const int64_t row_bytes = nb * kBB;  // a multiple of 16
  const int nchunks = (int)((nb + L::chunk_blocks - 1) / L::chunk_blocks);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), (short)0, (int)(N * row_bytes), 0x00020000);

  // loads: lane -> (row lr, 16-byte word lw of each 256-byte piece); rows past N reload the last
  const int lr = lane >> 4, lw = lane & 15;
  const uint32_t lbase = (uint32_t)((n0 + lr < N ? n0 + lr : N - 1) * row_bytes) + 16u * (uint32_t)lw;
  auto load = [&](int c, int j) __attribute__((always_inline)) -> v4u {
    const int off = 256 * j + 16 * lw;
    const bool ok = off < kChunk && (int64_t)c * kChunk + off < row_bytes;
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                       rs, ok ? lbase + (uint32_t)(c * kChunk + 256 * j) : 0x80000000u, 0, 2));
  };
  auto put = [&](int j, const v4u &v) __attribute__((always_inline)) {
    const int off = 256 * j + 16 * lw;
    if (off < kChunk) *reinterpret_cast<v4u *>(&stage[lr * kChunk + off]) = v;
  };

  // decode: lane -> (block bl of each step, part h of the block's codes)
  const int bl = lane / L::lanes_per_block, h = lane % L::lanes_per_block;
  const int dofs = (bl * kBB) & ~3;                // the dword holding d
  const int cofs = (bl * kBB + 2 + 8 * h) & ~3;    // the first of the three dwords holding the 8 code bytes
  const uint32_t dsel = bl & 1 ? 0x03020302u : 0x01000100u;  // d in the high / low half, twice
  const uint32_t csh = bl & 1 ? 0u : 16u;
  // activations of the lane's values for step s of chunk c (clamped in a partial chunk's idle lanes)
  auto act = [&](int c, int s, v4u (&av)[kActLoads][M]) __attribute__((always_inline)) {
    const int64_t b = (int64_t)c * L::chunk_blocks + s * kStepBlocks + bl;
    const int64_t k0 = (b < nb ? b : 0) * 32 + 8 * h;
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int t = 0; t < kActLoads; ++t) av[t][m] = *reinterpret_cast<const v4u *>(a + m * K + k0 + 16 * t);
  };

  float acc[kQsRows][M];
#pragma unroll
  for (int r = 0; r < kQsRows; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  const h2_t kM1032 = AsH2(0xE408E408u), kM72 = AsH2(0xD480D480u), kM1152 = AsH2(0xE480E480u);

  v4u wr[kQsPieces];
  v4u av[kQsSteps][kActLoads][M];
#pragma unroll
  for (int s = 0; s < kQsSteps; ++s) {
#pragma unroll
    for (int j = s ? QsLastPiece<TYPE>(s - 1) + 1 : 0; j <= QsLastPiece<TYPE>(s); ++j) wr[j] = load(0, j);
    act(0, s, av[s]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // chunk c; MORE: the next chunk's loads are issued as this one's land.  The
  // last chunk is a copy of its own, so every chunk before it issues the same
  // loads in the same order and the compiler's waits count them exactly.
  auto chunk = [&](int c, auto more_tag) __attribute__((always_inline)) {
    constexpr bool kMore = decltype(more_tag)::value;
    const int64_t cblocks = nb - (int64_t)c * L::chunk_blocks;  // blocks of this chunk: all when >= chunk_blocks
#pragma unroll
    for (int s = 0; s < kQsSteps; ++s) {
#pragma unroll
      for (int j = s ? QsLastPiece<TYPE>(s - 1) + 1 : 0; j <= QsLastPiece<TYPE>(s); ++j) {
        put(j, wr[j]);
        if (kMore) wr[j] = load(c + 1, j);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (s * kStepBlocks + bl < cblocks) {
#pragma unroll
        for (int r = 0; r < kQsRows; ++r) {
          const uint8_t *base = stage + r * kChunk + s * kStepBytes;
          const uint32_t dw = LdsDword(base, dofs);
          const uint32_t c0 = LdsDword(base, cofs), c1 = LdsDword(base, cofs + 4), c2 = LdsDword(base, cofs + 8);
          const h2_t dd = AsH2(__builtin_amdgcn_perm(dw, dw, dsel));
          const uint32_t cw[2] = {__builtin_amdgcn_alignbit(c1, c0, csh), __builtin_amdgcn_alignbit(c2, c1, csh)};
#pragma unroll
          for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {  // code bytes 4q + 2e, 4q + 2e + 1
              const int p = 2 * q + e;     // activation pair of these values
              if (TYPE == 2) {
                const uint32_t t = __builtin_amdgcn_perm(0u, cw[q], e ? 0x0c030c02u : 0x0c010c00u);
                const h2_t wl = (AsH2(AndOr(t, 0x000f000fu, 0x64006400u)) + kM1032) * dd;
                const h2_t wh = (AsH2(AndOr(t, 0x00f000f0u, 0x54005400u)) + kM72) * dd;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                  acc[r][m] = __builtin_amdgcn_fdot2(AsH2(av[s][0][m][p]), wl, acc[r][m], false);
                  acc[r][m] = __builtin_amdgcn_fdot2(AsH2(av[s][kActLoads - 1][m][p]), wh, acc[r][m], false);
                }
              } else {
                const uint32_t t = __builtin_amdgcn_perm(0x64646464u, cw[q] ^ 0x80808080u, e ? 0x04030402u : 0x04010400u);
                const h2_t wv = (AsH2(t) + kM1152) * dd;
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] = __builtin_amdgcn_fdot2(AsH2(av[s][0][m][p]), wv, acc[r][m], false);
              }
            }
          }
        }
      }
      if (kMore) act(c + 1, s, av[s]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int c = 0; c + 1 < nchunks; ++c) chunk(c, std::true_type{});
  chunk(nchunks - 1, std::false_type{});
#pragma unroll
  for (int r = 0; r < kQsRows; ++r) {
    const int64_t n = n0 + r;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = acc[r][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0 && n < N) y[m * N + n] = F32ToF16(s);
    }
  }
}

// The streamed kernel's conditions: 16-byte aligned operands, K % 256 == 0,
// M <= 2 (its activation registers grow with M) and byte offsets that fit a
// buffer descriptor.
template <int TYPE> bool GemvQ0StreamFits(int64_t M, int64_t N, int64_t K, const void *a, const void *w) {
  return M >= 1 && M <= 2 && K % 256 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
         N * (K / 32) * Q0Stream<TYPE>::block < (int64_t(1) << 31) - (int64_t(1) << 20);
}

template <int TYPE>
void LaunchGemvQ0Stream(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                        hipStream_t s) {
  const dim3 g((unsigned)((N + kQsRows - 1) / kQsRows));
  if (M == 1)
    hipLaunchKernelGGL((GemvQ0StreamKernel<TYPE, 1>), g, dim3(64), 0, s, a, w, N, K, y);
  else
    hipLaunchKernelGGL((GemvQ0StreamKernel<TYPE, 2>), g, dim3(64), 0, s, a, w, N, K, y);
}

// Fused q4_k / q6_k GEMV: y[m, n] = sum_k a[m, k] * W[n, k] with W the
// FLOAT16 DequantizePacked values of the [N, K] weight (ggml layout: the
// 256-value blocks of output n contiguous along k).  A workgroup computes 16
// outputs, 4 per wave; within a wave, lanes 0-31 and 32-63 take alternate
// blocks, each lane 8 consecutive values of its block.  A lane decodes its 8
// values per output with the reference's fp32 steps (two roundings, no
// contraction), rounds them to FLOAT16 (the chain's DequantizePacked output)
// and accumulates with the activations through v_dot2_f32_f16 in fp32.  A
// NaN weight makes the sum NaN whatever its sign, so the decode here skips
// the x86-64 NaN selection of the DequantizePacked kernel.
//
// Loads per lane and output: q4_k one 16-byte header (d, dmin, the 12 scale
// bytes; every block starts 16-byte aligned as 144 = 9 x 16) and one 8-byte
// run of codes; q6_k (210-byte blocks, 2-byte aligned) four 16-bit loads of
// low nibbles, four of high bits, the sub-block's scale byte and d.
// Byte B of a dword as a float in one v_cvt_f32_ubyteB.  Written as
// (float)((t >> 8B) & 0xff) the compiler folds the byte masks into the
// mask that isolated the codes and emits a bit-field extract plus
// v_cvt_f32_ubyte0: two instructions per value instead of one.
template <int B> __device__ __forceinline__ float UbyteF32(uint32_t t) {
  float r;
  if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(t));
  else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(t));
  else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(t));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(t));
  return r;
}

// Four codes, one per byte of t, as floats.
__device__ __forceinline__ void ByteFloats(uint32_t t, float *f) {
  f[0] = UbyteF32<0>(t);
  f[1] = UbyteF32<1>(t);
  f[2] = UbyteF32<2>(t);
  f[3] = UbyteF32<3>(t);
}

__device__ __forceinline__ void NibbleFloats(uint32_t dw, int sh, float *f) { ByteFloats((dw >> sh) & 0x0f0f0f0fu, f); }

// The raw bytes one lane needs from one block, loaded a block ahead of use.
template <int TYPE> struct KRaw;
template <> struct KRaw<12> {
  uint32_t h[4];  // d, dmin, the 12 scale bytes
  uint32_t q[2];  // 8 code bytes
};
template <> struct KRaw<14> {
  uint32_t l[2], hb[2];  // 8 low-nibble bytes, 8 high-bit bytes
  uint32_t d, sc;        // fp16 d, the sub-block's int8 scale
};

__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<12> &r) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  const v4u hdr = *reinterpret_cast<const v4u *>(p);
  const v2u q = *reinterpret_cast<const v2u *>(p + 16 + (i0 >> 6) * 32 + (i0 & 31));
  r.h[0] = hdr.x, r.h[1] = hdr.y, r.h[2] = hdr.z, r.h[3] = hdr.w;
  r.q[0] = q.x, r.q[1] = q.y;
}

__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<14> &r) {
  const uint16_t *ql = reinterpret_cast<const uint16_t *>(p + (i0 >> 7) * 64 + (i0 & 63));
  const uint16_t *qh = reinterpret_cast<const uint16_t *>(p + 128 + (i0 >> 7) * 32 + (i0 & 31));
  r.l[0] = ql[0] | (uint32_t)ql[1] << 16, r.l[1] = ql[2] | (uint32_t)ql[3] << 16;
  r.hb[0] = qh[0] | (uint32_t)qh[1] << 16, r.hb[1] = qh[2] | (uint32_t)qh[3] << 16;
  r.d = *reinterpret_cast<const uint16_t *>(p + 208);
  r.sc = p[192 + (i0 >> 4)];
}

__device__ __forceinline__ void DecodeK(const KRaw<12> &r, int i0, h2_t wp[4]) {
  const float d = F16ToF32((uint16_t)(r.h[0] & 0xffffu)), dmin = F16ToF32((uint16_t)(r.h[0] >> 16));
  const int g = i0 >> 5;
  // scale bytes 0..11 are h[1], h[2], h[3]; sub-block g uses byte g % 4 of
  // each (field extracts, no indexed access into r)
  const int sh = 8 * (g & 3);
  const uint32_t b1 = (r.h[1] >> sh) & 0xffu, b2 = (r.h[2] >> sh) & 0xffu, b3 = (r.h[3] >> sh) & 0xffu;
  const uint32_t scale = g < 4 ? b1 & 63u : (b3 & 15u) | ((b1 >> 6) << 4);
  const uint32_t minimum = g < 4 ? b2 & 63u : (b3 >> 4) | ((b2 >> 6) << 4);
  const float ds = d * (float)scale, dm = dmin * (float)minimum;
  float f[8];
  NibbleFloats(r.q[0], 4 * (g & 1), f);
  NibbleFloats(r.q[1], 4 * (g & 1), f + 4);
  // ds * q is exact in fp32 (ds = d * scale has at most 17 significant
  // bits, q at most 4), so one fused multiply-add rounds (ds * q) - dm
  // exactly as the reference's rounded product and rounded difference do
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float v0 = __builtin_fmaf(ds, f[2 * e], -dm), v1 = __builtin_fmaf(ds, f[2 * e + 1], -dm);
    wp[e] = h2_t{(_Float16)v0, (_Float16)v1};
  }
}

__device__ __forceinline__ void DecodeK(const KRaw<14> &r, int i0, h2_t wp[4]) {
  const float ds = F16ToF32((uint16_t)r.d) * (float)(int8_t)r.sc;
  const int shl = 4 * ((i0 >> 6) & 1), shh = 2 * ((i0 >> 5) & 3);
  float f[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // q = low nibble | (2 high bits << 4), as the bytes of a dword
    ByteFloats(((r.l[h] >> shl) & 0x0f0f0f0fu) | (((r.hb[h] >> shh) & 0x03030303u) << 4), f + 4 * h);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // (q - 32) is exact in fp32, then one rounded multiply, as the reference
    const float v0 = ds * (f[2 * e] - 32.f), v1 = ds * (f[2 * e + 1] - 32.f);
    wp[e] = h2_t{(_Float16)v0, (_Float16)v1};
  }
}

// q2_k, q3_k, q5_k and iq4_xs (field positions of DecodeX above).  A lane's
// 8 values share one sub-block, so each needs one scale (and minimum) and
// 8 consecutive code bytes per plane.
template <> struct KRaw<10> {
  uint32_t q[2];  // 8 bytes of 2-bit codes
  uint32_t sc;    // the dword holding the sub-block's scale / minimum byte
  uint32_t dd;    // fp16 d, fp16 dmin
};
template <> struct KRaw<11> {
  uint32_t hm[2], q[2];  // 8 high-mask bytes, 8 bytes of 2-bit codes
  uint32_t s;            // scale low-nibble byte | 2-bit byte << 8 | fp16 d << 16
};
template <> struct KRaw<13> {
  uint32_t h[4];   // d, dmin, the 12 scale bytes
  uint32_t hb[2];  // 8 high-bit bytes
  uint32_t q[2];   // 8 nibble bytes
};
template <> struct KRaw<23> {
  uint32_t hdr[2];  // fp16 d | high scale bits << 16, the 4 low-nibble scale bytes
  uint32_t q[2];    // 8 nibble bytes
};

// q2_k blocks are 4-byte aligned (84 = 4 x 21).
__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<10> &r) {
  const uint32_t *w = reinterpret_cast<const uint32_t *>(p);
  const int qo = (16 + (i0 >> 7) * 32 + (i0 & 31)) >> 2;
  r.q[0] = w[qo], r.q[1] = w[qo + 1];
  r.sc = w[i0 >> 6];  // byte i0 / 16 of the 16 scale bytes
  r.dd = w[20];       // bytes 80 .. 83
}

// q3_k blocks are 2-byte aligned (110 bytes).
__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<11> &r) {
  const uint16_t *h = reinterpret_cast<const uint16_t *>(p + (i0 & 31));
  const uint16_t *q = reinterpret_cast<const uint16_t *>(p + 32 + (i0 >> 7) * 32 + (i0 & 31));
  r.hm[0] = h[0] | (uint32_t)h[1] << 16, r.hm[1] = h[2] | (uint32_t)h[3] << 16;
  r.q[0] = q[0] | (uint32_t)q[1] << 16, r.q[1] = q[2] | (uint32_t)q[3] << 16;
  const int g = i0 >> 4;
  r.s = p[96 + (g & 7)] | (uint32_t)p[104 + (g & 3)] << 8 |
        (uint32_t)*reinterpret_cast<const uint16_t *>(p + 108) << 16;
}

// q5_k blocks are 16-byte aligned (176 = 16 x 11).
__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<13> &r) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  const v4u hdr = *reinterpret_cast<const v4u *>(p);
  const v2u hb = *reinterpret_cast<const v2u *>(p + 16 + (i0 & 31));
  const v2u q = *reinterpret_cast<const v2u *>(p + 48 + (i0 >> 6) * 32 + (i0 & 31));
  r.h[0] = hdr.x, r.h[1] = hdr.y, r.h[2] = hdr.z, r.h[3] = hdr.w;
  r.hb[0] = hb.x, r.hb[1] = hb.y, r.q[0] = q.x, r.q[1] = q.y;
}

// iq4_xs blocks are 8-byte aligned (136 = 8 x 17).
__device__ __forceinline__ void LoadK(const uint8_t *p, int i0, KRaw<23> &r) {
  typedef unsigned v2u __attribute__((ext_vector_type(2)));
  const v2u hdr = *reinterpret_cast<const v2u *>(p);
  const v2u q = *reinterpret_cast<const v2u *>(p + 8 + (i0 >> 5) * 16 + (i0 & 15));
  r.hdr[0] = hdr.x, r.hdr[1] = hdr.y, r.q[0] = q.x, r.q[1] = q.y;
}

// Reads of a block staged in LDS at byte offset o of the stage array s (16-
// byte aligned).  q3_k and q6_k blocks are only 2-byte aligned, and 16-bit
// LDS reads cost about 20 LDS cycles each there, so their fields are read as
// the aligned dwords around them and funnel-shifted into place
// (v_alignbit_b32, LdsDword above); offsets stay integers into s so the
// reads remain LDS reads.  The other formats read as LoadK does.
// the 8 bytes at offset o (o even): the three dwords around them
__device__ __forceinline__ void LdsBytes8(const uint8_t *s, int o, uint32_t out[2]) {
  const int b = o & ~3;
  const uint32_t sh = 8u * (uint32_t)(o & 3);
  const uint32_t d0 = LdsDword(s, b), d1 = LdsDword(s, b + 4), d2 = LdsDword(s, b + 8);
  out[0] = __builtin_amdgcn_alignbit(d1, d0, sh);
  out[1] = __builtin_amdgcn_alignbit(d2, d1, sh);
}
// the 16 bits at offset o (o even)
__device__ __forceinline__ uint32_t LdsHalf(const uint8_t *s, int o) {
  return (LdsDword(s, o & ~3) >> (8u * (uint32_t)(o & 3))) & 0xffffu;
}
template <class R> __device__ __forceinline__ void LoadKLds(const uint8_t *s, int o, int i0, R &r) {
  LoadK(s + o, i0, r);
}
__device__ __forceinline__ void LoadKLds(const uint8_t *s, int o, int i0, KRaw<11> &r) {
  LdsBytes8(s, o + (i0 & 31), r.hm);
  LdsBytes8(s, o + 32 + (i0 >> 7) * 32 + (i0 & 31), r.q);
  const int g = i0 >> 4;
  r.s = s[o + 96 + (g & 7)] | (uint32_t)s[o + 104 + (g & 3)] << 8 | LdsHalf(s, o + 108) << 16;
}
__device__ __forceinline__ void LoadKLds(const uint8_t *s, int o, int i0, KRaw<14> &r) {
  LdsBytes8(s, o + (i0 >> 7) * 64 + (i0 & 63), r.l);
  LdsBytes8(s, o + 128 + (i0 >> 7) * 32 + (i0 & 31), r.hb);
  r.d = LdsHalf(s, o + 208);
  r.sc = s[o + 192 + (i0 >> 4)];
}

// The products below are exact in fp32 wherever the reference rounds them
// (a 11-bit fp16 d times a scale of at most 6 bits, times a code of at most
// 5 bits), so ds * q - dm in one fused multiply-add, or ds * q, rounds as the
// reference's separately rounded steps do; iq4_xs's ds * value (8-bit
// values) is one rounded product, as in the reference.
// Four codes at a time: one shift and mask per dword leaves each code in
// its own byte, which v_cvt_f32_ubyte0..3 converts directly (ByteFloats).

__device__ __forceinline__ void DecodeK(const KRaw<10> &r, int i0, h2_t wp[4]) {
  const float d = F16ToF32((uint16_t)(r.dd & 0xffffu)), dmin = F16ToF32((uint16_t)(r.dd >> 16));
  const uint32_t b = (r.sc >> (8 * ((i0 >> 4) & 3))) & 0xffu;
  const float ds = d * (float)(b & 15u), dm = dmin * (float)(b >> 4);
  const int sh = 2 * ((i0 >> 5) & 3);
  float f[8];
  ByteFloats((r.q[0] >> sh) & 0x03030303u, f);
  ByteFloats((r.q[1] >> sh) & 0x03030303u, f + 4);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(ds, f[e], -dm);
#pragma unroll
  for (int e = 0; e < 4; ++e) wp[e] = h2_t{(_Float16)v[2 * e], (_Float16)v[2 * e + 1]};
}

__device__ __forceinline__ void DecodeK(const KRaw<11> &r, int i0, h2_t wp[4]) {
  const int g = i0 >> 4;
  const int lo = (int)((r.s & 0xffu) >> (4 * ((g >> 3) & 1))) & 15;
  const int hi = (int)(((r.s >> 8) & 0xffu) >> (2 * ((g >> 2) & 3))) & 3;
  const float ds = F16ToF32((uint16_t)(r.s >> 16)) * (float)((lo | hi << 4) - 32);
  const int hsh = (i0 >> 5) & 7, qsh = 2 * ((i0 >> 5) & 3);
  // u = code + 4 * high-mask bit (0..7 per byte) and q = u - 4.  For a
  // finite ds, ds * u - 4 ds in one fused step is the exact ds * q (both
  // products are exact), rounded as the reference rounds its product; an
  // infinite or NaN ds takes the reference's own steps (inf * 0 = NaN).
  float f[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    ByteFloats(((r.q[h] >> qsh) & 0x03030303u) | (((r.hm[h] >> hsh) & 0x01010101u) << 2), f + 4 * h);
  float v[8];
  if (__builtin_isfinite(ds)) {
    const float ds4 = 4.f * ds;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(ds, f[e], -ds4);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = ds * (f[e] - 4.f);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) wp[e] = h2_t{(_Float16)v[2 * e], (_Float16)v[2 * e + 1]};
}

__device__ __forceinline__ void DecodeK(const KRaw<13> &r, int i0, h2_t wp[4]) {
  const float d = F16ToF32((uint16_t)(r.h[0] & 0xffffu)), dmin = F16ToF32((uint16_t)(r.h[0] >> 16));
  const int g = i0 >> 5;
  const int sh8 = 8 * (g & 3);  // scale bytes as in q4_k
  const uint32_t b1 = (r.h[1] >> sh8) & 0xffu, b2 = (r.h[2] >> sh8) & 0xffu, b3 = (r.h[3] >> sh8) & 0xffu;
  const uint32_t scale = g < 4 ? b1 & 63u : (b3 & 15u) | ((b1 >> 6) << 4);
  const uint32_t minimum = g < 4 ? b2 & 63u : (b3 >> 4) | ((b2 >> 6) << 4);
  const float ds = d * (float)scale, dm = dmin * (float)minimum;
  const int nsh = 4 * (g & 1), hsh = g & 7;
  float f[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    ByteFloats(((r.q[h] >> nsh) & 0x0f0f0f0fu) | (((r.hb[h] >> hsh) & 0x01010101u) << 4), f + 4 * h);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(ds, f[e], -dm);
#pragma unroll
  for (int e = 0; e < 4; ++e) wp[e] = h2_t{(_Float16)v[2 * e], (_Float16)v[2 * e + 1]};
}

__device__ __forceinline__ void DecodeK(const KRaw<23> &r, int i0, h2_t wp[4]) {
  const int g = i0 >> 5;
  const float d = F16ToF32((uint16_t)(r.hdr[0] & 0xffffu));
  const uint32_t high = r.hdr[0] >> 16;
  const int lo = (int)(r.hdr[1] >> (8 * (g >> 1) + 4 * (g & 1))) & 15;
  const float ds = d * (float)((lo | (int)(((high >> (2 * g)) & 3u) << 4)) - 32);
  const int sh = 4 * ((i0 >> 4) & 1);
  float v[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // the 16 codebook values as bytes; v_perm picks 4 at once (codes 0-7 from
    // the low pair, 8-15 from the high pair, merged by bit 3)
    const uint32_t codes = (r.q[h] >> sh) & 0x0f0f0f0fu, sel = codes & 0x07070707u;
    const uint32_t lo4 = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);
    const uint32_t hi4 = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);
    // 0xff in each byte whose code has bit 3: (m << 8) - m, the subtraction
    // written as one instruction (the compiler folds the pair into a
    // quarter-rate v_mul_lo_u32 by 255)
    const uint32_t m = (codes >> 3) & 0x01010101u;
    uint32_t pick;
    asm("v_sub_u32 %0, %1, %2" : "=v"(pick) : "v"(m << 8), "v"(m));
    const uint32_t vals = (hi4 & pick) | (lo4 & ~pick);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * h + e] = ds * (float)(int8_t)(uint8_t)(vals >> (8 * e));
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) wp[e] = h2_t{(_Float16)v[2 * e], (_Float16)v[2 * e + 1]};
}

template <int TYPE, int M>
__global__ __launch_bounds__(256) void GemvKKernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ w,
                                                   int64_t N, int64_t K, uint16_t *__restrict__ y) {
  constexpr int kBytes = KLayout<TYPE>::bytes;
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, i0 = (lane & 31) * 8;
  const int64_t nb = K / 256;
  const int64_t n0 = (int64_t)blockIdx.x * kGvRows + wave * kGvCols;
  const uint8_t *row[kGvCols];  // columns past N decode the last and are not stored
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) row[c] = w + (n0 + c < N ? n0 + c : N - 1) * nb * kBytes;
  float acc[kGvCols][M];
#pragma unroll
  for (int c = 0; c < kGvCols; ++c)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[c][m] = 0.f;
  // the raw bytes and activations of the lane's next block load while the
  // current one is decoded (a lane with no block of its own, nb odd, reloads
  // its last one and adds nothing)
  KRaw<TYPE> cur[kGvCols], nxt[kGvCols];
  v4u av[M], avn[M];
  int64_t kb = half < nb ? half : nb - 1;
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) LoadK(row[c] + kb * kBytes, i0, cur[c]);
#pragma unroll
  for (int m = 0; m < M; ++m) av[m] = *reinterpret_cast<const v4u *>(a + m * K + kb * 256 + i0);
  for (kb = half; kb < nb; kb += 2) {
    const int64_t kn = kb + 2 < nb ? kb + 2 : kb;
#pragma unroll
    for (int c = 0; c < kGvCols; ++c) LoadK(row[c] + kn * kBytes, i0, nxt[c]);
#pragma unroll
    for (int m = 0; m < M; ++m) avn[m] = *reinterpret_cast<const v4u *>(a + m * K + kn * 256 + i0);  // 16-byte aligned
    h2_t wp[kGvCols][4];
#pragma unroll
    for (int c = 0; c < kGvCols; ++c) DecodeK(cur[c], i0, wp[c]);
#pragma unroll
    for (int m = 0; m < M; ++m) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const h2_t ap = AsH2(av[m][e]);
#pragma unroll
        for (int c = 0; c < kGvCols; ++c) acc[c][m] = __builtin_amdgcn_fdot2(ap, wp[c][e], acc[c][m], false);
      }
    }
#pragma unroll
    for (int c = 0; c < kGvCols; ++c) cur[c] = nxt[c];
#pragma unroll
    for (int m = 0; m < M; ++m) av[m] = avn[m];
  }
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) {
    const int64_t n = n0 + c;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = acc[c][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0 && n < N) y[m * N + n] = F32ToF16(s);
    }
  }
}

// The same GEMV with the weight streamed through LDS.  Per lane, the direct
// kernel above issues a few small loads per block (scale bytes, 8 code
// bytes), so little data is in flight and the small-block formats stay far
// below the bandwidth.  Here a workgroup streams its 16 rows CB blocks at a
// time: each row's CB * bytes window, widened to 16-byte boundaries, is read
// with coalesced 16-byte loads into registers while the previous stage is
// decoded, then written to the other half of a double-buffered LDS stage.
// A block keeps its global alignment modulo 16 inside its row slot, so the
// lanes decode it from LDS with the same LoadK / DecodeK as above, in the
// same order (half h of a wave takes the blocks h, h + 2, ... of its rows),
// which gives the same sums.  The stage's activations load before the next
// stage's weights so that their waits do not cover those loads.
template <int TYPE> constexpr int KStageWords(int cb) { return (cb * KLayout<TYPE>::bytes) / 16 + 2; }

template <int TYPE, int M, int CB>
__global__ __launch_bounds__(256) void GemvKLdsKernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ w,
                                                      int64_t N, int64_t K, uint16_t *__restrict__ y) {
  static_assert(CB % 2 == 0, "both halves of a wave take the same number of blocks per full stage");
  constexpr int kBytes = KLayout<TYPE>::bytes;
  constexpr int kWords = KStageWords<TYPE>(CB);  // 16-byte words of a row window at any start alignment
  constexpr int kSlot = kWords * 16;
  constexpr int kStageWords = kGvRows * kWords;
  constexpr int kPer = (kStageWords + 255) / 256;  // words per thread per stage
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) uint8_t stage[2][kGvRows * kSlot];
  // the wave index as a scalar: the per-row offsets below are then scalar
  // work, not 64-bit vector multiplies in the decode loop
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, i0 = (lane & 31) * 8;
  const int64_t nb = K / 256;
  const int64_t n0 = (int64_t)blockIdx.x * kGvRows;
  // The range check of a buffer load is per dword, and a 2-byte aligned
  // format (q3_k, q6_k) can end inside one: the descriptor covers the whole
  // 16-byte word holding the last byte (the same page as that byte; the bytes
  // past the weight are loaded but never decoded).  The launcher checks that
  // this stays below 2^31.
  const int64_t total = (N * nb * kBytes + 15) & ~int64_t(15);
  const __amdgpu_buffer_rsrc_t rsW =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w), (short)0, (int)total, 0x00020000);
  const int nstages = (int)((nb + CB - 1) / CB);

  // per thread: the row and word of each of its stage words (fixed over the stages)
  int wrow[kPer], wword[kPer];
  auto row_of = [&](int r) -> int64_t { return n0 + r < N ? n0 + r : N - 1; };  // rows past N decode the last
  int64_t wbase[kPer];  // byte offset of the row of each stage word
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int idx = tid + 256 * j;
    wrow[j] = idx / kWords;
    wword[j] = idx - wrow[j] * kWords;
    wbase[j] = row_of(wrow[j]) * nb * kBytes;
  }
  // a decoding row's block offsets modulo 16 (its window keeps the global
  // alignment): (row * nb * bytes) mod 16, plus the stage's part
  int rmod[kGvCols];
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) rmod[c] = (int)((row_of(wave * kGvCols + c) * nb * kBytes) & 15);
  v4u regs[kPer];
  auto load = [&](int s) __attribute__((always_inline)) {
    const int64_t kb0 = (int64_t)s * CB;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const bool ok = tid + 256 * j < kStageWords;
      const int64_t start = wbase[j] + kb0 * kBytes;
      const int64_t off = (start & ~int64_t(15)) + 16 * wword[j];
      regs[j] = __builtin_bit_cast(
          v4u, __builtin_amdgcn_raw_buffer_load_b128(rsW, ok ? (unsigned)off : 0x80000000u, 0, 2));
    }
  };
  auto put = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (tid + 256 * j < kStageWords) *reinterpret_cast<v4u *>(&stage[buf][wrow[j] * kSlot + wword[j] * 16]) = regs[j];
  };

  float acc[kGvCols][M];
#pragma unroll
  for (int c = 0; c < kGvCols; ++c)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[c][m] = 0.f;

  load(0);
  put(0);
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    const int64_t kb0 = (int64_t)s * CB;
    const int cb = (int)(nb - kb0 < CB ? nb - kb0 : CB);
    // this stage's activations, then the next stage's weights
    v4u av[CB / 2][M];
#pragma unroll
    for (int q = 0; q < CB / 2; ++q) {
      const int bb = 2 * q + half;
      const int64_t kb = kb0 + (bb < cb ? bb : 0);
#pragma unroll
      for (int m = 0; m < M; ++m) av[q][m] = *reinterpret_cast<const v4u *>(a + m * K + kb * 256 + i0);
    }
    if (s + 1 < nstages) load(s + 1);
#pragma unroll
    for (int q = 0; q < CB / 2; ++q) {
      const int bb = 2 * q + half;
      if (bb < cb) {
        h2_t wp[kGvCols][4];
#pragma unroll
        for (int c = 0; c < kGvCols; ++c) {
          const int r = wave * kGvCols + c;
          const int sm = (rmod[c] + (int)((kb0 * kBytes) & 15)) & 15;  // (row * nb + kb0) * bytes mod 16
          KRaw<TYPE> raw;
          LoadKLds(stage[buf], r * kSlot + sm + bb * kBytes, i0, raw);
          DecodeK(raw, i0, wp[c]);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const h2_t ap = AsH2(av[q][m][e]);
#pragma unroll
            for (int c = 0; c < kGvCols; ++c) acc[c][m] = __builtin_amdgcn_fdot2(ap, wp[c][e], acc[c][m], false);
          }
        }
      }
    }
    if (s + 1 < nstages) put(buf ^ 1);  // the other buffer: every wave left it at the last barrier
    __syncthreads();
  }
#pragma unroll
  for (int c = 0; c < kGvCols; ++c) {
    const int64_t n = n0 + wave * kGvCols + c;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float s = acc[c][m];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0 && n < N) y[m * N + n] = F32ToF16(s);
    }
  }
}

// Blocks per stage: about 10-18 KB of weight per stage for 16 rows, fewer
// blocks when 8 activation rows would hold too many registers.
template <int TYPE, int M> constexpr int KStageBlocks() {
  return KLayout<TYPE>::bytes <= 136 && M <= 4 ? 8 : 4;
}

// The staged kernel for every format while the weight's byte offsets fit a
// buffer descriptor; the direct kernel past that.
template <int TYPE, int M>
void LaunchGemvKM(const uint16_t *a, const uint8_t *w, int64_t N, int64_t K, uint16_t *y, hipStream_t s) {
  const dim3 g((unsigned)((N + kGvRows - 1) / kGvRows));
  if (N * (K / 256) * KLayout<TYPE>::bytes < (int64_t(1) << 31) - (int64_t(1) << 20))
    hipLaunchKernelGGL((GemvKLdsKernel<TYPE, M, KStageBlocks<TYPE, M>()>), g, dim3(256), 0, s, a, w, N, K, y);
  else
    hipLaunchKernelGGL((GemvKKernel<TYPE, M>), g, dim3(256), 0, s, a, w, N, K, y);
}

template <int TYPE>
void LaunchGemvKType(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                     hipStream_t s) {
  switch (M) {
  case 1: LaunchGemvKM<TYPE, 1>(a, w, N, K, y, s); break;
  case 2: LaunchGemvKM<TYPE, 2>(a, w, N, K, y, s); break;
  case 3: LaunchGemvKM<TYPE, 3>(a, w, N, K, y, s); break;
  case 4: LaunchGemvKM<TYPE, 4>(a, w, N, K, y, s); break;
  case 5: LaunchGemvKM<TYPE, 5>(a, w, N, K, y, s); break;
  case 6: LaunchGemvKM<TYPE, 6>(a, w, N, K, y, s); break;
  case 7: LaunchGemvKM<TYPE, 7>(a, w, N, K, y, s); break;
  case 8: LaunchGemvKM<TYPE, 8>(a, w, N, K, y, s); break;
  default: throw Unsupported("k-quant GEMV: M above 8");
  }
}

}  // namespace

void LaunchGemvK(int ggml_type, const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                 hipStream_t s) {
  if (N == 0) return;
  switch (ggml_type) {
  case 10: LaunchGemvKType<10>(a, w, M, N, K, y, s); break;
  case 11: LaunchGemvKType<11>(a, w, M, N, K, y, s); break;
  case 12: LaunchGemvKType<12>(a, w, M, N, K, y, s); break;
  case 13: LaunchGemvKType<13>(a, w, M, N, K, y, s); break;
  case 14: LaunchGemvKType<14>(a, w, M, N, K, y, s); break;
  case 23: LaunchGemvKType<23>(a, w, M, N, K, y, s); break;
  default: throw DeviceError("internal: no fused GEMV for this GGUF type");
  }
}

int GemvKAlignment(int ggml_type) {
  switch (ggml_type) {
  case 10: return 4;
  case 11: case 14: return 2;
  case 12: case 13: return 16;
  case 23: return 8;
  default: return 0;
  }
}

void LaunchGemvQ80(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                   hipStream_t s) {
  if (N == 0) return;
  if (GemvQ0StreamFits<8>(M, N, K, a, w)) return LaunchGemvQ0Stream<8>(a, w, M, N, K, y, s);
  const dim3 g((unsigned)((N + kGvRows - 1) / kGvRows));
  switch (M) {
  case 1: hipLaunchKernelGGL(GemvQ80Kernel<1>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 2: hipLaunchKernelGGL(GemvQ80Kernel<2>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 3: hipLaunchKernelGGL(GemvQ80Kernel<3>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 4: hipLaunchKernelGGL(GemvQ80Kernel<4>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 5: hipLaunchKernelGGL(GemvQ80Kernel<5>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 6: hipLaunchKernelGGL(GemvQ80Kernel<6>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 7: hipLaunchKernelGGL(GemvQ80Kernel<7>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 8: hipLaunchKernelGGL(GemvQ80Kernel<8>, g, dim3(256), 0, s, a, w, N, K, y); break;
  default: throw Unsupported("q8_0 GEMV: M above 8");
  }
}

bool GemvQ40Eligible(int64_t M, int64_t K, const void *a, const void *w) {
  return M >= 1 && M <= 8 && K % 64 == 0 && K > 0 && reinterpret_cast<uintptr_t>(w) % 4 == 0 &&
         reinterpret_cast<uintptr_t>(a) % 4 == 0;
}

void LaunchGemvQ40(const uint16_t *a, const uint8_t *w, int64_t M, int64_t N, int64_t K, uint16_t *y,
                   hipStream_t s) {
  if (N == 0) return;
  if (GemvQ0StreamFits<2>(M, N, K, a, w)) return LaunchGemvQ0Stream<2>(a, w, M, N, K, y, s);
  const dim3 g((unsigned)((N + kGvRows - 1) / kGvRows));
  switch (M) {
  case 1: hipLaunchKernelGGL(GemvQ40Kernel<1>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 2: hipLaunchKernelGGL(GemvQ40Kernel<2>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 3: hipLaunchKernelGGL(GemvQ40Kernel<3>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 4: hipLaunchKernelGGL(GemvQ40Kernel<4>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 5: hipLaunchKernelGGL(GemvQ40Kernel<5>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 6: hipLaunchKernelGGL(GemvQ40Kernel<6>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 7: hipLaunchKernelGGL(GemvQ40Kernel<7>, g, dim3(256), 0, s, a, w, N, K, y); break;
  case 8: hipLaunchKernelGGL(GemvQ40Kernel<8>, g, dim3(256), 0, s, a, w, N, K, y); break;
  default: throw Unsupported("q4_0 GEMV: M above 8");
  }
}

bool PackedFormatOnGpu(int ggml_type) {
  switch (ggml_type) {
  case 2: case 3: case 6: case 7: case 8: case 9: case 20: case 12: case 14:
  case 10: case 11: case 13: case 15: case 23: case 34: case 35: case 39: case 40: case 41: case 42:
  case 16: case 17: case 18: case 19: case 21: case 22: case 29:
    return true;
  default:
    return false;
  }
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
  case 12: LaunchPkKOut<12>(x, nblocks, out_dtype, y, vec, s); break;
  case 14: LaunchPkKOut<14>(x, nblocks, out_dtype, y, vec, s); break;
  case 10: LaunchPkXOut<10>(x, nblocks, out_dtype, y, vec, s); break;
  case 11: LaunchPkXOut<11>(x, nblocks, out_dtype, y, vec, s); break;
  case 13: LaunchPkXOut<13>(x, nblocks, out_dtype, y, vec, s); break;
  case 15: LaunchPkXOut<15>(x, nblocks, out_dtype, y, vec, s); break;
  case 23: LaunchPkXOut<23>(x, nblocks, out_dtype, y, vec, s); break;
  case 34: LaunchPkXOut<34>(x, nblocks, out_dtype, y, vec, s); break;
  case 35: LaunchPkXOut<35>(x, nblocks, out_dtype, y, vec, s); break;
  case 39: LaunchPkXOut<39>(x, nblocks, out_dtype, y, vec, s); break;
  case 40: LaunchPkXOut<40>(x, nblocks, out_dtype, y, vec, s); break;
  case 41: LaunchPkXOut<41>(x, nblocks, out_dtype, y, vec, s); break;
  case 42: LaunchPkXOut<42>(x, nblocks, out_dtype, y, vec, s); break;
  case 16: LaunchPkIqOut<16>(x, nblocks, out_dtype, y, vec, s); break;
  case 17: LaunchPkIqOut<17>(x, nblocks, out_dtype, y, vec, s); break;
  case 18: LaunchPkIqOut<18>(x, nblocks, out_dtype, y, vec, s); break;
  case 19: LaunchPkIqOut<19>(x, nblocks, out_dtype, y, vec, s); break;
  case 21: LaunchPkIqOut<21>(x, nblocks, out_dtype, y, vec, s); break;
  case 22: LaunchPkIqOut<22>(x, nblocks, out_dtype, y, vec, s); break;
  case 29: LaunchPkIqOut<29>(x, nblocks, out_dtype, y, vec, s); break;
  default: throw Unsupported("DequantizePacked: no GPU kernel for this format");
  }
}

}  // namespace onnxl_amd
