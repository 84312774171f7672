// Device-side element codecs with the reference's rounding rules
// (core/runtime/kernels/cast_helper.cc, cast_float8.cc, cast_sub_byte.cc).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace onnxl_amd {

// FLOAT16 bits -> float (exact; NaN payload kept).
__device__ __forceinline__ float F16ToF32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// float -> FLOAT16 bits, round to nearest even (hardware v_cvt_f16_f32 in the
// default round-to-nearest mode, fp16 denormals on).  NaN -> sign|0x7e00 as
// the reference writes it (cast_helper.cc:57-60).
__device__ __forceinline__ uint16_t F32ToF16(float f) {
  if (__builtin_isnan(f)) return (uint16_t)((__builtin_bit_cast(uint32_t, f) >> 16 & 0x8000u) | 0x7e00u);
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float Bf16ToF32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}

// float -> BFLOAT16 bits, round to nearest even; NaN keeps its upper half with
// the quiet bit set (cast_helper.cc:124-134).
__device__ __forceinline__ uint16_t F32ToBf16(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// FLOAT8E4M3FN bits -> float, exact (cast_float8.cc:83-118).
__device__ __forceinline__ float Fp8E4M3ToF32(uint8_t c) {
  const uint32_t s = (uint32_t)(c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
  if ((c & 0x7fu) == 0x7fu) return __builtin_bit_cast(float, s | 0x7fc00000u);
  if (e == 0) {
    const float mag = (float)m * 0.001953125f;  // m * 2^-9, exact
    return s ? -mag : mag;
  }
  return __builtin_bit_cast(float, s | ((e + 120u) << 23) | (m << 20));
}

// Round half to even of x / 2^sh for 1 <= sh <= 31.
__device__ __forceinline__ uint32_t ShrRne(uint32_t x, uint32_t sh) {
  const uint32_t q = x >> sh, rem = x & ((1u << sh) - 1u), half = 1u << (sh - 1u);
  return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

// float -> FLOAT8E4M3FN bits, saturating round to nearest even: NaN ->
// sign|0x7f, +-inf and magnitudes past 448 -> sign|0x7e, fp32 subnormals and
// magnitudes below 2^-10 -> signed zero (cast_float8.cc:27-81).
__device__ __forceinline__ uint8_t F32ToFp8E4M3Sat(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (a == 0x7f800000u) return (uint8_t)(sign | 0x7eu);
  const int e = (int)(a >> 23);
  if (e < 117) return (uint8_t)sign;
  const int E = e - 120;  // fp8 biased exponent of a normal result
  uint32_t mag = E >= 1 ? ShrRne(((uint32_t)E << 23) | (a & 0x7fffffu), 20)
                        : ShrRne((a & 0x7fffffu) | 0x800000u, (uint32_t)(21 - E));
  if (mag > 0x7eu) mag = 0x7eu;
  return (uint8_t)(sign | mag);
}

__device__ __forceinline__ int Int4ToInt(uint32_t nibble) {
  return (int)((nibble & 0xfu) ^ 8u) - 8;
}

// The NaN an fp32 step produces in the reference's x86-64 build, whose SSE
// arithmetic returns the first operand (quieted) when both are NaN, else the
// NaN one, and the negative default NaN 0xffc00000 for inf * 0 and inf - inf;
// the GPU's own choice of operand and default NaN is replaced by that.
__device__ __forceinline__ float SseNaN(float r, float a, float b) {
  if (r == r) return r;
  const uint32_t bits = a != a   ? __builtin_bit_cast(uint32_t, a) | 0x00400000u
                        : b != b ? __builtin_bit_cast(uint32_t, b) | 0x00400000u
                                 : 0xffc00000u;
  return __builtin_bit_cast(float, bits);
}
__device__ __forceinline__ float SseMul(float a, float b) { return SseNaN(a * b, a, b); }
__device__ __forceinline__ float SseSub(float a, float b) { return SseNaN(a - b, a, b); }

// FLOAT8E4M3FNUZ / FLOAT8E5M2FNUZ bits -> float, exact (cast_float8.cc:
// 174-215, 347-380): exponent bias 8 / 16, 0x80 the only NaN (0xffc00000).
template <int MB, int BIAS> __device__ __forceinline__ float Fp8FnuzToF32(uint8_t c) {
  if (c == 0x80u) return __builtin_bit_cast(float, 0xffc00000u);
  constexpr int EB = 7 - MB;
  const uint32_t e = (c >> MB) & ((1u << EB) - 1u), m = c & ((1u << MB) - 1u);
  const float mag = e == 0 ? (float)m * __builtin_bit_cast(float, (uint32_t)(128 - BIAS - MB) << 23)
                           : __builtin_bit_cast(float, ((e + 127u - BIAS) << 23) | (m << (23 - MB)));
  return (c & 0x80u) ? -mag : mag;
}

// FLOAT8E5M2 bits -> float, exact (cast_float8.cc:263-300): the fp16 layout's
// top byte; 0x7d-0x7f decode to 0x7fc00000 and 0xfd-0xff to 0xffc00000.
__device__ __forceinline__ float Fp8E5M2ToF32(uint8_t c) {
  if ((c & 0x7fu) > 0x7cu) return __builtin_bit_cast(float, (c & 0x80u) ? 0xffc00000u : 0x7fc00000u);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)((uint32_t)c << 8));
}

// FLOAT4E2M1 nibble -> float (cast_helper.cc:161-166): +-{0, .5, 1, 1.5, 2, 3, 4, 6}.
__device__ __forceinline__ float Fp4E2M1ToF32(uint32_t nib) {
  const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
  const float mag = e == 0 ? 0.5f * (float)m : __builtin_bit_cast(float, ((e + 126u) << 23) | (m << 22));
  return (nib & 8u) ? -mag : mag;
}

// FLOAT6E2M3 (MB = 3) / FLOAT6E3M2 (MB = 2) bits -> float (cast_helper.cc:
// 208-219): bias 2^(E-1) - 1, subnormals at exponent 0, sign bit 5.
template <int MB> __device__ __forceinline__ float Fp6ToF32(uint32_t bits) {
  constexpr int EB = 5 - MB, BIAS = (1 << (EB - 1)) - 1;
  const uint32_t e = (bits >> MB) & ((1u << EB) - 1u), m = bits & ((1u << MB) - 1u);
  const float mag = e == 0 ? (float)m * __builtin_bit_cast(float, (uint32_t)(128 - BIAS - MB) << 23)
                           : __builtin_bit_cast(float, ((e + 127u - BIAS) << 23) | (m << (23 - MB)));
  return (bits & 0x20u) ? -mag : mag;
}

// float -> FLOAT8E4M3FNUZ (MB 3, BIAS 8), FLOAT8E5M2 (MB 2, BIAS 15, FNUZ
// false) or FLOAT8E5M2FNUZ (MB 2, BIAS 16) bits, the saturating encoders of
// cast_float8.cc:124-173, 214-262 and 303-346: round to nearest even,
// +-inf and overflow to the largest finite code (0x7f FNUZ, 0x7b E5M2),
// magnitudes below half the smallest subnormal to zero, FNUZ zeros and NaN
// unsigned (NaN 0x80); E5M2 NaN is sign|0x7e with the sign the caller
// chooses, so this returns 0x7e for it.
template <int MB, int BIAS, bool FNUZ> __device__ __forceinline__ uint8_t F32ToFp8Sat(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7fffffffu;
  constexpr uint32_t kMax = FNUZ ? 0x7fu : 0x7bu;
  if (a > 0x7f800000u) return FNUZ ? 0x80u : 0x7eu;
  if (a == 0x7f800000u) return (uint8_t)(sign | kMax);
  const int e = (int)(a >> 23);
  const int E = e - 127 + BIAS;  // biased exponent of a normal result
  uint32_t mag = 0;
  if (e == 0) mag = 0;           // fp32 zeros and subnormals
  else if (E >= 1) mag = ShrRne(((uint32_t)E << 23) | (a & 0x7fffffu), 23 - MB);
  else if (24 - MB - E <= 25) mag = ShrRne((a & 0x7fffffu) | 0x800000u, (uint32_t)(24 - MB - E));
  if (mag > kMax) mag = kMax;
  if (FNUZ && mag == 0) return 0;
  return (uint8_t)(sign | mag);
}

// float -> FLOAT4E2M1 nibble (cast_helper.cc:168-203): NaN -> 0, beyond +-6
// saturates, else the nearest of the same-sign codes by fp32 distance, ties
// to the even code.  |v - c| of a negative v and code -c equals ||v| - c|
// exactly, so the scan runs on the magnitude.
__device__ __forceinline__ uint32_t F32ToFp4E2M1(float v) {
  if (v != v) return 0u;
  if (v > 6.0f) return 7u;
  if (v < -6.0f) return 15u;
  const uint32_t sign = __builtin_bit_cast(uint32_t, v) >> 31 ? 8u : 0u;
  const float m = __builtin_fabsf(v);
  uint32_t best = 0;
  float bd = m;
#pragma unroll
  for (uint32_t i = 1; i < 8; ++i) {
    const float d = __builtin_fabsf(m - Fp4E2M1ToF32(i));
    if (d < bd || (d == bd && !(i & 1u) && (best & 1u))) {
      best = i;
      bd = d;
    }
  }
  return best | sign;
}

// float -> FLOAT6E2M3 (MB 3) / FLOAT6E3M2 (MB 2) bits (cast_helper.cc:
// 220-246): NaN -> 0, +-inf -> +-0x1f, else the first magnitude code not
// below |v| (a binary search over the ordered codes) or the one before it,
// by fp32 distance with ties to the even code; past the largest, 0x1f.
template <int MB> __device__ __forceinline__ uint32_t F32ToFp6(float v) {
  if (v != v) return 0u;
  const uint32_t sign = __builtin_bit_cast(uint32_t, v) >> 31 ? 0x20u : 0u;
  const float m = __builtin_fabsf(v);
  if (m == __builtin_inff()) return 0x1fu | sign;
  uint32_t lo = 0, n = 32;  // lower_bound over codes [lo, lo + n)
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const uint32_t half = n >> 1;
    if (n > 0 && Fp6ToF32<MB>(lo + half) < m) {
      lo += half + 1;
      n -= half + 1;
    } else {
      n = half;
    }
  }
  uint32_t best = lo == 32 ? 0x1fu : lo;
  if (lo != 0 && lo != 32) {
    const float ld = m - Fp6ToF32<MB>(lo - 1), ud = Fp6ToF32<MB>(lo) - m;
    if (ld < ud || (ld == ud && !((lo - 1) & 1u))) best = lo - 1;
  }
  return best | sign;
}


// Element i of a tensor of type XT as float, as the reference's
// DequantizeLinear reads its input and QuantizeLinear its zero point
// (kernel_dequantizelinear.cc:85-155):
// 4-bit types two per byte (low nibble first), 2-bit four per byte from the
// low bits, 6-bit a little-endian bit stream.
template <int XT>
__device__ __forceinline__ float DecodeElement(const void *base, int64_t i) {
  const uint8_t *b = static_cast<const uint8_t *>(base);
  if constexpr (XT == kUint8) return (float)b[i];
  else if constexpr (XT == kInt8) return (float)static_cast<const int8_t *>(base)[i];
  else if constexpr (XT == kUint16) return (float)static_cast<const uint16_t *>(base)[i];
  else if constexpr (XT == kInt16) return (float)static_cast<const int16_t *>(base)[i];
  else if constexpr (XT == kInt32) return (float)static_cast<const int32_t *>(base)[i];
  else if constexpr (XT == kFloat8E4M3FN) return Fp8E4M3ToF32(b[i]);
  else if constexpr (XT == kFloat8E4M3FNUZ) return Fp8FnuzToF32<3, 8>(b[i]);
  else if constexpr (XT == kFloat8E5M2) return Fp8E5M2ToF32(b[i]);
  else if constexpr (XT == kFloat8E5M2FNUZ) return Fp8FnuzToF32<2, 16>(b[i]);
  else if constexpr (XT == kUint2 || XT == kInt2) {
    const uint32_t c = (b[i >> 2] >> (2 * (i & 3))) & 3u;
    return XT == kInt2 ? (float)((int)(c ^ 2u) - 2) : (float)c;
  } else if constexpr (XT == kFloat6E2M3 || XT == kFloat6E3M2) {
    const int64_t bit = 6 * i, byte = bit >> 3;
    const int sh = (int)(bit & 7);
    uint32_t v = (uint32_t)b[byte] >> sh;
    if (sh > 2) v |= (uint32_t)b[byte + 1] << (8 - sh);
    return Fp6ToF32<XT == kFloat6E2M3 ? 3 : 2>(v & 63u);
  } else {
    const uint8_t byte = b[i >> 1];
    const uint32_t nib = (i & 1) ? (byte >> 4) : (byte & 0xfu);
    if constexpr (XT == kInt4) return (float)Int4ToInt(nib);
    else if constexpr (XT == kFloat4E2M1) return Fp4E2M1ToF32(nib);
    else return (float)nib;  // kUint4
  }
}

}  // namespace onnxl_amd
