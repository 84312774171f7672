// Device-side element codecs with the reference's rounding rules
// (core/runtime/kernels/cast_helper.cc, cast_float8.cc, cast_sub_byte.cc).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

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

}  // namespace onnxl_amd
