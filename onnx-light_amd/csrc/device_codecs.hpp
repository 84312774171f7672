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

}  // namespace onnxl_amd
