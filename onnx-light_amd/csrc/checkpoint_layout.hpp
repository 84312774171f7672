// AWQ, GPTQ and BitBLAS checkpoint layouts: where the code of weight (k, n)
// and the zero point of (group, n) sit in the packed words
// (onnx_core/runtime/awq.cc:185-230 Code / Reconstructed,
// onnx_core/runtime/gptq.cc:166-205 Pieces / Code / Zero,
// onnx_core/runtime/bitblas.cc:239-290 Codes / Affine).  The functions
// are __host__ __device__: the host runs them for the formats' value checks
// on the few (group, column) pairs that need an exact scan, the preparation
// and decode kernels for every code.  Words are little-endian on both sides.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace onnxl_amd {

enum CkptKind : int {
  kAwqGemm = 0,   // AWQ "gemm": qweight INT32 [K, N * bits / 32] (4 or 8 bits)
  kAwqGemv = 1,   // AWQ "gemv": qweight INT32 [N, K / 8]
  kAwqFast = 2,   // AWQ "gemv_fast" / "llm-awq": qweight INT16 [N / 4, K], float zero terms
  kGptq = 3,      // GPTQ "gptq", "gptq_v2", "gptq_p"
  kBitblas = 4,   // BitBLAS "row-packed-v1": qweight INT8 [N, K * bits / 8], scales [N, groups]
};

struct CkptLayout {
  int kind, bits, width;   // width: bytes per packed word (GPTQ 1, 2, 4, 8)
  int planar;              // GPTQ: 32-code blocks split into 4-, 2- and 1-bit planes
  int zero_add;            // GPTQ "gptq" (v1): the stored zero field plus 1
  int signed_codes;        // BitBLAS from symmetric GPTQ: codes XOR the midpoint, zero = the midpoint
  int64_t K, N, group;     // group: rows per group (K for group_size -1)
  int64_t groups;          // scale / zero rows
  int64_t padded;          // AWQ gemv, gemv_fast: padded group count; BitBLAS: groups
  int64_t zero_columns;    // GPTQ: words per qzeros row
  const uint8_t *qweight, *qzeros;
};

__host__ __device__ inline uint64_t CkptWord(const uint8_t *p, int64_t index, int width) {
  switch (width) {
  case 1: return p[index];
  case 2: return reinterpret_cast<const uint16_t *>(p)[index];
  case 4: return reinterpret_cast<const uint32_t *>(p)[index];
  default: return reinterpret_cast<const uint64_t *>(p)[index];
  }
}

// AWQ's column order inside a 4-bit gemm word: column n % 8 sits at nibble
// {0, 4, 1, 5, 2, 6, 3, 7}[n % 8].
__host__ __device__ inline int AwqNibble(int64_t n) {
  const int j = (int)(n & 7);
  return (j >> 1) + 4 * (j & 1);
}

// One GPTQ field: logical code `index` of the stream `other` (a column of
// qweight, or a group row of qzeros).  Linear layouts take bits index * bits
// onwards of the stream, across a word boundary where the code crosses one;
// planar layouts keep each block of 32 codes in `bits` words, its 4-, 2- and
// 1-bit planes (those the width has, low bits first) one after the other.
__host__ __device__ inline uint32_t GptqField(const CkptLayout &L, const uint8_t *data, int64_t index, int64_t other,
                                              bool zeros) {
  const int wb = 8 * L.width;
  uint32_t r = 0;
  int64_t word[3];
  int shift[3], nb[3], off[3], pieces = 0;
  if (!L.planar) {
    const int64_t bit = index * L.bits;
    const int s = (int)(bit % wb);
    const int low = L.bits < wb - s ? L.bits : wb - s;
    word[0] = bit / wb, shift[0] = s, nb[0] = low, off[0] = 0, pieces = 1;
    if (low != L.bits) word[1] = bit / wb + 1, shift[1] = 0, nb[1] = L.bits - low, off[1] = low, pieces = 2;
  } else {
    int o = 0;
    int64_t w = (index / 32) * L.bits;
    for (int plane = 4; plane >= 1; plane >>= 1) {
      if (!(L.bits & plane)) continue;
      const int factor = 32 / plane;
      word[pieces] = w + (index % 32) / factor;
      shift[pieces] = (int)((index % 32) % factor) * plane;
      nb[pieces] = plane;
      off[pieces] = o;
      ++pieces;
      o += plane;
      w += plane;
    }
  }
  for (int i = 0; i < pieces; ++i) {
    const int64_t pos = zeros ? other * L.zero_columns + word[i] : word[i] * L.N + other;
    r |= (uint32_t)((CkptWord(data, pos, L.width) >> shift[i]) & ((1ull << nb[i]) - 1)) << off[i];
  }
  return r;
}

// A BitBLAS field: `bits` bits from bit `index * bits` of a little-endian
// byte stream (a code may span two bytes; bits <= 8).
__host__ __device__ inline uint32_t BitblasField(const uint8_t *data, int64_t index, int bits) {
  const int64_t bit = index * bits;
  const int s = (int)(bit & 7);
  uint32_t v = (uint32_t)data[bit >> 3] >> s;
  if (s + bits > 8) v |= (uint32_t)data[(bit >> 3) + 1] << (8 - s);
  return v & ((1u << bits) - 1);
}

// The code of weight row k, column n.
__host__ __device__ inline uint32_t CkptCode(const CkptLayout &L, int64_t k, int64_t n) {
  switch (L.kind) {
  case kBitblas: {  // row n of the [N, K] code matrix, K codes a row
    const uint32_t c = BitblasField(L.qweight, n * L.K + k, L.bits);
    return L.signed_codes ? c ^ (1u << (L.bits - 1)) : c;
  }
  case kAwqGemm:
    if (L.bits == 4)
      return (uint32_t)(CkptWord(L.qweight, k * (L.N / 8) + n / 8, 4) >> (4 * AwqNibble(n))) & 15u;
    return L.qweight[k * L.N + n];  // 8 bits: byte n % 4 of word k * (N / 4) + n / 4
  case kAwqGemv:
    return (uint32_t)(CkptWord(L.qweight, n * (L.K / 8) + k / 8, 4) >> (4 * (k % 8))) & 15u;
  case kAwqFast: {
    // the inverse of two 32-code permutations and a 4-row / 64-code interleave
    const int64_t i = k % 32;
    const int64_t first = ((i / 2) % 4) * 8 + (i / 8) * 2 + i % 2;
    const int64_t second = (first / 8) * 8 + (first % 2) * 4 + (first % 8) / 2;
    const int64_t flat = (n % 4) * 64 + (k % 64) / 32 * 32 + second;
    return (uint32_t)(CkptWord(L.qweight, (n / 4) * L.K + (k / 64) * 64 + flat / 4, 2) >> (4 * (flat % 4))) & 15u;
  }
  default:
    return GptqField(L, L.qweight, k, n, false);
  }
}

// The integer zero point of (group g, column n); AWQ gemv_fast / llm-awq
// has float zero terms instead (0 here).
__host__ __device__ inline uint32_t CkptZero(const CkptLayout &L, int64_t g, int64_t n) {
  switch (L.kind) {
  case kAwqGemm:
    if (L.bits == 4)
      return (uint32_t)(CkptWord(L.qzeros, g * (L.N / 8) + n / 8, 4) >> (4 * AwqNibble(n))) & 15u;
    return L.qzeros[g * L.N + n];
  case kAwqGemv:
    return (uint32_t)(CkptWord(L.qzeros, n * (L.padded / 8) + g / 8, 4) >> (4 * (g % 8))) & 15u;
  case kAwqFast:
    return 0;
  case kBitblas:  // qzeros [groups, N * bits / 8]: N codes a group row
    return L.signed_codes ? 1u << (L.bits - 1) : BitblasField(L.qzeros, g * L.N + n, L.bits);
  default:
    return GptqField(L, L.qzeros, n, g, true) + (uint32_t)L.zero_add;
  }
}

// Index of the scale (and AWQ fast zero term) of (group g, column n).
__host__ __device__ inline int64_t CkptScaleIndex(const CkptLayout &L, int64_t g, int64_t n) {
  return L.kind == kAwqGemv || L.kind == kBitblas ? n * L.padded + g : g * L.N + n;
}

}  // namespace onnxl_amd
