// ORT MatMulNBits weights (onnx_core/runtime/quantization.cc:916-930 plan,
// :1806-1880 decode): B [N, groups, block * bits / 8] holds the codes of
// column n, row g * block + j at bit (j % (8 / bits)) * bits of byte
// j / (8 / bits) of blob (n, g); scales [N, groups]; zero points packed
// UINT8 codes [N, ceil(groups * bits / 8)] or absent (then 2^(bits-1)).
// value = (code - zero point) * scale, rounded to the scale's dtype.
//
// Session-time preparation into the operands of the fused
// DequantizeLinear -> MatMul kernels, so the decode GEMV reads the weight
// directly in its own tiled layout:
//  - 4 bits: the tiled INT4 / UINT4 layout of TileInt4Kernel (each 16-column
//    tile's K range contiguous).  Without zero points the codes are offset
//    binary INT4 (code - 8 is the signed value, the tiled layout's own
//    encoding); with them UINT4 codes and UINT4 zero points [groups, N];
//  - 2 bits: the same 4-bit tiled layout (twice the bytes of the ORT blob),
//    so the same kernels run them: without zero points INT4 codes of
//    code - 2 (offset binary code + 6), with them UINT4 codes 0..3 and UINT4
//    zero points;
//  - 8 bits: [K, N] bytes, INT8 (code ^ 0x80 = code - 128) without zero
//    points, UINT8 codes with UINT8 zero points [groups, N];
//  - scales transposed to [groups, N] (blocked along K, axis 0).
// Every kernel is one thread per output word or element, reading the ORT
// bytes it needs; all of them run once per weight.
#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kGroupRows = 128;  // the tiled layout's row group (gemv_q4_tiled.hip)

// Tiled 4-bit words from ORT 4- or 2-bit codes (`bits`), each plus `add`:
// word idx = ((t * ngroups + q) * 64 + l) * 4 + c holds column 16 t + l % 16,
// rows 128 q + 32 c + 8 (l / 16) + (0..7), row 2i at bits 4i and row 2i + 1
// at bits 16 + 4i; `pad` fills rows past K and columns past N.
__global__ void OrtTileInt4Kernel(const uint8_t *__restrict__ B, int64_t K, int64_t N, int64_t block,
                                  int64_t groups, int64_t ngroups, int bits, uint32_t add, uint32_t pad,
                                  int64_t total, uint32_t *__restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx & 3);
  const int l = (int)((idx >> 2) & 63);
  const int64_t tq = idx >> 8;
  const int64_t t = tq / ngroups, q = tq % ngroups;
  const int64_t col = 16 * t + (l & 15);
  const int64_t row0 = kGroupRows * q + 32 * c + 8 * (l >> 4);
  const int64_t blob = block * bits / 8;
  const int per = 8 / bits;
  uint32_t word = 0;
  for (int j = 0; j < 8; ++j) {
    const int64_t row = row0 + j;
    uint32_t u = pad;
    if (row < K && col < N) {
      const int64_t g = row / block, jj = row % block;
      u = ((B[(col * groups + g) * blob + jj / per] >> (bits * (jj % per))) & ((1u << bits) - 1u)) + add;
    }
    word |= u << ((j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1));
  }
  out[idx] = word;
}

// 8-bit codes [N, groups, block] -> [K, N] bytes, xor `flip`.
__global__ void OrtBytesToRowsKernel(const uint8_t *__restrict__ B, int64_t K, int64_t N, int64_t block,
                                     int64_t groups, uint8_t flip, uint8_t *__restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= K * N) return;
  const int64_t r = e / N, n = e % N;
  out[e] = B[(n * groups + r / block) * block + r % block] ^ flip;
}

// scales [N, groups] -> [groups, N] (2-byte elements)
__global__ void OrtScaleTransposeKernel(const uint16_t *__restrict__ s, int64_t N, int64_t groups,
                                        uint16_t *__restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= N * groups) return;
  const int64_t g = e / N, n = e % N;
  out[e] = s[n * groups + g];
}

// zero points, packed `bits`-bit codes [N, zcol] -> [groups, N]: 4- and
// 2-bit codes as 4-bit ones two per byte, element g * N + n in the low nibble
// when even (ONNX packing); 8-bit one per byte.  One thread per output byte.
__global__ void OrtZeroPointsKernel(const uint8_t *__restrict__ z, int64_t N, int64_t groups, int64_t zcol,
                                    int bits, int64_t out_bytes, uint8_t *__restrict__ out) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= out_bytes) return;
  if (bits == 8) {
    const int64_t g = b / N, n = b % N;
    out[b] = z[n * zcol + g];
    return;
  }
  uint8_t v = 0;
  for (int h = 0; h < 2; ++h) {
    const int64_t e = 2 * b + h;
    if (e >= groups * N) break;
    const int64_t g = e / N, n = e % N;
    const int per = 8 / bits;
    const uint8_t code = (z[n * zcol + g / per] >> (bits * (g % per))) & ((1u << bits) - 1u);
    v |= (uint8_t)(code << (4 * h));
  }
  out[b] = v;
}

unsigned Blocks(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void LaunchPrepareNbits(const NbitsPrepParams &p, hipStream_t stream) {
  const int64_t groups = p.K / p.block;
  if (p.bits <= 4) {
    const int64_t ngroups = (p.K + kGroupRows - 1) / kGroupRows;
    const int64_t total = TiledInt4Bytes(p.K, p.N) / 4;
    // without zero points: INT4 offset binary of code - 2^(bits-1)
    const uint32_t add = p.zp ? 0u : 8u - (1u << (p.bits - 1));
    if (total > 0)
      hipLaunchKernelGGL(OrtTileInt4Kernel, dim3(Blocks(total)), dim3(256), 0, stream, p.B, p.K, p.N, p.block,
                         groups, ngroups, (int)p.bits, add, p.zp ? 0u : 8u, total, static_cast<uint32_t *>(p.weight));
  } else {
    if (p.K * p.N > 0)
      hipLaunchKernelGGL(OrtBytesToRowsKernel, dim3(Blocks(p.K * p.N)), dim3(256), 0, stream, p.B, p.K, p.N,
                         p.block, groups, (uint8_t)(p.zp ? 0 : 0x80), static_cast<uint8_t *>(p.weight));
  }
  if (p.N * groups > 0)
    hipLaunchKernelGGL(OrtScaleTransposeKernel, dim3(Blocks(p.N * groups)), dim3(256), 0, stream, p.scales, p.N,
                       groups, static_cast<uint16_t *>(p.scale_out));
  if (p.zp) {
    const int64_t zcol = (groups * p.bits + 7) / 8;
    const int64_t out_bytes = p.bits == 8 ? groups * p.N : (groups * p.N + 1) / 2;
    if (out_bytes > 0)
      hipLaunchKernelGGL(OrtZeroPointsKernel, dim3(Blocks(out_bytes)), dim3(256), 0, stream, p.zp, p.N, groups,
                         zcol, (int)p.bits, out_bytes, static_cast<uint8_t *>(p.zp_out));
  }
}

}  // namespace onnxl_amd
