// EXL3 weights (the ai.rt:Dequantize encoding "onnx_light.exl3_weights.v1",
// GPTQModel's EXL3 module; onnx_core/runtime/exl3.cc) on the device.
//
// A [k, n] weight as 16 x 16 tiles of trellis-coded 16-bit states: tile t
// (tile row t / (n / 16), tile column t % (n / 16)) holds 16 * bits INT16
// words, a cyclic bit stream of 256 symbols of `bits` bits; position p's
// state is the 16-bit window ending at bit (p + 1) * bits (State,
// :222-231), its value a codebook function of the state rounded to binary16
// (Codebook, :205-220), its place in the tile (lane p / 8, item p % 8) the
// MMA fragment order of :331-334.  The value matrix then goes through
// normalised 128-point Walsh-Hadamard butterflies down each 128-row block of
// every column, a row scale suh, the same butterflies along each 128-column
// block of every row and a column scale svh (:337-354), every operation one
// fp32 rounding (Hadamard :233-245).
//
// Exl3DecodeKernel: one 256-thread workgroup per 128 x 128 block, which is
// closed under both transforms.  The block's 64 tiles decode into an LDS
// array of 128 rows x 129 floats (the odd pitch keeps both the column and
// the row butterflies on distinct banks), the column butterflies run in 7
// stages with a barrier between them, then the suh scale, the row
// butterflies and the svh scale, and the block is written row by row.  No
// multiply is contracted into an add: each step is a separate rounding, as
// the reference's volatile steps are.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

#pragma clang fp contract(off)

constexpr int kPitch = 129;
constexpr float kInvSqrt128 = 0.08838834764831845f;

__device__ __forceinline__ float Half(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// Codebook (:205-220): 3INST (book 0), MCG (1) and MUL1 (2) of a state,
// rounded to binary16.
__device__ __forceinline__ float Exl3Codebook(uint32_t state, int book) {
  float r;
  if (book < 2) {
    uint32_t raw = book == 0 ? state * 89226354u + 64248484u : state * 0xcbac1fedu;
    raw = 0x3b603b60u ^ (raw & 0x8fff8fffu);
    r = __fadd_rn(Half(raw & 0xffffu), Half(raw >> 16));  // exact: both halves are binary16
  } else {
    const uint32_t raw = state * 0x83dcd12du;
    const uint32_t sum = (raw & 255u) + ((raw >> 8) & 255u) + ((raw >> 16) & 255u) + (raw >> 24);
    r = __builtin_fmaf(Half(sum + 0x6400u), Half(0x1eeeu), Half(0xc931u));
  }
  return Half(F32ToF16(r));
}

// The 16-bit state of `position` in a tile stream of 16 * bits words (State,
// :222-231): words are taken at index ^ 1 (the 32-bit words' halves).
__device__ __forceinline__ uint32_t Exl3State(const uint16_t *__restrict__ s, uint32_t bits, uint32_t position) {
  const uint32_t words = 16u * bits, span = 256u * bits;
  const uint32_t start = ((position + 1u) * bits + span - 16u) % span;
  const uint32_t word = start / 16u, shift = start % 16u;
  uint32_t state = s[word ^ 1u];
  if (shift) state = ((state << shift) | ((uint32_t)s[((word + 1u) % words) ^ 1u] >> (16u - shift))) & 0xffffu;
  return state;
}

template <int OUT>
__global__ __launch_bounds__(256) void Exl3DecodeKernel(const Exl3Params p, void *__restrict__ y) {
  __shared__ float lds[128 * kPitch];  // 66,048 bytes
  const int t = threadIdx.x;
  const int64_t br = blockIdx.y, bc = blockIdx.x;  // 128-row block, 128-column block
  const int64_t tiles_per_row = p.n / 16;
  // decode: tile i of the block (8 x 8 tiles), position t
  const uint32_t lane = (uint32_t)t / 8u, item = (uint32_t)t % 8u;
  const int r_in = (int)((lane % 4u) * 2u + (item & 1u) + ((item & 2u) ? 8u : 0u));
  const int c_in = (int)(lane / 4u + ((item & 4u) ? 8u : 0u));
  for (int i = 0; i < 64; ++i) {
    const int tr = i / 8, tc = i % 8;
    const int64_t tile = (br * 8 + tr) * tiles_per_row + bc * 8 + tc;
    const uint16_t *s = p.trellis + tile * 16 * p.bits;
    lds[(tr * 16 + r_in) * kPitch + tc * 16 + c_in] = Exl3Codebook(Exl3State(s, (uint32_t)p.bits, (uint32_t)t), p.book);
  }
  __syncthreads();
  // butterflies down the columns: thread t takes column t % 128 and pairs
  // t / 128, + 2, + 4, ...
  const int col = t % 128, p0 = t / 128;
  for (int w = 1; w < 128; w *= 2) {
    for (int q = p0; q < 64; q += 2) {
      const int j = (q / w) * 2 * w + q % w;
      const float a = lds[j * kPitch + col], b = lds[(j + w) * kPitch + col];
      lds[j * kPitch + col] = __fadd_rn(a, b);
      lds[(j + w) * kPitch + col] = __fsub_rn(a, b);
    }
    __syncthreads();
  }
  // normalisation, then the row scale suh
  for (int r = p0; r < 128; r += 2) {
    const float u = Half(p.suh[br * 128 + r]);
    lds[r * kPitch + col] = __fmul_rn(__fmul_rn(lds[r * kPitch + col], kInvSqrt128), u);
  }
  __syncthreads();
  // butterflies along the rows: thread t takes row t % 128
  const int row = t % 128;
  for (int w = 1; w < 128; w *= 2) {
    for (int q = p0; q < 64; q += 2) {
      const int j = (q / w) * 2 * w + q % w;
      const float a = lds[row * kPitch + j], b = lds[row * kPitch + j + w];
      lds[row * kPitch + j] = __fadd_rn(a, b);
      lds[row * kPitch + j + w] = __fsub_rn(a, b);
    }
    __syncthreads();
  }
  // normalisation, the column scale svh, the output
  const float v_scale = Half(p.svh[bc * 128 + col]);
  unsigned flag = 0;
  for (int r = p0; r < 128; r += 2) {
    const float v = __fmul_rn(__fmul_rn(lds[r * kPitch + col], kInvSqrt128), v_scale);
    if (!__builtin_isfinite(v)) flag |= kExl3BadValue;
    const int64_t o = (br * 128 + r) * p.n + bc * 128 + col;
    if constexpr (OUT == kFloat) {
      static_cast<float *>(y)[o] = v;
    } else if constexpr (OUT == kDouble) {
      static_cast<double *>(y)[o] = (double)v;
    } else {
      const uint16_t h = OUT == kFloat16 ? F32ToF16(v) : F32ToBf16(v);
      const bool inf = OUT == kFloat16 ? (h & 0x7c00u) == 0x7c00u : (h & 0x7f80u) == 0x7f80u;
      if (inf && __builtin_isfinite(v)) flag |= kExl3BadOutput;
      static_cast<uint16_t *>(y)[o] = h;
    }
  }
  if (flag) atomicOr(p.flag, flag);
}

}  // namespace

void LaunchExl3Decode(const Exl3Params &p, int out_dtype, void *y, hipStream_t s) {
  const dim3 g((unsigned)(p.n / 128), (unsigned)(p.k / 128)), b(256);
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL((Exl3DecodeKernel<kFloat>), g, b, 0, s, p, y); break;
  case kDouble: hipLaunchKernelGGL((Exl3DecodeKernel<kDouble>), g, b, 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL((Exl3DecodeKernel<kFloat16>), g, b, 0, s, p, y); break;
  default: hipLaunchKernelGGL((Exl3DecodeKernel<kBfloat16>), g, b, 0, s, p, y); break;
  }
}

}  // namespace onnxl_amd
