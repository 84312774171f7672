// bitsandbytes weights (the encoding "onnx_light.bitsandbytes_weights.v1" of
// ai.rt:Dequantize, onnx_core/runtime/bitsandbytes.cc) on the device.
//
// A weight of logical shape [rows, cols], flattened row-major.  nf4 / fp4:
// element i is the 4-bit code (codes[i / 2] >> (i % 2 ? 0 : 4)) & 15, its
// value table[code] * scale rounded to fp32 (:523-526), one scale per
// `block` consecutive elements: absmax[b], or with nested statistics
// fp32(fp32(nested_map[absmax[b]] * nested_absmax[b / 256]) + offset)
// (Scale, :339-346).  int8: the signed byte times its row's scale
// fp32(scb[row] / 127) (:519).  FLOAT16 / BFLOAT16 outputs round the fp32
// value to nearest even; a value that is not finite there (or in fp32) is the
// reference's "bitsandbytes nonfinite reconstruction." error, which the
// kernels report through a flag word.
//
// Kernels:
//  - BnbScalesKernel: one thread per block resolves its scale (the nested
//    form included) and flags an invalid FLOAT absmax (CheckParameters,
//    :348-379: finite and >= 0) or a scale that is not finite;
//  - BnbDecodeKernel: 8 consecutive values per thread into FLOAT, FLOAT16 or
//    BFLOAT16 (or into nothing: the finiteness check alone);
//  - BnbGemvKernel: y[m, n] = sum_k a[m, k] * W[n, k] for FLOAT16
//    activations and 4-bit codes, W the FLOAT16 decode above.  A workgroup
//    computes 16 outputs, 4 per wave; a lane takes 32 consecutive values of
//    each of its 4 rows per step (one 16-byte load of codes, one scale: 32
//    divides the block), so a wave covers 2048 values of a row per step, the
//    next step's loads in flight during this one's decode.  Per row and step
//    the lane builds the 16 possible FLOAT16 weights of the block,
//    fp16(fp32(table[j] * scale)), as two byte planes of 4 dwords (low and
//    high bytes); v_perm_b32 looks four codes up at once in each half of a
//    plane (codes & 7 select among 8 bytes) and a second v_perm_b32 picks the
//    half by bit 3 of each code.  The 16-bit weights of elements 2j and 2j+2
//    (high nibbles) and 2j+1 and 2j+3 (low nibbles) form the fp16 pairs, the
//    activations are paired the same way with v_perm_b32 (shared by the 4
//    rows), and v_dot2_f32_f16 accumulates in fp32.  The weights are exactly
//    the chain's; only the summation order differs.
#include <algorithm>

#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"

// the reference rounds the nested product, the offset sum and each value
// separately (its volatile float steps): no contraction into FMAs
#pragma clang fp contract(off)

namespace onnxl_amd {
namespace {

// nf4 (quantization.cc:126-141, as float) and fp4 (bitsandbytes' fp4 table
// over 12, bitsandbytes.cc:331-333), native index order
template <int FMT> __device__ __forceinline__ constexpr float BnbCode(int j) {
  constexpr float nf4[16] = {(float)-1.0,
                             (float)-0.6961928009986877,
                             (float)-0.5250730514526367,
                             (float)-0.39491748809814453,
                             (float)-0.28444138169288635,
                             (float)-0.18477343022823334,
                             (float)-0.09105003625154495,
                             (float)0.0,
                             (float)0.07958029955625534,
                             (float)0.16093020141124725,
                             (float)0.24611230194568634,
                             (float)0.33791524171829224,
                             (float)0.44070982933044434,
                             (float)0.5626170039176941,
                             (float)0.7229568362236023,
                             (float)1.0};
  constexpr float fp4[16] = {0.f, 1.f / 192, 2.f / 3, 1.f,  1.f / 3,  0.5f,  1.f / 6,  0.25f,
                             0.f, -1.f / 192, -2.f / 3, -1.f, -1.f / 3, -0.5f, -1.f / 6, -0.25f};
  return FMT == 0 ? nf4[j] : fp4[j];
}

// the same tables for run-time indices
__constant__ float kBnbTable[2][16] = {
    {BnbCode<0>(0), BnbCode<0>(1), BnbCode<0>(2), BnbCode<0>(3), BnbCode<0>(4), BnbCode<0>(5), BnbCode<0>(6),
     BnbCode<0>(7), BnbCode<0>(8), BnbCode<0>(9), BnbCode<0>(10), BnbCode<0>(11), BnbCode<0>(12), BnbCode<0>(13),
     BnbCode<0>(14), BnbCode<0>(15)},
    {BnbCode<1>(0), BnbCode<1>(1), BnbCode<1>(2), BnbCode<1>(3), BnbCode<1>(4), BnbCode<1>(5), BnbCode<1>(6),
     BnbCode<1>(7), BnbCode<1>(8), BnbCode<1>(9), BnbCode<1>(10), BnbCode<1>(11), BnbCode<1>(12), BnbCode<1>(13),
     BnbCode<1>(14), BnbCode<1>(15)}};

__device__ __forceinline__ bool Finite(float v) { return __builtin_isfinite(v); }

__global__ __launch_bounds__(256) void BnbScalesKernel(const BnbParams p) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= p.blocks) return;
  unsigned bad = 0;
  float m;
  if (p.format == 2 || !p.nested) {
    m = static_cast<const float *>(p.absmax)[b];
    if (!(Finite(m) && m >= 0.f)) bad |= kBnbBadAbsmax;
  } else {
    const float prod = p.nested_map[static_cast<const uint8_t *>(p.absmax)[b]] * p.nested_absmax[b >> 8];
    if (!Finite(prod)) bad |= kBnbBadScale;
    m = prod + p.offset;
    if (!Finite(m)) bad |= kBnbBadScale;
  }
  if (p.format == 2) {
    m = m / 127.f;
    if (!Finite(m)) bad |= kBnbBadScale;
  }
  if (p.scales) p.scales[b] = m;
  if (bad) atomicOr(p.flag, bad);
}

// OUT: kFloat, kFloat16, kBfloat16, or 0 (the fp32 finiteness check only);
// y == nullptr checks the values in OUT without storing them
template <int OUT>
__global__ __launch_bounds__(256) void BnbDecodeKernel(const BnbParams p, void *__restrict__ y) {
  __shared__ float table[16];
  if (threadIdx.x < 16) table[threadIdx.x] = kBnbTable[p.format & 1][threadIdx.x];
  __syncthreads();
  const int64_t count = p.rows * p.cols;
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= count) return;
  float v[8];
  unsigned bad = 0;
  if (p.format == 2) {
    int64_t row = i0 / p.cols, next = (row + 1) * p.cols;
    float s = p.scales[row];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t i = i0 + e;
      if (i >= count) {
        v[e] = 0.f;
        continue;
      }
      if (i == next) {
        ++row;
        next += p.cols;
        s = p.scales[row];
      }
      v[e] = (float)(int8_t)p.codes[i] * s;
    }
  } else {
    const float s = p.scales[i0 >> p.block_shift];  // 8 divides the block
    const int64_t nbytes = (count + 1) / 2;
    uint32_t w = 0;  // the 4 code bytes of these 8 values (those past the weight read as 0)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((i0 >> 1) + j < nbytes) w |= (uint32_t)p.codes[(i0 >> 1) + j] << (8 * j);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t code = (w >> (8 * (e >> 1) + ((e & 1) ? 0 : 4))) & 15u;
      v[e] = i0 + e < count ? table[code] * s : 0.f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (!Finite(v[e])) bad = 1;
  const bool full = i0 + 8 <= count;
  if (y == nullptr) {  // the finiteness check alone: convert, store nothing
    if constexpr (OUT == kFloat16 || OUT == kBfloat16) {
      const uint16_t em = OUT == kFloat16 ? 0x7c00u : 0x7f80u;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (((OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e])) & em) == em) bad = 1;
    }
  } else if constexpr (OUT == kFloat) {
    float *yo = static_cast<float *>(y) + i0;
    if (full && (reinterpret_cast<uintptr_t>(yo) & 15) == 0) {
      reinterpret_cast<float4 *>(yo)[0] = float4{v[0], v[1], v[2], v[3]};
      reinterpret_cast<float4 *>(yo)[1] = float4{v[4], v[5], v[6], v[7]};
    } else {
      for (int e = 0; e < 8 && i0 + e < count; ++e) yo[e] = v[e];
    }
  } else if constexpr (OUT == kFloat16 || OUT == kBfloat16) {
    uint16_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[e] = OUT == kFloat16 ? F32ToF16(v[e]) : F32ToBf16(v[e]);
      const uint16_t em = OUT == kFloat16 ? 0x7c00u : 0x7f80u;
      if ((h[e] & em) == em) bad = 1;
    }
    uint16_t *yo = static_cast<uint16_t *>(y) + i0;
    if (full && (reinterpret_cast<uintptr_t>(yo) & 15) == 0) {
      typedef unsigned v4u __attribute__((ext_vector_type(4)));
      *reinterpret_cast<v4u *>(yo) = v4u{h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16,
                                         h[4] | (uint32_t)h[5] << 16, h[6] | (uint32_t)h[7] << 16};
    } else {
      for (int e = 0; e < 8 && i0 + e < count; ++e) yo[e] = h[e];
    }
  }
  if (bad) atomicOr(p.flag, kBnbBadValue);
}

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t AsH2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }

// The 16 FLOAT16 weights of a block with scale s as byte planes: lo[d] holds
// the low bytes of entries 4d .. 4d+3, hi[d] their high bytes.  The prepared
// weight's values are finite in FLOAT16, so the hardware conversion (round
// to nearest even, v_cvt_pk_f16_f32 on pairs) needs no NaN handling.
template <int FMT> __device__ __forceinline__ void BuildPlanes(float s, uint32_t lo[4], uint32_t hi[4]) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  uint32_t pr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f2_t v = {BnbCode<FMT>(2 * i) * s, BnbCode<FMT>(2 * i + 1) * s};
    pr[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2_t));
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    lo[d] = __builtin_amdgcn_perm(pr[2 * d + 1], pr[2 * d], 0x06040200u);
    hi[d] = __builtin_amdgcn_perm(pr[2 * d + 1], pr[2 * d], 0x07050301u);
  }
}

// (x & mask) | bits in one v_and_or_b32 (the compiler splits it otherwise)
__device__ __forceinline__ uint32_t AndOr(uint32_t x, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(bits));
  return r;
}

// Four codes -> the low and high bytes of their weights.  sel: each code's
// bits 0-2 (one per byte); pick: byte j is j, plus 4 when the code's bit 3
// is set (the entries 8-15 lookup).
__device__ __forceinline__ void Lookup4(uint32_t sel, uint32_t pick, const uint32_t lo[4], const uint32_t hi[4],
                                        uint32_t &l, uint32_t &h) {
  const uint32_t la = __builtin_amdgcn_perm(lo[1], lo[0], sel), lb = __builtin_amdgcn_perm(lo[3], lo[2], sel);
  const uint32_t ha = __builtin_amdgcn_perm(hi[1], hi[0], sel), hb = __builtin_amdgcn_perm(hi[3], hi[2], sel);
  l = __builtin_amdgcn_perm(lb, la, pick);
  h = __builtin_amdgcn_perm(hb, ha, pick);
}

constexpr int kBnbRows = 16;  // outputs per workgroup, 4 per wave

template <int FMT, int M>
__global__ __launch_bounds__(256) void BnbGemvKernel(const uint16_t *__restrict__ a, const uint8_t *__restrict__ codes,
                                                     const float *__restrict__ scales, int64_t N, int64_t K,
                                                     int block_shift, uint16_t *__restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kBnbRows + wave * 4;
  int64_t row[4];  // rows past N decode the last and are not stored
#pragma unroll
  for (int r = 0; r < 4; ++r) row[r] = n0 + r < N ? n0 + r : N - 1;
  float acc[4][M];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.f;
  const int64_t nsteps = (K + 2047) / 2048;
  v4u cw[4], cwn[4], av[M][4], avn[M][4];
  float sc[4], scn[4];
  auto load = [&](int64_t st, v4u (&c)[4], float (&s)[4], v4u (&act)[M][4]) __attribute__((always_inline)) {
    int64_t k0 = st * 2048 + 32 * lane;
    if (k0 >= K) k0 = 0;  // an idle lane reloads the start and adds nothing
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      c[r] = *reinterpret_cast<const v4u *>(codes + ((row[r] * K + k0) >> 1));  // 16-byte aligned
      s[r] = scales[(row[r] * K + k0) >> block_shift];
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) act[m][q] = *reinterpret_cast<const v4u *>(a + m * K + k0 + 8 * q);
  };
  load(0, cw, sc, av);
  for (int64_t st = 0; st < nsteps; ++st) {
    const bool live = st * 2048 + 32 * lane < K;
    if (st + 1 < nsteps) load(st + 1, cwn, scn, avn);
    if (live) {
      // activation pairs (a[2j], a[2j + 2]) and (a[2j + 1], a[2j + 3]) of each 8-value group
      uint32_t ae[M][4][2], ao[M][4][2];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t x0 = av[m][q][2 * h], x1 = av[m][q][2 * h + 1];  // (a[4h], a[4h+1]), (a[4h+2], a[4h+3])
            ae[m][q][h] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
            ao[m][q][h] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
          }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t lo[4], hi[4];
        BuildPlanes<FMT>(sc[r], lo, hi);
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // 8 values: byte j holds element 2j (high nibble) and 2j + 1 (low)
          const uint32_t w = cw[r][q];
          uint32_t el, eh, ol, oh;
          // high nibbles: bits 4-6 and 7 of each byte; low nibbles: bits 0-2 and 3
          Lookup4((w >> 4) & 0x07070707u, AndOr(w >> 5, 0x04040404u, 0x03020100u), lo, hi, el, eh);
          Lookup4(w & 0x07070707u, AndOr(w >> 1, 0x04040404u, 0x03020100u), lo, hi, ol, oh);
          const uint32_t e01 = __builtin_amdgcn_perm(eh, el, 0x05010400u);  // (w[0], w[2])
          const uint32_t e23 = __builtin_amdgcn_perm(eh, el, 0x07030602u);  // (w[4], w[6])
          const uint32_t o01 = __builtin_amdgcn_perm(oh, ol, 0x05010400u);  // (w[1], w[3])
          const uint32_t o23 = __builtin_amdgcn_perm(oh, ol, 0x07030602u);  // (w[5], w[7])
#pragma unroll
          for (int m = 0; m < M; ++m) {
            float t = acc[r][m];
            t = __builtin_amdgcn_fdot2(AsH2(ae[m][q][0]), AsH2(e01), t, false);
            t = __builtin_amdgcn_fdot2(AsH2(ae[m][q][1]), AsH2(e23), t, false);
            t = __builtin_amdgcn_fdot2(AsH2(ao[m][q][0]), AsH2(o01), t, false);
            t = __builtin_amdgcn_fdot2(AsH2(ao[m][q][1]), AsH2(o23), t, false);
            acc[r][m] = t;
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      cw[r] = cwn[r];
      sc[r] = scn[r];
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) av[m][q] = avn[m][q];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
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

}  // namespace

void LaunchBnbScales(const BnbParams &p, hipStream_t s) {
  if (p.blocks == 0) return;
  hipLaunchKernelGGL(BnbScalesKernel, dim3((unsigned)((p.blocks + 255) / 256)), dim3(256), 0, s, p);
}

void LaunchBnbDecode(const BnbParams &p, int out_dtype, void *y, hipStream_t s) {
  const int64_t threads = (p.rows * p.cols + 7) / 8;
  if (threads == 0) return;
  const dim3 g((unsigned)((threads + 255) / 256));
  switch (out_dtype) {
  case kFloat: hipLaunchKernelGGL(BnbDecodeKernel<kFloat>, g, dim3(256), 0, s, p, y); break;
  case kFloat16: hipLaunchKernelGGL(BnbDecodeKernel<kFloat16>, g, dim3(256), 0, s, p, y); break;
  case kBfloat16: hipLaunchKernelGGL(BnbDecodeKernel<kBfloat16>, g, dim3(256), 0, s, p, y); break;
  default: hipLaunchKernelGGL(BnbDecodeKernel<0>, g, dim3(256), 0, s, p, y); break;
  }
}

bool BnbGemvEligible(int format, int64_t M, int64_t N, int64_t K, int64_t block, const void *a, const void *codes) {
  return (format == 0 || format == 1) && M >= 1 && M <= 4 && K % 32 == 0 && K % block == 0 &&
         reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(codes) % 16 == 0 && N > 0;
}

void LaunchBnbGemv(int format, const uint16_t *a, const uint8_t *codes, const float *scales, int64_t M, int64_t N,
                   int64_t K, int64_t block, uint16_t *y, hipStream_t s) {
  const dim3 g((unsigned)((N + kBnbRows - 1) / kBnbRows));
  const int sh = __builtin_ctzll((unsigned long long)block);
#define OLA_BNB(FMT)                                                                                             \
  switch (M) {                                                                                                   \
  case 1: hipLaunchKernelGGL((BnbGemvKernel<FMT, 1>), g, dim3(256), 0, s, a, codes, scales, N, K, sh, y); break; \
  case 2: hipLaunchKernelGGL((BnbGemvKernel<FMT, 2>), g, dim3(256), 0, s, a, codes, scales, N, K, sh, y); break; \
  case 3: hipLaunchKernelGGL((BnbGemvKernel<FMT, 3>), g, dim3(256), 0, s, a, codes, scales, N, K, sh, y); break; \
  default: hipLaunchKernelGGL((BnbGemvKernel<FMT, 4>), g, dim3(256), 0, s, a, codes, scales, N, K, sh, y); break; \
  }
  if (format == 0) {
    OLA_BNB(0)
  } else {
    OLA_BNB(1)
  }
#undef OLA_BNB
}

}  // namespace onnxl_amd
