// Decode-shaped fused DequantizeLinear(INT4 / UINT4, FLOAT16 scales) -> FLOAT16
// MatMul:  Y[M, N] = A[M, K] * W,  W[k, n] = fp16((x[k, n] - zp) * scale),
// for M <= 16 (one MFMA tile of activation rows).
//
// The weight stream dominates (K * N / 2 bytes read once), so the kernel is
// organised around HBM reads:
//  - A lane owns 8 consecutive columns (one dword of packed nibbles per k row)
//    and 8 consecutive k rows per 32-row chunk; 16 lanes span a 128-column
//    strip (64 contiguous bytes per k row), the 4 lane groups the 4 k groups.
//  - Dequantisation happens in registers.  Two k rows are merged byte-wise
//    with v_perm_b32 so that each 32-bit register holds the nibbles of one
//    column at rows k and k+1; OR-ing 0x6400 (fp16 1024) makes them exact fp16
//    values 1024 + u, a packed fp16 subtract of (1024 + bias + zero point)
//    recovers the integer, and a packed fp16 multiply by the column's scale
//    rounds exactly as fp16(float(q) * float(scale)) does (the fp32 product of
//    a 4-bit integer and an fp16 scale is exact, so one rounding remains).
//  - The decoded registers are already the A operand of
//    v_mfma_f32_16x16x32_f16 (row = column n of the strip, 8 consecutive k);
//    the activations are its B operand (column = row m of A).  Accumulation
//    is fp32.
//  - The 8 waves of a workgroup take consecutive K ranges of the same strip
//    and are reduced through LDS in a fixed order; when K is also split over
//    workgroups, each writes its fp32 partial and the last one to arrive (an
//    agent-scope counter per strip, reset by that workgroup) sums the
//    partials in slice order and stores fp16 (round to nearest even).  The
//    partials travel through agent-scope atomic loads and stores, which are
//    coherent across the XCDs' L2 caches without a cache-wide writeback.
#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kStrip = 128;        // columns per workgroup
constexpr int kChunk = 32;         // k rows per MFMA
constexpr int kMaxChunks = 4;      // chunks per wave (all loads in flight at once)
constexpr int kRedG = 33, kRedRow = 132;  // padded reduction layout

struct GemvArgs {
  const _Float16 *A;      // [M, K]
  const uint32_t *W;      // [K, N] packed 4-bit, N % 8 == 0 (rows are dword aligned)
  const _Float16 *scale;  // mode 2: [K / blk, N]; mode 1: [N]; mode 0: [1]
  const uint32_t *zp;     // packed 4-bit, same layout as scale, or nullptr
  _Float16 *Y;            // [M, N]
  float *partial;         // [slices, M, N] when slices > 1
  unsigned *counters;     // one per strip, zero between launches
  int M, N, K;
  int blk;                // k rows per scale row (mode 2)
  int mode;               // 0 per-tensor, 1 per-column, 2 blocked along K
  int slices;             // workgroups per strip along K
  int cpw;                // chunks per wave
};

// Nibbles of byte b of two k rows -> two fp16 pairs 0x6400 | u (= 1024 + u):
// column 2b at rows (r0, r1) and column 2b + 1 at rows (r0, r1).  `sel`
// gathers [x0.byte b, 0, x1.byte b, 0]; the AND-OR keeps one nibble per half
// and inserts the fp16 exponent of 1024.
__device__ __forceinline__ void DecodeBytePair(uint32_t x0, uint32_t x1, uint32_t sel, uint32_t mask,
                                               uint32_t magic, uint32_t &even, uint32_t &odd) {
  const uint32_t pb = __builtin_amdgcn_perm(x1, x0, sel);
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(even) : "v"(pb), "v"(mask), "v"(magic));
  const uint32_t sh = pb >> 4;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(odd) : "v"(sh), "v"(mask), "v"(magic));
}

constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = 0x80000000u;  // past every buffer: loads return zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kRsrcWord3);
}

template <bool SIGNED, bool HAS_ZP, int MODE>
__global__ __launch_bounds__(kThreads) void GemvQ4Kernel(const GemvArgs p) {
  // Per-wave partial sums; row m, strip column 8 * (4g + q) + e sits at
  // m * kRedRow + g * kRedG + 8q + e (padding makes the 64 lanes' writes hit 64
  // distinct banks).
  __shared__ float red[kWaves][16 * kRedRow];
  __shared__ unsigned last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int li = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin: give each XCD a run of
  // adjacent strips so the two halves of a 128-byte weight line (read by
  // neighbouring strips) meet in the same L2.
  // (XCD x owns the contiguous strips [x*base + min(x, extra), +count_x)).
  const int nstrips = gridDim.x;
  const int base = nstrips / 8, extra = nstrips % 8;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int strip = xcd * base + min(xcd, extra) + slot;
  const int slice = blockIdx.y;
  const int n0 = strip * kStrip + 8 * li;  // first of this lane's 8 columns
  const bool col_ok = n0 < p.N;
  const int64_t row_bytes = p.N >> 1;     // packed bytes per k row
  const int total = p.K / kChunk;
  const int c_begin = (slice * kWaves + wave) * p.cpw;
  const int nch = max(min(c_begin + p.cpw, total) - c_begin, 0);

  const int64_t s_rows = MODE == 2 ? p.K / p.blk : 1;
  const __amdgpu_buffer_rsrc_t rsW = Rsrc(p.W, (int64_t)p.K * row_bytes);
  const __amdgpu_buffer_rsrc_t rsS = Rsrc(p.scale, MODE == 0 ? 2 : s_rows * p.N * 2);
  const __amdgpu_buffer_rsrc_t rsZ = Rsrc(p.zp, HAS_ZP ? (MODE == 0 ? 1 : (s_rows * p.N) >> 1) : 0);
  const __amdgpu_buffer_rsrc_t rsA = Rsrc(p.A, (int64_t)p.M * p.K * 2);

  // ---- issue every load of this wave's K range (branch-free: out-of-range
  // lanes and chunks read from an offset past the buffer, which returns 0) ----
  uint32_t wq[kMaxChunks][8];
  v4i sc_raw[kMaxChunks];
  uint32_t zp_raw[kMaxChunks];
  v8h act[kMaxChunks];
  v4i sc_fixed = v4i{0, 0, 0, 0};
  uint32_t zp_fixed = 0;
  if constexpr (MODE == 0) {
    const uint32_t h = *static_cast<const uint16_t *>(static_cast<const void *>(p.scale));
    const int s2 = (int)(h | (h << 16));
    sc_fixed = v4i{s2, s2, s2, s2};
    if (HAS_ZP) zp_fixed = (*reinterpret_cast<const uint8_t *>(p.zp) & 0xfu) * 0x11111111u;
  } else if constexpr (MODE == 1) {
    sc_fixed = __builtin_amdgcn_raw_buffer_load_b128(rsS, col_ok ? (unsigned)n0 * 2u : kOob, 0, 0);
    if (HAS_ZP) zp_fixed = __builtin_amdgcn_raw_buffer_load_b32(rsZ, col_ok ? (unsigned)n0 >> 1 : kOob, 0, 0);
  }
  // Weight rows: the lane part of the offset is fixed, the row part is
  // wave-uniform and goes into the scalar offset (no per-load vector math).
  // Chunks past this wave's range re-read its first chunk (in bounds) and
  // meet zero activations.
  const unsigned w_lane = col_ok ? (unsigned)(8 * g * row_bytes + (n0 >> 1)) : kOob;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const bool live = c < nch;
    const int cc = live ? c_begin + c : min(c_begin, total - 1);
    const int k0 = cc * kChunk + 8 * g;  // first of this lane's 8 k rows
#pragma unroll
    for (int t = 0; t < 8; ++t)
      wq[c][t] = __builtin_amdgcn_raw_buffer_load_b32(
          rsW, w_lane, (int)((int64_t)(cc * kChunk + t) * row_bytes), 0);
    if constexpr (MODE == 2) {
      const int64_t si = (int64_t)(k0 / p.blk) * p.N + n0;
      sc_raw[c] = __builtin_amdgcn_raw_buffer_load_b128(rsS, col_ok ? (unsigned)(si * 2) : kOob, 0, 0);
      if (HAS_ZP) zp_raw[c] = __builtin_amdgcn_raw_buffer_load_b32(rsZ, col_ok ? (unsigned)(si >> 1) : kOob, 0, 0);
    }
    act[c] = __builtin_bit_cast(
        v8h, __builtin_amdgcn_raw_buffer_load_b128(
                 rsA, (live && li < p.M) ? (unsigned)(((int64_t)li * p.K + k0) * 2) : kOob, 0, 0));
  }
  if constexpr (MODE != 2) {
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
      sc_raw[c] = sc_fixed;
      zp_raw[c] = zp_fixed;
    }
  }

  v4f acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};

  const uint32_t mask = 0x000f000fu, magic = 0x64006400u;
  const uint32_t flip = SIGNED ? 0x88888888u : 0u;  // signed nibble s -> s + 8
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (c < nch) {  // wave-uniform
      // Per column e: scale pair (s_e, s_e) and bias pair (1024 + zb_e) twice,
      // zb = zero point (+ 8 for INT4, matching the weight's own offset), so
      // that (0x6400 | u) - bias = x - zp exactly.
      uint32_t sc2[8], bias2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = (uint32_t)sc_raw[c][e >> 1];
        sc2[e] = __builtin_amdgcn_perm(word, word, (e & 1) ? 0x03020302u : 0x01000100u);
      }
      if (HAS_ZP) {
        const uint32_t z = zp_raw[c] ^ flip;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          DecodeBytePair(z, z, 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b, mask, magic,
                         bias2[2 * b], bias2[2 * b + 1]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) bias2[e] = SIGNED ? 0x64086408u : 0x64006400u;  // 1032 / 1024
      }
      uint32_t wk[8][4];  // [column][row pair]: fp16 (1024 + u) at rows 2p, 2p+1
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        const uint32_t x0 = wq[c][2 * pr] ^ flip, x1 = wq[c][2 * pr + 1] ^ flip;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          DecodeBytePair(x0, x1, 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b, mask, magic,
                         wk[2 * b][pr], wk[2 * b + 1][pr]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v8h wop;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const v2h q = (__builtin_bit_cast(v2h, wk[e][pr]) - __builtin_bit_cast(v2h, bias2[e])) *
                        __builtin_bit_cast(v2h, sc2[e]);
          wop[2 * pr] = q.x;
          wop[2 * pr + 1] = q.y;
        }
        acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, act[c], acc[e], 0, 0, 0);
      }
    }
  }

  // ---- reduce the waves: lane (li, g), register q of acc[e] holds row m = li
  // of strip column 8 * (4g + q) + e ----
  if (li < p.M) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave][li * kRedRow + g * kRedG + 8 * q + e] = acc[e][q];
  }
  __syncthreads();
  const int M = p.M;
  const bool split = p.slices > 1;
  for (int idx = threadIdx.x; idx < M * kStrip; idx += kThreads) {
    const int m = idx / kStrip, col = idx % kStrip;
    const int n = strip * kStrip + col;
    const int ri = m * kRedRow + (col >> 5) * kRedG + 8 * ((col >> 3) & 3) + (col & 7);
    float v = red[0][ri];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += red[w][ri];  // fixed order
    if (n < p.N) {
      if (split) {
        // agent-scope atomic store: coherent across XCDs without a cache-wide fence
        __hip_atomic_store(p.partial + ((int64_t)slice * M + m) * p.N + n, v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      } else {
        p.Y[(int64_t)m * p.N + n] = (_Float16)v;
      }
    }
  }
  if (!split) return;

  // ---- K split over workgroups: the last one to arrive sums the partials.
  // The partials are written and read with agent-scope atomic accesses; every
  // wave waits for its stores to complete before the barrier that precedes the
  // counter update, so a workgroup that sees the final count reads complete
  // partials. ----
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(p.counters + strip, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(p.slices - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  for (int idx = threadIdx.x; idx < M * kStrip; idx += kThreads) {
    const int m = idx / kStrip, col = idx % kStrip;
    const int n = strip * kStrip + col;
    if (n < p.N) {
      float v = 0.f;
      for (int s = 0; s < p.slices; ++s)
        v += __hip_atomic_load(p.partial + ((int64_t)s * M + m) * p.N + n, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      p.Y[(int64_t)m * p.N + n] = (_Float16)v;
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(p.counters + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int Slices(const DqMatMulParams &p) {
  const int total = (int)(p.K / kChunk);
  return (total + kWaves * kMaxChunks - 1) / (kWaves * kMaxChunks);
}

}  // namespace

bool GemvQ4Eligible(const DqMatMulParams &p) {
  const bool four = p.w_dtype == kInt4 || p.w_dtype == kUint4;
  return four && p.M >= 1 && p.M <= 16 && !p.a_bf16 && p.scale_f16 && p.deq_round_f16 &&
         p.cast_round == 0 && p.K % kChunk == 0 && p.N % 8 == 0 &&
         p.K * p.N / 2 < (int64_t(1) << 31) - 64 && p.M * p.K * 2 < (int64_t(1) << 31) - 64 && (p.mode != 2 || (p.block % 8 == 0)) &&
         reinterpret_cast<uintptr_t>(p.A) % 16 == 0 && reinterpret_cast<uintptr_t>(p.W) % 4 == 0 &&
         reinterpret_cast<uintptr_t>(p.scale) % 16 == 0;
}

size_t GemvQ4ScratchBytes(const DqMatMulParams &p) {
  const int s = Slices(p);
  return s > 1 ? (size_t)s * p.M * p.N * sizeof(float) : 0;
}

size_t GemvQ4Counters(const DqMatMulParams &p) { return (size_t)((p.N + kStrip - 1) / kStrip); }

void LaunchGemvQ4(const DqMatMulParams &p, void *scratch, unsigned *counters, hipStream_t stream) {
  GemvArgs g{};
  g.A = static_cast<const _Float16 *>(p.A);
  g.W = reinterpret_cast<const uint32_t *>(p.W);
  g.scale = static_cast<const _Float16 *>(p.scale);
  g.zp = reinterpret_cast<const uint32_t *>(p.zp);
  g.Y = static_cast<_Float16 *>(p.Y);
  g.partial = static_cast<float *>(scratch);
  g.counters = counters;
  g.M = (int)p.M;
  g.N = (int)p.N;
  g.K = (int)p.K;
  g.blk = (int)(p.mode == 2 ? p.block : p.K);
  g.mode = p.mode;
  g.slices = Slices(p);
  const int total = (int)(p.K / kChunk);
  g.cpw = (total + kWaves * g.slices - 1) / (kWaves * g.slices);
  const dim3 grid((unsigned)((p.N + kStrip - 1) / kStrip), (unsigned)g.slices);
  const bool sgn = p.w_dtype == kInt4, zp = p.zp != nullptr;
  const int sel = (sgn ? 4 : 0) | (zp ? 2 : 0);
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, stream, g); };
  switch (p.mode * 8 + sel) {
  case 0: go(GemvQ4Kernel<false, false, 0>); break;
  case 2: go(GemvQ4Kernel<false, true, 0>); break;
  case 4: go(GemvQ4Kernel<true, false, 0>); break;
  case 6: go(GemvQ4Kernel<true, true, 0>); break;
  case 8: go(GemvQ4Kernel<false, false, 1>); break;
  case 10: go(GemvQ4Kernel<false, true, 1>); break;
  case 12: go(GemvQ4Kernel<true, false, 1>); break;
  case 14: go(GemvQ4Kernel<true, true, 1>); break;
  case 16: go(GemvQ4Kernel<false, false, 2>); break;
  case 18: go(GemvQ4Kernel<false, true, 2>); break;
  case 20: go(GemvQ4Kernel<true, false, 2>); break;
  default: go(GemvQ4Kernel<true, true, 2>); break;
  }
}

}  // namespace onnxl_amd
