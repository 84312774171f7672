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
//  - The 4 waves of a workgroup take consecutive K ranges of the same strip
//    and are reduced through LDS in a fixed order; when K is also split over
//    workgroups, each writes its fp32 partial and the last one to arrive (an
//    agent-scope counter per strip, reset by that workgroup) sums the
//    partials in slice order and stores fp16 (round to nearest even).
#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kStrip = 128;        // columns per workgroup
constexpr int kChunk = 32;         // k rows per MFMA
constexpr int kMaxChunks = 8;      // chunks per wave (all loads in flight at once)

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

// Zero-point nibble of column c (0..7) of a packed dword.
template <bool SIGNED> __device__ __forceinline__ int Nibble(uint32_t w, int c) {
  const int u = (int)((w >> (4 * c)) & 0xfu);
  return SIGNED ? ((u ^ 8) - 8) : u;
}

template <bool SIGNED, bool HAS_ZP>
__global__ __launch_bounds__(kThreads) void GemvQ4Kernel(const GemvArgs p) {
  __shared__ float red[4][16][kStrip];  // per-wave partial sums [wave][m][column]
  __shared__ unsigned last_flag;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int strip = blockIdx.x, slice = blockIdx.y;
  const int n0 = strip * kStrip + 8 * li;  // first of this lane's 8 columns
  const bool col_ok = n0 < p.N;
  const int nq = p.N >> 3;                 // dwords per packed row
  const int total = p.K / kChunk;
  const int c_begin = (slice * 4 + wave) * p.cpw;
  const int c_end = min(c_begin + p.cpw, total);
  const int nch = max(c_end - c_begin, 0);

  // ---- issue every load of this wave's K range ----
  uint32_t wq[kMaxChunks][8];
  v4i sc_raw[kMaxChunks];
  uint32_t zp_raw[kMaxChunks];
  v8h act[kMaxChunks];
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (c < nch) {
      const int k0 = (c_begin + c) * kChunk + 8 * g;  // first of this lane's 8 k rows
#pragma unroll
      for (int t = 0; t < 8; ++t)
        wq[c][t] = col_ok ? __builtin_nontemporal_load(p.W + (int64_t)(k0 + t) * nq + (n0 >> 3)) : 0u;
      int64_t si = 0;
      if (p.mode == 2) si = (int64_t)(k0 / p.blk) * p.N + n0;
      else if (p.mode == 1) si = n0;
      if (p.mode == 0) {
        const uint32_t s = *reinterpret_cast<const uint16_t *>(p.scale);
        const int s2 = (int)(s | (s << 16));
        sc_raw[c] = v4i{s2, s2, s2, s2};
        if (HAS_ZP) {
          const uint32_t z = *reinterpret_cast<const uint8_t *>(p.zp) & 0xfu;
          zp_raw[c] = z * 0x11111111u;
        }
      } else {
        sc_raw[c] = col_ok ? *reinterpret_cast<const v4i *>(p.scale + si) : v4i{0, 0, 0, 0};
        if (HAS_ZP) zp_raw[c] = col_ok ? p.zp[si >> 3] : 0u;
      }
      act[c] = li < p.M ? *reinterpret_cast<const v8h *>(p.A + (int64_t)li * p.K + k0) : v8h{};
    }
  }

  v4f acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    if (c < nch) {
      // per-column scale pair (s, s) and bias pair (1024 [+ 8] + zp)
      v2h sc2[8], sub2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = (uint32_t)sc_raw[c][e >> 1];
        const uint32_t h = (e & 1) ? (word >> 16) : (word & 0xffffu);
        sc2[e] = __builtin_bit_cast(v2h, h | (h << 16));
        const int bias = (SIGNED ? 1032 : 1024) + (HAS_ZP ? Nibble<SIGNED>(zp_raw[c], e) : 0);
        const _Float16 b = (_Float16)bias;  // exact: 1016 .. 1047
        sub2[e] = v2h{b, b};
      }
      uint32_t wk[8][4];  // [column][row pair]: fp16 (1024 + u) at rows 2p, 2p+1
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        uint32_t x0 = wq[c][2 * pr], x1 = wq[c][2 * pr + 1];
        if (SIGNED) {
          x0 ^= 0x88888888u;  // signed nibble s -> s + 8
          x1 ^= 0x88888888u;
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          // bytes: [x0.byte b, 0, x1.byte b, 0]  (selector 0x0c = zero byte)
          const uint32_t sel = 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
          const uint32_t pb = __builtin_amdgcn_perm(x1, x0, sel);
          wk[2 * b][pr] = (pb & 0x000f000fu) | 0x64006400u;
          wk[2 * b + 1][pr] = ((pb >> 4) & 0x000f000fu) | 0x64006400u;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v8h wop;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const v2h q = (__builtin_bit_cast(v2h, wk[e][pr]) - sub2[e]) * sc2[e];
          wop[2 * pr] = q.x;
          wop[2 * pr + 1] = q.y;
        }
        acc[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, act[c], acc[e], 0, 0, 0);
      }
    }
  }

  // ---- reduce the 4 waves: lane (li, g), register q holds row m = li of
  // strip columns 8 * (4g + q) + e ----
  if (li < p.M) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave][li][8 * (4 * g + q) + e] = acc[e][q];
  }
  __syncthreads();
  const int M = p.M;
  const bool split = p.slices > 1;
  for (int idx = threadIdx.x; idx < M * kStrip; idx += kThreads) {
    const int m = idx / kStrip, col = idx % kStrip;
    const int n = strip * kStrip + col;
    const float v = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
    if (n < p.N) {
      if (split) p.partial[((int64_t)slice * M + m) * p.N + n] = v;
      else p.Y[(int64_t)m * p.N + n] = (_Float16)v;
    }
  }
  if (!split) return;

  // ---- K split over workgroups: the last one to arrive sums the partials ----
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(p.counters + strip, 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(p.slices - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  for (int idx = threadIdx.x; idx < M * kStrip; idx += kThreads) {
    const int m = idx / kStrip, col = idx % kStrip;
    const int n = strip * kStrip + col;
    if (n < p.N) {
      float v = 0.f;
      for (int s = 0; s < p.slices; ++s)
        v += __builtin_nontemporal_load(p.partial + ((int64_t)s * M + m) * p.N + n);
      p.Y[(int64_t)m * p.N + n] = (_Float16)v;
    }
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(p.counters + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int Slices(const DqMatMulParams &p) {
  const int total = (int)(p.K / kChunk);
  return (total + 4 * kMaxChunks - 1) / (4 * kMaxChunks);
}

}  // namespace

bool GemvQ4Eligible(const DqMatMulParams &p) {
  const bool four = p.w_dtype == kInt4 || p.w_dtype == kUint4;
  return four && p.M >= 1 && p.M <= 16 && !p.a_bf16 && p.scale_f16 && p.deq_round_f16 &&
         p.cast_round == 0 && p.K % kChunk == 0 && p.N % 8 == 0 && p.K <= (1 << 30) &&
         p.N <= (1 << 30) && (p.mode != 2 || (p.block % 8 == 0)) &&
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
  g.cpw = (total + 4 * g.slices - 1) / (4 * g.slices);
  const dim3 grid((unsigned)((p.N + kStrip - 1) / kStrip), (unsigned)g.slices);
  const bool sgn = p.w_dtype == kInt4, zp = p.zp != nullptr;
  if (sgn) {
    if (zp) hipLaunchKernelGGL((GemvQ4Kernel<true, true>), grid, dim3(kThreads), 0, stream, g);
    else hipLaunchKernelGGL((GemvQ4Kernel<true, false>), grid, dim3(kThreads), 0, stream, g);
  } else {
    if (zp) hipLaunchKernelGGL((GemvQ4Kernel<false, true>), grid, dim3(kThreads), 0, stream, g);
    else hipLaunchKernelGGL((GemvQ4Kernel<false, false>), grid, dim3(kThreads), 0, stream, g);
  }
}

}  // namespace onnxl_amd
