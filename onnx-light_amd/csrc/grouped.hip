// GroupedMatMul (onnx-light opset 29): output[m, s, :] = input[m, :] @
// W[g] (+ bias[g]) with g = group_indices[m, s]; W[g] is [K, N], or [N, K]
// used transposed when transB != 0.  The MoE-shaped expert contraction.
//
// Two launches:
//  1. GroupRouteKernel (one workgroup) sorts the M * S (token, selection)
//     pairs by group: a count per group, an exclusive scan into the first
//     routed row and first GEMM tile of each group, then a scatter of the
//     pair indices.  The order of the pairs inside a group is arbitrary (LDS
//     atomics) and does not matter: each output row is computed by itself,
//     with the same summation order wherever it is routed.  Pairs whose group
//     index lies outside [0, G) get a NaN row (the reference raises; a call on
//     device-resident indices cannot report it before the work completes).
//  2. The MFMA GEMM core in grouped mode: each 256 x 128 tile belongs to one
//     group, gathers its A rows through the routing table, multiplies that
//     group's B (row-major [K, N], or [N, K] loaded and read like A) and
//     scatters its rows to Y.  Its grid is an upper bound of the tile count
//     (M * S / 256 + G tile-rows); workgroups past the routed tiles leave at
//     once.  Shapes the core does not take (K % 32 != 0, N % 16 != 0,
//     unaligned payloads) run GroupedSimpleKernel, one thread per output
//     element summing in order over k.
// The sums are fp32 over exact products of 16-bit values, as the reference's
// (km/kernel_grouped_matmul.cc:22-46); with a bias, the sum is rounded to the
// output dtype, the bias added in fp32 and the result rounded again.
#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"
#include "mfma_gemm.hpp"

namespace onnxl_amd {
namespace {

constexpr int kRouteThreads = 1024;

__device__ __forceinline__ int64_t GroupOf(const void *idx, int idx64, int64_t i) {
  return idx64 ? static_cast<const int64_t *>(idx)[i] : (int64_t) static_cast<const int32_t *>(idx)[i];
}

// One workgroup.  LDS: cnt[G], cursor[G] (dynamic), per-thread partial sums.
__global__ __launch_bounds__(kRouteThreads) void GroupRouteKernel(const GroupedParams p) {
  extern __shared__ int32_t lds[];
  int32_t *cnt = lds;            // [G]
  int32_t *cursor = lds + p.G;   // [G]
  __shared__ int32_t rsum[kRouteThreads], tsum[kRouteThreads];
  const int tid = threadIdx.x;
  const int G = p.G;
  const int64_t P = p.M * p.S;
  for (int g = tid; g < G; g += kRouteThreads) cnt[g] = 0;
  __syncthreads();
  for (int64_t i = tid; i < P; i += kRouteThreads) {
    const int64_t g = GroupOf(p.idx, p.idx64, i);
    if (g >= 0 && g < G) atomicAdd(&cnt[g], 1);
  }
  __syncthreads();
  // exclusive scans of the row counts and of the tile counts
  // (ceil(rows / 256) tile-rows of nbn tiles)
  const int per = (G + kRouteThreads - 1) / kRouteThreads;
  const int g0 = tid * per, g1 = min(G, g0 + per);
  int32_t rs = 0, ts = 0;
  for (int g = g0; g < g1; ++g) {
    rs += cnt[g];
    ts += (cnt[g] + mg::kBM - 1) / mg::kBM * p.nbn;
  }
  rsum[tid] = rs;
  tsum[tid] = ts;
  __syncthreads();
  for (int d = 1; d < kRouteThreads; d <<= 1) {  // inclusive Hillis-Steele scan
    const int32_t r = tid >= d ? rsum[tid - d] : 0, t = tid >= d ? tsum[tid - d] : 0;
    __syncthreads();
    rsum[tid] += r;
    tsum[tid] += t;
    __syncthreads();
  }
  int32_t rrun = rsum[tid] - rs, trun = tsum[tid] - ts;  // exclusive prefix of this thread's range
  for (int g = g0; g < g1; ++g) {
    p.row_off[g] = rrun;
    p.tile_off[g] = trun;
    cursor[g] = rrun;
    rrun += cnt[g];
    trun += (cnt[g] + mg::kBM - 1) / mg::kBM * p.nbn;
  }
  if (tid == kRouteThreads - 1) {
    p.row_off[G] = rsum[tid];
    p.tile_off[G] = tsum[tid];
  }
  __syncthreads();
  for (int64_t i = tid; i < P; i += kRouteThreads) {
    const int64_t g = GroupOf(p.idx, p.idx64, i);
    if (g >= 0 && g < G) {
      p.rows[atomicAdd(&cursor[g], 1)] = (int32_t)i;
    } else {
      uint16_t *y = static_cast<uint16_t *>(p.Y) + i * p.N;
      const uint16_t nan = p.bf16 ? 0x7fc0u : 0x7e00u;
      for (int64_t n = 0; n < p.N; ++n) y[n] = nan;
    }
  }
}

__device__ __forceinline__ float Dec(uint16_t h, bool bf16) {
  return bf16 ? __builtin_bit_cast(float, (uint32_t)h << 16) : (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t Enc(float f, bool bf16) {
  if (!bf16) return __builtin_bit_cast(uint16_t, (_Float16)f);
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                             // nearest even
  return (uint16_t)(u >> 16);
}

// One thread per output element: work item b covers columns 256 (b % nb) ..
// of pair b / nb, nb = ceil(N / 256); a grid of at most kSimpleMaxBlocks
// workgroups strides over the nb * pairs items, so any shape fits the grid.
constexpr int64_t kSimpleMaxBlocks = int64_t(1) << 20;

__global__ __launch_bounds__(256) void GroupedSimpleKernel(const GroupedParams p) {
  const int64_t nb = (p.N + 255) / 256;
  const int64_t items = nb * p.M * p.S;
  for (int64_t b = blockIdx.x; b < items; b += gridDim.x) {
    const int64_t i = b / nb;  // pair
    const int64_t n = (b % nb) * 256 + threadIdx.x;
    if (n >= p.N) continue;
    const int64_t g = GroupOf(p.idx, p.idx64, i);
    if (g < 0 || g >= p.G) continue;  // NaN row written by the routing kernel
    const uint16_t *x = static_cast<const uint16_t *>(p.A) + (i / p.S) * p.K;
    const uint16_t *w = static_cast<const uint16_t *>(p.W) + g * p.K * p.N;
    float v = 0.f;
    for (int64_t l = 0; l < p.K; ++l) {
      const uint16_t wb = p.transB ? w[n * p.K + l] : w[l * p.N + n];
      v = __fadd_rn(v, __fmul_rn(Dec(x[l], p.bf16), Dec(wb, p.bf16)));  // in order, no contraction
    }
    if (p.bias)
      v = __fadd_rn(Dec(Enc(v, p.bf16), p.bf16), Dec(static_cast<const uint16_t *>(p.bias)[g * p.N + n], p.bf16));
    static_cast<uint16_t *>(p.Y)[i * p.N + n] = Enc(v, p.bf16);
  }
}

// The quantized experts dequantized as the unfused chain does:
// DequantizeLinear's (x - zp) * scale in fp32, stored in the scale's dtype,
// then the optional Cast (kq/kernel_dequantizelinear.cc:57-63,259-285;
// kernel_cast.cc:360-370).  One thread per weight element, grid-stride.
__device__ __forceinline__ float QuantAt(const uint8_t *w, int dt, int64_t i) {
  switch (dt) {
  case kInt4: return (float)Int4ToInt((w[i >> 1] >> (4 * (i & 1))) & 0xfu);
  case kUint4: return (float)((w[i >> 1] >> (4 * (i & 1))) & 0xfu);
  case kInt8: return (float)(int8_t)w[i];
  case kUint8: return (float)w[i];
  default: return Fp8E4M3ToF32(w[i]);
  }
}

__global__ __launch_bounds__(256) void DequantExpertsKernel(const DqGroupedParams p, int64_t total) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t si = 0;
    if (p.scale_kind == 1) {
      si = (i / p.inner) % p.axis_dim;
    } else if (p.scale_kind == 2) {
      const int64_t o = i / (p.inner * p.axis_dim), a = (i / p.inner) % p.axis_dim, r = i % p.inner;
      si = (o * (p.axis_dim / p.block) + a / p.block) * p.inner + r;
    }
    const float s = p.scale_f16 ? F16ToF32(static_cast<const uint16_t *>(p.scale)[si])
                                : static_cast<const float *>(p.scale)[si];
    const float z = p.zp ? QuantAt(p.zp, p.x_dtype, si) : 0.f;
    const float v = (QuantAt(p.X, p.x_dtype, i) - z) * s;
    p.w16[i] = p.deq_round_f16 || p.cast_round != 16 ? F32ToF16(v) : F32ToBf16(v);
  }
}

}  // namespace

int64_t GroupedMaxTiles(const GroupedParams &p) {
  return ((p.M * p.S + mg::kBM - 1) / mg::kBM + p.G) * p.nbn;
}

size_t GroupedRouteLds(int64_t G) { return (size_t)(2 * G) * sizeof(int32_t); }

bool GroupedCoreEligible(const GroupedParams &p) {
  mg::GemmArgs g{};
  g.A = p.A;
  g.B = p.W;
  g.Y = p.Y;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  return mg::Eligible<mg::kH16>(g) && p.M * p.S * p.N * 2 < lim && p.N * p.K * 2 < lim &&
         (p.bias == nullptr || reinterpret_cast<uintptr_t>(p.bias) % 8 == 0);
}

void LaunchGroupedMatMul(const GroupedParams &p, hipStream_t stream) {
  const int64_t P = p.M * p.S;
  if (P == 0 || p.N == 0) return;
  hipLaunchKernelGGL(GroupRouteKernel, dim3(1), dim3(kRouteThreads), GroupedRouteLds(p.G), stream, p);
  if (p.K == 0 || !GroupedCoreEligible(p)) {
    const int64_t items = (p.N + 255) / 256 * P;
    hipLaunchKernelGGL(GroupedSimpleKernel, dim3((unsigned)std::min(items, kSimpleMaxBlocks)), dim3(256), 0, stream,
                       p);
    return;
  }
  mg::GemmArgs g{};
  g.A = p.A;
  g.B = p.W;
  g.Y = p.Y;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  g.batch = 1;
  g.grp_tile_off = p.tile_off;
  g.grp_row_off = p.row_off;
  g.grp_rows = p.rows;
  g.grp_count = (int)p.G;
  g.grp_sel = (int)p.S;
  g.grp_b_stride = p.K * p.N;
  g.grp_bias = p.bias;
  const int64_t tiles = GroupedMaxTiles(p);
  if (p.bf16) {
    if (p.transB) mg::LaunchGrouped<mg::kOutBf16, 2>(g, tiles, stream);
    else mg::LaunchGrouped<mg::kOutBf16, 1>(g, tiles, stream);
  } else {
    if (p.transB) mg::LaunchGrouped<mg::kOutF16, 2>(g, tiles, stream);
    else mg::LaunchGrouped<mg::kOutF16, 1>(g, tiles, stream);
  }
}

}  // namespace onnxl_amd

namespace onnxl_amd {

bool DqGroupedFusedEligible(const DqGroupedParams &p) {
  mg::GemmArgs g{};
  g.A = p.g.A;
  g.B = p.X;
  g.Y = p.g.Y;
  g.M = p.g.M;
  g.N = p.g.N;
  g.K = p.g.K;
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  return p.fused && !p.g.transB && p.g.bf16 && p.g.K > 0 && mg::Eligible<mg::kBf16F8>(g) &&
         p.g.M * p.g.S * p.g.N * 2 < lim && p.g.N * p.g.K < lim &&
         (p.g.bias == nullptr || reinterpret_cast<uintptr_t>(p.g.bias) % 8 == 0);
}

void LaunchDqGroupedMatMul(const DqGroupedParams &p, hipStream_t stream) {
  const int64_t P = p.g.M * p.g.S;
  if (P == 0 || p.g.N == 0) return;
  if (!DqGroupedFusedEligible(p)) {
    // general path: the weights dequantized into the workspace, then the
    // 16-bit grouped GEMM
    const int64_t total = p.g.G * p.g.K * p.g.N;
    if (total > 0) {
      const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
      hipLaunchKernelGGL(DequantExpertsKernel, dim3(blocks), dim3(256), 0, stream, p, total);
    }
    GroupedParams g = p.g;
    g.W = p.w16;
    LaunchGroupedMatMul(g, stream);
    return;
  }
  // 256 x 256 tiles (as configuration 4's fp8 GEMM) when K takes whole K
  // steps; the routing then counts 256-column tiles
  GroupedParams gp = p.g;
  const bool wide = p.g.K % 64 == 0;
  if (wide) gp.nbn = (p.g.N + 255) / 256;
  hipLaunchKernelGGL(GroupRouteKernel, dim3(1), dim3(kRouteThreads), GroupedRouteLds(gp.G), stream, gp);
  mg::GemmArgs g{};
  g.A = p.g.A;
  g.B = p.X;
  g.Y = p.g.Y;
  g.M = p.g.M;
  g.N = p.g.N;
  g.K = p.g.K;
  g.batch = 1;
  g.scale = p.scale;
  g.scale_f16 = p.scale_f16;
  g.scale_per_col = p.scale_per_col;
  g.scale_grp_stride = p.scale_grp_stride;
  g.grp_tile_off = p.g.tile_off;
  g.grp_row_off = p.g.row_off;
  g.grp_rows = p.g.rows;
  g.grp_count = (int)p.g.G;
  g.grp_sel = (int)p.g.S;
  g.grp_b_stride = p.g.K * p.g.N;
  g.grp_bias = p.g.bias;
  if (wide) mg::LaunchGrouped<mg::kOutBf16, 1, mg::kBf16F8, 4>(g, GroupedMaxTiles(gp), stream);
  else mg::LaunchGrouped<mg::kOutBf16, 1, mg::kBf16F8, 2>(g, GroupedMaxTiles(gp), stream);
}

}  // namespace onnxl_amd
