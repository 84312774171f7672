// Decode-shaped fused DequantizeLinear(INT4 / UINT4, FLOAT16 scales) -> FLOAT16
// MatMul on the tiled 4-bit weight layout (kernels.hpp, TiledInt4Bytes), the
// form a session prepares once for a constant weight (the way the reference
// Gemm kernel packs its constant B at preparation time,
// km/kernel_gemm.cc:378-405).
//
// With the ONNX row-major packing a workgroup can only read a long K range of
// a column strip as short row segments, so the K loop has to be split over
// workgroups and their partial sums reduced through memory.  In the tiled
// layout the full K range of a 16-column tile is one contiguous run, so:
//  - a workgroup owns T adjacent tiles over all of K (no split over
//    workgroups, no partial sums in memory); T is chosen so that the strips
//    spread over about 256 workgroups, one per CU;
//  - its 4 waves (one per SIMD) take consecutive 128-row groups, keeping two
//    groups' loads in flight, and each load instruction reads 1 KiB of
//    contiguous weight bytes (a 16-byte lane = 4 chunks of 8 k rows of one
//    column).  The decode is VALU-bound, and two waves sharing a SIMD left it
//    idle while both waited for data;
//  - a lane's dword already holds 8 consecutive k rows of one column with the
//    nibbles of rows 2j and 2j+1 at bits 4j and 16+4j, so one AND-OR yields
//    an fp16 pair of two rows: the A operand of v_mfma_f32_16x16x32_f16 needs
//    no byte permutation.  Pairs 0 and 2 (nibbles at bits 0-3 of each half)
//    OR into 0x6400 (1024, unit step 1) to give 1024 + u; pairs 1 and 3
//    (bits 4-7) OR into 0x5400 (64, step 1/16) to give 64 + u without a
//    shift; pairs 2 and 3 take the dword shifted right by 8.  One shift and
//    four AND-ORs per dword;
//  - the dequantised value is rounded exactly as the unfused chain rounds it:
//    (1024 + u) - (1024 + offset + zp) and (64 + u) - (64 + offset + zp) are
//    the exact integer x - zp, and one packed fp16 multiply by the scale
//    rounds fp16(float(x - zp) * scale) (the fp32 product of a 5-bit integer
//    and an fp16 scale is exact);
//  - the waves' fp32 partial sums are reduced through LDS in a fixed order
//    and stored as fp16 (round to nearest even).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;             // one wave per SIMD: no two waves of a CU compete for its VALU
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupRows = 128;      // k rows per 1 KiB group of a tile
constexpr int kGroupBytes = 1024;
constexpr int kDepth = 2;            // row groups whose loads are in flight ahead of use
constexpr int kMaxTiles = 4;         // tiles per workgroup
constexpr int kTargetGroups = 256;   // workgroups wanted: one per CU

constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = 0x80000000u;  // past every buffer: loads return zero, stores drop
// Cache policy of the weight loads: non-temporal (each weight byte is read
// once per call).  Measured on configuration 3: 8.2 us against 8.6-8.9 us
// with the default policy; the best plain read of the same bytes also uses
// it.
constexpr int kStreamPolicy = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kRsrcWord3);
}

struct TiledArgs {
  const _Float16 *A;      // [M, K]
  const uint8_t *W;       // tiled layout
  const _Float16 *scale;  // mode 2: [K / blk, N]; mode 1: [N]; mode 0: [1]
  const uint8_t *zp;      // 4-bit zero points in the scale's shape (ONNX packing), or nullptr
  _Float16 *Y;            // [M, N]
  int M, N, K;
  int blk_shift;          // log2 of the k rows per scale row (mode 2; a power of two >= 8)
  int ntiles;             // ceil(N / 16)
  int ngroups;            // ceil(K / 128)
  uint32_t bias2;         // fp16 pair 1024 + offset (8 for INT4, 0 for UINT4), no zero point
};

// fp16 pair of rows 2j, 2j+1 from a tiled dword w (w8 = w >> 8): 1024 + u
// for even j, 64 + u for odd j.
template <int J> __device__ __forceinline__ uint32_t RowPair(uint32_t w, uint32_t w8) {
  const uint32_t x = J < 2 ? w : w8;
  const uint32_t mask = J & 1 ? 0x00f000f0u : 0x000f000fu;
  const uint32_t magic = J & 1 ? 0x54005400u : 0x64006400u;
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(magic));
  return r;
}

// The bias of the odd pairs (64 + offset + zp) from that of the even pairs
// (0x6400 + offset + zp as fp16 bits): the integer moves to bits 4-7.
__device__ __forceinline__ uint32_t OddBias(uint32_t b) { return 0x5400u + ((b - 0x6400u) << 4); }

// MODE: 0 per-tensor, 1 per-column, 2 blocked along K, 3 blocked with blocks
// of 128 rows or more (one scale row per 128-row group, loaded once).
template <int T, bool HAS_ZP, bool SIGNED, int MODE>
__global__ __launch_bounds__(kThreads) void GemvQ4TiledKernel(const TiledArgs p) {
  constexpr bool kBlocked = MODE >= 2;
  constexpr int kPitch = 16 * T + 4;  // floats per activation row of a wave's partial sums
  __shared__ __attribute__((aligned(16))) float red[kWaves][16][kPitch];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int li = lane & 15, g = lane >> 4;
  const int tile0 = blockIdx.x * T;
  // this wave's 128-row groups [gb, gb + ng)
  const int gb = wave * p.ngroups / kWaves;
  const int ng = (wave + 1) * p.ngroups / kWaves - gb;
  const int64_t tile_bytes = (int64_t)p.ngroups * kGroupBytes;
  const int64_t s_rows = kBlocked ? p.K >> p.blk_shift : 1;

  const __amdgpu_buffer_rsrc_t rsW = Rsrc(p.W, p.ntiles * tile_bytes);
  const __amdgpu_buffer_rsrc_t rsA = Rsrc(p.A, (int64_t)p.M * p.K * 2);
  const __amdgpu_buffer_rsrc_t rsS = Rsrc(p.scale, kBlocked ? s_rows * p.N * 2 : (MODE == 1 ? p.N * 2 : 2));
  const __amdgpu_buffer_rsrc_t rsZ =
      Rsrc(p.zp, HAS_ZP ? (kBlocked ? (s_rows * p.N + 1) / 2 : (MODE == 1 ? (p.N + 1) / 2 : 1)) : 0);

  int col[T];
  unsigned w_lane[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int tl = tile0 + t;
    col[t] = 16 * tl + li;
    w_lane[t] = tl < p.ntiles ? (unsigned)(tl * tile_bytes + lane * 16) : kOob;
  }
  // zero-point nibble of an even / odd column (N is even when there are zero points)
  const int zsh = (li & 1) * 4;

  // Per-column scale and bias pairs that do not change along K (modes 0 and 1).
  uint32_t sfix[T], bfix[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    sfix[t] = 0;
    bfix[t] = p.bias2;
    if constexpr (!kBlocked) {
      const unsigned so = MODE == 1 ? (unsigned)min(col[t], p.N - 1) * 2u : 0u;
      const uint32_t s = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsS, so, 0, 0);
      sfix[t] = s | (s << 16);
      if constexpr (HAS_ZP) {
        const unsigned zo = MODE == 1 ? (unsigned)min(col[t], p.N - 1) >> 1 : 0u;
        const uint32_t zb = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rsZ, zo, 0, 0);
        const uint32_t z = MODE == 1 ? (zb >> zsh) & 15u : zb & 15u;
        const uint32_t b = 0x6400u + (SIGNED ? z ^ 8u : z);
        bfix[t] = b | (b << 16);
      }
    }
  }

  // ---- one slot per row group in flight: weights, activations, and (mode 2)
  // the scale / zero point of each chunk ----
  v4i wq[kDepth][T];
  v8h act[kDepth][4];
  uint32_t sc[kDepth][T][4];
  uint32_t zq[kDepth][T][4];
  v4f acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

  // Row group i of this wave into slot s.  Every offset is a per-lane
  // constant (vector offset) plus a wave-uniform part (scalar offset), so the
  // loads cost no vector instructions.  Groups past the wave's range, lanes
  // past M and rows past K read zero activations (a vector offset past the
  // buffer); the weights there are padding or zeros and the scale row is
  // clamped into the scale tensor, so those products are exactly 0.
  const bool m_ok = li < p.M;
  const unsigned a_lane = m_ok ? ((unsigned)(li * p.K) * 2u + 16u * (unsigned)g) : kOob;  // bytes
  // K % 32 == 0: a 32-row chunk lies wholly inside or wholly past K.  The
  // scale row of lane g is (rb >> shift) + g_srow; clamping the uniform part
  // to s_rows - 1 - (24 >> shift) keeps every lane inside the scale tensor and
  // changes no row of a chunk inside K.
  const int g_srow = (8 * g) >> p.blk_shift;
  const int su_max = (int)s_rows - 1 - (24 >> p.blk_shift);
  unsigned s_lane[T], z_lane[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int cc = min(col[t], p.N - 1);
    s_lane[t] = 2u * (unsigned)(p.N * g_srow + cc);     // scale bytes
    z_lane[t] = (unsigned)(p.N * g_srow + cc) >> 1;     // zero-point bytes (N even)
  }
  auto issue = [&](int s, int i) __attribute__((always_inline)) {
    const bool live = i < ng;  // wave-uniform
    const int q = live ? gb + i : 0;
#pragma unroll
    for (int t = 0; t < T; ++t)
      wq[s][t] = __builtin_amdgcn_raw_buffer_load_b128(rsW, live ? w_lane[t] : kOob, q * kGroupBytes, kStreamPolicy);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int rb = q * kGroupRows + 32 * c;  // first row of chunk c (wave-uniform)
      const bool in_k = live && rb < p.K;      // wave-uniform
      act[s][c] = __builtin_bit_cast(
          v8h, __builtin_amdgcn_raw_buffer_load_b128(rsA, in_k ? a_lane : kOob, in_k ? 2 * rb : 0, 0));
      if constexpr (kBlocked) {
        const int su = min(rb >> p.blk_shift, su_max);  // wave-uniform
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if (MODE == 3 && c > 0) {  // the group's one scale row (c is an unrolled constant)
            sc[s][t][c] = sc[s][t][0];
            if constexpr (HAS_ZP) zq[s][t][c] = zq[s][t][0];
            continue;
          }
          sc[s][t][c] = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsS, s_lane[t], 2 * p.N * su, 0);
          if constexpr (HAS_ZP)
            zq[s][t][c] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rsZ, z_lane[t], (p.N * su) >> 1, 0);
        }
      }
    }
  };

  auto compute = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // scale and bias enter the packed fp16 ops as broadcast low halves
        uint32_t s1 = sfix[t], b1 = bfix[t];
        if constexpr (kBlocked) {
          s1 = sc[s][t][c];
          if constexpr (HAS_ZP) {
            const uint32_t z = (zq[s][t][c] >> zsh) & 15u;
            b1 = 0x6400u + (SIGNED ? z ^ 8u : z);
          }
        }
        const _Float16 sv = __builtin_bit_cast(_Float16, (uint16_t)s1);
        const _Float16 bv = __builtin_bit_cast(_Float16, (uint16_t)(b1 & 0xffffu));
        const _Float16 bo = __builtin_bit_cast(_Float16, (uint16_t)OddBias(b1 & 0xffffu));
        const v2h s2 = v2h{sv, sv}, b2 = v2h{bv, bv}, b2o = v2h{bo, bo};
        const uint32_t w = (uint32_t)wq[s][t][c], w8 = w >> 8;
        const uint32_t pr[4] = {RowPair<0>(w, w8), RowPair<1>(w, w8), RowPair<2>(w, w8), RowPair<3>(w, w8)};
        v8h wop;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v2h v = (__builtin_bit_cast(v2h, pr[j]) - (j & 1 ? b2o : b2)) * s2;
          wop[2 * j] = v.x;
          wop[2 * j + 1] = v.y;
        }
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, act[s][c], acc[t], 0, 0, 0);
      }
    }
  };

#pragma unroll
  for (int s = 0; s < kDepth; ++s) {
    issue(s, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int r = 0; r < ng; r += kDepth) {
#pragma unroll
    for (int s = 0; s < kDepth; ++s) {
      compute(s);
      issue(s, r + kDepth + s);
      // group by group: decode work of a later group must not pull its data
      // waits into this one
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the last round's loads (past the range, all zero) retire before the waves
  // move on
  __builtin_amdgcn_s_waitcnt(0);

  // ---- reduce the waves: lane (li, g), register q of acc[t] holds row m = li
  // of column 16 * (tile0 + t) + 4g + q ----
  const int M = p.M;
  if (li < M) {
#pragma unroll
    for (int t = 0; t < T; ++t) *reinterpret_cast<v4f *>(&red[wave][li][16 * t + 4 * g]) = acc[t];
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rsY = Rsrc(p.Y, (int64_t)M * p.N * 2);
  const int col0 = 16 * tile0;
  for (int j = threadIdx.x; j < M * 4 * T; j += kThreads) {
    const int m = j / (4 * T), cq = 4 * (j % (4 * T));
    v4f v = *reinterpret_cast<const v4f *>(&red[0][m][cq]);
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += *reinterpret_cast<const v4f *>(&red[w][m][cq]);  // fixed order
    const int n = col0 + cq;
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = __builtin_bit_cast(uint16_t, (_Float16)v[e]);
    const int64_t yo = ((int64_t)m * p.N + n) * 2;
    if (p.N % 4 == 0) {  // a quad is wholly inside or outside; 8-byte aligned
      const v2i pk = v2i{(int)(h[0] | ((uint32_t)h[1] << 16)), (int)(h[2] | ((uint32_t)h[3] << 16))};
      __builtin_amdgcn_raw_buffer_store_b64(pk, rsY, n < p.N ? (unsigned)yo : kOob, 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __builtin_amdgcn_raw_buffer_store_b16(h[e], rsY, n + e < p.N ? (unsigned)(yo + 2 * e) : kOob, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Preparation: ONNX-packed 4-bit x [K, N] -> tiled layout, one thread per
// output dword (8 rows of one column).
__global__ __launch_bounds__(256) void TileInt4Kernel(const uint8_t *x, int64_t K, int64_t N, int is_signed,
                                                      int64_t ngroups, int64_t total, uint32_t *out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx & 3);
  const int l = (int)((idx >> 2) & 63);
  const int64_t tq = idx >> 8;  // tile * ngroups + group
  const int64_t t = tq / ngroups, q = tq % ngroups;
  const int64_t colm = 16 * t + (l & 15);
  const int64_t row0 = kGroupRows * q + 32 * c + 8 * (l >> 4);
  const uint32_t zero = is_signed ? 8u : 0u;
  uint32_t word = 0;
  for (int j = 0; j < 8; ++j) {
    const int64_t row = row0 + j;
    uint32_t u = zero;
    if (row < K && colm < N) {
      const int64_t e = row * N + colm;
      const uint32_t nib = (x[e >> 1] >> (4 * (e & 1))) & 15u;
      u = is_signed ? nib ^ 8u : nib;
    }
    word |= u << ((j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1));
  }
  out[idx] = word;
}

int TilesPerGroup(int64_t ntiles) {
  return (int)std::min<int64_t>(kMaxTiles, std::max<int64_t>(1, (ntiles + kTargetGroups - 1) / kTargetGroups));
}

}  // namespace

int64_t TiledInt4Bytes(int64_t K, int64_t N) {
  return ((N + 15) / 16) * ((K + kGroupRows - 1) / kGroupRows) * kGroupBytes;
}

void LaunchTileInt4(const uint8_t *x, int64_t K, int64_t N, int is_signed, uint32_t *out, hipStream_t stream) {
  const int64_t ngroups = (K + kGroupRows - 1) / kGroupRows;
  const int64_t total = TiledInt4Bytes(K, N) / 4;
  if (total == 0) return;
  hipLaunchKernelGGL(TileInt4Kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, x, K, N,
                     is_signed, ngroups, total, out);
}

bool GemvQ4TiledEligible(const DqMatMulParams &p) {
  const bool four = p.w_dtype == kInt4 || p.w_dtype == kUint4;
  const int64_t lim = (int64_t(1) << 31) - 64;
  return p.w_tiled && four && p.M >= 1 && p.M <= 16 && !p.a_bf16 && p.scale_f16 && p.deq_round_f16 &&
         p.cast_round == 0 && p.K % 32 == 0 &&
         (p.mode != 2 || (p.block >= 8 && (p.block & (p.block - 1)) == 0)) &&
         (p.zp == nullptr || p.N % 2 == 0) && TiledInt4Bytes(p.K, p.N) < lim && p.M * p.K * 2 < lim &&
         p.K * p.N * 2 < lim && reinterpret_cast<uintptr_t>(p.A) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.W) % 16 == 0 && reinterpret_cast<uintptr_t>(p.scale) % 2 == 0;
}

void LaunchGemvQ4Tiled(const DqMatMulParams &p, hipStream_t stream) {
  TiledArgs g{};
  g.A = static_cast<const _Float16 *>(p.A);
  g.W = p.W;
  g.scale = static_cast<const _Float16 *>(p.scale);
  g.zp = p.zp;
  g.Y = static_cast<_Float16 *>(p.Y);
  g.M = (int)p.M;
  g.N = (int)p.N;
  g.K = (int)p.K;
  g.blk_shift = p.mode == 2 ? __builtin_ctzll((unsigned long long)p.block) : 0;
  g.ntiles = (int)((p.N + 15) / 16);
  g.ngroups = (int)((p.K + kGroupRows - 1) / kGroupRows);
  const bool sgn = p.w_dtype == kInt4;
  const uint32_t b = 0x6400u + (sgn ? 8u : 0u);
  g.bias2 = b | (b << 16);
  const int T = TilesPerGroup(g.ntiles);
  const dim3 grid((unsigned)((g.ntiles + T - 1) / T));
  const bool zp = p.zp != nullptr;
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), 0, stream, g); };
  auto by_mode = [&](auto k0, auto k1, auto k2, auto k3) {
    if (p.mode == 0) go(k0);
    else if (p.mode == 1) go(k1);
    else if (g.blk_shift < 7) go(k2);
    else go(k3);
  };
#define OLA_TILED(TT, ZP, SG)                                                                    \
  by_mode(GemvQ4TiledKernel<TT, ZP, SG, 0>, GemvQ4TiledKernel<TT, ZP, SG, 1>, GemvQ4TiledKernel<TT, ZP, SG, 2>, \
          GemvQ4TiledKernel<TT, ZP, SG, 3>)
  auto by_zp = [&](auto tag) {
    constexpr int TT = decltype(tag)::value;
    if (!zp) OLA_TILED(TT, false, false);
    else if (sgn) OLA_TILED(TT, true, true);
    else OLA_TILED(TT, true, false);
  };
  switch (T) {
  case 1: by_zp(std::integral_constant<int, 1>{}); break;
  case 2: by_zp(std::integral_constant<int, 2>{}); break;
  case 3: by_zp(std::integral_constant<int, 3>{}); break;
  default: by_zp(std::integral_constant<int, 4>{}); break;
  }
#undef OLA_TILED
}

}  // namespace onnxl_amd
