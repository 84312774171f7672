// Decode-shaped fused DequantizeLinear(INT4 / UINT4, FLOAT16 scales) -> FLOAT16
// MatMul:  Y[M, N] = A[M, K] * W,  W[k, n] = fp16((x[k, n] - zp) * scale),
// for M <= 16 (one MFMA tile of activation rows).
//
// The weight stream dominates (K * N / 2 bytes read once), so the kernel is
// organised around HBM reads:
//  - A lane owns CPL consecutive columns (CPL = 16: 8 bytes of packed nibbles
//    per k row, one b64 load; CPL = 8 when N is not a multiple of 16) and 8
//    consecutive k rows per 32-row chunk; 16 lanes span a 16 * CPL-column
//    strip, so one load instruction reads 4 k rows of 8 * CPL contiguous
//    bytes.  With CPL = 16 that is a whole 128-byte line per row: row
//    segments of 64 bytes (CPL = 8) read HBM at about two thirds of the rate.
//  - Dequantisation happens in registers.  Two k rows are merged byte-wise
//    with v_perm_b32 so that each 32-bit register holds the nibbles of one
//    column at rows k and k+1; OR-ing 0x6400 (fp16 1024) into the low nibbles
//    makes them exact fp16 values 1024 + u, OR-ing 0x5400 (fp16 64, step
//    1/16) into the high nibbles where they lie makes them 64 + u (no shift),
//    a packed fp16 subtract of (1024 or 64 + bias + zero point) recovers the
//    integer, and a packed fp16 multiply by the column's scale
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
//    partials travel through sc1 (device-coherent) buffer loads and stores,
//    which are coherent across the XCDs' L2 caches without a cache-wide
//    writeback.
#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;          // k rows per MFMA
constexpr int kMaxChunks = 4;       // chunks per wave
constexpr int kDepth = 4;           // chunks whose loads are in flight ahead of use
constexpr int kTargetGroups = 256;  // workgroups wanted: about one per CU

// Strip geometry for CPL columns per lane.
template <int CPL> struct Strip {
  static constexpr int kCols = 16 * CPL;     // columns per workgroup
  static constexpr int kRedG = 4 * CPL + 1;  // padded reduction layout: a
  static constexpr int kRedRow = 4 * kRedG;  // wave's 64 lanes hit 64 banks
};

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

// Nibbles of byte b of two k rows -> two fp16 pairs: column 2b at rows
// (r0, r1) as 0x6400 | u (= 1024 + u, unit step 1) and column 2b + 1 at rows
// (r0, r1) as 0x5400 | u << 4 (= 64 + u, step 1/16: the nibble stays at bits
// 4-7, no shift).  `sel` gathers [x0.byte b, 0, x1.byte b, 0]; each AND-OR
// keeps one nibble per half and inserts the fp16 exponent.
__device__ __forceinline__ void DecodeBytePair(uint32_t x0, uint32_t x1, uint32_t sel, uint32_t &even,
                                               uint32_t &odd) {
  const uint32_t pb = __builtin_amdgcn_perm(x1, x0, sel);
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(even) : "v"(pb), "v"(0x000f000fu), "v"(0x64006400u));
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(odd) : "v"(pb), "v"(0x00f000f0u), "v"(0x54005400u));
}

__device__ __forceinline__ constexpr uint32_t ByteSel(int b) {
  return 0x0c000c00u | ((uint32_t)(4 + b) << 16) | (uint32_t)b;
}

constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = 0x80000000u;  // past every buffer: loads return zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Rsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kRsrcWord3);
}

// Buffer cache policy bit sc1 (gfx94x / gfx950): the access is coherent at
// device scope, i.e. it goes past the non-coherent L2 of the issuing XCD.
constexpr int kSc1 = 16;

// Four floats -> four fp16 (round to nearest even), packed in two dwords.
__device__ __forceinline__ v2i PackHalf4(v4f v) {
  v2i r;
  r.x = (int)((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[0]) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[1]) << 16));
  r.y = (int)((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2]) |
              ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[3]) << 16));
  return r;
}

// CPL / 8 dwords of packed nibbles (CPL columns) at byte offset off + soff,
// with the non-temporal cache policy (each weight byte is read once per call).
template <int CPL>
__device__ __forceinline__ void LoadNibbles(__amdgpu_buffer_rsrc_t rs, unsigned off, int soff,
                                            uint32_t (&dst)[CPL / 8]) {
  constexpr int kNonTemporal = 2;
  if constexpr (CPL == 16) {
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, soff, kNonTemporal);
    dst[0] = (uint32_t)v.x;
    dst[1] = (uint32_t)v.y;
  } else {
    dst[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, soff, kNonTemporal);
  }
}

template <int CPL, bool SIGNED, bool HAS_ZP, int MODE>
__global__ __launch_bounds__(kThreads) void GemvQ4Kernel(const GemvArgs p) {
  using S = Strip<CPL>;
  constexpr int kH = CPL / 8;  // dwords of nibbles per lane and k row
  // Per-wave partial sums (M rows per wave): row m, strip column
  // CPL * (4g + q) + e sits at m * kRedRow + g * kRedG + CPL * q + e.
  extern __shared__ float red[];
  __shared__ unsigned last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int li = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin: give each XCD a run of
  // adjacent strips (XCD x owns strips [x*base + min(x, extra), +count_x)).
  const int nstrips = gridDim.x;
  const int base = nstrips / 8, extra = nstrips % 8;
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const int strip = xcd * base + min(xcd, extra) + slot;
  const int slice = blockIdx.y;
  const int n0 = strip * S::kCols + CPL * li;  // first of this lane's CPL columns
  const bool col_ok = n0 < p.N;
  const int64_t row_bytes = p.N >> 1;          // packed bytes per k row
  const int total = p.K / kChunk;
  const int c_begin = (slice * kWaves + wave) * p.cpw;
  const int nch = max(min(c_begin + p.cpw, total) - c_begin, 0);

  const int64_t s_rows = MODE == 2 ? p.K / p.blk : 1;
  const __amdgpu_buffer_rsrc_t rsW = Rsrc(p.W, (int64_t)p.K * row_bytes);
  const __amdgpu_buffer_rsrc_t rsS = Rsrc(p.scale, MODE == 0 ? 2 : s_rows * p.N * 2);
  const __amdgpu_buffer_rsrc_t rsZ = Rsrc(p.zp, HAS_ZP ? (MODE == 0 ? 1 : (s_rows * p.N) >> 1) : 0);
  const __amdgpu_buffer_rsrc_t rsA = Rsrc(p.A, (int64_t)p.M * p.K * 2);

  // ---- loads of this wave's K range (branch-free: out-of-range lanes and
  // chunks read from an offset past the buffer, which returns 0) ----
  uint32_t wq[kMaxChunks][8][kH];
  v4i sc_raw[kMaxChunks][kH];
  uint32_t zp_raw[kMaxChunks][kH];
  v8h act[kMaxChunks];
  v4i sc_fixed[kH];
  uint32_t zp_fixed[kH];
#pragma unroll
  for (int h = 0; h < kH; ++h) {
    sc_fixed[h] = v4i{0, 0, 0, 0};
    zp_fixed[h] = 0;
  }
  if constexpr (MODE == 0) {
    const uint32_t hv = *static_cast<const uint16_t *>(static_cast<const void *>(p.scale));
    const int s2 = (int)(hv | (hv << 16));
    const uint32_t z = HAS_ZP ? (*reinterpret_cast<const uint8_t *>(p.zp) & 0xfu) * 0x11111111u : 0u;
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      sc_fixed[h] = v4i{s2, s2, s2, s2};
      zp_fixed[h] = z;
    }
  } else if constexpr (MODE == 1) {
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      sc_fixed[h] =
          __builtin_amdgcn_raw_buffer_load_b128(rsS, col_ok ? (unsigned)(n0 + 8 * h) * 2u : kOob, 0, 0);
      if (HAS_ZP)
        zp_fixed[h] =
            __builtin_amdgcn_raw_buffer_load_b32(rsZ, col_ok ? (unsigned)(n0 + 8 * h) >> 1 : kOob, 0, 0);
    }
  }
  // Weight rows: the lane part of the offset is fixed, the row part is
  // wave-uniform and goes into the scalar offset (no per-load vector math).
  // Chunks past this wave's range (c >= nch) read zero weights, scales and
  // activations, so they add exactly 0 and need no branch: a branch would let
  // the compiler sink chunk 0's loads behind the others, and the first MFMA
  // would then wait for every load of the wave.  The loads of chunk c are
  // issued kDepth chunks ahead of its use, in the order the chunks are
  // consumed.
  const unsigned w_lane = col_ok ? (unsigned)(8 * g * row_bytes + (n0 >> 1)) : kOob;
  auto issue = [&](int c) __attribute__((always_inline)) {
    const bool live = c < nch;  // wave-uniform
    const int cc = live ? c_begin + c : 0;
    const int k0 = cc * kChunk + 8 * g;  // first of this lane's 8 k rows
    const unsigned wl = live ? w_lane : kOob;
#pragma unroll
    for (int t = 0; t < 8; ++t)
      LoadNibbles<CPL>(rsW, wl, (int)((int64_t)(cc * kChunk + t) * row_bytes), wq[c][t]);
    if constexpr (MODE == 2) {
      const int64_t si = (int64_t)(k0 / p.blk) * p.N + n0;
#pragma unroll
      for (int h = 0; h < kH; ++h) {
        sc_raw[c][h] = __builtin_amdgcn_raw_buffer_load_b128(
            rsS, (live && col_ok) ? (unsigned)((si + 8 * h) * 2) : kOob, 0, 0);
        if (HAS_ZP)
          zp_raw[c][h] = __builtin_amdgcn_raw_buffer_load_b32(
              rsZ, (live && col_ok) ? (unsigned)((si + 8 * h) >> 1) : kOob, 0, 0);
      }
    } else {
#pragma unroll
      for (int h = 0; h < kH; ++h) {
        sc_raw[c][h] = live ? sc_fixed[h] : v4i{0, 0, 0, 0};
        zp_raw[c][h] = zp_fixed[h];
      }
    }
    act[c] = __builtin_bit_cast(
        v8h, __builtin_amdgcn_raw_buffer_load_b128(
                 rsA, (live && li < p.M) ? (unsigned)(((int64_t)li * p.K + k0) * 2) : kOob, 0, 0));
  };

  v4f acc[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) acc[e] = v4f{0.f, 0.f, 0.f, 0.f};

  const uint32_t flip = SIGNED ? 0x88888888u : 0u;  // signed nibble s -> s + 8
  auto compute = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      // Columns 8h + e of the lane: scale pair (s_e, s_e) and bias pair
      // (1024 + zb_e) (even e) or (64 + zb_e) (odd e) twice, zb = zero point
      // (+ 8 for INT4, matching the weight's own offset), decoded like the
      // weights, so that decoded weight - bias = x - zp exactly.
      uint32_t sc2[8], bias2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = (uint32_t)sc_raw[c][h][e >> 1];
        sc2[e] = __builtin_amdgcn_perm(word, word, (e & 1) ? 0x03020302u : 0x01000100u);
      }
      if (HAS_ZP) {
        const uint32_t z = zp_raw[c][h] ^ flip;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          DecodeBytePair(z, z, ByteSel(b), bias2[2 * b], bias2[2 * b + 1]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)  // 1032 / 1024 (even), 72 / 64 (odd)
          bias2[e] = (e & 1) ? (SIGNED ? 0x54805480u : 0x54005400u) : (SIGNED ? 0x64086408u : 0x64006400u);
      }
      uint32_t wk[8][4];  // [column][row pair]: fp16 1024 + u (even) / 64 + u (odd) at rows 2p, 2p+1
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        const uint32_t x0 = wq[c][2 * pr][h] ^ flip, x1 = wq[c][2 * pr + 1][h] ^ flip;
#pragma unroll
        for (int b = 0; b < 4; ++b)
          DecodeBytePair(x0, x1, ByteSel(b), wk[2 * b][pr], wk[2 * b + 1][pr]);
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
        acc[8 * h + e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wop, act[c], acc[8 * h + e], 0, 0, 0);
      }
    }
  };

#pragma unroll
  for (int c = 0; c < kDepth; ++c) {
    issue(c);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    compute(c);
    if (c + kDepth < kMaxChunks) issue(c + kDepth);
    // chunk by chunk: decode work of a later chunk must not pull its data
    // waits into this one
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- reduce the waves: lane (li, g), register q of acc[e] holds row m = li
  // of strip column CPL * (4g + q) + e ----
  const int M = p.M;
  if (li < M) {
    float *my = red + wave * M * S::kRedRow + li * S::kRedRow + g * S::kRedG;
#pragma unroll
    for (int e = 0; e < CPL; ++e)
#pragma unroll
      for (int q = 0; q < 4; ++q) my[CPL * q + e] = acc[e][q];
  }
  __syncthreads();
  // Each thread takes quads of 4 adjacent columns (N is a multiple of 8, so a
  // quad is wholly inside or wholly outside the matrix).
  const bool split = p.slices > 1;
  constexpr int kQuads = S::kCols / 4;
  const int nq = M * kQuads;
  const int64_t slice_bytes = (int64_t)M * p.N * 4;
  const __amdgpu_buffer_rsrc_t rsP = Rsrc(p.partial, split ? p.slices * slice_bytes : 0);
  const __amdgpu_buffer_rsrc_t rsY = Rsrc(p.Y, (int64_t)M * p.N * 2);
  for (int j = threadIdx.x; j < nq; j += kThreads) {
    const int m = j / kQuads, col = 4 * (j % kQuads);
    const int n = strip * S::kCols + col;
    const int ri = m * S::kRedRow + (col / (4 * CPL)) * S::kRedG + CPL * ((col / CPL) & 3) + (col % CPL);
    v4f v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = red[ri + i];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) v[i] += red[w * M * S::kRedRow + ri + i];  // fixed order
    }
    const bool ok = n < p.N;
    if (split) {
      // system-coherent (sc1) store: visible across the XCDs' L2 caches
      // without a cache-wide writeback
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(v4i, v), rsP, ok ? (unsigned)(slice * slice_bytes + ((int64_t)m * p.N + n) * 4) : kOob,
          0, kSc1);
    } else {
      __builtin_amdgcn_raw_buffer_store_b64(PackHalf4(v), rsY, ok ? (unsigned)(((int64_t)m * p.N + n) * 2) : kOob,
                                            0, 0);
    }
  }
  if (!split) return;

  // ---- K split over workgroups: the last one to arrive sums the partials.
  // Every wave waits for its partial stores to complete before the barrier
  // that precedes the counter update, so a workgroup that sees the final
  // count reads complete partials (sc1 loads, past the L2 of its XCD).  The
  // sum runs in slice order with up to 8 slices' loads in flight. ----
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(p.counters + strip, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(p.slices - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  for (int j = threadIdx.x; j < nq; j += kThreads) {
    const int m = j / kQuads, col = 4 * (j % kQuads);
    const int n = strip * S::kCols + col;
    const bool ok = n < p.N;
    const unsigned off0 = (unsigned)(((int64_t)m * p.N + n) * 4);
    v4f sum = v4f{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < p.slices; s0 += 8) {
      v4i part[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        part[u] = __builtin_amdgcn_raw_buffer_load_b128(
            rsP, (ok && s0 + u < p.slices) ? off0 + (unsigned)((s0 + u) * slice_bytes) : kOob, 0, kSc1);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s0 + u < p.slices) sum += __builtin_bit_cast(v4f, part[u]);
    }
    __builtin_amdgcn_raw_buffer_store_b64(PackHalf4(sum), rsY, ok ? (unsigned)(((int64_t)m * p.N + n) * 2) : kOob,
                                          0, 0);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(p.counters + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16 columns per lane (b64 loads, 128-byte row segments) when the rows allow.
int Cpl(const DqMatMulParams &p) {
  return p.N % 16 == 0 && reinterpret_cast<uintptr_t>(p.W) % 8 == 0 ? 16 : 8;
}

int Strips(const DqMatMulParams &p) {
  const int cols = 16 * Cpl(p);
  return (int)((p.N + cols - 1) / cols);
}

// Chunks per wave: at most kMaxChunks (the loads a wave keeps in flight),
// and no more than needed to spread the strips over about kTargetGroups
// workgroups.
int ChunksPerWave(const DqMatMulParams &p) {
  const int total = (int)(p.K / kChunk);
  const int want_slices = std::max(1, kTargetGroups / Strips(p));
  const int cpw = (total + kWaves * want_slices - 1) / (kWaves * want_slices);
  return std::min(kMaxChunks, std::max(1, cpw));
}

int Slices(const DqMatMulParams &p) {
  const int total = (int)(p.K / kChunk);
  const int span = kWaves * ChunksPerWave(p);
  return (total + span - 1) / span;
}

}  // namespace

bool GemvQ4Eligible(const DqMatMulParams &p) {
  const bool four = p.w_dtype == kInt4 || p.w_dtype == kUint4;
  return four && !p.w_tiled && p.M >= 1 && p.M <= 16 && !p.a_bf16 && p.scale_f16 && p.deq_round_f16 &&
         p.cast_round == 0 && p.K % kChunk == 0 && p.N % 8 == 0 &&
         p.K * p.N / 2 < (int64_t(1) << 31) - 64 && p.M * p.K * 2 < (int64_t(1) << 31) - 64 &&
         (p.mode != 2 || (p.block % 8 == 0)) && reinterpret_cast<uintptr_t>(p.A) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.W) % 4 == 0 && reinterpret_cast<uintptr_t>(p.scale) % 16 == 0 &&
         (int64_t)Slices(p) * p.M * p.N * 4 < (int64_t(1) << 31) - 64;  // partials: 32-bit offsets
}

size_t GemvQ4ScratchBytes(const DqMatMulParams &p) {
  const int s = Slices(p);
  return s > 1 ? (size_t)s * p.M * p.N * sizeof(float) : 0;
}

size_t GemvQ4Counters(const DqMatMulParams &p) { return (size_t)Strips(p); }

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
  g.cpw = ChunksPerWave(p);
  const int cpl = Cpl(p);
  const dim3 grid((unsigned)Strips(p), (unsigned)g.slices);
  // kWaves x M rows of 4 * kRedG floats (the padded reduction layout)
  const size_t lds = (size_t)kWaves * p.M * 4 * (4 * cpl + 1) * sizeof(float);
  const bool sgn = p.w_dtype == kInt4, zp = p.zp != nullptr;
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, dim3(kThreads), lds, stream, g); };
  auto by_mode = [&](auto k0, auto k1, auto k2) {
    if (p.mode == 0) go(k0);
    else if (p.mode == 1) go(k1);
    else go(k2);
  };
#define OLA_GEMV(CPL, SG, ZP) \
  by_mode(GemvQ4Kernel<CPL, SG, ZP, 0>, GemvQ4Kernel<CPL, SG, ZP, 1>, GemvQ4Kernel<CPL, SG, ZP, 2>)
  switch ((cpl == 16 ? 4 : 0) | (sgn ? 2 : 0) | (zp ? 1 : 0)) {
  case 0: OLA_GEMV(8, false, false); break;
  case 1: OLA_GEMV(8, false, true); break;
  case 2: OLA_GEMV(8, true, false); break;
  case 3: OLA_GEMV(8, true, true); break;
  case 4: OLA_GEMV(16, false, false); break;
  case 5: OLA_GEMV(16, false, true); break;
  case 6: OLA_GEMV(16, true, false); break;
  default: OLA_GEMV(16, true, true); break;
  }
#undef OLA_GEMV
}

}  // namespace onnxl_amd
