// int8 MFMA GEMM for gfx950, shared by MatMulInteger (int32 output) and
// QLinearMatMul (requantised u8/s8 output).
//
// Tile: 256 x 128 outputs per 256-thread workgroup (4 waves, 2 x 2), each
// wave 128 x 64 = 4 x 2 blocks of v_mfma_i32_32x32x32_i8, K step 64.
//  - A (row-major [M,K], K contiguous) is loaded straight into MFMA operand
//    registers with raw buffer loads: lane (r, g) holds row r, bytes
//    [k0 + 32g, k0 + 32g + 32).  The two waves sharing rows read the same
//    lines; the second read hits L2.
//  - B (row-major [K,N], N contiguous) must reach the MFMA as 16 consecutive k
//    of one column: each thread loads a 4(k) x 8(n) byte block, transposes it
//    with v_perm_b32 and stores 4-byte k-quads into an LDS tile laid out
//    [n][k] with XOR-swizzled 16-byte chunks (double-buffered, one barrier per
//    K step).
//  - Software pipeline: A for step it+1 and B for step it+2 are in flight
//    while step it computes; the LDS store of step it+1's B (loaded one step
//    earlier) is interleaved with step it's MFMAs.  The loop is unrolled twice
//    with ping-pong register sets so no loop-carried copy waits on a load.
//  - Every lane-constant address is computed once; per step only a scalar
//    K offset is added.  Out-of-range rows use an offset past the buffer end,
//    which the buffer load returns as zero (no branches in the loop).
//  - Operand bytes are a' = a ^ 0x80 for UINT8 (= a - 128) so the signed MFMA
//    applies; the zero-point algebra in kernels.hpp restores the exact result.
//    The row / column sums it needs come from extra MFMAs against an all-ones
//    operand, which land in exactly the lanes that hold the matching outputs.
//  - Workgroup ids are remapped so each XCD (8 on MI355X, ids dealt
//    round-robin) owns a contiguous run of tiles, grouped 8 tile-rows high,
//    so tiles sharing A rows / B columns share that XCD's L2.
#include <cstdlib>

#include "common.hpp"
#include "kernels.hpp"
#include "igemm_fast.hpp"

namespace onnxl_amd {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;
constexpr unsigned kFlip = 0x80808080u;
// Buffer resource word 3 for gfx9-family raw buffers; kOob is an offset past
// every buffer this kernel builds (their sizes stay below 2^31 - 2^24,
// checked on the host), so a load from it returns zero.
constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = 0x80000000u;

// Load paths: kFast (K % 64 == 0), kKTail (K % 16 == 0, partial last step),
// kBytes (any shape / alignment, byte loads).
enum Mode : int { kFast = 0, kKTail = 1, kBytes = 2 };

// LDS B tile [kBN][kBK] bytes; 16-byte chunk c of column n sits at chunk
// c ^ swz(n), which spreads both the transposing 4-byte stores and the
// 16-byte fragment reads over the banks.
__device__ __forceinline__ int BOff(int n, int chunk) {
  const int swz = ((n >> 1) ^ (n >> 3)) & 3;
  return n * kBK + ((chunk ^ swz) << 4);
}

// 4x4 byte transpose of rows r0..r3: d[j] = (r0.byte j, r1.byte j, r2.byte j,
// r3.byte j).  v_perm_b32 selects bytes of {S0, S1} (S1 = bytes 0-3).
__device__ __forceinline__ void Transpose4x4(unsigned r0, unsigned r1, unsigned r2, unsigned r3,
                                             unsigned d[4]) {
  const unsigned t0 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
  const unsigned t1 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);  // r2.b0 r3.b0 r2.b1 r3.b1
  const unsigned t2 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
  const unsigned t3 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);  // r2.b2 r3.b2 r2.b3 r3.b3
  d[0] = __builtin_amdgcn_perm(t1, t0, 0x05040100u);
  d[1] = __builtin_amdgcn_perm(t1, t0, 0x07060302u);
  d[2] = __builtin_amdgcn_perm(t3, t2, 0x05040100u);
  d[3] = __builtin_amdgcn_perm(t3, t2, 0x07060302u);
}

__device__ __forceinline__ int64_t MinI64(int64_t a, int64_t b) { return a < b ? a : b; }

template <int EPI, bool NEED_RA, bool NEED_CB, int MODE>
__global__ __launch_bounds__(kThreads, 1) void IGemmKernel(const IGemmParams p) {
  __shared__ __align__(16) int8_t lds_b[2][kBN * kBK];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;
  const int64_t M = p.M, N = p.N, K = p.K;

  // ---- tile selection (XCD-contiguous, grouped rows) ----
  const int64_t nbm = (M + kBM - 1) / kBM, nbn = (N + kBN - 1) / kBN;
  const int64_t tiles = nbm * nbn;
  const int64_t total = tiles * p.batch;
  const int64_t pid = blockIdx.x;
  const int64_t xcd = pid % kXcds, per = total / kXcds, extra = total % kXcds;
  const int64_t t_all = xcd * per + MinI64(xcd, extra) + pid / kXcds;
  const int64_t bt = t_all / tiles, t = t_all % tiles;
  const int64_t group = t / (kGroupM * nbn);
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = MinI64(nbm - first_m, kGroupM);
  const int64_t tm = first_m + (t % (kGroupM * nbn)) % gsize;
  const int64_t tn = (t % (kGroupM * nbn)) / gsize;
  const int64_t row0 = tm * kBM, col0 = tn * kBN;

  int64_t a_off, b_off;
  BatchOffsets(p.bm, bt, a_off, b_off);
  const int8_t *__restrict__ Ab = p.A + a_off;
  const int8_t *__restrict__ Bb = p.B + b_off;
  const unsigned aflip = p.a_u8 ? kFlip : 0u;
  const unsigned bflip = p.b_u8 ? kFlip : 0u;

  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(Ab), (short)0, (int)(MODE != kBytes ? M * K : 0), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(Bb), (short)0, (int)(MODE != kBytes ? K * N : 0), kRsrcWord3);

  // ---- lane-constant addressing ----
  unsigned a_voff[4];   // row start + 32*lg, or kOob for rows >= M
  unsigned a_mask[4];   // UINT8 flip of valid rows
  bool a_row_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + wm * 128 + i * 32 + lr;
    a_row_ok[i] = row < M;
    a_voff[i] = a_row_ok[i] ? (unsigned)(row * K + 32 * lg) : kOob;
    a_mask[i] = a_row_ok[i] ? aflip : 0u;
  }
  const int bno = tid & 15, bkq = tid >> 4;
  const int64_t b_col = col0 + 8 * bno;
  const bool b_col_ok = b_col < N;
  unsigned b_voff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) b_voff[r] = b_col_ok ? (unsigned)((4 * bkq + r) * N + b_col) : kOob;
  const unsigned b_mask = b_col_ok ? bflip : 0u;
  int b_st[2][4];  // LDS byte offsets of this thread's eight k-quad stores
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) b_st[h][j] = BOff(8 * bno + 4 * h + j, bkq >> 2) + 4 * (bkq & 3);
  int b_rd[2][2];  // LDS byte offsets of this lane's B fragments [kk][j]
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int j = 0; j < 2; ++j) b_rd[kk][j] = BOff(wn * 64 + j * 32 + lr, 2 * lg + kk);

  // ---- loads ----
  auto load_a = [&](int64_t k0, v4i(&dst)[4][2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (MODE == kBytes) {
        const int64_t row = row0 + wm * 128 + i * 32 + lr;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int64_t kc = k0 + 32 * lg + 16 * h;
          unsigned w[4] = {0, 0, 0, 0};
          if (row < M && kc < K) {
            const int8_t *src = Ab + row * K + kc;
            // byte path: flip each loaded byte here, padding stays zero
            for (int e = 0; e < 16; ++e)
              if (kc + e < K)
                w[e >> 2] |= (((unsigned)(uint8_t)src[e]) ^ (aflip & 0xffu)) << (8 * (e & 3));
          }
          dst[i][h] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
      } else {
        // raw bytes; the UINT8 flip is applied where the operand is used so
        // the prefetch never waits for its data here
        const unsigned off = a_voff[i] + (unsigned)k0;
        dst[i][0] = __builtin_amdgcn_raw_buffer_load_b128(rsA, off, 0, 0);
        dst[i][1] = __builtin_amdgcn_raw_buffer_load_b128(rsA, off + 16u, 0, 0);
      }
    }
  };
  auto load_b = [&](int64_t k0, unsigned(&dst)[4][2]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (MODE == kBytes) {
        const int64_t k = k0 + 4 * bkq + r;
        unsigned lo = 0, hi = 0;
        if (k < K && b_col_ok) {
          const int8_t *src = Bb + k * N + b_col;
          for (int e = 0; e < 8; ++e) {
            if (b_col + e < N) {
              const unsigned byte = ((unsigned)(uint8_t)src[e]) ^ (bflip & 0xffu);
              if (e < 4) lo |= byte << (8 * e); else hi |= byte << (8 * (e - 4));
            }
          }
        }
        dst[r][0] = lo;
        dst[r][1] = hi;
      } else {
        // rows k >= K lie past the buffer end and read zero
        const v2i v = __builtin_amdgcn_raw_buffer_load_b64(rsB, b_voff[r] + (unsigned)(k0 * N), 0, 0);
        dst[r][0] = (unsigned)v.x;
        dst[r][1] = (unsigned)v.y;
      }
    }
  };
  auto store_b = [&](int8_t *dst, const unsigned(&src)[4][2], int64_t k0) {
    unsigned f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // flip only bytes that were loaded: padding must stay zero
      f[r] = (MODE == kFast) ? b_mask
             : (MODE == kBytes ? 0u : ((k0 + 4 * bkq + r < K) ? b_mask : 0u));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      unsigned d[4];
      Transpose4x4(src[0][h] ^ f[0], src[1][h] ^ f[1], src[2][h] ^ f[2], src[3][h] ^ f[3], d);
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<unsigned *>(dst + b_st[h][j]) = d[j];
    }
  };

  v16i acc[4][2];
  v16i ra[4];
  v16i cb[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16i{0};
    if (NEED_RA) ra[i] = v16i{0};
  }
  if (NEED_CB) {
    cb[0] = v16i{0};
    cb[1] = v16i{0};
  }
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};

  // Pipeline: A for step it+1 and B for step it+2 are loaded during step it;
  // B of step it+1 (loaded one step earlier) is transposed into the other LDS
  // buffer while step it's MFMAs run, so no wait targets a just-issued load.
  // The loop is unrolled twice with ping-pong register sets: a loop-carried
  // register copy would force a wait on the prefetch at every iteration end.
  v4i a0[4][2], a1[4][2];
  unsigned b0[4][2], b1[4][2];
  const int nk = (int)((K + kBK - 1) / kBK);
  auto step = [&](int it, v4i(&a_use)[4][2], v4i(&a_fill)[4][2], unsigned(&b_use)[4][2],
                  unsigned(&b_fill)[4][2]) {
    load_a((int64_t)(it + 1) * kBK, a_fill);
    load_b((int64_t)(it + 2) * kBK, b_fill);
    const int8_t *bt_lds = lds_b[it & 1];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v4i bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const v4i *>(bt_lds + b_rd[kk][j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v4i av = a_use[i][kk];
        if (MODE == kFast) {
          av ^= (int)a_mask[i];
        } else {
          // partial last step: chunks at or past K hold bytes of the next row
          // (or were never loaded) and must read as zero
          const int64_t kc = (int64_t)it * kBK + 32 * lg + 16 * kk;
          const unsigned f = MODE == kBytes ? 0u : aflip;  // byte path flipped at load
          av = (a_row_ok[i] && kc < K) ? (av ^ (int)f) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bf[j], acc[i][j], 0, 0, 0);
        if (NEED_RA) ra[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, ones, ra[i], 0, 0, 0);
      }
      if (NEED_CB) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          cb[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ones, bf[j], cb[j], 0, 0, 0);
      }
    }
    store_b(lds_b[(it + 1) & 1], b_use, (int64_t)(it + 1) * kBK);
    __syncthreads();
  };
  if (nk > 0) {
    load_a(0, a0);
    load_b(0, b0);
    store_b(lds_b[0], b0, 0);
    load_b(kBK, b0);
  }
  __syncthreads();
  int it = 0;
  for (; it + 1 < nk; it += 2) {
    step(it, a0, a1, b0, b1);
    step(it + 1, a1, a0, b1, b0);
  }
  if (it < nk) step(it, a0, a1, b0, b1);

  // ---- epilogue: lane (lr, lg) of block (i, j) holds column j*32+lr,
  // rows (q/4)*8 + lg*4 + q%4 of register q ----
  const unsigned Ku = (unsigned)K;
  const QResolved qv = ResolveQ(p.dev, p.a_u8, p.b_u8, p.y_signed, p.alpha_scalar, p.beta_scalar, p.cs, p.zy);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int64_t row = row0 + wm * 128 + i * 32 + (q >> 2) * 8 + lg * 4 + (q & 3);
      if (row >= M) continue;
      const unsigned alpha =
          p.a_zp ? (unsigned)(p.a_u8 ? 128 - (int)p.a_zp[row] : -(int)(int8_t)p.a_zp[row])
                 : (unsigned)qv.alpha;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = col0 + wn * 64 + j * 32 + lr;
        if (col >= N) continue;
        const unsigned beta =
            p.b_zp ? (unsigned)(p.b_u8 ? 128 - (int)p.b_zp[col] : -(int)(int8_t)p.b_zp[col])
                   : (unsigned)qv.beta;
        unsigned v = (unsigned)acc[i][j][q];
        if (NEED_RA) v += beta * (unsigned)ra[i][q];
        if (NEED_CB) v += alpha * (unsigned)cb[j][q];
        v += Ku * alpha * beta;
        const int64_t yi = (bt * M + row) * N + col;
        if (EPI == kEpiInt32) {
          reinterpret_cast<int32_t *>(p.Y)[yi] = (int32_t)v;
        } else {
          float f = (float)(int32_t)v * qv.cs;
          f = __builtin_rintf(f) + qv.zy;
          f = f < p.qmin ? p.qmin : (f > p.qmax ? p.qmax : f);
          if (p.y_signed) {
            reinterpret_cast<int8_t *>(p.Y)[yi] = (int8_t)(int)f;
          } else {
            reinterpret_cast<uint8_t *>(p.Y)[yi] = (uint8_t)(int)f;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fast path (K % 64 == 0, N % 16 == 0, 16-byte aligned operands): both
// operands go global -> LDS with direct buffer loads (buffer_load_dwordx4 ...
// lds) into a 3-stage LDS ring, so two K steps are in flight without holding
// registers.
//  - A stage [256 rows][64 B] is stored as [row/16][16-byte chunk][row%16]:
//    one direct load per wave covers 16 rows x 4 chunks, and a 32-row MFMA
//    fragment read (ds_read_b128) touches 2 x 256 contiguous bytes.
//  - B stage [64 k][128 n] is stored row-major with 16-byte chunk c of row k
//    at chunk c ^ (k % 8).  The MFMA needs 16 consecutive k of one column per
//    lane: ds_read_b64_tr_b8 delivers that from the row-major tile.  Within a
//    16-lane group, result lane i byte t is byte (i % 8) of the 8-byte row
//    that lane 2t + i/8 addressed; so lane s addresses row k0 + s/2, column
//    block c0 + 8*(s % 2) and lane i receives column c0 + i, k0 .. k0 + 7.
//  - The UINT8 flip is applied to the fragments in registers; padding (rows
//    >= M, columns >= N) only feeds outputs that are never stored, and there
//    is no K padding on this path.
constexpr int kMaxStages = 6;
constexpr int kAStage = kBM * kBK;  // 16 KB
constexpr int kBStage = kBK * kBN;  //  8 KB

typedef int v2iL __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef __attribute__((address_space(3))) v2iL *lds_v2i_t;

// Waits until the oldest outstanding K step (six direct loads per thread) has
// landed, retires this wave's LDS reads, then joins the workgroup barrier.
// A plain __syncthreads() would drain every outstanding load (vmcnt(0)) and
// serialise the ring; the "memory" clobber keeps the compiler from moving LDS
// accesses across.
template <int S> __device__ __forceinline__ void RingBarrier() {
  static_assert(S >= 3 && S <= kMaxStages, "ring depth");
  if constexpr (S == 3) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (S == 4) asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (S == 5) asm volatile("s_waitcnt vmcnt(18) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if constexpr (S == 6) asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int EPI, bool NEED_RA, bool NEED_CB, int S>
__global__ __launch_bounds__(kThreads, 1) void IGemmLdsKernel(const IGemmParams p) {
  // One object per ring stage: the compiler's LDS-DMA wait tracking can then
  // tell a read of stage s from a direct load into another stage (with a
  // single array it waits for every outstanding load before each read).
  // Arrays past the ring depth are never referenced and not allocated.
  __shared__ __align__(16) int8_t lds_a0[kAStage], lds_a1[kAStage], lds_a2[kAStage],
      lds_a3[kAStage], lds_a4[kAStage], lds_a5[kAStage];
  __shared__ __align__(16) int8_t lds_b0[kBStage], lds_b1[kBStage], lds_b2[kBStage],
      lds_b3[kBStage], lds_b4[kBStage], lds_b5[kBStage];
  int8_t *const stage_a[kMaxStages] = {lds_a0, lds_a1, lds_a2, lds_a3, lds_a4, lds_a5};
  int8_t *const stage_b[kMaxStages] = {lds_b0, lds_b1, lds_b2, lds_b3, lds_b4, lds_b5};

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;
  const int64_t M = p.M, N = p.N, K = p.K;

  const int64_t nbm = (M + kBM - 1) / kBM, nbn = (N + kBN - 1) / kBN;
  const int64_t tiles = nbm * nbn;
  const int64_t total = tiles * p.batch;
  const int64_t pid = blockIdx.x;
  const int64_t xcd = pid % kXcds, per = total / kXcds, extra = total % kXcds;
  const int64_t t_all = xcd * per + MinI64(xcd, extra) + pid / kXcds;
  const int64_t bt = t_all / tiles, t = t_all % tiles;
  const int64_t group = t / (kGroupM * nbn);
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = MinI64(nbm - first_m, kGroupM);
  const int64_t tm = first_m + (t % (kGroupM * nbn)) % gsize;
  const int64_t tn = (t % (kGroupM * nbn)) / gsize;
  const int64_t row0 = tm * kBM, col0 = tn * kBN;

  int64_t a_off, b_off;
  BatchOffsets(p.bm, bt, a_off, b_off);
  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(p.A + a_off), (short)0, (int)(M * K), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(p.B + b_off), (short)0, (int)(K * N), kRsrcWord3);
  const int aflip = p.a_u8 ? (int)kFlip : 0;
  const int bflip = p.b_u8 ? (int)kFlip : 0;
  const int nk = (int)(K / kBK);

  // global offsets of this lane's direct loads (K step 0)
  unsigned a_g[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = row0 + 16 * (wave * 4 + q) + (lane & 15);
    a_g[q] = row < M ? (unsigned)(row * K + 16 * (lane >> 4)) : kOob;
  }
  unsigned b_g[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int krow = 8 * (wave * 2 + q) + (lane >> 3);
    const int64_t col = col0 + 16 * ((lane & 7) ^ (lane >> 3));
    b_g[q] = col < N ? (unsigned)(krow * N + col) : kOob;
  }
  // LDS read offsets within a stage
  int a_rd[2][4];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 128 + i * 32 + lr;
      a_rd[kk][i] = (r >> 4) * 1024 + (2 * kk + lg) * 256 + (r & 15) * 16;
    }
  int b_rd[2][2][2];
  {
    const int s16 = lane & 15, g16 = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int krow = kk * 32 + 16 * (g16 >> 1) + 8 * h + (s16 >> 1);
          const int col = wn * 64 + j * 32 + 16 * (g16 & 1) + 8 * (s16 & 1);
          b_rd[kk][j][h] = krow * kBN + 16 * ((col >> 4) ^ (krow & 7)) + (col & 15);
        }
  }

  auto issue = [&](int step, int stage) {
    const bool live = step < nk;
    const unsigned ka = (unsigned)step * kBK;
    const unsigned kb = (unsigned)((int64_t)step * kBK * N);
    int8_t *sa = stage_a[stage];
    int8_t *sb = stage_b[stage];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsA, (lds_ptr_t)(sa + (wave * 4 + q) * 1024), 16,
                                               live ? a_g[q] + ka : kOob, 0, 0, 0);
#pragma unroll
    for (int q = 0; q < 2; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsB, (lds_ptr_t)(sb + (wave * 2 + q) * 1024), 16,
                                               live ? b_g[q] + kb : kOob, 0, 0, 0);
  };

  v16i acc[4][2];
  v16i ra[4];
  v16i cb[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16i{0};
    if (NEED_RA) ra[i] = v16i{0};
  }
  if (NEED_CB) {
    cb[0] = v16i{0};
    cb[1] = v16i{0};
  }
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};

  // One K step on ring stage `stage` (a compile-time index after unrolling).
  auto step = [&](int it, int stage) {
    RingBarrier<S>();
    issue(it + S - 1, (stage + S - 1) % S);  // the stage every wave finished reading
    __builtin_amdgcn_sched_barrier(0);     // keep the loads at the top of the step
    const int8_t *sa = stage_a[stage];
    const int8_t *sb = stage_b[stage];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v4i bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const v2iL lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)(sb + b_rd[kk][j][0]));
        const v2iL hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)(sb + b_rd[kk][j][1]));
        bf[j] = v4i{lo.x, lo.y, hi.x, hi.y} ^ bflip;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4i av = *reinterpret_cast<const v4i *>(sa + a_rd[kk][i]) ^ aflip;
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bf[j], acc[i][j], 0, 0, 0);
        if (NEED_RA) ra[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, ones, ra[i], 0, 0, 0);
      }
      if (NEED_CB) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          cb[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ones, bf[j], cb[j], 0, 0, 0);
      }
    }
  };

#pragma unroll
  for (int s0 = 0; s0 < S - 1; ++s0) issue(s0, s0);
  int it = 0;
  for (; it + S <= nk; it += S) {
#pragma unroll
    for (int s0 = 0; s0 < S; ++s0) step(it + s0, s0);
  }
#pragma unroll
  for (int s0 = 0; s0 < S - 1; ++s0)
    if (it + s0 < nk) step(it + s0, s0);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): drain the look-ahead loads

  const unsigned Ku = (unsigned)K;
  const QResolved qv = ResolveQ(p.dev, p.a_u8, p.b_u8, p.y_signed, p.alpha_scalar, p.beta_scalar, p.cs, p.zy);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int64_t row = row0 + wm * 128 + i * 32 + (q >> 2) * 8 + lg * 4 + (q & 3);
      if (row >= M) continue;
      const unsigned alpha =
          p.a_zp ? (unsigned)(p.a_u8 ? 128 - (int)p.a_zp[row] : -(int)(int8_t)p.a_zp[row])
                 : (unsigned)qv.alpha;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = col0 + wn * 64 + j * 32 + lr;
        if (col >= N) continue;
        const unsigned beta =
            p.b_zp ? (unsigned)(p.b_u8 ? 128 - (int)p.b_zp[col] : -(int)(int8_t)p.b_zp[col])
                   : (unsigned)qv.beta;
        unsigned v = (unsigned)acc[i][j][q];
        if (NEED_RA) v += beta * (unsigned)ra[i][q];
        if (NEED_CB) v += alpha * (unsigned)cb[j][q];
        v += Ku * alpha * beta;
        const int64_t yi = (bt * M + row) * N + col;
        if (EPI == kEpiInt32) {
          reinterpret_cast<int32_t *>(p.Y)[yi] = (int32_t)v;
        } else {
          float f = (float)(int32_t)v * qv.cs;
          f = __builtin_rintf(f) + qv.zy;
          f = f < p.qmin ? p.qmin : (f > p.qmax ? p.qmax : f);
          if (p.y_signed) {
            reinterpret_cast<int8_t *>(p.Y)[yi] = (int8_t)(int)f;
          } else {
            reinterpret_cast<uint8_t *>(p.Y)[yi] = (uint8_t)(int)f;
          }
        }
      }
    }
  }
}

int g_ring_stages = 4;  // ring depth of the fast path (ONNXL_AMD_IGEMM_STAGES overrides)

template <int EPI, bool RA, bool CB>
void LaunchLds(const IGemmParams &p, dim3 grid, hipStream_t s) {
  switch (g_ring_stages) {
  case 3: hipLaunchKernelGGL((IGemmLdsKernel<EPI, RA, CB, 3>), grid, dim3(kThreads), 0, s, p); break;
  case 5: hipLaunchKernelGGL((IGemmLdsKernel<EPI, RA, CB, 5>), grid, dim3(kThreads), 0, s, p); break;
  case 6: hipLaunchKernelGGL((IGemmLdsKernel<EPI, RA, CB, 6>), grid, dim3(kThreads), 0, s, p); break;
  default: hipLaunchKernelGGL((IGemmLdsKernel<EPI, RA, CB, 4>), grid, dim3(kThreads), 0, s, p); break;
  }
}

template <int EPI, bool RA, bool CB, int MODE>
void Launch(const IGemmParams &p, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((IGemmKernel<EPI, RA, CB, MODE>), grid, dim3(kThreads), 0, s, p);
}

template <int EPI>
void LaunchEpi(const IGemmParams &p, int mode, dim3 grid, hipStream_t s) {
  if (mode != kFast) {
    // Rare shapes: always accumulate the row / column sums (exact: their
    // weights beta / alpha are zero when they are not needed).
    if (mode == kKTail) Launch<EPI, true, true, kKTail>(p, grid, s);
    else Launch<EPI, true, true, kBytes>(p, grid, s);
    return;
  }
  if (p.need_ra) {
    if (p.need_cb) LaunchLds<EPI, true, true>(p, grid, s);
    else LaunchLds<EPI, true, false>(p, grid, s);
  } else {
    if (p.need_cb) LaunchLds<EPI, false, true>(p, grid, s);
    else LaunchLds<EPI, false, false>(p, grid, s);
  }
}

}  // namespace

bool IGemmFastEligible(const IGemmParams &p) { return mg::Eligible<mg::kI8>(ToGemmArgs(p)); }

void LaunchIGemm(const IGemmParams &p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return;
  if (p.implicit_conv) {  // the caller checked the implicit operand's shape
    if (p.epilogue == kEpiInt32) LaunchIGemmConvI32(p, stream);
    else if (p.epilogue == kEpiQuant8Row) LaunchIGemmConvQ8Row(p, stream);
    else throw DeviceError("internal: implicit convolution with a per-tensor requantization");
    return;
  }
  // K % 128 == 0: the pipelined MFMA core (mfma_gemm.hpp).
  if (mg::Eligible<mg::kI8>(ToGemmArgs(p))) {
    if (p.epilogue == kEpiInt32) LaunchIGemmFastI32(p, stream);
    else if (p.epilogue == kEpiQuant8Row) LaunchIGemmFastQ8Row(p, stream);
    else LaunchIGemmFastQ8(p, stream);
    return;
  }
  if (p.epilogue == kEpiQuant8Row) throw DeviceError("internal: per-row requantization needs the pipelined GEMM");
  static const int stages_env = [] {
    const char *e = std::getenv("ONNXL_AMD_IGEMM_STAGES");
    return e ? std::atoi(e) : 0;
  }();
  if (stages_env >= 3 && stages_env <= kMaxStages) g_ring_stages = stages_env;
  const int64_t tiles = ((p.M + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN) * p.batch;
  // Buffer paths: 16-byte A rows, 8-byte B rows (every batch base and row
  // start aligned) and per-matrix byte counts, plus the look-ahead of two K
  // steps, below 2^31 - 2^24 so offsets never reach kOob by themselves.
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  const bool buf = (p.K % 16 == 0) && (p.N % 8 == 0) && p.M * p.K + 4 * kBK < lim &&
                   (p.K + 3 * kBK) * p.N < lim &&
                   (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.B) % 8 == 0);
  // kFast runs the LDS-ring kernel: it also needs 16-byte B chunks.
  const bool lds_ok = p.N % 16 == 0 && reinterpret_cast<uintptr_t>(p.B) % 16 == 0;
  const int mode = !buf ? kBytes : ((p.K % kBK == 0 && lds_ok) ? kFast : kKTail);
  const dim3 grid((unsigned)tiles);
  if (p.epilogue == kEpiInt32) LaunchEpi<kEpiInt32>(p, mode, grid, stream);
  else LaunchEpi<kEpiQuant8>(p, mode, grid, stream);
}


// ---------------------------------------------------------------------------
// QLinearMatMul past the int32-exact K.  One 16x16 output tile per
// workgroup, one output per thread; 64-deep K slices of (a - za) and
// (b - zb) staged in LDS.  A slice's 64 products (|.| <= 255 * 255 each)
// sum exactly in int32 and are added into an int64 total, so the sum is the
// reference's for every K; then the same requantization as the MFMA
// epilogue: rint((float)acc * cs) + zy, clamped, NaN -> 0.
namespace {
constexpr int kXT = 16, kXK = 64;

__global__ __launch_bounds__(256) void QlmExactKernel(const IGemmParams p, int32_t za, int32_t zb) {
  // device-resident zero points and scales (p.dev) replace the host values
  if (p.dev.za) za = p.a_u8 ? (int32_t)p.dev.za[0] : (int32_t)(int8_t)p.dev.za[0];
  if (p.dev.zb) zb = p.b_u8 ? (int32_t)p.dev.zb[0] : (int32_t)(int8_t)p.dev.zb[0];
  const QResolved qv = ResolveQ(p.dev, p.a_u8, p.b_u8, p.y_signed, 0, 0, p.cs, p.zy);
  __shared__ int32_t as[kXT][kXK + 1];
  __shared__ int32_t bs[kXK][kXT + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t row = (int64_t)blockIdx.y * kXT + ty, col = (int64_t)blockIdx.x * kXT + tx;
  const int64_t batch = blockIdx.z;
  int64_t a_off = 0, b_off = 0;
  BatchOffsets(p.bm, batch, a_off, b_off);
  const int8_t *A = p.A + a_off;
  const int8_t *B = p.B + b_off;
  int64_t acc = 0;
  for (int64_t k0 = 0; k0 < p.K; k0 += kXK) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = (int)threadIdx.x + 256 * e;
      const int ar = i / kXK, ak = i % kXK;  // A slice [16][64]
      const int64_t gr = (int64_t)blockIdx.y * kXT + ar, gk = k0 + ak;
      int32_t av = 0;
      if (gr < p.M && gk < p.K) {
        const int8_t v = A[gr * p.K + gk];
        av = (p.a_u8 ? (int32_t)(uint8_t)v : (int32_t)v) - za;
      }
      as[ar][ak] = av;
      const int bk = i / kXT, bc = i % kXT;  // B slice [64][16]
      const int64_t gk2 = k0 + bk, gc = (int64_t)blockIdx.x * kXT + bc;
      int32_t bv = 0;
      if (gk2 < p.K && gc < p.N) {
        const int8_t v = B[gk2 * p.N + gc];
        bv = (p.b_u8 ? (int32_t)(uint8_t)v : (int32_t)v) - zb;
      }
      bs[bk][bc] = bv;
    }
    __syncthreads();
    int32_t part = 0;
#pragma unroll 16
    for (int k = 0; k < kXK; ++k) part += as[ty][k] * bs[k][tx];
    acc += part;
    __syncthreads();
  }
  if (row < p.M && col < p.N) {
    const float v = __builtin_rintf((float)acc * qv.cs) + qv.zy;
    const uint8_t q = v != v ? 0 : (uint8_t)(int32_t)__builtin_amdgcn_fmed3f(v, p.qmin, p.qmax);
    static_cast<uint8_t *>(p.Y)[(batch * p.M + row) * p.N + col] = q;
  }
}
}  // namespace

void LaunchQlmExact(const IGemmParams &p, int32_t za, int32_t zb, hipStream_t stream) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return;
  const int64_t gx = (p.N + kXT - 1) / kXT, gy = (p.M + kXT - 1) / kXT;
  if (gx > 0x7fffffff || gy > 65535 || p.batch > 65535)
    throw Unsupported("QLinearMatMul: shape too large for the int64-exact GPU path");
  hipLaunchKernelGGL(QlmExactKernel, dim3((unsigned)gx, (unsigned)gy, (unsigned)p.batch), dim3(256), 0, stream, p,
                     za, zb);
}

}  // namespace onnxl_amd
