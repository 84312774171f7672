// Pipelined MFMA GEMM core for gfx950, shared by the int8 GEMM
// (MatMulInteger / QLinearMatMul), the fp8-weight bf16 GEMM (fused
// DequantizeLinear -> Cast -> MatMul) and the fp16 / bf16 MatMul.
//
// Y[b] = A[b] (M x K, row-major) * B[b] (K x N, row-major).
//
// Workgroup: 256 threads = 4 waves (2 x 2), one wave per SIMD, output tile
// 256 x (64 * WB); each wave owns 128 x (32 * WB) = 4 x WB blocks of 32 x 32
// MFMA outputs (WB = 2, or 4 for large GEMMs: the 256 accumulators then fill
// the AGPRs and each operand byte read from LDS feeds twice the MFMAs).
// A K step covers 128 bytes of every A row (128 int8 or 64 16-bit values).
//
// Memory path.
//  - Both operands go global -> LDS with direct buffer loads (16 bytes per
//    lane, 1 KB per wave instruction, no registers held) into a 3-stage ring:
//    while step t is multiplied, steps t+1 and t+2 are in flight.
//  - A stage [256 rows][128 B] is row-major with the 16-byte chunks of row r
//    permuted, chunk c at position c ^ h(r), h(r) = (r % 8) ^ ((r / 8) % 2).
//    A direct load puts lane i's
//    16 bytes at position i of its 1 KB, so lanes 8j .. 8j+7 fetch the eight
//    chunks of one row: every group of eight lanes reads one whole 128-byte
//    line (8 rows per load).  A layout with consecutive lanes on consecutive
//    rows (one load = the same 8 rows, column-wise) runs the address unit
//    about four times slower per byte and made the loads, not the MFMAs, the
//    bound.  A fragment read (ds_read_b128) has lanes on consecutive rows, one
//    chunk: any 8 consecutive rows hold it at 8 different positions, and any
//    16 at 16 different (row parity, position) pairs, so neither 8 lanes over
//    32 banks nor 16 lanes over 64 banks conflict.
//  - B stage [k rows][128 columns] is stored row-major with its 16-byte chunks
//    XOR-swizzled by the row index.  The MFMA wants consecutive k of one column
//    per lane; the transposing LDS reads (ds_read_b64_tr_b8 / _b16) deliver
//    exactly that from the row-major tile.  Within a 16-lane group, result
//    lane i element t is, for 8-bit elements, byte i%8 of the 8 bytes that
//    lane 2t + i/8 addressed; for 16-bit elements, element i%4 of the 4 that
//    lane 4t + i/4 addressed.  So lanes address (row k0 + s/2, columns
//    c0 + 8(s%2) ..) resp. (row k0 + s/4, columns c0 + 4(s%4) ..) and lane i
//    receives column c0 + i at k0, k0+1, ...
//
// Schedule (per K step of 4 sub-steps): the fragments of sub-step s are read
// from LDS two sub-steps ahead (three register sets); the fp8 B operand is
// decoded to bf16 under the MFMAs of sub-step s - 1, so neither LDS latency
// nor decode VALU work stalls the matrix pipe.  The single barrier per step sits inside sub-step 2, after
// half of its MFMAs are issued.  It waits only for the oldest ring stage
// (s_waitcnt vmcnt(L), L = direct loads per step), never for all loads.
//
// Epilogue: each wave converts its accumulators, stages 32 rows at a time in
// LDS and writes them back with 16-byte row-contiguous stores.
#pragma once

#include <type_traits>

#include "kernels.hpp"

namespace onnxl_amd {
namespace mg {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef __attribute__((address_space(3))) v2i *lds_v2i_t;
typedef __attribute__((address_space(3))) v4s *lds_v4s_t;

constexpr int kBM = 256, kStepBytes = 128, kStages = 3, kThreads = 256;
constexpr int kGroupM = 4, kXcds = 8;
constexpr int kAStage = kBM * kStepBytes;  // 32 KB
constexpr int kRsrcWord3 = 0x00020000;
constexpr unsigned kOob = 0x80000000u;
constexpr unsigned kFlip = 0x80808080u;
// Cache policy of the output stores: sc1 (device scope) writes through the
// XCD's L2.  Plain write-back stores leave up to the whole L2 dirty at the end
// of the kernel, and the kernel then completes only after that writeback: on
// C5 (33.5 MB of int32 output) 12.2 us per launch against 9.7 us with sc1.
constexpr int kStoreThrough = 16;

// Operand kinds.
//  kI8:     int8 / uint8 x int8 / uint8 -> int32 (v_mfma_i32_32x32x32_i8)
//  kBf16F8: bf16 A x float8e4m3fn B with a per-column (or single) fp32 scale;
//           B values enter the MFMA exactly (every e4m3fn value is a bf16
//           value: the high half of its fp32 decode) and the column's scale
//           multiplies the fp32 sum in the epilogue, Y = s_n * sum_k a q.
//           The DequantizeLinear(FLOAT) -> Cast(BFLOAT16) chain instead rounds
//           each s_n * q to bf16 first; the two differ by at most half a bf16
//           ulp of each product.
//  kH16:    fp16 x fp16 or bf16 x bf16 -> fp32 accumulate.
enum Kind : int { kI8 = 0, kBf16F8 = 1, kH16 = 2 };

// Output conversions.
// kOutQ8Row: the 8-bit requantization of kOutQ8 with a scale and an int32
// bias per output row (QLinearConv's per-output-channel w_scale and B).
enum Out : int { kOutI32 = 0, kOutQ8 = 1, kOutF16 = 2, kOutBf16 = 3, kOutQ8Row = 4 };

template <int KIND> struct Traits;
template <> struct Traits<kI8> {
  static constexpr int kKStep = 128;     // k values per step
  static constexpr int kBRows = 128;     // B rows per step
  static constexpr int kBsz = 1;         // bytes per B element
  using Acc = v16i;
};
template <> struct Traits<kBf16F8> {
  static constexpr int kKStep = 64;
  static constexpr int kBRows = 64;
  static constexpr int kBsz = 1;
  using Acc = v16f;
};
template <> struct Traits<kH16> {
  static constexpr int kKStep = 64;
  static constexpr int kBRows = 64;
  static constexpr int kBsz = 2;
  using Acc = v16f;
};
// The workgroup tile is 256 x BN with BN = 64 * WB: each wave owns 4 x WB
// blocks of 32 x 32 (WB = 2: 128 x 64 per wave; WB = 4: 128 x 128, which
// halves the operand bytes per MFMA and fills the 256 accumulator registers).
template <int KIND, int WB> constexpr int BPitch() { return 64 * WB * Traits<KIND>::kBsz; }
template <int KIND, int WB> constexpr int BStageBytes() { return Traits<KIND>::kBRows * BPitch<KIND, WB>(); }
// direct loads per wave per K step: A 32 KB + B stage, 1 KB per instruction
template <int KIND, int WB> constexpr int LoadsPerWave() { return (kAStage + BStageBytes<KIND, WB>()) / 1024 / 4; }
template <int KIND, int WB> constexpr int BLoadsPerWave() { return BStageBytes<KIND, WB>() / 1024 / 4; }

__device__ __forceinline__ int64_t MinI64(int64_t a, int64_t b) { return a < b ? a : b; }

// float pair -> packed bf16 pair (round to nearest even), lo in bits 0-15.
__device__ __forceinline__ unsigned PackBf16(float lo, float hi) {
  unsigned r;
  asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}

// Two floats that are bf16 values (fp8 decodes) -> packed bf16 pair, lo in
// bits 0-15: their high halves, exact for such values.  Inline asm: the
// compiler folds __builtin_amdgcn_perm of the two halves of one register pair
// into a perm of the low half with itself.
__device__ __forceinline__ unsigned HighHalves(v2f f) {
  unsigned r;
  asm("v_perm_b32 %0, %1, %2, %3" : "=v"(r) : "v"(f.y), "v"(f.x), "s"(0x07060302u));
  return r;
}

// One direct load: lane i's 16 bytes at `voffset` land at LDS address
// lds + 16 i (M0 holds the wave's LDS base).  Written as inline assembly so
// the compiler does not track the LDS write: it cannot tell which ring stage
// a load fills, and before LDS reads of another stage it waited for loads
// still in flight (s_waitcnt vmcnt(3..12) inside the K loop).  The ring's
// own waits (RingBarrier) order every read after the loads of its stage; the
// statements are volatile, so they keep their order against the barriers.
__device__ __forceinline__ void DirectLoad16(__amdgpu_buffer_rsrc_t rs, const char *lds, unsigned voffset) {
  const unsigned m0 = (unsigned)(size_t)(lds_ptr_t)lds;
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rs), "{m0}"(m0));
}

// Waits for all but the newest `L` direct loads (the oldest in-flight ring
// stage has then landed), retires this wave's LDS reads and joins the
// workgroup barrier.  A __syncthreads() would wait for every load.
template <int L> __device__ __forceinline__ void RingBarrier() {
  static_assert(L >= 0 && L < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(L) : "memory");
}

// Common launch-time description of one GEMM (all kinds).
struct GemmArgs {
  const void *A;
  const void *B;
  void *Y;
  int64_t M, N, K;
  int64_t batch;
  BatchMap bm;
  // kI8
  int a_u8, b_u8;
  const uint8_t *a_zp;
  const uint8_t *b_zp;
  int32_t alpha_scalar, beta_scalar;
  float cs, zy, qmin, qmax;
  int y_signed;
  QDevScalars dev;  // device-resident scalars replacing the four above (kI8 with ZP)
  // kBf16F8: dequantization scales (FLOAT or FLOAT16), one per column
  // (scale_per_col) or a single value; in grouped mode group g's scales start
  // scale_grp_stride elements after group g - 1's
  const void *scale;
  int scale_f16;
  int scale_per_col;
  int64_t scale_grp_stride;
  // Row pitches of B and Y in elements (0: N), so a launch can cover a
  // column range of larger matrices; N stays the width computed.
  int64_t ldb, ldy;
  // kOutQ8Row: row r is requantized with (row_xs * row_wscale[r] / row_ys)
  // (index 0 when !row_wscale_per) after adding row_bias[r] (none when null)
  // in exact integer arithmetic.
  const float *row_wscale;
  int row_wscale_per;
  float row_xs, row_ys;
  const int32_t *row_bias;
  // Grouped mode (GroupedMatMul; kernels with GM 1 or 2): the rows of A are
  // gathered and the rows of Y scattered through a routing table written on
  // the device, and each group of rows multiplies its own B.  M is then the
  // number of rows of A and Y has M * grp_sel rows.
  const int32_t *grp_tile_off;  // [grp_count + 1] first workgroup tile of each group
  const int32_t *grp_row_off;   // [grp_count + 1] first routed row of each group
  const int32_t *grp_rows;      // routed row -> row of Y (token * grp_sel + selection)
  int grp_count;
  int grp_sel;                  // row of A of Y row r: r / grp_sel
  int64_t grp_b_stride;         // elements from one group's B to the next
  const void *grp_bias;         // [grp_count, N] in the output dtype, or null
  // Implicit convolution (kernels with CV): B per batch entry is one image of
  // the padded NHWC input, read like A (rows = output positions).
  ImplicitConv cv;
};

// x / d for x, d < 2^16 from magic = ceil(2^32 / d) (0 for d = 1).
__device__ __forceinline__ uint32_t DivMagic(uint32_t x, uint32_t magic) {
  return magic ? __umulhi(x, magic) : x;
}

// GM: 0 one GEMM per batch entry; 1 grouped with each group's B [K, N]
// row-major; 2 grouped with each group's B given transposed, [N, K]
// row-major (kH16 only): its stage is then loaded and read like A's, rows of
// N with consecutive k, which is exactly the B operand of the MFMA; 3 one
// GEMM per batch entry with B given transposed like that (kH16 only: the
// fused DequantizePacked -> Transpose -> MatMul, whose decoded weight is
// [N, K]).
//
// CV: implicit convolution (int8): B is read like A, its row for output
// position n and K step t at the byte offset of GemmArgs::cv, so the im2col
// matrix is never written.
template <int KIND, int OUT, bool ZP, bool AU8, bool BU8, int WB, int GM = 0, bool CV = false>
__global__ __launch_bounds__(kThreads, 1) void MfmaGemmKernel(const GemmArgs p) {
  constexpr bool RA = ZP, CB = ZP;
  constexpr bool GRP = GM == 1 || GM == 2;  // grouped (routing tables)
  constexpr bool BT = GM == 2 || GM == 3 || CV;
  static_assert(GM == 0 || (((KIND == kH16 && WB == 2) || (KIND == kBf16F8 && GM == 1)) && !ZP),
                "grouped mode: 16-bit operands in 128-column tiles, or fp8 B [K, N] per group");
  static_assert(!CV || (KIND == kI8 && WB == 2 && GM == 0), "implicit convolution: int8, 128-column tiles");
  using T = Traits<KIND>;
  using Acc = typename T::Acc;
  constexpr int kBN = 64 * WB;                 // workgroup tile columns
  constexpr int kWN = 32 * WB;                 // wave tile columns
  constexpr int kBP = BPitch<KIND, WB>();      // bytes per B row in LDS
  // 1-byte B rows hold 8 (128-byte rows) or 16 (256-byte rows) chunks of 16
  // bytes; chunk c of row r sits at position c ^ (kBSwz * (r % 8)).  A
  // transposing read takes one chunk from each of 8 rows for 16 lanes, and the
  // next 16 lanes the neighbouring chunk of the same rows: with 256-byte rows
  // (all rows on the same banks) the doubled XOR puts the 16 chunks at 16
  // different positions, where the plain one put them on 8 twice.
  constexpr int kBSwz = kBP >= 256 ? 2 : 1;
  constexpr int kBStage = BStageBytes<KIND, WB>();
  constexpr int L = LoadsPerWave<KIND, WB>();
  constexpr int LB = BLoadsPerWave<KIND, WB>();
  static_assert(WB == 2 || (WB == 4 && KIND != kH16), "tile width");
  constexpr int kOsz = OUT == kOutI32 ? 4 : (OUT == kOutQ8 || OUT == kOutQ8Row ? 1 : 2);
  static_assert(LB >= 1 && LB <= 4, "B direct loads per wave");
  // One object per ring stage: the compiler's LDS-DMA wait tracking can then
  // tell a read of one stage from a direct load into another.
  __shared__ __align__(16) char sa0[kAStage], sa1[kAStage], sa2[kAStage];
  __shared__ __align__(16) char sb0[kBStage], sb1[kBStage], sb2[kBStage];
  __shared__ int32_t zsum[ZP ? (kThreads / 64) * 2 * kWN : 1];  // per wave: CB and beta of its columns
  __shared__ __align__(16) float cscale[KIND == kBf16F8 ? (kThreads / 64) * kWN : 4];  // per wave: column scales
  // stage index -> array (indices are compile-time constants after unrolling)
  auto SA = [&](int s) __attribute__((always_inline)) -> char * { return s == 0 ? sa0 : (s == 1 ? sa1 : sa2); };
  auto SB = [&](int s) __attribute__((always_inline)) -> char * { return s == 0 ? sb0 : (s == 1 ? sb1 : sb2); };

  const int tid = threadIdx.x;
  // the wave index as a scalar: the LDS destinations of the direct loads (M0)
  // then need no per-load readfirstlane
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = lane & 31, lg = lane >> 5;
  const int64_t M = p.M, N = p.N, K = p.K;
  const int64_t LDB = p.ldb ? p.ldb : N, LDY = p.ldy ? p.ldy : N;

  // ---- tile selection: each XCD owns a contiguous run of tiles, grouped
  // kGroupM tile-rows high, so tiles sharing A rows / B columns share an L2 ----
  const int64_t nbn = (N + kBN - 1) / kBN;
  int64_t bt = 0, row0, col0;
  // grouped mode: this tile's group, its routed rows [rbase, rbase + rcount)
  int grp = 0;
  int64_t rbase = 0, rcount = M;
  if constexpr (GRP) {
    // Workgroups past the routed tiles leave at once, before any load or
    // barrier (the whole workgroup takes the same branch).  The others are
    // spread as in the plain mode: each XCD a contiguous run of tiles (about
    // one group's worth when the groups are even), within a group kGroupM
    // tile-rows high and column by column, so each column tile of the group's
    // B is read once per run while its A rows stay in the caches.
    const int total = p.grp_tile_off[p.grp_count];
    const int pid = (int)blockIdx.x;
    if (pid >= total) return;
    const int xcd = pid % kXcds, per = total / kXcds, extra = total % kXcds;
    const int t = xcd * per + (xcd < extra ? xcd : extra) + pid / kXcds;
    // group g with grp_tile_off[g] <= t < grp_tile_off[g + 1] (non-empty)
    int lo = 0, hi = p.grp_count;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.grp_tile_off[mid] <= t) lo = mid;
      else hi = mid;
    }
    grp = lo;
    const int64_t local = t - p.grp_tile_off[grp];
    rbase = p.grp_row_off[grp];
    rcount = p.grp_row_off[grp + 1] - rbase;
    const int64_t nbm = (rcount + kBM - 1) / kBM;
    const int64_t first_m = local / (kGroupM * nbn) * kGroupM;
    const int64_t gsize = MinI64(nbm - first_m, kGroupM);
    row0 = (first_m + (local % (kGroupM * nbn)) % gsize) * kBM;
    col0 = (local % (kGroupM * nbn)) / gsize * kBN;
  } else {
    const int64_t nbm = (M + kBM - 1) / kBM;
    const int64_t tiles = nbm * nbn;
    const int64_t total = tiles * p.batch;
    const int64_t pid = blockIdx.x;
    const int64_t xcd = pid % kXcds, per = total / kXcds, extra = total % kXcds;
    const int64_t t_all = xcd * per + MinI64(xcd, extra) + pid / kXcds;
    bt = t_all / tiles;
    const int64_t tt = t_all % tiles;
    const int64_t group = tt / (kGroupM * nbn);
    const int64_t first_m = group * kGroupM;
    const int64_t gsize = MinI64(nbm - first_m, kGroupM);
    const int64_t tm = first_m + (tt % (kGroupM * nbn)) % gsize;
    const int64_t tn = (tt % (kGroupM * nbn)) / gsize;
    row0 = tm * kBM;
    col0 = tn * kBN;
  }

  constexpr int kAsz = KIND == kI8 ? 1 : 2;
  constexpr int kBsz = KIND == kH16 ? 2 : 1;
  int64_t a_off = 0, b_off = 0;
  if constexpr (GRP) b_off = grp * p.grp_b_stride;
  else BatchOffsets(p.bm, bt, a_off, b_off);
  const char *Ab = static_cast<const char *>(p.A) + a_off * kAsz;
  const char *Bb = static_cast<const char *>(p.B) + b_off * kBsz;
  const int64_t KA = K * kAsz;   // A row pitch in bytes
  const int64_t NB = LDB * kBsz;  // B row pitch in bytes
  const int64_t NW = N * kBsz;    // bytes of a B row inside the computed columns
  const __amdgpu_buffer_rsrc_t rsA =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(Ab), (short)0, (int)(M * KA), kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char *>(Bb), (short)0, (int)(CV ? p.cv.image_bytes : (BT ? N * KA : K * NB)), kRsrcWord3);
  // look-ahead loads past the last K step go through empty descriptors (every
  // access out of range): a scalar select instead of a per-lane one
  const __amdgpu_buffer_rsrc_t rsA0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(Ab), (short)0, 0, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsB0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(Bb), (short)0, 0, kRsrcWord3);
  const int64_t YR = GRP ? M * p.grp_sel : M;  // rows of Y
  const __amdgpu_buffer_rsrc_t rsY = __builtin_amdgcn_make_buffer_rsrc(
      static_cast<char *>(p.Y) + bt * M * LDY * kOsz, (short)0, (int)(YR * LDY * kOsz), kRsrcWord3);
  const int nfull = (int)(K / T::kKStep);                  // full K steps
  const bool half = K % T::kKStep != 0;                     // K % kKStep == kKStep / 2
  const int nk = nfull + (half ? 1 : 0);                    // K steps to load

  // ---- direct-load offsets (K step 0) ----
  unsigned a_g[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int64_t row = row0 + 8 * (8 * wave + q) + (lane >> 3);  // 8-row block 8 * wave + q
    int64_t src = row;  // row of A
    if constexpr (GRP) src = row < rcount ? p.grp_rows[rbase + row] / p.grp_sel : 0;
    a_g[q] = row < rcount ? (unsigned)(src * KA + 16 * ((lane & 7) ^ (lane >> 3) ^ (q & 1))) : kOob;
  }
  unsigned b_g[4];  // LB <= 4 (a fixed bound: a template-dependent size here
                    // makes the host compiler drop the kernel stub)
#pragma unroll
  for (int q = 0; q < LB; ++q) {
    const int i = wave * LB + q;  // 1 KB piece of the B stage
    if constexpr (CV) {
      // output position n: its input pixel for tap (0, 0) and channel chunk
      const int64_t n = col0 + 8 * i + (lane >> 3);
      const int64_t oh = n / p.cv.wo, ow = n - oh * p.cv.wo;
      b_g[q] = n < N ? (unsigned)(oh * p.cv.pix_row + ow * p.cv.pix_col + 16 * ((lane & 7) ^ (lane >> 3) ^ (i & 1)))
                     : kOob;
    } else if constexpr (BT) {
      // rows of N like A's rows of M: 8 rows of 128 bytes per piece
      const int64_t n = col0 + 8 * i + (lane >> 3);
      b_g[q] = n < N ? (unsigned)(n * KA + 16 * ((lane & 7) ^ (lane >> 3) ^ (i & 1))) : kOob;
    } else if constexpr (KIND == kH16) {
      const int krow = 4 * i + (lane >> 4);
      const int64_t cb = 2 * col0 + 16 * ((lane & 15) ^ (2 * ((lane >> 4) & 3)));
      b_g[q] = cb < NW ? (unsigned)(krow * NB + cb) : kOob;
    } else {
      // 1-byte B: a 1 KB piece is 1024 / kBP rows; lane -> (row, 16-byte
      // position p), holding global chunk p ^ BSwz(row)
      constexpr int kCpr = kBP / 16;
      const int krow = (1024 / kBP) * i + lane / kCpr;
      const int64_t cb = col0 + 16 * ((lane % kCpr) ^ (kBSwz * (krow & 7)));
      b_g[q] = cb < NW ? (unsigned)(krow * NB + cb) : kOob;
    }
  }
  // ---- LDS fragment offsets (sub-step 0; sub-step kk adds kk * const) ----
  // Sub-step kk reads chunk 2 kk + lg of row wm * 128 + 32 i + lr; block i
  // sits exactly 4096 bytes after block i-1, so one base per sub-step serves
  // all four blocks through the DS offset field.
  int a_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    a_rd[kk] = (wm * 128 + lr) * 128 + 16 * ((2 * kk + lg) ^ (lr & 7) ^ ((lr >> 3) & 1));
  const int s16 = lane & 15, g16 = lane >> 4;
  // One base per column block j; the second transposing read of a fragment
  // (h = 1) is 8 rows (int8) or 4 rows (16-bit) further, the same swizzle.
  int b_rd[WB];
#pragma unroll
  for (int j = 0; j < WB; ++j) {
    if constexpr (BT) {
      b_rd[j] = 0;  // bt_rd below
    } else if constexpr (KIND == kI8) {
      const int krow = 16 * (g16 >> 1) + (s16 >> 1);
      const int col = wn * kWN + j * 32 + 16 * (g16 & 1) + 8 * (s16 & 1);
      b_rd[j] = krow * kBP + 16 * ((col >> 4) ^ (kBSwz * (krow & 7))) + (col & 15);
    } else if constexpr (KIND == kBf16F8) {
      const int krow = 8 * (g16 >> 1) + (s16 >> 1);
      const int col = wn * kWN + j * 32 + 16 * (g16 & 1) + 8 * (s16 & 1);
      b_rd[j] = krow * kBP + 16 * ((col >> 4) ^ (kBSwz * (krow & 7))) + (col & 15);
    } else {
      const int krow = 8 * (g16 >> 1) + (s16 >> 2);
      const int col = wn * kWN + j * 32 + 16 * (g16 & 1) + 4 * (s16 & 3);
      b_rd[j] = krow * kBP + 16 * ((col >> 3) ^ (2 * (krow & 3))) + ((2 * col) & 15);
    }
  }
  // BT: sub-step kk reads chunk 2 kk + lg of B row (column of Y)
  // wn * kWN + 32 j + lr, block j 4096 bytes after block j - 1 (as for A)
  int bt_rd[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    bt_rd[kk] = BT ? (wn * kWN + lr) * 128 + 16 * ((2 * kk + lg) ^ (lr & 7) ^ ((lr >> 3) & 1)) : 0;
  // B rows per sub-step: 32 (int8) or 16 (16-bit k values)
  constexpr int kSubRows = KIND == kI8 ? 32 : 16;

  // per-column dequantization scales (kBf16F8)
  float bscale[WB];
#pragma unroll
  for (int j = 0; j < WB; ++j) bscale[j] = 1.f;
  if constexpr (KIND == kBf16F8) {
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const int64_t col = col0 + wn * kWN + j * 32 + lr;
      const int64_t si = grp * p.scale_grp_stride + (p.scale_per_col ? (col < N ? col : 0) : 0);
      bscale[j] = p.scale_f16 ? (float)static_cast<const _Float16 *>(p.scale)[si]
                              : static_cast<const float *>(p.scale)[si];
    }
  }
  // kOutQ8Row: the weight scale and bias of this lane's rows in the four
  // 32-row blocks, loaded here so that their latency hides under the K loop
  // instead of opening each block's epilogue
  float row_ws[OUT == kOutQ8Row ? 4 : 1] = {};
  int32_t row_b[OUT == kOutQ8Row ? 4 : 1] = {};
  if constexpr (OUT == kOutQ8Row) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + wm * 128 + i * 32 + lr;
      const int64_t rc = row < M ? row : 0;
      row_ws[i] = p.row_wscale[p.row_wscale_per ? rc : 0];
      row_b[i] = p.row_bias ? p.row_bias[rc] : 0;
    }
  }
  constexpr int aflip = (KIND == kI8 && AU8) ? (int)kFlip : 0;
  constexpr int bflip = (KIND == kI8 && BU8) ? (int)kFlip : 0;

  // Direct loads of K step `step` into ring stage `stage`: the L loads of a
  // step, numbered A pieces 0..7 then B pieces, in quarters (parts 0..3) or
  // all at once (part 4).
  auto issue = [&](int step, int stage, int part) __attribute__((always_inline)) {
    const bool live = step < nk;
    const unsigned ka = (unsigned)step * kStepBytes;
    unsigned kb = BT ? (unsigned)step * kStepBytes : (unsigned)((int64_t)step * T::kBRows * NB);
    if constexpr (CV) {
      // tap (i, j) and channel block of this step (scalar arithmetic)
      const uint32_t tap = DivMagic((uint32_t)step, p.cv.spt_magic);
      const uint32_t ti = DivMagic(tap, p.cv.kw_magic);
      kb = (unsigned)(ti * p.cv.tap_row + (tap - ti * (uint32_t)p.cv.kw) * p.cv.tap_col +
                      kStepBytes * ((uint32_t)step - tap * (uint32_t)p.cv.spt));
    }
    char *sa = SA(stage);
    char *sb = SB(stage);
    const __amdgpu_buffer_rsrc_t rsa = live ? rsA : rsA0, rsb = live ? rsB : rsB0;
    const int lo = part == 4 ? 0 : part * L / 4, hi = part == 4 ? L : (part + 1) * L / 4;
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q >= lo && q < hi)
        DirectLoad16(rsa, sa + (8 * wave + q) * 1024, a_g[q] + ka);
#pragma unroll
    for (int q = 0; q < LB; ++q)
      if (8 + q >= lo && 8 + q < hi)
        DirectLoad16(rsb, sb + (wave * LB + q) * 1024, b_g[q] + kb);
  };

  // ---- fragments ----
  // Sub-step s (4 per K step) multiplies A fragments ra[s % 3] by the B
  // fragments rb[s % 3] (kBf16F8: by the decoded operands bop[s % 2]).  Its
  // LDS reads were issued two sub-steps earlier and the fp8 decode ran under
  // the MFMAs of sub-step s - 1, so neither the LDS latency nor the decode
  // VALU work stalls the matrix pipe.
  v4i ra[3][4];
  v4i rb[3][WB];  // raw B: kI8 2 x tr8; kBf16F8 1 x tr8 (.xy); kH16 2 x tr16
  auto read = [&](int buf, const char *sa, const char *sb, int kk) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const char *base = sb + kk * kSubRows * kBP;
      if constexpr (BT) {
        rb[buf][j] = *reinterpret_cast<const v4i *>(sb + bt_rd[kk] + j * 4096);
      } else if constexpr (KIND == kI8) {
        const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)(base + b_rd[j]));
        const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)(base + b_rd[j] + 8 * kBP));
        rb[buf][j] = v4i{lo.x, lo.y, hi.x, hi.y};
      } else if constexpr (KIND == kBf16F8) {
        const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)(base + b_rd[j]));
        rb[buf][j] = v4i{v.x, v.y, 0, 0};
      } else {
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)(base + b_rd[j]));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)(base + b_rd[j] + 4 * kBP));
        rb[buf][j] = v4i{__builtin_bit_cast(v2i, lo).x, __builtin_bit_cast(v2i, lo).y,
                         __builtin_bit_cast(v2i, hi).x, __builtin_bit_cast(v2i, hi).y};
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[buf][i] = *reinterpret_cast<const v4i *>(sa + a_rd[kk] + i * 4096);
  };

  Acc acc[4][WB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < WB; ++j) acc[i][j] = Acc{0};
  int rsum[4] = {0, 0, 0, 0};  // kI8: partial row sums of a' (this lane's k group)
  int csum[WB];                // kI8: partial column sums of b'
#pragma unroll
  for (int j = 0; j < WB; ++j) csum[j] = 0;

  // kBf16F8: the decoded B operands, two sets.  The other kinds multiply the
  // fragments of the sub-step's own register set, so their B reads keep the
  // full two-sub-step look-ahead; uint8 fragments are turned into int8
  // (x ^ 0x80 = x - 128) in place one sub-step ahead, under the MFMAs of the
  // sub-step before (right before their own MFMAs the flips cost 4% more
  // cycles).
  v4i bop[KIND == kBf16F8 ? 2 : 1][WB];
  auto decode = [&](int rbuf, int bbuf) __attribute__((always_inline)) {
    if constexpr (KIND == kI8 && AU8) {
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[rbuf][i] ^= aflip;
    }
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      if constexpr (KIND == kI8 && BU8) {
        rb[rbuf][j] ^= bflip;
      } else if constexpr (KIND == kBf16F8) {
        // exact fp8 -> bf16: the high halves of the fp32 decode
        const v2f f0 = __builtin_amdgcn_cvt_pk_f32_fp8(rb[rbuf][j].x, false);
        const v2f f1 = __builtin_amdgcn_cvt_pk_f32_fp8(rb[rbuf][j].x, true);
        const v2f f2 = __builtin_amdgcn_cvt_pk_f32_fp8(rb[rbuf][j].y, false);
        const v2f f3 = __builtin_amdgcn_cvt_pk_f32_fp8(rb[rbuf][j].y, true);
        bop[bbuf][j] = v4i{(int)HighHalves(f0), (int)HighHalves(f1), (int)HighHalves(f2), (int)HighHalves(f3)};
      }
    }
  };
  // kI8 with zero points: this lane's partial column sums of b' over the
  // fragments in register set `buf` (one sub-step)
  auto colsum = [&](int buf) __attribute__((always_inline)) {
    if constexpr (KIND == kI8 && CB) {
#pragma unroll
      for (int j = 0; j < WB; ++j) {
        const v4i bv = rb[buf][j];
#pragma unroll
        for (int e = 0; e < 4; ++e) csum[j] = __builtin_amdgcn_sdot4(bv[e], 0x01010101, csum[j], false);
      }
    }
  };
  auto mma = [&](int abuf, int bbuf, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      if constexpr (KIND == kI8) {
        const v4i av = ra[abuf][i];
        if (RA) {
#pragma unroll
          for (int e = 0; e < 4; ++e) rsum[i] = __builtin_amdgcn_sdot4(av[e], 0x01010101, rsum[i], false);
        }
#pragma unroll
        for (int j = 0; j < WB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(rb[abuf][j], av, acc[i][j], 0, 0, 0);
      } else if constexpr (KIND == kBf16F8 || OUT == kOutBf16) {
        const v8bf av = __builtin_bit_cast(v8bf, ra[abuf][i]);
#pragma unroll
        for (int j = 0; j < WB; ++j) {
          v4i bv;
          if constexpr (KIND == kBf16F8) bv = bop[bbuf][j];
          else bv = rb[abuf][j];
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, bv), av, acc[i][j], 0, 0, 0);
        }
      } else {  // kH16 with FLOAT16 operands
        const v8h av = __builtin_bit_cast(v8h, ra[abuf][i]);
#pragma unroll
        for (int j = 0; j < WB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, rb[abuf][j]), av,
                                                             acc[i][j], 0, 0, 0);
      }
    }
  };

  // Instruction order inside a sub-step, pinned because the scheduler would
  // otherwise sink each LDS read next to its first use.
  constexpr int kReads = 4 + WB * (KIND == kBf16F8 ? 1 : 2);
  constexpr int kDecodeValu = KIND == kBf16F8 ? 8 * WB : (KIND == kI8 ? (AU8 ? 16 : 0) + (BU8 ? 4 * WB : 0) + (CB ? 4 * WB : 0) : 0);
  // A plain sub-step with `nvm` direct loads: each MFMA is preceded by its
  // share of the LDS reads two sub-steps ahead and followed by a direct load
  // and its share of the decode.  Reads issued all at once at the top of a
  // sub-step (4 waves x 8 reads) queue up in the LDS; one read per MFMA cost
  // 9% fewer cycles on C2.
  auto order_vm = [&](int nvm) __attribute__((always_inline)) {
    constexpr int kNM = 4 * WB;
#pragma unroll
    for (int x = 0; x < kNM; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x100, (kReads + kNM - 1) / kNM, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (x < nvm) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
      if constexpr (kDecodeValu > 0)
        __builtin_amdgcn_sched_group_barrier(0x002, (kDecodeValu + kNM - 1) / kNM, 0);  // VALU
    }
  };
  // second half of the barrier sub-step with `nvm` direct loads
  auto order_refill = [&](int nvm) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < 2 * WB; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x100, (kReads + 2 * WB - 1) / (2 * WB), 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);               // MFMA
      if (x < nvm) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
      if (x + 2 * WB < nvm) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if constexpr (kDecodeValu > 0)
        __builtin_amdgcn_sched_group_barrier(0x002, (kDecodeValu + 2 * WB - 1) / (2 * WB), 0);  // VALU
    }
  };
  // direct loads in refill quarter `part`
  auto quarter = [](int part) constexpr { return (part + 1) * L / 4 - part * L / 4; };

  // Sub-step s = 4 t + kk of K step t (ring stage t % 3); all buffer and
  // stage indices are compile-time after unrolling.  Sub-step kk == 2 holds
  // the step's barrier: every wave has retired its reads of stage t - 1 ... t
  // (its last reads of stage t were issued in sub-step kk == 1), and step
  // t + 1 has landed, so stage t is refilled with step t + 3 and the reads of
  // step t + 1 begin.  The refill is spread over four sub-steps (quarters in
  // sub-steps 2 and 3 of step t and 0 and 1 of step t + 1): issued in bursts,
  // the direct loads back up in the address unit and stall the MFMAs behind
  // them in each wave's instruction stream.
  auto substep = [&](int t, int kk, int sb3, int sb2, int cur, int nxt) __attribute__((always_inline)) {
    const int nb3 = (sb3 + 1) % 3, nb2 = (sb2 + 1) % 2, rb3 = (sb3 + 2) % 3;
    const int prv = (cur + 2) % 3;  // stage of step t - 1, being refilled with step t + 2
    if (kk != 2) {
      if (kk < 2) read(rb3, SA(cur), SB(cur), kk + 2);
      else read(rb3, SA(nxt), SB(nxt), kk - 2);
      if (kk == 3) issue(t + 3, cur, 1);
      else issue(t + 2, prv, 2 + kk);
      decode(nb3, nb2);
      colsum(sb3);
      mma(sb3, sb2, 0, 4);
      order_vm(kk == 3 ? quarter(1) : quarter(2 + kk));
      __builtin_amdgcn_sched_barrier(0);
    } else {
      mma(sb3, sb2, 0, 2);
      __builtin_amdgcn_sched_barrier(0);
      RingBarrier<L>();
      read(rb3, SA(nxt), SB(nxt), 0);
      issue(t + 3, cur, 0);  // first quarter of the refill
      decode(nb3, nb2);
      colsum(sb3);
      mma(sb3, sb2, 2, 4);
      order_refill(quarter(0));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // one full K step t whose first sub-step index s = 4t has s % 3 == r3
  auto step = [&](int t, int r3, int cur, int nxt) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) substep(t, kk, (r3 + kk) % 3, kk % 2, cur, nxt);
  };
  // A final half step (K % kKStep == kKStep / 2) runs 2 of the 4 sub-steps;
  // its stage was loaded whole (k past K: zero rows of B, unread bytes of A).
  auto half_step = [&](int r3) __attribute__((always_inline)) {
    decode((r3 + 1) % 3, 1);
    colsum(r3);
    colsum((r3 + 1) % 3);
    mma(r3, 0, 0, 4);
    mma((r3 + 1) % 3, 1, 0, 4);
  };

  // Zero points of this lane's rows (32i + lr) and columns (32j + lr).
  uint32_t za[4] = {0, 0, 0, 0}, zb[4] = {0, 0, 0, 0};  // raw zero-point bytes
  auto load_zp = [&]() __attribute__((always_inline)) {
    if constexpr (KIND == kI8 && ZP) {
      const __amdgpu_buffer_rsrc_t rsZa =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.a_zp), (short)0, (int)(p.a_zp ? M : 0), kRsrcWord3);
      const __amdgpu_buffer_rsrc_t rsZb =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p.b_zp), (short)0, (int)(p.b_zp ? N : 0), kRsrcWord3);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t row = row0 + wm * 128 + i * 32 + lr;
        za[i] = __builtin_amdgcn_raw_buffer_load_b8(rsZa, row < M ? (unsigned)row : kOob, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < WB; ++j) {
        const int64_t col = col0 + wn * kWN + j * 32 + lr;
        zb[j] = __builtin_amdgcn_raw_buffer_load_b8(rsZb, col < N ? (unsigned)col : kOob, 0, 0);
      }
    }
  };

  // A single half step (K <= kKStep / 2, e.g. attention scores over a 64-wide
  // head) needs one stage and no look-ahead: it and the zero points are
  // loaded together, and each 32-row block's MFMAs come right before its
  // epilogue, so the output stores start after the first block.
  // WB = 4 serves only whole K steps (the launcher checks K % kKStep == 0):
  // without the half-step and single-step paths the register allocator keeps
  // all 256 accumulators in registers through the loop.
  constexpr bool kWhole = WB == 4;
  const bool block_major = !kWhole && nfull == 0;  // then half is set (K > 0)
  if (block_major) {
    issue(0, 0, 4);
    load_zp();
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read(0, sa0, sb0, 0);
    read(1, sa0, sb0, 1);
    decode(0, 0);
    decode(1, 1);
    colsum(0);  // before the zero-point exchange; the MFMAs run block by block in the epilogue
    colsum(1);
  } else {
    // steps 0 and 1 whole, the first half of step 2 (sub-steps 0 and 1 of
    // step 0 issue the rest)
    issue(0, 0, 4);
    issue(1, 1, 4);
    issue(2, 2, 0);
    issue(2, 2, 1);
    RingBarrier<L + 2 * L / 4>();
    read(0, sa0, sb0, 0);
    read(1, sa0, sb0, 1);
    decode(0, 0);
    int t = 0;
    // 12 sub-steps per iteration: s % 3 and the stages repeat.  The last
    // iteration's missing steps are skipped by uniform branches inside the
    // loop: steps after the loop (another path with every accumulator live)
    // made the register allocator spill the 256 accumulators of WB = 4 inside
    // the loop.
    for (; t < nfull; t += 3) {
      step(t, 0, 0, 1);
      if (t + 1 < nfull) step(t + 1, 1, 1, 2);
      if (t + 2 < nfull) step(t + 2, 2, 2, 0);
    }
    if (!kWhole && half) {
      const int r3 = nfull % 3;  // (4 * nfull) % 3
      if (r3 == 0) half_step(0);
      else if (r3 == 1) half_step(1);
      else half_step(2);
    }
    // the zero points load after the last hand-counted wait (the K loop
    // keeps every register busy); then drain the look-ahead (out-of-range)
    // loads before the LDS is reused
    load_zp();
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // ---- zero-point terms (kI8 with zero points) ----
  // A wave holds the full K range of its 128 rows and kWN columns, so the
  // terms never cross waves: RA of row 32i + lr is rsum[i] plus its other lane
  // half, alpha is in zrow; CB and beta of the wave's columns go through the
  // wave's own LDS area to the lanes that store those columns.  Per element
  // Y = sum a'b' + beta_j RA_i + alpha_i Q_j with Q_j = CB_j + K beta_j
  // (mod 2^32); below K = 21845 every factor fits 24 signed bits, and the
  // full-rate 24-bit multiplies give the same low 32 bits.
  const bool mul24 = K < 21845;
  // the scalar constants, read here (after the last load of the ring) when
  // they are device-resident
  QResolved qv{p.alpha_scalar, p.beta_scalar, p.cs, p.zy};
  if constexpr (KIND == kI8) qv = ResolveQ(p.dev, p.a_u8, p.b_u8, p.y_signed, p.alpha_scalar, p.beta_scalar, p.cs, p.zy);
  int32_t *zc = zsum + (KIND == kI8 && ZP ? wave * 2 * kWN : 0);
  int zrow[4] = {0, 0, 0, 0};
  if constexpr (KIND == kI8 && ZP) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      zrow[i] = p.a_zp ? (p.a_u8 ? 128 - (int)za[i] : -(int)(int8_t)za[i]) : qv.alpha;
#pragma unroll
    for (int j = 0; j < WB; ++j) {
      const int v = csum[j] + __shfl_xor(csum[j], 32);
      if (lg == 0) {
        const int be = p.b_zp ? (p.b_u8 ? 128 - (int)zb[j] : -(int)(int8_t)zb[j]) : qv.beta;
        zc[j * 32 + lr] = (int)((unsigned)v + (unsigned)K * (unsigned)be);  // CB + K beta (mod 2^32)
        zc[kWN + j * 32 + lr] = be;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // kBf16F8: the scales of the wave's columns, to the lanes that store them
  float *csc = cscale + (KIND == kBf16F8 ? wave * kWN : 0);
  if constexpr (KIND == kBf16F8) {
#pragma unroll
    for (int j = 0; j < WB; ++j)
      if (lg == 0) csc[j * 32 + lr] = bscale[j];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- epilogue ----
  // The MFMAs compute the transposed block (B fragment as the row operand),
  // so lane (lr, lg) of block (i, j) holds output row 32i + lr and, in
  // registers 4g .. 4g+3, the four consecutive columns 32j + 8g + 4lg + 0..3.
  // Per 32-row block the wave packs those four values, stages the block in LDS
  // (row pitch padded by 16 bytes) and writes whole 16-byte row pieces.
  constexpr int kPitch = kWN * kOsz + 16;
  static_assert(32 * kPitch <= 16384 && 2 * 16384 <= kAStage, "epilogue staging: 32 rows per wave, two waves per stage");
  // Staging areas in ring stages 1 and 2: the block-major path (one half
  // step) loads only stage 0 and writes a block's outputs while the partner
  // wave (same wm) may still read its fragments from stage 0; the full path
  // has drained every stage behind a barrier.
  char *stg = (wave >> 1 ? sa2 : sa1) + (wave & 1) * 16384;
  // QLinearMatMul requantization constants (signed outputs biased by 128)
  const float q_bias = p.y_signed ? 128.f : 0.f;
  const float q_zy = qv.zy + q_bias, q_lo = p.qmin + q_bias, q_hi = p.qmax + q_bias;
  const unsigned q_flip = p.y_signed ? 0x80808080u : 0u;
  // Grouped mode with a bias: the bias of this lane's columns (4 per
  // (j, g) register group, the output dtype's bits).  GroupedMatMul adds it
  // as MatMul followed by Add does: the sum rounded to the output dtype, the
  // bias added in fp32, rounded again.
  v2i gbias[GRP ? WB : 1][4];
  const bool has_gbias = GRP && p.grp_bias != nullptr;
  if constexpr (GRP) {
    const __amdgpu_buffer_rsrc_t rsBias = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(p.grp_bias), (short)0, has_gbias ? (int)(p.grp_count * N * kOsz) : 0, kRsrcWord3);
#pragma unroll
    for (int j = 0; j < WB; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = col0 + wn * kWN + j * 32 + g * 8 + lg * 4;
        gbias[j][g] = __builtin_amdgcn_raw_buffer_load_b64(
            rsBias, col < N ? (unsigned)((grp * N + col) * kOsz) : kOob, 0, 0);
      }
  }
  // Epilogue of 32-row block i (use24: the 24-bit zero-point products).
  auto epi = [&](int i, auto use24) __attribute__((always_inline)) {
    int32_t ra_r = 0, al_r = 0;
    if constexpr (KIND == kI8 && ZP) {
      ra_r = rsum[i] + __shfl_xor(rsum[i], 32);
      al_r = zrow[i];
    }
    // kOutQ8Row: this lane's output row (row0 + wm * 128 + 32 i + lr) scale
    // and bias (loaded before the K loop), computed with the fp32 operations
    // of the reference
    float cs_r = qv.cs;
    double bias_r = 0.0;
    if constexpr (OUT == kOutQ8Row) {
      cs_r = p.row_xs * row_ws[i] / p.row_ys;
      bias_r = (double)row_b[i];
    }
#pragma unroll
    for (int j = 0; j < WB; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = j * 32 + g * 8 + lg * 4;  // first of the 4 columns (within the wave tile)
        char *dst = stg + lr * kPitch + cl * kOsz;
        if constexpr (KIND == kI8) {
          unsigned v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = (unsigned)acc[i][j][4 * g + e];
            if constexpr (ZP) {
              // Y = sum a'b' + beta_j RA_i + alpha_i CB_j + K alpha_i beta_j (mod 2^32)
              const int be = zc[kWN + cl + e], q = zc[cl + e];
              if constexpr (decltype(use24)::value)
                v[e] += (unsigned)(__mul24(be, ra_r) + __mul24(al_r, q));
              else
                v[e] += (unsigned)be * (unsigned)ra_r + (unsigned)al_r * (unsigned)q;
            }
          }
          if constexpr (OUT == kOutI32) {
            *reinterpret_cast<v4i *>(dst) = v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
          } else {
            // ties-to-even rounding before the zero point, then saturation.
            // Signed outputs are biased by 128 (exact on these integer
            // values) so one byte conversion packs both kinds; the XOR
            // removes the bias.
            unsigned packed = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float f;
              if constexpr (OUT == kOutQ8Row) {
                // (float) of the exact int64 sum acc + bias (the double sum is
                // exact below 2^53); NaN lands as 0 as through the x86-64 cast
                f = __builtin_rintf((float)((double)(int32_t)v[e] + bias_r) * cs_r) + q_zy;
                if (f != f) f = q_bias;
              } else {
                f = __builtin_rintf((float)(int32_t)v[e] * qv.cs) + q_zy;
              }
              packed = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(f, q_lo, q_hi), e, packed);
            }
            *reinterpret_cast<unsigned *>(dst) = packed ^ q_flip;
          }
        } else {
          Acc a = acc[i][j];
          if constexpr (KIND == kBf16F8) {  // the columns' dequantization scales
            const v4f sc4 = *reinterpret_cast<const v4f *>(csc + cl);
#pragma unroll
            for (int e = 0; e < 4; ++e) a[4 * g + e] *= sc4[e];
          }
          if constexpr (GRP) {
            if (has_gbias) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const unsigned bb = ((unsigned)gbias[j][g][e >> 1] >> (16 * (e & 1))) & 0xffffu;
                float r, bv;
                if constexpr (OUT == kOutBf16) {
                  r = __builtin_bit_cast(float, (PackBf16(a[4 * g + e], 0.f) & 0xffffu) << 16);
                  bv = __builtin_bit_cast(float, bb << 16);
                } else {
                  r = (float)(_Float16)a[4 * g + e];
                  bv = (float)__builtin_bit_cast(_Float16, (unsigned short)bb);
                }
                a[4 * g + e] = r + bv;
              }
            }
          }
          if constexpr (OUT == kOutBf16) {
            *reinterpret_cast<v2i *>(dst) = v2i{(int)PackBf16(a[4 * g], a[4 * g + 1]),
                                                (int)PackBf16(a[4 * g + 2], a[4 * g + 3])};
          } else {
            typedef _Float16 v4h __attribute__((ext_vector_type(4)));
            const v4h h = {(_Float16)a[4 * g], (_Float16)a[4 * g + 1], (_Float16)a[4 * g + 2],
                           (_Float16)a[4 * g + 3]};
            *reinterpret_cast<v4h *>(dst) = h;
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 32 rows x kWN columns x kOsz bytes in 16-byte pieces, WB * kOsz per lane
    constexpr int kChunksPerRow = kWN * kOsz / 16;
    // Branch-free stores: pieces outside the matrix get an offset past the
    // buffer, which the buffer store drops; all LDS reads issue first.
    const int64_t brow = row0 + wm * 128 + i * 32;
    const int64_t ncol = N - (col0 + wn * kWN);
    const unsigned ybase = (unsigned)((brow * LDY + col0 + wn * kWN) * kOsz);
    // grouped mode: each staged row goes to its own row of Y
    unsigned grow[WB * kOsz];
#pragma unroll
    for (int c = 0; c < WB * kOsz; ++c) {
      grow[c] = 0;
      if constexpr (GRP) {
        const int rr = (c * 64 + lane) / kChunksPerRow;
        if (brow + rr < rcount)
          grow[c] = (unsigned)(((int64_t)p.grp_rows[rbase + brow + rr] * LDY + col0 + wn * kWN) * kOsz);
      }
    }
    v4i piece[WB * kOsz];
#pragma unroll
    for (int c = 0; c < WB * kOsz; ++c) {
      const int id = c * 64 + lane;
      const int rr = id / kChunksPerRow, cc = id % kChunksPerRow;
      piece[c] = *reinterpret_cast<const v4i *>(stg + rr * kPitch + cc * 16);
    }
#pragma unroll
    for (int c = 0; c < WB * kOsz; ++c) {
      const int id = c * 64 + lane;
      const int rr = id / kChunksPerRow, cc = id % kChunksPerRow;
      const bool ok = brow + rr < rcount && cc * (16 / kOsz) < ncol;
      const unsigned at = GRP ? grow[c] + (unsigned)(cc * 16) : ybase + (unsigned)(rr * LDY * kOsz + cc * 16);
      __builtin_amdgcn_raw_buffer_store_b128(piece[c], rsY, ok ? at : kOob, 0, kStoreThrough);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (block_major) {
      mma(0, 0, i, i + 1);
      mma(1, 1, i, i + 1);
    }
    if (!(KIND == kI8 && ZP) || mul24) epi(i, std::true_type{});
    else epi(i, std::false_type{});
  }
}

// Host-side eligibility of the pipelined kernel for a problem: K a multiple
// of half the K step (a trailing half step is allowed), N a multiple of 16, 16-byte aligned operands and output, and
// every per-matrix byte offset (plus the look-ahead) below 2^31 - 2^24.
template <int KIND> inline bool Eligible(const GemmArgs &p) {
  constexpr int kAsz = KIND == kI8 ? 1 : 2, kBsz = KIND == kH16 ? 2 : 1;
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  const int64_t ldb = p.ldb ? p.ldb : p.N, ldy = p.ldy ? p.ldy : p.N;
  auto al = [](const void *q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  return p.K > 0 && p.K % (Traits<KIND>::kKStep / 2) == 0 && p.N % 16 == 0 && ldb % 16 == 0 && ldy % 16 == 0 &&
         ldb >= p.N && ldy >= p.N && al(p.A) && al(p.B) && al(p.Y) && p.M * p.K * kAsz + 4 * kStepBytes < lim &&
         p.M * ldy * 4 < lim && (p.K + 3 * Traits<KIND>::kKStep) * ldb * kBsz < lim;
}

template <int KIND, int OUT, bool ZP, bool AU8, bool BU8, int WB = 2, bool CV = false>
inline void Launch(const GemmArgs &p, hipStream_t s) {
  constexpr int kBN = 64 * WB;
  const int64_t tiles = ((p.M + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN) * p.batch;
  hipLaunchKernelGGL((MfmaGemmKernel<KIND, OUT, ZP, AU8, BU8, WB, 0, CV>), dim3((unsigned)tiles), dim3(kThreads),
                     0, s, p);
}

// Eligibility with B given transposed ([N, K] row-major, GM == 3): K a
// multiple of half the K step, N a multiple of 16, 16-byte aligned operands
// and output, and each matrix's bytes (plus the look-ahead) below 2^31 - 2^24.
inline bool EligibleBT(const GemmArgs &p) {
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  auto al = [](const void *q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  return p.K > 0 && p.K % (Traits<kH16>::kKStep / 2) == 0 && p.N % 16 == 0 && p.batch == 1 && al(p.A) &&
         al(p.B) && al(p.Y) && p.M * p.K * 2 + 4 * kStepBytes < lim && p.N * p.K * 2 + 4 * kStepBytes < lim &&
         p.M * p.N * 2 < lim;
}

template <int OUT> inline void LaunchBT(const GemmArgs &p, hipStream_t s) {
  const int64_t tiles = ((p.M + kBM - 1) / kBM) * ((p.N + 127) / 128);
  hipLaunchKernelGGL((MfmaGemmKernel<kH16, OUT, false, false, false, 2, 3>), dim3((unsigned)tiles), dim3(kThreads), 0,
                     s, p);
}

// Grouped launch: `max_tiles` workgroups, an upper bound of the tiles the
// routing table holds (the rest leave at once).
// WB = 4 (256-column tiles, fp8 B only) needs K % kKStep == 0 and routing
// tables counted in 256-column tiles.
template <int OUT, int GM, int KIND = kH16, int WB = 2>
inline void LaunchGrouped(const GemmArgs &p, int64_t max_tiles, hipStream_t s) {
  hipLaunchKernelGGL((MfmaGemmKernel<KIND, OUT, false, false, false, WB, GM>), dim3((unsigned)max_tiles),
                     dim3(kThreads), 0, s, p);
}

}  // namespace mg
}  // namespace onnxl_amd
