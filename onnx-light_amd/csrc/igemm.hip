// int8 MFMA GEMM for gfx950, shared by MatMulInteger (int32 output) and
// QLinearMatMul (requantised u8/s8 output).
//
// Tile: 256 x 128 outputs per 256-thread workgroup (4 waves, 2 x 2), each
// wave 128 x 64 = 4 x 2 blocks of v_mfma_i32_32x32x32_i8, K step 64.
//  - A (row-major [M,K], K contiguous) is loaded straight into MFMA operand
//    registers, one K step ahead: lane (r, g) holds row r, bytes
//    [k0 + 32g, k0 + 32g + 32).  The two waves that share rows read the same
//    lines; the second read hits L2.
//  - B (row-major [K,N], N contiguous) must reach the MFMA as 16 consecutive
//    k of one column, so each thread loads a 4(k) x 8(n) byte block, transposes
//    it in registers and stores 4-byte k-quads into an LDS tile laid out
//    [n][k] with XOR-swizzled 16-byte chunks; double-buffered, one barrier per
//    K step.
//  - Operand bytes are a' = a ^ 0x80 for UINT8 (= a - 128) so the signed MFMA
//    applies; the zero-point algebra in kernels.hpp restores the exact result.
//    The row / column sums it needs come from extra MFMAs against an all-ones
//    operand, which land in exactly the lanes that hold the matching outputs.
//  - Workgroup ids are remapped so each XCD (8 on MI355X, ids dealt
//    round-robin) owns a contiguous run of tiles, grouped 8 tile-rows high,
//    so tiles sharing A rows / B columns share that XCD's L2.
#include "kernels.hpp"

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

// LDS B tile [kBN][kBK] bytes; 16-byte chunk c of column n sits at chunk
// c ^ swz(n), which keeps both the transposing 4-byte stores and the 16-byte
// fragment reads spread over the banks.
__device__ __forceinline__ int BOff(int n, int chunk) {
  const int swz = ((n >> 1) ^ (n >> 3)) & 3;
  return n * kBK + ((chunk ^ swz) << 4);
}

// 4x4 byte transpose of rows r0..r3: d[j] = (r0.byte j, r1.byte j, r2.byte j, r3.byte j).
__device__ __forceinline__ void Transpose4x4(unsigned r0, unsigned r1, unsigned r2, unsigned r3,
                                             unsigned d[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int s = 8 * j;
    d[j] = ((r0 >> s) & 0xffu) | (((r1 >> s) & 0xffu) << 8) | (((r2 >> s) & 0xffu) << 16) |
           (((r3 >> s) & 0xffu) << 24);
  }
}

__device__ __forceinline__ int64_t MinI64(int64_t a, int64_t b) { return a < b ? a : b; }

template <int EPI, bool NEED_RA, bool NEED_CB, bool VEC>
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

  // ---- A: straight to operand registers ----
  auto load_a = [&](int64_t k0, v4i(&dst)[4][2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + wm * 128 + i * 32 + lr;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t kc = k0 + 32 * lg + 16 * h;
        v4i v = {0, 0, 0, 0};
        if (row < M && kc < K) {
          const int8_t *src = Ab + row * K + kc;
          if (VEC) {
            v = *reinterpret_cast<const v4i *>(src);
            v ^= (int)aflip;
          } else {
            unsigned w[4] = {0, 0, 0, 0};
            for (int e = 0; e < 16; ++e) {
              if (kc + e < K) {
                const unsigned byte = ((unsigned)(uint8_t)src[e]) ^ (aflip & 0xffu);
                w[e >> 2] |= byte << (8 * (e & 3));
              }
            }
            v = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
          }
        }
        dst[i][h] = v;
      }
    }
  };

  // ---- B: 4(k) x 8(n) block per thread -> transposed k-quads in LDS ----
  const int bno = tid & 15, bkq = tid >> 4;
  unsigned bst[4][2];
  auto load_b = [&](int64_t k0) {
    const int64_t n = col0 + 8 * bno;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t k = k0 + 4 * bkq + r;
      unsigned lo = 0, hi = 0;
      if (k < K && n < N) {
        const int8_t *src = Bb + k * N + n;
        if (VEC) {
          const v2i v = *reinterpret_cast<const v2i *>(src);
          lo = (unsigned)v.x ^ bflip;
          hi = (unsigned)v.y ^ bflip;
        } else {
          for (int e = 0; e < 8; ++e) {
            if (n + e < N) {
              const unsigned byte = ((unsigned)(uint8_t)src[e]) ^ (bflip & 0xffu);
              if (e < 4) lo |= byte << (8 * e); else hi |= byte << (8 * (e - 4));
            }
          }
        }
      }
      bst[r][0] = lo;
      bst[r][1] = hi;
    }
  };
  auto store_b = [&](int8_t *dst) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      unsigned d[4];
      Transpose4x4(bst[0][h], bst[1][h], bst[2][h], bst[3][h], d);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = 8 * bno + 4 * h + j;
        *reinterpret_cast<unsigned *>(dst + BOff(n, bkq >> 2) + 4 * (bkq & 3)) = d[j];
      }
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

  v4i a_cur[4][2], a_nxt[4][2];
  const int nk = (int)((K + kBK - 1) / kBK);
  if (nk > 0) {
    load_a(0, a_cur);
    load_b(0);
    store_b(lds_b[0]);
  }
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const bool more = it + 1 < nk;
    if (more) {
      load_a((int64_t)(it + 1) * kBK, a_nxt);
      load_b((int64_t)(it + 1) * kBK);
    }
    const int8_t *bt_lds = lds_b[it & 1];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      v4i bf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = wn * 64 + j * 32 + lr;
        bf[j] = *reinterpret_cast<const v4i *>(bt_lds + BOff(n, 2 * lg + kk));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur[i][kk], bf[j], acc[i][j], 0, 0, 0);
        if (NEED_RA) ra[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur[i][kk], ones, ra[i], 0, 0, 0);
      }
      if (NEED_CB) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          cb[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ones, bf[j], cb[j], 0, 0, 0);
      }
    }
    if (more) store_b(lds_b[(it + 1) & 1]);
    __syncthreads();
    if (more) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a_cur[i][0] = a_nxt[i][0];
        a_cur[i][1] = a_nxt[i][1];
      }
    }
  }

  // ---- epilogue: lane (lr, lg) of block (i, j) holds column j*32+lr,
  // rows (q/4)*8 + lg*4 + q%4 of register q ----
  const unsigned Ku = (unsigned)K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int64_t row = row0 + wm * 128 + i * 32 + (q >> 2) * 8 + lg * 4 + (q & 3);
      if (row >= M) continue;
      const unsigned alpha =
          p.a_zp ? (unsigned)(p.a_u8 ? 128 - (int)p.a_zp[row] : -(int)(int8_t)p.a_zp[row])
                 : (unsigned)p.alpha_scalar;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t col = col0 + wn * 64 + j * 32 + lr;
        if (col >= N) continue;
        const unsigned beta =
            p.b_zp ? (unsigned)(p.b_u8 ? 128 - (int)p.b_zp[col] : -(int)(int8_t)p.b_zp[col])
                   : (unsigned)p.beta_scalar;
        unsigned v = (unsigned)acc[i][j][q];
        if (NEED_RA) v += beta * (unsigned)ra[i][q];
        if (NEED_CB) v += alpha * (unsigned)cb[j][q];
        v += Ku * alpha * beta;
        const int64_t yi = (bt * M + row) * N + col;
        if (EPI == kEpiInt32) {
          reinterpret_cast<int32_t *>(p.Y)[yi] = (int32_t)v;
        } else {
          float f = (float)(int32_t)v * p.cs;
          f = __builtin_rintf(f) + p.zy;
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

template <int EPI, bool RA, bool CB>
void LaunchVec(const IGemmParams &p, bool vec, dim3 grid, hipStream_t s) {
  if (vec) {
    hipLaunchKernelGGL((IGemmKernel<EPI, RA, CB, true>), grid, dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((IGemmKernel<EPI, RA, CB, false>), grid, dim3(kThreads), 0, s, p);
  }
}

template <int EPI>
void LaunchEpi(const IGemmParams &p, bool vec, dim3 grid, hipStream_t s) {
  if (p.need_ra) {
    if (p.need_cb) LaunchVec<EPI, true, true>(p, vec, grid, s);
    else LaunchVec<EPI, true, false>(p, vec, grid, s);
  } else {
    if (p.need_cb) LaunchVec<EPI, false, true>(p, vec, grid, s);
    else LaunchVec<EPI, false, false>(p, vec, grid, s);
  }
}

}  // namespace

void LaunchIGemm(const IGemmParams &p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return;
  const int64_t tiles = ((p.M + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN) * p.batch;
  // 16-byte A rows and 8-byte B rows: every batch base and row start aligned.
  const bool vec = (p.K % 16 == 0) && (p.N % 8 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.A) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(p.B) % 8 == 0);
  const dim3 grid((unsigned)tiles);
  if (p.epilogue == kEpiInt32) LaunchEpi<kEpiInt32>(p, vec, grid, stream);
  else LaunchEpi<kEpiQuant8>(p, vec, grid, stream);
}

}  // namespace onnxl_amd
