// ConvInteger (nn/kernel_conv_integer.cc) and QLinearConv
// (kq/kernel_qlinearconv.cc) on the int8 GEMM core.
//
// For output channel m of group g and batch n the convolution is the GEMM
//   Y[n, g*Mg + r, p] = sum_k W[g*Mg + r, k] * Col[n, g, k, p]
// over k = (input channel of the group, kernel tap), with W in its ONNX
// layout [M, C/group, kernel...] (already the row-major A operand) and Col
// built by ImToColKernel: Col[n, g, k, p] is the input byte the tap reads for
// output position p, or x's zero point where the tap falls into the padding
// (which then contributes (x_zp - x_zp) * (w - w_zp) = 0, exactly the
// reference's skipped tap).  The GEMM output [n, g, Mg, P] is the NCHW output.
//
// DirectConvKernel computes the same sums one output per thread: the path for
// grouped convolutions with per-channel weight zero points (whose zero point
// would change along the GEMM batch), and for QLinearConv sums that int32
// does not hold exactly.  ConvRequantKernel applies QLinearConv's bias and
// requantization to the GEMM's int32 sums.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {
namespace {

constexpr int kCBlock = 256;

// Input coordinates of output position p and kernel tap (kz, ky, kx) along
// the three right-aligned spatial dims; false when the tap is in the padding.
__device__ __forceinline__ bool TapOffset(const ConvGeom &g, int64_t oz, int64_t oy, int64_t ox, int kz, int ky,
                                          int kx, int64_t &off) {
  const int64_t iz = oz * g.s[0] - g.pb[0] + kz * g.d[0];
  const int64_t iy = oy * g.s[1] - g.pb[1] + ky * g.d[1];
  const int64_t ix = ox * g.s[2] - g.pb[2] + kx * g.d[2];
  if (iz < 0 || iz >= g.in[0] || iy < 0 || iy >= g.in[1] || ix < 0 || ix >= g.in[2]) return false;
  off = (iz * g.in[1] + iy) * g.in[2] + ix;
  return true;
}

// Col[n, g, k, p] for a row (n, g, k) and 4 consecutive positions per thread.
__global__ __launch_bounds__(kCBlock) void ImToColKernel(const ConvGeom g, const uint8_t *x, uint8_t x_zp,
                                                          uint8_t *col) {
  const int64_t quads = (g.P + 3) / 4;
  const int64_t t = (int64_t)blockIdx.x * kCBlock + threadIdx.x;
  const int64_t rows = g.N * g.G * g.Kc;
  if (t >= rows * quads) return;
  const int64_t row = t / quads;
  const int64_t p0 = (t - row * quads) * 4;
  const int64_t k = row % g.Kc;
  const int64_t ng = row / g.Kc;  // n * G + grp
  const int64_t c = k / g.ks, tap = k - c * g.ks;
  const int kx = (int)(tap % g.k[2]), ky = (int)((tap / g.k[2]) % g.k[1]), kz = (int)(tap / (g.k[2] * g.k[1]));
  const int64_t grp = ng % g.G, n = ng / g.G;
  const uint8_t *plane = x + ((n * g.C + grp * g.cpg + c) * g.in_size);
  int64_t ox = p0 % g.out[2], oy = (p0 / g.out[2]) % g.out[1], oz = p0 / (g.out[2] * g.out[1]);
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint8_t v = x_zp;
    int64_t off;
    if (p0 + e < g.P && TapOffset(g, oz, oy, ox, kz, ky, kx, off)) v = plane[off];
    word |= (uint32_t)v << (8 * e);
    if (++ox == g.out[2]) {
      ox = 0;
      if (++oy == g.out[1]) {
        oy = 0;
        ++oz;
      }
    }
  }
  uint8_t *dst = col + row * g.P + p0;
  if (p0 + 4 <= g.P && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
    *reinterpret_cast<uint32_t *>(dst) = word;
  } else {
    for (int e = 0; e < 4 && p0 + e < g.P; ++e) dst[e] = (uint8_t)(word >> (8 * e));
  }
}

// Col rows of kPlanesPerBlock consecutive input planes (n, channel c of
// group grp) for every kernel tap: the planes are staged in LDS once, each
// thread decodes its 4 output positions once (32-bit arithmetic) and writes
// the ks rows Col[n, grp, c_in_group * ks + tap, p0 .. p0 + 3] of each plane.
// Several planes per workgroup keep enough loads in flight: one plane per
// workgroup left the pass waiting on plane loads.  For planes up to
// kPlaneMax bytes, 2-D or 1-D (the leading slot of the geometry is 1).
constexpr int kPlaneMax = 12 * 1024;  // per plane; kPlanesPerBlock of them share the LDS
constexpr int kPlanesPerBlock = 4;

template <int KH, int KW>  // 0: the kernel extent from the geometry
__global__ __launch_bounds__(kCBlock) void ImToColPlaneKernel(const ConvGeom g, const uint8_t *x, uint8_t x_zp,
                                                               uint8_t *col) {
  // kPlanesPerBlock planes of in_size bytes each (dynamic: occupancy follows
  // the plane size); their loads are all in flight before the first wait
  extern __shared__ __align__(16) uint8_t planes[];
  const uint32_t in_size = (uint32_t)g.in_size, P = (uint32_t)g.P;
  const int64_t nplanes = g.N * g.C;
  const int64_t first = (int64_t)blockIdx.x * kPlanesPerBlock;
  const int count = (int)std::min<int64_t>(kPlanesPerBlock, nplanes - first);
  const uint32_t lds_pitch = (in_size + 15) & ~15u;
  for (int pl = 0; pl < count; ++pl) {
    const uint8_t *src = x + (first + pl) * in_size;
    for (uint32_t i = threadIdx.x; i < in_size; i += kCBlock) planes[pl * lds_pitch + i] = src[i];
  }
  __syncthreads();
  const uint32_t C = (uint32_t)g.C, cpg = (uint32_t)g.cpg;
  const int H = (int)g.in[1], W = (int)g.in[2], OW = (int)g.out[2];
  const int sy = (int)g.s[1], sx = (int)g.s[2], dy = (int)g.d[1], dx = (int)g.d[2];
  const int py = (int)g.pb[1], px = (int)g.pb[2];
  const int kh = KH ? KH : g.k[1], kw = KW ? KW : g.k[2];
  for (uint32_t p0 = threadIdx.x * 4; p0 < P; p0 += kCBlock * 4) {
    int oy[4], ox[4];
    const uint32_t q = p0 / (uint32_t)OW;
    oy[0] = (int)q;
    ox[0] = (int)(p0 - q * (uint32_t)OW);
#pragma unroll
    for (int e = 1; e < 4; ++e) {
      ox[e] = ox[e - 1] + 1;
      oy[e] = oy[e - 1];
      if (ox[e] == OW) {
        ox[e] = 0;
        ++oy[e];
      }
    }
    const int nvalid = (int)min(4u, P - p0);
    for (int pl = 0; pl < count; ++pl) {
      const int64_t nc = first + pl;  // n * C + channel
      const uint32_t n = (uint32_t)(nc / C), ch = (uint32_t)(nc - (int64_t)n * C);
      const uint32_t grp = ch / cpg, ci = ch - grp * cpg;
      // first Col row of this plane: (n * G + grp) * Kc + ci * ks
      uint8_t *rows = col + (((int64_t)n * g.G + grp) * g.Kc + (int64_t)ci * kh * kw) * P;
      const uint8_t *plane = planes + pl * lds_pitch;
#pragma unroll
      for (int ky = 0; ky < kh; ++ky)
#pragma unroll
        for (int kx = 0; kx < kw; ++kx) {
          const int tap = ky * kw + kx;
          uint32_t word = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int iy = oy[e] * sy - py + ky * dy, ix = ox[e] * sx - px + kx * dx;
            const bool in = e < nvalid && iy >= 0 && iy < H && ix >= 0 && ix < W;
            word |= (uint32_t)(in ? plane[iy * W + ix] : x_zp) << (8 * e);
          }
          uint8_t *dst = rows + (int64_t)tap * P + p0;
          if (nvalid == 4 && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
            *reinterpret_cast<uint32_t *>(dst) = word;
          } else {
            for (int e = 0; e < nvalid; ++e) dst[e] = (uint8_t)(word >> (8 * e));
          }
        }
    }
  }
}

__device__ __forceinline__ int32_t ByteValue(const uint8_t *p, int64_t i, int is_u8) {
  return is_u8 ? (int32_t)p[i] : (int32_t)(int8_t)p[i];
}

// The reference's saturating requantization (kernel_qlinearconv.cc:127-138,
// :332-339): ties-to-even, zero point, clamp; NaN lands as 0 as it does
// through the x86-64 conversion.
__device__ __forceinline__ uint8_t Requant(int64_t acc, float cs, const ConvQuant &q) {
  const float v = __builtin_rintf((float)acc * cs) + q.zy;
  if (v != v) return 0;
  return (uint8_t)(int32_t)__builtin_amdgcn_fmed3f(v, q.qmin, q.qmax);
}

__device__ __forceinline__ float CombinedScale(const ConvQuant &q, int64_t m) {
  const float ws = q.w_scale[q.w_scale_per_channel ? m : 0];
  return q.x_scale * ws / q.y_scale;  // left to right, as :289
}

// One output per thread: (n, m, p) over the group's input channels and taps.
// QUANT: int64 sum, bias, requantization (QLinearConv); otherwise the int32
// wrap of ConvInteger.
template <bool QUANT>
__global__ __launch_bounds__(kCBlock) void DirectConvKernel(const ConvGeom g, const uint8_t *x, int x_u8,
                                                             uint8_t x_zp, const uint8_t *w, int w_u8,
                                                             const uint8_t *w_zp, int32_t w_zp_scalar,
                                                             const ConvQuant q, void *y) {
  const int64_t t = (int64_t)blockIdx.x * kCBlock + threadIdx.x;
  const int64_t total = g.N * g.M * g.P;
  if (t >= total) return;
  const int64_t p = t % g.P, nm = t / g.P;
  const int64_t m = nm % g.M, n = nm / g.M;
  const int64_t grp = m / g.Mg;
  const int32_t xz = x_u8 ? (int32_t)x_zp : (int32_t)(int8_t)x_zp;
  const int32_t wz = w_zp ? ByteValue(w_zp, m, w_u8) : w_zp_scalar;  // per channel, or the scalar
  const int64_t ox = p % g.out[2], oy = (p / g.out[2]) % g.out[1], oz = p / (g.out[2] * g.out[1]);
  int64_t acc = 0;
  uint32_t acc32 = 0;
  for (int64_t c = 0; c < g.cpg; ++c) {
    const uint8_t *plane = x + (n * g.C + grp * g.cpg + c) * g.in_size;
    const uint8_t *wrow = w + (m * g.cpg + c) * g.ks;
    int64_t tap = 0;
    for (int kz = 0; kz < g.k[0]; ++kz)
      for (int ky = 0; ky < g.k[1]; ++ky)
        for (int kx = 0; kx < g.k[2]; ++kx, ++tap) {
          int64_t off;
          if (!TapOffset(g, oz, oy, ox, kz, ky, kx, off)) continue;
          const int32_t prod = (ByteValue(plane, off, x_u8) - xz) * (ByteValue(wrow, tap, w_u8) - wz);
          if constexpr (QUANT) acc += prod;
          else acc32 += (uint32_t)prod;
        }
  }
  if constexpr (QUANT) {
    if (q.bias) acc += q.bias[m];
    static_cast<uint8_t *>(y)[t] = Requant(acc, CombinedScale(q, m), q);
  } else {
    static_cast<int32_t *>(y)[t] = (int32_t)acc32;
  }
}

// QLinearConv's bias and requantization of the GEMM's int32 sums [N, M, P]:
// workgroup y = (n, m) plane, 4 positions per thread (16-byte loads when P %
// 4 == 0).
typedef int v4i_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kCBlock) void ConvRequantKernel(const ConvGeom g, const int32_t *acc, const ConvQuant q,
                                                             uint8_t *y) {
  const uint32_t P = (uint32_t)g.P;
  const int64_t nm = (int64_t)blockIdx.y + (int64_t)blockIdx.z * 65535;
  const uint32_t p0 = (blockIdx.x * kCBlock + threadIdx.x) * 4;
  if (nm >= g.N * g.M || p0 >= P) return;
  const int64_t m = nm % g.M;
  const float cs = CombinedScale(q, m);
  const int64_t bias = q.bias ? q.bias[m] : 0;
  const int32_t *a = acc + nm * g.P + p0;
  uint8_t *dst = y + nm * g.P + p0;
  if ((P & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {  // acc is 16-byte aligned scratch
    const v4i_t v = *reinterpret_cast<const v4i_t *>(a);
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) word |= (uint32_t)Requant((int64_t)v[e] + bias, cs, q) << (8 * e);
    *reinterpret_cast<uint32_t *>(dst) = word;
  } else {
    for (uint32_t e = 0; e < 4 && p0 + e < P; ++e) dst[e] = Requant((int64_t)a[e] + bias, cs, q);
  }
}

unsigned Blocks(int64_t threads) { return (unsigned)((threads + kCBlock - 1) / kCBlock); }

// ---- implicit GEMM operands ----
// The padded input rows and columns a convolution reads: Hp = (Ho - 1) sh +
// (kh - 1) dh + 1 rows from input row -pt on (likewise Wp), so every tap of
// every output position lands inside the padded image.
constexpr int kCvChannels = 128;  // channels per K step
constexpr int64_t kCvMaxLds = 65536;  // staged input row (C * W) or weight row (Kc) bytes

int64_t PaddedRows(const ConvGeom &g) { return (g.out[1] - 1) * g.s[1] + (g.k[1] - 1) * g.d[1] + 1; }
int64_t PaddedCols(const ConvGeom &g) { return (g.out[2] - 1) * g.s[2] + (g.k[2] - 1) * g.d[2] + 1; }

// LDS layout of one staged input row on the dword path: channel row c (W / 4
// dwords) at dword c * ts + ((c >> 6) & 3), with ts odd and at least
// W / 4 + 3, so that the 64 lanes of a wavefront reading channel rows
// 4 qd + i (qd = 0..63, i fixed) hit 64 distinct banks.
__host__ __device__ inline int64_t RowTileStride(int64_t W) { return (W / 4 + 3) | 1; }  // dwords
int64_t RowTileBytes(int64_t C, int64_t W) { return W % 4 == 0 ? (C * RowTileStride(W) + 4) * 4 : C * W; }

// Word stores of the operands through the XCD's L2 (the device-scope sc1
// policy of the GEMM epilogue's stores): the kernel then ends without a
// writeback of dirty lines, and the GEMM, whose tiles read them from other
// XCDs, finds them in memory.  `rs` covers the block's own output row.
__device__ __forceinline__ void PutThrough(__amdgpu_buffer_rsrc_t rs, uint32_t e, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, rs, 4 * e, 0, 16);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t RowRsrc(void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0, (int)bytes, 0x00020000);
}

// One launch builds both operands.  Blocks 0 .. N * Hp - 1 write padded row
// hp of image n: xh[n, hp, wp, c] = x[n, c, hp - pt, wp - pl], or x's zero
// point outside the input; the C input rows of W bytes are staged in LDS,
// then written as Wp pixels of C bytes.  Dword path (W % 4 == 0, x dword
// aligned): loads of eight dwords in flight per thread; then each thread
// reads the 4 x 4 byte block of channels 4 qd .. 4 qd + 3 and pixels
// 4 q .. 4 q + 3 (four dword reads), transposes it with byte permutes, and
// writes the four pixels' channel dwords, a wavefront's 64 lanes on 64
// consecutive channel quads (256 contiguous bytes per store).  Otherwise
// byte reads, one channel dword per thread.  The remaining M blocks write
// one row of the tap-major weight each, wr[m, tap, c] = w[m, c, tap], from
// the row staged in LDS.
__global__ __launch_bounds__(kCBlock) void ImplicitOperandsKernel(const ConvGeom g, int64_t Hp, int64_t Wp,
                                                                  int dwords, const uint8_t *x, uint8_t x_zp,
                                                                  const uint8_t *w, uint8_t *xh, uint8_t *wr) {
  extern __shared__ uint8_t tile[];  // one staged input row or one weight row (Kc bytes), below 2^16
  // 32-bit index arithmetic inside the loops (64-bit division is a long
  // software sequence): every per-block count is below 2^16
  const uint32_t H = (uint32_t)g.in[1], W = (uint32_t)g.in[2], C = (uint32_t)g.C;
  // Workgroup i runs on XCD i % 8; logical block b is dealt so that each XCD
  // owns a contiguous run of blocks.  Consecutive padded rows of an image read
  // the same input cache lines (one 128-byte line holds parts of several
  // rows), and then read them through one L2 instead of eight.
  const int64_t nb = (int64_t)gridDim.x, pid = blockIdx.x;
  const int64_t xcd = pid % 8, per = nb / 8, extra = nb % 8;
  const int64_t b = xcd * per + (xcd < extra ? xcd : extra) + pid / 8;
  const uint32_t cq = C / 4, pl = (uint32_t)g.pb[2];
  const uint32_t zp4 = x_zp * 0x01010101u;
  if (b < g.N * Hp && dwords) {
    const int64_t n = b / Hp, hp = b - n * Hp, h = hp - g.pb[1];
    uint32_t *dst = reinterpret_cast<uint32_t *>(xh + (n * Hp + hp) * Wp * C);
    const uint32_t wpad = (uint32_t)Wp;
    const __amdgpu_buffer_rsrc_t rsD = RowRsrc(dst, Wp * C);
    if (h < 0 || h >= (int64_t)H) {
      for (uint32_t e = threadIdx.x; e < wpad * cq; e += kCBlock) PutThrough(rsD, e, zp4);
      return;
    }
    const uint32_t wd = W / 4, ts = (uint32_t)RowTileStride(W);
    uint32_t *t32 = reinterpret_cast<uint32_t *>(tile);
    const uint32_t *src = reinterpret_cast<const uint32_t *>(x + (n * C * H + h) * W);
    const uint32_t plane = H * W / 4, total = C * wd;
    for (uint32_t e0 = threadIdx.x; e0 < total; e0 += 8 * kCBlock) {
      uint32_t v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t e = e0 + k * kCBlock;
        if (e < total) {
          const uint32_t c = e / wd;
          v[k] = src[c * plane + (e - c * wd)];
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t e = e0 + k * kCBlock;
        if (e < total) {
          const uint32_t c = e / wd;
          t32[c * ts + ((c >> 6) & 3) + (e - c * wd)] = v[k];
        }
      }
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < wd * cq; t += kCBlock) {
      const uint32_t q = t / cq, qd = t - q * cq;
      const uint32_t *r0 = t32 + (4 * qd) * ts + ((qd >> 4) & 3) + q;
      const uint32_t a0 = r0[0], a1 = r0[ts], a2 = r0[2 * ts], a3 = r0[3 * ts];  // channels 4qd + i
      const uint32_t lo01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u), hi01 = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u), hi23 = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
      const uint32_t px[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u), __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                              __builtin_amdgcn_perm(hi23, hi01, 0x05040100u), __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t wp = 4 * q + j + pl;  // input columns past Wp are never read
        if (wp < wpad) PutThrough(rsD, wp * cq + qd, px[j]);
      }
    }
    // the padding columns [0, pl) and [pl + W, Wp): x's zero point
    const uint32_t left = pl < wpad ? pl : wpad, right0 = pl + W;
    const uint32_t pads = left + (wpad > right0 ? wpad - right0 : 0u);
    for (uint32_t e = threadIdx.x; e < pads * cq; e += kCBlock) {
      const uint32_t k = e / cq, wp = k < left ? k : right0 + (k - left);
      PutThrough(rsD, wp * cq + (e - k * cq), zp4);
    }
  } else if (b < g.N * Hp) {
    // one padded row, byte loads: xh[n, hp, wp, c] from the staged C x W bytes
    const int64_t n = b / Hp, hp = b - n * Hp, h = hp - g.pb[1];
    const bool row_in = h >= 0 && h < (int64_t)H;
    if (row_in) {
      const uint8_t *src = x + (n * C * H + h) * W;  // channel c at + c * H * W
      for (uint32_t e = threadIdx.x; e < C * W; e += kCBlock) {
        const uint32_t c = e / W;
        tile[e] = src[(size_t)c * H * W + (e - c * W)];
      }
    }
    __syncthreads();
    uint32_t *dst = reinterpret_cast<uint32_t *>(xh + (n * Hp + hp) * Wp * C);
    auto quad = [&](uint32_t wp, uint32_t qd) __attribute__((always_inline)) {
      const uint32_t wi = wp - pl;  // wraps above W when wp < pl
      uint32_t v = zp4;
      if (row_in && wp >= pl && wi < W) {
        const uint8_t *t = tile + (4 * qd) * W + wi;
        v = (uint32_t)t[0] | (uint32_t)t[W] << 8 | (uint32_t)t[2 * W] << 16 | (uint32_t)t[3 * W] << 24;
      }
      return v;
    };
    if (kCBlock % cq == 0) {
      // fixed channel dword per thread, kCBlock / cq pixels per pass
      const uint32_t qd = threadIdx.x % cq, step = kCBlock / cq;
      for (uint32_t wp = threadIdx.x / cq; wp < (uint32_t)Wp; wp += step) dst[wp * cq + qd] = quad(wp, qd);
    } else {
      for (uint32_t e = threadIdx.x; e < (uint32_t)Wp * cq; e += kCBlock) {
        const uint32_t wp = e / cq;
        dst[e] = quad(wp, e - wp * cq);
      }
    }
  } else {
    const int64_t m = b - g.N * Hp;
    const uint32_t T = (uint32_t)g.ks, Kc = (uint32_t)g.Kc, kq = Kc / 4;
    if (reinterpret_cast<uintptr_t>(w) % 4 == 0) {
      const uint32_t *src = reinterpret_cast<const uint32_t *>(w + m * Kc);
      for (uint32_t e = threadIdx.x; e < kq; e += kCBlock) reinterpret_cast<uint32_t *>(tile)[e] = src[e];
    } else {
      for (uint32_t e = threadIdx.x; e < Kc; e += kCBlock) tile[e] = w[m * Kc + e];
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rsD = RowRsrc(wr + m * Kc, Kc);
    for (uint32_t e = threadIdx.x; e < kq; e += kCBlock) {
      const uint32_t tap = (4 * e) / C, c = 4 * e - tap * C;
      const uint8_t *t = tile + c * T + tap;
      PutThrough(rsD, e, (uint32_t)t[0] | (uint32_t)t[T] << 8 | (uint32_t)t[2 * T] << 16 | (uint32_t)t[3 * T] << 24);
    }
  }
}

uint32_t Magic(int64_t d) { return d == 1 ? 0u : (uint32_t)(((uint64_t(1) << 32) + (uint64_t)d - 1) / (uint64_t)d); }

}  // namespace

bool ConvImplicitEligible(const ConvGeom &g) {
  const int64_t lim = (int64_t(1) << 31) - (int64_t(1) << 24);
  if (g.G != 1 || g.in[0] != 1 || g.k[0] != 1 || g.C % kCvChannels != 0 || g.P % 16 != 0 || g.P == 0) return false;
  const int64_t Hp = PaddedRows(g), Wp = PaddedCols(g);
  return RowTileBytes(g.C, g.in[2]) <= kCvMaxLds && g.Kc <= kCvMaxLds && g.N * Hp + g.M < (int64_t(1) << 31) &&
         Hp * Wp * g.C < lim && g.M * g.Kc < lim && g.M * g.P * 4 < lim;
}

size_t ConvImplicitInputBytes(const ConvGeom &g) { return (size_t)(g.N * PaddedRows(g) * PaddedCols(g) * g.C); }

ImplicitConv ConvImplicitDesc(const ConvGeom &g) {
  const int64_t Wp = PaddedCols(g), C = g.C;
  ImplicitConv cv{};
  cv.pix_row = g.s[1] * Wp * C;
  cv.pix_col = g.s[2] * C;
  cv.tap_row = g.d[1] * Wp * C;
  cv.tap_col = g.d[2] * C;
  cv.image_bytes = PaddedRows(g) * Wp * C;
  cv.wo = (int)g.out[2];
  cv.spt = (int)(C / kCvChannels);
  cv.kw = g.k[2];
  cv.spt_magic = Magic(cv.spt);
  cv.kw_magic = Magic(cv.kw);
  return cv;
}

void LaunchConvImplicitOperands(const ConvGeom &g, const uint8_t *x, uint8_t x_zp, const uint8_t *w, uint8_t *xh,
                                uint8_t *wr, hipStream_t s) {
  const int64_t Hp = PaddedRows(g), Wp = PaddedCols(g);
  const bool dwords = g.in[2] % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 4 == 0;
  const int64_t blocks = g.N * Hp + g.M;
  const unsigned lds = (unsigned)std::max<int64_t>(dwords ? RowTileBytes(g.C, g.in[2]) : g.C * g.in[2], g.Kc);
  if (blocks > 0)
    hipLaunchKernelGGL(ImplicitOperandsKernel, dim3((unsigned)blocks), dim3(kCBlock), lds, s, g, Hp, Wp, (int)dwords,
                       x, x_zp, w, xh, wr);
}

bool ConvColIsInput(const ConvGeom &g) {
  for (int i = 0; i < 3; ++i)
    if (g.k[i] != 1 || g.s[i] != 1 || g.pb[i] != 0 || g.in[i] != g.out[i]) return false;
  return true;
}

size_t ConvColBytes(const ConvGeom &g) { return ConvColIsInput(g) ? 0 : (size_t)(g.N * g.G * g.Kc * g.P); }

void LaunchImToCol(const ConvGeom &g, const uint8_t *x, uint8_t x_zp, uint8_t *col, hipStream_t s) {
  const int64_t threads = g.N * g.G * g.Kc * ((g.P + 3) / 4);
  if (threads == 0) return;
  const bool plane = g.in[0] == 1 && g.k[0] == 1 && g.in_size <= kPlaneMax && g.P < (1ll << 31) &&
                     g.N * g.C < (1ll << 31) * kPlanesPerBlock;
  const dim3 grid((unsigned)((g.N * g.C + kPlanesPerBlock - 1) / kPlanesPerBlock));
  const unsigned lds = (unsigned)(kPlanesPerBlock * ((g.in_size + 15) & ~15ll));
  if (plane && g.k[1] == 3 && g.k[2] == 3)
    hipLaunchKernelGGL((ImToColPlaneKernel<3, 3>), grid, dim3(kCBlock), lds, s, g, x, x_zp, col);
  else if (plane)
    hipLaunchKernelGGL((ImToColPlaneKernel<0, 0>), grid, dim3(kCBlock), lds, s, g, x, x_zp, col);
  else
    hipLaunchKernelGGL(ImToColKernel, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_zp, col);
}

void LaunchDirectConv(const ConvGeom &g, const uint8_t *x, int x_u8, uint8_t x_zp, const uint8_t *w, int w_u8,
                      const uint8_t *w_zp_per_channel, int32_t w_zp_scalar, const ConvQuant *q, void *y,
                      hipStream_t s) {
  const int64_t threads = g.N * g.M * g.P;
  if (threads == 0) return;
  if (q)
    hipLaunchKernelGGL(DirectConvKernel<true>, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_u8, x_zp, w,
                       w_u8, w_zp_per_channel, w_zp_scalar, *q, y);
  else
    hipLaunchKernelGGL(DirectConvKernel<false>, dim3(Blocks(threads)), dim3(kCBlock), 0, s, g, x, x_u8, x_zp, w,
                       w_u8, w_zp_per_channel, w_zp_scalar, ConvQuant{}, y);
}

void LaunchConvRequant(const ConvGeom &g, const int32_t *acc, const ConvQuant &q, uint8_t *y, hipStream_t s) {
  const int64_t planes = g.N * g.M;
  if (planes == 0 || g.P == 0) return;
  if (g.P >= (1ll << 31) || planes > 65535ll * 65535ll)
    throw Unsupported("QLinearConv: output planes beyond the requantization grid");
  const unsigned gx = Blocks((g.P + 3) / 4);
  const unsigned gy = (unsigned)std::min<int64_t>(planes, 65535), gz = (unsigned)((planes + 65534) / 65535);
  hipLaunchKernelGGL(ConvRequantKernel, dim3(gx, gy, gz), dim3(kCBlock), 0, s, g, acc, q, y);
}

}  // namespace onnxl_amd
