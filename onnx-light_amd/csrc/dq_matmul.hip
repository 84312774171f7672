// Dequantize-fused MatMul dispatch and the FLOAT16 / BFLOAT16 MatMul.
//
//  - int4 / uint4 weights with FLOAT16 scales, M <= 16 (decode): the
//    bandwidth-bound GEMV, on the ONNX packing (gemv_q4.hip) or on the tiled
//    layout of a prepared weight (gemv_q4_tiled.hip).
//  - float8e4m3fn weights, FLOAT scales per column or per tensor, Cast to
//    BFLOAT16, bf16 activations (prefill): the pipelined MFMA core with the
//    weight decoded exactly to bf16 as it is read from LDS and the scale
//    applied to the fp32 sums (mfma_gemm.hpp, kBf16F8).
//  - anything else the C ABI accepts: the weight is dequantised into scratch
//    with the chain's exact rounding, then multiplied by the 16-bit MatMul.
#include <algorithm>

#include "common.hpp"
#include "device_codecs.hpp"
#include "kernels.hpp"
#include "mfma_gemm.hpp"

namespace onnxl_amd {

bool GemvQ4Eligible(const DqMatMulParams &p);
bool GemvQ4TiledEligible(const DqMatMulParams &p);
void LaunchGemvQ4Tiled(const DqMatMulParams &p, hipStream_t stream);
size_t GemvQ4ScratchBytes(const DqMatMulParams &p);
size_t GemvQ4Counters(const DqMatMulParams &p);
void LaunchGemvQ4(const DqMatMulParams &p, void *scratch, unsigned *counters, hipStream_t stream);

namespace {

// ---------------------------------------------------------------------------
// Generic 16-bit MatMul for shapes the MFMA core does not take: one thread per
// output, fp32 accumulation in k order.  TB: B given transposed, [N, K].
template <bool BF16, bool TB = false>
__global__ __launch_bounds__(256) void HMatMulSimpleKernel(const HMatMulParams p) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t m = blockIdx.y;
  const int64_t b = blockIdx.z;
  if (n >= p.N) return;
  int64_t ao, bo;
  BatchOffsets(p.bm, b, ao, bo);
  const uint16_t *a = p.A + ao + m * p.K;
  const uint16_t *w = p.B + bo + (TB ? n * p.K : n);
  const int64_t wstep = TB ? 1 : p.N;
  float acc = 0.f;
  for (int64_t k = 0; k < p.K; ++k) {
    const float x = BF16 ? Bf16ToF32(a[k]) : F16ToF32(a[k]);
    const float y = BF16 ? Bf16ToF32(w[k * wstep]) : F16ToF32(w[k * wstep]);
    acc += x * y;
  }
  p.Y[(b * p.M + m) * p.N + n] = BF16 ? F32ToBf16(acc) : F32ToF16(acc);
}

mg::GemmArgs HArgs(const HMatMulParams &p) {
  mg::GemmArgs g{};
  g.A = p.A;
  g.B = p.B;
  g.Y = p.Y;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  g.batch = p.batch;
  g.bm = p.bm;
  return g;
}

// ---------------------------------------------------------------------------
// Weight dequantisation into a 16-bit [K, N] scratch matrix with the unfused
// chain's rounding: DequantizeLinear computes (x - zp) * scale in fp32 and
// stores the scale's dtype (FLOAT16: round to nearest even); an optional Cast
// rounds FLOAT to BFLOAT16 / FLOAT16
// (kq/kernel_dequantizelinear.cc:57-63,259-285; kernel_cast.cc:360-370).
__device__ __forceinline__ float DecodeWeight(const uint8_t *w, int dt, int64_t i) {
  switch (dt) {
  case kInt4: return (float)Int4ToInt((w[i >> 1] >> (4 * (i & 1))) & 0xfu);
  case kUint4: return (float)((w[i >> 1] >> (4 * (i & 1))) & 0xfu);
  case kInt8: return (float)(int8_t)w[i];
  case kUint8: return (float)w[i];
  default: return Fp8E4M3ToF32(w[i]);
  }
}

// Element (k, n) of a 4-bit weight in the tiled layout (kernels.hpp).
__device__ __forceinline__ float DecodeTiled(const uint8_t *w, int dt, int64_t ngroups, int64_t k, int64_t n) {
  const int64_t t = n >> 4, i = n & 15, q = k >> 7, c = (k >> 5) & 3, g = (k >> 3) & 3, j = k & 7;
  const uint32_t word = reinterpret_cast<const uint32_t *>(w)[((t * ngroups + q) * 64 + g * 16 + i) * 4 + c];
  const uint32_t u = (word >> ((j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1))) & 15u;
  return dt == kInt4 ? (float)((int)u - 8) : (float)u;
}

__global__ __launch_bounds__(256) void DequantWeightKernel(const DqMatMulParams p, uint16_t *out) {
  const int64_t total = p.K * p.N;
  const int64_t ngroups = (p.K + 127) / 128;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t k = i / p.N, n = i % p.N;
    int64_t si = 0;
    if (p.mode == 1) si = n;
    else if (p.mode == 2) si = (k / p.block) * p.N + n;
    const float s = p.scale_f16 ? F16ToF32(static_cast<const uint16_t *>(p.scale)[si])
                                : static_cast<const float *>(p.scale)[si];
    const float z = p.zp ? DecodeWeight(p.zp, p.w_dtype, si) : 0.f;
    const float x = p.w_tiled ? DecodeTiled(p.W, p.w_dtype, ngroups, k, n) : DecodeWeight(p.W, p.w_dtype, i);
    const float v = (x - z) * s;
    uint16_t bits;
    if (p.deq_round_f16) {
      bits = F32ToF16(v);  // DequantizeLinear output FLOAT16 (no Cast follows)
    } else if (p.cast_round == 16) {
      bits = F32ToBf16(v);
    } else {
      bits = F32ToF16(v);
    }
    out[i] = bits;
  }
}

bool Fp8Eligible(const DqMatMulParams &p) {
  return p.w_dtype == kFloat8E4M3FN && p.a_bf16 && p.cast_round == 16 && !p.scale_f16 &&
         (p.mode == 0 || p.mode == 1) && p.zp == nullptr;
}

// Compute units of the current device, queried once per device.
int64_t DeviceCUs() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// The fp8 GEMM in 256 x 256 tiles, except that when those tiles leave a last,
// partly filled round of workgroups, the trailing columns go to a second
// launch in 256 x 128 tiles.  C4 (4096 x 14336): 896 tiles are 3.5 rounds on
// 256 CUs; 768 tiles (12288 columns) make 3 whole rounds and the last 2048
// columns are 256 half-size tiles, one round of half the time.
void LaunchFp8Gemm(const mg::GemmArgs &g, hipStream_t stream) {
  const int64_t cus = DeviceCUs();
  const int64_t nbm = (g.M + 255) / 256, nbn = (g.N + 255) / 256;
  if (nbm * nbn < 512 || g.K % 64 != 0) {  // 256 x 256 tiles take whole K steps only
    mg::Launch<mg::kBf16F8, mg::kOutBf16, false, false, false, 2>(g, stream);
    return;
  }
  int64_t nb = nbn;  // tile-columns in 256 x 256 tiles
  if ((nbm * nbn) % cus != 0 && g.N % 256 == 0) {
    int64_t c = nbn - 1;
    while (c > 0 && (nbm * c) % cus != 0) --c;
    if (c > 0 && nbm * (nbn - c) * 2 <= cus) nb = c;
  }
  if (nb == nbn) {
    mg::Launch<mg::kBf16F8, mg::kOutBf16, false, false, false, 4>(g, stream);
    return;
  }
  const int64_t n0 = nb * 256;
  mg::GemmArgs g1 = g, g2 = g;
  g1.N = n0;
  g1.ldb = g.N;
  g1.ldy = g.N;
  g2.N = g.N - n0;
  g2.ldb = g.N;
  g2.ldy = g.N;
  g2.B = static_cast<const uint8_t *>(g.B) + n0;
  g2.Y = static_cast<uint16_t *>(g.Y) + n0;
  if (g.scale_per_col) g2.scale = static_cast<const float *>(g.scale) + n0;
  mg::Launch<mg::kBf16F8, mg::kOutBf16, false, false, false, 4>(g1, stream);
  mg::Launch<mg::kBf16F8, mg::kOutBf16, false, false, false, 2>(g2, stream);
}

mg::GemmArgs Fp8Args(const DqMatMulParams &p) {
  mg::GemmArgs g{};
  g.A = p.A;
  g.B = p.W;
  g.Y = p.Y;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  g.batch = 1;
  g.scale = p.scale;
  g.scale_f16 = 0;
  g.scale_per_col = p.mode == 1;
  return g;
}

}  // namespace

void LaunchHMatMul(const HMatMulParams &p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return;
  const mg::GemmArgs g = HArgs(p);
  if (mg::Eligible<mg::kH16>(g)) {
    if (p.bf16) mg::Launch<mg::kH16, mg::kOutBf16, false, false, false>(g, stream);
    else mg::Launch<mg::kH16, mg::kOutF16, false, false, false>(g, stream);
    return;
  }
  const dim3 grid((unsigned)((p.N + 255) / 256), (unsigned)p.M, (unsigned)p.batch);
  if (p.bf16) hipLaunchKernelGGL(HMatMulSimpleKernel<true>, grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(HMatMulSimpleKernel<false>, grid, dim3(256), 0, stream, p);
}

// Y = A @ B^T for B given as [N, K] (batch 1): the MFMA core reading B's rows
// like A's, else the simple kernel.
void LaunchHMatMulBT(const HMatMulParams &p, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return;
  const mg::GemmArgs g = HArgs(p);
  if (p.batch == 1 && mg::EligibleBT(g)) {
    if (p.bf16) mg::LaunchBT<mg::kOutBf16>(g, stream);
    else mg::LaunchBT<mg::kOutF16>(g, stream);
    return;
  }
  if (p.M > 65535 || p.batch > 65535) throw Unsupported("MatMul with B given as [N, K]: the one-thread-per-output "
                                                       "kernel for N % 16 != 0 takes at most 65535 rows");
  const dim3 grid((unsigned)((p.N + 255) / 256), (unsigned)p.M, (unsigned)p.batch);
  if (p.bf16) hipLaunchKernelGGL((HMatMulSimpleKernel<true, true>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((HMatMulSimpleKernel<false, true>), grid, dim3(256), 0, stream, p);
}

size_t DqMatMulScratchBytes(const DqMatMulParams &p) {
  if (GemvQ4TiledEligible(p)) return 0;
  if (GemvQ4Eligible(p)) return GemvQ4ScratchBytes(p);
  if (Fp8Eligible(p) && mg::Eligible<mg::kBf16F8>(Fp8Args(p))) return 0;
  return (size_t)(p.K * p.N) * sizeof(uint16_t);
}

size_t DqMatMulCounters(const DqMatMulParams &p) {
  return GemvQ4Eligible(p) ? GemvQ4Counters(p) : 0;
}

bool LaunchDqMatMul(const DqMatMulParams &p, void *scratch, size_t scratch_bytes, unsigned *counters,
                    size_t n_counters, hipStream_t stream) {
  if (p.M == 0 || p.N == 0) return true;
  if (GemvQ4TiledEligible(p)) {
    LaunchGemvQ4Tiled(p, stream);
    return true;
  }
  if (GemvQ4Eligible(p)) {
    if (scratch_bytes < GemvQ4ScratchBytes(p) || n_counters < GemvQ4Counters(p)) return false;
    LaunchGemvQ4(p, scratch, counters, stream);
    return true;
  }
  if (Fp8Eligible(p)) {
    const mg::GemmArgs g = Fp8Args(p);
    if (mg::Eligible<mg::kBf16F8>(g)) {
      LaunchFp8Gemm(g, stream);
      return true;
    }
  }
  // general path: dequantise into scratch, then the 16-bit MatMul (K == 0
  // leaves nothing to dequantise and the MatMul writes zeros)
  if (scratch_bytes < (size_t)(p.K * p.N) * sizeof(uint16_t)) return false;
  uint16_t *w16 = static_cast<uint16_t *>(scratch);
  const int64_t total = p.K * p.N;
  if (total > 0) {
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(DequantWeightKernel, dim3(blocks), dim3(256), 0, stream, p, w16);
  }
  HMatMulParams h{};
  h.A = static_cast<const uint16_t *>(p.A);
  h.B = w16;
  h.Y = static_cast<uint16_t *>(p.Y);
  h.M = p.M;
  h.N = p.N;
  h.K = p.K;
  h.batch = 1;
  h.bf16 = p.a_bf16;
  LaunchHMatMul(h, stream);
  return true;
}

}  // namespace onnxl_amd
