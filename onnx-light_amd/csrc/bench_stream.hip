// Measurement helper for bench.py, built as its own library
// (libonnxl_amd_bench.so), not part of the C ABI: read-only streaming kernels
// that give the achievable HBM read rate for a given byte count, so that a
// bandwidth-bound kernel's time can be set beside the time a plain read of
// the same bytes takes.  Several read designs, the bench keeps the fastest:
//
//   variant 0: one pass, 4 16-byte loads in flight per lane, one workgroup per
//              16 KiB;
//   variant 1: one pass, 8 loads in flight per lane (32 KiB per workgroup);
//   variant 2: one pass, 16 loads in flight per lane (64 KiB per workgroup);
//   variant 3: persistent, 1024 workgroups (4 per CU) looping over the bytes
//              with 4 loads in flight per lane;
//   variant 4: variant 1 with non-temporal loads (streaming cache policy).
//
// Consecutive lanes read consecutive 16-byte pieces, so a wave instruction
// reads 1 KiB of contiguous bytes.  The XOR of everything read is kept, and
// written only if it equals a value passed in by the host that it never
// equals in practice, so the loads cannot be removed and the kernel writes
// nothing.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;
constexpr int kPersistentBlocks = 1024;
typedef unsigned v4u __attribute__((ext_vector_type(4)));

template <int IN_FLIGHT, bool NT>
__global__ __launch_bounds__(kThreads) void StreamReadKernel(const v4u *__restrict__ p, int64_t n16,
                                                             unsigned never, unsigned *sink) {
  const int64_t span = (int64_t)gridDim.x * kThreads * IN_FLIGHT;
  unsigned acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * kThreads * IN_FLIGHT + threadIdx.x; base < n16; base += span) {
    v4u v[IN_FLIGHT];
#pragma unroll
    for (int u = 0; u < IN_FLIGHT; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      if constexpr (NT) v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : v4u{0, 0, 0, 0};
      else v[u] = i < n16 ? p[i] : v4u{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < IN_FLIGHT; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == never) sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

int InFlight(int variant) { return variant == 0 || variant == 3 ? 4 : (variant == 2 ? 16 : 8); }

}  // namespace

extern "C" {

int onnxl_amd_bench_stream_variants(void) { return 5; }

// Workgroups variant `variant` launches for `bytes`; `sink` must hold one
// unsigned per launched thread: blocks * 256.
int onnxl_amd_bench_stream_blocks_v(int64_t bytes, int variant) {
  const int64_t n16 = bytes / 16;
  const int64_t per_block = (int64_t)kThreads * InFlight(variant);
  const int64_t one_pass = (n16 + per_block - 1) / per_block;
  return (int)(variant == 3 ? (one_pass < kPersistentBlocks ? one_pass : kPersistentBlocks) : one_pass);
}

int onnxl_amd_bench_stream_blocks(int64_t bytes) { return onnxl_amd_bench_stream_blocks_v(bytes, 0); }

// Reads `bytes` (a multiple of 16, 16-byte aligned) at `p` once.
int onnxl_amd_bench_stream_read_v(const void *p, int64_t bytes, unsigned *sink, void *stream, int variant) {
  if (bytes % 16 != 0 || reinterpret_cast<uintptr_t>(p) % 16 != 0 || variant < 0 || variant > 4) return 1;
  const int blocks = onnxl_amd_bench_stream_blocks_v(bytes, variant);
  if (blocks == 0) return 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const v4u *q = static_cast<const v4u *>(p);
  const int64_t n16 = bytes / 16;
  const unsigned never = 0x9e3779b9u;
  switch (variant) {
  case 0: hipLaunchKernelGGL((StreamReadKernel<4, false>), dim3(blocks), dim3(kThreads), 0, s, q, n16, never, sink); break;
  case 1: hipLaunchKernelGGL((StreamReadKernel<8, false>), dim3(blocks), dim3(kThreads), 0, s, q, n16, never, sink); break;
  case 2: hipLaunchKernelGGL((StreamReadKernel<16, false>), dim3(blocks), dim3(kThreads), 0, s, q, n16, never, sink); break;
  case 3: hipLaunchKernelGGL((StreamReadKernel<4, false>), dim3(blocks), dim3(kThreads), 0, s, q, n16, never, sink); break;
  default: hipLaunchKernelGGL((StreamReadKernel<8, true>), dim3(blocks), dim3(kThreads), 0, s, q, n16, never, sink); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

int onnxl_amd_bench_stream_read(const void *p, int64_t bytes, unsigned *sink, void *stream) {
  return onnxl_amd_bench_stream_read_v(p, bytes, sink, stream, 0);
}

}  // extern "C"
