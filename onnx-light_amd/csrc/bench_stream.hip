// Measurement helper for bench.py, built as its own library
// (libonnxl_amd_bench.so), not part of the C ABI: a read-only streaming
// kernel that gives the achievable HBM read rate for a given byte count, so
// that a bandwidth-bound kernel's time can be set beside the time a plain read
// of the same bytes takes.
//
// Each thread keeps four 16-byte loads in flight; consecutive lanes read
// consecutive 16-byte pieces, so a wave instruction reads 1 KiB of contiguous
// bytes.  The XOR of everything read is kept, and written only if it equals a
// value passed in by the host that it never equals in practice, so the loads
// cannot be removed and the kernel writes nothing.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;
constexpr int kInFlight = 4;

__global__ __launch_bounds__(kThreads) void StreamReadKernel(const uint4 *__restrict__ p, int64_t n16,
                                                             unsigned never, unsigned *sink) {
  const int64_t span = (int64_t)gridDim.x * kThreads * kInFlight;
  unsigned acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * kThreads * kInFlight + threadIdx.x; base < n16; base += span) {
    uint4 v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      v[u] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == never) sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned) at `p` once.  `sink` must
// hold one unsigned per launched thread: blocks() * 256.
int onnxl_amd_bench_stream_blocks(int64_t bytes) {
  const int64_t n16 = bytes / 16;
  const int64_t per_block = (int64_t)kThreads * kInFlight;
  return (int)((n16 + per_block - 1) / per_block);
}

int onnxl_amd_bench_stream_read(const void *p, int64_t bytes, unsigned *sink, void *stream) {
  if (bytes % 16 != 0 || reinterpret_cast<uintptr_t>(p) % 16 != 0) return 1;
  const int blocks = onnxl_amd_bench_stream_blocks(bytes);
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(StreamReadKernel, dim3(blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4 *>(p), bytes / 16, 0x9e3779b9u, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
