// Dequantize-fused MatMul (placeholder until the GEMV / GEMM kernels land).
#include "common.hpp"
#include "kernels.hpp"

namespace onnxl_amd {

size_t DqMatMulScratchBytes(const DqMatMulParams &) { return 0; }
size_t DqMatMulCounters(const DqMatMulParams &) { return 0; }
bool LaunchDqMatMul(const DqMatMulParams &, void *, size_t, unsigned *, size_t, hipStream_t) {
  return false;
}
void LaunchHMatMul(const HMatMulParams &, hipStream_t) {
  throw Unsupported("MatMul FLOAT16/BFLOAT16: kernel not built yet");
}

}  // namespace onnxl_amd
