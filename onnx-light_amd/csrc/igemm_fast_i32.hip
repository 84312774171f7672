// Pipelined int8 GEMM instantiations with int32 output (MatMulInteger).
#include "igemm_fast.hpp"

namespace onnxl_amd {
void LaunchIGemmFastI32(const IGemmParams &p, hipStream_t s) { LaunchIGemmFastOut<mg::kOutI32>(p, s); }
}  // namespace onnxl_amd
