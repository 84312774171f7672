// Pipelined int8 GEMM instantiations with requantised u8/s8 output (QLinearMatMul).
#include "igemm_fast.hpp"

namespace onnxl_amd {
void LaunchIGemmFastQ8(const IGemmParams &p, hipStream_t s) { LaunchIGemmFastOut<mg::kOutQ8>(p, s); }
}  // namespace onnxl_amd
