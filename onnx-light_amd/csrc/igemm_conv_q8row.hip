// Implicit-convolution int8 GEMM instantiations with per-row requantised
// u8/s8 output (QLinearConv).
#include "igemm_fast.hpp"

namespace onnxl_amd {
void LaunchIGemmConvQ8Row(const IGemmParams &p, hipStream_t s) { LaunchIGemmFastOut<mg::kOutQ8Row, true>(p, s); }
}  // namespace onnxl_amd
