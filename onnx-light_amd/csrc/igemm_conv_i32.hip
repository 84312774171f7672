// Implicit-convolution int8 GEMM instantiations with int32 output
// (ConvInteger).
#include "igemm_fast.hpp"

namespace onnxl_amd {
void LaunchIGemmConvI32(const IGemmParams &p, hipStream_t s) { LaunchIGemmFastOut<mg::kOutI32, true>(p, s); }
}  // namespace onnxl_amd
