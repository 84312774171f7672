// Pipelined int8 GEMM instantiations with per-row requantised u8/s8 output
// (QLinearConv's per-output-channel scale and bias).
#include "igemm_fast.hpp"

namespace onnxl_amd {
void LaunchIGemmFastQ8Row(const IGemmParams &p, hipStream_t s) { LaunchIGemmFastOut<mg::kOutQ8Row>(p, s); }
}  // namespace onnxl_amd
