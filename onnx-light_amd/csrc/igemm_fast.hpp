// Launch glue of the pipelined int8 GEMM (mfma_gemm.hpp) for one output
// kind; included by igemm_fast_i32.hip and igemm_fast_q8.hip so the two
// instantiation sets compile in parallel.
#pragma once

#include "kernels.hpp"
#include "mfma_gemm.hpp"

namespace onnxl_amd {

inline mg::GemmArgs ToGemmArgs(const IGemmParams &p) {
  mg::GemmArgs g{};
  g.A = p.A;
  g.B = p.B;
  g.Y = p.Y;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  g.batch = p.batch;
  g.bm = p.bm;
  g.a_u8 = p.a_u8;
  g.b_u8 = p.b_u8;
  g.a_zp = p.a_zp;
  g.b_zp = p.b_zp;
  g.alpha_scalar = p.alpha_scalar;
  g.beta_scalar = p.beta_scalar;
  g.cs = p.cs;
  g.zy = p.zy;
  g.dev = p.dev;
  g.qmin = p.qmin;
  g.qmax = p.qmax;
  g.y_signed = p.y_signed;
  g.row_wscale = p.row_wscale;
  g.row_wscale_per = p.row_wscale_per;
  g.row_xs = p.row_xs;
  g.row_ys = p.row_ys;
  g.row_bias = p.row_bias;
  g.cv = p.cv;
  return g;
}

// Row / column sums are accumulated only when a zero point makes them count.
// CV: B is an implicit convolution operand (p.implicit_conv).
template <int OUT, bool CV = false> void LaunchIGemmFastOut(const IGemmParams &p, hipStream_t s) {
  const mg::GemmArgs g = ToGemmArgs(p);
  const bool zp = p.need_ra || p.need_cb;
  const int sel = (zp ? 4 : 0) | (p.a_u8 ? 2 : 0) | (p.b_u8 ? 1 : 0);
  switch (sel) {
  case 0: mg::Launch<mg::kI8, OUT, false, false, false, 2, CV>(g, s); break;
  case 1: mg::Launch<mg::kI8, OUT, false, false, true, 2, CV>(g, s); break;
  case 2: mg::Launch<mg::kI8, OUT, false, true, false, 2, CV>(g, s); break;
  case 3: mg::Launch<mg::kI8, OUT, false, true, true, 2, CV>(g, s); break;
  case 4: mg::Launch<mg::kI8, OUT, true, false, false, 2, CV>(g, s); break;
  case 5: mg::Launch<mg::kI8, OUT, true, false, true, 2, CV>(g, s); break;
  case 6: mg::Launch<mg::kI8, OUT, true, true, false, 2, CV>(g, s); break;
  default: mg::Launch<mg::kI8, OUT, true, true, true, 2, CV>(g, s); break;
  }
}

void LaunchIGemmFastI32(const IGemmParams &p, hipStream_t s);
void LaunchIGemmFastQ8(const IGemmParams &p, hipStream_t s);
void LaunchIGemmFastQ8Row(const IGemmParams &p, hipStream_t s);
void LaunchIGemmConvI32(const IGemmParams &p, hipStream_t s);
void LaunchIGemmConvQ8Row(const IGemmParams &p, hipStream_t s);

}  // namespace onnxl_amd
