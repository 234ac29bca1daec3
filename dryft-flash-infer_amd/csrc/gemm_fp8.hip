// FP8 e4m3 W8A8 linear: per-token activation quantization in the kernel, or done beforehand.
#include "gemm_launch.h"

extern "C" int qlx_linear_fp8_w8a8(const void* w, const void* w_scale, const void* x, void* y, int m,
                                   int n, int k, int tiled, const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = y;
  a.tiled = tiled;
  QLX_REQUIRE(k % 8 == 0, "K must be a multiple of 8");
  return qlx::launch_gemm<qlx::FmtFP8, true>("linear_fp8_w8a8", a, plan, m, n, k, stream);
}

// The same linear on an activation quantized beforehand by qlx_quantize_fp8_act (e4m3 codes
// [m][k], fp32 token scales [m]): batches of several tokens quantize once per projection
// instead of every workgroup reading every token's whole row for its maximum.
extern "C" int qlx_linear_fp8_w8a8_q(const void* w, const void* w_scale, const void* x_code, const float* x_scale,
                                     void* y, int m, int n, int k, int tiled, const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x_code;
  a.xs = x_scale;
  a.y = y;
  a.tiled = tiled;
  QLX_REQUIRE(k % 128 == 0, "K must be a multiple of 128");
  QLX_REQUIRE(x_scale != nullptr, "linear_fp8_w8a8_q: token scales are NULL");
  return qlx::launch_gemm<qlx::FmtFP8, true>("linear_fp8_w8a8_q", a, plan, m, n, k, stream);
}

// The fused residual add + RMSNorm form (qlx_linear_add_norm) of the same kernels.
int qlx::add_norm_fp8(const GemmArgs& a, const qlx_plan* plan, int m, int n, int k, void* stream) {
  return launch_gemm<FmtFP8, true>("linear_add_norm", a, plan, m, n, k, stream);
}
