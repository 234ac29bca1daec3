// W8A16 per-output-channel linear (signed int8, bf16 scales): instantiations and C entry point.
#include "gemm_launch.h"

extern "C" int qlx_linear_w8a16(const void* w, const void* w_scale, const void* x, void* y, int m,
                                int n, int k, int tiled, const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = y;
  a.tiled = tiled;
  return qlx::launch_gemm<qlx::FmtW8, true>("linear_w8a16", a, plan, m, n, k, stream);
}

// The fused residual add + RMSNorm form (qlx_linear_add_norm) of the same kernels.
int qlx::add_norm_w8a16(const GemmArgs& a, const qlx_plan* plan, int m, int n, int k, void* stream) {
  return launch_gemm<FmtW8, true>("linear_add_norm", a, plan, m, n, k, stream);
}
