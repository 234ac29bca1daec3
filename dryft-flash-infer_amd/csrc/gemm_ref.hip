// cuda_fp8 reference formats (offset codes, fp16 per-64 scales, permuted/tiled layouts).
#include "gemm_launch.h"

extern "C" int qlx_linear_ref(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                              int k, int bits, int tiled, const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = y;
  a.tiled = tiled;
  QLX_REQUIRE(bits == 8 || bits == 4, "weights are 8 or 4 bits");
  QLX_REQUIRE(bits == 8 || tiled, "4-bit weights are stored tiled");
  if (bits == 8) return qlx::launch_gemm<qlx::FmtRef<8>, true>("linear_ref8", a, plan, m, n, k, stream);
  return qlx::launch_gemm<qlx::FmtRef<4>, true>("linear_ref4", a, plan, m, n, k, stream);
}

// The fused residual add + RMSNorm form (qlx_linear_add_norm) of the same kernels.
int qlx::add_norm_ref(const GemmArgs& a, int bits, const qlx_plan* plan, int m, int n, int k, void* stream) {
  if (bits == 8) return launch_gemm<FmtRef<8>, true>("linear_add_norm", a, plan, m, n, k, stream);
  return launch_gemm<FmtRef<4>, true>("linear_add_norm", a, plan, m, n, k, stream);
}
