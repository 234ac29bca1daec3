// FP8 e4m3 W8A8 linear with in-kernel per-token activation quantization.
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
  return qlx::launch_gemm<qlx::FmtFP8>("linear_fp8_w8a8", a, plan, m, n, k, stream);
}
