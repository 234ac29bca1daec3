// fp8.fp8_matmul (E4M3 weight-only, group scales) and cuda_int8 W8A8 linears.
#include "gemm_launch.h"

extern "C" int qlx_linear_fp8wo(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                                int k, int group, const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = y;
  a.group = group;
  QLX_REQUIRE(group >= 64 && group % 64 == 0 && k % group == 0,
              "fp8 group %d must be a multiple of 64 dividing K=%d", group, k);
  return qlx::launch_gemm<qlx::FmtFP8WO>("linear_fp8wo", a, plan, m, n, k, stream);
}

extern "C" int qlx_linear_int8(const void* w, const void* w_scale, const void* xq, const float* x_scale,
                               const void* xq2, const float* x_scale2, void* y, int m, int n, int k,
                               const qlx_plan* plan, void* stream) {
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = xq;
  a.xs = x_scale;
  a.x2 = xq2;
  a.xs2 = x_scale2;
  a.comp = xq2 ? 2 : 1;
  a.y = y;
  QLX_REQUIRE(!xq2 || x_scale2, "a second activation component needs its scales");
  return qlx::launch_gemm<qlx::FmtInt8>("linear_int8", a, plan, m, n, k, stream);
}
