// GEMM + residual add + RMSNorm in one launch (cuda_fp8.matmul_add_norm).
#include "gemm_launch.h"

extern "C" int qlx_linear_add_norm(int fmt, const void* w, const void* w_scale, const void* x, int m, int n, int k,
                                   int tiled, const void* residual, const void* norm_w, float eps, void* delta,
                                   int* counter, void* res_out, void* normed, const qlx_plan* plan, void* stream) {
  QLX_REQUIRE(counter != nullptr && delta != nullptr, "linear_add_norm: delta and counter are required");
  QLX_REQUIRE(n <= 65536, "linear_add_norm: n=%d rows exceed 65536", n);
  qlx::GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = delta;
  a.tiled = tiled;
  a.resid = residual;
  a.norm_w = norm_w;
  a.res_out = res_out;
  a.normed = normed;
  a.an_counter = counter;
  a.eps = eps;
  switch (fmt) {
    case QLX_FMT_W8A16: return qlx::add_norm_w8a16(a, plan, m, n, k, stream);
    case QLX_FMT_W4A16: return qlx::add_norm_w4a16(a, plan, m, n, k, stream);
    case QLX_FMT_FP8:
      QLX_REQUIRE(k % 8 == 0, "K must be a multiple of 8");
      return qlx::add_norm_fp8(a, plan, m, n, k, stream);
    case QLX_FMT_REF8:
    case QLX_FMT_REF4:
      QLX_REQUIRE(fmt == QLX_FMT_REF8 || tiled, "4-bit weights are stored tiled");
      return qlx::add_norm_ref(a, fmt == QLX_FMT_REF8 ? 8 : 4, plan, m, n, k, stream);
    default:
      QLX_REQUIRE(false, "linear_add_norm serves W8A16, W4A16, FP8 W8A8 and the cuda_fp8 formats (format %d)", fmt);
  }
}
