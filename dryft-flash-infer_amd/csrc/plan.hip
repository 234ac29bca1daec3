// Default launch plans for the quantized linears.
//
// The reference races a fixed list of (warps, split-K) configurations per projection at
// warmup (engine/kernels/gemm.py:134-261, engine/kernels/cuda_fp8.py:1404-1423). Here the
// default comes from the shape: enough waves in flight to cover HBM latency on 256 CUs,
// K split inside a workgroup first (kw waves per tile, reduced in LDS) and across
// workgroups only when a projection has too few 16-row tiles, and enough steps per wave
// to keep its loads pipelined. Callers may pass any other valid plan.
#include "gemm_launch.h"

namespace {

qlx::FmtInfo fmt_info(int fmt) {
  switch (fmt) {
    case QLX_FMT_W8A16: return qlx::info<qlx::FmtW8>();
    case QLX_FMT_W4A16: return qlx::info<qlx::FmtW4>();
    case QLX_FMT_FP8: return qlx::info<qlx::FmtFP8>();
    case QLX_FMT_REF8: return qlx::info<qlx::FmtRef<8>>();
    case QLX_FMT_REF4: return qlx::info<qlx::FmtRef<4>>();
    case QLX_FMT_FP8WO: return qlx::info<qlx::FmtFP8WO>();
    case QLX_FMT_INT8: return qlx::info<qlx::FmtInt8>();
    default: return qlx::FmtInfo{0, 0, 0, 0};
  }
}

// Waves the chip should have in flight for a streaming GEMV: 256 CUs x 8.
constexpr int kTargetWaves = 2048;

}  // namespace

extern "C" int qlx_plan_linear(int fmt, int mode, int m, int n, int k, qlx_plan* plan) {
  QLX_REQUIRE(plan != nullptr, "plan is NULL");
  const qlx::FmtInfo fi = fmt_info(fmt);
  QLX_REQUIRE(fi.kstep > 0, "unknown format %d", fmt);
  QLX_REQUIRE(m >= 1 && m <= 64 && n >= 16 && n % 16 == 0 && k >= fi.kstep && k % fi.kstep == 0,
              "shape m=%d n=%d k=%d does not fit format %d", m, n, k, fmt);
  qlx_plan p = {};
  p.mode = mode;
  p.waves = 4;
  p.rw = m > 16 ? 2 : 1;
  const int nsteps = k / fi.kstep;
  const int ntiles = n / 16;
  const int slots = (ntiles + p.rw - 1) / p.rw;  // waves if every wave took whole tiles
  int need = slots >= kTargetWaves ? 1 : (kTargetWaves + slots - 1) / slots;
  int max_par = nsteps / 2 > 1 ? nsteps / 2 : 1;  // keep >= 2 steps per wave
  if (need > max_par) need = max_par;
  p.kw = need >= 4 ? 4 : (need >= 2 ? 2 : 1);
  p.splits = (need + p.kw - 1) / p.kw;
  // Large m stages a wide activation slice: split K further until LDS fits.
  qlx::GemmArgs a = {};
  for (;;) {
    const int lds = qlx::layout(fi, p, m, n, k, a);
    if (lds <= qlx::kLdsLimit || p.splits >= nsteps) break;
    ++p.splits;
  }
  qlx::layout(fi, p, m, n, k, a);
  p.splits = a.splits;  // normalised: every slice non-empty
  if (mode == QLX_MODE_PLANES && p.splits < 1) p.splits = 1;
  *plan = p;
  return QLX_OK;
}

extern "C" int qlx_plan_tickets(const qlx_plan* plan, int fmt, int m, int n, int k) {
  QLX_REQUIRE(plan != nullptr, "plan is NULL");
  const qlx::FmtInfo fi = fmt_info(fmt);
  QLX_REQUIRE(fi.kstep > 0, "unknown format %d", fmt);
  qlx::GemmArgs a = {};
  qlx::layout(fi, *plan, m, n, k, a);
  return a.tile_groups;
}
