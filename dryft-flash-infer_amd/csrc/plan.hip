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
    default: return qlx::FmtInfo{0, 0, 0, 0, 0};
  }
}

// Workgroups a streaming GEMV should at least have. Measured on MI355X at M = 1..8 over the
// Qwen3-4B shapes: fewer, larger workgroups win (each pays the activation staging and a
// reduction once) as long as there are about 150 or more of them (gate_up's 152 whole tiles
// per 8 waves: 13.4 us against 16.9 with 304 half tiles, W4A16).
constexpr int kMinGroups = 150;
// Workgroups of 8 waves that run in one round (one per CU).
constexpr int kOneRound = 256;

}  // namespace

extern "C" int qlx_plan_linear(int fmt, int mode, int m, int n, int k, qlx_plan* plan) {
  QLX_REQUIRE(plan != nullptr, "plan is NULL");
  const qlx::FmtInfo fi = fmt_info(fmt);
  QLX_REQUIRE(fi.kstep > 0, "unknown format %d", fmt);
  QLX_REQUIRE(m >= 1 && m <= 64 && n >= 1 && k >= fi.kstep && k % fi.kstep == 0,
              "shape m=%d n=%d k=%d does not fit format %d", m, n, k, fmt);
  qlx_plan p = {};
  p.mode = mode;
  p.waves = 8;
  p.rw = m > 16 ? 2 : 1;
  p.splits = 1;
  const int nsteps = k / fi.kstep;
  const int ntiles = (n + 15) / 16;
  // kw: waves sharing one tile's K range, the smallest that still gives kMinGroups groups
  // (and at least one step per wave).
  p.kw = 8;
  for (int kw = 1; kw <= 8; kw *= 2) {
    const int groups = (ntiles + (p.waves / kw) * p.rw - 1) / ((p.waves / kw) * p.rw);
    if (groups >= kMinGroups || kw >= nsteps) {
      p.kw = kw;
      break;
    }
  }
  qlx::GemmArgs a = {};
  if (m <= 16) {
    // Up to 16 tokens the staged activation slice may use the whole LDS while the workgroups
    // fit one round (one per CU): o at 8 tokens whole-K 8.5 us against 13.0 with two K slices
    // (W4A16). Where K must be sliced to fit, take fewer waves per tile and as many slices as
    // still fit one round: down at 4-8 tokens (W4A16) 4 waves per tile x 3 slices (240
    // workgroups) 12.0-12.7 us against 16.8-17.5 with 8 x 2-3 (320-480 workgroups).
    const int kw0 = p.kw;
    for (int kw = kw0; kw >= 1; kw /= 2) {
      qlx_plan q = p;
      q.kw = kw;
      const int groups = (ntiles + (q.waves / kw) * q.rw - 1) / ((q.waves / kw) * q.rw);
      if (kw < kw0 && groups * 2 > kOneRound) break;  // fewer waves per tile would not help
      int smin = 1;  // the fewest K slices whose staged slice fits
      for (; smin <= nsteps; ++smin) {
        q.splits = smin;
        if (qlx::layout(fi, q, m, n, k, a) <= qlx::kLdsLimit) break;
      }
      if (smin > nsteps) continue;
      const int s = std::max(smin, smin > 1 ? kOneRound / groups : 1);
      if (groups * s > kOneRound && !(s == 1 && kw == kw0)) continue;
      q.splits = std::min(s, nsteps);
      qlx::layout(fi, q, m, n, k, a);
      q.splits = a.splits;
      // 8-bit weights have twice W4A16's K steps per byte of row, and there more, smaller
      // workgroups win on the whole-K shapes the rule above gives 8 tiles or 2 tile slots per
      // workgroup. Measured on MI355X, us per call over 24 distinct Qwen3-4B weights (this rule's
      // plan / the one above): SwiGLU gate_up at 4 waves, 2 per tile -- FP8 13.02 / 13.80,
      // 15.09 / 15.49, 15.05 / 15.83, 15.72 / 16.13 at M = 1 / 2 / 4 / 8; W8A16 13.29 / 15.68,
      // 14.33 / 14.63, 14.65 / 14.89 at M = 1 / 2 / 4 (15.42 / 15.28 at 8); FP8 qkv with a whole
      // workgroup per tile -- 7.03 / 7.42, 9.15 / 9.30, 9.29 / 9.52, 9.57 / 9.89 (W8A16 qkv and
      // every W4A16 shape are faster as above).
      const bool bits8 = fmt == QLX_FMT_FP8 || fmt == QLX_FMT_W8A16;
      if (bits8 && mode == QLX_MODE_SWIGLU && q.splits == 1 && q.waves == 8 && q.kw == 1 && q.rw == 1 &&
          m <= (fmt == QLX_FMT_FP8 ? 8 : 4)) {
        q.waves = 4;
        q.kw = 2;
        qlx::layout(fi, q, m, n, k, a);
        q.splits = a.splits;
      } else if (fmt == QLX_FMT_FP8 && mode == QLX_MODE_BF16 && q.splits == 1 && q.waves == 8 && q.kw == 4 &&
                 q.rw == 1 && m <= 8) {
        q.kw = 8;
        qlx::layout(fi, q, m, n, k, a);
        q.splits = a.splits;
      }
      *plan = q;
      return QLX_OK;
    }
  }
  // Large m stages a wide activation slice: split K until the workgroup's LDS fits the
  // 64 KB target; a plan whose reduction buffer alone is larger drops to 4 waves.
  for (;;) {
    const int lds = qlx::layout(fi, p, m, n, k, a);
    if (lds <= qlx::kLdsTarget) break;
    if (p.splits >= nsteps) {
      if (p.waves == 8) {
        p.waves = 4;
        if (p.kw > 4) p.kw = 4;
        p.splits = 1;
        continue;
      }
      break;  // <= 160 KB is still launchable
    }
    ++p.splits;
  }
  qlx::layout(fi, p, m, n, k, a);
  p.splits = a.splits;  // normalised: every slice non-empty
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

// Normalise a plan's K splits (every slice non-empty); with `grow`, first raise them until
// the LDS fits, as the reference's _plan grows split-K until shared memory fits
// (engine/kernels/cuda_fp8.py:1255-1276). comp: activation components (FMT_INT8).
extern "C" int qlx_plan_fit(qlx_plan* plan, int fmt, int m, int n, int k, int comp, int grow) {
  QLX_REQUIRE(plan != nullptr, "plan is NULL");
  const qlx::FmtInfo fi = fmt_info(fmt);
  QLX_REQUIRE(fi.kstep > 0, "unknown format %d", fmt);
  int rc = qlx::check_plan(plan, m, n, k, fi.kstep);
  if (rc) return rc;
  qlx::GemmArgs a = {};
  a.comp = comp;
  const int nsteps = k / fi.kstep;
  if (plan->splits > nsteps) plan->splits = nsteps;
  while (grow) {
    const int lds = qlx::layout(fi, *plan, m, n, k, a);
    if (lds <= qlx::kLdsTarget || plan->splits >= nsteps) break;
    ++plan->splits;
  }
  qlx::layout(fi, *plan, m, n, k, a);
  plan->splits = a.splits;
  return QLX_OK;
}
