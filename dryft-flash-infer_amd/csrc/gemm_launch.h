// Host side of the quantized GEMM: plan validation, LDS layout, template dispatch.
#pragma once

#include <type_traits>

#include "gemm.h"

namespace qlx {

// LDS per workgroup: plans aim at <= 64 KB (two or more workgroups per CU); gfx950 allows up
// to 160 KB for one workgroup, used when a wide batch cannot fit otherwise.
constexpr int kLdsTarget = 64 * 1024;
constexpr int kLdsLimit = 159 * 1024;  // 160 KB less room for the kernel's static LDS

struct FmtInfo {
  int kstep, nsc, xbytes;
  int bias;    // the codes carry a bias that the sums remove
  int totals;  // ... by bias totals staged in LDS (not by compute() itself)
};

template <class F>
constexpr FmtInfo info() {
  return FmtInfo{F::KSTEP, F::NSC, F::XBYTES, F::BIAS != 0.f, needs_bias_totals<F>()};
}

inline int round16(int v) { return (v + 15) & ~15; }

// Fill the derived fields of GemmArgs for (plan, shape); returns total LDS bytes or -1.
inline int layout(const FmtInfo& fi, const qlx_plan& p, int m, int n, int k, GemmArgs& a) {
  a.m = m;
  a.n = n;
  a.k = k;
  a.mode = p.mode;
  a.nsteps = k / fi.kstep;
  a.sps = (a.nsteps + p.splits - 1) / p.splits;
  a.splits = (a.nsteps + a.sps - 1) / a.sps;
  // SwiGLU tiles hold 8 gate + 8 up rows: (n/2)/8 = n/16; otherwise the last tile may be partial.
  a.ntiles = p.mode == QLX_MODE_SWIGLU ? n / 16 : (n + 15) / 16;
  const int copies = a.comp > 1 ? a.comp : 1;  // activation components staged
  a.kw = p.kw;
  a.rt = (p.waves / p.kw) * p.rw;
  a.tile_groups = (a.ntiles + a.rt - 1) / a.rt;
  a.half = n / 2;
  const int mt = m <= 16 ? 1 : (m <= 32 ? 2 : 4);
  a.xstride = round16(a.sps * fi.kstep * fi.xbytes + 16);
  const int xbytes = copies * m * a.xstride;
  const int red = p.waves * p.rw * 16 * 16 * mt * 4;
  a.off_sc = round16(xbytes > red ? xbytes : red);
  a.sc_stride = 16 * a.rt;
  const int sc_floats = fi.nsc == 0 ? a.sc_stride : a.sps * fi.nsc * a.sc_stride;
  a.off_xb = round16(a.off_sc + sc_floats * 4);
  a.xb_stride = a.sps * (fi.nsc > 1 ? fi.nsc : 1);
  const int xb_floats = fi.totals ? m * a.xb_stride : 0;
  a.off_sx = round16(a.off_xb + xb_floats * 4);
  return a.off_sx + copies * m * (a.xb_stride > 2 ? a.xb_stride : 2) * 4;
}

inline int check_plan(const qlx_plan* p, int m, int n, int k, int kstep) {
  QLX_REQUIRE(p != nullptr, "plan is NULL");
  QLX_REQUIRE(m >= 1 && m <= 64, "m=%d must be in 1..64", m);
  QLX_REQUIRE(n >= 1, "n=%d must be positive", n);
  QLX_REQUIRE(p == nullptr || p->mode != QLX_MODE_SWIGLU || n % 16 == 0, "SwiGLU needs 2I rows with I %% 8 == 0");
  QLX_REQUIRE(k >= kstep && k % kstep == 0, "K=%d must be a positive multiple of %d", k, kstep);
  QLX_REQUIRE(p->mode >= 0 && p->mode <= 2, "bad mode %d", p->mode);
  QLX_REQUIRE(p->waves == 4 || p->waves == 8, "waves must be 4 or 8");
  QLX_REQUIRE(p->kw >= 1 && p->waves % p->kw == 0, "kw must divide waves");
  QLX_REQUIRE(p->rw == 1 || p->rw == 2, "rw must be 1 or 2");
  QLX_REQUIRE(p->splits >= 1, "splits must be >= 1");
  return QLX_OK;
}

// Opt a kernel into more than 64 KB of dynamic LDS (raised to what the launch needs).
template <class F, int MT, int RW, int WAVES, bool SW, bool AN = false>
hipError_t allow_lds(int lds) {
  static int allowed = 64 * 1024;
  if (lds <= allowed) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<F, MT, RW, WAVES, SW, AN>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e == hipSuccess) allowed = lds;
  return e;
}

// Persistent single calls (gemm_persist_kernel): workgroups per CU, or 0 where the format keeps
// one workgroup per row block. Measured on the 151936-row lm_head at M = 1 (us per call over
// 1 GiB of distinct weights): W4A16 54.5 as one workgroup per row block, 45.0 with one
// persistent workgroup per CU, 45.9 with two; FP8 68.1 / 67.2 / 64.9; W8A16 70.8 / 72.6 /
// 73.3 (before the bias-total cache).
template <class F>
constexpr int persist_per_cu() {
  if constexpr (std::is_same<F, FmtW4>::value) return 1;
  if constexpr (std::is_same<F, FmtFP8>::value) return 2;
  return 0;
}

inline int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  return cus[dev];
}

// Launch the persistent kernel when the call suits it: whole K (one slice), bf16 or SwiGLU
// output, whole 16-row tiles, and at least two row blocks per workgroup. Returns false (nothing
// launched) otherwise.
template <class F, int MT, int RW, int WAVES>
bool launch_persist(const GemmArgs& a, int lds, hipStream_t st, hipError_t* err) {
  constexpr int wpc = persist_per_cu<F>();
  if constexpr (wpc == 0) {
    return false;
  } else {
    if (a.splits != 1 || a.an_counter || a.n % 16 || (a.mode != QLX_MODE_BF16 && a.mode != QLX_MODE_SWIGLU))
      return false;
    const int cus = device_cus();
    const int grid = cus * wpc;
    if (cus <= 0 || a.tile_groups < 2 * grid) return false;
    constexpr int NJ = std::is_same<F, FmtW4>::value ? 2 : (std::is_same<F, FmtW8>::value ? 1 : 0);
    GemmArgs b = a;
    b.off_red = round16(lds);
    b.off_bt = b.off_red + WAVES * RW * 16 * 16 * MT * 4;
    const int total = b.off_bt + a.nsteps * NJ * MT * 16 * 4;
    if (total > kLdsLimit) return false;
    const void* fn = a.mode == QLX_MODE_SWIGLU
                         ? reinterpret_cast<const void*>(&gemm_persist_kernel<F, MT, RW, WAVES, true>)
                         : reinterpret_cast<const void*>(&gemm_persist_kernel<F, MT, RW, WAVES, false>);
    static int allowed[2] = {64 * 1024, 64 * 1024};  // per instantiation: [SwiGLU]
    int& ok = allowed[a.mode == QLX_MODE_SWIGLU];
    if (total > ok) {
      if ((*err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, total)) != hipSuccess)
        return true;
      ok = total;
    }
    if (a.mode == QLX_MODE_SWIGLU)
      gemm_persist_kernel<F, MT, RW, WAVES, true><<<grid, WAVES * 64, total, st>>>(b);
    else
      gemm_persist_kernel<F, MT, RW, WAVES, false><<<grid, WAVES * 64, total, st>>>(b);
    *err = hipGetLastError();
    return true;
  }
}

// The ring kernel (gemm_ring_w4_kernel) where it applies: 4-bit weights, at most 16 tokens,
// one tile per wave (kw = 1), bf16 outputs, the persistent launch's other conditions, at least
// 4 steps per row block, and LDS for a ring of 8 steps per wave (4 where the activation leaves
// less room). One workgroup per CU.
template <class F, int MT, int RW, int WAVES>
bool launch_ring(const GemmArgs& a, int lds, hipStream_t st, hipError_t* err) {
  if constexpr (!std::is_same<F, FmtW4>::value || RW != 1 || MT != 1) {
    return false;
  } else {
    if (a.kw != 1 || a.splits != 1 || a.an_counter || a.n % 16 || a.mode != QLX_MODE_BF16 || a.nsteps < 4)
      return false;
    const int grid = device_cus();
    if (grid <= 0 || a.tile_groups < 2 * grid) return false;
    GemmArgs b = a;
    b.off_bt = round16(a.off_sc + 2 * ring_scale_words(a.nsteps, a.rt) * 4);
    b.off_ring = round16(b.off_bt + a.nsteps * 2 * 16 * 4);
    const int slot = F::LOADS * 1024 * WAVES;  // one step of every wave
    // Two workgroups per CU (four waves per SIMD, whose issue overlaps) with 3-step rings where
    // LDS allows, else one with 8 or 4 steps.
    struct Shape { int wpc, depth; const void* fn; };
    const Shape shapes[] = {{2, 3, reinterpret_cast<const void*>(&gemm_ring_w4_kernel<WAVES, 3, 2>)},
                            {1, 8, reinterpret_cast<const void*>(&gemm_ring_w4_kernel<WAVES, 8, 1>)},
                            {1, 4, reinterpret_cast<const void*>(&gemm_ring_w4_kernel<WAVES, 4, 1>)}};
    int pick = -1;
    for (int i = 0; i < 3 && pick < 0; ++i) {
      const int lds_i = b.off_ring + shapes[i].depth * slot;
      if (lds_i * shapes[i].wpc <= kLdsLimit && a.tile_groups >= 2 * grid * shapes[i].wpc) pick = i;
    }
    if (pick < 0) return false;
    const int total = b.off_ring + shapes[pick].depth * slot;
    const void* fn = shapes[pick].fn;
    static int allowed[3] = {64 * 1024, 64 * 1024, 64 * 1024};
    int& ok = allowed[pick];
    if (total > ok) {
      if ((*err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, total)) != hipSuccess)
        return true;
      ok = total;
    }
    void* args[] = {&b};
    *err = hipLaunchKernel(fn, dim3(grid * shapes[pick].wpc), dim3(WAVES * 64), args, (size_t)total, st);
    return true;
  }
}

// AN_OK: this format's entry points include the fused add-norm (qlx_linear_add_norm), which
// launches the AN instantiation when a.an_counter is set.
template <class F, int MT, int RW, int WAVES, bool AN_OK>
hipError_t launch_one(const GemmArgs& a, int lds, hipStream_t st) {
  const int grid = a.tile_groups * a.splits;
  hipError_t e;
  if (launch_ring<F, MT, RW, WAVES>(a, lds, st, &e)) return e;
  if (launch_persist<F, MT, RW, WAVES>(a, lds, st, &e)) return e;
  if constexpr (AN_OK) {
    if (a.an_counter) {
      if ((e = allow_lds<F, MT, RW, WAVES, false, true>(lds)) != hipSuccess) return e;
      gemm_kernel<F, MT, RW, WAVES, false, true><<<grid, WAVES * 64, lds, st>>>(a);
      return hipGetLastError();
    }
  }
  if (a.mode == QLX_MODE_SWIGLU) {
    if ((e = allow_lds<F, MT, RW, WAVES, true>(lds)) != hipSuccess) return e;
    gemm_kernel<F, MT, RW, WAVES, true><<<grid, WAVES * 64, lds, st>>>(a);
  } else {
    if ((e = allow_lds<F, MT, RW, WAVES, false>(lds)) != hipSuccess) return e;
    gemm_kernel<F, MT, RW, WAVES, false><<<grid, WAVES * 64, lds, st>>>(a);
  }
  return hipGetLastError();
}

template <class F, int MT, bool AN_OK>
hipError_t launch_mt(const GemmArgs& a, const qlx_plan& p, int lds, hipStream_t st) {
  if (p.waves == 4)
    return p.rw == 1 ? launch_one<F, MT, 1, 4, AN_OK>(a, lds, st) : launch_one<F, MT, 2, 4, AN_OK>(a, lds, st);
  return p.rw == 1 ? launch_one<F, MT, 1, 8, AN_OK>(a, lds, st) : launch_one<F, MT, 2, 8, AN_OK>(a, lds, st);
}

template <class F, bool AN_OK = false>
int launch_gemm(const char* name, GemmArgs a, const qlx_plan* plan, int m, int n, int k, void* stream) {
  int rc = check_plan(plan, m, n, k, F::KSTEP);
  if (rc) return rc;
  QLX_REQUIRE(!a.tiled || n % 16 == 0, "%s: tiled weights have rows %% 16 == 0 (n=%d)", name, n);
  const qlx_plan& p = *plan;
  const int lds = layout(info<F>(), p, m, n, k, a);
  QLX_REQUIRE(lds <= kLdsLimit, "%s: plan needs %d bytes of LDS (> %d); use more splits", name, lds, kLdsLimit);
  QLX_REQUIRE(p.mode != QLX_MODE_PLANES || a.splits == p.splits,
              "%s: %d splits over %d steps leave %d non-empty planes", name, p.splits, a.nsteps, a.splits);
  if (p.mode == QLX_MODE_PLANES || a.splits > 1)
    QLX_REQUIRE(p.workspace != nullptr, "%s: split-K needs a workspace", name);
  if (p.mode != QLX_MODE_PLANES && a.splits > 1) QLX_REQUIRE(p.tickets != nullptr, "%s: split-K needs tickets", name);
  a.work = p.workspace;
  a.tickets = p.tickets;
  const int mt = (m + 15) / 16;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (a.an_counter) {
    QLX_REQUIRE(AN_OK && p.mode == QLX_MODE_BF16, "%s: the fused add-norm takes bf16 output (mode 0)", name);
    QLX_REQUIRE(n % 8 == 0, "%s: the fused add-norm needs n %% 8 == 0 (n=%d)", name, n);
    QLX_REQUIRE(a.resid && a.norm_w && a.res_out && a.normed, "%s: add-norm operand is NULL", name);
  }
  if (mt == 1)
    e = launch_mt<F, 1, AN_OK>(a, p, lds, st);
  else if (mt == 2)
    e = launch_mt<F, 2, AN_OK>(a, p, lds, st);
  else
    e = launch_mt<F, 4, AN_OK>(a, p, lds, st);
  return hip_status(e, name);
}

// Fused residual add + RMSNorm launches (a.an_counter and the add-norm operands set), one per
// format, each defined in the file that instantiates that format's GEMM.
int add_norm_w8a16(const GemmArgs& a, const qlx_plan* plan, int m, int n, int k, void* stream);
int add_norm_w4a16(const GemmArgs& a, const qlx_plan* plan, int m, int n, int k, void* stream);
int add_norm_fp8(const GemmArgs& a, const qlx_plan* plan, int m, int n, int k, void* stream);
int add_norm_ref(const GemmArgs& a, int bits, const qlx_plan* plan, int m, int n, int k, void* stream);

}  // namespace qlx
