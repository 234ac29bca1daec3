// Decode-step executor: every quantized projection of a decode step in one launch.
//
// The reference runs each projection as its own CUDA launch inside a graph and hides the
// launch gap with programmatic dependent launch: a GEMM's weight loads start while the
// previous kernel drains (engine/kernels/cuda_fp8.py:47-50, 150-169, 252;
// engine/kernels/cuda_jit.py:218-262). HIP has
// no such launch attribute, and at M = 1 most projections are 10-25 MB, so a separate launch
// (about 1.6 us) plus first-load latency, activation staging and the epilogue cost as much as
// the weight stream itself.
//
// Here one cooperative launch walks the projections in order. Projection c may read what
// projections < c wrote, so a workgroup starts projection c only after every workgroup has
// finished c - 1 (a stage counter of arrivals), but it issues c's first weight loads before
// it waits: weights do not depend on activations. Activations are read and outputs written
// device-coherently, since other workgroups of the same launch produce and consume them.
//
// Every wait is bounded: cooperative launch guarantees all workgroups are resident, and a
// spin that still exceeds its limit records an error flag and leaves the wait, so the
// kernel always ends.
#include <vector>

#include "gemm_launch.h"

namespace qlx {

// One projection of the stack, as the executor reads it from device memory.
struct StackDesc {
  GemmArgs a;
  int items;  // work items: tile_groups * splits
  int sw;     // SwiGLU epilogue
  int pad[2];
};

// sync[0]: arrivals (P per projection), sync[1]: exits, sync[2]: error flag. Zero at launch;
// the last workgroup to exit zeroes [0] and [1] again.
__device__ __forceinline__ void stage_arrive(int* sync) {
  publish_stores();  // this workgroup's outputs are device-visible before it is counted
  if (threadIdx.x == 0) __hip_atomic_fetch_add(&sync[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void stage_wait(int* sync, int target, int spin_limit) {
  if (threadIdx.x == 0) {
    int spins = 0;
    while (__hip_atomic_load(&sync[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > spin_limit) {
        __hip_atomic_store(&sync[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <class F, int WAVES>
__global__ void __launch_bounds__(WAVES * 64)
stack_kernel(const StackDesc* __restrict__ calls, int ncalls, int* sync, int spin_limit) {
  extern __shared__ __align__(16) char lds[];
  constexpr int PF = PipeDepth<1>::PF;
  const int P = gridDim.x, p = blockIdx.x;
  Item<1> it;
  uint4 buf[PF][1][F::LOADS];
  auto coords = [&](const GemmArgs& a, int item, int& tg, int& s) {
    tg = item / a.splits;
    s = item - tg * a.splits;
  };
  // The first item of projection 0 needs no wait.
  bool prefetched = false;
  if (p < calls[0].items) {
    int tg, s;
    coords(calls[0].a, p, tg, s);
    item_prefetch<F, 1>(calls[0].a, tg, s, it, buf);
    prefetched = true;
  }
  for (int c = 0; c < ncalls; ++c) {
    const StackDesc& d = calls[c];
    if (c > 0) stage_wait(sync, P * c, spin_limit);
    for (int item = p; item < d.items; item += P) {
      if (!prefetched) {
        int tg, s;
        coords(d.a, item, tg, s);
        item_prefetch<F, 1>(d.a, tg, s, it, buf);
      }
      prefetched = false;
      if (d.sw)
        item_run<F, 1, 1, WAVES, true, true>(d.a, lds, it, buf);
      else
        item_run<F, 1, 1, WAVES, false, true>(d.a, lds, it, buf);
      __syncthreads();  // LDS is reused by the next item
    }
    stage_arrive(sync);
    // Projection c + 1's weights start streaming before its wait.
    if (c + 1 < ncalls && p < calls[c + 1].items) {
      int tg, s;
      coords(calls[c + 1].a, p, tg, s);
      item_prefetch<F, 1>(calls[c + 1].a, tg, s, it, buf);
      prefetched = true;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&sync[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == P - 1) {  // everyone has left every wait: reset for the next launch
      __hip_atomic_store(&sync[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&sync[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

constexpr int kStackWaves = 8;

template <class F>
const void* stack_fn() {
  return reinterpret_cast<const void*>(&stack_kernel<F, kStackWaves>);
}

const void* stack_fn_for(int fmt) {
  switch (fmt) {
    case QLX_FMT_W8A16: return stack_fn<FmtW8>();
    case QLX_FMT_W4A16: return stack_fn<FmtW4>();
    case QLX_FMT_FP8: return stack_fn<FmtFP8>();
    default: return nullptr;
  }
}

FmtInfo stack_info(int fmt) {
  switch (fmt) {
    case QLX_FMT_W8A16: return info<FmtW8>();
    case QLX_FMT_W4A16: return info<FmtW4>();
    default: return info<FmtFP8>();
  }
}

// Plan of one projection for P resident workgroups of 8 waves: the (kw, splits) whose busiest
// workgroup streams the fewest bytes, counting each extra item as 64 KB of overhead; ties go
// to fewer items.
qlx_plan stack_plan(const FmtInfo& fi, int mode, int m, int n, int k, int P, int bytes_per_k) {
  qlx_plan best = {};
  double best_cost = 1e300;
  const int nsteps = k / fi.kstep;
  const int ntiles = n / 16;
  for (int kw = 1; kw <= kStackWaves; kw *= 2) {
    for (int splits = 1; splits <= 8 && splits <= nsteps; ++splits) {
      qlx_plan p = {};
      p.mode = mode;
      p.waves = kStackWaves;
      p.kw = kw;
      p.rw = 1;
      p.splits = splits;
      GemmArgs a = {};
      if (layout(fi, p, m, n, k, a) > kLdsTarget) continue;
      if (a.splits != splits) continue;  // not a normalised split count
      const int items = a.tile_groups * a.splits;
      const int per_wg = (items + P - 1) / P;
      const double item_bytes = (double)a.rt * 16 * (double)a.sps * fi.kstep * bytes_per_k;
      const double cost = per_wg * (item_bytes + 65536.0) + 1e-3 * items;
      (void)ntiles;
      if (cost < best_cost) {
        best_cost = cost;
        best = p;
      }
    }
  }
  return best;
}

}  // namespace qlx

using namespace qlx;

extern "C" {

int qlx_stack_desc_size(void) { return (int)sizeof(StackDesc); }

int qlx_stack_build(int fmt, int m, const qlx_stack_call* calls, int ncalls, int groups_per_cu, void* desc,
                    qlx_plan* plans, float* workspace, int* tickets, long long* workspace_floats,
                    int* tickets_needed, int* grid, int* lds_bytes) {
  const void* fn = stack_fn_for(fmt);
  QLX_REQUIRE(fn != nullptr, "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(m >= 1 && m <= 16, "the decode executor serves m = 1..16 (got %d)", m);
  QLX_REQUIRE(calls != nullptr && ncalls >= 1, "no projections");
  QLX_REQUIRE(groups_per_cu >= 1 && groups_per_cu <= 4, "groups_per_cu must be 1..4");
  int dev = 0, cus = 0, occ = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_status(e, "stack_build");
  const FmtInfo fi = stack_info(fmt);
  const int bytes_num = fmt == QLX_FMT_W4A16 ? 1 : 2;  // bytes per 2 k values
  // LDS of the widest projection decides occupancy.
  int lds = 0;
  std::vector<qlx_plan> plans_v;  // per projection, for the final P
  int P = 0;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      if (lds > 64 * 1024) {
        e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return hip_status(e, "stack_build");
      }
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kStackWaves * 64, lds);
      if (e != hipSuccess) return hip_status(e, "stack_build");
      QLX_REQUIRE(occ >= 1, "the executor does not fit a CU with %d bytes of LDS", lds);
      P = cus * (occ < groups_per_cu ? occ : groups_per_cu);
    }
    const int Pp = pass == 0 ? cus * groups_per_cu : P;
    plans_v.clear();
    lds = 0;
    for (int c = 0; c < ncalls; ++c) {
      const qlx_stack_call& q = calls[c];
      QLX_REQUIRE(q.n >= 16 && q.n % 16 == 0 && q.k % fi.kstep == 0 && q.k > 0,
                  "projection %d: n=%d k=%d do not fit the tiled format", c, q.n, q.k);
      QLX_REQUIRE(q.mode == QLX_MODE_BF16 || q.mode == QLX_MODE_SWIGLU, "projection %d: mode %d", c, q.mode);
      qlx_plan p = stack_plan(fi, q.mode, m, q.n, q.k, Pp, bytes_num);
      QLX_REQUIRE(p.waves == kStackWaves, "projection %d: no plan fits", c);
      GemmArgs a = {};
      const int l = layout(fi, p, m, q.n, q.k, a);
      if (l > lds) lds = l;
      plans_v.push_back(p);
    }
  }
  long long ws = 0;
  int tk = 0;
  StackDesc* out = reinterpret_cast<StackDesc*>(desc);
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    StackDesc d = {};
    d.a.w = q.w;
    d.a.ws = q.w_scale;
    d.a.x = q.x;
    d.a.y = q.y;
    d.a.tiled = 1;
    layout(fi, plans_v[c], m, q.n, q.k, d.a);
    d.a.work = workspace;
    d.a.tickets = tickets;
    d.items = d.a.tile_groups * d.a.splits;
    d.sw = q.mode == QLX_MODE_SWIGLU;
    if (d.a.splits > 1) {
      const long long need = (long long)d.a.splits * m * q.n;
      if (need > ws) ws = need;
      if (d.a.tile_groups > tk) tk = d.a.tile_groups;
    }
    if (out) out[c] = d;
    if (plans) {
      plans[c] = plans_v[c];
      plans[c].splits = d.a.splits;
      plans[c].workspace = d.a.splits > 1 ? workspace : nullptr;
      plans[c].tickets = d.a.splits > 1 ? tickets : nullptr;
    }
  }
  if (workspace_floats) *workspace_floats = ws;
  if (tickets_needed) *tickets_needed = tk;
  if (grid) *grid = P;
  if (lds_bytes) *lds_bytes = lds;
  return QLX_OK;
}

int qlx_stack_run(int fmt, const void* desc, int ncalls, int grid, int lds_bytes, int* sync, int spin_limit,
                  void* stream) {
  const void* fn = stack_fn_for(fmt);
  QLX_REQUIRE(fn != nullptr, "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(desc && sync && ncalls >= 1 && grid >= 1 && spin_limit >= 1, "bad executor arguments");
  void* args[] = {(void*)&desc, (void*)&ncalls, (void*)&sync, (void*)&spin_limit};
  hipError_t e = hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kStackWaves * 64), args, (unsigned)lds_bytes,
                                            (hipStream_t)stream);
  return hip_status(e, "stack_run");
}

}  // extern "C"
