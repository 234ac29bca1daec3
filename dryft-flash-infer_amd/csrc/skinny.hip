// Skinny GEMM for 16..64 tokens (speculative verification, small batches).
//
// The decode kernel (gemm.h) stages a workgroup's whole K slice of the activation in LDS
// before its MFMA loop, and each wave keeps MT token fragments of every tile in registers.
// Past 16 tokens that costs too much: the staged slice outgrows LDS, so K is cut into many
// slices (each re-staging 64 tokens of x and writing fp32 partials), and at 64 tokens the
// registers spill. Here the activation streams through LDS one K step at a time instead:
//   * a workgroup owns WAVES x RW 16-row tiles (RW = 2 per wave up to 32 tokens: every
//     activation fragment read from LDS feeds two tiles' MFMAs) and one K slice; every wave runs the same steps, so
//     the waves share each staged activation chunk [m][KSTEP] and its scales, in two
//     buffers: while a step's MFMAs run, the next step's activation is fetched and written
//     to the other buffer, and one barrier per step publishes it;
//   * weights stream into registers PF steps ahead, in the MI355X tile layout, and go
//     through the format's MFMA step with the decode kernel's arithmetic: per-group fp32
//     partials times the group scale, the code bias removed by the same MFMA chain with
//     every code at the bias (run here on the fragments the step reads anyway);
//   * K slices write fp32 planes [slices][m][n] that the plane consumers reduce in slice
//     order (qlx_reduce_planes, qlx_swiglu): deterministic, like the reference's split-K
//     planes (engine/kernels/cuda_fp8.py:965-981).
// The reference serves these batches with the same kernels as decode, up to 64 rows in
// tiles of 8 tokens (engine/kernels/cuda_fp8.py:1227-1234, 1404-1423).
#include "gemm_launch.h"

namespace qlx {

// Weight steps in flight per wave (even: the two activation register sets alternate with
// the step's parity): 4 where the registers allow it.
__host__ __device__ constexpr int skinny_pf(int mt) { return mt == 1 ? 4 : 2; }
// 16-row tiles per wave, sharing each activation fragment read from LDS: two up to 32 tokens,
// one at 64 (two would need more than the 256 registers of two waves per SIMD).
__host__ __device__ constexpr int skinny_rw(int mt) { return mt >= 4 ? 1 : 2; }
// Token fragments (16 tokens each) a batch is computed with: 1, 2 or 4 (33..48 tokens run as 4).
__host__ __device__ constexpr int skinny_mt_of(int m) { return m <= 16 ? 1 : (m <= 32 ? 2 : 4); }

// LDS of one activation chunk: [m rows][xstride bytes] of x in the format's B order, then
// the group scales [NSC][16 rows x the workgroup's tiles] as floats.
struct SkinnyLayout {
  int xstride, off_sc, sc_stride, chunk;
};

__host__ __device__ constexpr int up16(int v) { return (v + 15) & ~15; }

template <class F>
__host__ __device__ inline SkinnyLayout skinny_layout(int m, int waves) {
  SkinnyLayout L{};
  L.xstride = F::KSTEP * F::XBYTES + 16;  // rows 4 banks apart: a B read of 16 rows is conflict-free
  L.sc_stride = 16 * waves * skinny_rw(skinny_mt_of(m));
  L.off_sc = up16(m * L.xstride);
  L.chunk = up16(L.off_sc + (F::NSC > 0 ? F::NSC : 0) * L.sc_stride * 4);
  return L;
}

// x chunks (16 bytes, 8 values) of one K step that each thread stages.
template <class F, int WAVES>
struct SkinnyStage {
  static constexpr int PER_ROW = F::KSTEP / 8;
  static constexpr int MAX = (64 * PER_ROW + WAVES * 64 - 1) / (WAVES * 64);
};

// One K step of RW tiles against MT token fragments of the staged chunk `ch`, the format's
// arithmetic (FmtW4::compute, FmtW8::compute) with two changes: each activation fragment read
// from LDS feeds the MFMAs of all RW tiles, and the code bias is removed with the bias chain
// run on the same fragment (A = the bias in every position; the chain FmtW4/FmtW8::bias_chain
// runs, so it rounds the same and a zero row still gives exactly zero). W4: per-group scales
// from the chunk at sc[j][row]; W8: the per-channel scale comes in the epilogue.
template <class F, int MT, int RW>
__device__ __forceinline__ void skinny_step(f32x4 (&acc)[RW][MT], const uint4 (&c)[RW][F::LOADS], const char* ch,
                                            const SkinnyLayout& L, int lane, const int (&xoff)[MT],
                                            const int (&rowl)[RW]) {
  if constexpr (std::is_same<F, FmtW4>::value) {
    const uint4 ab = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136 = the code bias
    const float* sc = reinterpret_cast<const float*>(ch + L.off_sc);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 tmp[RW][MT], tb[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        tb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < RW; ++r) tmp[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      const int kb = (j * 128 + (lane >> 4) * 32) * 2;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint4 av[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const uint32_t wd = t == 0 ? c[r][j].x : t == 1 ? c[r][j].y : t == 2 ? c[r][j].z : c[r][j].w;
          av[r] = uint4{nib_pair(wd, 0), nib_pair(wd, 4), nib_pair(wd, 8), nib_pair(wd, 12)};
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(ch + xoff[mt] + kb + t * 16);
#pragma unroll
          for (int r = 0; r < RW; ++r)
            tmp[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[r]), as_bf16x8(bv), tmp[r][mt], 0, 0, 0);
          tb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ab), as_bf16x8(bv), tb[mt], 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc + j * L.sc_stride + rowl[r]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[r][mt][i] = fmaf(s4[i], tmp[r][mt][i] - tb[mt][i], acc[r][mt][i]);
      }
    }
  } else {
    static_assert(std::is_same<F, FmtW8>::value, "skinny_step: W4A16 or W8A16");
    const uint4 ab = {0x43004300u, 0x43004300u, 0x43004300u, 0x43004300u};  // bf16 128
    f32x4 tmp[RW][MT], tb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      tb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < RW; ++r) tmp[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = (j * 64 + (lane >> 4) * 16) * 2;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        uint4 av[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const uint32_t w0 = (t == 0 ? c[r][j].x : c[r][j].z) ^ 0x80808080u;
          const uint32_t w1 = (t == 0 ? c[r][j].y : c[r][j].w) ^ 0x80808080u;
          const uint2 lo = bytes_to_bf16(w0), hi = bytes_to_bf16(w1);
          av[r] = uint4{lo.x, lo.y, hi.x, hi.y};
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(ch + xoff[mt] + kb + t * 16);
#pragma unroll
          for (int r = 0; r < RW; ++r)
            tmp[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[r]), as_bf16x8(bv), tmp[r][mt], 0, 0, 0);
          tb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ab), as_bf16x8(bv), tb[mt], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][mt][i] += tmp[r][mt][i] - tb[mt][i];
  }
}

// Two workgroups per CU: each wave at most 256 registers.
template <class F, int MT, int WAVES, bool SW>
__global__ void __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WAVES == 4 ? 2 : 1)))
skinny_kernel(GemmArgs a, SkinnyLayout L, int steps_per_slice) {
  static_assert(F::LOADS == 2, "a tile step is two 1 KB loads per wave");
  static_assert(F::NSC == 0 || std::is_same<F, FmtW4>::value, "group scales as W4A16 lays them out");
  extern __shared__ __align__(16) char lds[];
  constexpr int PF = skinny_pf(MT), RW = skinny_rw(MT);
  constexpr int SPR = SkinnyStage<F, WAVES>::PER_ROW, SMAX = SkinnyStage<F, WAVES>::MAX;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tg = blockIdx.x / a.splits, s = blockIdx.x - tg * a.splits;
  const int step0 = s * steps_per_slice;
  const int nst = min(a.nsteps, step0 + steps_per_slice) - step0;
  const int last = step0 + nst - 1;
  // Wave w holds tiles RW w .. RW w + RW - 1 of the workgroup's RW WAVES tiles.
  int tile[RW], wrow[RW], rowl[RW];
  bool act[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    tile[r] = (tg * WAVES + wave) * RW + r;
    act[r] = tile[r] < a.ntiles;
    wrow[r] = act[r] ? weight_row(a, tile[r], lane & 15) : 0;
    rowl[r] = (wave * RW + r) * 16 + 4 * (lane >> 4);
  }

  // Weight steps step0 .. step0 + PF - 1 first: nothing else they wait for. A tile past the
  // end streams tile 0 of the workgroup (always real); its results are dropped.
  uint4 buf[PF][RW][F::LOADS];
#pragma unroll
  for (int p = 0; p < PF; ++p)
#pragma unroll
    for (int r = 0; r < RW; ++r) load_chunk<F>(buf[p][r], a, act[r] ? wrow[r] : weight_row(a, tg * WAVES * RW, lane & 15),
                                               min(step0 + p, last), lane);

  // A step's staged data: SMAX 16-byte activation chunks and (group formats) SCMAX raw bf16
  // scales per thread, fetched into registers ahead of time and written to LDS later.
  constexpr int SCMAX = F::NSC > 0 ? (F::NSC * 16 * WAVES * RW + WAVES * 64 - 1) / (WAVES * 64) : 1;
  struct Staged {
    uint4 x[SMAX];
    uint32_t sc[SCMAX];
  };
  const uint16_t* x = reinterpret_cast<const uint16_t*>(a.x);
  auto fetch_x = [&](int step, Staged& st) {
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const int q = threadIdx.x + u * WAVES * 64;
      if (q < a.m * SPR) {
        const int mm = q / SPR, c = q - mm * SPR;
        const u32x4 v = *gmem(reinterpret_cast<const u32x4*>(x + (size_t)mm * a.k + step * F::KSTEP + c * 8));
        st.x[u] = uint4{v[0], v[1], v[2], v[3]};
      }
    }
    if constexpr (F::NSC > 0) {
#pragma unroll
      for (int u = 0; u < SCMAX; ++u) {
        const int q = threadIdx.x + u * WAVES * 64;
        st.sc[u] = 0u;
        if (q < F::NSC * L.sc_stride) {
          const int j = q / L.sc_stride, rl = q - j * L.sc_stride;
          const int t = tg * WAVES * RW + (rl >> 4);
          if (t < a.ntiles)  // group 2 step + j of the tile row's weight row, as F::scale reads it
            st.sc[u] = gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)weight_row(a, t, rl & 15) * (a.k >> 7) +
                                                                      F::NSC * step + j];
        }
      }
    }
  };
  auto put_x = [&](char* ch, const Staged& st) {
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const int q = threadIdx.x + u * WAVES * 64;
      if (q < a.m * SPR) {
        const int mm = q / SPR, c = q - mm * SPR;
        *reinterpret_cast<uint4*>(ch + mm * L.xstride + c * 16) = F::order(st.x[u]);
      }
    }
    if constexpr (F::NSC > 0) {
      float* sc = reinterpret_cast<float*>(ch + L.off_sc);
#pragma unroll
      for (int u = 0; u < SCMAX; ++u) {
        const int q = threadIdx.x + u * WAVES * 64;
        if (q < F::NSC * L.sc_stride) sc[q] = bf2f(st.sc[u]);  // [j][row]: q = j sc_stride + row
      }
    }
  };

  // Two chunk buffers and two register sets: step i's MFMAs run from buffer i & 1; the
  // activation of step i + 2 is fetched into register set i & 1 (its previous contents, step
  // i, went to LDS a step ago), and step i + 1's, fetched a whole step earlier, is written to
  // the other buffer (whose step i - 1 every wave finished before the last barrier); one
  // barrier per step publishes it. The fetches thus have a step of MFMAs to arrive in.
  Staged rr[2];
  fetch_x(step0, rr[0]);
  if (nst > 1) fetch_x(step0 + 1, rr[1]);
  put_x(lds, rr[0]);
  __syncthreads();
  f32x4 acc[RW][MT];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  int xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xoff[mt] = min(16 * mt + (lane & 15), a.m - 1) * L.xstride;

  for (int i0 = 0; i0 < nst; i0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int i = i0 + p;
      if (i < nst) {  // uniform across the workgroup
        if (i + 2 < nst) fetch_x(step0 + i + 2, rr[p & 1]);
        skinny_step<F, MT, RW>(acc, buf[p], lds + (i & 1) * L.chunk, L, lane, xoff, rowl);
#pragma unroll
        for (int r = 0; r < RW; ++r)
          load_chunk<F>(buf[p][r], a, act[r] ? wrow[r] : weight_row(a, tg * WAVES * RW, lane & 15),
                        min(step0 + i + PF, last), lane);
        if (i + 1 < nst) put_x(lds + ((i + 1) & 1) * L.chunk, rr[(p + 1) & 1]);
        __syncthreads();
      }
    }
  }

  // Epilogue: lane holds rows 4 (lane >> 4) + 0..3 of each tile for token 16 mt + (lane & 15).
  const int r0 = 4 * (lane >> 4);
  const uint16_t* ws = reinterpret_cast<const uint16_t*>(a.ws);
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    if (!act[r]) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int mm = 16 * mt + (lane & 15);
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // per-channel formats scale once here; group formats scaled every group in the step
        v[i] = acc[r][mt][i];
        if constexpr (F::NSC == 0) v[i] *= bf2f(gmem(ws)[weight_row(a, tile[r], r0 + i)]);
      }
      if (a.splits > 1) {  // fp32 plane s, rows in natural order
        if (mm < a.m) {
          float* plane = a.work + ((size_t)s * a.m + mm) * a.n;
#pragma unroll
          for (int i = 0; i < 4; ++i) plane[weight_row(a, tile[r], r0 + i)] = v[i];
        }
      } else if constexpr (SW) {
        // Tile rows 0..7 are gate rows 8 tile + 0..7 (lanes 0..31), rows 8..15 the matching up
        // rows (lanes 32..63): gate lane l pairs with up lane l + 32.
        float u[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) u[i] = __shfl_down(v[i], 32, 64);
        if (lane < 32 && mm < a.m) {
          const int o = 8 * tile[r] + r0;
          store_pair(y, (size_t)mm * a.half + o, swiglu_bf(v[0], u[0]), swiglu_bf(v[1], u[1]));
          store_pair(y, (size_t)mm * a.half + o + 2, swiglu_bf(v[2], u[2]), swiglu_bf(v[3], u[3]));
        }
      } else if (mm < a.m) {
        const int o = 16 * tile[r] + r0;
        store_pair(y, (size_t)mm * a.n + o, v[0], v[1]);
        store_pair(y, (size_t)mm * a.n + o + 2, v[2], v[3]);
      }
    }
  }
}

template <class F, int MT, int WAVES>
hipError_t skinny_launch(const GemmArgs& a, const SkinnyLayout& L, int sps, hipStream_t st) {
  const int lds = 2 * L.chunk;
  const dim3 grid(a.tile_groups * a.splits), block(WAVES * 64);
  const void* fn = a.mode == QLX_MODE_SWIGLU ? reinterpret_cast<const void*>(&skinny_kernel<F, MT, WAVES, true>)
                                              : reinterpret_cast<const void*>(&skinny_kernel<F, MT, WAVES, false>);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  if (a.mode == QLX_MODE_SWIGLU)
    skinny_kernel<F, MT, WAVES, true><<<grid, block, lds, st>>>(a, L, sps);
  else
    skinny_kernel<F, MT, WAVES, false><<<grid, block, lds, st>>>(a, L, sps);
  return hipGetLastError();
}

template <class F, int WAVES>
hipError_t skinny_mt(const GemmArgs& a, const SkinnyLayout& L, int sps, hipStream_t st) {
  const int mt = skinny_mt_of(a.m);  // the plan and the layout derive the tiles per wave from it too
  if (mt == 1) return skinny_launch<F, 1, WAVES>(a, L, sps, st);
  if (mt == 2) return skinny_launch<F, 2, WAVES>(a, L, sps, st);
  return skinny_launch<F, 4, WAVES>(a, L, sps, st);
}

// Waves and K slices: 4 waves per workgroup (two workgroups per CU), and K slices until about
// 240 workgroups, each slice at least 2 steps (the weight pipeline).
template <class F>
void skinny_plan(int m, int n, int k, int* waves, int* splits) {
  const int nsteps = k / F::KSTEP;
  const int ntiles = n / 16;  // SwiGLU tiles hold 8 gate + 8 up rows: also n / 16
  *waves = 4;
  const int rt = 4 * skinny_rw(skinny_mt_of(m));
  const int groups = (ntiles + rt - 1) / rt;
  int s = (240 + groups - 1) / groups;
  const int most = nsteps / 2 > 1 ? nsteps / 2 : 1;
  if (s > most) s = most;
  if (s < 1) s = 1;
  *splits = s;
}

template <class F>
int skinny_run(const char* name, GemmArgs a, int m, int n, int k, int mode, const qlx_plan* plan, void* stream) {
  QLX_REQUIRE(plan != nullptr, "%s: plan is NULL", name);
  QLX_REQUIRE(m >= 1 && m <= 64, "%s: m=%d must be in 1..64", name, m);
  QLX_REQUIRE(n >= 16 && n % 16 == 0 && k >= F::KSTEP && k % F::KSTEP == 0,
              "%s: n=%d k=%d do not fit the tiled format", name, n, k);
  QLX_REQUIRE(mode == QLX_MODE_BF16 || mode == QLX_MODE_SWIGLU, "%s: mode %d", name, mode);
  QLX_REQUIRE(plan->waves == 4 || plan->waves == 8, "%s: waves must be 4 or 8", name);
  const int nsteps = k / F::KSTEP;
  QLX_REQUIRE(plan->splits >= 1 && plan->splits <= nsteps, "%s: splits must be 1..%d", name, nsteps);
  const int sps = (nsteps + plan->splits - 1) / plan->splits;
  const int splits = (nsteps + sps - 1) / sps;  // every slice non-empty
  QLX_REQUIRE(splits == 1 || plan->workspace != nullptr, "%s: K slices need a workspace", name);
  a.m = m;
  a.n = n;
  a.k = k;
  a.mode = mode;
  a.nsteps = nsteps;
  a.splits = splits;
  a.sps = sps;
  a.kw = 1;
  a.rt = plan->waves * skinny_rw(skinny_mt_of(m));
  a.ntiles = n / 16;
  a.tile_groups = (a.ntiles + a.rt - 1) / a.rt;
  a.half = n / 2;
  a.tiled = 1;
  a.work = plan->workspace;
  const SkinnyLayout L = plan->waves == 8 ? skinny_layout<F>(m, 8) : skinny_layout<F>(m, 4);
  QLX_REQUIRE(2 * L.chunk <= kLdsLimit, "%s: %d bytes of LDS", name, 2 * L.chunk);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = plan->waves == 8 ? skinny_mt<F, 8>(a, L, sps, st) : skinny_mt<F, 4>(a, L, sps, st);
  if (e != hipSuccess) return hip_status(e, name);
  if (splits > 1) {
    if (mode == QLX_MODE_SWIGLU) return qlx_swiglu(nullptr, plan->workspace, splits, a.y, m, n / 2, stream);
    return qlx_reduce_planes(plan->workspace, a.y, (long long)m * n, splits, stream);
  }
  return QLX_OK;
}

}  // namespace qlx

using namespace qlx;

extern "C" {

int qlx_plan_skinny(int fmt, int mode, int m, int n, int k, qlx_plan* plan) {
  QLX_REQUIRE(plan != nullptr, "plan is NULL");
  QLX_REQUIRE(fmt == QLX_FMT_W4A16 || fmt == QLX_FMT_W8A16, "the skinny GEMM serves W4A16 and W8A16 (format %d)", fmt);
  const int kstep = fmt == QLX_FMT_W4A16 ? FmtW4::KSTEP : FmtW8::KSTEP;
  QLX_REQUIRE(m >= 1 && m <= 64 && n >= 16 && n % 16 == 0 && k >= kstep && k % kstep == 0,
              "shape m=%d n=%d k=%d does not fit format %d", m, n, k, fmt);
  qlx_plan p = {};
  p.mode = mode;
  p.kw = 1;
  p.rw = 1;
  if (fmt == QLX_FMT_W4A16)
    skinny_plan<FmtW4>(m, n, k, &p.waves, &p.splits);
  else
    skinny_plan<FmtW8>(m, n, k, &p.waves, &p.splits);
  const int nsteps = k / kstep;
  const int sps = (nsteps + p.splits - 1) / p.splits;
  p.splits = (nsteps + sps - 1) / sps;
  *plan = p;
  return QLX_OK;
}

int qlx_linear_skinny(int fmt, const void* w, const void* w_scale, const void* x, void* y, int m, int n, int k,
                      const qlx_plan* plan, void* stream) {
  GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x;
  a.y = y;
  QLX_REQUIRE(w && w_scale && x && y, "linear_skinny: NULL pointer");
  QLX_REQUIRE(plan != nullptr, "linear_skinny: plan is NULL");
  if (fmt == QLX_FMT_W4A16) return skinny_run<FmtW4>("linear_skinny", a, m, n, k, plan->mode, plan, stream);
  if (fmt == QLX_FMT_W8A16) return skinny_run<FmtW8>("linear_skinny", a, m, n, k, plan->mode, plan, stream);
  QLX_REQUIRE(false, "the skinny GEMM serves W4A16 and W8A16 (format %d)", fmt);
}

}  // extern "C"
