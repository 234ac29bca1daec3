// Skinny GEMM for 16..64 tokens (speculative verification, small batches).
//
// The decode kernel (gemm.h) stages a workgroup's whole K slice of the activation in LDS
// before its MFMA loop, and each wave keeps MT token fragments of every tile in registers.
// Past 16 tokens that costs too much: the staged slice outgrows LDS, so K is cut into many
// slices (each re-staging 64 tokens of x and writing fp32 partials), and at 64 tokens the
// registers spill. Here the activation streams through LDS one K step at a time instead:
//   * a workgroup owns WAVES x RW 16-row tiles (RW = 1 by default; 2, up to 32 tokens, lets
//     every activation fragment read from LDS feed two tiles' MFMAs) and one K slice; every
//     wave runs the same steps, so the waves share each staged activation chunk
//     [16 MT rows][KSTEP] and its scales, in two LDS buffers, one barrier per step;
//   * the activation and the weights of step i + PF are fetched together, PF steps ahead,
//     with every load unconditional, so the in-order memory counter waits only for what a
//     step needs; weights come in the MI355X tile layout and go through the format's MFMA
//     step with the decode kernel's arithmetic: per-group fp32 partials times the group
//     scale, the code bias removed by the same MFMA chain with every code at the bias (run
//     here on the fragments the step reads anyway);
//   * K slices write fp32 planes [slices][m][n] reduced in slice order, by the plane
//     consumers (qlx_reduce_planes, qlx_swiglu) or, with tickets, by the row group's last
//     workgroup: deterministic, like the reference's split-K planes
//     (engine/kernels/cuda_fp8.py:965-981).
// The reference serves these batches with the same kernels as decode, up to 64 rows in
// tiles of 8 tokens (engine/kernels/cuda_fp8.py:1227-1234, 1404-1423).
#include "gemm_launch.h"

namespace qlx {

// Weight steps in flight per wave, and activation chunks in flight per thread (the same
// depth: the activation of step i + PF is fetched with the weights of step i + PF).
__host__ __device__ constexpr int skinny_pf(int mt, bool wide) { return wide || mt == 1 ? 3 : 2; }
// 4-bit weights at 33..64 tokens run one workgroup per CU, each wave with the 512 registers of
// a whole SIMD: two activation sets of 64 rows, the MT = 4 accumulators and the code-bias
// chains spill at 256.
// 16-row tiles per wave, sharing each activation fragment read from LDS: two up to 32 tokens,
// one at 64 (two would need more than the 256 registers of two waves per SIMD).
__host__ __device__ constexpr int skinny_rw_max(int mt) { return mt >= 4 ? 1 : 2; }
// Token fragments (16 tokens each) a batch is computed with: 1, 2 or 4 (33..48 tokens run as 4).
__host__ __device__ constexpr int skinny_mt_of(int m) { return m <= 16 ? 1 : (m <= 32 ? 2 : 4); }

// LDS of one activation chunk: [16 MT rows][xstride bytes] of x in the format's B order (rows
// past m hold zeros and are never read), then the group scales [NSC][16 rows x
// the workgroup's tiles] as floats.
struct SkinnyLayout {
  int xstride, off_sc, sc_stride, chunk;
};

__host__ __device__ constexpr int up16(int v) { return (v + 15) & ~15; }

template <class F>
__host__ __device__ inline SkinnyLayout skinny_layout(int m, int waves, int rw) {
  SkinnyLayout L{};
  L.xstride = F::KSTEP * F::XBYTES + 16;  // rows 4 banks apart: a B read of 16 rows is conflict-free
  L.sc_stride = 16 * waves * rw;
  L.off_sc = up16(16 * skinny_mt_of(m) * L.xstride);
  L.chunk = up16(L.off_sc + (F::NSC > 0 ? F::NSC : 0) * L.sc_stride * 4);
  return L;
}

// LDS of a launch: the two chunk buffers, then (4-bit weights) the shared code-bias totals of
// two steps, [2][2 groups][MT][16 tokens] floats.
template <class F, int MT>
__host__ __device__ inline int skinny_lds(const SkinnyLayout& L) {
  return 2 * L.chunk + (std::is_same<F, FmtW4>::value ? 2 * 2 * MT * 16 * 4 : 0);
}

// x chunks (16 bytes, 8 values) of one K step that each thread stages: 16 MT rows.
template <class F, int WAVES, int MT>
struct SkinnyStage {
  static constexpr int PER_ROW = F::KSTEP * F::XBYTES / 16;
  static constexpr int CHUNKS = 16 * MT * PER_ROW;
  static constexpr int MAX = (CHUNKS + WAVES * 64 - 1) / (WAVES * 64);
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
  } else if constexpr (std::is_same<F, FmtFP8>::value) {
    // FP8 W8A8: e4m3 weights against the e4m3 codes of the activation (quantized per token
    // beforehand); both scales come in the epilogue. Chunk bytes 64 j + 16 c of a row hold the
    // codes of k 64 j + 16 c .., as the weight bytes of lane 16 c + r.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = j * 64 + (lane >> 4) * 16;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 bv = *reinterpret_cast<const uint4*>(ch + xoff[mt] + kb);
        const long b0 = (long)(((unsigned long)bv.y << 32) | bv.x), b1 = (long)(((unsigned long)bv.w << 32) | bv.z);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const long a0 = (long)(((unsigned long)c[r][j].y << 32) | c[r][j].x);
          const long a1 = (long)(((unsigned long)c[r][j].w << 32) | c[r][j].z);
          acc[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a0, b0, acc[r][mt], 0, 0, 0);
          acc[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a1, b1, acc[r][mt], 0, 0, 0);
        }
      }
    }
  } else {
    static_assert(std::is_same<F, FmtW8>::value, "skinny_step: W4A16, W8A16 or FP8 W8A8");
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

// W4A16 step with the code-bias chains shared: the chain of (group j, token fragment mt) depends
// on the staged activation only, the same for every tile of the workgroup, so wave
// (j MT + mt) % WAVES alone runs it and leaves its totals in bt_cur[j][mt][16 tokens]; the others
// read them after the step's barrier. So each wave keeps its step's partials (pend) and group
// scales (ps: the chunk buffer they came from is restaged during the next step) and adds them
// one step later: skinny_apply_w4(step i - 1) then skinny_step_w4s(step i). The sums, their
// roundings and their order are skinny_step's, so the output is the same bits.
template <int MT, int RW>
__device__ __forceinline__ void skinny_apply_w4(f32x4 (&acc)[RW][MT], const f32x4 (&pend)[2][RW][MT],
                                                const f32x4 (&ps)[2][RW], const float* bt, int lane) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float tb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) tb[mt] = bt[(j * MT + mt) * 16 + (lane & 15)];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const f32x4 s4 = ps[j][r];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][mt][i] = fmaf(s4[i], pend[j][r][mt][i] - tb[mt], acc[r][mt][i]);
    }
  }
}

template <int MT, int RW, int WAVES>
__device__ __forceinline__ void skinny_step_w4s(f32x4 (&pend)[2][RW][MT], f32x4 (&ps)[2][RW], const uint4 (&c)[RW][2],
                                                const char* ch, const SkinnyLayout& L, float* bt_cur, int lane, int wave,
                                                const int (&xoff)[MT], const int (&rowl)[RW]) {
  const uint4 ab = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136 = the code bias
  const float* sc = reinterpret_cast<const float*>(ch + L.off_sc);
  // The chains this wave runs: q = wave, wave + WAVES, .. below 2 MT, or wave % 2 MT once
  // when the waves outnumber the chains (duplicates write the same bits). No branch: each chain
  // reads its own fragments at a computed address.
  constexpr int NCH = 2 * MT, PER = NCH > WAVES ? NCH / WAVES : 1;
  static_assert(NCH <= WAVES || NCH % WAVES == 0, "chains spread evenly over the waves");
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int q = NCH > WAVES ? wave + u * WAVES : wave % NCH;
    const int jq = q / MT, mq = q - jq * MT;
    int xq = xoff[0];
#pragma unroll
    for (int mt = 1; mt < MT; ++mt) xq = mq == mt ? xoff[mt] : xq;
    const char* bq = ch + xq + (jq * 128 + (lane >> 4) * 32) * 2;
    f32x4 tb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ab), as_bf16x8(*reinterpret_cast<const uint4*>(bq + t * 16)),
                                                   tb, 0, 0, 0);
    if (lane < 16) bt_cur[q * 16 + lane] = tb[0];  // every row of the chain's result is the same
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int r = 0; r < RW; ++r) ps[j][r] = *reinterpret_cast<const f32x4*>(sc + j * L.sc_stride + rowl[r]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < RW; ++r) pend[j][r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
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
          pend[j][r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[r]), as_bf16x8(bv), pend[j][r][mt], 0, 0, 0);
      }
    }
  }
}

// Buffer resource over `bytes` of device memory (base address uniform across the workgroup).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t skinny_rsrc(const void* p, unsigned bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, (int)bytes,
                                           0x00020000);
}

// Buffer access policy sc1: device scope (past this XCD's L2, which other XCDs' stores do not update).
constexpr int kSc1 = 16;

// fn(integral_constant<int, P>) for P = B .. E - 1, unrolled at compile time.
template <int B, int E, class Fn>
__device__ __forceinline__ void static_for(Fn&& fn) {
  if constexpr (B < E) {
    fn(std::integral_constant<int, B>{});
    static_for<B + 1, E>(fn);
  }
}

// Two workgroups per CU (each wave at most 256 registers), or one for the wide instances.
template <class F, int MT, int RW, int WAVES, bool SW>
__global__ void __launch_bounds__(WAVES * 64)
__attribute__((amdgpu_waves_per_eu(WAVES == 4 && !(MT == 4 && F::NSC > 0) ? 2 : 1)))
skinny_kernel(GemmArgs a0, SkinnyLayout L, int steps_per_slice) {
  static_assert(F::LOADS == 2, "a tile step is two 1 KB loads per wave");
  static_assert(F::NSC == 0 || std::is_same<F, FmtW4>::value, "group scales as W4A16 lays them out");
  extern __shared__ __align__(16) char lds[];
  static_assert(RW >= 1 && RW <= skinny_rw_max(MT), "tiles per wave");
  constexpr int PF = skinny_pf(MT, WAVES == 4 && MT == 4 && F::NSC > 0);
  constexpr int SPR = SkinnyStage<F, WAVES, MT>::PER_ROW, SMAX = SkinnyStage<F, WAVES, MT>::MAX;
  constexpr int CHUNKS = SkinnyStage<F, WAVES, MT>::CHUNKS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  GemmArgs a = a0;
  int bid = blockIdx.x;
  int b = 0;      // token block
  int prow = a.m;  // rows of one fp32 plane
  if (a.tblocks == 2) {  // token blocks: block ids 16 q + 8 b + x are row group 8 q + x, tokens 32 b..
    // (ids 8 apart share an XCD, so the second block finds the weights in that XCD's L2)
    b = (bid >> 3) & 1;
    prow = a.pm;
    bid = 8 * (bid >> 4) + (bid & 7);
    a.x = static_cast<const char*>(a.x) + (size_t)b * 32 * a.k * F::XBYTES;
    if (a.xs) a.xs += b * 32;
    a.y = static_cast<char*>(a.y) + (size_t)b * 32 * (SW ? a.half : a.n) * 2;
    a.work += (size_t)b * 32 * a.n;  // K-slice planes keep the whole batch's rows (a.pm)
    a.m = min(32, a.m - 32 * b);
  }
  const int tg = bid / a.splits, s = bid - tg * a.splits;
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

  // Every load below is issued unconditionally (indices clamped to real rows, tiles and steps),
  // so the compiler counts the in-order memory queue exactly: a wait for step i's data never
  // waits for loads issued after it. (Loads under branches made it drain the whole queue,
  // vmcnt(0), several times per step.) A tile past the end streams tile 0 of the workgroup
  // (always real); its results are dropped.
  int lrow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) lrow[r] = act[r] ? wrow[r] : weight_row(a, tg * WAVES * RW, lane & 15);

  // A step's staged data: SMAX 16-byte activation chunks and (group formats) SCMAX raw bf16
  // scales per thread, fetched into registers ahead of time and written to LDS later.
  constexpr int SCMAX = F::NSC > 0 ? (F::NSC * 16 * WAVES * RW + WAVES * 64 - 1) / (WAVES * 64) : 1;
  struct Staged {
    uint4 x[SMAX];
    uint16_t sc[SCMAX];  // widened only when written to LDS: no copy of an in-flight load
  };
  // The activation through a buffer resource over its m rows: a thread's chunks u = 0, 1, ..
  // are rows row0 + u XROWS of one column, so one 32-bit offset serves every chunk (the row
  // step is a scalar offset), and rows past m read as zeros (the resource's bounds check).
  constexpr int XROWS = WAVES * 64 / SPR;
  static_assert(WAVES * 64 % SPR == 0, "a thread's chunks share their column");
  // (FP8: the e4m3 codes, one byte per value.)
  constexpr unsigned XB = F::XBYTES;
  const __amdgpu_buffer_rsrc_t xr = skinny_rsrc(a.x, (unsigned)a.m * (unsigned)a.k * XB);
  const int xrow0 = threadIdx.x / SPR, xcol = threadIdx.x - xrow0 * SPR;
  const unsigned xoff0 = (unsigned)xrow0 * (unsigned)a.k * XB + (unsigned)xcol * 16u;
  auto fetch_x = [&](int step, Staged& st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(xoff0 + (unsigned)step * (F::KSTEP * XB)),
                                                            u * XROWS * a.k * (int)XB, 0);
      st.x[u] = uint4{v[0], v[1], v[2], v[3]};
    }
    if constexpr (F::NSC > 0) {
#pragma unroll
      for (int u = 0; u < SCMAX; ++u) {
        const int q = min((int)threadIdx.x + u * WAVES * 64, F::NSC * L.sc_stride - 1);
        const int j = q / L.sc_stride, rl = q - j * L.sc_stride;
        const int t = min(tg * WAVES * RW + (rl >> 4), a.ntiles - 1);  // a tile past the end: dropped
        // group 2 step + j of the tile row's weight row, as F::scale reads it
        st.sc[u] = gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)weight_row(a, t, rl & 15) * (a.k >> 7) +
                                                                  F::NSC * step + j];
      }
    }
  };
  auto put_x = [&](char* ch, const Staged& st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < SMAX; ++u) {
      const int mm = xrow0 + u * XROWS;  // rows past m hold zeros and are never read
      if (CHUNKS % (WAVES * 64) == 0 || mm < 16 * MT) {
        if constexpr (std::is_same<F, FmtFP8>::value)
          *reinterpret_cast<uint4*>(ch + mm * L.xstride + xcol * 16) = st.x[u];  // codes in k order
        else
          *reinterpret_cast<uint4*>(ch + mm * L.xstride + xcol * 16) = F::order(st.x[u]);
      }
    }
    if constexpr (F::NSC > 0) {
      float* sc = reinterpret_cast<float*>(ch + L.off_sc);
#pragma unroll
      for (int u = 0; u < SCMAX; ++u) {
        const int q = min((int)threadIdx.x + u * WAVES * 64, F::NSC * L.sc_stride - 1);
        sc[q] = bf2f((uint32_t)st.sc[u]);  // [j][row]: q = j sc_stride + row
      }
    }
  };

  // Pipeline: register sets rr[p] hold the activation of the steps = p (mod PF), buf[p] their
  // weights; both are fetched PF steps ahead, the activation of a step just before its weights.
  // Step i: its MFMAs read chunk buffer i & 1 and buf[i % PF]; then the activation and weights
  // of step i + PF refill rr/buf[i % PF]; then the activation of step i + 1 (fetched before the
  // weights of step i + 1, so waiting for it waits for nothing the MFMAs did not) goes to the
  // other chunk buffer, whose step i - 1 every wave finished before the last barrier; one
  // barrier per step publishes it. Steps past the slice are clamped to its last (cache hits).
  uint4 buf[PF][RW][F::LOADS];
  Staged rr[PF];
  // Weights through a buffer resource (WBUF): a tile's K steps are consecutive 2 KB blocks, so a
  // lane's chunk of step s sits s * 2048 bytes past its step-0 offset (woff, fixed for the
  // launch: a wave keeps its tiles) and the step is the scalar offset -- no per-lane address
  // arithmetic per refill. Measured per call over 24 distinct Qwen3-4B weights (us, per-lane
  // addresses / buffer): W4A16 at 16 tokens gate_up 11.8 / 11.4, down 9.4 / 9.1; at 32 tokens
  // gate_up (8 waves) 15.3 / 14.9; W8A16 at 16 tokens gate_up 16.6 / 15.2, down 11.4 / 11.2. The
  // other instances measured as fast or slower with it (the 4-wave 33-64 token launches: W4A16
  // down 15.7 / 15.9, W8A16 gate_up 28.4 / 30.1; FP8 at 32-64 tokens up to 0.7 us slower).
  constexpr bool WBUF = (std::is_same<F, FmtW4>::value && (MT == 1 || WAVES == 8)) ||
                        (std::is_same<F, FmtW8>::value && MT == 1);
  const __amdgpu_buffer_rsrc_t wrs = skinny_rsrc(a.w, WBUF ? (unsigned)a.ntiles * (unsigned)a.nsteps * 2048u : 0u);
  uint32_t woff[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r)
    woff[r] = WBUF ? (uint32_t)(reinterpret_cast<const char*>(F::chunk_ptr(a, lrow[r], 0, lane, 0)) -
                                static_cast<const char*>(a.w))
                   : 0u;
  auto wload = [&](uint4 (&c)[F::LOADS], int r, int step) __attribute__((always_inline)) {
    if constexpr (WBUF) {
#pragma unroll
      for (int j = 0; j < F::LOADS; ++j) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wrs, (int)(woff[r] + (uint32_t)j * 1024u), step * 2048, 2);
        c[j] = uint4{v[0], v[1], v[2], v[3]};
      }
    } else {
      load_chunk<F>(c, a, lrow[r], step, lane);
    }
  };
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    fetch_x(min(step0 + p, last), rr[p]);
#pragma unroll
    for (int r = 0; r < RW; ++r) wload(buf[p][r], r, min(step0 + p, last));
  }
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

  // The SwiGLU instance of 4-bit weights at two token fragments on 4 waves (gate_up's 33-64
  // token launches, two 32-token blocks) shares the code-bias chains (skinny_step_w4s):
  // [step parity][2][MT][16] totals behind the two chunk buffers, a step's partials added after
  // the next barrier. Measured per call over 36 distinct Qwen3-4B weights (us, own chains /
  // shared): gate_up at 48 and 64 tokens 24.5 / 21.1 and 24.4 / 21.4; every other instance as
  // fast or slower shared -- gate_up at 16 and 32 tokens (8 waves) 11.8 / 12.7 and 15.2 / 15.6,
  // down at 16 / 32 / 64 tokens 9.4 / 10.0, 12.7 / 12.8, 15.8 / 15.8.
  constexpr bool SB = std::is_same<F, FmtW4>::value && MT == 2 && WAVES == 4 && SW;
  float* const btb = reinterpret_cast<float*>(lds + 2 * L.chunk);
  f32x4 pend[2][RW][MT], ps[2][RW];
  // Every lambda is inlined: an outlined one would take the register arrays by address (scratch).
  auto body = [&](int i, auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value;
    if constexpr (SB) {
      if (i > 0) skinny_apply_w4<MT, RW>(acc, pend, ps, btb + ((i - 1) & 1) * (2 * MT * 16), lane);
      skinny_step_w4s<MT, RW, WAVES>(pend, ps, buf[p], lds + (i & 1) * L.chunk, L, btb + (i & 1) * (2 * MT * 16),
                                     lane, wave, xoff, rowl);
    } else {
      skinny_step<F, MT, RW>(acc, buf[p], lds + (i & 1) * L.chunk, L, lane, xoff, rowl);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int nx = min(step0 + i + PF, last);
    fetch_x(nx, rr[p]);
#pragma unroll
    for (int r = 0; r < RW; ++r) wload(buf[p][r], r, nx);
    __builtin_amdgcn_sched_barrier(0);
    put_x(lds + ((i + 1) & 1) * L.chunk, rr[(p + 1) % PF]);
    __syncthreads();
  };
  int i0 = 0;
  for (; i0 + PF <= nst; i0 += PF) static_for<0, PF>([&](auto pc) __attribute__((always_inline)) { body(i0 + decltype(pc)::value, pc); });
  static_for<0, PF>([&](auto pc) __attribute__((always_inline)) {  // the last nst % PF steps (uniform branches)
    if (i0 + decltype(pc)::value < nst) body(i0 + decltype(pc)::value, pc);
  });
  if constexpr (SB)  // the last step's partials: its totals were published by the last barrier
    skinny_apply_w4<MT, RW>(acc, pend, ps, btb + ((nst - 1) & 1) * (2 * MT * 16), lane);

  // Epilogue: lane holds rows 4 (lane >> 4) + 0..3 of each tile for token 16 mt + (lane & 15).
  // K-slice planes shared through tickets go through a buffer resource at device scope.
  // (over this block's rows of every plane: planes are prow rows apart)
  const __amdgpu_buffer_rsrc_t wr = skinny_rsrc(
      a.work, a.tickets != nullptr ? ((unsigned)(a.splits - 1) * (unsigned)prow + (unsigned)a.m) * (unsigned)a.n * 4u : 0u);
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
        if constexpr (std::is_same<F, FmtFP8>::value) v[i] *= a.xs[min(mm, a.m - 1)];  // the token's scale
      }
      if (a.splits > 1) {  // fp32 plane s, rows in natural order
        if (mm < a.m) {
          float* plane = a.work + ((size_t)s * prow + mm) * a.n;
          if (a.tickets != nullptr) {  // read by the row group's last workgroup below
            // rows r0 .. r0 + 3 of a tile are consecutive weight rows: one 16-byte store
            const unsigned off = (unsigned)(((size_t)s * prow + mm) * a.n + weight_row(a, tile[r], r0)) * 4u;
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
                wr, (int)off, 0, kSc1);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) plane[weight_row(a, tile[r], r0 + i)] = v[i];
          }
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
  if (a.splits == 1 || a.tickets == nullptr) return;

  // K slices with tickets: the row group's last workgroup to finish sums the planes in slice
  // order, as qlx_reduce_planes / qlx_swiglu would in a second launch (the same sums, so the
  // same bits). The partials went out with device-coherent stores; every wave waits for its
  // stores before the ticket is taken (a workgroup-scope release does not wait for them).
  __shared__ int s_last;
  publish_stores();
  if (threadIdx.x == 0) {
    int* ticket = &a.tickets[a.tblocks == 2 ? 2 * tg + b : tg];  // per (row group, token block)
    const int prev = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == a.splits - 1;
    if (s_last) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  // Thread items: 4 consecutive output rows of one token (SwiGLU: 4 gate rows and their up
  // rows), each plane's chunk one 16-byte device-scope load, 4 planes in flight at a time.
  constexpr int RT = WAVES * RW, QUADS = SW ? 2 : 4;  // 4-row chunks per tile
  const int per_tok = RT * QUADS;
  const unsigned pstride = (unsigned)prow * (unsigned)a.n * 4u;
  auto f4 = [](const u32x4& u) { return f32x4{__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]),
                                              __uint_as_float(u[3])}; };
  for (int idx = threadIdx.x; idx < per_tok * a.m; idx += WAVES * 64) {
    const int mm = idx / per_tok, c = idx - mm * per_tok;
    const int t = tg * RT + c / QUADS, q4 = 4 * (c - (c / QUADS) * QUADS);
    if (t >= a.ntiles) continue;
    const int row = SW ? 8 * t + q4 : 16 * t + q4;  // first of the 4 rows (SwiGLU: gate rows)
    const unsigned off = (unsigned)((size_t)mm * a.n + row) * 4u;
    f32x4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = 0; sp0 < a.splits; sp0 += 4) {
      u32x4 lg[4], lu[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int sp = min(sp0 + j, a.splits - 1);
        lg[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)(off + sp * pstride), 0, kSc1);
        if constexpr (SW) lu[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)(off + sp * pstride + a.half * 4), 0, kSc1);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (sp0 + j < a.splits) {  // slice order
          const f32x4 vg = f4(lg[j]);
#pragma unroll
          for (int i = 0; i < 4; ++i) g[i] += vg[i];
          if constexpr (SW) {
            const f32x4 vu = f4(lu[j]);
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] += vu[i];
          }
        }
      }
    }
    if constexpr (SW) {
      store_pair(y, (size_t)mm * a.half + row, swiglu_bf(g[0], u[0]), swiglu_bf(g[1], u[1]));
      store_pair(y, (size_t)mm * a.half + row + 2, swiglu_bf(g[2], u[2]), swiglu_bf(g[3], u[3]));
    } else {
      store_pair(y, (size_t)mm * a.n + row, g[0], g[1]);
      store_pair(y, (size_t)mm * a.n + row + 2, g[2], g[3]);
    }
  }
}

template <class F, int MT, int RW, int WAVES>
hipError_t skinny_launch(const GemmArgs& a, const SkinnyLayout& L, int sps, hipStream_t st) {
  const int lds = skinny_lds<F, MT>(L);
  const dim3 grid(a.tile_groups * a.splits * (a.tblocks == 2 ? 2 : 1)), block(WAVES * 64);
  const void* fn = a.mode == QLX_MODE_SWIGLU ? reinterpret_cast<const void*>(&skinny_kernel<F, MT, RW, WAVES, true>)
                                              : reinterpret_cast<const void*>(&skinny_kernel<F, MT, RW, WAVES, false>);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
  }
  if (a.mode == QLX_MODE_SWIGLU)
    skinny_kernel<F, MT, RW, WAVES, true><<<grid, block, lds, st>>>(a, L, sps);
  else
    skinny_kernel<F, MT, RW, WAVES, false><<<grid, block, lds, st>>>(a, L, sps);
  return hipGetLastError();
}

template <class F, int WAVES>
hipError_t skinny_mt(const GemmArgs& a, const SkinnyLayout& L, int sps, hipStream_t st) {
  const int mt = skinny_mt_of(a.m), rw = a.rt / WAVES;
  if (mt == 1) return rw == 2 ? skinny_launch<F, 1, 2, WAVES>(a, L, sps, st) : skinny_launch<F, 1, 1, WAVES>(a, L, sps, st);
  if (mt == 2) return rw == 2 ? skinny_launch<F, 2, 2, WAVES>(a, L, sps, st) : skinny_launch<F, 2, 1, WAVES>(a, L, sps, st);
  return skinny_launch<F, 4, 1, WAVES>(a, L, sps, st);
}

// Waves, tiles per wave and K slices: 4 waves per workgroup, one tile per wave (two, which reuse
// each activation fragment read from LDS twice, measured no faster on any config-4 shape: gate_up
// 12.6 vs 12.7 us at 16 tokens, 17.4 vs 16.6 at 32; down 13.1 vs 11.0 at 16), and K slices until
// about 240 workgroups (down: 40 row groups x 6 slices), each slice at least 2 steps. A shape with
// row groups for at least 256 whole-K workgroups (gate_up: 1216 tiles) at up to 32 tokens runs 8
// waves per workgroup instead, one per CU: every staged activation chunk then serves 8 tiles, half
// the activation reads from L2 (gate_up 12.7 -> 11.7 us at 16 tokens, 17.1 -> 15.7 at 32; taking
// a tile's steps two waves at a time, which doubles them, measured 13.6 and 21.6). Measured on the
// Qwen3 config-4 shapes over every slice count, waves per workgroup and tiles per wave.
template <class F>
void skinny_plan(int m, int n, int k, int* waves, int* rw, int* splits) {
  const int nsteps = k / F::KSTEP;
  const int ntiles = n / 16;  // SwiGLU tiles hold 8 gate + 8 up rows: also n / 16
  *waves = 4;
  *rw = 1;
  const int rt = 4 * *rw;
  const int groups = (ntiles + rt - 1) / rt;
  int s = 240 / groups;
  const int most = nsteps / 2 > 1 ? nsteps / 2 : 1;
  if (s > most) s = most;
  if (s < 1) s = 1;
  *splits = s;
  if (s == 1 && m <= 32 && groups >= 256) *waves = 8;
}

template <class F>
int skinny_run(const char* name, GemmArgs a, int m, int n, int k, int mode, const qlx_plan* plan, void* stream) {
  QLX_REQUIRE(plan != nullptr, "%s: plan is NULL", name);
  QLX_REQUIRE(m >= 1 && m <= 64, "%s: m=%d must be in 1..64", name, m);
  QLX_REQUIRE(n >= 16 && n % 16 == 0 && k >= F::KSTEP && k % F::KSTEP == 0,
              "%s: n=%d k=%d do not fit the tiled format", name, n, k);
  QLX_REQUIRE((long long)(n / 16) * (k / F::KSTEP) * 2048 < (1ll << 31),
              "%s: the skinny GEMM reads weights of under 2 GiB (n=%d k=%d)", name, n, k);
  QLX_REQUIRE(mode == QLX_MODE_BF16 || mode == QLX_MODE_SWIGLU, "%s: mode %d", name, mode);
  QLX_REQUIRE(plan->waves == 4 || plan->waves == 8, "%s: waves must be 4 or 8", name);
  QLX_REQUIRE(plan->rw >= 1 && plan->rw <= skinny_rw_max(skinny_mt_of(m)),
              "%s: rw=%d tiles per wave (1, or 2 up to 32 tokens)", name, plan->rw);
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
  a.rt = plan->waves * plan->rw;
  a.ntiles = n / 16;
  a.tile_groups = (a.ntiles + a.rt - 1) / a.rt;
  a.half = n / 2;
  a.tiled = 1;
  a.work = plan->workspace;
  a.tickets = splits > 1 ? plan->tickets : nullptr;
  QLX_REQUIRE(a.tickets == nullptr || (long long)splits * m * n * 4 < (1ll << 31),
              "%s: %d planes of %d x %d floats exceed the 2 GiB a shared reduction addresses", name, splits, m, n);
  hipStream_t st = (hipStream_t)stream;
  const int wgs = a.tile_groups * splits;
  if (skinny_mt_of(m) == 4 && F::NSC > 0 && plan->waves == 4 && splits > 1 && wgs % 8 == 0 && 2 * wgs <= 512) {
    // K-sliced batches of 33..64 tokens whose two 32-token blocks still fit the two-per-CU
    // instance in one round (down: 40 row groups x 6 slices = 240 per block): one launch, a
    // (row group, slice)'s two blocks on one XCD; each block writes its rows of the planes, and
    // with tickets the last workgroup of each (row group, block) reduces them (2 counters per
    // row group).
    a.tblocks = 2;
    a.pm = m;
    const hipError_t e = skinny_launch<F, 2, 1, 4>(a, skinny_layout<F>(32, 4, plan->rw), sps, st);
    if (e != hipSuccess) return hip_status(e, name);
    if (a.tickets != nullptr) return QLX_OK;
    if (mode == QLX_MODE_SWIGLU) return qlx_swiglu(nullptr, plan->workspace, splits, a.y, m, n / 2, stream);
    return qlx_reduce_planes(plan->workspace, a.y, (long long)m * n, splits, stream);
  }
  if (skinny_mt_of(m) == 4 && F::NSC > 0 && plan->waves == 4 && splits == 1 && a.tile_groups > 256) {
    // Token blocks: 33..64 tokens over more whole-K row groups than CUs (gate_up: 304) run as
    // two blocks of at most 32 tokens on the two-workgroups-per-CU instance; the one-per-CU
    // 64-token instance would run 48 CUs' second workgroup after the first round. With row
    // groups a multiple of 8, both blocks go in one launch, a row group's two blocks on one XCD
    // (its L2 serves the second weight read); else two launches, the second block's weights
    // mostly from the Infinity Cache. Each token's sums are the same: bit-identical output.
    const SkinnyLayout Lb = skinny_layout<F>(32, 4, plan->rw);
    if (a.tile_groups % 8 == 0) {
      a.tblocks = 2;
      const hipError_t e = skinny_launch<F, 2, 1, 4>(a, Lb, sps, st);
      return e == hipSuccess ? QLX_OK : hip_status(e, name);
    }
    const size_t ybytes = (size_t)(mode == QLX_MODE_SWIGLU ? n / 2 : n) * 2;
    for (int m0 = 0; m0 < m; m0 += 32) {
      GemmArgs b = a;
      b.m = min(32, m - m0);
      b.x = static_cast<const char*>(a.x) + (size_t)m0 * k * 2;
      b.y = static_cast<char*>(a.y) + (size_t)m0 * ybytes;
      const hipError_t e = skinny_mt<F, 4>(b, skinny_layout<F>(b.m, 4, plan->rw), sps, st);
      if (e != hipSuccess) return hip_status(e, name);
    }
    return QLX_OK;
  }
  const SkinnyLayout L = skinny_layout<F>(m, plan->waves, plan->rw);
  const int lds_bytes = skinny_lds<F, 4>(L);  // the widest token count's totals
  QLX_REQUIRE(lds_bytes <= kLdsLimit, "%s: %d bytes of LDS", name, lds_bytes);
  hipError_t e = plan->waves == 8 ? skinny_mt<F, 8>(a, L, sps, st) : skinny_mt<F, 4>(a, L, sps, st);
  if (e != hipSuccess) return hip_status(e, name);
  if (splits > 1 && a.tickets == nullptr) {  // without tickets: the planes reduced in a second launch
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
  QLX_REQUIRE(fmt == QLX_FMT_W4A16 || fmt == QLX_FMT_W8A16 || fmt == QLX_FMT_FP8,
              "the skinny GEMM serves W4A16, W8A16 and FP8 W8A8 (format %d)", fmt);
  const int kstep = fmt == QLX_FMT_W4A16 ? FmtW4::KSTEP : (fmt == QLX_FMT_W8A16 ? FmtW8::KSTEP : FmtFP8::KSTEP);
  QLX_REQUIRE(m >= 1 && m <= 64 && n >= 16 && n % 16 == 0 && k >= kstep && k % kstep == 0,
              "shape m=%d n=%d k=%d does not fit format %d", m, n, k, fmt);
  qlx_plan p = {};
  p.mode = mode;
  p.kw = 1;
  if (fmt == QLX_FMT_W4A16)
    skinny_plan<FmtW4>(m, n, k, &p.waves, &p.rw, &p.splits);
  else if (fmt == QLX_FMT_W8A16)
    skinny_plan<FmtW8>(m, n, k, &p.waves, &p.rw, &p.splits);
  else
    skinny_plan<FmtFP8>(m, n, k, &p.waves, &p.rw, &p.splits);
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
  QLX_REQUIRE(false, "qlx_linear_skinny serves W4A16 and W8A16 (format %d; FP8: qlx_linear_skinny_fp8)", fmt);
}

int qlx_linear_skinny_fp8(const void* w, const void* w_scale, const void* x_code, const float* x_scale, void* y,
                          int m, int n, int k, const qlx_plan* plan, void* stream) {
  GemmArgs a = {};
  a.w = w;
  a.ws = w_scale;
  a.x = x_code;
  a.xs = x_scale;
  a.y = y;
  QLX_REQUIRE(w && w_scale && x_code && x_scale && y, "linear_skinny_fp8: NULL pointer");
  QLX_REQUIRE(plan != nullptr, "linear_skinny_fp8: plan is NULL");
  return skinny_run<FmtFP8>("linear_skinny_fp8", a, m, n, k, plan->mode, plan, stream);
}

}  // extern "C"
