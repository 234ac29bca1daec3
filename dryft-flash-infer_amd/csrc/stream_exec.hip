// Stream executor: every quantized projection of a decode step in one launch, with the weight
// stream taken off the dependency chain.
//
// The reference runs each projection as its own launch in a captured graph and overlaps a
// GEMM's weight loads with the previous kernel through programmatic dependent launch
// (engine/kernels/cuda_fp8.py:47-50, 150-169; engine/kernels/cuda_jit.py:218-262). The first
// executor here (decode_stack.hip) does it in one cooperative launch, but its waves both
// stream weights into registers and poll for the activations earlier projections publish, and
// a wave's memory operations complete in issue order: a poll waits behind every weight load
// the wave has in flight. This executor splits the two jobs between two kinds of wave in each
// workgroup (one per CU):
//
//   * kSxCompute compute waves stream weights with direct-to-LDS loads (global_load_lds, 1 KB
//     per instruction) into a private LDS ring each, and run the MFMAs from the ring and the
//     staged activation. They issue no other memory operation, so their loads complete in
//     order and `s_waitcnt vmcnt(n)` says exactly which ring line has landed. A ring line is
//     refilled as soon as it is consumed, so the stream runs as far ahead as the ring allows
//     -- across projections, while inputs are still being produced. (Measured on MI355X: four
//     such waves per CU stream 6.9 TB/s; one wave draws at most ~9 GB/s, so fewer waves cannot.)
//   * kSxIo IO waves poll the published activation of the next projection this workgroup has
//     work in, copy it into LDS as bf16 (FP8: with the per-token maxima), signal the compute
//     waves through an LDS word each, then reduce each tile's partial sums from the compute
//     waves, apply the epilogue and publish the outputs. The per-step work on the staged
//     activation (FP8 codes, W8A16/W4A16 bias sums) is done by the compute wave that owns the
//     step, for itself: the link from one projection to the next is a poll and a copy.
//
// Work: each projection's 16-row tiles are dealt to workgroups whole (all of K), in
// contiguous ranges chosen so that every workgroup's running total of weight bytes stays
// balanced over the chain; within a workgroup the compute waves split each tile's K steps
// (step s to wave s % kSxCompute) and the tile's output is their sum in wave order, so results
// do not depend on timing. Dependencies between workgroups are the published words of the
// first executor (exec_common.h): no grid barrier, no counter.
#include <algorithm>
#include <numeric>
#include <vector>

#include "exec_common.h"

namespace qlx {

constexpr int kSxCompute = 8;  // compute waves per workgroup
constexpr int kSxIo = 4;       // IO waves per workgroup
constexpr int kSxSlots = 8;    // tiles whose partial sums may be in flight between the two
constexpr int kSxMaxTilesPerEntry = 48;         // per-row scales staged per work entry
constexpr int kSxNormU = 3;    // chunks per IO thread of a residual + RMSNorm stage (one pass)
constexpr int kSxNormMaxM = 2;  // tokens of such a stage: m * k / 8 <= kSxNormU * 256

// One projection, as the IO waves read it (global memory).
struct alignas(16) SxProj {
  const void* w;          // codes in the MI355X tile layout
  const void* ws;         // scales: bf16 [n] (per channel) or [n][k/128] (W4A16)
  const void* x;          // input in memory (bf16 [m][k]), or null
  const uint64_t* xwire;  // input published by an earlier projection, or null
  void* y;                // output, bf16 [m][n_out]
  uint64_t* ywire;        // published copy of the output for later projections, or null
  int n, k, nsteps, ntiles;
  int sw;                 // SwiGLU epilogue (tile = 8 gate + 8 up rows)
  int xpitch;             // values per token row of xwire
  int half;               // n / 2
  int norm;               // input stage: residual add + RMSNorm (xwire, if any, is the delta)
  // Residual add + RMSNorm input stage (norm != 0): r = bf16(resid + delta), input =
  // bf16(bf16(r * rsqrt(mean(r^2) + eps)) * nw).
  const void* nw;         // RMSNorm weight, bf16 [k]
  const void* rmem;       // residual in memory (bf16 [m][k]), or null
  const uint64_t* rwire;  // residual published by an earlier projection's stage, or null
  void* rout;             // r to memory (by the workgroup holding tile 0), or null
  uint64_t* rwire_out;    // r published for later stages, or null
  void* nout;             // the normed input to memory (tile 0's workgroup), or null
  float eps;
  int pad2;
};

// What the compute waves need of a projection (copied to LDS once per launch).
struct alignas(16) SxComp {
  const void* w;
  const void* ws;
  int nsteps, kgroups, sw, half;  // sw: tile = gate rows 8t.. and up rows half + 8t..
};

// A workgroup's share of one projection: tiles [tile0, tile0 + ntile).
struct alignas(16) SxWork {
  int proj, tile0, ntile, pad;
};

// Descriptor image (one allocation): header, SxProj[ncalls], SxComp[ncalls], int work_start[nwg + 1],
// SxWork[...]. Offsets are relative to the image, so the host image is copied as is.
struct alignas(16) SxHeader {
  int ncalls, nwg, proj_off, comp_off, start_off, work_off, max_work, pad;
};

// LDS layout of a launch (bytes), the same for every workgroup.
struct SxLayout {
  int ring_off, ring_lines;
  int part_stride;   // bytes of one wave's partial sums of one tile (16 rows x m floats)
  int stage_off[2], stage_bytes;
  int part_off;      // kSxSlots x kSxCompute x 1 KB of partial sums
  int ctl_off;       // control words
  int comp_off;      // SxComp[ncalls]
  int work_off;      // this workgroup's SxWork entries
  int sws_off;       // per-row scales of work entries e & 1 (floats, 2 x kSxMaxTilesPerEntry x 16)
  int m;
};

// Control words (uint32 each, at ctl_off).
enum SxCtl {
  kCtlStaged = 0,  // [2][kSxIo]: IO wave i's part of staging buffer b holds work entry k: word = k + 1
  kCtlIoBar = 2 * kSxIo,  // IO-team barrier counter (residual + RMSNorm stages)
  kCtlPart = 2 * kSxIo + 4,  // [kSxSlots][kSxCompute]: generation of the partial sums compute wave c left in the slot
  kCtlFree = kCtlPart + kSxSlots * kSxCompute,  // [kSxSlots]: generations of the slot consumed by the IO waves
  kCtlAmax = kCtlFree + kSxSlots,  // [3][16]: FP8 per-token maxima of entries e % 3 (zeroed between uses)
  kCtlWords = kCtlAmax + 48,
};

// LDS views of generic pointers into the dynamic LDS array: accesses through them compile to
// ds_* instructions (a generic access would be a flat one, which also counts as a vector
// memory operation).
typedef __attribute__((address_space(3))) uint32_t lds_u32;
__device__ __forceinline__ lds_u32* as_lds(uint32_t* p) { return (lds_u32*)p; }
__device__ __forceinline__ const lds_u32* as_lds(const uint32_t* p) { return (const lds_u32*)p; }

__device__ __forceinline__ uint32_t lds_load(const uint32_t* p) {
  return __hip_atomic_load(as_lds(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(uint32_t* p, uint32_t v) {
  __hip_atomic_store(as_lds(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Spin on an LDS word until it reaches `want` (or the run's deadline passes).
__device__ __forceinline__ void lds_wait_ge(const uint32_t* p, uint32_t want, const Waits& w, WaitSite site) {
  while (lds_load(p) < want) {
    if (ll_expired(w, site)) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// Plain (volatile) LDS word access for the compute waves. An atomic LDS access makes the
// compiler wait for every outstanding memory operation first (vmcnt(0): the whole weight ring);
// a wave's LDS operations are performed in issue order, so a flag written after data is seen
// after it by a wave that reads the flag, then the data.
__device__ __forceinline__ uint32_t lds_vload(const uint32_t* p) { return *(const volatile lds_u32*)as_lds(p); }
__device__ __forceinline__ void lds_vstore(uint32_t* p, uint32_t v) { *(volatile lds_u32*)as_lds(p) = v; }

// The wait of the compute waves, which give up silently at the deadline: flagging the error
// takes a global atomic, and any global operation besides the ring loads would make their
// memory operations complete out of order (the IO waves' waits flag it instead).
__device__ __forceinline__ void lds_wait_ge_quiet(const uint32_t* p, uint32_t want, const Waits& w) {
  while (lds_vload(p) < want) {
    if (__builtin_amdgcn_s_memrealtime() > w.deadline) return;
    __builtin_amdgcn_s_sleep(1);
  }
}

// ---- compute waves: the weight ring -----------------------------------------------------

// s_waitcnt vmcnt(N): every wait is exact because a compute wave's only memory operations are
// its ring loads, which complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Direct-to-LDS loads (each lane's 16 or 4 bytes to LDS address lds + 16 lane or + 4 lane),
// non-temporal (one wait state after the M0 write, which the LDS-DMA form reads), written as
// inline assembly: the compiler then inserts no wait of its own for
// them (it would wait for every such load before any LDS access it cannot prove apart, which
// drains the ring at every step); the ring's waits are the explicit vmcnt waits below.
__device__ __forceinline__ void dma16(const void* g, const void* l) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)l);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(la), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* g, const void* l) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)l);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt" ::"s"(la), "v"(g) : "memory", "m0");
}

// Wave-uniform copies (scalar registers) of values read from LDS descriptors.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const char* uni(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

// The sequence of ring loads of compute wave `cw`: for each work entry, each tile, each of
// the wave's steps (s = cw, cw + kSxCompute, ...): [W4A16: every fourth of the wave's steps, one
// gather of the group scales of its next four steps], then the step's two 1 KB lines. The
// cursor keeps the current entry's fields in scalar registers and the current tile's
// addresses per lane, so an op costs a few scalar instructions and one address add.
template <class F>
struct SxCursor {
  static constexpr bool GS = F::NSC > 0;  // group scales come through the ring
  const SxWork* work;
  const SxComp* comp;
  int nwork, cw;
  int e, t, j, sub;        // entry, tile within the entry, local step, op within the step
  int ns, ntile, nsteps;   // this wave's steps per tile, tiles of the entry, K steps
  bool done;
  int tile0, sw, half, kgroups;
  const char* w;
  const char* ws;
  const char* lw;  // this lane's address of line 0 of the wave's first step in the current tile
  const char* lg;  // W4A16: this lane's row of group scales in the current tile

  __device__ int my_steps(int n) const { return n > cw ? (n - cw + kSxCompute - 1) / kSxCompute : 0; }
  __device__ int ops_in_step(int jj) const { return 2 + (GS && (jj & 3) == 0 ? 1 : 0); }

  // Tile t of the current entry: lane (c, r) reads tile row r (the gate rows 8 t.. then the up
  // rows half + 8 t.. of a SwiGLU tile) at byte 64 jj + 16 c of each step (tile_offset).
  __device__ void enter_tile(int lane) {
    const int tile = tile0 + t, r = lane & 15;
    const int wrow = sw ? (r < 8 ? 8 * tile + r : half + 8 * tile + r - 8) : 16 * tile + r;
    lw = w + tile_offset(wrow, cw, 0, lane, nsteps * 128);
    if constexpr (GS) lg = ws + (size_t)wrow * kgroups * 2;
  }
  // Entry e or the next one in which this wave has steps; done when there is none.
  __device__ void enter_entry(int lane) {
    for (; e < nwork; ++e) {
      const SxWork wk = work[e];
      const SxComp d = comp[uni(wk.proj)];
      nsteps = uni(d.nsteps);
      ns = my_steps(nsteps);
      ntile = uni(wk.ntile);
      if (ns > 0 && ntile > 0) {
        tile0 = uni(wk.tile0);
        sw = uni(d.sw);
        half = uni(d.half);
        kgroups = uni(d.kgroups);
        w = uni(d.w);
        ws = uni(d.ws);
        t = j = sub = 0;
        enter_tile(lane);
        return;
      }
    }
    done = true;
  }
  __device__ void start(const SxWork* wk, const SxComp* cp, int nw, int wave, int lane) {
    work = wk;
    comp = cp;
    nwork = nw;
    cw = wave;
    e = 0;
    done = false;
    enter_entry(lane);
  }
  __device__ void advance(int lane) {
    if (++sub < ops_in_step(j)) return;
    sub = 0;
    if (++j < ns) return;
    j = 0;
    if (++t < ntile) {
      enter_tile(lane);
      return;
    }
    ++e;
    enter_entry(lane);
  }
  // Issue the op at the cursor into ring line `line`.
  __device__ void issue(char* line, int lane) const {
    if (GS && (j & 3) == 0 && sub == 0) {
      // lane = 16 q + r: groups (2 s_q, 2 s_q + 1) of its row, s_q = the wave's step j + q (clamped)
      const int q = lane >> 4;
      int sq = cw + (j + q) * kSxCompute;
      if (sq >= nsteps) sq = cw + j * kSxCompute;
      dma4(lg + sq * 4, line);
    } else {
      const int jj = sub - (GS && (j & 3) == 0 ? 1 : 0);
      dma16(lw + (size_t)j * (kSxCompute * 2048) + jj * 1024, line);
    }
  }
};

// s_waitcnt vmcnt(n) for a run-time n in [0, HI], by binary search over immediates.
template <int LO, int HI>
__device__ __forceinline__ void wait_vm_bs(int n) {
  if constexpr (LO == HI) {
    wait_vm<LO>();
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID)
      wait_vm_bs<LO, MID>(n);
    else
      wait_vm_bs<MID + 1, HI>(n);
  }
}

// The ring of one compute wave: R slots of 1 KB, kept full. The consumer takes a group of up
// to four of the wave's steps at once (k = 2 lines per step, plus the W4A16 scale gather):
// one wait for the group's oldest k loads, k LDS reads, the group's MFMAs, then k new loads
// into the freed slots -- so the bookkeeping and the waits are paid per group, not per line.
template <class F, int R>
struct SxRing {
  char* base;
  int islot, cslot;  // next slot to issue into / take from
  int pending;       // ops issued and not yet freed
  SxCursor<F> cur;

  // Issue loads into free slots, up to the end of work entry `last` (every entry: INT_MAX).
  __device__ void fill(int lane, int last) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the freed slots' reads are done
    while (!cur.done && pending < R && cur.e <= last) {
      cur.issue(base + islot * 1024, lane);
      islot = islot + 1 == R ? 0 : islot + 1;
      ++pending;
      cur.advance(lane);
    }
  }
  // Wait until the oldest k ops in flight have landed.
  __device__ void wait_oldest(int k) {
    if (pending == R)
      wait_vm_bs<0, R - 1>(R - k);
    else
      wait_vm_bs<0, R - 1>(pending - k);
  }
  // Slot of the i-th op of the group that starts at cslot.
  __device__ const char* at(int i) const {
    const int sl = cslot + i;
    return base + (sl >= R ? sl - R : sl) * 1024;
  }
  __device__ void free(int k) {
    cslot += k;
    if (cslot >= R) cslot -= R;
    pending -= k;
  }
};

// One K step of W4A16 from ring lines c[0..1] and the group scales of this wave's rows (bf16
// pairs (group 2s, 2s + 1) for rows rowl..rowl+3): the arithmetic of FmtW4::compute (the code
// bias from the same fragments, in the same MFMA order) with the scales taken from the ring's
// gather instead of the staged scale table.
__device__ __forceinline__ void sx_w4_step(f32x4& acc, const uint4 (&c)[2], const uint4& scw, const char* stage,
                                           const GemmArgs& a, int s, int lane, int xoff, int) {
  const uint32_t sw4[4] = {scw.x, scw.y, scw.z, scw.w};
  const uint4 avb = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x4 tmp = {0.f, 0.f, 0.f, 0.f}, tb = {0.f, 0.f, 0.f, 0.f};
    const uint32_t wd[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
    const int kb = (s * 256 + j * 128 + (lane >> 4) * 32) * 2;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint4 av;
      av.x = nib_pair(wd[t], 0);
      av.y = nib_pair(wd[t], 4);
      av.z = nib_pair(wd[t], 8);
      av.w = nib_pair(wd[t], 12);
      const uint4 bv = *reinterpret_cast<const uint4*>(stage + xoff + kb + t * 16);
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), tmp, 0, 0, 0);
      tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(avb), as_bf16x8(bv), tb, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sc = bf2f(j ? sw4[i] >> 16 : sw4[i] & 0xffffu);
      acc[i] = fmaf(sc, tmp[i] - tb[i], acc[i]);
    }
  }
}

// Staging geometry of a projection with k inputs (the staged slice is all of K). Every format
// stages the bf16 activation (FP8: the compute wave that owns a step turns its 256 bytes per
// token into the step's 128 e4m3 codes in place, at the start of the region).
__device__ __host__ inline void sx_stage_args(const FmtInfo& fi, int m, int k, GemmArgs& a) {
  a.m = m;
  a.k = k;
  a.nsteps = k / fi.kstep;
  a.sps = a.nsteps;
  a.xstride = ((k * 2 + 16) + 15) & ~15;
  a.off_sx = (m * a.xstride + 15) & ~15;
  a.off_xb = a.off_sx + 64 + 64;  // after the token scales (16 floats) and spare
  a.xb_stride = fi.nsc > 1 ? a.nsteps * fi.nsc : a.nsteps;
}
__host__ __device__ inline int sx_stage_bytes(const FmtInfo& fi, int m, int k) {
  GemmArgs a = {};
  sx_stage_args(fi, m, k, a);
  return a.off_xb + (fi.totals ? m * a.xb_stride * 4 : 0);
}
// A residual + RMSNorm stage keeps its sums of squares (one double per 8-value chunk, then the
// token totals) in its staging buffer after what the compute waves read: kSxCssBytes from here.
constexpr int kSxCssBytes = (kSxNormU * kSxIo * 64 + kSxNormMaxM) * 8;
__host__ __device__ inline int sx_css_offset(const FmtInfo& fi, int m, int k) {
  return (sx_stage_bytes(fi, m, k) + 15) & ~15;
}

// FP8 per-token scale from the token's maximum |x| (bits of a non-negative float), as the
// reference takes it: max(amax / 448, 1e-12) (engine/kernels/fp8.py:20-28).
__device__ __forceinline__ float sx_token_scale(uint32_t amax_bits) {
  return fmaxf(__uint_as_float(amax_bits) / 448.f, 1e-12f);
}

// Per-step prologue of compute wave cw for its own steps s = cw, cw + kSxCompute, ... of a
// staged entry; only this wave reads what it writes, so no other wave waits for it.
//   FP8: the e4m3 codes of each token's 128 values of step s (per-token scale from the
//        entry's maxima), written over the first half of the step's bf16 region. Items are
//        (step, token, 16-byte chunk), 16 chunks per region and 64 lanes per pass, so every
//        region is read whole by one instruction before the codes overwrite it.
//   W8A16 / W4A16: the bias sums of the step's scale groups (stage_bias's work).
template <class F>
__device__ __forceinline__ void sx_own_steps_prologue(const GemmArgs& a, char* stage, const uint32_t* amax, int ns,
                                                      int cw, int lane, int m) {
  if constexpr (std::is_same<F, FmtFP8>::value) {
    // lane r < m holds token r's scale and its IEEE reciprocal; items fetch theirs by shuffle
    const int mr = min(lane & 15, m - 1);
    const float scr = sx_token_scale(lds_vload(&amax[mr]));
    const float yr = 1.f / scr;
    const int items = ns * m * 16;
    for (int i0 = 0; i0 < items; i0 += 64) {
      const int it = i0 + lane;
      const int c = it & 15, rs = it >> 4;
      const int mm = it < items ? rs % m : 0;
      const float sc = __shfl(scr, mm, 64), y = __shfl(yr, mm, 64);
      if (it < items) {
        char* p = stage + mm * a.xstride + (cw + (rs / m) * kSxCompute) * 256;
        const uint4 v = *reinterpret_cast<const uint4*>(p + c * 16);
        *reinterpret_cast<uint2*>(p + c * 8) = e4m3_chunk(v, sc, y);
      }
    }
  } else if constexpr (needs_bias_totals<F>()) {
    constexpr int NJ = F::NSC > 1 ? F::NSC : 1;
    const int mm = lane & 15, mrow = min(mm, m - 1);
    float* xb = reinterpret_cast<float*>(stage + a.off_xb);
    for (int jj = 0; jj < ns; ++jj) {
      const int s = cw + jj * kSxCompute;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const f32x4 d = F::bias_chain(stage, s, j, lane, mrow * a.xstride);
        if ((lane >> 4) == 0 && mm < m) xb[mm * a.xb_stride + s * NJ + j] = d[0];
      }
    }
  }
}

// The compute waves: stream the ring, run each tile's MFMAs over this wave's steps, hand the
// tile's partial sums to the IO waves.
template <class F, int R>
__device__ __forceinline__ void sx_compute(const SxLayout& L, char* lds, const SxWork* work, int nwork,
                                           const SxComp* comp, const Waits& w) {
  constexpr bool W4 = std::is_same<F, FmtW4>::value;
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  const int lane = threadIdx.x & 63, cw = uni((int)threadIdx.x >> 6);
  uint32_t* ctl = reinterpret_cast<uint32_t*>(lds + L.ctl_off);
  SxRing<F, R> rg;
  rg.base = lds + L.ring_off + cw * R * 1024;
  rg.islot = rg.cslot = rg.pending = 0;
  rg.cur.start(work, comp, nwork, cw, lane);
  rg.fill(lane, 0x7fffffff);
  const FmtInfo fi = info<F>();
  const int mrow = min(lane & 15, L.m - 1);
  const int rowl = 4 * (lane >> 4);
  int q = 0;  // tiles so far (all entries)
  for (int e = 0; e < nwork; ++e) {
    const SxWork wk = work[e];
    const SxComp d = comp[uni(wk.proj)];
    const int nsteps = uni(d.nsteps), ntile = uni(wk.ntile);
    const int ns = nsteps > cw ? (nsteps - cw + kSxCompute - 1) / kSxCompute : 0;
    GemmArgs a = {};
    sx_stage_args(fi, L.m, nsteps * fi.kstep, a);
    const char* stage = lds + L.stage_off[e & 1];
    const int xoff = mrow * a.xstride;
#pragma unroll
    for (int i = 0; i < kSxIo; ++i) lds_wait_ge_quiet(&ctl[kCtlStaged + (e & 1) * kSxIo + i], (uint32_t)e + 1, w);
    if (ntile > 0) sx_own_steps_prologue<F>(a, const_cast<char*>(stage), &ctl[kCtlAmax + 16 * (e % 3)], ns, cw, lane, L.m);
    for (int t = 0; t < ntile; ++t, ++q) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      // Groups of up to four of this wave's steps (the step within the group is a compile-time
      // index, so the lines and W4A16 scales stay in registers).
      for (int j0 = 0; j0 < ns; j0 += 4) {
        const int n = ns - j0 < 4 ? ns - j0 : 4;
        const int g = W4 ? 1 : 0;  // the scale gather leads the group
        const int k = 2 * n + g;
        rg.wait_oldest(k);
        uint4 scw[4], c[4][2];
        if constexpr (W4) {
          const char* gp = rg.at(0);  // this lane's rows' scales, steps j0..j0+3
#pragma unroll
          for (int v = 0; v < 4; ++v) scw[v] = *reinterpret_cast<const uint4*>(gp + (v * 16 + rowl) * 4);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (u < n) {
            c[u][0] = *reinterpret_cast<const uint4*>(rg.at(g + 2 * u) + lane * 16);
            c[u][1] = *reinterpret_cast<const uint4*>(rg.at(g + 2 * u + 1) + lane * 16);
          }
        rg.free(k);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (u < n) {
            const int s = cw + (j0 + u) * kSxCompute;
            if constexpr (W4) {
              sx_w4_step(acc, c[u], scw[u], stage, a, s, lane, xoff, mrow);
            } else {
              f32x4 accs[1] = {acc};
              const int xo[1] = {xoff}, mr[1] = {mrow};
              // FP8: the step's codes sit at the start of its 256-byte bf16 region
              F::template compute<1>(accs, c[u], stage, a, FP8 ? 2 * s : s, lane, xo, mr, rowl);
              acc = accs[0];
            }
          }
        }
        // While computing entry e, refill only with entry e's loads: a load issue occupies the
        // wave (about 1 KB per 110 ns), and later entries' loads can wait for the time this wave
        // spends waiting for the next entry's input.
        rg.fill(lane, e);
      }
      // Partial sums of tile q to its slot, once the IO waves are done with the slot's
      // previous tile; then the flag that says they are there.
      const int slot = q % kSxSlots;
      lds_wait_ge_quiet(&ctl[kCtlFree + slot], (uint32_t)(q / kSxSlots), w);
      float* red = reinterpret_cast<float*>(lds + L.part_off + (slot * kSxCompute + cw) * L.part_stride);
      if ((lane & 15) < L.m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(rowl + i) * L.m + (lane & 15)] = acc[i];
      }
      asm volatile("" ::: "memory");
      if (lane == 0) lds_vstore(&ctl[kCtlPart + slot * kSxCompute + cw], (uint32_t)(q / kSxSlots + 1));
    }
    rg.fill(lane, 0x7fffffff);  // the entry is done: stream ahead while the next input is produced
  }
  wait_vm<0>();  // no ring load may land after the workgroup's LDS is released
}

// ---- IO waves ---------------------------------------------------------------------------

// The IO waves' staging of one entry: each thread fetches chunks of 8 values (U in flight),
// waits until they have all been published, and stores them as bf16 (in the format's chunk
// order) -- nothing else, so the link from the producers to the compute waves is a poll and a
// copy. FP8: the per-token maxima |x| too: each thread keeps the maximum of its chunks of one
// token and adds it with one LDS atomic at the end (a chunk of another token, where a token's
// row ends inside the thread's chunks, takes its own). No barrier: the compute waves wait for
// every IO wave's flag.
template <class F, class XS, int U>
__device__ __forceinline__ void sx_stage_raw(const GemmArgs& a, const XS& xs, char* stage, int tid, int nthr,
                                             uint32_t* amax) {
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  const int cpr = a.k >> 3;
  const int total = a.m * cpr;
  int row = -1;      // FP8: the token of this thread's running maximum
  float rmax = 0.f;  // and the maximum
  for (int q0 = tid; q0 < total; q0 += U * nthr) {
    typename XS::Raw r[U];
    auto chunk = [&](int u, int& mm, int& kabs) {
      const int q = q0 + u * nthr;
      mm = q / cpr;
      kabs = (q - mm * cpr) * 8;
      return q < total;
    };
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int mm, kabs;
      if (chunk(u, mm, kabs)) xs.fetch(a, mm, kabs, r[u]);
    }
    settle_batch<XS, U>(a, xs, r, chunk);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int mm, kabs;
      if (chunk(u, mm, kabs)) {
        const uint4 v = xs.value(r[u]);
        if constexpr (FP8) {
          *reinterpret_cast<uint4*>(stage + mm * a.xstride + kabs * 2) = v;
          const uint32_t d[4] = {v.x, v.y, v.z, v.w};
          float mx = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fmaxf(fabsf(bf2f(d[j] & 0xffffu)), fabsf(bf2f(d[j] >> 16))));
          if (row < 0) row = mm;
          if (mm == row)
            rmax = fmaxf(rmax, mx);
          else
            atomicMax(&amax[mm], __float_as_uint(mx));
        } else {
          *reinterpret_cast<uint4*>(stage + mm * a.xstride + kabs * 2) = F::order(v);
        }
      }
    }
  }
  if constexpr (FP8) {
    if (row >= 0) atomicMax(&amax[row], __float_as_uint(rmax));
  }
}

// Barrier of the IO waves (residual + RMSNorm stages only): an LDS counter each IO wave adds
// to; `gen` counts the barriers this wave has passed, the same number in every IO wave.
__device__ __forceinline__ void sx_io_barrier(uint32_t* bar, uint32_t& gen, const Waits& w) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  ++gen;
  if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(as_lds(bar), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  lds_wait_ge(bar, gen * kSxIo, w, kWaitInput);
}

// Residual add + RMSNorm input stage (engine/kernels/reference.py:13-28, norm.py:125-139; the
// arithmetic of qlx_add_rms_norm): r = bf16(resid + delta) with delta the published output of an
// earlier projection (DELTA) and resid published by an earlier stage (RWIRE) or in memory; the
// sum of r^2 per token in fp64 in a fixed order (per 8-value chunk, then chunk by chunk), the
// mean rounded to fp32, scale = 1 / sqrt(mean + eps) in fp32; the input bf16(bf16(r * scale) * w)
// goes to the staging buffer as bf16 like any other activation (FP8: with its per-token maxima,
// so the compute waves' codes are the FP8 per-token quantization of the normed row). Every
// workgroup with work in the projection computes the same r and input from the same words in the
// same order; the one holding tile 0 also writes r (memory and published) and the input. One
// pass: m * k / 8 <= kSxNormU * 256 and k a multiple of 512, checked on the host.
template <class F, bool RWIRE, bool DELTA>
__device__ __forceinline__ void sx_stage_norm(const GemmArgs& a, const SxProj& P, char* stage, int tid, int nthr,
                                              uint32_t* amax, double* css, uint32_t* bar, uint32_t& gen, bool owner,
                                              const Waits& w) {
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  constexpr int U = kSxNormU;
  const int lane = threadIdx.x & 63, iw = tid >> 6;
  const int cpr = a.k >> 3, total = a.m * cpr;
  const XWire dx(DELTA ? P.xwire : nullptr, DELTA ? P.xpitch : 0, a.m, w);
  const XWire rx(RWIRE ? P.rwire : nullptr, RWIRE ? a.k : 0, a.m, w);
  GemmArgs ar = a;  // the residual in memory, [m][k]
  ar.x = P.rmem;
  auto chunk = [&](int u, int& mm, int& kabs) {
    const int q = tid + u * nthr;
    mm = q / cpr;
    kabs = (q - mm * cpr) * 8;
    return q < total;
  };
  XWire::Raw rd[U], rr[U];
  XPlain::Raw rp[U];
  uint4 wv[U], rv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int mm, kabs;
    if (chunk(u, mm, kabs)) {
      if constexpr (DELTA) dx.fetch(a, mm, kabs, rd[u]);
      if constexpr (RWIRE)
        rx.fetch(a, mm, kabs, rr[u]);
      else
        XPlain{}.fetch(ar, mm, kabs, rp[u]);
      const u32x4 t = *gmem(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(P.nw) + kabs));
      wv[u] = uint4{t[0], t[1], t[2], t[3]};
    }
  }
  if constexpr (DELTA) settle_batch<XWire, U>(a, dx, rd, chunk);
  if constexpr (RWIRE) settle_batch<XWire, U>(a, rx, rr, chunk);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int mm, kabs;
    if (chunk(u, mm, kabs)) {
      const uint4 x = RWIRE ? rx.value(rr[u]) : rp[u].v;
      uint4 r = x;
      if constexpr (DELTA) {
        const uint4 d = dx.value(rd[u]);
        const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ds[4] = {d.x, d.y, d.z, d.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[i] = bf16_pair(bf2f(xs[i] & 0xffffu) + bf2f(ds[i] & 0xffffu), bf2f(xs[i] >> 16) + bf2f(ds[i] >> 16));
        r = uint4{o[0], o[1], o[2], o[3]};
      }
      rv[u] = r;
      const uint32_t rs[4] = {r.x, r.y, r.z, r.w};
      double ss = 0.0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double lo = bf2f(rs[i] & 0xffffu), hi = bf2f(rs[i] >> 16);
        ss += lo * lo;
        ss += hi * hi;
      }
      css[tid + u * nthr] = ss;
    }
  }
  sx_io_barrier(bar, gen, w);
  // Token t's total, by IO wave t: lane l sums chunks l, l + 64, ... in order, then the wave's
  // lanes pairwise (a fixed tree).
  double* tot = css + kSxNormU * 256;
  if (iw < a.m) {
    double t = 0.0;
    for (int c = lane; c < cpr; c += 64) t += css[iw * cpr + c];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if (lane == 0) tot[iw] = t;
  }
  sx_io_barrier(bar, gen, w);
  int row = -1;
  float rmax = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    int mm, kabs;
    if (chunk(u, mm, kabs)) {
      // mean rounded to fp32, + eps and 1/sqrt in fp32, as torch's rsqrt(mean + eps)
      const float scale = 1.0f / sqrtf((float)(tot[mm] / (double)a.k) + P.eps);
      const uint32_t rs[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w}, ws[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
      uint32_t o[4];
      float mx = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y0 = round_bf(round_bf(bf2f(rs[i] & 0xffffu) * scale) * bf2f(ws[i] & 0xffffu));
        const float y1 = round_bf(round_bf(bf2f(rs[i] >> 16) * scale) * bf2f(ws[i] >> 16));
        o[i] = bf16_pair(y0, y1);
        mx = fmaxf(mx, fmaxf(fabsf(y0), fabsf(y1)));
      }
      const uint4 y = uint4{o[0], o[1], o[2], o[3]};
      if constexpr (FP8) {
        *reinterpret_cast<uint4*>(stage + mm * a.xstride + kabs * 2) = y;
        if (row < 0) row = mm;
        if (mm == row)
          rmax = fmaxf(rmax, mx);
        else
          atomicMax(&amax[mm], __float_as_uint(mx));
      } else {
        *reinterpret_cast<uint4*>(stage + mm * a.xstride + kabs * 2) = F::order(y);
      }
      if (owner) {
        const size_t at = (size_t)mm * a.k + kabs;
        if (P.rout) *gmem(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(P.rout) + at)) = u32x4{rs[0], rs[1], rs[2], rs[3]};
        if (P.nout) *gmem(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(P.nout) + at)) = u32x4{o[0], o[1], o[2], o[3]};
        if (P.rwire_out) {
#pragma unroll
          for (int i = 0; i < 4; ++i) wire_store_pair(P.rwire_out + (at >> 1) + i, rs[i], w.epoch);
        }
      }
    }
  }
  if constexpr (FP8) {
    if (row >= 0) atomicMax(&amax[row], __float_as_uint(rmax));
  }
}

template <class F>
__device__ __forceinline__ void sx_io(const SxLayout& L, char* lds, const SxProj* projs, const SxWork* work, int nwork,
                                      const Waits& w) {
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  constexpr int UNROLL = 5;  // chunks per IO thread in flight: one pass over k <= 10240 at m = 1
  const int lane = threadIdx.x & 63, iw = ((int)threadIdx.x >> 6) - kSxCompute;
  uint32_t* ctl = reinterpret_cast<uint32_t*>(lds + L.ctl_off);
  const int tid = (int)threadIdx.x - kSxCompute * 64;  // within the IO waves
  constexpr int nthr = kSxIo * 64;
  const FmtInfo fi = info<F>();
  float* sws = reinterpret_cast<float*>(lds + L.sws_off);
  int q0 = 0;       // first tile (workgroup-wide count) of the entry
  int q0_prev = 0;  // first tile of the previous entry
  uint32_t bar_gen = 0;  // IO-team barriers passed
  for (int e = 0; e < nwork; ++e) {
    const SxWork wk = work[e];
    const SxProj& P = projs[wk.proj];
    char* stage = lds + L.stage_off[e & 1];
    GemmArgs a = {};
    sx_stage_args(fi, L.m, P.k, a);
    a.x = P.x;
    a.mode = P.sw ? QLX_MODE_SWIGLU : QLX_MODE_BF16;
    a.half = P.half;
    a.n = P.n;
    // Entry e reuses entry e - 2's buffers. Every IO wave has staged entry e - 1, so every IO
    // wave is done with entry e - 2's epilogues (per-row scales e & 1, FP8 maxima (e + 1) % 3);
    // the compute waves have left partial sums of entry e - 2's last tile, so they are done with
    // its staged activation (buffer e & 1).
    if (e >= 1) {
#pragma unroll
      for (int i = 0; i < kSxIo; ++i) lds_wait_ge(&ctl[kCtlStaged + ((e - 1) & 1) * kSxIo + i], (uint32_t)e, w, kWaitInput);
    }
    if (e >= 2) {
      const int ql = q0_prev - 1, slot = ql % kSxSlots;
#pragma unroll
      for (int c = 0; c < kSxCompute; ++c)
        lds_wait_ge(&ctl[kCtlPart + slot * kSxCompute + c], (uint32_t)(ql / kSxSlots + 1), w, kWaitPartial);
    }
    // Per-row scales of the entry's tiles: loaded before the polls and stored after staging, so
    // their memory latency overlaps the wait for the input.
    constexpr int NSW = kSxMaxTilesPerEntry * 16 / (kSxIo * 64);
    uint32_t swv[NSW];
    if constexpr (F::NSC == 0) {
#pragma unroll
      for (int u = 0; u < NSW; ++u) {
        const int i = tid + u * nthr;
        swv[u] = 0u;
        if (i < wk.ntile * 16)
          swv[u] = gmem(reinterpret_cast<const uint16_t*>(P.ws))[weight_row(a, wk.tile0 + i / 16, i & 15)];
      }
    }
    // FP8 maxima: entry e's buffer was cleared at the start of entry e - 1, before IO wave 0
    // raised its flag for entry e - 1, which every IO wave waited for above. Clear entry e + 1's:
    // its last readers, entry e - 2's epilogues, are done.
    uint32_t* amax = &ctl[kCtlAmax + 16 * (e % 3)];
    if constexpr (FP8) {
      if (tid < 16) lds_store(&ctl[kCtlAmax + 16 * ((e + 1) % 3) + tid], 0u);
    }
    float* swe = sws + (e & 1) * kSxMaxTilesPerEntry * 16;
    if (P.norm) {
      double* css = reinterpret_cast<double*>(stage + sx_css_offset(fi, L.m, P.k));
      const bool owner = wk.tile0 == 0;
      if (P.rwire) {
        if (P.xwire)
          sx_stage_norm<F, true, true>(a, P, stage, tid, nthr, amax, css, &ctl[kCtlIoBar], bar_gen, owner, w);
        else
          sx_stage_norm<F, true, false>(a, P, stage, tid, nthr, amax, css, &ctl[kCtlIoBar], bar_gen, owner, w);
      } else {
        if (P.xwire)
          sx_stage_norm<F, false, true>(a, P, stage, tid, nthr, amax, css, &ctl[kCtlIoBar], bar_gen, owner, w);
        else
          sx_stage_norm<F, false, false>(a, P, stage, tid, nthr, amax, css, &ctl[kCtlIoBar], bar_gen, owner, w);
      }
    } else if (P.xwire) {
      const XWire xs(P.xwire, P.xpitch, L.m, w);
      sx_stage_raw<F, XWire, UNROLL>(a, xs, stage, tid, nthr, amax);
    } else {
      sx_stage_raw<F, XPlain, UNROLL>(a, XPlain{}, stage, tid, nthr, amax);
    }
    if constexpr (F::NSC == 0) {
#pragma unroll
      for (int u = 0; u < NSW; ++u) {
        const int i = tid + u * nthr;
        if (i < wk.ntile * 16) swe[i] = bf2f(swv[u]);
      }
    }
    // This wave's part of the staged activation (and of the maxima) is in place: its flag.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) lds_store(&ctl[kCtlStaged + (e & 1) * kSxIo + iw], (uint32_t)e + 1);
    // Epilogues: tile q of the workgroup goes to IO wave q % kSxIo.
    const int nout = P.sw ? P.half : P.n;
    constexpr int NVMAX = 4;
    for (int t = (iw - q0 % kSxIo + kSxIo) % kSxIo; t < wk.ntile; t += kSxIo) {
      const int q = q0 + t, slot = q % kSxSlots;
#pragma unroll
      for (int c = 0; c < kSxCompute; ++c)
        lds_wait_ge(&ctl[kCtlPart + slot * kSxCompute + c], (uint32_t)(q / kSxSlots + 1), w, kWaitPartial);
      const float* red = reinterpret_cast<const float*>(lds + L.part_off + slot * kSxCompute * L.part_stride);
      const int wstride = L.part_stride / 4;  // floats between two compute waves' partials
      const int tile = wk.tile0 + t;
      const int rows_out = P.sw ? 8 : 16;
      const int pairs = (rows_out / 2) * L.m;
      for (int idx = lane; idx < pairs; idx += 64) {
        const int mm = idx / (rows_out / 2), nl = 2 * (idx - mm * (rows_out / 2));
        const int nv = P.sw ? 4 : 2;
        const int rl[NVMAX] = {nl, nl + 1, nl + 8, nl + 9};
        float v[NVMAX];
#pragma unroll
        for (int i = 0; i < NVMAX; ++i) {
          if (i >= nv) break;
          float s = 0.f;
#pragma unroll
          for (int c = 0; c < kSxCompute; ++c) s += red[c * wstride + rl[i] * L.m + mm];
          if constexpr (F::NSC == 0) s *= swe[t * 16 + rl[i]];
          if constexpr (FP8) s *= sx_token_scale(lds_load(&amax[mm]));
          v[i] = s;
        }
        float o0 = v[0], o1 = v[1];
        int oi = 16 * tile + nl;
        if (P.sw) {
          o0 = swiglu_bf(v[0], v[2]);
          o1 = swiglu_bf(v[1], v[3]);
          oi = 8 * tile + nl;
        }
        const uint32_t pair = bf16_pair(o0, o1);
        *gmem(reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(P.y) + (size_t)mm * nout + oi)) = pair;
        if (P.ywire) wire_store_pair(P.ywire + (size_t)mm * (nout >> 1) + (oi >> 1), pair, w.epoch);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's reads are done
      if (lane == 0) lds_store(&ctl[kCtlFree + slot], (uint32_t)(q / kSxSlots + 1));
    }
    q0_prev = q0;
    q0 += wk.ntile;
  }
}

template <class F, int R>
__global__ void __launch_bounds__((kSxCompute + kSxIo) * 64)
stream_kernel(const char* __restrict__ desc, SxLayout L, uint32_t epoch, int* err, long long budget_ticks) {
  extern __shared__ __align__(16) char lds[];
  const SxHeader hd = *reinterpret_cast<const SxHeader*>(desc);
  const Waits w{epoch, __builtin_amdgcn_s_memrealtime() + (unsigned long long)budget_ticks, err};
  const int* start = reinterpret_cast<const int*>(desc + hd.start_off);
  const int w0 = start[blockIdx.x], nwork = start[blockIdx.x + 1] - w0;
  // Copy the compute waves' descriptors and this workgroup's work list to LDS, zero the
  // control words: the launch's one workgroup barrier.
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(desc + hd.comp_off);
    u32x4* dst = reinterpret_cast<u32x4*>(lds + L.comp_off);
    const int n16 = hd.ncalls * (int)(sizeof(SxComp) / 16);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
    const u32x4* ws = reinterpret_cast<const u32x4*>(desc + hd.work_off) + w0;
    u32x4* wd = reinterpret_cast<u32x4*>(lds + L.work_off);
    for (int i = threadIdx.x; i < nwork; i += blockDim.x) wd[i] = ws[i];
    uint32_t* ctl = reinterpret_cast<uint32_t*>(lds + L.ctl_off);
    for (int i = threadIdx.x; i < kCtlWords; i += blockDim.x) ctl[i] = 0u;
  }
  __syncthreads();
  const SxWork* work = reinterpret_cast<const SxWork*>(lds + L.work_off);
  if ((int)threadIdx.x < kSxCompute * 64)
    sx_compute<F, R>(L, lds, work, nwork, reinterpret_cast<const SxComp*>(lds + L.comp_off), w);
  else
    sx_io<F>(L, lds, reinterpret_cast<const SxProj*>(desc + hd.proj_off), work, nwork, w);
}

// Ring sizes the kernel is built for (1 KB lines per compute wave); a launch takes the largest
// its LDS allows. A group of four steps takes 8 lines at once, W4A16's 9 (8 is not built for it).
constexpr int kSxRings[] = {16, 14, 12, 10, 8};

template <class F>
const void* sx_fn_r(int ring) {
  if (ring == 16) return reinterpret_cast<const void*>(&stream_kernel<F, 16>);
  if (ring == 14) return reinterpret_cast<const void*>(&stream_kernel<F, 14>);
  if (ring == 12) return reinterpret_cast<const void*>(&stream_kernel<F, 12>);
  if (ring == 10) return reinterpret_cast<const void*>(&stream_kernel<F, 10>);
  if constexpr (F::NSC == 0)
    if (ring == 8) return reinterpret_cast<const void*>(&stream_kernel<F, 8>);
  return nullptr;
}
const void* sx_fn(int fmt, int ring) {
  switch (fmt) {
    case QLX_FMT_W8A16: return sx_fn_r<FmtW8>(ring);
    case QLX_FMT_W4A16: return sx_fn_r<FmtW4>(ring);
    case QLX_FMT_FP8: return sx_fn_r<FmtFP8>(ring);
    default: return nullptr;
  }
}

FmtInfo sx_info(int fmt) {
  switch (fmt) {
    case QLX_FMT_W8A16: return info<FmtW8>();
    case QLX_FMT_W4A16: return info<FmtW4>();
    default: return info<FmtFP8>();
  }
}

bool sx_overlaps(const void* a, long long na, const void* b, long long nb) {
  const char* x = static_cast<const char*>(a);
  const char* y = static_cast<const char*>(b);
  return x < y + nb && y < x + na;
}

}  // namespace qlx

using namespace qlx;

extern "C" {

int qlx_stream_build(int fmt, int m, const qlx_stack_call* calls, int ncalls, const qlx_norm_input* norms,
                     void* desc, long long* desc_bytes, void* arena, long long* arena_bytes,
                     qlx_stream_launch* launch) {
  QLX_REQUIRE(sx_fn(fmt, kSxRings[0]) != nullptr, "the stream executor serves W8A16, W4A16 and FP8 W8A8 (format %d)",
              fmt);
  QLX_REQUIRE(m >= 1 && m <= 16, "the stream executor serves m = 1..16 (got %d)", m);
  QLX_REQUIRE(calls != nullptr && ncalls >= 1, "no projections");
  const FmtInfo fi = sx_info(fmt);
  auto normed = [&](int c) { return norms != nullptr && norms[c].norm_w != nullptr; };
  std::vector<int> src(ncalls, -1), published(ncalls, 0), rsrc(ncalls, -1), rpublished(ncalls, 0);
  int knorm = 0;  // widest residual + RMSNorm stage
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    QLX_REQUIRE(q.n >= 16 && q.n % 16 == 0 && q.k > 0 && q.k % fi.kstep == 0 && q.k % 8 == 0,
                "projection %d: n=%d k=%d do not fit the tiled format", c, q.n, q.k);
    QLX_REQUIRE(q.mode == QLX_MODE_BF16 || q.mode == QLX_MODE_SWIGLU, "projection %d: mode %d", c, q.mode);
    QLX_REQUIRE(q.w && q.w_scale && q.y && (normed(c) ? q.x == nullptr : q.x != nullptr),
                "projection %d: NULL pointer (x must be NULL exactly when the input is a norm stage)", c);
    if (normed(c)) {
      QLX_REQUIRE(norms[c].resid != nullptr, "projection %d: a norm stage needs its residual", c);
      QLX_REQUIRE(q.k % 512 == 0 && m <= kSxNormMaxM && m * (q.k / 8) <= kSxNormU * kSxIo * 64,
                  "projection %d: a norm stage takes k a multiple of 512 and m * k <= %d (m=%d, k=%d)", c,
                  kSxNormU * kSxIo * 64 * 8, m, q.k);
      knorm = std::max(knorm, q.k);
    }
  }
  auto nout = [&](int c) { return calls[c].mode == QLX_MODE_SWIGLU ? calls[c].n / 2 : calls[c].n; };
  // memory a projection or a norm stage writes
  auto written = [&](const void* p, long long bytes) {
    for (int j = 0; j < ncalls; ++j) {
      if (sx_overlaps(p, bytes, calls[j].y, 2LL * m * nout(j))) return true;
      if (normed(j) && norms[j].resid_out && sx_overlaps(p, bytes, norms[j].resid_out, 2LL * m * calls[j].k))
        return true;
      if (normed(j) && norms[j].normed_out && sx_overlaps(p, bytes, norms[j].normed_out, 2LL * m * calls[j].k))
        return true;
    }
    return false;
  };
  for (int c = 0; c < ncalls; ++c) {
    const long long ybytes = 2LL * m * nout(c);
    for (int j = 0; j < ncalls; ++j)
      if (j != c)
        QLX_REQUIRE(!sx_overlaps(calls[c].y, ybytes, calls[j].y, 2LL * m * nout(j)),
                    "outputs of projections %d and %d overlap", c, j);
    if (normed(c)) {
      const qlx_norm_input& nd = norms[c];
      if (nd.delta) {
        for (int j = 0; j < c; ++j)
          if (nd.delta == calls[j].y && calls[c].k == nout(j)) {
            src[c] = j;
            published[j] = 1;
            break;
          }
        QLX_REQUIRE(src[c] >= 0, "projection %d: the delta of a norm stage is the whole output of an earlier "
                    "projection", c);
      }
      for (int j = 0; j < c; ++j)
        if (normed(j) && norms[j].resid_out && nd.resid == norms[j].resid_out && calls[j].k == calls[c].k) {
          rsrc[c] = j;
          rpublished[j] = 1;
          break;
        }
      QLX_REQUIRE(rsrc[c] >= 0 || !written(nd.resid, 2LL * m * calls[c].k),
                  "projection %d: the residual is memory the chain writes (only an earlier stage's resid_out can "
                  "be)", c);
      QLX_REQUIRE(!nd.resid_out || !sx_overlaps(nd.resid_out, 2LL * m * calls[c].k, nd.resid, 2LL * m * calls[c].k),
                  "projection %d: resid_out overlaps the residual", c);
      continue;
    }
    for (int j = 0; j < c; ++j)
      if (calls[c].x == calls[j].y && calls[c].k <= nout(j)) {
        src[c] = j;
        published[j] = 1;
        break;
      }
    if (src[c] < 0)
      QLX_REQUIRE(!written(calls[c].x, 2LL * m * calls[c].k),
                  "projection %d reads memory the chain writes (only the whole output of an earlier projection "
                  "can be an input)", c);
  }
  int dev = 0, P = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&P, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_status(e, "stream_build");

  // Tiles to workgroups: per projection, contiguous tile ranges, the larger shares to the
  // workgroups with the least weight bytes so far (stable order, so ties rotate).
  std::vector<double> load(P, 0.0);
  std::vector<std::vector<SxWork>> works(P);
  int kmax = 0;
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    const int ntiles = q.n / 16, nsteps = q.k / fi.kstep;
    kmax = std::max(kmax, q.k);
    const double tile_bytes = 2048.0 * nsteps;
    std::vector<int> order(P);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return load[a] < load[b]; });
    const int base = ntiles / P, extra = ntiles % P;
    // the extra tiles go to the least-loaded workgroups; ranges in workgroup order
    std::vector<int> cnt(P, base);
    for (int i = 0; i < extra; ++i) cnt[order[i]] += 1;
    int t0 = 0;
    for (int g = 0; g < P; ++g) {
      if (cnt[g] > 0) {
        QLX_REQUIRE(cnt[g] <= kSxMaxTilesPerEntry, "projection %d: %d tiles per workgroup (max %d)", c, cnt[g],
                    kSxMaxTilesPerEntry);
        works[g].push_back(SxWork{c, t0, cnt[g], 0});
        t0 += cnt[g];
        load[g] += cnt[g] * tile_bytes;
      }
    }
  }
  int max_work = 0, total_work = 0;
  for (int g = 0; g < P; ++g) {
    max_work = std::max(max_work, (int)works[g].size());
    total_work += (int)works[g].size();
  }
  // LDS: [comp descriptors][work list][control][partials][per-row scales][staging x2][rings]
  SxLayout L = {};
  L.m = m;
  int off = 0;
  L.comp_off = off;
  off += ncalls * (int)sizeof(SxComp);
  L.work_off = off;
  off += max_work * (int)sizeof(SxWork);
  L.ctl_off = off;
  off += kCtlWords * 4;
  off = (off + 15) & ~15;
  L.part_off = off;
  L.part_stride = 16 * m * 4;
  off += kSxSlots * kSxCompute * L.part_stride;
  off = (off + 15) & ~15;
  L.sws_off = off;
  off += 2 * kSxMaxTilesPerEntry * 16 * 4;
  L.stage_bytes = (sx_stage_bytes(fi, m, kmax) + 15) & ~15;
  if (knorm > 0) L.stage_bytes = std::max(L.stage_bytes, sx_css_offset(fi, m, knorm) + kSxCssBytes);
  L.stage_off[0] = off;
  L.stage_off[1] = off + L.stage_bytes;
  off += 2 * L.stage_bytes;
  off = (off + 1023) & ~1023;
  L.ring_off = off;
  const int room = (kLdsLimit - off) / (kSxCompute * 1024);
  L.ring_lines = 0;
  for (int r : kSxRings)
    if (r <= room && sx_fn(fmt, r) != nullptr) {
      L.ring_lines = r;
      break;
    }
  QLX_REQUIRE(L.ring_lines > 0, "the stream executor needs %d KB of LDS before its rings (m=%d, k=%d)", off / 1024, m,
              kmax);
  const int lds = off + kSxCompute * L.ring_lines * 1024;
  {  // every workgroup must be resident (cooperative launch): one per CU with this LDS
    const void* fn = sx_fn(fmt, L.ring_lines);
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    int occ = 0;
    if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, (kSxCompute + kSxIo) * 64, lds);
    if (e != hipSuccess) return hip_status(e, "stream_build");
    QLX_REQUIRE(occ >= 1, "the stream executor does not fit a CU with %d bytes of LDS", lds);
  }
  // Arena: published outputs.
  long long aoff = 0;
  std::vector<long long> wire_off(ncalls, -1), rwire_off(ncalls, -1);
  for (int c = 0; c < ncalls; ++c) {
    if (published[c]) {
      wire_off[c] = aoff;
      aoff += ((8LL * m * (nout(c) / 2)) + 255) & ~255LL;
    }
    if (rpublished[c]) {
      rwire_off[c] = aoff;
      aoff += ((8LL * m * (calls[c].k / 2)) + 255) & ~255LL;
    }
  }
  // Descriptor image.
  SxHeader hd = {};
  hd.ncalls = ncalls;
  hd.nwg = P;
  hd.proj_off = (int)sizeof(SxHeader);
  hd.comp_off = hd.proj_off + ncalls * (int)sizeof(SxProj);
  hd.start_off = hd.comp_off + ncalls * (int)sizeof(SxComp);
  hd.work_off = (hd.start_off + (P + 1) * 4 + 15) & ~15;
  hd.max_work = max_work;
  const long long bytes = hd.work_off + (long long)total_work * (long long)sizeof(SxWork);
  if (desc_bytes) *desc_bytes = bytes;
  if (arena_bytes) *arena_bytes = aoff;
  if (launch) {
    launch->grid = P;
    launch->lds_bytes = lds;
    launch->ring_lines = L.ring_lines;
    launch->layout_words = (int)(sizeof(SxLayout) / 4);
    static_assert(sizeof(SxLayout) <= sizeof(launch->layout), "layout does not fit the launch struct");
    memcpy(launch->layout, &L, sizeof(SxLayout));
  }
  if (!desc) return QLX_OK;
  QLX_REQUIRE(arena != nullptr || aoff == 0, "the chain needs an arena of %lld bytes", aoff);
  char* out = static_cast<char*>(desc);
  memset(out, 0, (size_t)bytes);
  memcpy(out, &hd, sizeof(hd));
  char* base = static_cast<char*>(arena);
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    SxProj pj = {};
    pj.w = q.w;
    pj.ws = q.w_scale;
    pj.y = q.y;
    pj.n = q.n;
    pj.k = q.k;
    pj.nsteps = q.k / fi.kstep;
    pj.ntiles = q.n / 16;
    pj.sw = q.mode == QLX_MODE_SWIGLU;
    pj.half = q.n / 2;
    pj.ywire = wire_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + wire_off[c]) : nullptr;
    if (src[c] >= 0) {
      pj.xwire = reinterpret_cast<const uint64_t*>(base + wire_off[src[c]]);
      pj.xpitch = nout(src[c]);
    } else {
      pj.x = q.x;
    }
    if (normed(c)) {
      const qlx_norm_input& nd = norms[c];
      pj.norm = 1;
      pj.nw = nd.norm_w;
      pj.eps = nd.eps;
      if (rsrc[c] >= 0)
        pj.rwire = reinterpret_cast<const uint64_t*>(base + rwire_off[rsrc[c]]);
      else
        pj.rmem = nd.resid;
      pj.rout = nd.resid_out;
      pj.nout = nd.normed_out;
      pj.rwire_out = rwire_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + rwire_off[c]) : nullptr;
    }
    memcpy(out + hd.proj_off + c * sizeof(SxProj), &pj, sizeof(pj));
    SxComp cp = {};
    cp.w = q.w;
    cp.ws = q.w_scale;
    cp.nsteps = pj.nsteps;
    cp.kgroups = q.k / 128;
    cp.sw = pj.sw;
    cp.half = pj.half;
    memcpy(out + hd.comp_off + c * sizeof(SxComp), &cp, sizeof(cp));
  }
  int* start = reinterpret_cast<int*>(out + hd.start_off);
  int wi = 0;
  for (int g = 0; g < P; ++g) {
    start[g] = wi;
    for (const SxWork& wk : works[g]) memcpy(out + hd.work_off + (size_t)(wi++) * sizeof(SxWork), &wk, sizeof(wk));
  }
  start[P] = wi;
  return QLX_OK;
}

int qlx_stream_run(int fmt, const void* desc, const qlx_stream_launch* launch, unsigned epoch, int* error,
                   long long budget_us, void* stream) {
  QLX_REQUIRE(launch != nullptr && desc != nullptr && error != nullptr, "bad stream executor arguments");
  const void* fn = sx_fn(fmt, launch->ring_lines);
  QLX_REQUIRE(fn != nullptr, "the stream executor serves W8A16, W4A16 and FP8 W8A8 (format %d) with rings of 12, 14 or "
              "16 lines (got %d)", fmt, launch->ring_lines);
  QLX_REQUIRE(launch->layout_words == (int)(sizeof(SxLayout) / 4), "launch layout from another library version");
  QLX_REQUIRE(launch->grid >= 1 && launch->lds_bytes > 0 && launch->lds_bytes <= kLdsLimit,
              "bad stream executor launch configuration");
  QLX_REQUIRE((epoch & 0xffffu) != 0, "epoch %u: its low 16 bits tag published values and must not be 0", epoch);
  QLX_REQUIRE(budget_us >= 0 && budget_us <= 600000000LL, "budget_us must be 0..600e6");
  SxLayout L;
  memcpy(&L, launch->layout, sizeof(SxLayout));
  QLX_REQUIRE(L.ring_lines == launch->ring_lines, "bad ring size %d", L.ring_lines);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, launch->lds_bytes);
  if (e != hipSuccess) return hip_status(e, "stream_run");
  long long ticks = budget_us * 100;  // the real-time counter runs at 100 MHz
  const char* d = static_cast<const char*>(desc);
  void* args[] = {(void*)&d, (void*)&L, (void*)&epoch, (void*)&error, (void*)&ticks};
  e = hipLaunchCooperativeKernel(fn, dim3(launch->grid), dim3((kSxCompute + kSxIo) * 64), args,
                                 (unsigned)launch->lds_bytes, (hipStream_t)stream);
  return hip_status(e, "stream_run");
}

}  // extern "C"
