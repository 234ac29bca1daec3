// Decode-step executor: every quantized projection of a decode step in one launch.
//
// The reference runs each projection as its own CUDA launch inside a graph and hides the
// launch gap with programmatic dependent launch: a GEMM's weight loads start while the
// previous kernel drains (engine/kernels/cuda_fp8.py:47-50, 150-169, 252;
// engine/kernels/cuda_jit.py:218-262). HIP has no such launch attribute, and at M = 1 most
// projections are 5-25 MB, so per-launch latency (launch, first loads, activation staging,
// epilogue) costs as much as the weight stream itself.
//
// Here one cooperative launch runs the whole chain on `lanes` sets of workgroups, one
// workgroup per CU in each; lane l runs projections l, l + lanes, ... so a CU works on
// several projections at once and their memory latencies overlap.
//   * Work: a projection's weight is cut into row blocks of rt tiles, each ns K steps long.
//     Each workgroup gets one contiguous, equal share of the projection's block-steps (or
//     of its whole row blocks, when cutting K is not worth it). Each row block a share
//     touches is one work item. A row block cut into several pieces is summed, in piece
//     order, by the workgroup holding piece 0 (its last item of the projection), so results
//     do not depend on timing.
//   * Overlap: a workgroup issues the first weight loads of its next item -- in this
//     projection or a later one -- before it finishes the current item. Weights never
//     depend on activations, so they stream while inputs are still being produced.
//   * Dependencies without barriers: values another workgroup needs (a chained projection's
//     output, a row block's partial sums) are published as 64-bit words {32-bit value, run
//     epoch} with one device-coherent store each, and the reader polls exactly the words it
//     needs until their epoch is the current run's. A dependency costs one store-to-load
//     trip instead of a store, its acknowledgement, a counter update and a counter poll.
//     Every run has a new nonzero epoch, so words left by earlier runs never match.
//   * Every wait is bounded by a per-run deadline on the 100 MHz real-time counter: a wait
//     past it sets the error flag and moves on (that run's outputs are undefined), so the
//     kernel always ends. Cooperative launch guarantees that every workgroup is resident.
#include <vector>

#include "gemm_launch.h"

namespace qlx {

constexpr int kMaxPieces = 4;  // pieces of one row block (the reducer has all in flight)

// One projection of the chain, as the executor reads it (from LDS when the chain's
// descriptors fit next to the items' LDS: read once per launch instead of missing the
// caches, which the weight stream keeps flushing, on every item).
struct alignas(16) StackDesc {
  GemmArgs a;      // a.sps: most steps of one item (LDS layout); a.splits: most pieces of a row block
  uint64_t* xwire;  // the activation as published by an earlier projection, or null (read a.x)
  uint64_t* ywire;  // publish the output here ([m][n_out/2] words), or null
  uint64_t* part;   // partial sums of pieces 1.. ([np-1][m][n] words), or null
  int units;        // work units: block-steps (gran 1) or row blocks (gran ns)
  int pe;           // workgroups with work: min(P, units)
  int gran;         // block-steps per unit
  int sw;           // SwiGLU epilogue
  int xpitch;       // words per token row of xwire (the producer's n_out / 2)
  int off_red;      // LDS byte offset of the waves' partial sums (apart from the staged x)
  int rot;          // workgroup p holds share (p - rot) mod nwg of this projection
  int nwg;          // workgroups per lane
};

// Workgroup p's share of a projection. Shares are rotated from projection to projection (each
// starts where the previous one's workgroups ended), so that when a projection has fewer
// shares than workgroups the extra work does not fall on the same workgroups every layer.
__host__ __device__ inline int share_slot(const StackDesc& d, int p) {
  const int v = p - d.rot;
  return v < 0 ? v + d.nwg : v;
}

// ---- shares of a projection ---------------------------------------------------------

// Workgroup p holds units [p*U/pe, (p+1)*U/pe); owner(u) is the workgroup holding unit u.
// 32-bit arithmetic (64-bit division is a long software sequence on the GPU): the planner
// keeps (U + 1) * (pe + 1) and U * gran below 2^31.
__host__ __device__ inline unsigned share_begin(unsigned p, unsigned U, unsigned pe) { return p * U / pe; }
__host__ __device__ inline unsigned share_owner(unsigned u, unsigned U, unsigned pe) {
  const unsigned o = ((u + 1) * pe + U - 1) / U - 1;
  return o < pe - 1 ? o : pe - 1;
}

// Item of workgroup p in row block g: steps [*step0, *step0 + *nst), piece *piece of *np.
__host__ __device__ inline void share_item(int p, int g, int U, int pe, int gran, int ns, int* step0, int* nst,
                                           int* piece, int* np) {
  const unsigned b0 = share_begin(p, U, pe) * gran, b1 = share_begin(p + 1, U, pe) * gran;
  const unsigned gs = (unsigned)g * ns;
  const unsigned s0 = b0 > gs ? b0 : gs;
  const unsigned s1 = b1 < gs + ns ? b1 : gs + ns;
  *step0 = (int)(s0 - gs);
  *nst = (int)(s1 - s0);
  unsigned first, last;
  if (gran == ns) {  // whole row blocks: unit g
    first = last = share_owner(g, U, pe);
  } else {           // gran 1: units are block-steps
    first = share_owner(gs, U, pe);
    last = share_owner(gs + ns - 1, U, pe);
  }
  *np = (int)(last - first + 1);
  *piece = p - (int)first;
}

// ---- published words -------------------------------------------------------------------

struct Waits {
  uint32_t epoch;
  unsigned long long deadline;  // real-time counter value
  int* err;
};

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load(gmem(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, uint32_t v, uint32_t epoch) {
  __hip_atomic_store(gmem(p), ((uint64_t)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Kinds of wait: the first one of a run to give up leaves (1 << kind) in the error word.
enum WaitSite { kWaitInput = 0, kWaitPartial = 1, kWaitTeam = 2, kWaitChunk = 3, kWaitSlot = 4 };

// True (and the run flagged as failed) once the run's deadline has passed: waits stop there.
__device__ __forceinline__ bool ll_expired(const Waits& w, WaitSite site) {
  if (__builtin_amdgcn_s_memrealtime() <= w.deadline) return false;
  int expect = 0;
  __hip_atomic_compare_exchange_strong(gmem(w.err), &expect, 1 << site, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Activation published by an earlier projection: bf16 pairs, `pitch` words per token row
// (the activation may be the first k columns of a wider output).
struct XWire {
  static constexpr bool POLLS = true;
  const uint64_t* wire;
  int pitch;
  Waits w;
  struct Raw {
    uint64_t v[4];
  };
  __device__ __forceinline__ void fetch(const GemmArgs&, int mm, int kabs, Raw& r) const {
    const uint64_t* p = wire + (size_t)mm * pitch + (kabs >> 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = ll_load(p + i);
  }
  __device__ __forceinline__ bool ready(const Raw& r) const {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 4; ++i) ok &= (uint32_t)(r.v[i] >> 32) == w.epoch;
    return ok;
  }
  __device__ __forceinline__ void refetch(const GemmArgs&, int mm, int kabs, Raw& r) const {
    const uint64_t* p = wire + (size_t)mm * pitch + (kabs >> 1);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if ((uint32_t)(r.v[i] >> 32) != w.epoch) r.v[i] = ll_load(p + i);
  }
  __device__ __forceinline__ bool expired() const { return ll_expired(w, kWaitInput); }
  __device__ __forceinline__ uint4 value(const Raw& r) const {
    return uint4{(uint32_t)r.v[0], (uint32_t)r.v[1], (uint32_t)r.v[2], (uint32_t)r.v[3]};
  }
};

// ---- work items --------------------------------------------------------------------------

// Weight steps in flight per wave: most workgroups' whole share of a decode projection
// (fewer for 4-bit weights, whose dequantization needs more registers).
template <class F>
struct ExecDepth {
  static constexpr int PF = 6;
};
template <>
struct ExecDepth<FmtW4> {
  static constexpr int PF = 4;
};

// Per-wave state of one executor work item: row block tg, steps [step0, step0 + nst), K
// piece s of np; the wave streams tile row wrow at steps step0 + kwi + j * kw, j < my, the
// last being `last`; plus the item's per-row scale for formats with one scale per row.
struct ExecItem {
  int tg, s, np, step0, nst, wt, kwi, my, last, wrow;
  uint32_t scb;  // the per-row scale's bf16 bits, converted only when staged
};

// Issue the wave's first ExecDepth<F>::PF weight steps (and the per-row scale) of a work
// item. A wave without steps in the item (my == 0) loads nothing.
template <class F>
__device__ __forceinline__ void exec_prefetch(const GemmArgs& a, int tg, int step0, int nst, int s, int np,
                                              ExecItem& it, uint4 (&buf)[ExecDepth<F>::PF][F::LOADS]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  it.tg = tg;
  it.s = s;
  it.np = np;
  it.step0 = step0;
  it.nst = nst;
  it.wt = wave / a.kw;
  it.kwi = wave - it.wt * a.kw;
  const int tile0 = tg * a.rt + it.wt;
  const bool active = tile0 < a.ntiles;
  it.wrow = active ? weight_row(a, tile0, lane & 15) : 0;
  it.my = active ? (nst - it.kwi + a.kw - 1) / a.kw : 0;  // this wave's steps: kwi, kwi + kw, ...
  it.last = step0 + it.kwi + (it.my - 1) * a.kw;
  // The scale first: memory counters complete in order, so reading it then waits for no
  // weight load. It stays raw bits here: converting it now would wait for every memory
  // operation still in flight (the previous item's output stores among them).
  it.scb = 0u;
  if constexpr (F::NSC == 0) {
    const int rl = threadIdx.x, tile = tg * a.rt + (rl >> 4);
    if (rl < 16 * a.rt && tile < a.ntiles)
      it.scb = gmem(reinterpret_cast<const uint16_t*>(a.ws))[weight_row(a, tile, rl & 15)];
  }
#pragma unroll
  for (int p = 0; p < ExecDepth<F>::PF; ++p)
    if (p < it.my) load_chunk<F>(buf[p], a, it.wrow, step0 + it.kwi + p * a.kw, lane);
}

// Stage what the item needs in LDS and stream its weight steps through the MFMAs. With
// `reuse`, the activation slice (and its bias sums) staged for the previous item -- same
// projection, same steps -- is still in place.
template <class F, int WAVES, class XS>
__device__ __forceinline__ void exec_main(const GemmArgs& a, const XS& xs, char* lds, const ExecItem& it, bool reuse,
                                          uint4 (&buf)[ExecDepth<F>::PF][F::LOADS], f32x4 (&acc)[1][1]) {
  constexpr int PF = ExecDepth<F>::PF;
  const int lane = threadIdx.x & 63;
  const int step0 = it.step0, nst = it.nst, kwi = it.kwi, my = it.my;
  if (!reuse) {
    if constexpr (std::is_same<F, FmtFP8>::value)
      stage_fp8_act(a, xs, lds, step0, nst);
    else
      stage_bf16<F>(a, xs, lds, step0, nst);
  }
  if constexpr (F::NSC == 0) {
    // Read on every path, so the register is not left pending for the next item's prefetch.
    const float scv = bf2f(it.scb);
    if (threadIdx.x < 16 * a.rt) reinterpret_cast<float*>(lds + a.off_sc)[threadIdx.x] = scv;
  } else {
    stage_scales<F>(a, lds, it.tg, step0, nst);
  }
  __syncthreads();
  if constexpr (F::BIAS != 0.f) {
    if (!reuse) {
      stage_bias<F, WAVES>(a, lds, nst);
      __syncthreads();
    }
  }
  acc[0][0] = f32x4{0.f, 0.f, 0.f, 0.f};
  int xoff[1], mrow[1];
  mrow[0] = min(lane & 15, a.m - 1);
  xoff[0] = mrow[0] * a.xstride;
  const int rowl = it.wt * 16 + 4 * (lane >> 4);
  // Steps j0 .. j0 + PF - 1 are in buf. Every load issued is consumed: a load nobody reads
  // leaves its register pending, and the next item's first use of that register would wait for
  // every memory operation in flight.
  int j0 = 0;
  for (; j0 + 2 * PF <= my; j0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      F::template compute<1>(acc[0], buf[p], lds, a, kwi + (j0 + p) * a.kw, lane, xoff, mrow, rowl);
      load_chunk<F>(buf[p], a, it.wrow, step0 + kwi + (j0 + p + PF) * a.kw, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (j0 + PF <= my) {  // the last block that still refills some buffers
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      F::template compute<1>(acc[0], buf[p], lds, a, kwi + (j0 + p) * a.kw, lane, xoff, mrow, rowl);
      if (j0 + p + PF < my) load_chunk<F>(buf[p], a, it.wrow, step0 + kwi + (j0 + p + PF) * a.kw, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
    j0 += PF;
  }
#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (j0 + p < my) F::template compute<1>(acc[0], buf[p], lds, a, kwi + (j0 + p) * a.kw, lane, xoff, mrow, rowl);
}

// ---- epilogue ----------------------------------------------------------------------------

// Combine the item's waves; then, per output pair: write it (np == 1), publish this piece's
// partial sums (piece > 0), or add the other pieces' partials in piece order and write
// (piece 0). Outputs go to y and, when a later projection reads them, to ywire.
template <class F, bool SW, class Team = BlockTeam>
__device__ __forceinline__ void exec_finish(const StackDesc& d, char* lds, const ExecItem& it,
                                            const f32x4 (&acc)[1][1], const Waits& w, const Team& team = {},
                                            bool guard = true) {
  const GemmArgs& a = d.a;
  char* red = lds + d.off_red;
  acc_to_lds<1, 1>(red, acc, team, guard);
  constexpr int NV = SW ? 4 : 2;  // values per output pair: (g0, g1, u0, u1) or (v0, v1)
  constexpr int rows_out = SW ? 8 : 16;
  const int per_tile = (rows_out / 2) * a.m;
  const int total = a.rt * per_tile;
  const int nout = SW ? a.half : a.n;
  const int piece = it.s, np = it.np;
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
  for (int idx = team.tid(); idx < total; idx += team.size()) {
    const int tl = idx / per_tile, rem = idx - tl * per_tile;
    const int mm = rem / (rows_out / 2), nl = 2 * (rem - mm * (rows_out / 2));
    const int tile = it.tg * a.rt + tl;
    if (tile >= a.ntiles) continue;
    int row[NV];  // weight rows of the values
    float v[NV];
    if constexpr (SW) {
      row[0] = 8 * tile + nl;
      row[1] = row[0] + 1;
      row[2] = a.half + row[0];
      row[3] = row[2] + 1;
      v[0] = tile_value<F, 1, 1>(a, red, lds, tl, nl, mm);
      v[1] = tile_value<F, 1, 1>(a, red, lds, tl, nl + 1, mm);
      v[2] = tile_value<F, 1, 1>(a, red, lds, tl, nl + 8, mm);
      v[3] = tile_value<F, 1, 1>(a, red, lds, tl, nl + 9, mm);
    } else {
      row[0] = 16 * tile + nl;
      row[1] = row[0] + 1;
      v[0] = tile_value<F, 1, 1>(a, red, lds, tl, nl, mm);
      v[1] = tile_value<F, 1, 1>(a, red, lds, tl, nl + 1, mm);
    }
    if (np > 1) {
      if (piece > 0) {
        uint64_t* part = d.part + ((size_t)(piece - 1) * a.m + mm) * a.n;
#pragma unroll
        for (int i = 0; i < NV; ++i) ll_store(part + row[i], __float_as_uint(v[i]), w.epoch);
        continue;
      }
      uint64_t raw[kMaxPieces - 1][NV];
#pragma unroll
      for (int q = 1; q < kMaxPieces; ++q)
        if (q < np) {
          const uint64_t* part = d.part + ((size_t)(q - 1) * a.m + mm) * a.n;
#pragma unroll
          for (int i = 0; i < NV; ++i) raw[q - 1][i] = ll_load(part + row[i]);
        }
      // Re-poll every stale word together until all pieces are in (bounded).
      while (true) {
        bool all = true;
#pragma unroll
        for (int q = 1; q < kMaxPieces; ++q)
#pragma unroll
          for (int i = 0; i < NV; ++i)
            if (q < np && (uint32_t)(raw[q - 1][i] >> 32) != w.epoch) all = false;
        if (all || ll_expired(w, kWaitPartial)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 1; q < kMaxPieces; ++q)
          if (q < np) {
            const uint64_t* part = d.part + ((size_t)(q - 1) * a.m + mm) * a.n;
#pragma unroll
            for (int i = 0; i < NV; ++i)
              if ((uint32_t)(raw[q - 1][i] >> 32) != w.epoch) raw[q - 1][i] = ll_load(part + row[i]);
          }
      }
#pragma unroll
      for (int q = 1; q < kMaxPieces; ++q)
        if (q < np)
#pragma unroll
          for (int i = 0; i < NV; ++i) v[i] += __uint_as_float((uint32_t)raw[q - 1][i]);
    }
    float o0 = v[0], o1 = v[1];
    if constexpr (SW) {
      o0 = swiglu_bf(v[0], v[2]);
      o1 = swiglu_bf(v[1], v[3]);
    }
    const int oi = row[0];  // first output of the pair (even; for SwiGLU the gate row index)
    const uint32_t pair = bf16_pair(o0, o1);
    *gmem(reinterpret_cast<uint32_t*>(y + (size_t)mm * nout + oi)) = pair;
    if (d.ywire) ll_store(d.ywire + (size_t)mm * (nout >> 1) + (oi >> 1), pair, w.epoch);
  }
}

// ---- the chain ---------------------------------------------------------------------------

// The work item after (c, g) for workgroup p of its lane: (c, g + 1) inside its share, else
// the first row block of the lane's next projection in which p has work. False when there is
// none. Lane l runs projections l, l + lanes, l + 2 lanes, ...
__device__ __forceinline__ bool next_work(const StackDesc* calls, int ncalls, int lanes, int lane, int p, int& c,
                                          int& g) {
  if (c >= 0) {
    const StackDesc& d = calls[c];
    if ((unsigned)(g + 1) * d.a.nsteps < share_begin(share_slot(d, p) + 1, d.units, d.pe) * d.gran) {
      ++g;
      return true;
    }
  }
  for (c = c < 0 ? lane : c + lanes; c < ncalls; c += lanes) {
    const StackDesc& d = calls[c];
    const int v = share_slot(d, p);
    if (v < d.pe) {
      const unsigned u = share_begin(v, d.units, d.pe);
      g = d.gran == d.a.nsteps ? (int)u : (int)(u / d.a.nsteps);
      return true;
    }
  }
  return false;
}

template <class F>
__device__ __forceinline__ void prefetch_work(const StackDesc& d, int p, int g, ExecItem& it,
                                              uint4 (&buf)[ExecDepth<F>::PF][F::LOADS]) {
  int step0, nst, piece, np;
  share_item(share_slot(d, p), g, d.units, d.pe, d.gran, d.a.nsteps, &step0, &nst, &piece, &np);
  exec_prefetch<F>(d.a, g, step0, nst, piece, np, it, buf);
}

// A workgroup's next work item, found ahead of time: finding it is arithmetic, and arithmetic
// that runs after the item's output stores may wait for them (a register it reuses can still
// be the target of a load), which would delay the next item's weight loads.
struct NextItem {
  bool have;
  int c, g, step0, nst, piece, np;
};
__device__ __forceinline__ NextItem find_next(const StackDesc* calls, int ncalls, int lanes, int lane, int p, int c,
                                              int g) {
  NextItem n;
  n.c = c;
  n.g = g;
  n.have = next_work(calls, ncalls, lanes, lane, p, n.c, n.g);
  if (n.have) {
    const StackDesc& d = calls[n.c];
    share_item(share_slot(d, p), n.g, d.units, d.pe, d.gran, d.a.nsteps, &n.step0, &n.nst, &n.piece, &n.np);
  }
  return n;
}

template <class F, int WAVES, bool DLDS>
__global__ void __launch_bounds__(WAVES * 64)
stack_kernel(const StackDesc* __restrict__ gcalls, int ncalls, uint32_t epoch, int* err, long long budget_ticks,
             int desc_off, int lanes) {
  extern __shared__ __align__(16) char lds[];
  const int per_lane = gridDim.x / lanes;
  const int lane = blockIdx.x / per_lane, p = blockIdx.x - lane * per_lane;
  const Waits w{epoch, __builtin_amdgcn_s_memrealtime() + (unsigned long long)budget_ticks, err};
  const StackDesc* calls = gcalls;
  if constexpr (DLDS) {
    const int n16 = ncalls * (int)(sizeof(StackDesc) / 16);
    const auto src = gmem(reinterpret_cast<const u32x4*>(gcalls));
    u32x4* dst = reinterpret_cast<u32x4*>(lds + desc_off);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
    calls = reinterpret_cast<const StackDesc*>(lds + desc_off);
  }
  ExecItem cur, nxt;
  uint4 buf[ExecDepth<F>::PF][F::LOADS];
  f32x4 acc[1][1];
  int nc = -1, ng = 0;
  int staged_c = -1, staged_step0 = -1, staged_nst = -1;  // activation slice now in LDS
  bool have = next_work(calls, ncalls, lanes, lane, p, nc, ng);
  if (have) prefetch_work<F>(calls[nc], p, ng, nxt, buf);
  while (have) {
    const int c = nc;
    const StackDesc& d = calls[c];
    cur = nxt;
    const bool reuse = staged_c == c && staged_step0 == cur.step0 && staged_nst == cur.nst;
    if (d.xwire)
      exec_main<F, WAVES>(d.a, XWire{d.xwire, d.xpitch, w}, lds, cur, reuse, buf, acc);
    else
      exec_main<F, WAVES>(d.a, XPlain{}, lds, cur, reuse, buf, acc);
    staged_c = c;
    staged_step0 = cur.step0;
    staged_nst = cur.nst;
    // Outputs first: later projections wait for them. Anything before them -- finding the
    // next item, issuing its loads (the stores would queue behind them) -- delays the chain
    // (measured: 60-160 us per decode step).
    if (d.sw)
      exec_finish<F, true>(d, lds, cur, acc, w);
    else
      exec_finish<F, false>(d, lds, cur, acc, w);
    const NextItem after = find_next(calls, ncalls, lanes, lane, p, nc, ng);
    have = after.have;
    nc = after.c;
    ng = after.g;
    if (have) exec_prefetch<F>(calls[nc].a, ng, after.step0, after.nst, after.piece, after.np, nxt, buf);
    __syncthreads();  // LDS is reused by the next item
  }
}

template <class F>
const void* stack_fn(int waves, bool dlds) {
  if (waves == 4)
    return dlds ? reinterpret_cast<const void*>(&stack_kernel<F, 4, true>)
                : reinterpret_cast<const void*>(&stack_kernel<F, 4, false>);
  return dlds ? reinterpret_cast<const void*>(&stack_kernel<F, 8, true>)
              : reinterpret_cast<const void*>(&stack_kernel<F, 8, false>);
}

// ---- ring executor: weight-loading waves feed the compute waves through LDS -------------
//
// In the executor above every wave streams its own weights, so the loads it issues for its
// next item sit in the same in-order memory queue as the polls of that item's activation:
// a poll's answer waits for every weight load issued before it, and while a dependency is
// outstanding the wave can keep only a few steps in flight. Here the workgroup has NC compute
// waves and NL loader waves. The loaders walk the same work items and copy every weight step
// (and, for per-row-scale formats, each item's scales) into an LDS ring of 1 KB chunks, as far
// ahead as the ring allows; they never wait for an activation. The compute waves stage
// activations, wait only for the words they need and read weights from the ring. Weights
// never depend on activations, so the HBM stream goes on while the chain waits for a
// dependency. One wave streams about one 1 KB chunk per 150 ns however many loads it keeps in
// flight (measured on MI355X, for plain loads and for LDS-direct loads alike), so a CU needs
// four to six loader waves to draw its share of 7 TB/s; they keep eight plain 16-byte-per-lane
// loads in flight each and write every chunk to its slot once the slot is free.
//
// Stream order of one workgroup: item after item, each [scale chunk], then its steps in
// order, in each step the rt tiles in order, each tile step as two 1 KB chunks (the two
// 16-byte loads of every lane). Loader l copies the chunks q with q % NL == l; chunk q lives
// in ring slot q % R. Counters in LDS: landed[l] = chunks of loader l in place (its chunks
// in stream order, so chunk q is in place once landed[q % NL] > q / NL); pos[w] = first
// chunk compute wave w still needs (monotonic). A loader writes chunk q once q < min(pos) + R.
// Compute waves wait for each other through an LDS counter (the hardware barrier would wait
// for the loaders too).

constexpr int kCtlBytes = 256;
constexpr int kCtlBar = 0, kCtlLanded = 4, kCtlAmax = 16, kCtlPos = 32;  // uint32 indices
constexpr int kLoaderDepth = 8;  // loads each loader wave keeps in flight
// A compute wave reads its next step (two chunks, NC waves x 2 chunks further on) before it
// releases the current one, so it needs chunk pos + 2 NC + 1 while holding pos: the ring must
// hold more than 17 chunks, or the slowest wave could never get its next step.
constexpr int kRingMinChunks = 32;

template <int NC>
struct RingTeam {
  uint32_t* bar;
  Waits w;
  __device__ __forceinline__ int tid() const { return threadIdx.x; }
  __device__ __forceinline__ int size() const { return NC * 64; }
  // Arrival k (counting from 0) belongs to barrier k / NC: no wave reaches barrier b + 1
  // before all have reached b, so the counter needs no reset.
  __device__ __forceinline__ void sync() const {
    uint32_t old = 0;
    if ((threadIdx.x & 63) == 0) old = __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    const uint32_t target = (old / NC + 1) * NC;
    while (__hip_atomic_load(bar, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
      if (ll_expired(w, kWaitTeam)) break;
      __builtin_amdgcn_s_sleep(1);
    }
  }
};

// The geometry of a workgroup's item that both roles derive from the descriptor.
struct RingItem {
  int tg, step0, nst, piece, np, lrt;
  uint32_t n;  // chunks
};
template <class F>
__device__ __forceinline__ RingItem ring_item(const StackDesc& d, int p, int g) {
  RingItem r;
  r.tg = g;
  share_item(share_slot(d, p), g, d.units, d.pe, d.gran, d.a.nsteps, &r.step0, &r.nst, &r.piece, &r.np);
  r.lrt = 31 - __builtin_clz((unsigned)d.a.rt);
  r.n = (F::NSC == 0 ? 1u : 0u) + ((uint32_t)r.nst << (r.lrt + 1));
  return r;
}

// The 16 bytes (8 bf16 per-row scales) that lane `lane` copies for row block tg: rows in
// block order ([gate rows][up rows] for SwiGLU blocks); lanes past the block copy a valid
// block that nobody reads.
__device__ __forceinline__ const u32x4* scale_block(const GemmArgs& a, int tg, int lane) {
  const u32x4* ws = reinterpret_cast<const u32x4*>(a.ws);
  const int tile0 = tg * a.rt;
  int b = 0;
  if (a.mode == QLX_MODE_SWIGLU) {  // rt blocks of gate rows (8 per tile), then rt of up rows
    if (lane < a.rt) b = min(tile0 + lane, a.half / 8 - 1);
    else if (lane < 2 * a.rt) b = min((a.half + 8 * tile0) / 8 + lane - a.rt, a.n / 8 - 1);
  } else if (lane < 2 * a.rt) {
    b = min(2 * tile0 + lane, a.n / 8 - 1);
  }
  return ws + b;
}

// Wave-uniform value (kept in scalar registers: the loader's bookkeeping is scalar work).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Loader wave l: chunks l, l + NL, l + 2 NL, ... of the workgroup's stream. Loads run
// kLoaderDepth chunks ahead of the writes (chunk t of this loader is in buf[t % depth]); a
// chunk is written once its slot is free, then counted in landed[l]. The item's geometry is
// held in scalar registers; a weight chunk's address is tile_offset() of the tiled layout
// with the wave-uniform part computed once per chunk.
template <class F, int NC, int NL>
__device__ __forceinline__ void ring_loader(const StackDesc* calls, int ncalls, int p, char* lds, uint32_t* ctl,
                                            int ring_off, uint32_t rmask, const Waits& w) {
  static_assert(F::LOADS == 2, "one tile step is two 1 KB chunks");
  constexpr int D = kLoaderDepth;
  constexpr int nsc = F::NSC == 0 ? 1 : 0;
  const int l = uni((int)(threadIdx.x >> 6) - NC), lane = threadIdx.x & 63;
  uint32_t* landed = ctl + kCtlLanded;
  const uint32_t* pos = ctl + kCtlPos;
  char* ring = lds + ring_off;
  int c = -1, g = 0;
  bool more = next_work(calls, ncalls, 1, 0, p, c, g);
  if (!more) return;
  // The current item, as scalars, and this lane's part of its addresses.
  const char* wb = nullptr;
  int spr = 0, rt = 1, lrt = 0, ntiles = 1, tile0 = 0, step0 = 0, n = 0, sw = 0, rowsel = 0;
  const u32x4* sptr = nullptr;
  auto enter = [&]() {
    const StackDesc& d = calls[c];
    const RingItem it = ring_item<F>(d, p, g);
    wb = reinterpret_cast<const char*>(d.a.w);
    spr = uni((std::is_same<F, FmtW4>::value ? d.a.k >> 1 : d.a.k) >> 7);  // 128-byte steps per row
    rt = uni(d.a.rt);
    lrt = uni(it.lrt);
    ntiles = uni(d.a.ntiles);
    tile0 = uni(it.tg * d.a.rt);
    step0 = uni(it.step0);
    n = uni((int)it.n);
    sw = uni(d.a.mode == QLX_MODE_SWIGLU);
    const int r = lane & 15;
    rowsel = sw ? (r < 8 ? r : d.a.half + r - 8) : r;  // weight row of tile row r, less 8 * tile
    if (nsc) sptr = scale_block(d.a, it.tg, lane);
  };
  enter();
  int idx = l;  // this loader's next chunk, within the current item
  // The next chunk's address for this lane; false once the stream has ended. The flag (not the
  // per-lane address) steers the loop, so the bookkeeping stays wave-uniform.
  auto next_chunk = [&](const u32x4*& ptr) -> bool {
    while (more && idx >= n) {
      idx -= n;
      more = next_work(calls, ncalls, 1, 0, p, c, g);
      if (more) enter();
    }
    if (!more) return false;
    if (nsc && idx == 0) {
      ptr = sptr;
    } else {
      const int e = idx - nsc;
      const int j = e & 1, t = (e >> 1) & (rt - 1), step = step0 + (e >> (lrt + 1));
      const int tile = min(tile0 + t, ntiles - 1);
      size_t off;
      if (!sw) {  // rows 16 tile .. 16 tile + 15: the chunk is 1 KB of consecutive bytes
        off = ((size_t)(tile * spr + step) * 2 + j) * 1024 + lane * 16;
      } else {
        const int wrow = 8 * tile + rowsel;
        off = ((size_t)((wrow >> 4) * spr + step) * 2 + j) * 1024 + (lane >> 4) * 256 + (wrow & 15) * 16;
      }
      ptr = reinterpret_cast<const u32x4*>(wb + off);
    }
    idx += NL;
    return true;
  };
  auto load = [](const u32x4* ptr) { return __builtin_nontemporal_load(gmem(ptr)); };
  u32x4 buf[D];
  uint32_t issued = 0;
  const u32x4* any = nullptr;  // an address already read: where loads past the end go
#pragma unroll
  for (int k = 0; k < D; ++k) {
    if (next_chunk(any)) ++issued;
    buf[k] = load(any);
  }
  uint32_t t = 0, limit = rmask + 1;
  bool live = true;  // false once the run's deadline has passed: stop waiting for slots
  while (t < issued) {
#pragma unroll
    for (int k = 0; k < D; ++k) {
      if (t < issued) {
        const uint32_t q = (uint32_t)l + NL * t;
        while (q >= limit && live) {  // ring full: wait for the compute waves to free slots
          uint32_t mn = __hip_atomic_load(&pos[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
          for (int v = 1; v < NC; ++v)
            mn = min(mn, __hip_atomic_load(&pos[v], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP));
          limit = (uint32_t)uni((int)mn) + rmask + 1;
          if (q < limit) break;
          if (ll_expired(w, kWaitSlot)) live = false;
          else __builtin_amdgcn_s_sleep(1);
        }
        *reinterpret_cast<u32x4*>(ring + ((q & rmask) << 10) + lane * 16) = buf[k];
        ++t;
        __hip_atomic_store(&landed[l], t, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (next_chunk(any)) ++issued;
      }
      buf[k] = load(any);
    }
  }
}

// Compute side: wait until chunk q is in its slot (cached counters; bounded by the deadline).
template <int NL>
struct Landed {
  const uint32_t* landed;
  uint32_t c[NL];  // last value read of each loader's counter
  __device__ __forceinline__ void wait(uint32_t q, const Waits& w) {
    const int l = (int)(q % NL);
    const uint32_t t = q / NL;
    uint32_t have = 0;
#pragma unroll
    for (int i = 0; i < NL; ++i)
      if (i == l) have = c[i];
    if (have > t) return;
    while (true) {
      have = __hip_atomic_load(&landed[l], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (have > t) break;
      if (ll_expired(w, kWaitChunk)) {
        have = 0xffffffffu;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < NL; ++i)
      if (i == l) c[i] = have;
  }
};

template <class F, int NC, int NL, bool DLDS>
__global__ void __launch_bounds__((NC + NL) * 64)
ring_kernel(const StackDesc* __restrict__ gcalls, int ncalls, uint32_t epoch, int* err, long long budget_ticks,
            int desc_off, int ctl_off, int ring_off, uint32_t rmask) {
  extern __shared__ __align__(16) char lds[];
  const int p = blockIdx.x, wave = uni((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const Waits w{epoch, __builtin_amdgcn_s_memrealtime() + (unsigned long long)budget_ticks, err};
  uint32_t* ctl = reinterpret_cast<uint32_t*>(lds + ctl_off);
  if (threadIdx.x < kCtlBytes / 4) ctl[threadIdx.x] = 0u;
  const StackDesc* calls = gcalls;
  if constexpr (DLDS) {
    const int n16 = ncalls * (int)(sizeof(StackDesc) / 16);
    const auto src = gmem(reinterpret_cast<const u32x4*>(gcalls));
    u32x4* dst = reinterpret_cast<u32x4*>(lds + desc_off);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
    calls = reinterpret_cast<const StackDesc*>(lds + desc_off);
  }
  __syncthreads();  // the only barrier of all waves
  if (wave >= NC) {
    ring_loader<F, NC, NL>(calls, ncalls, p, lds, ctl, ring_off, rmask, w);
    return;
  }
  const RingTeam<NC> team{ctl + kCtlBar, w};
  uint32_t* pos = ctl + kCtlPos;
  uint32_t* amax = ctl + kCtlAmax;
  const char* ring = lds + ring_off;
  Landed<NL> landed{ctl + kCtlLanded, {}};
  auto release = [&](uint32_t v) {
    if (lane == 0) __hip_atomic_store(&pos[wave], v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  uint32_t q = 0;
  int c = -1, g = 0;
  int staged_c = -1, staged_step0 = -1, staged_nst = -1;  // activation slice now in LDS
  while (next_work(calls, ncalls, 1, 0, p, c, g)) {
    const StackDesc& d = calls[c];
    const GemmArgs& a = d.a;
    const RingItem it = ring_item<F>(d, p, g);
    constexpr uint32_t nsc = F::NSC == 0 ? 1u : 0u;
    const int lkw = 31 - __builtin_clz((unsigned)a.kw);
    const int wt = wave >> lkw, kwi = wave & (a.kw - 1);
    const bool active = it.tg * a.rt + wt < a.ntiles;
    const int my = active && it.nst > kwi ? (it.nst - kwi + a.kw - 1) >> lkw : 0;
    const bool reuse = staged_c == c && staged_step0 == it.step0 && staged_nst == it.nst;
    // Per-row scales: from the item's scale chunk (bf16, rows in block order).
    if constexpr (F::NSC == 0) {
      landed.wait(q, w);
      if (threadIdx.x < 16 * a.rt) {
        const uint16_t* sl = reinterpret_cast<const uint16_t*>(ring + ((q & rmask) << 10));
        const int rl = threadIdx.x, t = rl >> 4, r = rl & 15;
        const int at = a.mode == QLX_MODE_SWIGLU ? (r < 8 ? 8 * t + r : 8 * a.rt + 8 * t + r - 8) : rl;
        reinterpret_cast<float*>(lds + a.off_sc)[rl] = bf2f(sl[at]);
      }
      release(q + nsc);
    } else {
      stage_scales<F>(a, lds, it.tg, it.step0, it.nst, team);
    }
    if (!reuse) {
      if constexpr (std::is_same<F, FmtFP8>::value) {
        if (d.xwire)
          stage_fp8_act(a, XWire{d.xwire, d.xpitch, w}, lds, it.step0, it.nst, team, amax);
        else
          stage_fp8_act(a, XPlain{}, lds, it.step0, it.nst, team, amax);
      } else {
        if (d.xwire)
          stage_bf16<F>(a, XWire{d.xwire, d.xpitch, w}, lds, it.step0, it.nst, team);
        else
          stage_bf16<F>(a, XPlain{}, lds, it.step0, it.nst, team);
      }
      staged_c = c;
      staged_step0 = it.step0;
      staged_nst = it.nst;
    }
    if (!reuse || F::NSC != 0) team.sync();
    if constexpr (F::BIAS != 0.f) {
      if (!reuse) {
        stage_bias<F, NC>(a, lds, it.nst);
        team.sync();
      }
    }
    // Main loop: this wave's steps kwi, kwi + kw, ... of tile wt, two chunks each, the next
    // step's chunks read while the current one is in the MFMAs.
    f32x4 acc[1][1];
    acc[0][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    int xoff[1], mrow[1];
    mrow[0] = min(lane & 15, a.m - 1);
    xoff[0] = mrow[0] * a.xstride;
    const int rowl = wt * 16 + 4 * (lane >> 4);
    auto chunk_of = [&](int jj) {
      return q + nsc + ((uint32_t)(((kwi + (jj << lkw)) << it.lrt) + wt) << 1);
    };
    auto fetch = [&](uint4 (&cb)[2], int jj) {
      const uint32_t cq = chunk_of(jj);
      landed.wait(cq, w);
      landed.wait(cq + 1, w);
      cb[0] = *reinterpret_cast<const uint4*>(ring + ((cq & rmask) << 10) + lane * 16);
      cb[1] = *reinterpret_cast<const uint4*>(ring + (((cq + 1) & rmask) << 10) + lane * 16);
    };
    uint4 ca[2], cb[2];
    if (my > 0) fetch(ca, 0);
    for (int jj = 0; jj < my; jj += 2) {
      if (jj + 1 < my) fetch(cb, jj + 1);
      F::template compute<1>(acc[0], ca, lds, a, kwi + (jj << lkw), lane, xoff, mrow, rowl);
      release(jj + 1 < my ? chunk_of(jj + 1) : q + it.n);
      if (jj + 1 >= my) break;
      if (jj + 2 < my) fetch(ca, jj + 2);
      F::template compute<1>(acc[0], cb, lds, a, kwi + ((jj + 1) << lkw), lane, xoff, mrow, rowl);
      release(jj + 2 < my ? chunk_of(jj + 2) : q + it.n);
    }
    release(q + it.n);
    ExecItem ei;
    ei.tg = it.tg;
    ei.s = it.piece;
    ei.np = it.np;
    if (d.sw)
      exec_finish<F, true>(d, lds, ei, acc, w, team, false);
    else
      exec_finish<F, false>(d, lds, ei, acc, w, team, false);
    if constexpr (std::is_same<F, FmtFP8>::value) {
      if (threadIdx.x < a.m) amax[threadIdx.x] = 0u;  // for the next staging
    }
    team.sync();  // the next item overwrites scales, partial sums and maybe the activation
    q += it.n;
  }
}

// Compute and loader waves per workgroup the ring executor is built for: 8, 10 or 12 waves
// (at most three per SIMD, so each wave keeps 168 registers).
bool ring_shape_ok(int waves, int loaders) {
  return (waves == 4 && (loaders == 4 || loaders == 6)) || (waves == 8 && loaders == 4);
}

template <class F, int NC, int NL>
const void* ring_fn2(bool dlds) {
  return dlds ? reinterpret_cast<const void*>(&ring_kernel<F, NC, NL, true>)
              : reinterpret_cast<const void*>(&ring_kernel<F, NC, NL, false>);
}

template <class F>
const void* ring_fn(int waves, int loaders, bool dlds) {
  if (waves == 8) return ring_fn2<F, 8, 4>(dlds);
  return loaders == 6 ? ring_fn2<F, 4, 6>(dlds) : ring_fn2<F, 4, 4>(dlds);
}

const void* ring_fn_for(int fmt, int waves, int loaders, bool dlds) {
  if (!ring_shape_ok(waves, loaders)) return nullptr;
  switch (fmt) {
    case QLX_FMT_W8A16: return ring_fn<FmtW8>(waves, loaders, dlds);
    case QLX_FMT_W4A16: return ring_fn<FmtW4>(waves, loaders, dlds);
    case QLX_FMT_FP8: return ring_fn<FmtFP8>(waves, loaders, dlds);
    default: return nullptr;
  }
}

const void* stack_fn_for(int fmt, int waves, bool dlds) {
  switch (fmt) {
    case QLX_FMT_W8A16: return stack_fn<FmtW8>(waves, dlds);
    case QLX_FMT_W4A16: return stack_fn<FmtW4>(waves, dlds);
    case QLX_FMT_FP8: return stack_fn<FmtFP8>(waves, dlds);
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

// ---- planning (host) -------------------------------------------------------------------

// LDS of one executor item: the single-call layout plus the waves' partial sums kept apart
// from the staged activation (which later items of the same projection reuse).
int exec_lds(const FmtInfo& fi, const qlx_plan& p, int m, int n, int k, GemmArgs& a) {
  const int base = (layout(fi, p, m, n, k, a) + 15) & ~15;
  return base + p.waves * 16 * 16 * 4;  // [wave][16 rows][16 tokens] floats (rw = 1, mt = 1)
}

struct StackPlan {
  qlx_plan plan;
  int units, pe, gran, sps, max_np;
};

// Checks the shares of one candidate: every row block's pieces are consecutive workgroups
// whose step ranges tile [0, ns) in order, each within sps steps. Returns the most pieces of
// one row block, or -1.
int check_shares(int groups, int ns, int U, int pe, int gran, int sps) {
  int max_np = 1;
  for (int g = 0; g < groups; ++g) {
    const unsigned gs = (unsigned)g * ns;
    const int first = (int)share_owner(gs / gran, U, pe);
    int step = 0, np0 = -1;
    for (int q = first; q < pe && share_begin(q, U, pe) * gran < gs + ns; ++q) {
      int s0, nst, piece, np;
      share_item(q, g, U, pe, gran, ns, &s0, &nst, &piece, &np);
      if (s0 != step || nst < 1 || nst > sps || piece != q - first || (np0 >= 0 && np != np0)) return -1;
      np0 = np;
      step += nst;
    }
    if (step != ns || np0 < 1) return -1;
    if (np0 > max_np) max_np = np0;
  }
  return max_np;
}

// kw (so rt = waves / kw tiles per row block) and the unit size (one block-step, or one
// whole row block). Cost, in bytes of the busiest workgroup: its weight bytes (a tile step is
// 2 KB in every executor format), a fixed charge per item, and one extra dependency trip
// when row blocks are cut into pieces.
bool plan_projection(const FmtInfo& fi, int mode, int m, int n, int k, int P, int waves, int force_kw,
                     int lds_limit, bool ring, StackPlan& out) {
  // Where every wave loads its own weights, an item costs about one memory round trip more
  // than its bytes (staging, epilogue) and a cut row block one more dependency trip: ~4 us,
  // ~128 KB of one workgroup's stream. With loader waves the stream does not stop for either:
  // an item costs its barriers and epilogue (~1 us), a cut row block the reducer's wait; and
  // every workgroup streams all the time, so a projection is spread over all of them (the
  // same workgroups would otherwise carry the extra work in every layer).
  const double kStepBytes = 2048.0, kItemBytes = ring ? 24576.0 : 131072.0, kPieceBytes = ring ? 49152.0 : 98304.0;
  const int ns = k / fi.kstep;
  const int ntiles = n / 16;
  double best = 1e300;
  bool found = false;
  for (int kw = 1; kw <= waves; kw *= 2) {
    if (force_kw && kw != force_kw) continue;
    const int rt = waves / kw;
    const int groups = (ntiles + rt - 1) / rt;
    for (int whole = 0; whole < 2; ++whole) {
      const int gran = whole ? ns : 1;
      const long long U = (long long)groups * ns / gran;
      if ((U + 1) * (P + 1) >= (1LL << 31) || U * gran >= (1LL << 31)) continue;  // 32-bit share math
      // Fewer workgroups than P give bigger shares: fewer pieces per row block, more LDS;
      // with fewer block-steps than workgroups, a few pieces per row block.
      long long cand[8];
      int nc = 0;
      for (int div = 1; div <= (ring ? 1 : 8); div *= 2) cand[nc++] = U < P / div ? U : P / div;
      for (int np = 2; np <= kMaxPieces; ++np) cand[nc++] = !whole && groups * np < U ? (long long)groups * np : 0;
      for (int ci = 0; ci < nc; ++ci) {
        const int pe = (int)cand[ci];
        bool seen = false;
        for (int cj = 0; cj < ci; ++cj) seen |= cand[cj] == cand[ci];
        if (pe < 1 || pe > P || seen) continue;
        const long long per = (U + pe - 1) / pe * gran;  // most block-steps of one workgroup
        const int sps = (int)(per < ns ? per : ns);
        qlx_plan p = {};
        p.mode = mode;
        p.waves = waves;
        p.kw = kw;
        p.rw = 1;
        p.splits = ns / sps;  // layout() then sizes LDS for ceil(ns / splits) >= sps steps
        GemmArgs a = {};
        const int lds = exec_lds(fi, p, m, n, k, a);
        if (a.sps < sps || lds > lds_limit) continue;
        const int max_np = check_shares(groups, ns, (int)U, pe, gran, sps);
        if (max_np < 1 || max_np > kMaxPieces) continue;
        const long long items = whole ? per / ns : (per + ns - 1) / ns + 1;
        const double cost = (double)per * rt * kStepBytes + items * kItemBytes + (max_np > 1 ? kPieceBytes : 0.0);
        if (cost < best) {
          best = cost;
          found = true;
          out.plan = p;
          out.units = (int)U;
          out.pe = pe;
          out.gran = gran;
          out.sps = a.sps;
          out.max_np = max_np;
        }
      }
    }
  }
  return found;
}

bool overlaps(const void* a, long long na, const void* b, long long nb) {
  const char* x = static_cast<const char*>(a);
  const char* y = static_cast<const char*>(b);
  return x < y + nb && y < x + na;
}

}  // namespace qlx

using namespace qlx;

extern "C" {

int qlx_stack_desc_size(void) { return (int)sizeof(StackDesc); }

int qlx_stack_build(int fmt, int m, const qlx_stack_call* calls, int ncalls, int waves, int groups_per_cu,
                    int loaders, int ring_chunks, void* desc, qlx_plan* plans, void* arena,
                    long long* arena_bytes, qlx_stack_launch* launch) {
  QLX_REQUIRE(stack_fn_for(fmt, 8, false) != nullptr,
              "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(waves == 4 || waves == 8, "waves must be 4 or 8 (got %d)", waves);
  QLX_REQUIRE(m >= 1 && m <= 16, "the decode executor serves m = 1..16 (got %d)", m);
  QLX_REQUIRE(calls != nullptr && ncalls >= 1, "no projections");
  QLX_REQUIRE(groups_per_cu >= 1 && groups_per_cu <= 4, "groups_per_cu must be 1..4");
  QLX_REQUIRE(loaders == -1 || loaders == 0 || loaders == 4 || loaders == 6, "loaders must be -1, 0, 4 or 6 (got %d)",
              loaders);
  QLX_REQUIRE(ring_chunks == 0 || (ring_chunks >= kRingMinChunks && (ring_chunks & (ring_chunks - 1)) == 0),
              "ring_chunks must be 0 or a power of two >= %d (got %d)", kRingMinChunks, ring_chunks);
  if (loaders < 0) loaders = groups_per_cu == 1 ? (waves == 4 ? 6 : 4) : 0;
  QLX_REQUIRE(loaders == 0 || (ring_shape_ok(waves, loaders) && groups_per_cu == 1),
              "loader waves: 4 compute waves with 4 or 6 loaders, or 8 with 4, and one lane (waves=%d, loaders=%d, "
              "groups_per_cu=%d)", waves, loaders, groups_per_cu);
  const FmtInfo fi = stack_info(fmt);
  // Shapes, and which earlier projection (if any) produces each activation. Outputs may not
  // overlap each other or an activation read from memory: the chain has no ordering between
  // projections other than these data dependencies.
  std::vector<int> src(ncalls, -1), published(ncalls, 0);
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    QLX_REQUIRE(q.kw == 0 || q.kw == 1 || q.kw == 2 || q.kw == 4 || q.kw == 8,
                "projection %d: kw must be 0 (planner) or 1, 2, 4, 8", c);
    QLX_REQUIRE(q.n >= 16 && q.n % 16 == 0 && q.k > 0 && q.k % fi.kstep == 0,
                "projection %d: n=%d k=%d do not fit the tiled format", c, q.n, q.k);
    QLX_REQUIRE(q.mode == QLX_MODE_BF16 || q.mode == QLX_MODE_SWIGLU, "projection %d: mode %d", c, q.mode);
    QLX_REQUIRE(q.w && q.w_scale && q.x && q.y, "projection %d: NULL pointer", c);
  }
  auto nout = [&](int c) { return calls[c].mode == QLX_MODE_SWIGLU ? calls[c].n / 2 : calls[c].n; };
  for (int c = 0; c < ncalls; ++c) {
    const long long ybytes = 2LL * m * nout(c);
    for (int j = 0; j < ncalls; ++j) {
      if (j != c) QLX_REQUIRE(!overlaps(calls[c].y, ybytes, calls[j].y, 2LL * m * nout(j)),
                              "outputs of projections %d and %d overlap", c, j);
    }
    const long long xbytes = 2LL * m * calls[c].k;
    for (int j = 0; j < ncalls; ++j) {
      if (calls[c].x == calls[j].y && j < c && calls[c].k <= nout(j)) {
        src[c] = j;
        published[j] = 1;
        break;
      }
    }
    if (src[c] < 0)
      for (int j = 0; j < ncalls; ++j)
        QLX_REQUIRE(!overlaps(calls[c].x, xbytes, calls[j].y, 2LL * m * nout(j)),
                    "projection %d reads memory that projection %d writes (only the whole output of an "
                    "earlier projection can be an input)", c, j);
  }
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_status(e, "stack_build");
  std::vector<StackPlan> sp(ncalls);
  int lds = 0, lanes = groups_per_cu, desc_lds = -1;
  int ctl_off = 0, ring_off = 0, rchunks = 0;
  const int P = cus;  // workgroups per lane
  const long long desc_bytes = (long long)ncalls * sizeof(StackDesc);
  // Plan for P workgroups, then shrink P to what fits the CUs with that LDS; repeat until
  // plan and grid agree.
  // Item LDS may take what the weight ring (at least 32 slots, or the requested size) leaves.
  const int item_limit =
      loaders ? kLdsLimit - kCtlBytes - 1024 - (ring_chunks ? ring_chunks : kRingMinChunks) * 1024 : kLdsLimit;
  for (int round = 0;; ++round) {
    QLX_REQUIRE(round < 4, "no stable executor grid");
    int items_lds = 0;
    for (int c = 0; c < ncalls; ++c) {
      const qlx_stack_call& q = calls[c];
      QLX_REQUIRE(plan_projection(fi, q.mode, m, q.n, q.k, P, waves, q.kw, item_limit, loaders > 0, sp[c]),
                  "projection %d: no executor plan for n=%d k=%d", c, q.n, q.k);
      GemmArgs a = {};
      const int l = exec_lds(fi, sp[c].plan, m, q.n, q.k, a);
      if (l > items_lds) items_lds = l;
    }
    items_lds = (items_lds + 15) & ~15;
    const void* fn = nullptr;
    if (loaders == 0) {
      desc_lds = items_lds + desc_bytes <= kLdsLimit ? items_lds : -1;
      lds = desc_lds >= 0 ? (int)(items_lds + desc_bytes) : items_lds;
      fn = stack_fn_for(fmt, waves, desc_lds >= 0);
    } else {
      // [items][counters][ring][descriptors, if the ring keeps >= 32 slots beside them]
      ctl_off = items_lds;
      ring_off = (ctl_off + kCtlBytes + 1023) & ~1023;
      auto fit = [&](long long room) {
        int r = 0;
        for (int c = kRingMinChunks; (long long)c * 1024 <= room; c *= 2) r = c;
        return ring_chunks ? (ring_chunks * 1024LL <= room ? ring_chunks : 0) : r;
      };
      // Descriptors go to LDS only beside a ring of 128 slots (or the requested size): a
      // deeper ring hides longer dependency waits than descriptor reads cost.
      rchunks = fit(kLdsLimit - ring_off - desc_bytes);
      desc_lds = rchunks >= (ring_chunks ? ring_chunks : 128) ? ring_off + rchunks * 1024 : -1;
      if (desc_lds < 0) rchunks = fit(kLdsLimit - ring_off);
      QLX_REQUIRE(rchunks >= kRingMinChunks, "the executor's weight ring does not fit beside %d bytes of item LDS",
                  items_lds);
      lds = ring_off + rchunks * 1024 + (desc_lds >= 0 ? (int)desc_bytes : 0);
      fn = ring_fn_for(fmt, waves, loaders, desc_lds >= 0);
    }
    if (lds > 64 * 1024) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) return hip_status(e, "stack_build");
    }
    int occ = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, (waves + loaders) * 64, lds);
    if (e != hipSuccess) return hip_status(e, "stack_build");
    QLX_REQUIRE(occ >= 1, "the executor does not fit a CU with %d bytes of LDS", lds);
    if (occ >= lanes) break;
    lanes = occ;
  }
  // Arena: published outputs and partial sums, 256-byte aligned regions.
  long long off = 0;
  std::vector<long long> wire_off(ncalls, -1), part_off(ncalls, -1);
  for (int c = 0; c < ncalls; ++c) {
    if (published[c]) {
      wire_off[c] = off;
      off += ((8LL * m * (nout(c) / 2)) + 255) & ~255LL;
    }
    if (sp[c].max_np > 1) {
      part_off[c] = off;
      off += ((8LL * (sp[c].max_np - 1) * m * calls[c].n) + 255) & ~255LL;
    }
  }
  StackDesc* out = reinterpret_cast<StackDesc*>(desc);
  int rot = 0;  // each projection's shares start where the previous projection's ended
  if (out) QLX_REQUIRE(arena != nullptr || off == 0, "the chain needs an arena of %lld bytes", off);
  char* base = static_cast<char*>(arena);
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    StackDesc d = {};
    d.a.w = q.w;
    d.a.ws = q.w_scale;
    d.a.x = q.x;
    d.a.y = q.y;
    d.a.tiled = 1;
    d.off_red = (layout(fi, sp[c].plan, m, q.n, q.k, d.a) + 15) & ~15;
    d.a.splits = sp[c].max_np;
    if (base) {
      d.ywire = wire_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + wire_off[c]) : nullptr;
      d.part = part_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + part_off[c]) : nullptr;
      d.xwire = src[c] >= 0 ? reinterpret_cast<uint64_t*>(base + wire_off[src[c]]) : nullptr;
      d.xpitch = src[c] >= 0 ? nout(src[c]) / 2 : 0;
    }
    d.units = sp[c].units;
    d.nwg = P;
    d.rot = rot;
    rot = (rot + sp[c].pe) % P;
    d.pe = sp[c].pe;
    d.gran = sp[c].gran;
    d.sw = q.mode == QLX_MODE_SWIGLU;
    if (out) out[c] = d;
    if (plans) {
      plans[c] = sp[c].plan;
      plans[c].splits = sp[c].max_np;
      plans[c].workspace = nullptr;
      plans[c].tickets = nullptr;
    }
  }
  if (arena_bytes) *arena_bytes = off;
  if (launch) {
    launch->grid = P * lanes;
    launch->lanes = lanes;
    launch->lds_bytes = lds;
    launch->waves = waves;
    launch->desc_lds = desc_lds;
    launch->loaders = loaders;
    launch->ring_off = ring_off;
    launch->ring_chunks = rchunks;
    launch->ctl_off = ctl_off;
    launch->inflight = loaders ? kLoaderDepth : 0;
  }
  return QLX_OK;
}

int qlx_stack_run(int fmt, const void* desc, int ncalls, const qlx_stack_launch* launch, unsigned epoch,
                  int* error, long long budget_us, void* stream) {
  QLX_REQUIRE(launch != nullptr && (launch->waves == 4 || launch->waves == 8) && launch->grid >= 1,
              "bad executor launch configuration");
  const int loaders = launch->loaders;
  QLX_REQUIRE(loaders == 0 || ring_shape_ok(launch->waves, loaders), "bad executor loaders");
  const void* fn = loaders ? ring_fn_for(fmt, launch->waves, loaders, launch->desc_lds >= 0)
                           : stack_fn_for(fmt, launch->waves, launch->desc_lds >= 0);
  QLX_REQUIRE(fn != nullptr, "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(desc && error && ncalls >= 1, "bad executor arguments");
  QLX_REQUIRE(launch->desc_lds < 0 || launch->desc_lds + (long long)ncalls * (long long)sizeof(StackDesc) <=
                                          launch->lds_bytes,
              "descriptor copy does not fit the launch's LDS");
  QLX_REQUIRE(epoch != 0, "epoch 0 is reserved (a zeroed arena carries it)");
  QLX_REQUIRE(budget_us >= 0 && budget_us <= 600000000LL, "budget_us must be 0..600e6");
  long long ticks = budget_us * 100;  // the real-time counter runs at 100 MHz
  int desc_off = launch->desc_lds, lanes = launch->lanes;
  QLX_REQUIRE(lanes >= 1 && launch->grid % lanes == 0, "bad executor lanes");
  if (loaders) {
    const int rc = launch->ring_chunks, ctl = launch->ctl_off, ro = launch->ring_off;
    QLX_REQUIRE(lanes == 1 && rc >= kRingMinChunks && (rc & (rc - 1)) == 0 && ctl >= 0 && ctl + kCtlBytes <= ro &&
                    ro % 1024 == 0 && (long long)ro + rc * 1024LL <= launch->lds_bytes &&
                    (launch->desc_lds < 0 || launch->desc_lds >= ro + rc * 1024),
                "bad ring executor launch configuration");
    uint32_t rmask = (uint32_t)rc - 1;
    int ctl_off = ctl, ring_off = ro;
    void* args[] = {(void*)&desc,     (void*)&ncalls,  (void*)&epoch,    (void*)&error, (void*)&ticks,
                    (void*)&desc_off, (void*)&ctl_off, (void*)&ring_off, (void*)&rmask};
    hipError_t e = hipLaunchCooperativeKernel(fn, dim3(launch->grid), dim3((launch->waves + loaders) * 64), args,
                                              (unsigned)launch->lds_bytes, (hipStream_t)stream);
    return hip_status(e, "stack_run");
  }
  void* args[] = {(void*)&desc, (void*)&ncalls, (void*)&epoch, (void*)&error, (void*)&ticks, (void*)&desc_off,
                  (void*)&lanes};
  hipError_t e = hipLaunchCooperativeKernel(fn, dim3(launch->grid), dim3(launch->waves * 64), args,
                                            (unsigned)launch->lds_bytes, (hipStream_t)stream);
  return hip_status(e, "stack_run");
}

}  // extern "C"
