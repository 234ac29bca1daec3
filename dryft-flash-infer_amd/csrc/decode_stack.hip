// Decode-step executor: every quantized projection of a decode step in one launch.
//
// The reference runs each projection as its own CUDA launch inside a graph and hides the
// launch gap with programmatic dependent launch: a GEMM's weight loads start while the
// previous kernel drains (engine/kernels/cuda_fp8.py:47-50, 150-169, 252;
// engine/kernels/cuda_jit.py:218-262). HIP has no such launch attribute, and at M = 1 most
// projections are 5-25 MB, so per-launch latency (launch, first loads, activation staging,
// epilogue) costs as much as the weight stream itself.
//
// Here one launch runs the whole chain on `lanes` sets of workgroups, one
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
//     Every run has a new nonzero epoch, so words left by earlier runs never match. The
//     epoch lives in the arena's first words, one per workgroup: each workgroup reads the
//     last run's at its start, uses the next one and stores it at its end. Every workgroup
//     runs every run, so all of them hold the same epoch, and none waits at its end for a
//     shared counter. The launch takes no per-run argument, so a run captures into a HIP graph
//     and every replay is a new run.
//   * Every wait is bounded by a per-run deadline on the 100 MHz real-time counter: a wait
//     past it sets the error flag and moves on (that run's outputs are undefined), so the
//     kernel always ends. The grid is one workgroup per CU per lane and the planner checks
//     that this many fit the device at once (occupancy), so on an otherwise idle GPU every
//     workgroup is resident; where other work holds CUs, waits run out the deadline rather
//     than hang.
#include <vector>

#include "attn_common.h"
#include "exec_common.h"
#include "rope_common.h"

namespace qlx {

constexpr int kMaxPieces = 4;  // pieces of one row block (the reducer has all in flight)
constexpr int kMaxGrid = 1024;  // workgroups of one launch (one epoch word each)
constexpr long long kArenaCtlBytes = 4 * kMaxGrid;  // arena head: each workgroup's last run epoch

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
  int xpitch;       // words (values) per token row of xwire (the producer's n_out)
  int off_red;      // LDS byte offset of the waves' partial sums (apart from the staged x)
  int rot;          // workgroup p holds share (p - rot) mod nwg of this projection
  int nwg;          // workgroups per lane
  // FP8 chains: a published output also carries, per token and 16-row weight tile, the
  // largest magnitude of the tile's bf16 outputs (words {16-bit run tag, bf16}); a projection
  // reading it combines the xmax_n tiles of its k columns instead of reading whole rows for its
  // token scales. Token row mm, row block g, tile tl of the block: word
  // mm * pitch + g * kMaxLine + tl (each row block's words on a cache line of their own: one
  // workgroup writes them, and small stores of many workgroups into one line queue up).
  uint32_t* ymax;        // publish this projection's maxima here, or null
  const uint32_t* xmax;  // the producer's maxima, or null (read whole rows)
  int ymax_pitch;        // words per token row of ymax: row blocks x kMaxLine
  int xmax_pitch;        // the producer's ymax_pitch
  int xmax_n;            // the producer's tiles that make up this projection's k columns
  int xmax_rt;           // the producer's tiles per row block
  // Residual add + RMSNorm input stage (nw non-null): the input is
  // bf16(bf16(r * rsqrt(mean(r^2) + eps)) * nw) with r = bf16(resid + delta), delta the
  // published output xwire points at (if any), resid in memory (rmem) or published by an
  // earlier stage (rwire, [m][k] words). The workgroup holding row block 0 (piece 0) writes r
  // to rout and the input to nout (either may be null) and publishes r to rpub.
  const void* nw;
  const void* rmem;
  const uint64_t* rwire;
  void* rout;
  void* nout;
  uint64_t* rpub;
  float eps;
  // 0: a projection. 1: the splits of an attention stage, 2: their merge (see exec_attention;
  // GemmArgs fields hold that stage's parameters there).
  int kind;
};

constexpr int kMaxLine = 32;  // maxima words per row block: one 128-byte line
// The published maxima pay from 5 tokens on. Every item of a Qwen3-4B chain covers the whole
// K range, so below that one pass reads each row (token maxima and slice from the same
// registers) and the maxima only add work; beyond it the whole-row prologue reads x twice.
// Measured on the Qwen3-4B FP8 chain (us per step, without / with): M=1 1180 / 1319, M=2
// 1486 / 1568, M=4 2029 / 2027, M=8 3287 / 2918, M=16 5148 / 3928.
constexpr int kMaximaMinM = 4;
// FP8 projections below this many weight bytes run on half the workgroups in chains of at most
// kMaximaMinM tokens (the planner's loop says why): Qwen3-4B's qkv, o and down, not gate_up.
constexpr long long kHalfBytes = 32LL << 20;

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

// ---- work items --------------------------------------------------------------------------

// Weight steps in flight per wave: most workgroups' whole share of a decode projection
// (fewer for 4-bit weights, whose dequantization needs more registers). A chain whose row
// blocks are never cut into K pieces runs a kernel without the piece reduction, whose
// registers allow FP8 a deeper prefetch. Measured on the Qwen3-4B M=1 chain (us per step):
// FP8 1217 / 1223 / 1205 / 1203 / 1229 at 6 / 8 / 9 / 10 / 11 steps, and since its qkv, o and
// down run on half the workgroups (twice the share each) 1219 / 1148 / 1107 / 1089 / 1167 at
// 6 / 8 / 10 / 12 / 14 (12 spills 6 registers, 14 spills 25; M = 2 1572 / 1559 at 10 / 12,
// M = 4 2062-2070 / 2059-2064); W8A16 1383 / 1405 /
// 1400 at 6 / 7 / 8; W4A16 1224 / 1242 at 4 / 5. FP8 with the piece reduction (chains of
// more than 4 tokens) at 6 steps spilled 5 registers; at 4 it spills none (M = 8 / 16 chains
// 2411-2416 / 3541-3548 us at 6, 2386-2393 / 3518-3522 at 4 or 5); W4A16's at 4 spilled 14-20,
// at 3 none (M = 8 chain 1541-1543 us at 4, 1478 at 3, 1484-1485 at 2). The instance with
// attention stages (ATT) holds the attention path's registers too; the 36-layer one-launch
// step (8 / 4 splits) at 7 / 8 / 9 / 10 steps: FP8 1657 / 1612 / 1595 / 1627 us (with the
// halves 1493 at 9, 1535 at 11); W8A16 at 4 / 5 / 6 / 7: 1627 / 1651 / 1683 / 1723 (4 splits);
// W4A16 at 3 / 4 / 5: 1364 / 1369 / 1505.
template <class F, bool PIECES, bool ATT = false>
struct ExecDepth {
  static constexpr int PF = ATT ? 4 : 6;
};
template <bool ATT>
struct ExecDepth<FmtFP8, false, ATT> {
  static constexpr int PF = ATT ? 9 : 12;
};
template <bool ATT>
struct ExecDepth<FmtFP8, true, ATT> {
  static constexpr int PF = 4;
};
template <bool PIECES, bool ATT>
struct ExecDepth<FmtW4, PIECES, ATT> {
  static constexpr int PF = PIECES || ATT ? 3 : 4;
};

// Group scales a workgroup's threads hold for one item (formats with per-group scales): up
// to kScaleRegs pairs of bf16 values (a step's two groups) per thread, loaded with the weights
// instead of after staging (5 x 512 pairs: every Qwen3-4B item at M = 1).
constexpr int kScaleRegs = 5;

struct ExecItem {
  int tg, s, np, step0, nst, wt, kwi, my, last, wrow;
  uint32_t scb;  // the per-row scale's bf16 bits, converted only when staged
  bool scpre;    // the item's group scales are in scw (else staged from memory)
  uint32_t scw[kScaleRegs];  // group scale pairs (bf16 bits), slot q = tid + u * threads
};

// Issue the wave's first PF weight steps (and the per-row scale) of a work
// item. A wave without steps in the item (my == 0) loads nothing.
template <class F, int WAVES, bool PIECES, int PF>
__device__ __forceinline__ void exec_prefetch(const GemmArgs& a, int tg, int step0, int nst, int s, int np,
                                              ExecItem& it, uint4 (&buf)[PF][F::LOADS]) {
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
  it.scpre = false;
  if constexpr (F::NSC == 0) {
    const int rl = threadIdx.x, tile = tg * a.rt + (rl >> 4);
    if (rl < 16 * a.rt && tile < a.ntiles)
      it.scb = gmem(reinterpret_cast<const uint16_t*>(a.ws))[weight_row(a, tile, rl & 15)];
  } else {
    // Group scales of the item, a step's two per 4-byte load: slot q is step q >> lg, row
    // q & (rows - 1) (rows = 16 rt, a power of two: a shift and a mask, no division).
    const int rows = 16 * a.rt, lg = __builtin_ctz(rows), total = nst * rows;
    it.scpre = total <= kScaleRegs * WAVES * 64;
    if (it.scpre) {
#pragma unroll
      for (int u = 0; u < kScaleRegs; ++u) {
        const int q = threadIdx.x + u * WAVES * 64;
        const int rl = q & (rows - 1), tile = tg * a.rt + (rl >> 4);
        it.scw[u] = 0u;
        if (q < total && tile < a.ntiles) it.scw[u] = F::scale_pair(a, weight_row(a, tile, rl & 15), step0 + (q >> lg));
      }
    }
  }
#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (p < it.my) load_chunk<F>(buf[p], a, it.wrow, step0 + it.kwi + p * a.kw, lane);
}

// The team of an executor workgroup's waves (threads 0 .. 64 WAVES - 1): they stream weights,
// stage activations, run the MFMAs and the epilogue.
template <int WAVES>
struct ComputeTeam {
  __device__ int tid() const { return threadIdx.x; }
  __device__ int size() const { return WAVES * 64; }
  __device__ void sync() const { __syncthreads(); }
};

// The producer's published per-token maxima an FP8 item combines (StackDesc.xmax), or none.
struct MaxIn {
  const uint32_t* p;
  int pitch, n, rt;
};

// FP8 prologue of a published activation whose producer also published per-token maxima of
// each weight tile's outputs: the token maxima are combined from those n words per token, so
// the item reads only its slice of x. They are maxima of the same bf16 values, so the token
// scales and codes equal those of the whole-row prologue (stage_fp8_act). When the slice fits
// one batch, its chunks are polled together with the first batch of maxima words (the last of
// them lands with the producer's last output). `amax` is zeroed.
template <class XS>
__device__ __forceinline__ void stage_fp8_maxima(const GemmArgs& a, const XS& xs, const MaxIn& mi, char* lds,
                                                 int step0, int nst, uint32_t* amax) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  constexpr int U_ = stage_unroll<XS, true>();
  constexpr int MW = 4;  // 16-byte loads of maxima words per thread in flight
  const int cps = nst * 16, total = a.m * cps;  // the slice's 8-value chunks
  const bool one_pass = total <= U_ * nthr;
  typename XS::Raw r[U_];
  auto first = [&](int u, int& mm, int& kabs) {
    const int q = tid + u * nthr;
    mm = q / cps;
    kabs = step0 * 128 + (q - mm * cps) * 8;
    return q < total;
  };
  unsigned sstale = 0;  // bit u: slice chunk u has not arrived
  if (one_pass) {
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      int mm, kabs;
      if (first(u, mm, kabs)) xs.fetch(a, mm, kabs, r[u]);
    }
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      int mm, kabs;
      if (first(u, mm, kabs) && !xs.ready(r[u])) sstale |= 1u << u;
    }
  }
  const __amdgpu_buffer_rsrc_t mrs = wire_rsrc(mi.p, (unsigned)a.m * (unsigned)mi.pitch * 4u);
  const uint32_t tag = wire_tag(xs.w.epoch);
  // 16-byte loads: per row block, per token row, in all
  const int lpb = (mi.rt + 3) >> 2, per = (mi.n + mi.rt - 1) / mi.rt * lpb, nl = a.m * per;
  auto word_ok = [&](const u32x4& v, int valid) {
    bool ok = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) ok &= e >= valid || (v[e] >> 16) == tag;
    return ok;
  };
  // Every thread takes the first round (its slice chunks are polled there), with or without
  // maxima words of its own.
  for (int l0 = tid; l0 == tid || l0 < nl; l0 += MW * nthr) {
    u32x4 mv[MW];
    unsigned off[MW];
    int valid[MW], tok[MW];
    unsigned stale = 0;
#pragma unroll
    for (int j = 0; j < MW; ++j) {
      const int q = l0 + j * nthr;
      tok[j] = q / per;
      const int c = q - tok[j] * per, blk = c / lpb, i4 = 4 * (c - blk * lpb);
      valid[j] = q < nl ? max(0, min(4, min(mi.rt - i4, mi.n - blk * mi.rt - i4))) : 0;
      off[j] = ((unsigned)tok[j] * mi.pitch + blk * kMaxLine + i4) * 4u;
      if (q < nl) mv[j] = wire_load16(mrs, off[j]);
    }
#pragma unroll
    for (int j = 0; j < MW; ++j)
      if (valid[j] && !word_ok(mv[j], valid[j])) stale |= 1u << j;
    while ((stale | sstale) && !xs.expired()) {
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int j = 0; j < MW; ++j)
        if (stale >> j & 1u) mv[j] = wire_load16(mrs, off[j]);
#pragma unroll
      for (int u = 0; u < U_; ++u) {
        int mm, kabs;
        if (sstale >> u & 1u) {
          first(u, mm, kabs);
          xs.refetch(a, mm, kabs, r[u]);
        }
      }
#pragma unroll
      for (int j = 0; j < MW; ++j)
        if ((stale >> j & 1u) && word_ok(mv[j], valid[j])) stale &= ~(1u << j);
#pragma unroll
      for (int u = 0; u < U_; ++u)
        if ((sstale >> u & 1u) && xs.ready(r[u])) sstale &= ~(1u << u);
    }
#pragma unroll
    for (int j = 0; j < MW; ++j) {
      if (!valid[j]) continue;
      uint32_t b = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < valid[j]) b = max(b, mv[j][e] & 0xffffu);
      atomicMax(&amax[tok[j]], b << 16);
    }
  }
  __syncthreads();
  float* sx = reinterpret_cast<float*>(lds + a.off_sx);
  auto token_scale = [&](int mm) { return fmaxf(__uint_as_float(amax[mm]) / 448.f, 1e-12f); };
  for (int i = tid; i < a.m; i += nthr) sx[i] = token_scale(i);
  if (one_pass) {
    settle_batch<XS, U_>(a, xs, r, first);  // arrived with the maxima (nothing left, but a run past its deadline)
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      int mm, kabs;
      if (first(u, mm, kabs))
        store_e4m3_chunk(lds + mm * a.xstride + (kabs - step0 * 128), xs.value(r[u]), token_scale(mm));
    }
    return;
  }
  for (int q0 = tid; q0 < total; q0 += U_ * nthr) {
    auto chunk = [&](int u, int& mm, int& kabs) {
      const int q = q0 + u * nthr;
      mm = q / cps;
      kabs = step0 * 128 + (q - mm * cps) * 8;
      return q < total;
    };
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      int mm, kabs;
      if (chunk(u, mm, kabs)) xs.fetch(a, mm, kabs, r[u]);
    }
    settle_batch<XS, U_>(a, xs, r, chunk);
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      int mm, kabs;
      if (chunk(u, mm, kabs))
        store_e4m3_chunk(lds + mm * a.xstride + (kabs - step0 * 128), xs.value(r[u]), token_scale(mm));
    }
  }
}

// Chunks of 8 values each thread holds through a pass of a norm stage. A token row's chunks
// take norm_row_slots(k) slots (k / 8 rounded up to whole waves, so the 64 slots of a wave in
// one round belong to one token); a pass takes as many whole rows as fit kNormU slots per
// thread (one row at least, checked on the host); more tokens take more passes.
constexpr int kNormU = 3;
__host__ __device__ inline int norm_row_slots(int k) { return ((k >> 3) + 63) & ~63; }
constexpr int kNormWpr = 8;  // wave sums of one token row read together (rows up to k = 4096)

// Token rows one pass of a norm stage takes.
__host__ __device__ inline int norm_pass_tokens(int m, int k, int u, int threads) {
  const int t = (u * threads) / norm_row_slots(k);
  return t < m ? t : m;
}

// LDS (doubles) a norm stage's wave sums and wave maxima take: one of each per wave and round.
__host__ __device__ inline int norm_lds_doubles(int waves) { return 2 * kNormU * waves; }

// Residual add + RMSNorm input stage of an item (see StackDesc.nw): every workgroup with work in
// the projection computes r and the normed input from the same words in the same order -- the
// sum of r^2 per token in fp64: per 8-value chunk, then per wave (wave_sum_last), then the
// waves in slot order; mean rounded to fp32, scale = 1 / sqrt(mean + eps) in fp32; input
// bf16(bf16(r * scale) * w) (norm.py:53-80, reference.py:13-28) -- and stages its slice of that
// input like any activation (FP8: quantized per token over the whole normed row, its maximum
// taken per wave the same way). The squares of bf16 values are exact in fp64 and their sums
// agree to the last fp64 bits in any order, below what rounding the mean to fp32 can see. The
// owner (row block 0) also writes r and the input and publishes r. Tokens t0 .. t0 + tn - 1
// (one pass); `css` holds norm_lds_doubles(waves) doubles.
template <class F, int U>
__device__ __forceinline__ void stage_norm_pass(const StackDesc& d, char* lds, int step0, int nst, double* css,
                                                bool owner, const Waits& w, int t0, int tn) {
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  const GemmArgs& a = d.a;
  const int tid = threadIdx.x, nthr = blockDim.x, lane = tid & 63, nw = nthr >> 6;
  const int cpr = a.k >> 3, cpw = norm_row_slots(a.k), slots = tn * cpw;
  const bool has_delta = d.xwire != nullptr, rwire = d.rwire != nullptr;
  const XWire dx(has_delta ? d.xwire : nullptr, has_delta ? d.xpitch : 0, a.m, w);
  const XWire rx(rwire ? d.rwire : nullptr, rwire ? a.k : 0, a.m, w);
  // Round u: slot q = tid + u * threads = 64 (u * waves + wave) + lane, token q / cpw, chunk
  // q % cpw (slots past the row's cpr chunks hold nothing).
  int tok[U], kab[U];
  bool on[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int q = tid + u * nthr;
    tok[u] = q / cpw;
    kab[u] = (q - tok[u] * cpw) * 8;
    on[u] = q < slots && kab[u] < a.k;
    tok[u] += t0;
  }
  auto chunk = [&](int u, int& mm, int& kabs) {
    mm = tok[u];
    kabs = kab[u];
    return on[u];
  };
  XWire::Raw rd[U], rr[U];
  uint4 rp[U], wv[U], rv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (on[u]) {
      if (has_delta) dx.fetch(a, tok[u], kab[u], rd[u]);
      if (rwire) {
        rx.fetch(a, tok[u], kab[u], rr[u]);
      } else {
        const u32x4 t = *gmem(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(d.rmem) +
                                                              (size_t)tok[u] * a.k + kab[u]));
        rp[u] = uint4{t[0], t[1], t[2], t[3]};
      }
      const u32x4 t = *gmem(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(d.nw) + kab[u]));
      wv[u] = uint4{t[0], t[1], t[2], t[3]};
    }
  }
  if (has_delta) settle_batch<XWire, U>(a, dx, rd, chunk);
  if (rwire) settle_batch<XWire, U>(a, rx, rr, chunk);
  const int wave = tid >> 6;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double ss = 0.0;
    rv[u] = uint4{0u, 0u, 0u, 0u};
    if (on[u]) {
      const uint4 x = rwire ? rx.value(rr[u]) : rp[u];
      uint4 r = x;
      if (has_delta) {
        const uint4 dv = dx.value(rd[u]);
        const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ds[4] = {dv.x, dv.y, dv.z, dv.w};
        uint32_t o[4], nan = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[i] = bf16_pair_hw(bf2f(xs[i] & 0xffffu) + bf2f(ds[i] & 0xffffu), bf2f(xs[i] >> 16) + bf2f(ds[i] >> 16));
          nan |= bf16_nan_bits(o[i]);
        }
        if (nan != 0u) {  // a NaN: the integer rounding's sign | 0x7FC0 form
#pragma unroll
          for (int i = 0; i < 4; ++i)
            o[i] = bf16_pair(bf2f(xs[i] & 0xffffu) + bf2f(ds[i] & 0xffffu), bf2f(xs[i] >> 16) + bf2f(ds[i] >> 16));
        }
        r = uint4{o[0], o[1], o[2], o[3]};
      }
      rv[u] = r;
      const uint32_t rs[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const double lo = bf2f(rs[i] & 0xffffu), hi = bf2f(rs[i] >> 16);
        ss += lo * lo;
        ss += hi * hi;
      }
    }
    ss = wave_sum_last(ss);
    if (lane == 63 && u * nthr < slots) css[u * nw + wave] = ss;
  }
  __syncthreads();
  // Each thread adds up the wave sums of its tokens, in slot order (entry e = u * waves + wave
  // covers slots 64 e .. 64 e + 63, all of one token; token t's are [t * wpr, (t + 1) * wpr)).
  // Up to kNormWpr of them are read together; longer rows (k > 4096) read the rest one by one.
  const int ne = min(U * nw, (slots + 63) >> 6), wpr = cpw >> 6;
  int e0[U], e1[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    e0[u] = (tok[u] - t0) * wpr;
    e1[u] = min(e0[u] + wpr, ne);
  }
  float scale[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    double v[kNormWpr], tot = 0.0;
#pragma unroll
    for (int i = 0; i < kNormWpr; ++i) v[i] = e0[u] + i < e1[u] ? css[e0[u] + i] : 0.0;
#pragma unroll
    for (int i = 0; i < kNormWpr; ++i)
      if (e0[u] + i < e1[u]) tot += v[i];
    for (int e = e0[u] + kNormWpr; e < e1[u]; ++e) tot += css[e];
    scale[u] = 1.0f / sqrtf((float)(tot / (double)a.k) + d.eps);
  }
  // The normed input (kept for the codes) and, for FP8, its largest magnitude per wave.
  uint4 yv[U];
  float mx[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t rs[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w}, ws2[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
    uint32_t o[4], nan = 0u;
    float m = 0.f;
    // bf16(bf16(r * scale) * w) by the hardware's pair conversion; a wave with a NaN anywhere
    // redoes its values with the integer rounding (same bits but for a NaN's).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = bf16_pair_hw(bf2f(rs[i] & 0xffffu) * scale[u], bf2f(rs[i] >> 16) * scale[u]);
      o[i] = bf16_pair_hw(bf2f(t & 0xffffu) * bf2f(ws2[i] & 0xffffu), bf2f(t >> 16) * bf2f(ws2[i] >> 16));
      nan |= bf16_nan_bits(t) | bf16_nan_bits(o[i]);
      m = fmaxf(m, fmaxf(fabsf(bf2f(o[i] & 0xffffu)), fabsf(bf2f(o[i] >> 16))));
    }
    if (nan != 0u) {
      m = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y0 = round_bf(round_bf(bf2f(rs[i] & 0xffffu) * scale[u]) * bf2f(ws2[i] & 0xffffu));
        const float y1 = round_bf(round_bf(bf2f(rs[i] >> 16) * scale[u]) * bf2f(ws2[i] >> 16));
        o[i] = bf16_pair(y0, y1);
        m = fmaxf(m, fmaxf(fabsf(y0), fabsf(y1)));
      }
    }
    yv[u] = uint4{o[0], o[1], o[2], o[3]};
    mx[u] = on[u] ? m : 0.f;
  }
  const int c0 = step0 * (F::KSTEP / 8), c1 = c0 + nst * (F::KSTEP / 8);  // the slice's chunks of a row
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!on[u]) continue;
    const int mm = tok[u], kabs = kab[u];
    if constexpr (!FP8) {
      const int kc = kabs >> 3;
      if (kc >= c0 && kc < c1)
        *reinterpret_cast<uint4*>(lds + mm * a.xstride + (kabs - step0 * F::KSTEP) * 2) = F::order(yv[u]);
    }
    if (owner) {
      const size_t e = (size_t)mm * a.k + kabs;
      if (d.rout) *gmem(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(d.rout) + e)) =
                      u32x4{rv[u].x, rv[u].y, rv[u].z, rv[u].w};
      if (d.nout) *gmem(reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(d.nout) + e)) =
                      u32x4{yv[u].x, yv[u].y, yv[u].z, yv[u].w};
      if (d.rpub) {
        const uint32_t rs2[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) wire_store_pair(d.rpub + (e >> 1) + i, rs2[i], w.epoch);
      }
    }
  }
  if constexpr (FP8) {  // the codes of the slice, at the token scales of the whole normed rows
    float* wm = reinterpret_cast<float*>(css + kNormU * 8);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float m = wave_max_last(mx[u]);
      if (lane == 63 && u * nthr < slots) wm[u * nw + wave] = m;
    }
    __syncthreads();
    float* sx = reinterpret_cast<float*>(lds + a.off_sx);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v[kNormWpr], m = 0.f;
#pragma unroll
      for (int i = 0; i < kNormWpr; ++i) v[i] = e0[u] + i < e1[u] ? wm[e0[u] + i] : 0.f;
#pragma unroll
      for (int i = 0; i < kNormWpr; ++i) m = fmaxf(m, v[i]);
      for (int e = e0[u] + kNormWpr; e < e1[u]; ++e) m = fmaxf(m, wm[e]);
      const float ts = fmaxf(m / 448.f, 1e-12f);
      if (!on[u]) continue;
      if (kab[u] == 0) sx[tok[u]] = ts;
      const int kc = kab[u] >> 3;
      if (kc >= c0 && kc < c1) store_e4m3_chunk(lds + tok[u] * a.xstride + (kc - c0) * 8, yv[u], ts);
    }
  }
}


// The whole stage: its token rows in passes of norm_pass_tokens (one pass at M = 1..4 with
// k = 2560 and 8 waves). A pass's LDS sums are reused by the next after a barrier.
template <class F, int U>
__device__ __forceinline__ void stage_norm(const StackDesc& d, char* lds, int step0, int nst, double* css, bool owner,
                                           const Waits& w) {
  const int tpp = norm_pass_tokens(d.a.m, d.a.k, U, blockDim.x);
  for (int t0 = 0; t0 < d.a.m; t0 += tpp) {
    if (t0) __syncthreads();
    stage_norm_pass<F, U>(d, lds, step0, nst, css, owner, w, t0, min(tpp, d.a.m - t0));
  }
}

// Stage what the item needs in LDS and stream its weight steps through the MFMAs. With
// `reuse`, the activation slice (and its bias sums) staged for the previous item -- same
// projection, same steps -- is still in place. `amax` is the zeroed FP8 scratch of the token
// maxima (and, behind its 64 bytes, a norm stage's sums).
template <class F, int WAVES, bool PIECES, class XS, int PF>
__device__ __forceinline__ void exec_main(const GemmArgs& a, const XS& xs, char* lds, const ExecItem& it, bool reuse,
                                          uint4 (&buf)[PF][F::LOADS], f32x4 (&acc)[1][1],
                                          uint32_t* amax, const MaxIn& mi = {}, const StackDesc* nd = nullptr,
                                          const Waits* nw = nullptr) {
  constexpr bool FP8 = std::is_same<F, FmtFP8>::value;
  const int lane = threadIdx.x & 63;
  const int step0 = it.step0, nst = it.nst, kwi = it.kwi, my = it.my;
  if (!reuse) {
    if (nd) {  // a residual add + RMSNorm stage
      double* css = reinterpret_cast<double*>(reinterpret_cast<char*>(amax) + 64);
      const bool owner = it.tg == 0 && it.s == 0;
      if (a.m * norm_row_slots(a.k) <= (int)blockDim.x)  // one chunk per thread (every M = 1 stage)
        stage_norm<F, 1>(*nd, lds, step0, nst, css, owner, *nw);
      else
        stage_norm<F, kNormU>(*nd, lds, step0, nst, css, owner, *nw);
    } else if constexpr (FP8) {
      bool done = false;
      if constexpr (XS::POLLS) {
        if (mi.p) {
          stage_fp8_maxima(a, xs, mi, lds, step0, nst, amax);
          done = true;
        }
      }
      if (!done) stage_fp8_act(a, xs, lds, step0, nst, BlockTeam{}, amax);
    } else
      stage_bf16<F>(a, xs, lds, step0, nst);
  }
  if constexpr (F::NSC == 0) {
    // Read on every path, so the register is not left pending for the next item's prefetch.
    const float scv = bf2f(it.scb);
    if (threadIdx.x < 16 * a.rt) reinterpret_cast<float*>(lds + a.off_sc)[threadIdx.x] = scv;
  } else if (it.scpre) {
    const int rows = 16 * a.rt, lg = __builtin_ctz(rows), total = nst * rows;
    float* sc = reinterpret_cast<float*>(lds + a.off_sc);
#pragma unroll
    for (int u = 0; u < kScaleRegs; ++u) {
      const int q = threadIdx.x + u * WAVES * 64;
      const int rl = q & (rows - 1), st = q >> lg;
      if (q < total) {
        sc[(2 * st) * a.sc_stride + rl] = F::scale_of(it.scw[u] & 0xffffu);
        sc[(2 * st + 1) * a.sc_stride + rl] = F::scale_of(it.scw[u] >> 16);
      }
    }
  } else {
    stage_scales<F>(a, lds, it.tg, step0, nst, ComputeTeam<WAVES>{});
  }
  __syncthreads();
  // The token maxima are read (into the token scales) before that barrier: clear them for
  // the next staging, which the end-of-item barrier orders after this.
  if constexpr (FP8)
    if (threadIdx.x < 16) amax[threadIdx.x] = 0u;
  if constexpr (needs_bias_totals<F>()) {
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
// (piece 0). Outputs go to y and, when a later projection reads them, to ywire. With MAXIMA
// (FP8 chains) and d.ymax, the writer of each tile's outputs also
// publishes each token's largest magnitude among them.
template <class F, bool SW, bool PIECES, bool MAXIMA = false, class Team = BlockTeam>
__device__ __forceinline__ void exec_finish(const StackDesc& d, char* lds, const ExecItem& it,
                                            const f32x4 (&acc)[1][1], const Waits& w, const Team& team = {},
                                            bool guard = true) {
  const GemmArgs& a = d.a;
  char* red = lds + d.off_red;
  acc_to_lds<1, 1>(red, acc, team, guard);
  if constexpr (!PIECES) {
    if (!(MAXIMA && d.ymax)) {
      // One output value per thread, (tile, token, row) in thread order so that a row pair is
      // two neighbouring lanes: its kw partial sums read together (one LDS round trip) and
      // added in wave order, as tile_value adds them; the even lane takes its neighbour's
      // value by a DPP move and stores the pair.
      constexpr int RO = SW ? 8 : 16;  // output rows per tile
      const int m = a.m, kw = a.kw, per_tile = RO * m, total = a.rt * per_tile;
      const int nout = SW ? a.half : a.n;
      const float* rf = reinterpret_cast<const float*>(red);
      uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
      uint64_t* const ywire = d.ywire;
      for (int idx = team.tid(); idx < total; idx += team.size()) {
        const int tl = idx / per_tile, rem = idx - tl * per_tile;
        const int mm = rem / RO, r = rem - mm * RO;
        const int tile = it.tg * a.rt + tl;
        // partial (wave tl * kw + q, row, token mm): rf[((tl * kw + q) * 16 + row) * 16 + mm]
        const float* base = rf + ((tl * kw) * 16 + r) * 16 + mm;
        float pg[8], pu[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          pg[q] = q < kw ? base[q * 256] : 0.f;
          if constexpr (SW) pu[q] = q < kw ? base[q * 256 + 8 * 16] : 0.f;
        }
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (q < kw) {
            g += pg[q];
            if constexpr (SW) u += pu[q];
          }
        float o;
        if constexpr (SW)
          o = swiglu_bf(F::finish(a, lds, g, tl * 16 + r, mm), F::finish(a, lds, u, tl * 16 + r + 8, mm));
        else
          o = F::finish(a, lds, g, tl * 16 + r, mm);
        const float o1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(o), 0x101, 0xf, 0xf, false));
        if ((r & 1) == 0 && tile < a.ntiles) {
          const int oi = (SW ? 8 : 16) * tile + r;
          const uint32_t pair = bf16_pair(o, o1);
          *gmem(reinterpret_cast<uint32_t*>(y + (size_t)mm * nout + oi)) = pair;
          if (ywire) wire_store_pair(ywire + (size_t)mm * (nout >> 1) + (oi >> 1), pair, w.epoch);
        }
      }
      return;
    }
  }
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
    if (PIECES && np > 1) {
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
    if (d.ywire) wire_store_pair(d.ywire + (size_t)mm * (nout >> 1) + (oi >> 1), pair, w.epoch);
    if constexpr (MAXIMA) {
      if (d.ymax) {
        // The tile's pairs of this token are rows_out / 2 consecutive lanes (idx steps by whole
        // waves, and tiles and tokens by rows_out / 2), all active together: their largest
        // magnitude (fmaxf drops a NaN, as the staging's maxima do) goes out from the first.
        float mx = fmaxf(0.f, fmaxf(fabsf(bf2f(pair & 0xffffu)), fabsf(bf2f(pair >> 16))));
#pragma unroll
        for (int sh = 1; sh < rows_out / 2; sh <<= 1) mx = fmaxf(mx, __shfl_xor(mx, sh));
        if (nl == 0)
          __hip_atomic_store(gmem(d.ymax + (size_t)mm * d.ymax_pitch + it.tg * kMaxLine + tl),
                             (wire_tag(w.epoch) << 16) | (__float_as_uint(mx) >> 16), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// ---- attention stage ---------------------------------------------------------------------
//
// One token (m = 1, batch 1), head_dim 128, bf16 caches, G = n_q / n_kv = 4 query heads per KV
// head. The stage's parameters sit in the descriptor's GemmArgs: w, ws = cos, sin tables;
// resid, norm_w = q and k norm gains; res_out, normed = k and v caches; tickets = the position
// (int32); n = capacity; k = table rows; half = n_q; group = n_kv; splits = items per KV head;
// eps = the RMSNorm epsilon; the descriptor's eps = head_dim^-0.5 * log2(e). xwire = the
// published qkv row; part = the splits' partials, kAttnWords 64-bit words per (KV head, split,
// query row): the accumulator's 128 values, the maximum, the total.
constexpr int kAttnWords = 130;
constexpr int kAttnG = 4;  // query heads per KV head (query rows of an item)

// LDS of an attention item: the KV head's q/k/v values [6][128] bf16 (2 KB), then the waves'
// accumulators [waves][4][128] and their maxima and totals [waves][4] (fp32).
__host__ __device__ inline int attn_lds_bytes(int waves) { return 2048 + waves * kAttnG * 130 * 4 + 2 * waves * kAttnG * 4; }

// Splits item (KV head kvh, split part): poll the KV head's q, k, v words; head norm + RoPE of
// the 4 query heads and the key (rope_norm_rotate: the arithmetic of qlx_qkv_norm_rope); the item
// that reads the key's block writes k and v into the caches at the position; then S^T = K Q^T,
// the online softmax and P V over the item's blocks (block j = part + S (wave + waves i)), with
// the arithmetic of attn_kernel (the new key's values taken from LDS where its block was read
// from memory before they were written); the waves merged through LDS; the item's partials
// published.
template <int WAVES>
__device__ __forceinline__ void exec_attention(const StackDesc& d, char* lds, int item, const Waits& w) {
  const GemmArgs& a = d.a;
  const int S = a.splits, NQ = a.half, H = a.group, cap = a.n;
  const int kvh = item / S, part = item - kvh * S;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  uint16_t* hs = reinterpret_cast<uint16_t*>(lds);  // [6][128]: q heads 0..3, k, v of the KV head
  float* wacc = reinterpret_cast<float*>(lds + 2048);
  float* wm = wacc + WAVES * kAttnG * 128;
  float* wl = wm + WAVES * kAttnG;
  // Loads in the order they are needed (memory operations complete in order): the position,
  // the KV head's words (6 heads x 16 chunks of 8 values, one chunk per thread), this wave's
  // first block (its index does not depend on the position), then the rotation inputs.
  const int pos0 = *gmem(reinterpret_cast<const int*>(a.tickets));
  const XWire xs(d.xwire, d.xpitch, 1, w);
  XWire::Raw r;
  const int hsl = tid >> 4, c8 = tid & 15;
  const bool poll = tid < 96;
  const int col = (hsl < 4 ? (kvh * kAttnG + hsl) * 128 : (NQ + (hsl == 4 ? 0 : H) + kvh) * 128) + 8 * c8;
  if (poll) xs.fetch(a, 0, col, r);
  const int j1 = part + S * wv, jstep = S * WAVES;
  const size_t hb = (size_t)kvh * cap * 128;
  const KVSrc kv{a.res_out, a.normed, nullptr, nullptr};
  KVBlock<false> cur;
  if (32 * j1 < cap) cur.load(kv, hb, 32 * j1, cap, n, g);
  const int pos = __builtin_amdgcn_readfirstlane(pos0);
  const int end = min(pos + 1, cap);  // keys at or past end are live for no row
  const int nblk = end > 0 ? (end + 31) >> 5 : 0;
  const int nb = j1 < nblk ? (nblk - j1 + jstep - 1) / jstep : 0;
  // Rotation inputs of wave 0's lanes 8 h + j (h = 0..3: query heads, 4: the key).
  const bool in_table = pos >= 0 && pos < a.k;
  const int hr = min(lane >> 3, 4), jr = lane & 7;
  float cl[8], ch[8], sl[8], sh[8], gl[8], gh[8];
  if (wv == 0) {
    const size_t tp = (size_t)(in_table ? pos : 0) * 128;
    const uint16_t* cs = reinterpret_cast<const uint16_t*>(a.w) + tp;
    const uint16_t* sn = reinterpret_cast<const uint16_t*>(a.ws) + tp;
    unpack8(*gmem(reinterpret_cast<const u32x4*>(cs + 8 * jr)), cl);
    unpack8(*gmem(reinterpret_cast<const u32x4*>(cs + 64 + 8 * jr)), ch);
    unpack8(*gmem(reinterpret_cast<const u32x4*>(sn + 8 * jr)), sl);
    unpack8(*gmem(reinterpret_cast<const u32x4*>(sn + 64 + 8 * jr)), sh);
    const uint16_t* gain = reinterpret_cast<const uint16_t*>(hr < 4 ? a.resid : a.norm_w);
    unpack8(*gmem(reinterpret_cast<const u32x4*>(gain + 8 * jr)), gl);
    unpack8(*gmem(reinterpret_cast<const u32x4*>(gain + 64 + 8 * jr)), gh);
  }
  if (poll) {
    while (!xs.ready(r) && !xs.expired()) {
      __builtin_amdgcn_s_sleep(1);
      xs.refetch(a, 0, col, r);
    }
    const uint4 v = xs.value(r);
    *reinterpret_cast<u32x4*>(hs + hsl * 128 + 8 * c8) = u32x4{v.x, v.y, v.z, v.w};
  }
  __syncthreads();
  // The item holding the key's block (when the key is written at all) writes k and v.
  const bool writes = in_table && pos < cap;
  const bool owner = writes && ((pos >> 5) % S) == part;
  if (wv == 0) {
    float xl[8], xh[8], yl[8], yh[8];
    uint32_t ylp[4], yhp[4];
    unpack8(*reinterpret_cast<const u32x4*>(hs + hr * 128 + 8 * jr), xl);
    unpack8(*reinterpret_cast<const u32x4*>(hs + hr * 128 + 64 + 8 * jr), xh);
    rope_norm_rotate(xl, xh, gl, gh, cl, ch, sl, sh, a.eps, yl, yh, ylp, yhp);
    if (lane < 40) {
      u32x4 lo = u32x4{ylp[0], ylp[1], ylp[2], ylp[3]}, hi = u32x4{yhp[0], yhp[1], yhp[2], yhp[3]};
      if (!in_table) {  // outside the cos/sin table: the query reads as NaN
#pragma unroll
        for (int i = 0; i < 8; ++i) yl[i] = yh[i] = __builtin_nanf("");
        lo = pack8(yl);
        hi = pack8(yh);
      }
      if (hr < 4 || writes) {  // (a key that is not written leaves the cache's values in place)
        *reinterpret_cast<u32x4*>(hs + hr * 128 + 8 * jr) = lo;
        *reinterpret_cast<u32x4*>(hs + hr * 128 + 64 + 8 * jr) = hi;
      }
    } else if (lane < 56) {  // the value row, as the cache stores it (bf16 of its bf16 values)
      const int c = lane - 40;
      float f[8];
      unpack8(*reinterpret_cast<const u32x4*>(hs + 5 * 128 + 8 * c), f);
      *reinterpret_cast<u32x4*>(hs + 5 * 128 + 8 * c) = pack8(f);
    }
  }
  __syncthreads();
  if (owner && tid < 32) {  // k, then v: 16 chunks each
    const int which = tid >> 4, c = tid & 15;
    uint16_t* dst = reinterpret_cast<uint16_t*>(which ? a.normed : a.res_out) + hb + (size_t)pos * 128 + 8 * c;
    *gmem(reinterpret_cast<u32x4*>(dst)) = *reinterpret_cast<const u32x4*>(hs + (4 + which) * 128 + 8 * c);
  }
  // Query fragments: row n (query head G kvh + n for n < 4), dims kdim(s, g).
  u32x4 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    qf[s] = n < kAttnG ? *reinterpret_cast<const u32x4*>(hs + n * 128 + kdim<false>(s, g)) : u32x4{0u, 0u, 0u, 0u};
  const int lim = end;  // one token: every query row sees keys 0 .. pos
  float m = kNegInf, l = 0.f;
  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The block holding the key read the cache before the key was written: its values come from
  // LDS (the ones just written to the cache).
  auto patch = [&](KVBlock<false>& b, int kb) __attribute__((always_inline)) {
    if (!writes || pos < kb || pos >= kb + 32) return;
    const int o = pos - kb;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
      if (o == 16 * kt + n) {
#pragma unroll
        for (int s = 0; s < 4; ++s) b.k[kt][s] = *reinterpret_cast<const u32x4*>(hs + 4 * 128 + kdim<false>(s, g));
      }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (slot_key(g, j) == o) b.v[j] = *reinterpret_cast<const u32x4*>(hs + 5 * 128 + 8 * n);
  };
  auto compute = [&](const KVBlock<false>& b, int kb) __attribute__((always_inline)) {
    f32x4 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
        st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf8(b.kfrag(kt, s)), bf8(qf[s]), st[kt], 0, 0, 0);
    }
    float sc[8], bm = kNegInf;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + 16 * kt + 4 * g + i;
        sc[4 * kt + i] = key < lim ? st[kt][i] * d.eps : kNegInf;
        bm = fmaxf(bm, sc[4 * kt + i]);
      }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    const float mu = mn == kNegInf ? 0.f : mn;
    const float carry = ex2(m - mu);
    m = mn;
    float p[8], ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = ex2(sc[j] - mu);
      ps += p[j];
    }
    l = l * carry + ps;
    const u32x4 pf = u32x4{pack_bf(p[0], p[1]), pack_bf(p[2], p[3]), pack_bf(p[4], p[5]), pack_bf(p[6], p[7])};
    float cr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cr[i] = __shfl(carry, 4 * g + i, 64);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      f32x4 t = acc[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] *= cr[i];
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf8(pf), bf8(b.vfrag(c)), t, 0, 0, 0);
    }
  };
  auto run = [&](KVBlock<false>& b, int j) __attribute__((always_inline)) {
    const int kb = 32 * j;
    patch(b, kb);
    if (kb + 32 > end) b.zero_from(kb, end, g);
    compute(b, kb);
  };
  // One block in registers at a time (the executor's registers are its weight pipeline's): at
  // decode lengths a wave has one or two blocks, the first fetched at the item's start.
  for (int i = 0; i < nb; ++i) {
    if (i > 0) cur.load(kv, hb, 32 * (j1 + jstep * i), cap, n, g);
    run(cur, j1 + jstep * i);
  }
  // Merge the waves (maxima and totals, then each accumulator rescaled to the item's maximum,
  // summed over waves in order) and publish the item's partial of each query row.
  {
    float lt = l + __shfl_xor(l, 16, 64);
    lt = lt + __shfl_xor(lt, 32, 64);
    if (g == 0 && n < kAttnG) {
      wm[wv * kAttnG + n] = m;
      wl[wv * kAttnG + n] = lt;
    }
  }
  __syncthreads();
  if (g == 0) {  // rows 4 g + i = i: lanes 0..15 hold rows 0..3 of dims 8 n + c
#pragma unroll
    for (int i = 0; i < kAttnG; ++i) {
      float M = kNegInf;
#pragma unroll
      for (int q = 0; q < WAVES; ++q) M = fmaxf(M, wm[q * kAttnG + i]);
      const float f = wm[wv * kAttnG + i] == kNegInf ? 0.f : ex2(wm[wv * kAttnG + i] - M);
      float* dst = wacc + ((size_t)wv * kAttnG + i) * 128 + 8 * n;
#pragma unroll
      for (int c = 0; c < 8; ++c) dst[c] = acc[c][i] * f;
    }
  }
  __syncthreads();
  uint64_t* out = d.part + ((size_t)kvh * S + part) * kAttnG * kAttnWords;
  for (int idx = tid; idx < kAttnG * kAttnWords; idx += WAVES * 64) {
    const int row = idx / kAttnWords, e = idx - row * kAttnWords;
    float M = kNegInf;
#pragma unroll
    for (int q = 0; q < WAVES; ++q) M = fmaxf(M, wm[q * kAttnG + row]);
    float v;
    if (e < 128) {
      v = 0.f;
#pragma unroll
      for (int q = 0; q < WAVES; ++q) v += wacc[((size_t)q * kAttnG + row) * 128 + e];
    } else if (e == 128) {
      v = M;
    } else {
      v = 0.f;
#pragma unroll
      for (int q = 0; q < WAVES; ++q) {
        const float mq = wm[q * kAttnG + row];
        v += mq == kNegInf ? 0.f : wl[q * kAttnG + row] * ex2(mq - M);
      }
    }
    ll_store(out + idx, __float_as_uint(v), w.epoch);
  }
}

// Merge item: query row qr (query head qr of the token, KV head qr / 4): every split's partial
// polled, then combined as attn_merge_kernel does -- weights exp(max_s - max), weighted
// accumulators over weighted totals, splits in order -- and the row written to y and, for later
// projections, published.
template <int WAVES>
__device__ __forceinline__ void exec_merge(const StackDesc& d, int qr, const Waits& w) {
  const GemmArgs& a = d.a;
  const int S = a.splits, kvh = qr / kAttnG, row = qr - kvh * kAttnG;
  const int t = threadIdx.x;
  if (t >= 128) return;
  const uint64_t* base = d.part + ((size_t)kvh * S * kAttnG + row) * kAttnWords;
  constexpr int kMaxS = 4;  // splits polled together
  float M = kNegInf, L = 0.f, A = 0.f;
  for (int s0 = 0; s0 < S; s0 += kMaxS) {
    uint64_t av[kMaxS], mv[kMaxS], lv[kMaxS];
#pragma unroll
    for (int j = 0; j < kMaxS; ++j) {
      if (s0 + j >= S) continue;
      const uint64_t* p = base + (size_t)(s0 + j) * kAttnG * kAttnWords;
      av[j] = ll_load(p + t);
      mv[j] = ll_load(p + 128);
      lv[j] = ll_load(p + 129);
    }
    auto ok = [&](uint64_t x) { return (uint32_t)(x >> 32) == w.epoch; };
    while (true) {
      bool all = true;
#pragma unroll
      for (int j = 0; j < kMaxS; ++j)
        if (s0 + j < S && !(ok(av[j]) && ok(mv[j]) && ok(lv[j]))) all = false;
      if (all || ll_expired(w, kWaitInput)) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int j = 0; j < kMaxS; ++j) {
        if (s0 + j >= S) continue;
        const uint64_t* p = base + (size_t)(s0 + j) * kAttnG * kAttnWords;
        if (!ok(av[j])) av[j] = ll_load(p + t);
        if (!ok(mv[j])) mv[j] = ll_load(p + 128);
        if (!ok(lv[j])) lv[j] = ll_load(p + 129);
      }
    }
    float Mb = M;
#pragma unroll
    for (int j = 0; j < kMaxS; ++j)
      if (s0 + j < S) Mb = fmaxf(Mb, __uint_as_float((uint32_t)mv[j]));
    const float Mu = Mb == kNegInf ? 0.f : Mb;
    const float c = M == kNegInf ? 0.f : ex2(M - Mu);
    A *= c;
    L *= c;
#pragma unroll
    for (int j = 0; j < kMaxS; ++j) {
      const float mj = __uint_as_float((uint32_t)mv[j]);
      if (s0 + j >= S || mj == kNegInf) continue;
      const float f = ex2(mj - Mu);
      A += f * __uint_as_float((uint32_t)av[j]);
      L += f * __uint_as_float((uint32_t)lv[j]);
    }
    M = Mb;
  }
  const float o = A / L;
  const float o1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(o), 0x101, 0xf, 0xf, false));
  if ((t & 1) == 0) {
    const int oi = qr * 128 + t;
    const uint32_t pair = pack_bf(o, o1);
    *gmem(reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.y) + oi)) = pair;
    if (d.ywire) wire_store_pair(d.ywire + (oi >> 1), pair, w.epoch);
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

template <class F, int WAVES, bool PIECES, int PF>
__device__ __forceinline__ void prefetch_work(const StackDesc& d, int p, int g, ExecItem& it,
                                              uint4 (&buf)[PF][F::LOADS]) {
  int step0, nst, piece, np;
  share_item(share_slot(d, p), g, d.units, d.pe, d.gran, d.a.nsteps, &step0, &nst, &piece, &np);
  exec_prefetch<F, WAVES, PIECES>(d.a, g, step0, nst, piece, np, it, buf);
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

// ATT: the chain has attention stages (its own instance, so that chains without keep the
// projection path's registers and code unchanged).
template <class F, int WAVES, bool DLDS, bool PIECES, bool ATT = false>
__global__ void __launch_bounds__(WAVES * 64)
stack_kernel(const StackDesc* __restrict__ gcalls, int ncalls, uint32_t* ctl, int* err, long long budget_ticks,
             int desc_off, int lanes, int amax_off) {
  extern __shared__ __align__(16) char lds[];
  const int per_lane = gridDim.x / lanes;
  const int lane = blockIdx.x / per_lane, p = blockIdx.x - lane * per_lane;
  constexpr bool MAXIMA = std::is_same<F, FmtFP8>::value;  // published row-block maxima
  uint32_t* amax = reinterpret_cast<uint32_t*>(lds + amax_off);  // FP8 staging: per-token maxima
  if (threadIdx.x < 16) amax[threadIdx.x] = 0u;
  const StackDesc* calls = gcalls;
  if constexpr (DLDS) {
    const int n16 = ncalls * (int)(sizeof(StackDesc) / 16);
    const auto src = gmem(reinterpret_cast<const u32x4*>(gcalls));
    u32x4* dst = reinterpret_cast<u32x4*>(lds + desc_off);
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
    calls = reinterpret_cast<const StackDesc*>(lds + desc_off);
  }
  // This run's epoch: the next after this workgroup's last run's, skipping low 16 bits of 0
  // (the tag of a zeroed arena). Read after the descriptors, so that the first weight prefetch
  // (which needs them, not the epoch) does not wait for this device-scope load.
  uint32_t epoch = __hip_atomic_load(gmem(ctl + blockIdx.x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  if ((epoch & 0xffffu) == 0u) epoch += 1u;
  const Waits w{epoch, __builtin_amdgcn_s_memrealtime() + (unsigned long long)budget_ticks, err};
  __syncthreads();
  ExecItem cur, nxt;
  uint4 buf[ExecDepth<F, PIECES, ATT>::PF][F::LOADS];
  f32x4 acc[1][1];
  int nc = -1, ng = 0;
  int staged_c = -1, staged_step0 = -1, staged_nst = -1;  // activation slice now in LDS
  bool have = next_work(calls, ncalls, lanes, lane, p, nc, ng);
  if (have) {
    if (!ATT || calls[nc].kind == 0)
      prefetch_work<F, WAVES, PIECES>(calls[nc], p, ng, nxt, buf);
    else
      nxt.tg = ng;
  }
  while (have) {
    const int c = nc;
    const StackDesc& d = calls[c];
    cur = nxt;
    if (ATT && d.kind != 0) {  // an attention stage's item: its splits, or their merge
      // No weights are in flight for it: the registers of the weight pipeline are free.
#pragma unroll
      for (int q = 0; q < ExecDepth<F, PIECES, ATT>::PF; ++q)
#pragma unroll
        for (int j = 0; j < F::LOADS; ++j) buf[q][j] = uint4{0u, 0u, 0u, 0u};
      if (d.kind == 1)
        exec_attention<WAVES>(d, lds, cur.tg, w);
      else
        exec_merge<WAVES>(d, cur.tg, w);
      staged_c = -1;
      const NextItem after = find_next(calls, ncalls, lanes, lane, p, nc, ng);
      have = after.have;
      nc = after.c;
      ng = after.g;
      if (have) {
        if (calls[nc].kind == 0)
          exec_prefetch<F, WAVES, PIECES>(calls[nc].a, ng, after.step0, after.nst, after.piece, after.np, nxt, buf);
        else
          nxt.tg = ng;
      }
      __syncthreads();  // LDS is reused by the next item
      continue;
    }
    const bool reuse = staged_c == c && staged_step0 == cur.step0 && staged_nst == cur.nst;
    if (d.xwire && !d.nw)
      exec_main<F, WAVES, PIECES>(d.a, XWire(d.xwire, d.xpitch, d.a.m, w), lds, cur, reuse, buf, acc, amax,
                                  MaxIn{d.xmax, d.xmax_pitch, d.xmax_n, d.xmax_rt});
    else  // x in memory, or a norm stage (one call site: the kernel's code stays as small)
      exec_main<F, WAVES, PIECES>(d.a, XPlain{}, lds, cur, reuse, buf, acc, amax, MaxIn{}, d.nw ? &d : nullptr, &w);
    staged_c = c;
    staged_step0 = cur.step0;
    staged_nst = cur.nst;
    // Outputs first: later projections wait for them. Anything before them -- finding the
    // next item, issuing its loads (the stores would queue behind them) -- delays the chain
    // (measured: 60-160 us per decode step).
    if (d.sw) {
      exec_finish<F, true, PIECES, MAXIMA>(d, lds, cur, acc, w, ComputeTeam<WAVES>{}, false);
    } else {
      exec_finish<F, false, PIECES, MAXIMA>(d, lds, cur, acc, w, ComputeTeam<WAVES>{}, false);
    }
    const NextItem after = find_next(calls, ncalls, lanes, lane, p, nc, ng);
    have = after.have;
    nc = after.c;
    ng = after.g;
    if (have) {
      if (!ATT || calls[nc].kind == 0)
        exec_prefetch<F, WAVES, PIECES>(calls[nc].a, ng, after.step0, after.nst, after.piece, after.np, nxt, buf);
      else
        nxt.tg = ng;
    }
    __syncthreads();  // LDS is reused by the next item
  }
  // This run's epoch for this workgroup's next run (no wait: nothing here reads it back).
  if (threadIdx.x == 0) __hip_atomic_store(gmem(ctl + blockIdx.x), epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <class F, int WAVES>
const void* stack_fn2(bool dlds, bool pieces, bool att) {
  if (att)  // attention stages: chains without K pieces (one token)
    return pieces ? nullptr
                  : dlds ? reinterpret_cast<const void*>(&stack_kernel<F, WAVES, true, false, true>)
                         : reinterpret_cast<const void*>(&stack_kernel<F, WAVES, false, false, true>);
  if (pieces)
    return dlds ? reinterpret_cast<const void*>(&stack_kernel<F, WAVES, true, true>)
                : reinterpret_cast<const void*>(&stack_kernel<F, WAVES, false, true>);
  return dlds ? reinterpret_cast<const void*>(&stack_kernel<F, WAVES, true, false>)
              : reinterpret_cast<const void*>(&stack_kernel<F, WAVES, false, false>);
}

template <class F>
const void* stack_fn(int waves, bool dlds, bool pieces, bool att) {
  return waves == 8 ? stack_fn2<F, 8>(dlds, pieces, att) : stack_fn2<F, 4>(dlds, pieces, att);
}

// The kernel for a launch of `waves` (4 or 8) waves per workgroup: `pieces` when some row block
// of the chain is cut into K pieces, `att` when the chain has attention stages.
const void* stack_fn_for(int fmt, int waves, bool dlds, bool pieces, bool att = false) {
  if (waves != 4 && waves != 8) return nullptr;
  switch (fmt) {
    case QLX_FMT_W8A16: return stack_fn<FmtW8>(waves, dlds, pieces, att);
    case QLX_FMT_W4A16: return stack_fn<FmtW4>(waves, dlds, pieces, att);
    case QLX_FMT_FP8: return stack_fn<FmtFP8>(waves, dlds, pieces, att);
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
                     int lds_limit, StackPlan& out, double stage_bytes = 0.0) {
  // An item costs about one memory round trip more than its bytes (staging, epilogue) and a
  // cut row block one more dependency trip: ~4 us, ~128 KB of one workgroup's stream.
  const double kStepBytes = 2048.0, kItemBytes = 131072.0, kPieceBytes = 98304.0;
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
      for (int div = 1; div <= 8; div *= 2) cand[nc++] = U < P / div ? U : P / div;
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
        const double cost = (double)per * rt * kStepBytes + items * kItemBytes + (max_np > 1 ? kPieceBytes : 0.0) +
                            (double)per * stage_bytes;
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
                    void* desc, qlx_plan* plans, void* arena, long long* arena_bytes, qlx_stack_launch* launch) {
  return qlx_stack_build_step(fmt, m, calls, ncalls, nullptr, nullptr, waves, groups_per_cu, desc, plans, arena,
                              arena_bytes, launch);
}

int qlx_stack_build_normed(int fmt, int m, const qlx_stack_call* calls, int ncalls, const qlx_norm_input* norms,
                           int waves, int groups_per_cu, void* desc, qlx_plan* plans, void* arena,
                           long long* arena_bytes, qlx_stack_launch* launch) {
  return qlx_stack_build_step(fmt, m, calls, ncalls, norms, nullptr, waves, groups_per_cu, desc, plans, arena,
                              arena_bytes, launch);
}

int qlx_stack_build_step(int fmt, int m, const qlx_stack_call* calls, int ncalls, const qlx_norm_input* norms,
                         const qlx_stack_attention* attns, int waves, int groups_per_cu, void* desc,
                         qlx_plan* plans, void* arena, long long* arena_bytes, qlx_stack_launch* launch) {
  QLX_REQUIRE(stack_fn_for(fmt, 8, false, false) != nullptr,
              "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(waves == 4 || waves == 8, "waves must be 4 or 8 (got %d)", waves);
  QLX_REQUIRE(m >= 1 && m <= 16, "the decode executor serves m = 1..16 (got %d)", m);
  QLX_REQUIRE(calls != nullptr && ncalls >= 1, "no projections");
  QLX_REQUIRE(groups_per_cu >= 1 && groups_per_cu <= 4, "groups_per_cu must be 1..4");
  const FmtInfo fi = stack_info(fmt);
  auto normed = [&](int c) { return norms != nullptr && norms[c].norm_w != nullptr; };
  auto kind = [&](int c) { return attns != nullptr ? attns[c].kind : 0; };
  // Work items of an attention stage's entry: (KV head, split), or query rows for the merge.
  auto attn_items = [&](int c) { return kind(c) == 1 ? attns[c].n_kv * attns[c].splits : attns[c].n_q; };
  // Shapes, and which earlier projection (if any) produces each activation. Outputs may not
  // overlap each other or an activation read from memory: the chain has no ordering between
  // projections other than these data dependencies.
  std::vector<int> src(ncalls, -1), published(ncalls, 0), rsrc(ncalls, -1), rpublished(ncalls, 0);
  int css_doubles = 0;  // LDS of the widest norm stage's per-chunk sums
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    if (kind(c) != 0) {
      const qlx_stack_attention& at = attns[c];
      QLX_REQUIRE(kind(c) == 1 || kind(c) == 2, "entry %d: attention kind %d", c, kind(c));
      QLX_REQUIRE(m == 1, "entry %d: an attention stage takes one token (m = 1, got %d)", c, m);
      QLX_REQUIRE(at.n_kv >= 1 && at.n_q == kAttnG * at.n_kv, "entry %d: n_q must be %d x n_kv", c, kAttnG);
      QLX_REQUIRE(at.splits >= 1 && at.splits <= 64, "entry %d: splits must be 1..64", c);
      QLX_REQUIRE(at.capacity >= 1 && at.table_rows >= 1 && (long long)at.n_kv * at.capacity * 128 < (1ll << 40),
                  "entry %d: bad capacity or table rows", c);
      QLX_REQUIRE(at.q_norm_w && at.k_norm_w && at.cos && at.sin && at.positions && at.k_cache && at.v_cache,
                  "entry %d: NULL attention pointer", c);
      QLX_REQUIRE(q.n == at.n_q * 128 && q.mode == QLX_MODE_BF16, "entry %d: n must be n_q x 128, mode bf16", c);
      if (kind(c) == 1) {
        QLX_REQUIRE(q.x != nullptr && q.y == nullptr && q.k == (at.n_q + 2 * at.n_kv) * 128,
                    "entry %d: the splits read the qkv row (x, k = (n_q + 2 n_kv) x 128) and write no y", c);
        QLX_REQUIRE(c + 1 < ncalls && kind(c + 1) == 2, "entry %d: the splits must be followed by their merge", c);
        const qlx_stack_attention& mg = attns[c + 1];
        QLX_REQUIRE(mg.n_q == at.n_q && mg.n_kv == at.n_kv && mg.splits == at.splits && mg.capacity == at.capacity &&
                        mg.table_rows == at.table_rows && mg.q_norm_w == at.q_norm_w && mg.k_norm_w == at.k_norm_w &&
                        mg.cos == at.cos && mg.sin == at.sin && mg.positions == at.positions &&
                        mg.k_cache == at.k_cache && mg.v_cache == at.v_cache && mg.eps == at.eps &&
                        mg.scale == at.scale,
                    "entry %d: the merge's attention fields differ from its splits'", c + 1);
      } else {
        QLX_REQUIRE(c >= 1 && kind(c - 1) == 1, "entry %d: a merge must follow its splits", c);
        QLX_REQUIRE(q.x == nullptr && q.y != nullptr && q.k == 0, "entry %d: the merge writes y and reads no x", c);
      }
      QLX_REQUIRE(!normed(c), "entry %d: an attention stage has no norm stage", c);
      continue;
    }
    QLX_REQUIRE(q.kw == 0 || q.kw == 1 || q.kw == 2 || q.kw == 4 || q.kw == 8,
                "projection %d: kw must be 0 (planner) or 1, 2, 4, 8", c);
    QLX_REQUIRE(q.n >= 16 && q.n % 16 == 0 && q.k > 0 && q.k % fi.kstep == 0,
                "projection %d: n=%d k=%d do not fit the tiled format", c, q.n, q.k);
    QLX_REQUIRE(q.mode == QLX_MODE_BF16 || q.mode == QLX_MODE_SWIGLU, "projection %d: mode %d", c, q.mode);
    QLX_REQUIRE(q.w && q.w_scale && q.y && (normed(c) ? q.x == nullptr : q.x != nullptr),
                "projection %d: NULL pointer (x must be NULL exactly when the input is a norm stage)", c);
    if (normed(c)) {
      QLX_REQUIRE(norms[c].resid != nullptr, "projection %d: a norm stage needs its residual", c);
      QLX_REQUIRE(norm_row_slots(q.k) <= kNormU * waves * 64,
                  "projection %d: a norm stage takes k <= %d (one token row per pass; k=%d)", c, kNormU * waves * 64 * 8,
                  q.k);
      css_doubles = std::max(css_doubles, norm_lds_doubles(8));
    }
  }
  auto nout = [&](int c) {
    return kind(c) == 1 ? 0 : (calls[c].mode == QLX_MODE_SWIGLU ? calls[c].n / 2 : calls[c].n);
  };
  // memory a projection or a norm stage writes
  auto written = [&](const void* p, long long bytes) {
    for (int j = 0; j < ncalls; ++j) {
      if (overlaps(p, bytes, calls[j].y, 2LL * m * nout(j))) return true;
      if (normed(j) && norms[j].resid_out && overlaps(p, bytes, norms[j].resid_out, 2LL * m * calls[j].k)) return true;
      if (normed(j) && norms[j].normed_out && overlaps(p, bytes, norms[j].normed_out, 2LL * m * calls[j].k))
        return true;
    }
    return false;
  };
  // Everything the launch writes -- projection outputs, and the residual and normed input a
  // stage writes back -- must be disjoint: two writers of one range race, and a stage's
  // residual is looked up by the address an earlier stage wrote it to.
  struct Range { const void* p; long long bytes; int call; const char* what; };
  std::vector<Range> outs;
  for (int c = 0; c < ncalls; ++c) {
    outs.push_back({calls[c].y, 2LL * m * nout(c), c, "output"});
    if (normed(c) && norms[c].resid_out) outs.push_back({norms[c].resid_out, 2LL * m * calls[c].k, c, "resid_out"});
    if (normed(c) && norms[c].normed_out) outs.push_back({norms[c].normed_out, 2LL * m * calls[c].k, c, "normed_out"});
  }
  for (size_t a = 0; a < outs.size(); ++a)
    for (size_t b = a + 1; b < outs.size(); ++b)
      QLX_REQUIRE(!overlaps(outs[a].p, outs[a].bytes, outs[b].p, outs[b].bytes),
                  "the %s of projection %d and the %s of projection %d overlap", outs[a].what, outs[a].call,
                  outs[b].what, outs[b].call);
  for (int c = 0; c < ncalls; ++c) {
    if (normed(c)) {
      const qlx_norm_input& nd = norms[c];
      const long long rbytes = 2LL * m * calls[c].k;
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
      for (int j = c - 1; j >= 0; --j)  // resid_out ranges are disjoint: at most one matches
        if (normed(j) && norms[j].resid_out && nd.resid == norms[j].resid_out && calls[j].k == calls[c].k) {
          rsrc[c] = j;
          rpublished[j] = 1;
          break;
        }
      QLX_REQUIRE(rsrc[c] >= 0 || !written(nd.resid, rbytes),
                  "projection %d: the residual is memory the chain writes (only an earlier stage's resid_out can "
                  "be)", c);
      QLX_REQUIRE(!nd.resid_out || !overlaps(nd.resid_out, rbytes, nd.resid, rbytes),
                  "projection %d: resid_out overlaps the residual", c);
      continue;
    }
    if (kind(c) == 2) continue;  // reads its splits' partials
    const long long xbytes = 2LL * m * calls[c].k;
    for (int j = 0; j < ncalls; ++j) {
      if (kind(j) != 1 && calls[c].x == calls[j].y && j < c && calls[c].k <= nout(j)) {
        src[c] = j;
        published[j] = 1;
        break;
      }
    }
    if (src[c] < 0)
      QLX_REQUIRE(!written(calls[c].x, xbytes),
                  "projection %d reads memory the chain writes (only the whole output of an earlier projection "
                  "can be an input)", c);
    QLX_REQUIRE(kind(c) != 1 || (src[c] >= 0 && calls[c].k == nout(src[c])),
                "entry %d: the splits read the whole output of an earlier projection", c);
  }
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_status(e, "stack_build");
  std::vector<StackPlan> sp(ncalls);
  int lds = 0, lanes = groups_per_cu, desc_lds = -1, amax_off = 0;
  bool att = false;  // attention stages: the kernel instance with their items
  for (int c = 0; c < ncalls; ++c) att |= kind(c) != 0;
  const int P = cus;  // workgroups per lane
  QLX_REQUIRE(P >= 1 && (long long)P * lanes <= kMaxGrid, "%d CUs x %d lanes exceed %d workgroups", P, lanes, kMaxGrid);
  const long long desc_bytes = (long long)ncalls * sizeof(StackDesc);
  // Plan for P workgroups, then shrink P to what fits the CUs with that LDS; repeat until
  // plan and grid agree. LDS: [items][64 B of FP8 row maxima][descriptors, if they fit].
  bool pieces = false;  // some row block is cut into K pieces: the kernel with their reduction
  for (int round = 0;; ++round) {
    QLX_REQUIRE(round < 4, "no stable executor grid");
    int items_lds = 0;
    for (int c = 0; c < ncalls; ++c) {
      const qlx_stack_call& q = calls[c];
      if (kind(c) != 0) {  // attention items: whole items on as many workgroups
        sp[c] = StackPlan{};
        sp[c].plan.waves = waves;
        sp[c].plan.kw = 1;
        sp[c].plan.rw = 1;
        sp[c].plan.splits = 1;
        sp[c].units = attn_items(c);
        sp[c].pe = std::min(P, sp[c].units);
        sp[c].gran = 1;
        sp[c].sps = 1;
        sp[c].max_np = 1;
        if (kind(c) == 1) items_lds = std::max(items_lds, attn_lds_bytes(waves));
        continue;
      }
      // With published token maxima an FP8 item reads only its slice of a published input, 4
      // bytes per value and token, after the input arrives (the weights were prefetched while
      // it was awaited): the planner charges those bytes 4x a weight byte (measured on the
      // Qwen3-4B FP8 chain, us per step at M = 8 / 16 by the factor: none 2914 / 3932, 1x 2641 /
      // 3930, 2x 2642 / 3475, 3x 2462 / 3490, 4x 2412 / 3488, 6x 2422 / 3483).
      const bool slice_staged = fmt == QLX_FMT_FP8 && m > kMaximaMinM && src[c] >= 0 && !normed(c);
      const double stage_bytes = slice_staged ? 4.0 * 4.0 * fi.kstep * m : 0.0;
      // FP8 chains without published maxima: a projection of under kHalfBytes of weights is
      // planned on half the workgroups. Shares start where the previous projection's ended, so
      // two such projections in a row (qkv -> o, down -> the next qkv) run on disjoint halves,
      // and a consumer's poll never queues behind the weight prefetch its workgroup issued
      // right after producing (memory counters complete in order). Measured on the Qwen3-4B
      // chains, us per step, all workgroups / half: FP8 M=1 1175 / 1103, M=2 1610 / 1566, M=4
      // 2085 / 2054, the one-launch decode step with attention 1579 / 1488; 3/8 of them the
      // same, 3/4 no gain (the halves overlap), gate_up (50 MB) halved too 1789. W8A16 (1276 /
      // 1411) and W4A16 (1047 / 1165), whose items compute more after their input arrives, and
      // FP8 above kMaximaMinM tokens (2647 / 3097 at M=8) keep every workgroup.
      const bool half = fmt == QLX_FMT_FP8 && m <= kMaximaMinM && (long long)q.n * q.k < kHalfBytes;
      const int Pp = half ? std::max(1, P / 2) : P;
      QLX_REQUIRE(plan_projection(fi, q.mode, m, q.n, q.k, Pp, waves, q.kw, kLdsLimit - 64, sp[c], stage_bytes),
                  "projection %d: no executor plan for n=%d k=%d", c, q.n, q.k);
      GemmArgs a = {};
      const int l = exec_lds(fi, sp[c].plan, m, q.n, q.k, a);
      if (l > items_lds) items_lds = l;
    }
    amax_off = (items_lds + 15) & ~15;
    const int items_end = amax_off + 64 + 8 * css_doubles;  // FP8 row maxima, norm stages' sums
    desc_lds = items_end + desc_bytes <= kLdsLimit ? items_end : -1;
    lds = desc_lds >= 0 ? (int)(items_end + desc_bytes) : items_end;
    pieces = false;
    for (int c = 0; c < ncalls; ++c) pieces |= sp[c].max_np > 1;
    QLX_REQUIRE(!(att && pieces), "a chain with attention stages cannot cut row blocks into K pieces");
    const void* fn = stack_fn_for(fmt, waves, desc_lds >= 0, pieces, att);
    if (lds > 64 * 1024) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
      if (e != hipSuccess) return hip_status(e, "stack_build");
    }
    int occ = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, waves * 64, lds);
    if (e != hipSuccess) return hip_status(e, "stack_build");
    QLX_REQUIRE(occ >= 1, "the executor does not fit a CU with %d bytes of LDS", lds);
    if (occ >= lanes) break;
    lanes = occ;
  }
  // FP8 chains of more than kMaximaMinM tokens: a published output also
  // carries its per-token maxima per weight tile, and a projection reading it combines those of
  // its k columns instead of reading whole rows for its token scales.
  const bool maxima = fmt == QLX_FMT_FP8 && m > kMaximaMinM;
  auto tile_cols = [&](int c) { return calls[c].mode == QLX_MODE_SWIGLU ? 8 : 16; };  // outputs per tile
  auto max_pitch = [&](int c) {
    GemmArgs a = {};
    layout(fi, sp[c].plan, m, calls[c].n, calls[c].k, a);
    return a.tile_groups * kMaxLine;
  };
  auto max_rt = [&](int c) {
    GemmArgs a = {};
    layout(fi, sp[c].plan, m, calls[c].n, calls[c].k, a);
    return a.rt;
  };
  // Arena: published outputs (and their maxima) and partial sums, 256-byte aligned regions.
  long long off = kArenaCtlBytes;  // [0, 4 kMaxGrid): each workgroup's last run epoch
  std::vector<long long> wire_off(ncalls, -1), part_off(ncalls, -1), max_off(ncalls, -1), rpub_off(ncalls, -1);
  for (int c = 0; c < ncalls; ++c) {
    if (published[c]) {
      wire_off[c] = off;
      off += ((8LL * m * (nout(c) / 2)) + 255) & ~255LL;
      if (maxima) {
        QLX_REQUIRE(max_rt(c) <= kMaxLine, "projection %d: %d tiles per row block", c, max_rt(c));
        max_off[c] = off;
        off += (4LL * m * max_pitch(c) + 255) & ~255LL;
      }
    }
    if (kind(c) == 1) {  // the splits' partials: [n_kv][splits][4 rows][kAttnWords] words
      part_off[c] = off;
      off += (8LL * attns[c].n_kv * attns[c].splits * kAttnG * kAttnWords + 255) & ~255LL;
    }
    if (sp[c].max_np > 1) {
      part_off[c] = off;
      off += ((8LL * (sp[c].max_np - 1) * m * calls[c].n) + 255) & ~255LL;
    }
    if (rpublished[c]) {  // a norm stage's r, read by later stages
      rpub_off[c] = off;
      off += ((4LL * m * calls[c].k) + 255) & ~255LL;
    }
  }
  StackDesc* out = reinterpret_cast<StackDesc*>(desc);
  int rot = 0;  // each projection's shares start where the previous projection's ended
  if (out) QLX_REQUIRE(arena != nullptr || off == 0, "the chain needs an arena of %lld bytes", off);
  char* base = static_cast<char*>(arena);
  for (int c = 0; c < ncalls; ++c) {
    const qlx_stack_call& q = calls[c];
    if (kind(c) != 0) {
      const qlx_stack_attention& at = attns[c];
      StackDesc d = {};
      d.kind = kind(c);
      d.a.w = at.cos;
      d.a.ws = at.sin;
      d.a.resid = at.q_norm_w;
      d.a.norm_w = at.k_norm_w;
      d.a.res_out = at.k_cache;
      d.a.normed = at.v_cache;
      d.a.tickets = const_cast<int*>(at.positions);
      d.a.y = q.y;
      d.a.m = 1;
      d.a.n = at.capacity;
      d.a.k = at.table_rows;
      d.a.half = at.n_q;
      d.a.group = at.n_kv;
      d.a.splits = at.splits;
      d.a.eps = at.eps;
      d.a.nsteps = 1;
      d.a.tile_groups = sp[c].units;
      d.eps = at.scale * 1.4426950408889634f;  // scores pre-multiplied by log2(e): base-2 exponentials
      if (base) {
        d.part = reinterpret_cast<uint64_t*>(base + part_off[kind(c) == 1 ? c : c - 1]);
        if (kind(c) == 1) {
          d.xwire = reinterpret_cast<uint64_t*>(base + wire_off[src[c]]);
          d.xpitch = nout(src[c]);
        } else {
          d.ywire = wire_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + wire_off[c]) : nullptr;
        }
      }
      d.units = sp[c].units;
      d.nwg = P;
      d.rot = rot;
      rot = (rot + sp[c].pe) % P;
      d.pe = sp[c].pe;
      d.gran = 1;
      if (out) out[c] = d;
      if (plans) plans[c] = sp[c].plan;
      continue;
    }
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
      d.xpitch = src[c] >= 0 ? nout(src[c]) : 0;
      if (max_off[c] >= 0) {
        d.ymax = reinterpret_cast<uint32_t*>(base + max_off[c]);
        d.ymax_pitch = max_pitch(c);
      }
      const int j = src[c];
      if (j >= 0 && max_off[j] >= 0 && q.k % tile_cols(j) == 0) {
        d.xmax = reinterpret_cast<const uint32_t*>(base + max_off[j]);
        d.xmax_pitch = max_pitch(j);
        d.xmax_n = q.k / tile_cols(j);
        d.xmax_rt = max_rt(j);
      }
    }
    d.units = sp[c].units;
    if (normed(c)) {
      const qlx_norm_input& nd = norms[c];
      d.nw = nd.norm_w;
      d.eps = nd.eps;
      d.rout = nd.resid_out;
      d.nout = nd.normed_out;
      if (base) {
        if (rsrc[c] >= 0)
          d.rwire = reinterpret_cast<const uint64_t*>(base + rpub_off[rsrc[c]]);
        else
          d.rmem = nd.resid;
        d.rpub = rpub_off[c] >= 0 ? reinterpret_cast<uint64_t*>(base + rpub_off[c]) : nullptr;
      }
    }
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
    launch->amax_off = amax_off;
    launch->pieces = pieces ? 1 : 0;
    launch->attention = att ? 1 : 0;
  }
  return QLX_OK;
}

int qlx_stack_run(int fmt, const void* desc, int ncalls, const qlx_stack_launch* launch, void* arena, int* error,
                  long long budget_us, void* stream) {
  QLX_REQUIRE(launch != nullptr && (launch->waves == 4 || launch->waves == 8) && launch->grid >= 1 &&
                  launch->grid <= kMaxGrid,
              "bad executor launch configuration");
  QLX_REQUIRE(launch->pieces == 0 || launch->pieces == 1, "launch.pieces must be 0 or 1 (got %d)", launch->pieces);
  QLX_REQUIRE(launch->attention == 0 || launch->attention == 1, "launch.attention must be 0 or 1");
  const void* fn = stack_fn_for(fmt, launch->waves, launch->desc_lds >= 0, launch->pieces != 0, launch->attention != 0);
  QLX_REQUIRE(fn != nullptr, "the decode executor serves W8A16, W4A16 and FP8 W8A8 (format %d)", fmt);
  QLX_REQUIRE(desc && arena && error && ncalls >= 1, "bad executor arguments");
  QLX_REQUIRE(reinterpret_cast<uintptr_t>(arena) % 256 == 0, "the arena must be 256-byte aligned");
  QLX_REQUIRE(launch->desc_lds < 0 || launch->desc_lds + (long long)ncalls * (long long)sizeof(StackDesc) <=
                                          launch->lds_bytes,
              "descriptor copy does not fit the launch's LDS");
  QLX_REQUIRE(launch->amax_off >= 0 && launch->amax_off % 16 == 0 && launch->amax_off + 64 <= launch->lds_bytes,
              "bad executor LDS layout");
  QLX_REQUIRE(budget_us >= 0 && budget_us <= 600000000LL, "budget_us must be 0..600e6");
  long long ticks = budget_us * 100;  // the real-time counter runs at 100 MHz
  int desc_off = launch->desc_lds, lanes = launch->lanes, amax_off = launch->amax_off;
  QLX_REQUIRE(lanes >= 1 && launch->grid % lanes == 0, "bad executor lanes");
  uint32_t* ctl = static_cast<uint32_t*>(arena);
  void* args[] = {(void*)&desc,     (void*)&ncalls, (void*)&ctl,     (void*)&error,
                  (void*)&ticks,    (void*)&desc_off, (void*)&lanes, (void*)&amax_off};
  hipError_t e = hipLaunchKernel(fn, dim3(launch->grid), dim3(launch->waves * 64), args,
                                 (size_t)launch->lds_bytes, (hipStream_t)stream);
  return hip_status(e, "stack_run");
}

}  // extern "C"
