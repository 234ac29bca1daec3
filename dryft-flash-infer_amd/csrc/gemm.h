// Quantized skinny GEMM / GEMV for gfx950: y[m][n] = sum_k x[m][k] * deq(W)[n][k].
//
// One kernel skeleton serves every weight format; a small policy struct per format says
// how a wave loads its weight chunk, turns it into MFMA operands and applies scales.
//
// Work decomposition (decode shapes: m = 1..64, n = 2560..151936, k = 2560..9728):
//   * the weight is cut into 16-row tiles; a tile's k range is cut into "steps" of KSTEP
//     values, and one step of one tile is what a wave's lanes load in one 16-byte-per-lane
//     instruction (1 KB for 4-bit and 8-bit formats; 2 KB, two loads, for the reference's
//     8-bit tiles);
//   * a workgroup owns RT = (waves / kw) * rw consecutive tiles and one K slice of `sps`
//     steps. kw waves split the slice of one tile step by step (interleaved), rw is the
//     number of tiles each wave streams side by side so one activation fragment feeds rw
//     MFMAs;
//   * `splits` K slices of a row block are separate workgroups. The last one to finish
//     (a ticket counter per row block) sums the fp32 partials in slice order and writes
//     the output, so results do not depend on scheduling (engine/kernels/cuda_fp8.py:975
//     sums split-K planes in the same fixed order).
//
// MFMA operand layout (v_mfma_f32_16x16x32_{bf16,fp8}, v_mfma_i32_16x16x64_i8): lane l
// supplies A row (l & 15) and B column (l & 15) for the k chunk (l >> 4), and receives D
// rows 4*(l >> 4) + 0..3 of column (l & 15). A rows are weight rows, B columns are
// activation rows (tokens), so m <= 16 per fragment; lanes whose token index is past m
// read the last real token and their output column is dropped.
//
// The k order inside an MFMA is free as long as A and B agree, so the activation is staged
// into LDS in whatever order the weight chunk unpacks in ("B order"). Integer codes are
// turned into exact bf16 by the magic-number method (Kim et al., 2022: OR the code into
// the mantissa of 128.0 for 4-bit codes; v_cvt_f32_ubyte for bytes), which adds a bias
// per value. The bias times the activation sum is subtracted per scale group, computed by
// the same MFMA chain with the codes all at the bias, so zero weights cancel exactly.
#pragma once

#include "common.h"
#include "../../include/qlinear.h"

namespace qlx {

struct GemmArgs {
  const void* w;
  const void* ws;   // weight scales
  const void* x;    // activation (bf16, or int8 for FMT_INT8)
  const float* xs;  // activation scales (FMT_INT8)
  const void* x2;   // FMT_INT8 second (residual) activation component, or null
  const float* xs2;
  int comp;         // FMT_INT8 activation components (1 or 2)
  void* y;
  float* work;
  int* tickets;
  int m, n, k;
  int mode, splits, sps, nsteps;
  int ntiles, kw, rt, tile_groups;
  int group;         // FP8WO scale group
  int tiled;         // weight stored in tiles (see tile_offset; REF8: the reference's tiles)
  int half;          // SWIGLU: I = n / 2
  int xstride;       // LDS bytes per staged activation row
  int off_sc, off_xb, off_sx;  // LDS byte offsets (x region starts at 0)
  int sc_stride;     // floats per staged scale row ([step*nsc + j][16*rt])
  int xb_stride;     // floats per token in xb ([m][sps*nsc])
  int tblocks;       // skinny GEMM: 2 = two 32-token blocks in one launch (else 0)
  int off_red;       // persistent kernel: LDS offset of the waves' partial sums (apart from x)
  int off_bt;        // persistent kernel: LDS offset of the code-bias totals [step][group][MT][16]
  int off_ring;      // ring kernel: LDS offset of the waves' weight rings [wave][slot][LOADS KB]
  int pm;            // skinny GEMM token blocks: rows of a K-slice plane (the whole batch)
  // Fused residual add + RMSNorm (qlx_linear_add_norm): y receives delta = bf16(x W^T)
  // with device-coherent stores; the workgroup that completes the last row block adds
  // `resid`, normalises with `norm_w` and writes `res_out` and `normed`.
  const void* resid;
  const void* norm_w;
  void* res_out;
  void* normed;
  int* an_counter;   // row blocks completed; zero before the launch, zero again after it
  float eps;
};

// Weight row held by tile row r (0..15). SwiGLU tiles pair gate rows 8t..8t+7 with the
// matching up rows I+8t..I+8t+7 (engine/kernels/cuda_fp8.py:208-212 pairs them per lane).
// Rows past n (a partial last tile of a row-major weight) read row n - 1; their outputs are
// dropped.
__device__ __forceinline__ int weight_row(const GemmArgs& a, int tile, int r) {
  if (a.mode == QLX_MODE_SWIGLU) return r < 8 ? 8 * tile + r : a.half + 8 * tile + r - 8;
  return min(16 * tile + r, a.n - 1);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// MI355X tile layout of a row-major [rows][row_bytes] weight (row_bytes % 128 == 0): a
// 16-row x 128-byte step is one contiguous 2 KB block, ordered [j][c][r][16 B] -- exactly
// the order in which a wave's two 16-byte-per-lane loads consume it (lane = 16c + r, load j
// takes bytes 64j + 16c of row r) -- and a tile's steps follow each other. Each load
// instruction then reads 1 KB of consecutive bytes.
__device__ __forceinline__ size_t tile_offset(int wrow, int step_bytes_idx, int j, int lane, int row_bytes) {
  return ((size_t)(wrow >> 4) * (row_bytes >> 7) + step_bytes_idx) * 2048 +
         (size_t)((j * 4 + (lane >> 4)) * 16 + (wrow & 15)) * 16;
}

// Device-coherent (agent scope) store/load: written through to / read from the level all
// XCDs share, so split-K partials need no cache-wide write-back to be seen by another CU.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Publish this workgroup's device-coherent stores before one thread signals another
// workgroup (ticket or arrival counter). Each wave waits until its own stores are
// acknowledged (s_waitcnt 0), then the barrier orders every wave before the signal. A
// workgroup-scope release alone does not wait for outstanding stores on gfx950 (the
// barrier does not either), and an agent-scope release would also write back the whole L2.
__device__ __forceinline__ void publish_stores() {
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __syncthreads();
}

// Where a work item's bf16 activation comes from. Staging reads it 8 values (16 bytes) at
// a time: fetch issues the loads of a chunk, so a thread has several chunks in flight;
// sources whose data may not have arrived yet (POLLS) also say whether a fetched chunk is
// ready and re-fetch its stale parts; value gives the 8 values. The single-call kernels read
// x from device memory.
struct XPlain {
  static constexpr bool POLLS = false;
  struct Raw {
    uint4 v;
  };
  __device__ __forceinline__ void fetch(const GemmArgs& a, int mm, int kabs, Raw& r) const {
    const u32x4 v = *gmem(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.x) + (size_t)mm * a.k + kabs));
    r.v = uint4{v[0], v[1], v[2], v[3]};
  }
  __device__ __forceinline__ bool ready(const Raw&) const { return true; }
  __device__ __forceinline__ void refetch(const GemmArgs&, int, int, Raw&) const {}
  __device__ __forceinline__ bool expired() const { return false; }
  __device__ __forceinline__ uint4 value(const Raw& r) const { return r.v; }
};

// Settle a batch of fetched chunks of a source whose data may not have arrived: every round
// re-fetches all of the batch's stale chunks together and waits for them, until all are ready
// or the source's deadline has passed. Chunks written by different producers then cost one
// round trip after the last of them lands, not one per chunk. chunk(u, mm, kabs) says whether
// slot u holds a chunk and where it is.
template <class XS, int U, class Chunk>
__device__ __forceinline__ void settle_batch(const GemmArgs& a, const XS& xs, typename XS::Raw (&r)[U], Chunk chunk) {
  if constexpr (XS::POLLS) {
    unsigned stale = 0;  // bit u: slot u holds a chunk that has not arrived
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int mm, kabs;
      if (chunk(u, mm, kabs) && !xs.ready(r[u])) stale |= 1u << u;
    }
    while (stale && !xs.expired()) {
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int mm, kabs;
        if (stale >> u & 1u) {
          chunk(u, mm, kabs);
          xs.refetch(a, mm, kabs, r[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if ((stale >> u & 1u) && xs.ready(r[u])) stale &= ~(1u << u);
    }
  }
}

// Two exact small-integer floats -> bf16 pair (the high halves are exact: <= 8 significant bits).
__device__ __forceinline__ uint32_t pack_hi(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 4 bytes -> 4 bf16 values (byte value as float), natural order.
__device__ __forceinline__ uint2 bytes_to_bf16(uint32_t d) {
  uint2 r;
  r.x = pack_hi((float)(d & 0xffu), (float)((d >> 8) & 0xffu));
  r.y = pack_hi((float)((d >> 16) & 0xffu), (float)(d >> 24));
  return r;
}

// Low nibbles of bytes (0,2) and (1,3) of d, shifted by `sh` (0, 4, 8 or 12), as bf16(128 +
// code) pairs, i.e. ((d >> sh) & 0x000f000f) | 0x43004300. Built with a byte permute from the
// dword's low or high nibbles (d & 0x0f0f0f0f, shared by the four calls on one dword): 7
// instructions per dword instead of 11 (the compiler splits (x & m) | c with two literal
// constants into two instructions).
__device__ __forceinline__ uint32_t nib_pair(uint32_t d, int sh) {
  const uint32_t n = ((sh & 4) ? d >> 4 : d) & 0x0f0f0f0fu;
  return __builtin_amdgcn_perm(0x43434343u, n, (sh & 8) ? 0x04030401u : 0x04020400u);
}

__device__ __forceinline__ uint32_t bf16_at(const uint16_t* p, int i) { return p[i]; }

// ====================================================================================
// Format policies. Each provides:
//   KSTEP, LOADS (16-byte loads per lane per step), NSC (scales per step; 0 = per
//   channel), BIAS (code bias removed via activation sums; 0 = none), XBYTES (staged
//   bytes per activation value), load(), compute(), stage_chunk(), finish().
// ====================================================================================

// ---- W4A16: int32 [n][k/8] words (nibble i of word j = k 8j+i, code = q + 8),
//      bf16 scale [n][k/128]. Step = 256 k = 128 bytes of a row = two groups; lane chunk j
//      (j = 0, 1) is the 4 words at byte 64j + 16c, i.e. group 2*step + j, so one wave's two
//      loads complete 16 full 128-byte lines.
struct FmtW4 {
  static constexpr int KSTEP = 256, LOADS = 2, NSC = 2, XBYTES = 2;
  static constexpr bool SCALE_PAIR = true;  // scale_pair(): a step's two group scales
  static constexpr float BIAS = 136.f;  // bf16(128 + code) = q + 136
  static constexpr bool FUSED_BIAS = true;  // compute() runs the bias chain itself (no xb)
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    if (a.tiled)
      return reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.w) +
                                            tile_offset(wrow, step, j, lane, a.k >> 1));
    return reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(a.w) +
                                          (size_t)wrow * (a.k >> 3) + step * 32 + j * 16 + (lane >> 4) * 4);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int step, int j) {
    return bf2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)wrow * (a.k >> 7) + 2 * step + j]);
  }
  // Both group scales of a step, one 4-byte load (a row's k/128 groups are an even count).
  __device__ static uint32_t scale_pair(const GemmArgs& a, int wrow, int step) {
    return gmem(reinterpret_cast<const uint32_t*>(a.ws))[(size_t)wrow * (a.k >> 8) + step];
  }
  __device__ static float scale_of(uint32_t bits16) { return bf2f(bits16); }
  // A element order per word: k offsets [0,4,1,5,2,6,3,7] (nibble j and j+4 per dword);
  // the staged activation chunk (8 values in k order) is permuted to match.
  static constexpr bool GATHER = false;
  __device__ static uint4 order(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return o;
  }
  // The same MFMA chain with every code at the bias (q = 0): bias * sum(x) rounded exactly
  // as the main loop rounds it, so an all-zero weight row gives exactly zero.
  __device__ static f32x4 bias_chain(const char* lds, int srel, int j, int lane, int xoff) {
    const uint4 av = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136
    const int kb = (srel * 256 + j * 128 + (lane >> 4) * 32) * 2;
    f32x4 t4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff + kb + t * 16);
      t4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), t4, 0, 0, 0);
    }
    return t4;
  }
  // BMODE 0: the code-bias chain runs with every step; 1: it runs and its totals go to the
  // LDS table at a.off_bt ([step][group][MT][16 tokens]); 2: the totals are read back from that
  // table instead (a persistent workgroup's later items: same activation, same steps). All
  // rows of the bias chain's A operand are equal, so every row of its result is the same value.
  template <int MT, int BMODE = 0>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs& a, int srel, int lane, const int (&xoff)[MT],
                                 const int (&mrow)[MT], int rowl) {
    const float* sc = reinterpret_cast<const float*>(lds + a.off_sc);
    float* bt = reinterpret_cast<float*>(const_cast<char*>(lds) + a.off_bt);
    // The code bias: the same MFMA chain with every code at the bias, on the fragments the
    // step reads anyway -- bias_chain's value bit for bit (same operands, same order), with no
    // staging pass, barrier or LDS table before the first step.
    const uint4 avb = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f32x4 tmp[MT], tb[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) tmp[mt] = tb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint32_t wd[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
      const int kb = (srel * 256 + j * 128 + (lane >> 4) * 32) * 2;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint4 av;
        av.x = nib_pair(wd[t], 0);
        av.y = nib_pair(wd[t], 4);
        av.z = nib_pair(wd[t], 8);
        av.w = nib_pair(wd[t], 12);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb + t * 16);
          tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), tmp[mt], 0, 0, 0);
          if constexpr (BMODE < 2)
            tb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(avb), as_bf16x8(bv), tb[mt], 0, 0, 0);
        }
      }
      const int bti = (srel * 2 + j) * MT * 16 + (lane & 15);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (BMODE == 1) {
          if (lane < 16) bt[bti + mt * 16] = tb[mt][0];
        } else if constexpr (BMODE == 2) {
          const float v = bt[bti + mt * 16];
          tb[mt] = f32x4{v, v, v, v};
        }
      }
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc + (srel * 2 + j) * a.sc_stride + rowl);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(s4[i], tmp[mt][i] - tb[mt][i], acc[mt][i]);
    }
  }
  __device__ static float finish(const GemmArgs&, const char*, float v, int, int) { return v; }
};

// ---- W8A16 per output channel: int8 [n][k], bf16 scale [n]. Step = 128 k (a full
//      128-byte row segment); lane chunk j is the 16 bytes at 64j + 16c.
struct FmtW8 {
  static constexpr int KSTEP = 128, LOADS = 2, NSC = 0, XBYTES = 2;
  static constexpr float BIAS = 128.f;  // (byte ^ 0x80) = q + 128
  static constexpr bool FUSED_BIAS = true;  // compute() runs the bias chain itself (no xb)
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    if (a.tiled)
      return reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.w) + tile_offset(wrow, step, j, lane, a.k));
    return reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(a.w) + (size_t)wrow * a.k +
                                          step * 128 + j * 64 + (lane >> 4) * 16);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int, int) {
    return bf2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[wrow]);
  }
  static constexpr bool GATHER = false;
  __device__ static uint4 order(uint4 v) { return v; }
  __device__ static f32x4 bias_chain(const char* lds, int srel, int, int lane, int xoff) {
    const uint4 av = {0x43004300u, 0x43004300u, 0x43004300u, 0x43004300u};  // bf16 128
    f32x4 t4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = (srel * 128 + j * 64 + (lane >> 4) * 16) * 2;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff + kb + t * 16);
        t4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), t4, 0, 0, 0);
      }
    }
    return t4;
  }
  // BMODE as in FmtW4::compute (one bias total per step: [step][MT][16 tokens]).
  template <int MT, int BMODE = 0>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs& a, int srel, int lane, const int (&xoff)[MT],
                                 const int (&mrow)[MT], int) {
    float* bt = reinterpret_cast<float*>(const_cast<char*>(lds) + a.off_bt);
    // The code bias as in FmtW4::compute: bias_chain's value bit for bit, from the same fragments.
    const uint4 avb = {0x43004300u, 0x43004300u, 0x43004300u, 0x43004300u};  // bf16 128
    f32x4 tmp[MT], tb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) tmp[mt] = tb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t wd[4] = {c[j].x ^ 0x80808080u, c[j].y ^ 0x80808080u, c[j].z ^ 0x80808080u,
                              c[j].w ^ 0x80808080u};
      const int kb = (srel * 128 + j * 64 + (lane >> 4) * 16) * 2;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint2 lo = bytes_to_bf16(wd[2 * t]), hi = bytes_to_bf16(wd[2 * t + 1]);
        const uint4 av = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb + t * 16);
          tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), tmp[mt], 0, 0, 0);
          if constexpr (BMODE < 2)
            tb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(avb), as_bf16x8(bv), tb[mt], 0, 0, 0);
        }
      }
    }
    const int bti = srel * MT * 16 + (lane & 15);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (BMODE == 1) {
        if (lane < 16) bt[bti + mt * 16] = tb[mt][0];
      } else if constexpr (BMODE == 2) {
        const float v = bt[bti + mt * 16];
        tb[mt] = f32x4{v, v, v, v};
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][i] += tmp[mt][i] - tb[mt][i];
  }
  // Per-channel scale once, after the K sum.
  __device__ static float finish(const GemmArgs& a, const char* lds, float v, int rl, int) {
    return v * reinterpret_cast<const float*>(lds + a.off_sc)[rl];
  }
};

// ---- FP8 W8A8: e4m3 [n][k], bf16 scale [n]; activation quantized per token in the
//      prologue. Step = 128 k (a full 128-byte row segment), chunk j at byte 64j + 16c.
struct FmtFP8 {
  static constexpr int KSTEP = 128, LOADS = 2, NSC = 0, XBYTES = 1;
  static constexpr float BIAS = 0.f;
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    if (a.tiled)
      return reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.w) + tile_offset(wrow, step, j, lane, a.k));
    return reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.w) + (size_t)wrow * a.k +
                                          step * 128 + j * 64 + (lane >> 4) * 16);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int, int) {
    return bf2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[wrow]);
  }
  template <int MT>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs&, int srel, int lane, const int (&xoff)[MT],
                                 const int (&)[MT], int) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int kb = srel * 128 + j * 64 + (lane >> 4) * 16;
      const long a0 = (long)(((unsigned long)c[j].y << 32) | c[j].x);
      const long a1 = (long)(((unsigned long)c[j].w << 32) | c[j].z);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb);
        const long b0 = (long)(((unsigned long)bv.y << 32) | bv.x);
        const long b1 = (long)(((unsigned long)bv.w << 32) | bv.z);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a0, b0, acc[mt], 0, 0, 0);
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(a1, b1, acc[mt], 0, 0, 0);
      }
    }
  }
  __device__ static float finish(const GemmArgs& a, const char* lds, float v, int rl, int mm) {
    const float sx = reinterpret_cast<const float*>(lds + a.off_sx)[mm];
    return v * sx * reinterpret_cast<const float*>(lds + a.off_sc)[rl];
  }
};

// Natural column at permuted position p of a 64-block (engine/kernels/cuda_fp8.py:1117-1124).
__device__ __forceinline__ int ref_pos_natural(int p) {
  const int t = p >> 4, s = (p >> 2) & 3, i = p & 3;
  return 16 * s + 2 * t + ((i & 1) | ((i >> 1) << 3));
}

// ---- cuda_fp8 reference formats: offset codes, fp16 scale per 64 [n][k/64], columns of each
//      64-block permuted (cuda_fp8.py:1117-1124). Step = 128 k = blocks j = 0, 1.
//      BITS 8: tiled [rows/16][K/128][half][j][g][t][16 B] or row-major permuted;
//      BITS 4: tiled [rows/16][K/128][half][g][t][16 B], block 0 low nibble, block 1 high.
//      Lane (r, c) takes the chunk of row r at t = c, so B position
//      64j + 16c + 8u + e holds permuted position 16c + 8u + e' of block j.
template <int BITS>
struct FmtRef {
  static constexpr int KSTEP = 128, LOADS = BITS == 8 ? 2 : 1, NSC = 2, XBYTES = 2;
  static constexpr bool SCALE_PAIR = true;
  static constexpr float BIAS = BITS == 8 ? 128.f : 136.f;
  static constexpr bool FUSED_BIAS = true;  // compute() runs the bias chain itself (no xb)
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    const int r = wrow & 15, tile = wrow >> 4, c = lane >> 4;
    const uint8_t* w = reinterpret_cast<const uint8_t*>(a.w);
    if (BITS == 4) {
      const size_t tb = ((size_t)tile * (a.k >> 7) + step) * 1024;
      return reinterpret_cast<const uint4*>(w + tb + (((r >> 3) * 8 + (r & 7)) * 4 + c) * 16);
    }
    if (a.tiled) {  // [half][j][g][t][16 B]
      const size_t tb = ((size_t)tile * (a.k >> 7) + step) * 2048;
      return reinterpret_cast<const uint4*>(w + tb + ((((r >> 3) * 2 + j) * 8 + (r & 7)) * 4 + c) * 16);
    }
    return reinterpret_cast<const uint4*>(w + (size_t)wrow * a.k + step * 128 + j * 64 + c * 16);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int step, int j) {
    return h2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)wrow * (a.k >> 6) + 2 * step + j]);
  }
  // Both block scales of a step, one 4-byte load (k is a multiple of 128).
  __device__ static uint32_t scale_pair(const GemmArgs& a, int wrow, int step) {
    return gmem(reinterpret_cast<const uint32_t*>(a.ws))[(size_t)wrow * (a.k >> 7) + step];
  }
  __device__ static float scale_of(uint32_t bits16) { return h2f((uint16_t)bits16); }
  // B position e (0..7) of chunk (c, u) of a 64-block holds permuted position 16c + 8u + sw(e):
  // 8-bit codes unpack in byte order, 4-bit codes as bytes (0,2),(1,3) per dword.
  __device__ static f32x4 bias_chain(const char* lds, int srel, int j, int lane, int xoff) {
    const uint32_t b = BITS == 8 ? 0x43004300u : 0x43084308u;  // bf16 128 / 136
    const uint4 av = {b, b, b, b};
    const int kb = (srel * 128 + j * 64 + (lane >> 4) * 16) * 2;
    f32x4 t4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff + kb + u * 16);
      t4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), t4, 0, 0, 0);
    }
    return t4;
  }
  static constexpr bool GATHER = true;  // staged from permuted positions (stage_chunk)
  // Chunk (c, u) of a 64-block -- permuted positions 16c + 8u + 0..7 -- holds the natural
  // values 32u + 2c + {0, 1, 8, 9, 16, 17, 24, 25} (ref_pos_natural): four aligned pairs of
  // consecutive values, read as four 4-byte loads. 8-bit codes take them in that order; 4-bit
  // codes pair the values 8 apart (bytes (0, 2), (1, 3) of a dword).
  __device__ static uint4 stage_chunk(const GemmArgs& a, int mm, int kabs) {
    const uint32_t* row = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(a.x) + (size_t)mm * a.k);
    const int blk = kabs & ~63, p0 = kabs & 63;  // p0 = 16c + 8u
    const int base = (blk + 32 * ((p0 >> 3) & 1) + 2 * (p0 >> 4)) >> 1;  // dword index of the first pair
    const uint32_t d0 = gmem(row)[base], d1 = gmem(row)[base + 4], d2 = gmem(row)[base + 8],
                   d3 = gmem(row)[base + 12];
    if constexpr (BITS == 8) return uint4{d0, d1, d2, d3};
    return uint4{__builtin_amdgcn_perm(d1, d0, 0x05040100u), __builtin_amdgcn_perm(d1, d0, 0x07060302u),
                 __builtin_amdgcn_perm(d3, d2, 0x05040100u), __builtin_amdgcn_perm(d3, d2, 0x07060302u)};
  }
  template <int MT>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs& a, int srel, int lane, const int (&xoff)[MT],
                                 const int (&mrow)[MT], int rowl) {
    const float* sc = reinterpret_cast<const float*>(lds + a.off_sc);
    // The code bias as in FmtW4::compute: bias_chain's value bit for bit, from the same fragments.
    const uint32_t bb = BITS == 8 ? 0x43004300u : 0x43084308u;  // bf16 128 / 136
    const uint4 avb = {bb, bb, bb, bb};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint4 av[2];
      if (BITS == 8) {
        const uint4 ch = c[j];
        const uint2 p0 = bytes_to_bf16(ch.x), p1 = bytes_to_bf16(ch.y);
        const uint2 p2 = bytes_to_bf16(ch.z), p3 = bytes_to_bf16(ch.w);
        av[0] = uint4{p0.x, p0.y, p1.x, p1.y};
        av[1] = uint4{p2.x, p2.y, p3.x, p3.y};
      } else {
        const uint4 ch = c[0];
        const int sh = 4 * j;
        av[0] = uint4{nib_pair(ch.x, sh), nib_pair(ch.x, sh + 8), nib_pair(ch.y, sh), nib_pair(ch.y, sh + 8)};
        av[1] = uint4{nib_pair(ch.z, sh), nib_pair(ch.z, sh + 8), nib_pair(ch.w, sh), nib_pair(ch.w, sh + 8)};
      }
      f32x4 tmp[MT], tb[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) tmp[mt] = tb[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int kb = (srel * 128 + j * 64 + (lane >> 4) * 16) * 2;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb + u * 16);
          tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[u]), as_bf16x8(bv), tmp[mt], 0, 0, 0);
          tb[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(avb), as_bf16x8(bv), tb[mt], 0, 0, 0);
        }
      }
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc + (srel * 2 + j) * a.sc_stride + rowl);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(s4[i], tmp[mt][i] - tb[mt][i], acc[mt][i]);
    }
  }
  __device__ static float finish(const GemmArgs&, const char*, float v, int, int) { return v; }
};

// ---- fp8.fp8_matmul: e4m3 [n][k] weights, bf16 scale [n][k/group], bf16 activation.
//      Step = 128 k, chunk j (64-wide block 2*step + j) at byte 64j + 16c; e4m3 -> fp32 by
//      v_cvt_pk_f32_fp8 (exact), -> bf16 by truncation (exact: e4m3 has 4 significant bits).
struct FmtFP8WO {
  static constexpr int KSTEP = 128, LOADS = 2, NSC = 2, XBYTES = 2;
  static constexpr bool SCALE_PAIR = false;
  static constexpr float BIAS = 0.f;
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    return reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(a.w) + (size_t)wrow * a.k +
                                          step * 128 + j * 64 + (lane >> 4) * 16);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int step, int j) {
    return bf2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)wrow * (a.k / a.group) +
                                                        (step * 128 + j * 64) / a.group]);
  }
  static constexpr bool GATHER = false;
  __device__ static uint4 order(uint4 v) { return v; }
  template <bool HI>
  __device__ static uint32_t fp8pair(uint32_t d) {
    typedef __attribute__((ext_vector_type(2))) float f2;
    const f2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)d, HI);
    return pack_hi(f[0], f[1]);
  }
  template <int MT>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs& a, int srel, int lane, const int (&xoff)[MT],
                                 const int (&)[MT], int rowl) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t wd[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
      const int kb = (srel * 128 + j * 64 + (lane >> 4) * 16) * 2;
      f32x4 tmp[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) tmp[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint4 av = {fp8pair<false>(wd[2 * t]), fp8pair<true>(wd[2 * t]),
                          fp8pair<false>(wd[2 * t + 1]), fp8pair<true>(wd[2 * t + 1])};
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb + t * 16);
          tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(bv), tmp[mt], 0, 0, 0);
        }
      }
      const f32x4 sc = *reinterpret_cast<const f32x4*>(
          reinterpret_cast<const float*>(lds + a.off_sc) + (srel * 2 + j) * a.sc_stride + rowl);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf(sc[i], tmp[mt][i], acc[mt][i]);
    }
  }
  __device__ static float finish(const GemmArgs&, const char*, float v, int, int) { return v; }
};

// ---- cuda_int8 W8A8: int8 [n][k] and int8 activation [m][k], both in fragment order
//      (engine/kernels/cuda_int8.py:64, 100-108); fp16 weight scale [n][k/64], fp32
//      activation scale [m][k/64]; per group acc = fma(float(dot) * sx, sw, acc)
//      (engine/kernels/cuda_int8.py:198-199). Step = 128 k = groups 2*step + j, chunk j at
//      byte 64j + 16c.
struct FmtInt8 {
  static constexpr int KSTEP = 128, LOADS = 2, NSC = 2, XBYTES = 1;
  static constexpr bool SCALE_PAIR = false;
  static constexpr float BIAS = 0.f;
  __device__ static const uint4* chunk_ptr(const GemmArgs& a, int wrow, int step, int lane, int j) {
    return reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(a.w) + (size_t)wrow * a.k +
                                          step * 128 + j * 64 + (lane >> 4) * 16);
  }
  __device__ static float scale(const GemmArgs& a, int wrow, int step, int j) {
    return h2f(gmem(reinterpret_cast<const uint16_t*>(a.ws))[(size_t)wrow * (a.k >> 6) + 2 * step + j]);
  }
  // Both block scales of a step, one 4-byte load (k is a multiple of 128).
  __device__ static uint32_t scale_pair(const GemmArgs& a, int wrow, int step) {
    return gmem(reinterpret_cast<const uint32_t*>(a.ws))[(size_t)wrow * (a.k >> 7) + step];
  }
  __device__ static float scale_of(uint32_t bits16) { return h2f((uint16_t)bits16); }
  template <int MT>
  __device__ static void compute(f32x4 (&acc)[MT], const uint4* c, const char* lds,
                                 const GemmArgs& a, int srel, int lane, const int (&xoff)[MT],
                                 const int (&mrow)[MT], int rowl) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const i32x4 av = {(int)c[j].x, (int)c[j].y, (int)c[j].z, (int)c[j].w};
      const int kb = srel * 128 + j * 64 + (lane >> 4) * 16;
      const f32x4 sw = *reinterpret_cast<const f32x4*>(
          reinterpret_cast<const float*>(lds + a.off_sc) + (srel * 2 + j) * a.sc_stride + rowl);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 bv = *reinterpret_cast<const uint4*>(lds + xoff[mt] + kb);
        const i32x4 b = {(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w};
        const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b, i32x4{0, 0, 0, 0}, 0, 0, 0);
        const float* sxp = reinterpret_cast<const float*>(lds + a.off_sx);
        const float sx = sxp[mrow[mt] * a.xb_stride + srel * 2 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf((float)d[i] * sx, sw[i], acc[mt][i]);
        if (a.comp == 2) {  // the residual component, accumulated after the first (cuda_int8.py:207-216)
          const uint4 rv = *reinterpret_cast<const uint4*>(lds + a.m * a.xstride + xoff[mt] + kb);
          const i32x4 rb = {(int)rv.x, (int)rv.y, (int)rv.z, (int)rv.w};
          const i32x4 d2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, rb, i32x4{0, 0, 0, 0}, 0, 0, 0);
          const float sr = sxp[(a.m + mrow[mt]) * a.xb_stride + srel * 2 + j];
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][i] = fmaf((float)d2[i] * sr, sw[i], acc[mt][i]);
        }
      }
    }
  }
  __device__ static float finish(const GemmArgs&, const char*, float v, int, int) { return v; }
};

// ====================================================================================
// Prologue: stage the workgroup's activation slice (B order), its scales, bias sums.
// ====================================================================================

// Chunks each thread keeps in flight while staging: 4 from device memory; from published
// activations (the decode executor's polls) 3 for the FP8 prologue and 1 for bf16, the
// fastest on the Qwen3-4B M=1 chain (FP8 1223 / 1190 / 1202 / 1218 us at 2 / 3 / 4 / 6;
// W4A16 1185 / 1190 / 1213 / 1221 us at 1 / 2 / 3 / 4).
template <class XS, bool FP8>
__host__ __device__ constexpr int stage_unroll() {
  return XS::POLLS ? (FP8 ? 3 : 1) : 4;
}

// The threads that stage and finish a work item, and how they wait for each other: the
// whole workgroup and its barrier here; the decode executor passes its own team (the same
// threads, counted at compile time).
struct BlockTeam {
  __device__ int tid() const { return threadIdx.x; }
  __device__ int size() const { return blockDim.x; }
  __device__ void sync() const { __syncthreads(); }
};

// UNROLL (0: stage_unroll's choice) sets the chunks each thread keeps in flight.
template <class F, class XS, class Team = BlockTeam, int UNROLL = 0>
__device__ __forceinline__ void stage_bf16(const GemmArgs& a, const XS& xs, char* lds, int step0, int nst, const Team& team = {}) {
  const int tid = team.tid(), nthr = team.size();
  constexpr int U_ = UNROLL ? UNROLL : stage_unroll<XS, false>();
  constexpr int CPS = F::KSTEP / 8;  // 16-byte chunks per step
  const int cpr = nst * CPS;
  const int total = a.m * cpr;
  if constexpr (F::GATHER) {
    static_assert(std::is_same<XS, XPlain>::value, "gathered staging reads x from device memory");
    for (int q = tid; q < total; q += nthr) {
      const int mm = q / cpr, kc = q - mm * cpr;
      *reinterpret_cast<uint4*>(lds + mm * a.xstride + kc * 16) = F::stage_chunk(a, mm, step0 * F::KSTEP + kc * 8);
    }
  } else {
    for (int q0 = tid; q0 < total; q0 += U_ * nthr) {
      typename XS::Raw r[U_];
      auto chunk = [&](int u, int& mm, int& kabs) {
        const int q = q0 + u * nthr;
        mm = q / cpr;
        kabs = step0 * F::KSTEP + (q - mm * cpr) * 8;
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
          *reinterpret_cast<uint4*>(lds + mm * a.xstride + (kabs - step0 * F::KSTEP) * 2) = F::order(xs.value(r[u]));
      }
    }
  }
}

// Formats whose compute() removes the code bias itself (FUSED_BIAS) need no bias totals.
template <class F, class = void>
struct fused_bias : std::false_type {};
template <class F>
struct fused_bias<F, std::void_t<decltype(F::FUSED_BIAS)>> : std::bool_constant<F::FUSED_BIAS> {};
template <class F>
constexpr bool needs_bias_totals() { return F::BIAS != 0.f && !fused_bias<F>::value; }

// Bias totals per (token, scale group) from the staged activation, one MFMA chain per
// (group, 16-token fragment), spread over the workgroup's waves. Needs the staged x.
template <class F, int WAVES>
__device__ void stage_bias(const GemmArgs& a, char* lds, int nst) {
  constexpr int NJ = F::NSC > 1 ? F::NSC : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int frags = (a.m + 15) >> 4;
  float* xb = reinterpret_cast<float*>(lds + a.off_xb);
  for (int item = wave; item < nst * NJ * frags; item += WAVES) {
    const int mt = item % frags, sj = item / frags;
    const int mm = 16 * mt + (lane & 15);
    const int mrow = min(mm, a.m - 1);
    const f32x4 d = F::bias_chain(lds, sj / NJ, sj % NJ, lane, mrow * a.xstride);
    if ((lane >> 4) == 0 && mm < a.m) xb[mm * a.xb_stride + sj] = d[0];
  }
}

// e4m3 codes of 8 activation values (bf16 pairs in v) at per-token scale sc, to LDS.
__device__ __forceinline__ void store_e4m3_chunk(char* dst, uint4 v, float sc) {
  *reinterpret_cast<uint2*>(dst) = e4m3_chunk(v, sc, 1.f / sc);
}

// The per-token bf16 maxima (as uint bits) of the FP8 prologue, after the token scales.
__device__ __forceinline__ uint32_t* fp8_amax(const GemmArgs& a, char* lds) {
  return reinterpret_cast<uint32_t*>(lds + a.off_sx) + a.m;
}

// FP8 W8A8 prologue: per-token scale over the whole row, then e4m3 codes of the slice. When
// one batch of loads covers the rows, the values stay in registers for the codes (one pass
// over x); otherwise the slice is read again. With `zeroed_amax`, the per-token maxima live
// there, already cleared and visible to the team.
template <class XS, class Team = BlockTeam, int UNROLL = 0>
__device__ __forceinline__ void stage_fp8_act(const GemmArgs& a, const XS& xs, char* lds, int step0, int nst, const Team& team = {},
                              uint32_t* zeroed_amax = nullptr) {
  const int tid = team.tid(), nthr = team.size();
  constexpr int U_ = UNROLL ? UNROLL : stage_unroll<XS, true>();
  float* sx = reinterpret_cast<float*>(lds + a.off_sx);
  uint32_t* amax = zeroed_amax ? zeroed_amax : fp8_amax(a, lds);
  if (!zeroed_amax) {
    for (int i = tid; i < a.m; i += nthr) amax[i] = 0u;
    team.sync();
  }
  const int cpr = a.k >> 3;
  const int total = a.m * cpr;
  const bool one_pass = total <= U_ * nthr;
  uint4 kept[U_];
  for (int q0 = tid; q0 < total; q0 += U_ * nthr) {
    typename XS::Raw r[U_];
    auto chunk = [&](int u, int& mm, int& kabs) {
      const int q = q0 + u * nthr;
      mm = q / cpr;
      kabs = (q - mm * cpr) * 8;
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
      const int q = q0 + u * nthr;
      if (q < total) {
        const uint4 v = xs.value(r[u]);
        kept[u] = v;
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
        float mx = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fmaxf(fabsf(bf2f(d[j] & 0xffffu)), fabsf(bf2f(d[j] >> 16))));
        atomicMax(&amax[q / cpr], __float_as_uint(mx));
      }
    }
  }
  team.sync();
  // Every thread derives the token scales it needs from the maxima (no second barrier); the
  // epilogue reads sx after later barriers.
  auto token_scale = [&](int mm) { return fmaxf(__uint_as_float(amax[mm]) / 448.f, 1e-12f); };
  for (int i = tid; i < a.m; i += nthr) sx[i] = token_scale(i);
  const int c0 = step0 * 16, c1 = c0 + nst * 16;  // the slice's 8-value chunks within a row
  if (one_pass) {
#pragma unroll
    for (int u = 0; u < U_; ++u) {
      const int q = tid + u * nthr;
      if (q < total) {
        const int mm = q / cpr, kc = q - mm * cpr;
        if (kc >= c0 && kc < c1) store_e4m3_chunk(lds + mm * a.xstride + (kc - c0) * 8, kept[u], token_scale(mm));
      }
    }
    return;
  }
  const int cps = nst * 16;  // 8-value chunks per row of the slice
  for (int q0 = tid; q0 < a.m * cps; q0 += U_ * nthr) {
    typename XS::Raw r[U_];
    auto chunk = [&](int u, int& mm, int& kabs) {
      const int q = q0 + u * nthr;
      mm = q / cps;
      kabs = step0 * 128 + (q - mm * cps) * 8;
      return q < a.m * cps;
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

// FP8 W8A8 prologue from an activation quantized beforehand (qlx_quantize_fp8_act: the same
// per-token scale and codes the in-kernel prologue computes): the slice's e4m3 codes and the
// token scales are copied, so no workgroup reads whole rows for the maxima.
__device__ __forceinline__ void stage_fp8_pre(const GemmArgs& a, char* lds, int step0, int nst) {
  const uint8_t* xq = reinterpret_cast<const uint8_t*>(a.x);
  float* sx = reinterpret_cast<float*>(lds + a.off_sx);
  for (int i = threadIdx.x; i < a.m; i += blockDim.x) sx[i] = a.xs[i];
  const int cps = nst * 8;  // 16-byte chunks of a row's slice (128 codes per step)
  for (int q = threadIdx.x; q < a.m * cps; q += blockDim.x) {
    const int mm = q / cps, kc = q - mm * cps;
    const u32x4 v = *gmem(reinterpret_cast<const u32x4*>(xq + (size_t)mm * a.k + step0 * 128 + kc * 16));
    *reinterpret_cast<u32x4*>(lds + mm * a.xstride + kc * 16) = v;
  }
}

// cuda_int8 prologue: int8 activation slice and its fp32 group scales.
__device__ void stage_int8_act(const GemmArgs& a, char* lds, int step0, int nst) {
  const int cps = nst * 8;
  float* sx = reinterpret_cast<float*>(lds + a.off_sx);
  const int gps = 2 * nst;
  for (int c = 0; c < a.comp; ++c) {  // component c at token rows c*m .. c*m + m - 1
    const int8_t* xq = reinterpret_cast<const int8_t*>(c ? a.x2 : a.x);
    const float* xsc = c ? a.xs2 : a.xs;
    for (int q = threadIdx.x; q < a.m * cps; q += blockDim.x) {
      const int mm = q / cps, kc = q - mm * cps;
      *reinterpret_cast<uint4*>(lds + (c * a.m + mm) * a.xstride + kc * 16) =
          *reinterpret_cast<const uint4*>(xq + (size_t)mm * a.k + step0 * 128 + kc * 16);
    }
    for (int q = threadIdx.x; q < a.m * gps; q += blockDim.x) {
      const int mm = q / gps, j = q - mm * gps;
      sx[(c * a.m + mm) * a.xb_stride + j] = xsc[(size_t)mm * (a.k >> 6) + 2 * step0 + j];
    }
  }
}

template <class F, class Team = BlockTeam>
__device__ void stage_scales(const GemmArgs& a, char* lds, int tg, int step0, int nst, const Team& team = {}) {
  const int tid = team.tid(), nthr = team.size();
  float* sc = reinterpret_cast<float*>(lds + a.off_sc);
  const int rows = 16 * a.rt;
  if constexpr (F::NSC == 0) {
    for (int rl = tid; rl < rows; rl += nthr) {
      const int tile = tg * a.rt + (rl >> 4);
      sc[rl] = tile < a.ntiles ? F::scale(a, weight_row(a, tile, rl & 15), 0, 0) : 0.f;
    }
  } else {
    if constexpr (F::SCALE_PAIR) {
      if ((rows & (rows - 1)) == 0) {
        // A step's two scales of a row with one 4-byte load; with rows (16 rt) a power of two the
        // (step, row) of an index is a shift and a mask. Four loads in flight per thread.
        const int lg = __builtin_ctz(rows);
        const int total = nst * rows;
        for (int q0 = tid; q0 < total; q0 += 4 * nthr) {
          uint32_t v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * nthr, st = q >> lg, rl = q & (rows - 1);
            const int tile = tg * a.rt + (rl >> 4);
            v[u] = q < total && tile < a.ntiles ? F::scale_pair(a, weight_row(a, tile, rl & 15), step0 + st) : 0u;
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int q = q0 + u * nthr, st = q >> lg, rl = q & (rows - 1);
            if (q < total) {
              sc[(2 * st) * a.sc_stride + rl] = F::scale_of(v[u] & 0xffffu);
              sc[(2 * st + 1) * a.sc_stride + rl] = F::scale_of(v[u] >> 16);
            }
          }
        }
        return;
      }
    }
    // Four loads in flight per thread, then their stores: one memory round trip per batch.
    const int total = nst * F::NSC * rows;
    for (int q0 = tid; q0 < total; q0 += 4 * nthr) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = q0 + u * nthr, sj = q / rows, rl = q - sj * rows;
        const int tile = tg * a.rt + (rl >> 4);
        v[u] = q < total && tile < a.ntiles
                   ? F::scale(a, weight_row(a, tile, rl & 15), step0 + sj / F::NSC, sj % F::NSC)
                   : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = q0 + u * nthr, sj = q / rows, rl = q - sj * rows;
        if (q < total) sc[sj * a.sc_stride + rl] = v[u];
      }
    }
  }
}

// ====================================================================================
// One work item (a row block's K slice): prefetch, then stage + stream + epilogue.
// ====================================================================================

__device__ __forceinline__ void block_coords(const GemmArgs& a, int b, int& tg, int& s) {
  const int total = a.tile_groups * a.splits;
  int logical = b;
  if (total >= 8) {  // consecutive logical blocks (the splits of a row block) share an XCD
    const int per = total >> 3, rem = total & 7, xcd = b & 7, idx = b >> 3;
    logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
  }
  tg = logical / a.splits;
  s = logical - tg * a.splits;
}

template <class F>
__device__ __forceinline__ void load_chunk(uint4 (&c)[F::LOADS], const GemmArgs& a, int wrow, int step,
                                           int lane) {
#pragma unroll
  for (int j = 0; j < F::LOADS; ++j) {
    const u32x4 v = __builtin_nontemporal_load(gmem(reinterpret_cast<const u32x4*>(F::chunk_ptr(a, wrow, step, lane, j))));
    c[j] = uint4{v[0], v[1], v[2], v[3]};
  }
}

template <class F, int RW>
struct PipeDepth {
  static constexpr int PF = RW == 1 ? 4 : 2;  // steps in flight per wave (each 2 KB for RW = 1)
};
// W4A16 at one tile per wave: 3 steps. Measured on single calls at M = 1 (us, 4 / 3 steps):
// lm_head 45.5 / 43.4, gate_up 11.25 / 11.0, down 8.36 / 7.9, qkv 6.13 / 6.6 (2 steps: 45.4,
// 11.4, 7.8, 6.3); its dequantization keeps more registers live per step than the 8-bit formats.
template <>
struct PipeDepth<FmtW4, 1> {
  static constexpr int PF = 3;
};

// Per-wave state of one work item, fixed by item_prefetch: row block tg, steps
// [step0, step0 + nst), K piece s of the np pieces the row block is cut into.
template <int RW>
struct Item {
  int tg, s, np, step0, nst, wt, kwi, tile0, my, last;
  int wrow[RW];  // a tile past the end streams its neighbour's rows; its output is dropped
};

// Issue the wave's first PF steps of weight loads for a work item. They depend on nothing
// else, so they are in flight while the activation is staged (or, in the decode executor,
// while the previous item finishes or the previous projection completes).
template <class F, int RW>
__device__ __forceinline__ void item_prefetch_range(const GemmArgs& a, int tg, int step0, int nst, int s, int np,
                                                    Item<RW>& it,
                                                    uint4 (&buf)[PipeDepth<F, RW>::PF][RW][F::LOADS]) {
  constexpr int PF = PipeDepth<F, RW>::PF;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  it.tg = tg;
  it.s = s;
  it.np = np;
  it.step0 = step0;
  it.nst = nst;
  it.wt = wave / a.kw;
  it.kwi = wave - it.wt * a.kw;
  it.tile0 = tg * a.rt + it.wt * RW;
  const bool active = it.tile0 < a.ntiles;
#pragma unroll
  for (int r = 0; r < RW; ++r)
    it.wrow[r] = active ? weight_row(a, it.tile0 + r < a.ntiles ? it.tile0 + r : it.tile0, lane & 15) : 0;
  it.my = active ? (it.nst - it.kwi + a.kw - 1) / a.kw : 0;  // this wave's steps: kwi, kwi + kw, ...
  it.last = it.step0 + it.kwi + (it.my - 1) * a.kw;
#pragma unroll
  for (int p = 0; p < PF; ++p)
    if (p < it.my)
#pragma unroll
      for (int r = 0; r < RW; ++r) load_chunk<F>(buf[p][r], a, it.wrow[r], it.step0 + it.kwi + p * a.kw, lane);
}

// Work item (tg, s) of a launch whose row blocks are cut into a.splits equal K slices.
template <class F, int RW>
__device__ __forceinline__ void item_prefetch(const GemmArgs& a, int tg, int s, Item<RW>& it,
                                              uint4 (&buf)[PipeDepth<F, RW>::PF][RW][F::LOADS]) {
  const int step0 = s * a.sps;
  item_prefetch_range<F, RW>(a, tg, step0, min(a.nsteps, step0 + a.sps) - step0, s, a.splits, it, buf);
}

// bf16 pair (rows idx, idx + 1) as one 32-bit word, and its store.
__device__ __forceinline__ uint32_t bf16_pair(float v0, float v1) {
  return (uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16);
}
__device__ __forceinline__ void store_pair(uint16_t* y, size_t idx, float v0, float v1) {
  *gmem(reinterpret_cast<uint32_t*>(y + idx)) = bf16_pair(v0, v1);
}
// The same pair written device-coherent (agent scope), for values another workgroup of the
// launch reads back (the fused add-norm tail).
__device__ __forceinline__ void store_pair_coherent(uint16_t* y, size_t idx, float v0, float v1) {
  __hip_atomic_store(gmem(reinterpret_cast<uint32_t*>(y + idx)), bf16_pair(v0, v1), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// 8 bf16 values (16 bytes at element e of p) that other workgroups of this launch wrote: two
// device-coherent 8-byte loads, each single-copy atomic.
__device__ __forceinline__ uint4 load8_coherent(const uint16_t* p, size_t e) {
  const auto q = gmem(reinterpret_cast<const uint64_t*>(p + e));
  const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return uint4{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
}

__device__ __forceinline__ uint4 load8_plain(const uint16_t* p, size_t e) {
  const u32x4 v = *gmem(reinterpret_cast<const u32x4*>(p + e));
  return uint4{v[0], v[1], v[2], v[3]};
}

// Residual add + RMSNorm of the whole [m][n] output, run by the workgroup that completes the
// last row block: res = bf16(resid + delta), normed = bf16(bf16(res * rsqrt(mean res^2 + eps)) * w)
// (the fused epilogue of engine/kernels/cuda_fp8.py:1339-1374 with the rounding of
// engine/kernels/reference.py:19-28; the same arithmetic as qlx_add_rms_norm). Each token row
// is taken by a group of G threads (a power of two), which reads it 8 values at a time: the sum
// of squares (fp64, reduced over the group in a fixed order), then the outputs.
__device__ __noinline__ void add_norm_tail(const GemmArgs& a) {
  __shared__ double s_part[16];
  const int tid = threadIdx.x;
  int mp = 1;
  while (mp < a.m) mp <<= 1;
  const int G = (int)blockDim.x / mp;  // threads per row
  const int mm = tid / G, gi = tid - mm * G;
  const bool live = mm < a.m;
  const int nch = a.n >> 3;
  const size_t base = (size_t)(live ? mm : 0) * a.n;
  const uint16_t* dl = reinterpret_cast<const uint16_t*>(a.y);
  const uint16_t* xr = reinterpret_cast<const uint16_t*>(a.resid);
  const uint16_t* wn = reinterpret_cast<const uint16_t*>(a.norm_w);
  auto residual = [](uint4 x, uint4 d, float (&r)[8]) {
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ds[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t xb = e & 1 ? xs[e >> 1] >> 16 : xs[e >> 1] & 0xffffu;
      const uint32_t db = e & 1 ? ds[e >> 1] >> 16 : ds[e >> 1] & 0xffffu;
      r[e] = round_bf(bf2f(xb) + bf2f(db));
    }
  };
  // Rows of up to kTailChunks chunks per thread (the hidden width at M <= 8) take one pass:
  // delta, residual and norm weight are loaded together and kept in registers, so the tail is
  // one memory round trip; wider rows stream twice.
  constexpr int U = 4;  // chunks in flight per thread (two-pass rows)
  constexpr int kTailChunks = 6;
  double ss = 0.0;
  uint16_t* ro = reinterpret_cast<uint16_t*>(a.res_out);
  uint16_t* yo = reinterpret_cast<uint16_t*>(a.normed);
  auto row_total = [&](double part_ss) {
    const int lanes = G < 64 ? G : 64;
    for (int o = lanes >> 1; o > 0; o >>= 1) part_ss += __shfl_xor(part_ss, o, 64);
    double total = part_ss;
    if (G > 64) {  // a row spans G / 64 waves: their sums in wave order
      const int wpg = G >> 6;
      if ((tid & 63) == 0) s_part[tid >> 6] = part_ss;
      __syncthreads();
      total = 0.0;
      if (live)
        for (int w = 0; w < wpg; ++w) total += s_part[mm * wpg + w];
    }
    return total;
  };
  auto write_chunk = [&](int c, const float (&r)[8], uint4 w, float scale) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t rb[4], yb[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float w0 = bf2f(ws[e >> 1] & 0xffffu), w1 = bf2f(ws[e >> 1] >> 16);
      rb[e >> 1] = bf16_pair(r[e], r[e + 1]);
      yb[e >> 1] = bf16_pair(round_bf(round_bf(r[e] * scale) * w0), round_bf(round_bf(r[e + 1] * scale) * w1));
    }
    *gmem(reinterpret_cast<u32x4*>(ro + base + (size_t)c * 8)) = u32x4{rb[0], rb[1], rb[2], rb[3]};
    *gmem(reinterpret_cast<u32x4*>(yo + base + (size_t)c * 8)) = u32x4{yb[0], yb[1], yb[2], yb[3]};
  };
  if (nch <= kTailChunks * G) {
    uint4 d[kTailChunks], x[kTailChunks], w[kTailChunks];
#pragma unroll
    for (int u = 0; u < kTailChunks; ++u) {
      const int c = gi + u * G;
      if (live && c < nch) {
        d[u] = load8_coherent(dl, base + (size_t)c * 8);
        x[u] = load8_plain(xr, base + (size_t)c * 8);
        w[u] = load8_plain(wn, (size_t)c * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < kTailChunks; ++u) {
      if (live && gi + u * G < nch) {
        float r[8];
        residual(x[u], d[u], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (double)r[e] * (double)r[e];
      }
    }
    const double total = row_total(ss);
    const float scale = 1.0f / sqrtf((float)(total / (double)a.n) + a.eps);
#pragma unroll
    for (int u = 0; u < kTailChunks; ++u) {
      if (live && gi + u * G < nch) {
        float r[8];
        residual(x[u], d[u], r);
        write_chunk(gi + u * G, r, w[u], scale);
      }
    }
    return;
  }
  for (int c0 = gi; live && c0 < nch; c0 += U * G) {
    uint4 d[U], x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * G;
      if (c < nch) {
        d[u] = load8_coherent(dl, base + (size_t)c * 8);
        x[u] = load8_plain(xr, base + (size_t)c * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (c0 + u * G < nch) {
        float r[8];
        residual(x[u], d[u], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (double)r[e] * (double)r[e];
      }
    }
  }
  const double total = row_total(ss);
  // mean rounded to fp32, + eps and 1/sqrt in fp32, as torch's rsqrt(mean + eps)
  const float scale = 1.0f / sqrtf((float)(total / (double)a.n) + a.eps);
  for (int c0 = gi; live && c0 < nch; c0 += U * G) {
    uint4 d[U], x[U], w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * G;
      if (c < nch) {
        d[u] = load8_coherent(dl, base + (size_t)c * 8);
        x[u] = load8_plain(xr, base + (size_t)c * 8);
        w[u] = load8_plain(wn, (size_t)c * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * G;
      if (c < nch) {
        float r[8];
        residual(x[u], d[u], r);
        write_chunk(c, r, w[u], scale);
      }
    }
  }
}

// After a workgroup has written a completed row block of delta (device-coherent stores): count
// it, and let the workgroup that completes the last row block run the add-norm tail. The
// counter is left at zero for the next launch.
__device__ __forceinline__ void add_norm_ticket(const GemmArgs& a) {
  __shared__ int s_tail;
  publish_stores();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(a.an_counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_tail = prev == a.tile_groups - 1;
    if (s_tail) __hip_atomic_store(a.an_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_tail) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  add_norm_tail(a);
}

// y = bf16(bf16(silu(g)) * u) with g and u rounded to bf16 first (swiglu.py:12-30).
__device__ __forceinline__ float swiglu_bf(float g, float u) {
  const float gb = round_bf(g), ub = round_bf(u);
  return round_bf(gb / (1.f + expf(-gb))) * ub;
}

// Stage the activation (from xs), then stream the item's weight steps through the MFMAs into
// acc. On return the weight buffer is free (the next item may be prefetched into it) and LDS
// still holds what the epilogue needs.
// One K step of the wave's MFMA work; BMODE (formats with the fused code bias only) as in
// FmtW4::compute.
template <class F, int MT, int BMODE>
__device__ __forceinline__ void compute_step(f32x4 (&acc)[MT], const uint4* c, const char* lds, const GemmArgs& a,
                                             int srel, int lane, const int (&xoff)[MT], const int (&mrow)[MT],
                                             int rowl) {
  if constexpr (BMODE == 0)
    F::template compute<MT>(acc, c, lds, a, srel, lane, xoff, mrow, rowl);
  else
    F::template compute<MT, BMODE>(acc, c, lds, a, srel, lane, xoff, mrow, rowl);
}

// Stage the item's activation slice (unless `stage_x` is false: a persistent workgroup's later
// items find it in place) and scales, then run its steps. BMODE as in FmtW4::compute.
template <class F, int MT, int RW, int WAVES, class XS, int BMODE = 0>
__device__ __forceinline__ void item_main(const GemmArgs& a, const XS& xs, char* lds, const Item<RW>& it,
                                          uint4 (&buf)[PipeDepth<F, RW>::PF][RW][F::LOADS], f32x4 (&acc)[RW][MT],
                                          bool stage_x = true) {
  constexpr int PF = PipeDepth<F, RW>::PF;
  const int lane = threadIdx.x & 63;
  const int tg = it.tg, step0 = it.step0, nst = it.nst, wt = it.wt, kwi = it.kwi, my = it.my;

  // ---- prologue
  if (!stage_x) {
  } else if constexpr (std::is_same<F, FmtFP8>::value) {
    bool pre = false;  // quantized beforehand: x holds e4m3 codes, xs the token scales
    if constexpr (std::is_same<XS, XPlain>::value) pre = a.xs != nullptr;
    if (pre)
      stage_fp8_pre(a, lds, step0, nst);
    else
      stage_fp8_act(a, xs, lds, step0, nst);
  } else if constexpr (std::is_same<F, FmtInt8>::value) {
    static_assert(std::is_same<XS, XPlain>::value, "int8 activations are read from device memory");
    stage_int8_act(a, lds, step0, nst);
  } else {
    stage_bf16<F>(a, xs, lds, step0, nst);
  }
  stage_scales<F>(a, lds, tg, step0, nst);
  __syncthreads();
  if constexpr (needs_bias_totals<F>()) {
    if (stage_x) {
      stage_bias<F, WAVES>(a, lds, nst);
      __syncthreads();
    }
  }

  // ---- main loop
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  int xoff[MT], mrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    mrow[mt] = min(16 * mt + (lane & 15), a.m - 1);
    xoff[mt] = mrow[mt] * a.xstride;
  }
  // Steady state: PF steps per trip, every load unconditional. Prefetch addresses past the
  // wave's last step are clamped to it (a cache hit), so the body has no branches and the
  // compiler keeps PF steps of loads in flight instead of draining at every join.
  int j0 = 0;
  for (; j0 + PF <= my; j0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int srel = kwi + (j0 + p) * a.kw;
#pragma unroll
      for (int r = 0; r < RW; ++r)
        compute_step<F, MT, BMODE>(acc[r], buf[p][r], lds, a, srel, lane, xoff, mrow, (wt * RW + r) * 16 + 4 * (lane >> 4));
      // Refill the slot just consumed (same registers: no copies across the loop edge),
      // and keep the refill here rather than letting the scheduler sink it to the end.
      const int nxt = min(step0 + kwi + (j0 + p + PF) * a.kw, it.last);
#pragma unroll
      for (int r = 0; r < RW; ++r) load_chunk<F>(buf[p][r], a, it.wrow[r], nxt, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // Tail: the remaining (< PF) steps are already loaded.
#pragma unroll
  for (int p = 0; p < PF; ++p) {
    if (j0 + p < my) {
      const int srel = kwi + (j0 + p) * a.kw;
#pragma unroll
      for (int r = 0; r < RW; ++r)
        compute_step<F, MT, BMODE>(acc[r], buf[p][r], lds, a, srel, lane, xoff, mrow, (wt * RW + r) * 16 + 4 * (lane >> 4));
    }
  }

}

// Epilogue, first half: every wave's accumulators to LDS ([wave][RW][16 rows][16*MT]). With
// `guard`, first wait until every wave is done with what was there.
template <int MT, int RW, class Team = BlockTeam>
__device__ __forceinline__ void acc_to_lds(char* lds, const f32x4 (&acc)[RW][MT], const Team& team = {},
                                           bool guard = true) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (guard) team.sync();
  float* red = reinterpret_cast<float*>(lds);
  constexpr int RC = 16 * MT;
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[((wave * RW + r) * 16 + 4 * (lane >> 4) + i) * RC + 16 * mt + (lane & 15)] = acc[r][mt][i];
  team.sync();
}

// Output (tile tl of the block, tile row nl, token mm): the kw waves' sums (acc_to_lds at
// `redp`) added in wave order, then the format's scales (staged in `lds`).
template <class F, int MT, int RW>
__device__ __forceinline__ float tile_value(const GemmArgs& a, const char* redp, const char* lds, int tl, int nl,
                                            int mm) {
  constexpr int RC = 16 * MT, WSTRIDE = RW * 16 * RC;  // floats between two waves' partials
  const float* red = reinterpret_cast<const float*>(redp);
  const int slot = tl / RW, r = tl - slot * RW;  // tile tl of the block = slot's r-th tile
  const float* base = red + ((slot * a.kw * RW + r) * 16 + nl) * RC + mm;
  // Four waves' partials are read before any is added (one LDS round trip per four waves, not
  // one per wave); indices past kw repeat the last partial and are not added. The sum keeps
  // wave order.
  float v = 0.f;
  for (int w0 = 0; w0 < a.kw; w0 += 4) {
    float part[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) part[w] = base[min(w0 + w, a.kw - 1) * WSTRIDE];
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (w0 + w < a.kw) v += part[w];
  }
  return F::finish(a, lds, v, tl * 16 + nl, mm);
}

// Combine the kw waves of each tile, write the output (bf16, SwiGLU or fp32 planes), and
// when the row block is cut into pieces let the last workgroup to finish reduce the
// planes in piece order.
template <class F, int MT, int RW, int WAVES, bool SW, bool AN = false>
__device__ __forceinline__ void item_finish(const GemmArgs& a, char* lds, const Item<RW>& it,
                                            const f32x4 (&acc)[RW][MT]) {
  const int tg = it.tg, s = it.s, np = it.np;
  acc_to_lds<MT, RW>(lds, acc);
  auto combined = [&](int tl, int nl, int mm) -> float { return tile_value<F, MT, RW>(a, lds, lds, tl, nl, mm); };
  auto swiglu = [](float g, float u) -> float { return swiglu_bf(g, u); };

  // Outputs go out in row pairs (one 32-bit store of two bf16).
  constexpr int rows_out = SW ? 8 : 16;
  const int per_tile = (rows_out / 2) * a.m;
  const int total = a.rt * per_tile;
  const bool direct = np == 1 || a.mode == QLX_MODE_PLANES;
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int tl = idx / per_tile, rem = idx - tl * per_tile;
    const int mm = rem / (rows_out / 2), nl = 2 * (rem - mm * (rows_out / 2));
    const int tile = tg * a.rt + tl;
    if (tile >= a.ntiles) continue;
    if (SW) {
      const float g0 = combined(tl, nl, mm), u0 = combined(tl, nl + 8, mm);
      const float g1 = combined(tl, nl + 1, mm), u1 = combined(tl, nl + 9, mm);
      if (direct) {
        store_pair(y, (size_t)mm * a.half + 8 * tile + nl, swiglu(g0, u0), swiglu(g1, u1));
      } else {
        float* pl = a.work + ((size_t)s * a.m + mm) * a.n + 8 * tile + nl;
        store_coherent(pl, g0);
        store_coherent(pl + 1, g1);
        store_coherent(pl + a.half, u0);
        store_coherent(pl + a.half + 1, u1);
      }
    } else {
      const int row = 16 * tile + nl;
      if (row >= a.n) continue;
      const bool two = row + 1 < a.n;
      const float v0 = combined(tl, nl, mm), v1 = two ? combined(tl, nl + 1, mm) : 0.f;
      float* pl = a.work + ((size_t)s * a.m + mm) * a.n + row;
      if (a.mode == QLX_MODE_PLANES) {
        pl[0] = v0;
        if (two) pl[1] = v1;
      } else if (!direct) {
        store_coherent(pl, v0);
        if (two) store_coherent(pl + 1, v1);
      } else if (two && (a.n & 1) == 0) {
        if constexpr (AN)
          store_pair_coherent(y, (size_t)mm * a.n + row, v0, v1);
        else
          store_pair(y, (size_t)mm * a.n + row, v0, v1);
      } else {
        y[(size_t)mm * a.n + row] = f2bf(v0);
        if (two) y[(size_t)mm * a.n + row + 1] = f2bf(v1);
      }
    }
  }
  if (direct) {
    if constexpr (AN) add_norm_ticket(a);
    return;
  }

  // ---- split-K: the last workgroup of this row block reduces the planes in slice order.
  // The partials went out with device-coherent stores; every wave waits for its stores to
  // complete before the ticket is taken, and the last workgroup reads them with
  // device-coherent loads. No L2 write-back/invalidate of the whole cache is needed (an
  // agent-scope fence would emit one per workgroup).
  __shared__ int s_last;
  publish_stores();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&a.tickets[tg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == np - 1;
    if (s_last) __hip_atomic_store(&a.tickets[tg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const size_t plane = (size_t)a.m * a.n;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int tl = idx / per_tile, rem = idx - tl * per_tile;
    const int mm = rem / (rows_out / 2), nl = 2 * (rem - mm * (rows_out / 2));
    const int tile = tg * a.rt + tl;
    if (tile >= a.ntiles) continue;
    if (SW) {
      const float* pg = a.work + (size_t)mm * a.n + 8 * tile + nl;
      float g0 = 0.f, u0 = 0.f, g1 = 0.f, u1 = 0.f;
      for (int sp = 0; sp < np; ++sp) {
        g0 += load_coherent(pg + sp * plane);
        g1 += load_coherent(pg + sp * plane + 1);
        u0 += load_coherent(pg + sp * plane + a.half);
        u1 += load_coherent(pg + sp * plane + a.half + 1);
      }
      store_pair(y, (size_t)mm * a.half + 8 * tile + nl, swiglu(g0, u0), swiglu(g1, u1));
    } else {
      const int row = 16 * tile + nl;
      if (row >= a.n) continue;
      const bool two = row + 1 < a.n;
      const float* p = a.work + (size_t)mm * a.n + row;
      float v0 = 0.f, v1 = 0.f;
      for (int sp = 0; sp < np; ++sp) {
        v0 += load_coherent(p + sp * plane);
        if (two) v1 += load_coherent(p + sp * plane + 1);
      }
      if (two && (a.n & 1) == 0) {
        if constexpr (AN)
          store_pair_coherent(y, (size_t)mm * a.n + row, v0, v1);
        else
          store_pair(y, (size_t)mm * a.n + row, v0, v1);
      } else {
        y[(size_t)mm * a.n + row] = f2bf(v0);
        if (two) y[(size_t)mm * a.n + row + 1] = f2bf(v1);
      }
    }
  }
  if constexpr (AN) add_norm_ticket(a);
}

// One launch = one linear call. SW: the SwiGLU epilogue (a separate instantiation, so
// profiles tell it apart); AN: the fused residual add + RMSNorm after the last row block.
template <class F, int MT, int RW, int WAVES, bool SW, bool AN = false>
__global__ void __launch_bounds__(WAVES * 64) gemm_kernel(GemmArgs a) {
  extern __shared__ __align__(16) char lds[];
  int tg, s;
  block_coords(a, blockIdx.x, tg, s);
  Item<RW> it;
  uint4 buf[PipeDepth<F, RW>::PF][RW][F::LOADS];
  item_prefetch<F, RW>(a, tg, s, it, buf);
  f32x4 acc[RW][MT];
  item_main<F, MT, RW, WAVES>(a, XPlain{}, lds, it, buf, acc);
  item_finish<F, MT, RW, WAVES, SW, AN>(a, lds, it, acc);
}

// Epilogue of the persistent kernel: the waves' sums go to their own LDS area (a.off_red), so
// the staged activation stays for the workgroup's next item; bf16 or SwiGLU outputs (whole K,
// whole 16-row tiles).
template <class F, int MT, int RW, int WAVES, bool SW>
__device__ __forceinline__ void persist_finish(const GemmArgs& a, char* lds, const Item<RW>& it,
                                               const f32x4 (&acc)[RW][MT]) {
  char* red = lds + a.off_red;
  acc_to_lds<MT, RW>(red, acc, BlockTeam{}, false);  // the area's last readers passed a barrier since
  constexpr int rows_out = SW ? 8 : 16;
  const int per_tile = (rows_out / 2) * a.m;
  const int total = a.rt * per_tile;
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int tl = idx / per_tile, rem = idx - tl * per_tile;
    const int mm = rem / (rows_out / 2), nl = 2 * (rem - mm * (rows_out / 2));
    const int tile = it.tg * a.rt + tl;
    if (tile >= a.ntiles) continue;
    if constexpr (SW) {
      const float g0 = tile_value<F, MT, RW>(a, red, lds, tl, nl, mm);
      const float u0 = tile_value<F, MT, RW>(a, red, lds, tl, nl + 8, mm);
      const float g1 = tile_value<F, MT, RW>(a, red, lds, tl, nl + 1, mm);
      const float u1 = tile_value<F, MT, RW>(a, red, lds, tl, nl + 9, mm);
      store_pair(y, (size_t)mm * a.half + 8 * tile + nl, swiglu_bf(g0, u0), swiglu_bf(g1, u1));
    } else {
      const float v0 = tile_value<F, MT, RW>(a, red, lds, tl, nl, mm);
      const float v1 = tile_value<F, MT, RW>(a, red, lds, tl, nl + 1, mm);
      store_pair(y, (size_t)mm * a.n + 16 * tile + nl, v0, v1);
    }
  }
}

// A single call as a persistent launch: workgroup b takes row blocks b, b + grid, ... (whole
// K). The activation (FP8: its codes and token scales) is staged once; the next row block's
// first weight steps are issued before the current one's epilogue, so the weight stream does
// not stop at row-block boundaries and no workgroup launch sits between them. Formats with the
// fused code bias compute its totals on the first row block only (BMODE 1) and read them back
// on the rest (BMODE 2): bit-identical sums, about half the MFMAs. The launch guarantees every
// workgroup at least two row blocks, so each first row block is a whole one.
template <class F, int MT, int RW, int WAVES, bool SW>
__global__ void __launch_bounds__(WAVES * 64) gemm_persist_kernel(GemmArgs a) {
  extern __shared__ __align__(16) char lds[];
  constexpr bool CACHE = std::is_same<F, FmtW4>::value || std::is_same<F, FmtW8>::value;
  int tg = blockIdx.x;
  Item<RW> it;
  uint4 buf[PipeDepth<F, RW>::PF][RW][F::LOADS];
  item_prefetch<F, RW>(a, tg, 0, it, buf);
  f32x4 acc[RW][MT];
  for (bool first = true;; first = false) {
    if constexpr (CACHE) {
      if (first)
        item_main<F, MT, RW, WAVES, XPlain, 1>(a, XPlain{}, lds, it, buf, acc, true);
      else
        item_main<F, MT, RW, WAVES, XPlain, 2>(a, XPlain{}, lds, it, buf, acc, false);
    } else {
      item_main<F, MT, RW, WAVES, XPlain, 0>(a, XPlain{}, lds, it, buf, acc, first);
    }
    const int nt = tg + (int)gridDim.x;
    const Item<RW> cur = it;
    if (nt < a.tile_groups) item_prefetch<F, RW>(a, nt, 0, it, buf);
    persist_finish<F, MT, RW, WAVES, SW>(a, lds, cur, acc);
    if (nt >= a.tile_groups) break;
    tg = nt;
    __syncthreads();  // scales and partial sums are restaged for the next row block
  }
}

// ---- persistent single calls with a direct-to-LDS weight ring (4-bit weights) ---------
//
// The register pipeline keeps PipeDepth steps in flight per wave, and 4-bit weights, whose
// dequantization holds many registers, get 3: 48 KB per CU, too few bytes to cover HBM
// latency. Here each wave streams its steps into a ring of D slots in LDS instead
// (global_load_lds_dwordx4: lane i's 16 bytes land at slot + 16 i, counted by vmcnt like any
// load), D steps ahead of its MFMAs, and the ring runs on across row blocks: a workgroup's
// steps form one sequence, so the next row block's first steps are in flight while the current
// one finishes. The row block's group scales come the same way, one row block ahead, into a
// double buffer. One 16-row tile per wave over the whole K (kw = 1), so a wave's outputs need
// no cross-wave sum and are stored from its registers. The arithmetic and its order are the
// register pipeline's (FmtW4::compute): the outputs are bit-identical.
//
// Waits are explicit. Every LDS access of the steady state is an assembler instruction, and
// global loads are all LDS DMA: a compiler-visible LDS access after an LDS DMA would make the
// compiler wait for every DMA in flight. A ring slot is read after s_waitcnt vmcnt((D - 1) *
// LOADS): the D - 1 later steps may still be out. Loads complete in order, and anything else
// issued in between (scales, stores) only makes that wait longer, never short.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
__device__ __forceinline__ u32x4 ds_read16(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ float ds_read4f(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void ds_write4f(uint32_t addr, float v) {
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left open).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt holds 0..63");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier that waits for this wave's LDS operations but not for its loads in flight
// (a __syncthreads fence would wait for the ring's DMA); the memory clobber keeps the compiler
// from moving memory operations across it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void dma16(const void* src, char* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 2);
}
// 16 bytes per lane at buffer offset voff + soff into LDS at dst + 16 lane (the same non-temporal
// policy as dma16): the vector offset can stay fixed while the scalar one advances.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, int soff, char* dst) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)dst, 16, (int)voff, soff, 0, 2);
}
__device__ __forceinline__ void dma4(const void* src, char* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
}

// LDS of the ring kernel, after the activation (a.off_sc .. : [2][scale words] raw scale
// pairs, then the code-bias totals [step][2][16] floats, then the rings [wave][D][2 KB]).
__host__ __device__ inline int ring_scale_words(int nsteps, int rt) { return (nsteps * 16 * rt + 63) & ~63; }

template <int WAVES, bool BM1>
__device__ __forceinline__ void ring_step_w4(f32x4& acc, const u32x4 (&c)[2], uint32_t xa, uint32_t sa, uint32_t ba,
                                             int lane) {
  // xa: this lane's activation bytes of the step (token row, lane group), sa: its four rows'
  // scale pairs of the step, ba: the step's code-bias totals (its token column).
  u32x4 bv[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int t = 0; t < 4; ++t) bv[j][t] = ds_read16(xa + j * 256 + t * 16);
  u32x4 sp = ds_read16(sa);
  float bt[2] = {0.f, 0.f};
  if constexpr (!BM1) {
    bt[0] = ds_read4f(ba);
    bt[1] = ds_read4f(ba + 64);
  }
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(bv[0][0]), "+v"(bv[0][1]), "+v"(bv[0][2]), "+v"(bv[0][3]), "+v"(bv[1][0]), "+v"(bv[1][1]),
                 "+v"(bv[1][2]), "+v"(bv[1][3]), "+v"(bt[0]), "+v"(bt[1]), "+v"(sp)
               :
               : "memory");
  const uint4 avb = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};  // bf16 136
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    f32x4 tmp = {0.f, 0.f, 0.f, 0.f}, tb = {0.f, 0.f, 0.f, 0.f};
    const uint32_t wd[4] = {c[j][0], c[j][1], c[j][2], c[j][3]};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      uint4 av;
      av.x = nib_pair(wd[t], 0);
      av.y = nib_pair(wd[t], 4);
      av.z = nib_pair(wd[t], 8);
      av.w = nib_pair(wd[t], 12);
      const uint4 b = uint4{bv[j][t][0], bv[j][t][1], bv[j][t][2], bv[j][t][3]};
      tmp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av), as_bf16x8(b), tmp, 0, 0, 0);
      if constexpr (BM1) tb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(avb), as_bf16x8(b), tb, 0, 0, 0);
    }
    if constexpr (BM1) {
      // Through a VALU copy (an identity DPP move): the compiler pads an MFMA result's readers
      // with the wait states it needs, but not an assembler statement's.
      const float v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(tb[0]), 0xe4, 0xf, 0xf, false));
      if (lane < 16) ds_write4f(ba + j * 64, v);
    } else {
      tb = f32x4{bt[j], bt[j], bt[j], bt[j]};
    }
    // scale of row i, group j: half j of the row's pair (bf16 bits)
    f32x4 s4;
#pragma unroll
    for (int i = 0; i < 4; ++i) s4[i] = bf2f(j ? sp[i] >> 16 : sp[i] & 0xffffu);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(s4[i], tmp[i] - tb[i], acc[i]);
  }
}

template <int WAVES, int D, int WPC>
__global__ void __launch_bounds__(WAVES * 64, WPC * WAVES / 4) gemm_ring_w4_kernel(GemmArgs a) {
  extern __shared__ __align__(16) char lds[];
  static_assert(D >= 2 && (D - 1) * 2 <= 63, "vmcnt holds at most 63");
  using F = FmtW4;
  constexpr int L = F::LOADS, SLOT = L * 1024;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = gridDim.x, ns = a.nsteps, rows = 16 * a.rt;
  const int nitems = (a.tile_groups - (int)blockIdx.x + G - 1) / G;  // row blocks b, b + G, ...
  const int total = nitems * ns;                                      // this wave's steps
  const int sw = ring_scale_words(ns, a.rt);
  char* sbuf = lds + a.off_sc;  // [2][sw] scale pairs
  char* ring = lds + a.off_ring + wave * (D * SLOT);
  const uint32_t ring_a = lds_addr(ring) + lane * 16;
  const uint32_t* ws = reinterpret_cast<const uint32_t*>(a.ws);
  // The scale pairs of row block `item` into buffer `item & 1`, word q = step * rows + row;
  // each DMA moves 64 words, and this wave moves every WAVES-th of them.
  auto scales = [&](int item) {
    const int tg = (int)blockIdx.x + item * G;
    char* dst = sbuf + (item & 1) * (sw * 4);
    for (int t = wave; t * 64 < sw; t += WAVES) {
      int q = t * 64 + lane;
      q = q < ns * rows ? q : ns * rows - 1;  // lanes past the end reread the last word
      const int st = q / rows, rl = q - st * rows, tile = tg * a.rt + (rl >> 4);
      const int row = weight_row(a, tile < a.ntiles ? tile : a.ntiles - 1, rl & 15);
      dma4(ws + (size_t)row * (a.k >> 8) + st, dst + t * 256);
    }
  };
  auto tile_of = [&](int item) {  // the wave's tile of row block `item` (past the end: dropped)
    const int tile = ((int)blockIdx.x + item * G) * a.rt + wave;
    return __builtin_amdgcn_readfirstlane(tile < a.ntiles ? tile : a.ntiles - 1);
  };
  auto wrow_of = [&](int item) { return weight_row(a, tile_of(item), lane & 15); };
  // Tile-layout weights (the launch takes whole tiles and bf16 outputs): step s of a tile is the
  // 2 KB block (tile * k / 256 + s) * 2048, lane l's 16 bytes of half j at j * 1024 + 16 l --
  // read through a buffer resource with that block's offset as the scalar offset and the lane's
  // as a fixed vector offset, so issuing a step costs no vector instruction. Row-major weights
  // (or tiles past 4 GB) go through chunk_ptr.
  const int spr = a.k >> 8;
  const uint32_t lane_off = (uint32_t)lane * 16u;
  const unsigned long long wbytes = (unsigned long long)a.ntiles * spr * 2048ull;
  const bool by_buffer = a.tiled && wbytes < (1ull << 31);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.w), (short)0, by_buffer ? (int)wbytes : 0, 0x00020000);
  int ig = 0, ii = 0, is = 0, it = tile_of(0), iw = wrow_of(0);  // next step to issue: row block ii, step is
  auto issue = [&]() {
    char* slot = ring + (ig % D) * SLOT;
    if (by_buffer) {
      const int soff = (it * spr + is) * 2048;
#pragma unroll
      for (int j = 0; j < L; ++j) dma16_buf(wr, lane_off + j * 1024u, soff, slot + j * 1024);
    } else {
#pragma unroll
      for (int j = 0; j < L; ++j) dma16(F::chunk_ptr(a, iw, is, lane, j), slot + j * 1024);
    }
    ++ig;
    if (++is == ns) {
      is = 0;
      if (++ii < nitems) {
        it = tile_of(ii);
        iw = wrow_of(ii);
      }
    }
  };
  // Prologue: row block 0's scales, the activation (its LDS writes wait for nothing else in
  // flight), then the ring's first D steps (the launch guarantees total >= D).
  scales(0);
  stage_bf16<F>(a, XPlain{}, lds, 0, ns);
#pragma unroll
  for (int p = 0; p < D; ++p) issue();
  wait_vm<D * L>();  // this wave's scale DMAs, issued before the ring's
  barrier_lds();
  const int mrow = min(lane & 15, a.m - 1);
  const uint32_t xa0 = lds_addr(lds) + mrow * a.xstride + (lane >> 4) * 64;
  const uint32_t bt0 = lds_addr(lds) + a.off_bt + (lane & 15) * 4;
  const int rowl = wave * 16 + 4 * (lane >> 4);
  uint16_t* y = reinterpret_cast<uint16_t*>(a.y);
  for (int item = 0, g = 0; item < nitems; ++item) {
    if (item + 1 < nitems) scales(item + 1);
    const int ig0 = ig;
    const uint32_t sa0 = lds_addr(sbuf) + (item & 1) * (sw * 4) + rowl * 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < ns; ++s, ++g) {
      if (ig - g == D)
        wait_vm<(D - 1) * L>();
      else
        wait_vm<0>();
      u32x4 c[L];
#pragma unroll
      for (int j = 0; j < L; ++j) c[j] = ds_read16(ring_a + (g % D) * SLOT + j * 1024);
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(c[0]), "+v"(c[1]) : : "memory");
      if (ig < total) issue();  // the slot just read is free again
      const uint32_t xa = xa0 + s * 512, sa = sa0 + s * rows * 4, ba = bt0 + s * 128;
      if (item == 0)
        ring_step_w4<WAVES, true>(acc, c, xa, sa, ba, lane);
      else
        ring_step_w4<WAVES, false>(acc, c, xa, sa, ba, lane);
    }
    // Outputs from registers: lane (r, c) holds rows 4 (lane >> 4) .. + 3 of the wave's tile
    // for token lane & 15 (0 + v: a -0 sum leaves as +0, as the LDS sum in tile_value does).
    const int tile = ((int)blockIdx.x + item * G) * a.rt + wave, mm = lane & 15;
    if (tile < a.ntiles && mm < a.m) {
      const int r0 = 16 * tile + 4 * (lane >> 4);
      if (r0 + 1 < a.n) store_pair(y, (size_t)mm * a.n + r0, 0.f + acc[0], 0.f + acc[1]);
      if (r0 + 3 < a.n) store_pair(y, (size_t)mm * a.n + r0 + 2, 0.f + acc[2], 0.f + acc[3]);
    }
    // The next row block's scales (issued before this one's ring refills) have landed once all
    // but the refills since are in; then the buffer and the code-bias totals are shared.
    if (item + 1 < nitems) {
      if (ig - ig0 >= D - 1)
        wait_vm<(D - 1) * L>();
      else
        wait_vm<0>();
    }
    barrier_lds();
  }
}

}  // namespace qlx
