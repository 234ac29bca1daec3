// Grouped-query decode attention over the KV cache, split along the key length
// (engine/kernels/attention.py:37-227: split kernel, merge kernel, DecodeAttention).
//
// One workgroup per (sequence x KV head, split); its four waves take 32-key blocks in turn.
// The R = tokens x group query rows of a KV head share every key and value it reads:
//
//   S^T = K Q^T   on v_mfma_f32_16x16x32_bf16: A = 16 keys x 32 dims (a lane's 16-byte load
//                 of one key row), B = Q^T (the rows' query fragments, held in registers).
//                 The C fragment leaves each lane 8 keys of one query row, which is exactly
//                 the A fragment the P V product needs, so P never goes through LDS.
//   O += P V      A = bf16(P) 16 rows x 32 keys, B = V. A lane loads 8 consecutive values of 8
//                 keys (eight 16-byte loads) and transposes that 8 x 8 block in registers; the
//                 8 products of a block take output columns d = 8 n + j (j = 0..7), which
//                 covers the 128 dims with every lane's block used once.
//
// Softmax follows the reference: fp32 scores and running maximum, p = exp(s - max), the
// row total summed from fp32 p, the P V product from bf16 p, acc / total at the end
// (attention.py:102-137). Exponentials are base 2 on scores pre-multiplied by log2(e).
// The split partials merge as in attention.py:144-178: weights exp(max_s - max), sum of
// weighted accumulators over sum of weighted totals, in a small second kernel (one workgroup per
// head). Merging in the attention launch itself -- the last workgroup of a head, found with a
// ticket -- measured slower: the partial stores' acknowledgement, the ticket and the merge's
// loads are three device-scope round trips (6 us of 12.9 at batch 1, 4096 keys, 32 splits).
//
// Splits are a parallelism knob, not a fixed key range: 32-key blocks are dealt round-robin
// (block j to split j % S, then to wave (j / S) % 4), so the live blocks -- the live length
// pos + tokens is read on the device -- spread over the splits whatever the capacity, a
// wave's first block can be fetched before the position arrives, and the grid stays fixed for
// graph capture. A short context uses fewer splits (one block per wave at least); with one,
// the workgroup writes the output itself.
#include "attn_common.h"
#include "../../include/qlinear.h"

#include <algorithm>

namespace qlx {

struct AttnArgs {
  const uint16_t* q;   // bf16 [B*T][H*G*128]
  const void* k;       // bf16 or int8 [B][H][cap][128]
  const void* v;
  const float* ks;     // fp32 [B][H][cap] (INT8 cache)
  const float* vs;
  const int* pos;      // base position of token 0
  uint16_t* out;       // bf16 [B*T][H*G*128]
  float* pacc;         // split partials: [B*H][S][R][128], then maxima and totals [B*H][S][R]
  float scale2;        // head_dim^-0.5 * log2(e)
  int cap, splits, T, G, H, R, heads;
};

// RT tiles of 16 query rows (R <= 16 RT). 256 threads; dynamic LDS 4 x R x 128 fp32.
template <int RT, bool Q8>
__global__ void __launch_bounds__(256) attn_kernel(AttnArgs a) {
  extern __shared__ float wacc[];  // [4 waves][R][128]
  __shared__ float wm[4][64], wl[4][64];
  const int head = blockIdx.x, part = blockIdx.y;
  // wave index and position in scalar registers: block bounds and loop trips are wave-uniform
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int seq = head / a.H, kvh = head - seq * a.H;
  const int NQ = a.H * a.G;
  const size_t hb = (size_t)head * a.cap * 128;
  // Key blocks of 32 are dealt round-robin: block j to split j % S, and within the split to
  // wave (j / S) % 4. A wave's first block is then known before the position is: its K/V loads
  // (clamped to the capacity, always valid memory) and the query loads go out at entry, and
  // the position read overlaps them.
  const int j0 = part + a.splits * w;
  constexpr bool PF = RT <= 2;  // prefetch the next block (registers allow it up to 2 row tiles)
  KVBlock<Q8> cur, nxt;
  const KVSrc kv{a.k, a.v, a.ks, a.vs};
  if (PF && 32 * j0 < a.cap) cur.load(kv, hb, 32 * j0, a.cap, n, g);

  // Query fragments (B operand of S^T = K Q^T): row 16 rt + n, dims kdim(s, g). Up to two row
  // tiles live in registers; more are read from LDS each block (the four waves share them),
  // which with no prefetched block keeps the wave within its registers.
  constexpr bool QLDS = RT >= 3;
  __shared__ u32x4 qlds[QLDS ? RT * 4 * 64 : 1];
  u32x4 qf[QLDS ? 1 : RT][4];
  auto qload = [&](int rt, int s) -> u32x4 {
    const int r = 16 * rt + n;
    if (r >= a.R) return u32x4{0u, 0u, 0u, 0u};
    const int t = r / a.G, gi = r - t * a.G;
    const uint16_t* qp = a.q + ((size_t)(seq * a.T + t) * NQ + kvh * a.G + gi) * 128 + kdim<Q8>(s, g);
    return *gmem(reinterpret_cast<const u32x4*>(qp));
  };
  if constexpr (QLDS) {
    for (int i = w; i < RT * 4; i += 4) qlds[i * 64 + lane] = qload(i >> 2, i & 3);
    __syncthreads();
  } else {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int s = 0; s < 4; ++s) qf[rt][s] = qload(rt, s);
  }
  auto qfrag = [&](int rt, int s) -> u32x4 {
    if constexpr (QLDS) return qlds[(rt * 4 + s) * 64 + lane];
    else return qf[rt][s];
  };
  const int base = __builtin_amdgcn_readfirstlane(a.pos[0]);
  const int end = min(base + a.T, a.cap);  // keys at or past end are live for no row
  const int nblk = end > 0 ? (end + 31) >> 5 : 0;
  // Splits in use: at least one block per wave each (a short context on many splits would
  // only add partials and merge work). Workgroups past them leave now; when fewer splits
  // are used than launched, waves past the first fetch their first block again.
  const int se = max(1, min(a.splits, (nblk + 3) >> 2));
  if (part >= se) return;
  const int j1 = part + se * w, jstep1 = 4 * se;
  const int nb = j1 < nblk ? (nblk - j1 + jstep1 - 1) / jstep1 : 0;  // this wave's blocks
  if (PF && j1 != j0 && nb > 0) cur.load(kv, hb, 32 * j1, a.cap, n, g);
  // Last live key + 1 of row 16 rt + n (padding rows: every live key).
  int lim[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = 16 * rt + n;
    lim[rt] = r < a.R ? min(base + r / a.G + 1, end) : end;
  }

  float m[RT], l[RT];
  f32x4 acc[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    m[rt] = kNegInf;
    l[rt] = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](const KVBlock<Q8>& b, int kb) __attribute__((always_inline)) {
    u32x4 kf[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[kt][s] = b.kfrag(kt, s);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      f32x4 st[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        st[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s)
          st[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf8(kf[kt][s]), bf8(qfrag(rt, s)), st[kt], 0, 0, 0);
      }
      // lane: row 16 rt + n, keys kb + 16 kt + 4 g + i
      float sc[8];
      float bm = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb + 16 * kt + 4 * g + i;
          sc[4 * kt + i] = key < lim[rt] ? st[kt][i] * a.scale2 : kNegInf;
          bm = fmaxf(bm, sc[4 * kt + i]);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m[rt], bm);
      const float mu = mn == kNegInf ? 0.f : mn;  // a row with no live key yet keeps p = 0
      const float carry = ex2(m[rt] - mu);
      m[rt] = mn;
      float p[8], ps = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = ex2(sc[j] - mu);
        ps += p[j];
      }
      l[rt] = l[rt] * carry + ps;
      const u32x4 pf = u32x4{pack_bf(p[0], p[1]), pack_bf(p[2], p[3]), pack_bf(p[4], p[5]), pack_bf(p[6], p[7])};
      // acc rows 4 g + i of this tile take the carry of the lane holding that row
      float cr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) cr[i] = __shfl(carry, 4 * g + i, 64);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        f32x4 t = acc[rt][c];
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] *= cr[i];
        acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf8(pf), bf8(b.vfrag(c)), t, 0, 0, 0);
      }
    }
  };

  // The last block may run past `end`: its values there are zeroed (P is 0 there, and 0 times
  // whatever the cache holds past the live keys could be NaN).
  auto run = [&](KVBlock<Q8>& b, int j) __attribute__((always_inline)) {
    const int kb = 32 * j;
    if (kb + 32 > end) b.zero_from(kb, end, g);
    compute(b, kb);
  };
  if constexpr (PF) {
    if (nb > 0) {
      int i = 0;
      // (sched_barrier: the scheduler would otherwise sink the prefetch below the first
      // products of the current block, behind a wait for every load in flight)
      for (; i + 2 < nb; i += 2) {
        nxt.load(kv, hb, 32 * (j1 + jstep1 * (i + 1)), a.cap, n, g);
        __builtin_amdgcn_sched_barrier(0);
        run(cur, j1 + jstep1 * i);
        cur.load(kv, hb, 32 * (j1 + jstep1 * (i + 2)), a.cap, n, g);
        __builtin_amdgcn_sched_barrier(0);
        run(nxt, j1 + jstep1 * (i + 1));
      }
      if (i + 1 < nb) {
        nxt.load(kv, hb, 32 * (j1 + jstep1 * (i + 1)), a.cap, n, g);
        __builtin_amdgcn_sched_barrier(0);
        run(cur, j1 + jstep1 * i);
        run(nxt, j1 + jstep1 * (i + 1));
      } else {
        run(cur, j1 + jstep1 * i);
      }
    }
  } else {
    for (int i = 0; i < nb; ++i) {
      cur.load(kv, hb, 32 * (j1 + jstep1 * i), a.cap, n, g);
      run(cur, j1 + jstep1 * i);
    }
  }

  // Merge the four waves: wave maxima and totals, then each wave's accumulator rescaled to
  // the workgroup maximum, summed over waves in order.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float lt = l[rt] + __shfl_xor(l[rt], 16, 64);
    lt = lt + __shfl_xor(lt, 32, 64);
    const int r = 16 * rt + n;
    if (g == 0 && r < a.R) {
      wm[w][r] = m[rt];
      wl[w][r] = lt;
    }
  }
  __syncthreads();
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rt + 4 * g + i;
      if (r >= a.R) continue;
      const float M = fmaxf(fmaxf(wm[0][r], wm[1][r]), fmaxf(wm[2][r], wm[3][r]));
      const float f = wm[w][r] == kNegInf ? 0.f : ex2(wm[w][r] - M);
      float* dst = wacc + ((size_t)w * a.R + r) * 128 + 8 * n;
      f32x4 lo, hi;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        lo[c] = acc[rt][c][i] * f;
        hi[c] = acc[rt][c + 4][i] * f;
      }
      *reinterpret_cast<f32x4*>(dst) = lo;
      *reinterpret_cast<f32x4*>(dst + 4) = hi;
    }
  }
  __syncthreads();

  // Workgroup result per (row, 4 dims): maximum M, total L, accumulator A (waves in order).
  auto wg_result = [&](int r, int d4, float& M, float& L) -> f32x4 {
    M = fmaxf(fmaxf(wm[0][r], wm[1][r]), fmaxf(wm[2][r], wm[3][r]));
    L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float f = wm[q][r] == kNegInf ? 0.f : ex2(wm[q][r] - M);
      L += wl[q][r] * f;
      A += *reinterpret_cast<const f32x4*>(wacc + ((size_t)q * a.R + r) * 128 + d4);
    }
    return A;
  };
  auto store_out = [&](int r, int d4, f32x4 A, float L) {
    const int t = r / a.G, gi = r - t * a.G;
    uint16_t* o = a.out + ((size_t)(seq * a.T + t) * NQ + kvh * a.G + gi) * 128 + d4;
    *gmem(reinterpret_cast<u32x2*>(o)) = u32x2{pack_bf(A[0] / L, A[1] / L), pack_bf(A[2] / L, A[3] / L)};
  };
  const int items = a.R * 32;
  if (se == 1) {
    for (int idx = threadIdx.x; idx < items; idx += 256) {
      const int r = idx >> 5, d4 = (idx & 31) * 4;
      float M, L;
      const f32x4 A = wg_result(r, d4, M, L);
      store_out(r, d4, A, L);
    }
    return;
  }

  // Several splits: this split's partial goes out with plain stores; the merge kernel that
  // follows on the stream (the kernel boundary makes them visible) combines the live splits.
  // Partials: acc [heads][S][R][128], then maxima and totals [heads][S][R].
  const size_t pb = ((size_t)head * a.splits + part) * a.R;
  const size_t nslot = (size_t)a.heads * a.splits * a.R;
  for (int idx = threadIdx.x; idx < items; idx += 256) {
    const int r = idx >> 5, d4 = (idx & 31) * 4;
    float M, L;
    const f32x4 A = wg_result(r, d4, M, L);
    *gmem(reinterpret_cast<f32x4*>(a.pacc + (pb + r) * 128 + d4)) = A;
    if (d4 == 0) {
      gmem(a.pacc)[nslot * 128 + pb + r] = M;
      gmem(a.pacc)[nslot * 129 + pb + r] = L;
    }
  }
}

// Merge of the split partials of one query row of one head (a workgroup per sequence x KV head
// x row: its loads spread over that many CUs, not one per head): the splits in use (se, from
// the same position) combine as in attention.py:144-178 -- weights exp(max_s - max), weighted
// accumulators over weighted totals -- in a fixed order. ng thread groups share an item's
// splits (contiguous ranges); a thread issues the loads of up to 16 splits at once (one memory
// round trip), merges them, and the groups' results combine in group order through LDS. With
// one split in use the attention kernel wrote the output itself.
__global__ void __launch_bounds__(256) attn_merge_kernel(AttnArgs a) {
  extern __shared__ float gbuf[];  // the groups' results: 6 floats per slot
  const int head = blockIdx.x;
  const int seq = head / a.H, kvh = head - seq * a.H;
  const int NQ = a.H * a.G;
  const int base = __builtin_amdgcn_readfirstlane(a.pos[0]);
  const int end = min(base + a.T, a.cap);
  const int nblk = end > 0 ? (end + 31) >> 5 : 0;
  const int se = max(1, min(a.splits, (nblk + 3) >> 2));
  if (se == 1) return;
  const int items = 32, row = blockIdx.y;  // items: the row's 4-value chunks
  const int ng = 256 / items;
  const int per = (se + ng - 1) / ng;
  const int slots = items * ng;
  const size_t nslot = (size_t)a.heads * a.splits * a.R;
  const size_t hb0 = (size_t)head * a.splits * a.R;
  const float* P = a.pacc;
  f32x4* ga = reinterpret_cast<f32x4*>(gbuf);
  float* gm = gbuf + 4 * slots;
  float* gl = gm + slots;
  for (int w0 = threadIdx.x; w0 < slots; w0 += 256) {
    const int item = w0 % items, sg = w0 / items;
    const int r = row, d4 = (item & 31) * 4;
    const int s_lo = sg * per, s_hi = min(se, s_lo + per);
    float Mt = kNegInf, Lt = 0.f;
    f32x4 At = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = s_lo; b0 < s_hi; b0 += 16) {
      float mv[16], lv[16];
      f32x4 av[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const size_t o = hb0 + (size_t)min(b0 + j, s_hi - 1) * a.R + r;
        mv[j] = gmem(P)[nslot * 128 + o];
        lv[j] = gmem(P)[nslot * 129 + o];
        av[j] = *gmem(reinterpret_cast<const f32x4*>(P + o * 128 + d4));
      }
      float Mb = Mt;
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (b0 + j < s_hi) Mb = fmaxf(Mb, mv[j]);
      const float Mu = Mb == kNegInf ? 0.f : Mb;
      const float c = Mt == kNegInf ? 0.f : ex2(Mt - Mu);
      At *= c;
      Lt *= c;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (b0 + j >= s_hi || mv[j] == kNegInf) continue;
        const float f = ex2(mv[j] - Mu);
        At += f * av[j];
        Lt += f * lv[j];
      }
      Mt = Mb;
    }
    ga[w0] = At;
    gm[w0] = Mt;
    gl[w0] = Lt;
  }
  __syncthreads();
  for (int item = threadIdx.x; item < items; item += 256) {
    float M = kNegInf;
    for (int g2 = 0; g2 < ng; ++g2) M = fmaxf(M, gm[g2 * items + item]);
    float L = 0.f;
    f32x4 A = {0.f, 0.f, 0.f, 0.f};
    for (int g2 = 0; g2 < ng; ++g2) {
      const float mg = gm[g2 * items + item];
      if (mg == kNegInf) continue;
      const float f = ex2(mg - M);
      A += f * ga[g2 * items + item];
      L += f * gl[g2 * items + item];
    }
    const int r = row, d4 = (item & 31) * 4;
    const int t = r / a.G, gi = r - t * a.G;
    uint16_t* o = a.out + ((size_t)(seq * a.T + t) * NQ + kvh * a.G + gi) * 128 + d4;
    *gmem(reinterpret_cast<u32x2*>(o)) = u32x2{pack_bf(A[0] / L, A[1] / L), pack_bf(A[2] / L, A[3] / L)};
  }
}

template <int RT, bool Q8>
static int launch_attn(const AttnArgs& a, int heads, hipStream_t st) {
  attn_kernel<RT, Q8><<<dim3(heads, a.splits), 256, (size_t)4 * a.R * 128 * sizeof(float), st>>>(a);
  if (a.splits > 1) {
    attn_merge_kernel<<<dim3(heads, a.R), 256, 6 * 256 * sizeof(float), st>>>(a);
  }
  QLX_LAUNCH_CHECK("decode attention");
}

}  // namespace qlx

using namespace qlx;

extern "C" int qlx_attention_workspace(int batch, int n_kv, int group, int tokens, int splits, size_t* bytes) {
  QLX_REQUIRE(bytes != nullptr, "attention workspace: null size pointer");
  QLX_REQUIRE(batch > 0 && n_kv > 0 && group > 0 && tokens > 0 && splits > 0, "attention workspace: sizes must be positive");
  const size_t heads = (size_t)batch * n_kv, rows = (size_t)tokens * group;
  // the split partials: accumulators [heads][S][R][128], maxima and totals [heads][S][R]
  *bytes = splits == 1 ? 0 : heads * splits * rows * (128 + 2) * sizeof(float);
  return QLX_OK;
}

extern "C" int qlx_decode_attention(const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
                                    const float* v_scale, const int* pos, void* out, void* workspace,
                                    size_t workspace_bytes, int batch, int n_kv, int group, int head_dim, int tokens,
                                    int capacity, int splits, float scale, void* stream) {
  QLX_REQUIRE(head_dim == 128, "decode attention: head_dim must be 128 (got %d)", head_dim);
  QLX_REQUIRE(batch > 0 && n_kv > 0 && group > 0 && tokens > 0 && capacity > 0, "decode attention: sizes must be positive");
  QLX_REQUIRE(tokens * group <= 64, "decode attention: tokens x group must be <= 64 (got %d)", tokens * group);
  QLX_REQUIRE(splits >= 1 && splits <= 256, "decode attention: splits must be in 1..256 (got %d)", splits);
  QLX_REQUIRE(q && k_cache && v_cache && pos && out, "decode attention: null pointer");
  QLX_REQUIRE((k_scale == nullptr) == (v_scale == nullptr), "decode attention: give both scales or neither");
  QLX_REQUIRE((size_t)batch * n_kv * capacity * 128 < (1ull << 40), "decode attention: cache too large");
  size_t need = 0;
  qlx_attention_workspace(batch, n_kv, group, tokens, splits, &need);
  QLX_REQUIRE(splits == 1 || (workspace != nullptr && workspace_bytes >= need),
              "decode attention: workspace of %zu bytes needed for %d splits", need, splits);
  AttnArgs a{};
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.k = k_cache;
  a.v = v_cache;
  a.ks = k_scale;
  a.vs = v_scale;
  a.pos = pos;
  a.out = reinterpret_cast<uint16_t*>(out);
  const int heads = batch * n_kv;
  a.R = tokens * group;
  a.heads = heads;
  QLX_REQUIRE(need < (1ull << 31), "decode attention: split workspace beyond 2 GiB (%zu bytes)", need);
  if (splits > 1) a.pacc = reinterpret_cast<float*>(workspace);
  a.scale2 = scale * 1.4426950408889634f;
  a.cap = capacity;
  a.splits = splits;
  a.T = tokens;
  a.G = group;
  a.H = n_kv;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool q8 = k_scale != nullptr;
  const int rt = (a.R + 15) / 16;
  switch (rt) {
    case 1: return q8 ? launch_attn<1, true>(a, heads, st) : launch_attn<1, false>(a, heads, st);
    case 2: return q8 ? launch_attn<2, true>(a, heads, st) : launch_attn<2, false>(a, heads, st);
    case 3: return q8 ? launch_attn<3, true>(a, heads, st) : launch_attn<3, false>(a, heads, st);
    default: return q8 ? launch_attn<4, true>(a, heads, st) : launch_attn<4, false>(a, heads, st);
  }
}
