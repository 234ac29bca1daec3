// Per-head RMSNorm + RoPE of the fused QKV projection, K and V written into the cache
// (engine/kernels/rope.py:24-60 `_norm_rope`, :63-92 q/kv kernels, :125-166 the fused Q/K/V
// kernel, :169-218 the split-K planes variant, :96-122 the INT8 cache writes).
//
// Eight lanes per 128-value head (rope_common.h: the lane layout and the roundings, those of
// engine/kernels/reference.py:31-46). A workgroup of 256 threads covers 32 heads of one row:
// Q heads, then K heads (whose lanes also move the V head).
// From planes, x = bf16(sum of the fp32 planes in slice order) (rope.py:169-176).
// INT8 cache: per (token, head) scale max(amax |y|, 1e-12) / 127, codes
// clamp(floor(y / scale + 0.5), -127, 127) (rope.py:108-118).
#include "rope_common.h"
#include "../../include/qlinear.h"

namespace qlx {

struct RopeArgs {
  qlx_rope_args p;
  int heads;  // n_q + n_kv
};

// 8 values of row `row` at column `col`: bf16 from qkv, or bf16(sum of the planes).
__device__ __forceinline__ void load8(const qlx_rope_args& p, int row, long long col, float* f) {
  if (p.planes == nullptr) {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(p.qkv) + (size_t)row * p.stride + col;
    unpack8(*gmem(reinterpret_cast<const u32x4*>(x)), f);
    return;
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.splits; ++s) {
    const float* pp = p.planes + ((size_t)s * p.rows + row) * p.stride + col;
    const f32x4 lo = *gmem(reinterpret_cast<const f32x4*>(pp));
    const f32x4 hi = *gmem(reinterpret_cast<const f32x4*>(pp + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[i] += lo[i];
      acc[4 + i] += hi[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = round_bf(acc[i]);
}

__device__ __forceinline__ void store_int8(int8_t* dst, const float* f, float sc) {
  uint32_t d[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float c = fminf(fmaxf(floorf(f[i] / sc + 0.5f), -127.f), 127.f);
    d[i >> 2] |= ((uint32_t)(int)c & 0xffu) << (8 * (i & 3));
  }
  *gmem(reinterpret_cast<u32x2*>(dst)) = u32x2{d[0], d[1]};
}

// Max over the 8 lanes of a head (lanes 8 h .. 8 h + 7 of the wave).
__device__ __forceinline__ float head_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 1, 64));
  v = fmaxf(v, __shfl_xor(v, 2, 64));
  return fmaxf(v, __shfl_xor(v, 4, 64));
}

__global__ void __launch_bounds__(256) rope_kernel(RopeArgs ra) {
  const qlx_rope_args& p = ra.p;
  const int row = blockIdx.x;
  const int hh = blockIdx.y * 32 + (threadIdx.x >> 3);
  const int j = threadIdx.x & 7;
  // Lanes past the last head compute on head 0's data and store nothing (a head's 8 lanes
  // take the same branch, and no lane leaves before the shuffles).
  const bool active = hh < ra.heads;
  const int h = active ? hh : 0;
  const bool is_q = h < p.n_q;
  const int kvh = h - p.n_q;
  const long long col = is_q ? p.q_col + (long long)h * 128 : p.k_col + (long long)kvh * 128;

  // The position first: the cos/sin rows it selects are the second of two dependent loads.
  const int tok = row % p.seq_len;
  const long long pos = p.pos_int64 ? reinterpret_cast<const long long*>(p.positions)[tok]
                                    : (long long)reinterpret_cast<const int*>(p.positions)[tok];
  const bool in_table = pos >= 0 && pos < p.table_rows;
  const long long tp = in_table ? pos : 0;
  float cl[8], ch[8], sl[8], sh[8];
  const uint16_t* cs = reinterpret_cast<const uint16_t*>(p.cos) + (size_t)tp * 128;
  const uint16_t* sn = reinterpret_cast<const uint16_t*>(p.sin) + (size_t)tp * 128;
  unpack8(*gmem(reinterpret_cast<const u32x4*>(cs + 8 * j)), cl);
  unpack8(*gmem(reinterpret_cast<const u32x4*>(cs + 64 + 8 * j)), ch);
  unpack8(*gmem(reinterpret_cast<const u32x4*>(sn + 8 * j)), sl);
  unpack8(*gmem(reinterpret_cast<const u32x4*>(sn + 64 + 8 * j)), sh);

  float xl[8], xh[8];
  load8(p, row, col + 8 * j, xl);
  load8(p, row, col + 64 + 8 * j, xh);
  const uint16_t* gain = reinterpret_cast<const uint16_t*>(is_q ? p.q_norm_w : p.k_norm_w);
  float wl[8], wh[8];
  unpack8(*gmem(reinterpret_cast<const u32x4*>(gain + 8 * j)), wl);
  unpack8(*gmem(reinterpret_cast<const u32x4*>(gain + 64 + 8 * j)), wh);
  float yl[8], yh[8];
  uint32_t ylp[4], yhp[4];
  rope_norm_rotate(xl, xh, wl, wh, cl, ch, sl, sh, p.eps, yl, yh, ylp, yhp);

  if (is_q) {
    if (!active) return;
    uint16_t* q = reinterpret_cast<uint16_t*>(p.q_out) + (size_t)row * p.n_q * 128 + (size_t)h * 128;
    if (!in_table) {  // a position outside the cos/sin table: the head reads as NaN
#pragma unroll
      for (int i = 0; i < 8; ++i) yl[i] = yh[i] = __builtin_nanf("");
    }
    if (!in_table) {
      *gmem(reinterpret_cast<u32x4*>(q + 8 * j)) = pack8(yl);
      *gmem(reinterpret_cast<u32x4*>(q + 64 + 8 * j)) = pack8(yh);
    } else {
      *gmem(reinterpret_cast<u32x4*>(q + 8 * j)) = u32x4{ylp[0], ylp[1], ylp[2], ylp[3]};
      *gmem(reinterpret_cast<u32x4*>(q + 64 + 8 * j)) = u32x4{yhp[0], yhp[1], yhp[2], yhp[3]};
    }
    return;
  }

  // K head kvh: rotated K and the raw V head to slot pos of sequence row / seq_len.
  float vl[8], vh[8];
  const long long vcol = p.v_col + (long long)kvh * 128;
  load8(p, row, vcol + 8 * j, vl);
  load8(p, row, vcol + 64 + 8 * j, vh);
  const bool writes = active && in_table && pos < p.capacity;
  const int seq = row / p.seq_len;
  const size_t hs = (size_t)seq * p.n_kv + kvh;
  const size_t slot = (hs * p.capacity + (size_t)(writes ? pos : 0)) * 128;
  if (p.k_copy != nullptr && active) {
    const size_t cslot = (hs * p.seq_len + tok) * 128;
    uint16_t* kc = reinterpret_cast<uint16_t*>(p.k_copy) + cslot;
    uint16_t* vc = reinterpret_cast<uint16_t*>(p.v_copy) + cslot;
    *gmem(reinterpret_cast<u32x4*>(kc + 8 * j)) = u32x4{ylp[0], ylp[1], ylp[2], ylp[3]};
    *gmem(reinterpret_cast<u32x4*>(kc + 64 + 8 * j)) = u32x4{yhp[0], yhp[1], yhp[2], yhp[3]};
    *gmem(reinterpret_cast<u32x4*>(vc + 8 * j)) = pack8(vl);
    *gmem(reinterpret_cast<u32x4*>(vc + 64 + 8 * j)) = pack8(vh);
  }
  if (p.k_scale != nullptr) {
    float ka = 0.f, va = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ka = fmaxf(ka, fmaxf(fabsf(yl[i]), fabsf(yh[i])));
      va = fmaxf(va, fmaxf(fabsf(vl[i]), fabsf(vh[i])));
    }
    const float ks = fmaxf(head_max(ka), 1e-12f) / 127.0f;
    const float vs = fmaxf(head_max(va), 1e-12f) / 127.0f;
    if (!writes) return;
    int8_t* kc = reinterpret_cast<int8_t*>(p.k_cache) + slot;
    int8_t* vc = reinterpret_cast<int8_t*>(p.v_cache) + slot;
    store_int8(kc + 8 * j, yl, ks);
    store_int8(kc + 64 + 8 * j, yh, ks);
    store_int8(vc + 8 * j, vl, vs);
    store_int8(vc + 64 + 8 * j, vh, vs);
    if (j == 0) {
      p.k_scale[slot >> 7] = ks;
      p.v_scale[slot >> 7] = vs;
    }
    return;
  }
  if (!writes) return;
  uint16_t* kc = reinterpret_cast<uint16_t*>(p.k_cache) + slot;
  uint16_t* vc = reinterpret_cast<uint16_t*>(p.v_cache) + slot;
  *gmem(reinterpret_cast<u32x4*>(kc + 8 * j)) = u32x4{ylp[0], ylp[1], ylp[2], ylp[3]};
  *gmem(reinterpret_cast<u32x4*>(kc + 64 + 8 * j)) = u32x4{yhp[0], yhp[1], yhp[2], yhp[3]};
  *gmem(reinterpret_cast<u32x4*>(vc + 8 * j)) = pack8(vl);
  *gmem(reinterpret_cast<u32x4*>(vc + 64 + 8 * j)) = pack8(vh);
}

}  // namespace qlx

using namespace qlx;

extern "C" int qlx_qkv_norm_rope(const qlx_rope_args* args, void* stream) {
  QLX_REQUIRE(args != nullptr, "norm_rope: null arguments");
  const qlx_rope_args& p = *args;
  QLX_REQUIRE(p.rows >= 0 && p.n_q >= 0 && p.n_kv >= 0 && p.n_q + p.n_kv > 0, "norm_rope: bad row or head counts");
  QLX_REQUIRE(p.seq_len >= 1 && p.rows % p.seq_len == 0, "norm_rope: rows (%d) must be a multiple of seq_len (%d)",
              p.rows, p.seq_len);
  QLX_REQUIRE((p.qkv == nullptr) != (p.planes == nullptr), "norm_rope: give qkv or planes, not both");
  QLX_REQUIRE(p.planes == nullptr || p.splits >= 1, "norm_rope: planes need splits >= 1");
  QLX_REQUIRE(p.stride > 0 && p.stride % 8 == 0, "norm_rope: row stride must be a positive multiple of 8");
  QLX_REQUIRE(p.table_rows >= 1 && p.cos && p.sin && p.positions, "norm_rope: cos/sin tables and positions needed");
  QLX_REQUIRE(p.n_q == 0 || (p.q_out && p.q_norm_w && p.q_col >= 0 && p.q_col % 8 == 0 &&
                             p.q_col + (long long)p.n_q * 128 <= p.stride),
              "norm_rope: Q heads need q_out, q_norm_w and columns inside the row");
  QLX_REQUIRE(p.n_kv == 0 || (p.k_cache && p.v_cache && p.k_norm_w && p.capacity >= 1 && p.k_col >= 0 &&
                              p.v_col >= 0 && p.k_col % 8 == 0 && p.v_col % 8 == 0 &&
                              p.k_col + (long long)p.n_kv * 128 <= p.stride &&
                              p.v_col + (long long)p.n_kv * 128 <= p.stride),
              "norm_rope: K/V heads need caches, k_norm_w, capacity and columns inside the row");
  QLX_REQUIRE((p.k_scale == nullptr) == (p.v_scale == nullptr), "norm_rope: give both cache scales or neither");
  QLX_REQUIRE((p.k_copy == nullptr) == (p.v_copy == nullptr), "norm_rope: give both bf16 copies or neither");
  if (p.rows == 0) return QLX_OK;
  RopeArgs ra{p, p.n_q + p.n_kv};
  const dim3 grid(p.rows, (ra.heads + 31) / 32);
  rope_kernel<<<grid, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(ra);
  QLX_LAUNCH_CHECK("norm_rope");
}
