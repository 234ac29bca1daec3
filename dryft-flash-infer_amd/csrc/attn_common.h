// Pieces of grouped-query decode attention shared by the attention kernel (attention.hip) and
// the decode-step executor's attention stage (decode_stack.hip): the key/value block a wave
// holds in registers and the fragment layout of S^T = K Q^T and P V on bf16 MFMA
// (engine/kernels/attention.py:37-178 computes the same quantities).
#pragma once

#include "common.h"

namespace qlx {

// Where a block's keys and values come from: bf16 caches [heads][cap][128], or INT8 codes with
// one fp32 scale per (token, head).
struct KVSrc {
  const void* k;
  const void* v;
  const float* ks;
  const float* vs;
};

constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Dim slot of MFMA k-step s for lane group g. The order inside a product is free as long as
// the query and key fragments agree: bf16 keys take dims 32 s + 8 g (each load instruction
// reads 64 consecutive bytes of 16 keys), INT8 keys 32 g + 8 s (a lane's four steps are 32
// consecutive bytes, two 16-byte loads).
template <bool Q8>
__device__ __forceinline__ int kdim(int s, int g) { return Q8 ? 32 * g + 8 * s : 32 * s + 8 * g; }

// Key of slot j (0..7) of lane group g in a 32-key block: the keys the S^T fragment leaves
// in that lane (key tile j / 4, row 4 g + j % 4).
__device__ __forceinline__ int slot_key(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

__device__ __forceinline__ bf16x8 bf8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

template <bool Q8>
struct KVBlock;

template <>
struct KVBlock<false> {
  u32x4 k[2][4];  // [key tile][k-step]: 8 dims of key 16 kt + n
  u32x4 v[8];     // [slot]: V[key(slot)][8 n .. 8 n + 7]
  __device__ __forceinline__ void load(const KVSrc& a, size_t hb, int kb, int kcap, int n, int g) {
    const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k) + hb;
    const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v) + hb;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = min(kb + 16 * kt + n, kcap - 1);
#pragma unroll
      for (int s = 0; s < 4; ++s) k[kt][s] = *gmem(reinterpret_cast<const u32x4*>(K + (size_t)key * 128 + kdim<false>(s, g)));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = min(kb + slot_key(g, j), kcap - 1);
      v[j] = *gmem(reinterpret_cast<const u32x4*>(V + (size_t)key * 128 + 8 * n));
    }
  }
  __device__ __forceinline__ void zero_from(int kb, int end, int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (kb + slot_key(g, j) >= end) v[j] = u32x4{0u, 0u, 0u, 0u};
  }
  __device__ __forceinline__ u32x4 kfrag(int kt, int s) const { return k[kt][s]; }
  // Column c (0..7) of the lane's 8 keys x 8 dims block: 8 keys of dim 8 n + c, slot order.
  __device__ __forceinline__ u32x4 vfrag(int c) const {
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = reinterpret_cast<const uint32_t*>(&v[2 * q])[c >> 1];
      const uint32_t hi = reinterpret_cast<const uint32_t*>(&v[2 * q + 1])[c >> 1];
      d[q] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
    return u32x4{d[0], d[1], d[2], d[3]};
  }
};

// INT8 cache: codes with one fp32 scale per (token, head); each value is dequantised to
// bf16(code * scale) as it is loaded (attention.py:94-99).
template <>
struct KVBlock<true> {
  u32x4 k[2][2];  // [key tile][half]: dims 32 g .. 32 g + 31 of key 16 kt + n
  u32x2 v[8];     // [slot]: codes of V[key(slot)][8 n .. 8 n + 7]
  float ksc[2], vsc[8];
  __device__ __forceinline__ void load(const KVSrc& a, size_t hb, int kb, int kcap, int n, int g) {
    const int8_t* K = reinterpret_cast<const int8_t*>(a.k) + hb;
    const int8_t* V = reinterpret_cast<const int8_t*>(a.v) + hb;
    const size_t sb = hb >> 7;  // scale index of key 0 of this head
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = min(kb + 16 * kt + n, kcap - 1);
      k[kt][0] = *gmem(reinterpret_cast<const u32x4*>(K + (size_t)key * 128 + 32 * g));
      k[kt][1] = *gmem(reinterpret_cast<const u32x4*>(K + (size_t)key * 128 + 32 * g + 16));
      ksc[kt] = gmem(a.ks)[sb + key];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = min(kb + slot_key(g, j), kcap - 1);
      v[j] = *gmem(reinterpret_cast<const u32x2*>(V + (size_t)key * 128 + 8 * n));
      vsc[j] = gmem(a.vs)[sb + key];
    }
  }
  __device__ __forceinline__ void zero_from(int kb, int end, int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (kb + slot_key(g, j) >= end) {
        v[j] = u32x2{0u, 0u};
        vsc[j] = 0.f;
      }
  }
  static __device__ __forceinline__ float deq(uint32_t w, int b, float sc) {
    return round_bf((float)(int)(int8_t)(w >> (8 * b)) * sc);
  }
  __device__ __forceinline__ u32x4 kfrag(int kt, int s) const {
    const uint32_t* c = reinterpret_cast<const uint32_t*>(&k[kt][s >> 1]) + 2 * (s & 1);
    const float sc = ksc[kt];
    return u32x4{pack_bf(deq(c[0], 0, sc), deq(c[0], 1, sc)), pack_bf(deq(c[0], 2, sc), deq(c[0], 3, sc)),
                 pack_bf(deq(c[1], 0, sc), deq(c[1], 1, sc)), pack_bf(deq(c[1], 2, sc), deq(c[1], 3, sc))};
  }
  __device__ __forceinline__ u32x4 vfrag(int c) const {
    uint32_t d[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w0 = reinterpret_cast<const uint32_t*>(&v[2 * q])[c >> 2];
      const uint32_t w1 = reinterpret_cast<const uint32_t*>(&v[2 * q + 1])[c >> 2];
      d[q] = pack_bf(deq(w0, c & 3, vsc[2 * q]), deq(w1, c & 3, vsc[2 * q + 1]));
    }
    return u32x4{d[0], d[1], d[2], d[3]};
  }
};

}  // namespace qlx
