// Per-head RMSNorm + RoPE arithmetic shared by the head norm + RoPE kernel (rope.hip) and the
// decode-step executor's attention stage (decode_stack.hip), with the reference's roundings
// (engine/kernels/reference.py:31-46, engine/kernels/rope.py:24-60):
//   scale = 1 / sqrt(mean(x^2) + eps)          (fp32; the sum of squares exact in fp64)
//   n     = bf16(bf16(x * scale) * w)
//   y     = bf16(bf16(n * cos) + bf16(rotate_half(n) * sin)),  rotate_half(n) = (-n[64:], n[:64])
// Eight lanes per 128-value head: lane j holds dims 8 j .. 8 j + 7 and their rotate_half partners
// 64 + 8 j .. 64 + 8 j + 7, so the rotation stays in the lane and only the sum of squares
// crosses lanes (shuffles among the 8 lanes of a head).
#pragma once

#include "common.h"

namespace qlx {

typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf2f(d[i] & 0xffffu);
    f[2 * i + 1] = bf2f(d[i] >> 16);
  }
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = (uint32_t)f2bf(f[2 * i]) | ((uint32_t)f2bf(f[2 * i + 1]) << 16);
  return u32x4{d[0], d[1], d[2], d[3]};
}

// The lane's 16 values of a head (xl: dims 8 j + 0..7, xh: 64 + 8 j + 0..7), its norm gains
// (wl, wh), cos and sin (cl/ch, sl/sh) -> the rotated values, as floats (yl, yh) and bf16 pairs
// (ylp, yhp). Every lane of the wave takes part (the head's lanes are 8 consecutive lanes whose
// index differs in bits 0..2). Every rounding is to bf16, by the hardware's pair conversion
// (the integer rounding's bits for every value but a NaN, checked on all 2^32 inputs); a lane
// meeting a NaN redoes its values with the integer rounding.
__device__ __forceinline__ void rope_norm_rotate(const float* xl, const float* xh, const float* wl, const float* wh,
                                                 const float* cl, const float* ch, const float* sl, const float* sh,
                                                 float eps, float* yl, float* yh, uint32_t* ylp, uint32_t* yhp) {
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += (double)xl[i] * (double)xl[i] + (double)xh[i] * (double)xh[i];
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  const float scale = 1.0f / sqrtf((float)(ss / 128.0) + eps);
  uint32_t nan = 0u;
  auto lo = [](uint32_t p) { return bf2f(p & 0xffffu); };
  auto hi = [](uint32_t p) { return bf2f(p >> 16); };
  auto pr = [&nan](float x0, float x1) {
    const uint32_t p = bf16_pair_hw(x0, x1);
    nan |= bf16_nan_bits(p);
    return p;
  };
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const uint32_t ta = pr(xl[i] * scale, xl[i + 1] * scale), tb = pr(xh[i] * scale, xh[i + 1] * scale);
    const uint32_t a = pr(lo(ta) * wl[i], hi(ta) * wl[i + 1]);  // n[8 j + i], n[8 j + i + 1]
    const uint32_t b = pr(lo(tb) * wh[i], hi(tb) * wh[i + 1]);  // n[64 + 8 j + i], ...
    const uint32_t p1 = pr(lo(a) * cl[i], hi(a) * cl[i + 1]), p2 = pr(-lo(b) * sl[i], -hi(b) * sl[i + 1]);
    const uint32_t p3 = pr(lo(b) * ch[i], hi(b) * ch[i + 1]), p4 = pr(lo(a) * sh[i], hi(a) * sh[i + 1]);
    ylp[i >> 1] = pr(lo(p1) + lo(p2), hi(p1) + hi(p2));
    yhp[i >> 1] = pr(lo(p3) + lo(p4), hi(p3) + hi(p4));
  }
  if (nan == 0u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      yl[i] = bf2f((ylp[i >> 1] >> (16 * (i & 1))) & 0xffffu);
      yh[i] = bf2f((yhp[i >> 1] >> (16 * (i & 1))) & 0xffffu);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = round_bf(round_bf(xl[i] * scale) * wl[i]);  // n[8 j + i]
      const float b = round_bf(round_bf(xh[i] * scale) * wh[i]);  // n[64 + 8 j + i]
      yl[i] = round_bf(round_bf(a * cl[i]) + round_bf(-b * sl[i]));
      yh[i] = round_bf(round_bf(b * ch[i]) + round_bf(a * sh[i]));
    }
    const u32x4 l = pack8(yl), h = pack8(yh);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ylp[i] = l[i];
      yhp[i] = h[i];
    }
  }
}

}  // namespace qlx
