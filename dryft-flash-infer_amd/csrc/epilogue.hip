// Split-K plane consumers and the small epilogues between projections.
//
// The bf16 roundings land where the reference puts them:
//   reduce_planes     bf16(sum_s P[s]) in slice order      engine/kernels/cuda_fp8.py:965-981
//   residual_planes   bf16(x + bf16(sum_s P[s]))           engine/kernels/cuda_small.py:43-55
//   rms_norm          bf16(bf16(x * rsqrt(mean x^2 + eps)) * w)  engine/kernels/reference.py:13-16
//   add_rms_norm      residual then rms_norm               engine/kernels/reference.py:19-28
//   swiglu            bf16(bf16(silu(bf16 g)) * bf16 u)    engine/kernels/swiglu.py:37-53
//   add_norm_quant    residual, rms_norm, INT8 quantize    engine/kernels/cuda_int8.py:17-44
//   add_norm_fp8      residual, rms_norm, per-token e4m3 quantize (the FP8 W8A8 activation
//                     of qlx_quantize_fp8_act, from the normed row held on chip)
#include "common.h"
#include "../../include/qlinear.h"

namespace qlx {

__global__ void __launch_bounds__(256)
reduce_planes_kernel(const float* __restrict__ p, uint16_t* __restrict__ out, size_t width, int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= width) return;
  float acc = 0.f;
  for (int s = 0; s < splits; ++s) acc += p[(size_t)s * width + i];
  out[i] = f2bf(acc);
}

__global__ void __launch_bounds__(256)
residual_planes_kernel(const uint16_t* __restrict__ x, const float* __restrict__ p,
                       uint16_t* __restrict__ out, size_t width, int splits) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= width) return;
  float acc = 0.f;
  for (int s = 0; s < splits; ++s) acc += p[(size_t)s * width + i];
  out[i] = f2bf(bf2f(x[i]) + round_bf(acc));
}

// Chunks of 8 values a thread of add_rms_norm_kernel loads at once (n <= 256 * 8 * 8 = 16384).
constexpr int kNormChunks = 8;

__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
  return uint4{v[0], v[1], v[2], v[3]};
}

// delta: bf16 [rows][n] or (planes != null) fp32 planes [splits][rows][n]; res may be null
// (plain rms_norm of x). One workgroup of 256 threads per row. When n % 8 == 0 every thread
// issues all of its 16-byte loads (x, delta or each plane, w) before it uses any, so a row
// costs one memory round trip per input rather than one per value a thread holds.
__global__ void __launch_bounds__(256)
add_rms_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ delta,
                    const float* __restrict__ planes, int splits, const uint16_t* __restrict__ w,
                    uint16_t* __restrict__ res, uint16_t* __restrict__ y, int8_t* __restrict__ q,
                    float* __restrict__ qs, uint8_t* __restrict__ q8, float* __restrict__ q8s, int rows, int n,
                    float eps) {
  extern __shared__ float rbuf[];  // the row's residual, fp32
  __shared__ double part[4];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * n;
  const bool add = delta != nullptr || planes != nullptr;
  // Sum of squares in fp64: each square of a bf16 value is exact there and so is the sum of
  // a hidden row's worth, which makes the scale independent of the summation order.
  double ss = 0.0;
  const bool vec = (n & 7) == 0;
  if (vec) {
    const int nc = n >> 3;
    uint4 xv[kNormChunks], dv[kNormChunks];
#pragma unroll
    for (int u = 0; u < kNormChunks; ++u) {
      const int c = threadIdx.x + u * 256;
      if (c < nc) {
        xv[u] = ld16(x + base + 8 * c);
        if (delta) dv[u] = ld16(delta + base + 8 * c);
      }
    }
    float d[kNormChunks][8];
    if (planes) {  // slice-order fp32 sums, each slice's loads of every chunk issued together
#pragma unroll
      for (int u = 0; u < kNormChunks; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) d[u][i] = 0.f;
      for (int sl = 0; sl < splits; ++sl) {
        const float* pl = planes + (size_t)sl * rows * n + base;
        u32x4 pv[kNormChunks][2];
#pragma unroll
        for (int u = 0; u < kNormChunks; ++u) {
          const int c = threadIdx.x + u * 256;
          if (c < nc) {
            pv[u][0] = *reinterpret_cast<const u32x4*>(pl + 8 * c);
            pv[u][1] = *reinterpret_cast<const u32x4*>(pl + 8 * c + 4);
          }
        }
#pragma unroll
        for (int u = 0; u < kNormChunks; ++u) {
          const int c = threadIdx.x + u * 256;
          if (c < nc)
#pragma unroll
            for (int i = 0; i < 8; ++i) d[u][i] += __uint_as_float(pv[u][i >> 2][i & 3]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kNormChunks; ++u) {
      const int c = threadIdx.x + u * 256;
      if (c >= nc) continue;
      const uint32_t xs[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
      float r[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = bf2f((xs[i >> 1] >> (16 * (i & 1))) & 0xffffu);
      if (add) {
        const uint32_t ds[4] = {dv[u].x, dv[u].y, dv[u].z, dv[u].w};
        // bf16 rounding by the hardware's pair conversion (the integer rounding's bits for every
        // value but a NaN); a chunk meeting a NaN is redone the integer way.
        uint32_t rp[4], nan = 0u;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          float dd0, dd1;
          if (planes) {
            const uint32_t dp = bf16_pair_hw(d[u][i], d[u][i + 1]);
            nan |= bf16_nan_bits(dp);
            dd0 = bf2f(dp & 0xffffu);
            dd1 = bf2f(dp >> 16);
          } else {
            dd0 = bf2f(ds[i >> 1] & 0xffffu);
            dd1 = bf2f(ds[i >> 1] >> 16);
          }
          rp[i >> 1] = bf16_pair_hw(r[i] + dd0, r[i + 1] + dd1);
          nan |= bf16_nan_bits(rp[i >> 1]);
        }
        if (nan == 0u) {
#pragma unroll
          for (int i = 0; i < 8; ++i) r[i] = bf2f((rp[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float dd = planes ? round_bf(d[u][i]) : bf2f((ds[i >> 1] >> (16 * (i & 1))) & 0xffffu);
            r[i] = round_bf(r[i] + dd);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) rp[i] = pack_bf2(r[2 * i], r[2 * i + 1]);
        }
        if (res) *reinterpret_cast<u32x4*>(res + base + 8 * c) = u32x4{rp[0], rp[1], rp[2], rp[3]};
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        rbuf[8 * c + i] = r[i];
        ss += (double)r[i] * (double)r[i];
      }
    }
  } else {
    for (int c = threadIdx.x; c < n; c += 256) {
      float r = bf2f(x[base + c]);
      if (add) {
        float d;
        if (planes) {
          d = 0.f;
          for (int sl = 0; sl < splits; ++sl) d += planes[(size_t)sl * rows * n + base + c];
          d = round_bf(d);
        } else {
          d = bf2f(delta[base + c]);
        }
        r = round_bf(r + d);
        if (res) res[base + c] = f2bf(r);
      }
      rbuf[c] = r;
      ss += (double)r * (double)r;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const double total = ((part[0] + part[1]) + part[2]) + part[3];
  // mean rounded to fp32, + eps and 1/sqrt in fp32, as torch's rsqrt(mean + eps)
  const float scale = 1.0f / sqrtf((float)(total / (double)n) + eps);
  if (vec) {
    const int nc = n >> 3;
    uint4 wv[kNormChunks];
#pragma unroll
    for (int u = 0; u < kNormChunks; ++u) {
      const int c = threadIdx.x + u * 256;
      if (c < nc) wv[u] = ld16(w + 8 * c);
    }
#pragma unroll
    for (int u = 0; u < kNormChunks; ++u) {
      const int c = threadIdx.x + u * 256;
      if (c >= nc) continue;
      const uint32_t ws[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
      float v[8];
      uint32_t vp[4], nan = 0u;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {  // as above: the pair conversion, the integer way on a NaN
        const uint32_t t = bf16_pair_hw(rbuf[8 * c + i] * scale, rbuf[8 * c + i + 1] * scale);
        vp[i >> 1] = bf16_pair_hw(bf2f(t & 0xffffu) * bf2f(ws[i >> 1] & 0xffffu),
                                  bf2f(t >> 16) * bf2f(ws[i >> 1] >> 16));
        nan |= bf16_nan_bits(t) | bf16_nan_bits(vp[i >> 1]);
      }
      if (nan == 0u) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = bf2f((vp[i >> 1] >> (16 * (i & 1))) & 0xffffu);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          v[i] = round_bf(round_bf(rbuf[8 * c + i] * scale) * bf2f((ws[i >> 1] >> (16 * (i & 1))) & 0xffffu));
#pragma unroll
        for (int i = 0; i < 4; ++i) vp[i] = pack_bf2(v[2 * i], v[2 * i + 1]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) rbuf[8 * c + i] = v[i];
      if (y) *reinterpret_cast<u32x4*>(y + base + 8 * c) = u32x4{vp[0], vp[1], vp[2], vp[3]};
    }
  } else {
    for (int c = threadIdx.x; c < n; c += 256) {
      const float v = round_bf(round_bf(rbuf[c] * scale) * bf2f(w[c]));
      rbuf[c] = v;
      if (y) y[base + c] = f2bf(v);
    }
  }
  if (q8) {
    // FP8 per-token activation quantize of the normed row (every value is a bf16 value, so its
    // top 16 bits are its bf16 bits, a NaN's the integer rounding's sign | 0x7FC0 form):
    // scale = max(amax / 448, 1e-12), codes e4m3(x / scale).
    __shared__ float pmax[4];
    __syncthreads();
    float mx = 0.f;
    for (int c = threadIdx.x; c < n; c += 256) mx = fmaxf(mx, fabsf(rbuf[c]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) pmax[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float sc = fmaxf(fmaxf(fmaxf(pmax[0], pmax[1]), fmaxf(pmax[2], pmax[3])) / 448.f, 1e-12f);
    const float yr = 1.f / sc;
    if (threadIdx.x == 0) q8s[row] = sc;
    for (int c8 = threadIdx.x; c8 < (n >> 3); c8 += 256) {
      uint32_t pk[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pk[i] = (__float_as_uint(rbuf[8 * c8 + 2 * i]) >> 16) | (__float_as_uint(rbuf[8 * c8 + 2 * i + 1]) & 0xffff0000u);
      *reinterpret_cast<uint2*>(q8 + base + 8 * c8) = e4m3_chunk(uint4{pk[0], pk[1], pk[2], pk[3]}, sc, yr);
    }
    return;
  }
  if (!q) return;
  // INT8 activation quantize per 64-group, fragment order (cuda_int8.py:30-44).
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int groups = n / 64;
  for (int g = threadIdx.x >> 6; g < groups; g += 4) {
    const int nat = (lane >> 4) * 4 + ((lane & 15) >> 2) * 16 + (lane & 3);
    const float v = rbuf[g * 64 + nat];
    const float amax = wave_max(fabsf(v));
    const float s = fmaxf(amax / 127.f, 1e-20f);
    q[base + g * 64 + lane] = (int8_t)(int)rintf(v / s);
    if (lane == 0) qs[(size_t)row * groups + g] = s;
  }
}

// gate_up: bf16 [rows][2I] or (planes != null) fp32 planes [splits][rows][2I].
__global__ void __launch_bounds__(256)
swiglu_kernel(const uint16_t* __restrict__ gu, const float* __restrict__ planes, int splits,
              uint16_t* __restrict__ out, int rows, int inter) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int row = blockIdx.y;
  if (c >= inter) return;
  const size_t base = (size_t)row * 2 * inter + c;
  float g, u;
  if (planes) {
    g = 0.f;
    u = 0.f;
    const size_t plane = (size_t)rows * 2 * inter;
    for (int s = 0; s < splits; ++s) {
      g += planes[s * plane + base];
      u += planes[s * plane + base + inter];
    }
    g = round_bf(g);
    u = round_bf(u);
  } else {
    g = bf2f(gu[base]);
    u = bf2f(gu[base + inter]);
  }
  const float silu = round_bf(g / (1.f + expf(-g)));
  out[(size_t)row * inter + c] = f2bf(silu * u);
}

static inline unsigned blocks_for(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace qlx

using namespace qlx;

extern "C" {

int qlx_reduce_planes(const float* planes, void* out, long long width, int splits, void* stream) {
  QLX_REQUIRE(width > 0 && splits >= 1, "bad reduce shape");
  reduce_planes_kernel<<<blocks_for(width), 256, 0, (hipStream_t)stream>>>(planes, (uint16_t*)out,
                                                                          (size_t)width, splits);
  QLX_LAUNCH_CHECK("reduce_planes");
}

int qlx_residual_planes(const void* x, const float* planes, void* out, long long width, int splits,
                        void* stream) {
  QLX_REQUIRE(width > 0 && splits >= 1, "bad residual shape");
  residual_planes_kernel<<<blocks_for(width), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, planes, (uint16_t*)out, (size_t)width, splits);
  QLX_LAUNCH_CHECK("residual_planes");
}

int qlx_add_rms_norm(const void* x, const void* delta, const float* planes, int splits, const void* w,
                     void* res, void* y, int rows, int n, float eps, void* stream) {
  QLX_REQUIRE(rows > 0 && n > 0 && n <= 16384, "rows=%d n=%d: rows must be > 0 and n in 1..16384", rows, n);
  QLX_REQUIRE(planes == nullptr || splits >= 1, "planes need splits >= 1");
  add_rms_norm_kernel<<<rows, 256, n * sizeof(float), (hipStream_t)stream>>>(
      (const uint16_t*)x, (const uint16_t*)delta, planes, splits, (const uint16_t*)w, (uint16_t*)res,
      (uint16_t*)y, nullptr, nullptr, nullptr, nullptr, rows, n, eps);
  QLX_LAUNCH_CHECK("add_rms_norm");
}

int qlx_add_norm_quant_int8(const void* x, const void* delta, const float* planes, int splits,
                            const void* w, void* res, void* q, float* q_scale, int rows, int n, float eps,
                            void* stream) {
  QLX_REQUIRE(rows > 0 && n > 0 && n <= 16384 && n % 64 == 0, "n=%d must be a multiple of 64 up to 16384", n);
  QLX_REQUIRE(planes == nullptr || splits >= 1, "planes need splits >= 1");
  add_rms_norm_kernel<<<rows, 256, n * sizeof(float), (hipStream_t)stream>>>(
      (const uint16_t*)x, (const uint16_t*)delta, planes, splits, (const uint16_t*)w, (uint16_t*)res,
      nullptr, (int8_t*)q, q_scale, nullptr, nullptr, rows, n, eps);
  QLX_LAUNCH_CHECK("add_norm_quant_int8");
}

int qlx_add_norm_quant_fp8(const void* x, const void* delta, const float* planes, int splits, const void* w,
                           void* res, void* y, void* code, float* scale, int rows, int n, float eps, void* stream) {
  QLX_REQUIRE(rows > 0 && n > 0 && n <= 16384 && n % 8 == 0, "n=%d must be a multiple of 8 up to 16384", n);
  QLX_REQUIRE(planes == nullptr || splits >= 1, "planes need splits >= 1");
  QLX_REQUIRE(code != nullptr && scale != nullptr, "codes and scales are required");
  add_rms_norm_kernel<<<rows, 256, n * sizeof(float), (hipStream_t)stream>>>(
      (const uint16_t*)x, (const uint16_t*)delta, planes, splits, (const uint16_t*)w, (uint16_t*)res,
      (uint16_t*)y, nullptr, nullptr, (uint8_t*)code, scale, rows, n, eps);
  QLX_LAUNCH_CHECK("add_norm_quant_fp8");
}

int qlx_swiglu(const void* gate_up, const float* planes, int splits, void* out, int rows, int inter,
               void* stream) {
  QLX_REQUIRE(rows > 0 && inter > 0, "bad swiglu shape");
  QLX_REQUIRE(gate_up != nullptr || (planes != nullptr && splits >= 1), "swiglu needs gate_up or planes");
  dim3 grid((inter + 255) / 256, rows);
  swiglu_kernel<<<grid, 256, 0, (hipStream_t)stream>>>((const uint16_t*)gate_up, planes, splits,
                                                      (uint16_t*)out, rows, inter);
  QLX_LAUNCH_CHECK("swiglu");
}

}  // extern "C"
