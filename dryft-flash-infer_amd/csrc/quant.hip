// Quantize, pack and relayout kernels (load-time work) and the library's error state.
//
// Every kernel here is bit-exact with the CPU statement of the reference:
//   quantize_weight   engine/kernels/cuda_fp8.py:1127-1151 (plus the north-star
//                     generalisations: bf16 scales, signed int8, int4 k32 words)
//   dequantize        engine/kernels/cuda_fp8.py:1154-1161
//   prepare_ref       engine/kernels/cuda_fp8.py:1117-1124, 1164-1205
//   row_major_ref     engine/kernels/cuda_fp8.py:1207-1214
//   quantize_fp8_*    engine/kernels/fp8.py:20-28 (weights; per-token activations)
//   int8_prepare      engine/kernels/cuda_int8.py:100-108
//   quantize_act_int8 engine/kernels/cuda_int8.py:58-77
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/qlinear.h"

namespace qlx {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return QLX_OK;
  set_error("%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
  return QLX_EHIP;
}

// Natural column held at permuted position p of a 64-wide block (cuda_fp8.py:1117-1124):
// p = 16t + 4s + i holds 16s + 2t + (0,1,8,9)[i].
__device__ __forceinline__ int ref_natural(int p) {
  const int t = p >> 4, s = (p >> 2) & 3, i = p & 3;
  return 16 * s + 2 * t + ((i & 1) | ((i >> 1) << 3));
}

// ---- weight quantize (one wave per (row, group)) ------------------------------------------

// storage: 0 = offset bytes (q + offset, uint8, one per byte), 1 = signed int8,
// 2 = int4 codes (q + 8) packed eight per int32 along K (nibble i of word j is k = 8j + i).
__global__ void __launch_bounds__(256)
quantize_weight_kernel(const uint16_t* __restrict__ w, void* __restrict__ data,
                       uint16_t* __restrict__ scale, int rows, int k, int group, int bits,
                       int scale_fp16, int nudge, int storage) {
  const int lane = threadIdx.x & 63;
  const long long gid = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int groups = k / group;
  if (gid >= (long long)rows * groups) return;
  const int row = (int)(gid / groups), g = (int)(gid % groups);
  const uint16_t* src = w + (size_t)row * k + (size_t)g * group;
  const int octets = group >> 3;
  float amax = 0.f;
  for (int o = lane; o < octets; o += 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * o);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(bf2f(d[j] & 0xffffu)));
      amax = fmaxf(amax, fabsf(bf2f(d[j] >> 16)));
    }
  }
  amax = wave_max(amax);
  const float limit = bits == 8 ? 127.f : 7.f;
  const float offset = bits == 8 ? 128.f : 8.f;
  float s = fmaxf(amax / limit, 1e-12f);
  if (nudge) s = s * (1.0f + 0.0009765625f);
  uint16_t sbits;
  float sval;
  if (scale_fp16) {
    sbits = f2h(s);
    sval = h2f(sbits);
  } else {
    sbits = f2bf(s);
    sval = bf2f(sbits);
  }
  if (lane == 0) scale[(size_t)row * groups + g] = sbits;
  for (int o = lane; o < octets; o += 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * o);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    uint32_t codes[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = bf2f(e & 1 ? d[e >> 1] >> 16 : d[e >> 1] & 0xffffu);
      float q = clamp_keep_nan(rintf(x / sval), limit);
      if (storage == 1) {
        codes[e] = q != q ? 0u : (uint32_t)(int32_t)q & 0xffu;
      } else {
        const float b = q + offset;
        codes[e] = b != b ? 0u : (uint32_t)b;
      }
    }
    const size_t kk = (size_t)g * group + 8 * o;
    if (storage == 2) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) word |= (codes[e] & 0xfu) << (4 * e);
      reinterpret_cast<uint32_t*>(data)[((size_t)row * k + kk) >> 3] = word;
    } else {
      uint2 out;
      out.x = codes[0] | (codes[1] << 8) | (codes[2] << 16) | (codes[3] << 24);
      out.y = codes[4] | (codes[5] << 8) | (codes[6] << 16) | (codes[7] << 24);
      *reinterpret_cast<uint2*>(reinterpret_cast<uint8_t*>(data) + (size_t)row * k + kk) = out;
    }
  }
}

// ---- dequantize: bf16((q - offset) * float(scale)) -------------------------------------

__global__ void __launch_bounds__(256)
dequantize_kernel(const void* __restrict__ data, const uint16_t* __restrict__ scale,
                  uint16_t* __restrict__ out, int rows, int k, int groups, int bits,
                  int scale_fp16, int storage) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * k) return;
  const int row = (int)(i / k), col = (int)(i % k);
  const int g = col / (k / groups);
  const uint16_t sb = scale[(size_t)row * groups + g];
  const float s = scale_fp16 ? h2f(sb) : bf2f(sb);
  float q;
  if (storage == 1) {
    q = (float)reinterpret_cast<const int8_t*>(data)[i];
  } else if (storage == 2) {
    const uint32_t word = reinterpret_cast<const uint32_t*>(data)[i >> 3];
    q = (float)((word >> (4 * (i & 7))) & 0xfu) - 8.f;
  } else {
    q = (float)reinterpret_cast<const uint8_t*>(data)[i] - (bits == 8 ? 128.f : 8.f);
  }
  out[i] = f2bf(q * s);
}

// ---- reference layouts (cuda_fp8.Prepared) --------------------------------------------------

// Output byte o of the prepared weight, gathered from the [rows, K] quantize output.
__global__ void __launch_bounds__(256)
prepare_ref_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int rows,
                   int k, int bits, int tiled) {
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int width = bits == 4 ? k / 2 : k;
  if (o >= (size_t)rows * width) return;
  if (!tiled) {  // 8-bit row-major, fragment-permuted columns
    const int r = (int)(o / k), pos = (int)(o % k);
    dst[o] = src[(size_t)r * k + (pos & ~63) + ref_natural(pos & 63)];
    return;
  }
  const int groups = k / 128;
  if (bits == 8) {
    // (tile, group, half, j, g, t, byte) = 16 * 2048-byte tiles per row block
    size_t rest = o;
    const int byte = rest % 16; rest /= 16;
    const int t = rest % 4; rest /= 4;
    const int gg = rest % 8; rest /= 8;
    const int j = rest % 2; rest /= 2;
    const int half = rest % 2; rest /= 2;
    const int grp = rest % groups; rest /= groups;
    const int tile = (int)rest;
    const int row = tile * 16 + half * 8 + gg;
    const int pos = j * 64 + t * 16 + byte;
    dst[o] = src[(size_t)row * k + grp * 128 + (pos & ~63) + ref_natural(pos & 63)];
  } else {
    // (tile, group, half, g, t, byte); block 0 in the low nibble, block 1 in the high one
    size_t rest = o;
    const int byte = rest % 16; rest /= 16;
    const int t = rest % 4; rest /= 4;
    const int gg = rest % 8; rest /= 8;
    const int half = rest % 2; rest /= 2;
    const int grp = rest % groups; rest /= groups;
    const int tile = (int)rest;
    const int row = tile * 16 + half * 8 + gg;
    const size_t base = (size_t)row * k + grp * 128;
    const int nat = ref_natural(t * 16 + byte);
    dst[o] = (uint8_t)((src[base + nat] & 0xf) | ((src[base + 64 + nat] & 0xf) << 4));
  }
}

// Tiled 8-bit prepared weight -> fragment-permuted row-major bytes.
__global__ void __launch_bounds__(256)
row_major_ref_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int rows,
                     int k) {
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= (size_t)rows * k) return;
  const int r = (int)(o / k), pos = (int)(o % k);
  const int tile = r / 16, half = (r / 8) % 2, gg = r % 8;
  const int grp = pos / 128, j = (pos / 64) % 2, t = (pos / 16) % 4, byte = pos % 16;
  const size_t idx = ((((((size_t)tile * (k / 128) + grp) * 2 + half) * 2 + j) * 8 + gg) * 4 + t) * 16 + byte;
  dst[o] = src[idx];
}

// ---- FP8 e4m3 (fp8.py:20-28) ------------------------------------------------------------------

// One wave per (row, group): s = max(amax/448, 1e-12); code = e4m3(clamp(w/s)); scale out bf16(s).
__global__ void __launch_bounds__(256)
quantize_fp8_weight_kernel(const uint16_t* __restrict__ w, uint8_t* __restrict__ code,
                           uint16_t* __restrict__ scale, int rows, int k, int group) {
  const int lane = threadIdx.x & 63;
  const long long gid = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int groups = k / group;
  if (gid >= (long long)rows * groups) return;
  const int row = (int)(gid / groups), g = (int)(gid % groups);
  const uint16_t* src = w + (size_t)row * k + (size_t)g * group;
  uint8_t* dst = code + (size_t)row * k + (size_t)g * group;
  const int octets = group >> 3;
  float amax = 0.f;
  for (int o = lane; o < octets; o += 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * o);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(bf2f(d[j] & 0xffffu)));
      amax = fmaxf(amax, fabsf(bf2f(d[j] >> 16)));
    }
  }
  amax = wave_max(amax);
  const float s = fmaxf(amax / 448.f, 1e-12f), y = 1.f / s;
  if (lane == 0) scale[(size_t)row * groups + g] = f2bf(s);
  for (int o = lane; o < octets; o += 64)
    *reinterpret_cast<uint2*>(dst + 8 * o) = e4m3_chunk(*reinterpret_cast<const uint4*>(src + 8 * o), s, y);
}

// Per-token activation quantize: one block of 256 threads per row.
__global__ void __launch_bounds__(256)
quantize_fp8_act_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ code,
                        float* __restrict__ scale, int k) {
  __shared__ float part[4];
  const int row = blockIdx.x;
  const uint16_t* src = x + (size_t)row * k;
  const int octets = k >> 3;
  float amax = 0.f;
  for (int o = threadIdx.x; o < octets; o += 256) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + 8 * o);
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      amax = fmaxf(amax, fabsf(bf2f(d[j] & 0xffffu)));
      amax = fmaxf(amax, fabsf(bf2f(d[j] >> 16)));
    }
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float s = fmaxf(amax / 448.f, 1e-12f), y = 1.f / s;
  if (threadIdx.x == 0) scale[row] = s;
  for (int o = threadIdx.x; o < octets; o += 256)
    *reinterpret_cast<uint2*>(code + (size_t)row * k + 8 * o) =
        e4m3_chunk(*reinterpret_cast<const uint4*>(src + 8 * o), s, y);
}

// Every input the FP8 quantizers can see, through e4m3_chunk and through e4m3_of_quotient: a
// finite or infinite bf16 maximum `amax` (block y), its scale max(amax / 448, 1e-12), and each
// bf16 x with |x| <= amax, plus every NaN x. counts[0] = codes that differ, counts[2 + i] the
// first 64 of them as (amax bits << 48 | x bits << 32 | fast code << 8 | reference code).
__global__ void __launch_bounds__(256) fp8_selfcheck_kernel(unsigned long long* counts) {
  const uint32_t ab = blockIdx.y;  // 0 .. 0x7f80 (+inf)
  const float amax = bf2f(ab);
  const float s = fmaxf(amax / 448.f, 1e-12f), y = 1.f / s;
  unsigned long long bad = 0;
  // 8 consecutive x bit patterns per thread: one chunk
  for (uint32_t x0 = (blockIdx.x * 256 + threadIdx.x) * 8; x0 < 0x10000u; x0 += gridDim.x * 256 * 8) {
    uint32_t pk[4];
    bool live[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t xb = x0 + e, mag = xb & 0x7fffu;
      live[e] = mag <= ab || mag > 0x7f80u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // values outside the domain are replaced by 0 so that the chunk stays a possible input
      const uint32_t lo = live[2 * i] ? x0 + 2 * i : 0u, hi = live[2 * i + 1] ? x0 + 2 * i + 1 : 0u;
      pk[i] = lo | (hi << 16);
    }
    const uint2 f = e4m3_chunk(uint4{pk[0], pk[1], pk[2], pk[3]}, s, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t bits = e & 1 ? pk[e >> 1] >> 16 : pk[e >> 1] & 0xffffu;
      const uint32_t r = e4m3_of_quotient(bf2f(bits), s);
      const uint32_t fc = ((e < 4 ? f.x : f.y) >> (8 * (e & 3))) & 0xffu;
      if (fc != r) {
        ++bad;
        const unsigned long long i = atomicAdd(&counts[1], 1ull);
        if (i < 64) counts[2 + i] = ((unsigned long long)ab << 48) | ((unsigned long long)bits << 32) | (fc << 8) | r;
      }
    }
  }
  if (bad) atomicAdd(&counts[0], bad);
}

// ---- INT8 W8A8 (cuda_int8.py) ---------------------------------------------------------------

// Natural index held at INT8 fragment position p (cuda_int8.py:64).
__device__ __forceinline__ int i8_natural(int p) {
  return (p >> 4) * 4 + ((p & 15) >> 2) * 16 + (p & 3);
}

// out[r][p] = row_major_ref[r][position holding natural i8_natural(p)] ^ 128.
__global__ void __launch_bounds__(256)
int8_prepare_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ dst, int rows, int k) {
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= (size_t)rows * k) return;
  const int r = (int)(o / k), pos = (int)(o % k);
  const int n = i8_natural(pos & 63);
  const int old = ((n % 8) / 2) * 16 + (n / 16) * 4 + ((n % 16) / 8) * 2 + n % 2;
  dst[o] = (int8_t)(src[(size_t)r * k + (pos & ~63) + old] ^ 128u);
}

// One wave per (row, 64-group): s = max(amax/127, 1e-20); q = rint(x/s) at fragment position.
// With q2 != null the residual x - q*s is quantized the same way (cuda_int8.py:69-74).
__global__ void __launch_bounds__(256)
quantize_act_int8_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                         float* __restrict__ scale, int8_t* __restrict__ q2, float* __restrict__ scale2,
                         int m, int k) {
  const int lane = threadIdx.x & 63;
  const long long gid = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int groups = k / 64;
  if (gid >= (long long)m * groups) return;
  const int row = (int)(gid / groups), g = (int)(gid % groups);
  const float v = bf2f(x[(size_t)row * k + g * 64 + i8_natural(lane)]);
  const float amax = wave_max(fabsf(v));
  const float s = fmaxf(amax / 127.f, 1e-20f);
  const float qv = rintf(v / s);
  q[(size_t)row * k + g * 64 + lane] = (int8_t)(int)qv;
  if (lane == 0) scale[(size_t)row * groups + g] = s;
  if (q2) {
    const float r = v - qv * s;
    const float ramax = wave_max(fabsf(r));
    const float sr = fmaxf(ramax / 127.f, 1e-20f);
    q2[(size_t)row * k + g * 64 + lane] = (int8_t)(int)rintf(r / sr);
    if (lane == 0) scale2[(size_t)row * groups + g] = sr;
  }
}

static inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

}  // namespace qlx

using namespace qlx;

extern "C" {

const char* qlx_last_error(void) { return g_error; }

int qlx_abi_version(void) { return QLX_ABI_VERSION; }

int qlx_quantize_weight(const void* w, void* data, void* scale, int rows, int k, int group,
                        int bits, int scale_kind, int nudge, int storage, void* stream) {
  QLX_REQUIRE(bits == 8 || bits == 4, "weights are 8 or 4 bits, got %d", bits);
  QLX_REQUIRE(rows > 0 && k > 0 && group > 0 && k % group == 0, "%d is not a multiple of %d", k, group);
  QLX_REQUIRE(group % 8 == 0, "group %d must be a multiple of 8", group);
  QLX_REQUIRE(storage >= 0 && storage <= 2, "bad storage %d", storage);
  QLX_REQUIRE(storage != 2 || bits == 4, "int4 k32 packing needs bits=4");
  QLX_REQUIRE(storage != 1 || bits == 8, "signed storage needs bits=8");
  QLX_REQUIRE(scale_kind == QLX_SCALE_F16 || scale_kind == QLX_SCALE_BF16, "bad scale kind");
  const size_t work = (size_t)rows * (k / group);
  quantize_weight_kernel<<<blocks_for(work, 4), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)w, data, (uint16_t*)scale, rows, k, group, bits,
      scale_kind == QLX_SCALE_F16, nudge, storage);
  QLX_LAUNCH_CHECK("quantize_weight");
}

int qlx_dequantize(const void* data, const void* scale, void* out, int rows, int k, int groups,
                   int bits, int scale_kind, int storage, void* stream) {
  QLX_REQUIRE(rows > 0 && k > 0 && groups > 0 && k % groups == 0, "bad dequantize shape");
  QLX_REQUIRE(storage != 2 || k % 8 == 0, "k32 words need K % 8 == 0");
  dequantize_kernel<<<blocks_for((size_t)rows * k, 256), 256, 0, (hipStream_t)stream>>>(
      data, (const uint16_t*)scale, (uint16_t*)out, rows, k, groups, bits,
      scale_kind == QLX_SCALE_F16, storage);
  QLX_LAUNCH_CHECK("dequantize");
}

int qlx_prepare_ref(const void* data, void* out, int rows, int k, int bits, int tiled, void* stream) {
  QLX_REQUIRE(k % 128 == 0, "K=%d is not a multiple of 128", k);
  QLX_REQUIRE(rows % 16 == 0, "rows=%d is not a multiple of 16", rows);
  QLX_REQUIRE(bits == 8 || bits == 4, "weights are 8 or 4 bits");
  QLX_REQUIRE(bits == 8 || tiled, "4-bit weights are stored tiled");
  const size_t n = (size_t)rows * (bits == 4 ? k / 2 : k);
  prepare_ref_kernel<<<blocks_for(n, 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)data, (uint8_t*)out, rows, k, bits, tiled);
  QLX_LAUNCH_CHECK("prepare_ref");
}

int qlx_row_major_ref(const void* weight, void* out, int rows, int k, void* stream) {
  QLX_REQUIRE(k % 128 == 0 && rows % 16 == 0, "bad row_major shape");
  row_major_ref_kernel<<<blocks_for((size_t)rows * k, 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)weight, (uint8_t*)out, rows, k);
  QLX_LAUNCH_CHECK("row_major_ref");
}

int qlx_quantize_fp8_weight(const void* w, void* code, void* scale, int rows, int k, int group,
                            void* stream) {
  QLX_REQUIRE(rows > 0 && k > 0 && group > 0 && k % group == 0, "%d is not a multiple of %d", k, group);
  QLX_REQUIRE(group % 8 == 0, "group %d must be a multiple of 8", group);
  const size_t work = (size_t)rows * (k / group);
  quantize_fp8_weight_kernel<<<blocks_for(work, 4), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)w, (uint8_t*)code, (uint16_t*)scale, rows, k, group);
  QLX_LAUNCH_CHECK("quantize_fp8_weight");
}

int qlx_quantize_fp8_act(const void* x, void* code, float* scale, int m, int k, void* stream) {
  QLX_REQUIRE(m > 0 && k > 0 && k % 8 == 0, "activation K=%d must be a positive multiple of 8", k);
  quantize_fp8_act_kernel<<<m, 256, 0, (hipStream_t)stream>>>((const uint16_t*)x, (uint8_t*)code,
                                                              scale, k);
  QLX_LAUNCH_CHECK("quantize_fp8_act");
}

int qlx_fp8_selfcheck(unsigned long long* counts, void* stream) {
  QLX_REQUIRE(counts != nullptr, "counts is null");
  fp8_selfcheck_kernel<<<dim3(32, 0x7f81), 256, 0, (hipStream_t)stream>>>(counts);
  QLX_LAUNCH_CHECK("fp8_selfcheck");
}

int qlx_int8_prepare(const void* row_major_ref, void* out, int rows, int k, void* stream) {
  QLX_REQUIRE(k % 64 == 0 && rows > 0, "bad int8_prepare shape");
  int8_prepare_kernel<<<blocks_for((size_t)rows * k, 256), 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)row_major_ref, (int8_t*)out, rows, k);
  QLX_LAUNCH_CHECK("int8_prepare");
}

int qlx_quantize_act_int8(const void* x, void* q, float* scale, void* q2, float* scale2, int m, int k,
                          void* stream) {
  QLX_REQUIRE(m > 0 && k > 0 && k % 64 == 0, "activation K=%d must be a multiple of 64", k);
  QLX_REQUIRE(!q2 || scale2, "a second component needs its scales");
  const size_t work = (size_t)m * (k / 64);
  quantize_act_int8_kernel<<<blocks_for(work, 4), 256, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, (int8_t*)q, scale, (int8_t*)q2, scale2, m, k);
  QLX_LAUNCH_CHECK("quantize_act_int8");
}

}  // extern "C"

// ---- MI355X tile layout (load time) ------------------------------------------------------

namespace qlx {

// dst block (tile t, step s) = 2 KB ordered [j][c][r][16 B], taken from row 16t + r, bytes
// 128s + 64j + 16c of the row-major source. One thread per 16-byte chunk.
__global__ void __launch_bounds__(256)
tile_rows_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, int rows, int row_bytes) {
  const size_t o = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t total = (size_t)rows * row_bytes / 16;
  if (o >= total) return;
  const int within = (int)(o & 127);  // 128 chunks per 2 KB block
  const size_t blk = o >> 7;
  const int steps = row_bytes >> 7;
  const int t = (int)(blk / steps), s = (int)(blk % steps);
  const int j = within >> 6, c = (within >> 4) & 3, r = within & 15;
  dst[o] = src[((size_t)(16 * t + r) * row_bytes + 128 * s + 64 * j + 16 * c) / 16];
}

}  // namespace qlx

extern "C" int qlx_tile_rows(const void* src, void* dst, int rows, int row_bytes, void* stream) {
  QLX_REQUIRE(rows > 0 && rows % 16 == 0, "rows=%d must be a positive multiple of 16", rows);
  QLX_REQUIRE(row_bytes > 0 && row_bytes % 128 == 0, "row bytes %d must be a multiple of 128", row_bytes);
  const size_t chunks = (size_t)rows * row_bytes / 16;
  qlx::tile_rows_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (const uint4*)src, (uint4*)dst, rows, row_bytes);
  QLX_LAUNCH_CHECK("tile_rows");
}
