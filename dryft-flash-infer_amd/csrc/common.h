// Shared device helpers for the gfx950 quantized-linear library.
//
// Number formats travel as raw bits: bf16 and fp16 as uint16_t, OCP e4m3fn as
// uint8_t. Every conversion here rounds to nearest even, the way torch's casts
// do, so quantize and pack kernels are bit-exact with the CPU statement of the
// reference (engine/kernels/cuda_fp8.py:1127-1151, engine/kernels/fp8.py:20-28).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

namespace qlx {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

// ---- bf16 / fp16 -------------------------------------------------------------------

// Global-memory view of a generic pointer to device memory. Accesses through it compile to
// global_* instead of flat_* instructions; flat accesses also count against the LDS/scalar
// counter, so a wait for an LDS result would wait for every flat load in flight (pointers
// read from memory, unlike kernel arguments, are not known to be global).
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* gmem(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, RNE by integer add (cuda_fp8.py:64-68); NaN -> sign | 0x7FC0. Both
// results are formed and one selected: no divergent branch in the epilogues that call it.
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t nan = ((u >> 16) & 0x8000u) | 0x7fc0u;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? nan : rne);
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Two fp32 values to a bf16 pair (lo in the low half) by the hardware's round-to-nearest-even
// conversion (v_cvt_pk_bf16_f32): the same bits as f2bf for every value but a NaN (checked on
// MI355X over all 2^32 inputs; a NaN keeps its payload's top bits instead of becoming
// sign | 0x7FC0). Callers test bf16_nan_bits on the result and redo a NaN's pair with f2bf.
__device__ __forceinline__ uint32_t bf16_pair_hw(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) __bf16 b2;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}
// Bits 15 / 31 set where the low / high bf16 half of p is a NaN.
__device__ __forceinline__ uint32_t bf16_nan_bits(uint32_t p) { return ((p & 0x7fff7fffu) + 0x007f007fu) & 0x80008000u; }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// fp32 -> fp16 bits, RNE (hardware v_cvt_f16_f32 rounds to nearest even).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// ---- OCP e4m3fn ------------------------------------------------------------------------

// fp32 -> e4m3fn byte, RNE. Below 2^-6 the subnormal code is rint(|f| * 2^9);
// above, 20 mantissa bits are dropped with round-half-even by integer add.
// Anything that rounds past 448 (and Inf/NaN) becomes NaN (0x7F), as torch's cast.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  // Branches, not selects: in a wave almost every value takes the normal path, so only that
  // path runs (computing every case and selecting measured ~15 us slower per FP8 decode step).
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  uint32_t code;
  if (a > 0x7f800000u) {
    code = 0x7fu;
  } else if (a < (121u << 23)) {
    code = (uint32_t)rintf(__uint_as_float(a) * 512.0f);
  } else {
    const uint32_t ar = a + 0x7ffffu + ((a >> 20) & 1u);
    code = (ar >> 20) - (120u << 3);
    if (code > 0x7eu) code = 0x7fu;
  }
  return code | sign;
}

// Clamp to +-lim keeping NaN (torch.clamp propagates NaN; fminf/fmaxf would not).
__device__ __forceinline__ float clamp_keep_nan(float v, float lim) {
  return v < -lim ? -lim : (v > lim ? lim : v);
}

// The FP8 quantizers' code for x / sc, the reference's way: IEEE division, clamp to +-448,
// RNE cast (engine/kernels/fp8.py:20-28).
__device__ __forceinline__ uint32_t e4m3_of_quotient(float x, float sc) {
  return f32_to_e4m3(clamp_keep_nan(x / sc, 448.f));
}

// x / sc as IEEE division rounds it, from y = 1 / sc (IEEE-rounded): the product x * y is
// within an ulp of the quotient, and one correction with its exact residual (fma) lands on the
// correctly rounded quotient (Markstein's theorem for a correctly rounded reciprocal). The sign
// is taken from x so that -0 stays -0 (the residual of -0 is +0).
__device__ __forceinline__ float quotient_by_reciprocal(float x, float sc, float y) {
  const float q0 = x * y;
  const float r = __builtin_fmaf(-q0, sc, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
}

// e4m3 codes of 8 bf16 values (pairs in v) over the scale sc, y = 1 / sc, natural byte order:
// the same codes as e4m3_of_quotient, at about a seventh of its instructions. The quotient comes
// from quotient_by_reciprocal and the cast from the hardware's RNE conversion (v_cvt_pk_fp8_f32,
// OCP e4m3 on gfx950). Both hold for every input the quantizers can see, a bf16 value no larger
// in magnitude than the bf16 maximum its scale was taken from: qlx_fp8_selfcheck compares the two
// paths on all of them. The clamp is not needed there: |x / sc| <= 448 (1 + 2^-23) rounds to 448.
// A chunk holding a NaN, or a non-finite scale, takes e4m3_of_quotient (the hardware gives 0xFF
// for every NaN; torch keeps the sign).
__device__ __forceinline__ uint2 e4m3_chunk(uint4 v, float sc, float y) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  // bit 15 / 31 of (h & 0x7fff) + 0x7f per half: set when that bf16 half is a NaN (> 0x7f80)
  const uint32_t nan = (((d[0] & 0x7fff7fffu) + 0x007f007fu) | ((d[1] & 0x7fff7fffu) + 0x007f007fu) |
                        ((d[2] & 0x7fff7fffu) + 0x007f007fu) | ((d[3] & 0x7fff7fffu) + 0x007f007fu)) &
                       0x80008000u;
  uint32_t o[2];
  if (nan != 0u || !(sc <= 3.40282347e38f)) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t c = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t bits = (e & 1) ? d[2 * h + (e >> 1)] >> 16 : d[2 * h + (e >> 1)] & 0xffffu;
        c |= e4m3_of_quotient(bf2f(bits), sc) << (8 * e);
      }
      o[h] = c;
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float q0 = quotient_by_reciprocal(bf2f(d[2 * h] & 0xffffu), sc, y);
      const float q1 = quotient_by_reciprocal(bf2f(d[2 * h] >> 16), sc, y);
      const float q2 = quotient_by_reciprocal(bf2f(d[2 * h + 1] & 0xffffu), sc, y);
      const float q3 = quotient_by_reciprocal(bf2f(d[2 * h + 1] >> 16), sc, y);
      const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false);
      o[h] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q2, q3, lo, true);
    }
  }
  return uint2{o[0], o[1]};
}

// ---- wave reductions (64 lanes) ----------------------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Lane values moved by one DPP pattern; lanes without a source (or in rows the row mask
// leaves out) read 0. DPP moves cost no LDS round trip, unlike the shuffles above.
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, ROWS, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROWS, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, false));
}

// Sum (fp64) and maximum (fp32, of values >= 0) of the 64 lanes, valid in lane 63: inclusive
// prefix sums within rows of 16 (row_shr 1, 2, 4, 8), then lane 15 of rows 0 and 2 into rows 1
// and 3 (row_bcast:15), then lane 31 into rows 2 and 3 (row_bcast:31). A fixed order: the
// same inputs give the same bits.
__device__ __forceinline__ double wave_sum_last(double v) {
  v += dpp_f64<0x111, 0xf>(v);
  v += dpp_f64<0x112, 0xf>(v);
  v += dpp_f64<0x114, 0xf>(v);
  v += dpp_f64<0x118, 0xf>(v);
  v += dpp_f64<0x142, 0xa>(v);
  v += dpp_f64<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ float wave_max_last(float v) {
  v = fmaxf(v, dpp_f32<0x111, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x112, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x114, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x118, 0xf>(v));
  v = fmaxf(v, dpp_f32<0x142, 0xa>(v));
  v = fmaxf(v, dpp_f32<0x143, 0xc>(v));
  return v;
}

// ---- error reporting --------------------------------------------------------------------

void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);

}  // namespace qlx

#define QLX_OK 0
#define QLX_EINVAL (-1)
#define QLX_EHIP (-2)

#define QLX_REQUIRE(cond, ...)                  \
  do {                                          \
    if (!(cond)) {                              \
      qlx::set_error(__VA_ARGS__);              \
      return QLX_EINVAL;                        \
    }                                           \
  } while (0)

#define QLX_LAUNCH_CHECK(what) return qlx::hip_status(hipGetLastError(), what)
