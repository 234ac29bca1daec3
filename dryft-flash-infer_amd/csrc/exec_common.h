// Shared pieces of the decode-step executor (decode_stack.hip): bounded
// waits on the real-time counter, and the published-word ("wire") protocol by which a
// projection's output reaches the workgroups of later projections without a grid barrier.
#pragma once

#include "gemm_launch.h"

namespace qlx {

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
enum WaitSite { kWaitInput = 0, kWaitPartial = 1 };

// True (and the run flagged as failed) once the run's deadline has passed: waits stop there.
__device__ __forceinline__ bool ll_expired(const Waits& w, WaitSite site) {
  if (__builtin_amdgcn_s_memrealtime() <= w.deadline) return false;
  int expect = 0;
  __hip_atomic_compare_exchange_strong(gmem(w.err), &expect, 1 << site, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Published activations ("wire"): one 32-bit word per value, {16-bit run tag, bf16}. Every
// word is single-copy atomic on its own, so a reader can take 16 bytes (4 values) per lane
// with one device-coherent load and check each value's tag: half the load instructions of
// 64-bit {value pair, 32-bit tag} words, and each lane's loads are the wave's bottleneck
// (a wave draws about 1 KB per 110 ns however deep its queue, measured on MI355X).
__device__ __forceinline__ uint32_t wire_tag(uint32_t epoch) { return epoch & 0xffffu; }

// Both values of an output pair as two tagged words, in one 64-bit device-coherent store.
__device__ __forceinline__ void wire_store_pair(uint64_t* p, uint32_t pair, uint32_t epoch) {
  const uint32_t t = wire_tag(epoch) << 16;
  const uint64_t v = ((uint64_t)(t | (pair >> 16)) << 32) | (t | (pair & 0xffffu));
  __hip_atomic_store(gmem(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Buffer resource over `bytes` of device memory, in scalar registers (the pointer is the
// same for every lane: descriptors are read from LDS, which the compiler cannot see).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wire_rsrc(const void* p, unsigned bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a), hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, (int)bytes,
                                           0x00020000);
}
// 16 bytes at `off`, read at device scope (sc1: past this XCD's L2, which other XCDs'
// stores do not update).
__device__ __forceinline__ u32x4 wire_load16(__amdgpu_buffer_rsrc_t rs, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 16);
}

// Activation published by an earlier projection: `pitch` words per token row (the
// activation may be the first k columns of a wider output).
struct XWire {
  static constexpr bool POLLS = true;
  __amdgpu_buffer_rsrc_t rs;
  int pitch;
  uint32_t tag;
  Waits w;
  __device__ XWire(const uint64_t* wire, int pitch_, int m, const Waits& w_)
      : rs(wire_rsrc(wire, (unsigned)m * (unsigned)pitch_ * 4u)), pitch(pitch_), tag(wire_tag(w_.epoch)), w(w_) {}
  struct Raw {
    u32x4 v[2];
  };
  __device__ __forceinline__ static bool half_ready(const u32x4& h, uint32_t tag) {
    return (h[0] >> 16) == tag && (h[1] >> 16) == tag && (h[2] >> 16) == tag && (h[3] >> 16) == tag;
  }
  __device__ __forceinline__ void fetch(const GemmArgs&, int mm, int kabs, Raw& r) const {
    const unsigned off = ((unsigned)mm * pitch + kabs) * 4u;
    r.v[0] = wire_load16(rs, off);
    r.v[1] = wire_load16(rs, off + 16);
  }
  __device__ __forceinline__ bool ready(const Raw& r) const { return half_ready(r.v[0], tag) && half_ready(r.v[1], tag); }
  __device__ __forceinline__ void refetch(const GemmArgs&, int mm, int kabs, Raw& r) const {
    const unsigned off = ((unsigned)mm * pitch + kabs) * 4u;
    if (!half_ready(r.v[0], tag)) r.v[0] = wire_load16(rs, off);
    if (!half_ready(r.v[1], tag)) r.v[1] = wire_load16(rs, off + 16);
  }
  __device__ __forceinline__ bool expired() const { return ll_expired(w, kWaitInput); }
  __device__ __forceinline__ uint4 value(const Raw& r) const {
    return uint4{(r.v[0][0] & 0xffffu) | (r.v[0][1] << 16), (r.v[0][2] & 0xffffu) | (r.v[0][3] << 16),
                 (r.v[1][0] & 0xffffu) | (r.v[1][1] << 16), (r.v[1][2] & 0xffffu) | (r.v[1][3] << 16)};
  }
};

}  // namespace qlx
