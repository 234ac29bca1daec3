// HBM stream floor: read `bytes` with 16-byte loads, fold them into one word per workgroup.
//
// The counterpart of the reference's pure-read probe (bench/tiled_probe.py:20-31): the
// best a read-only kernel reaches over the same bytes is the floor the quantized linears
// are measured against, next to the 8 TB/s vendor peak.
#include "common.h"
#include "../../include/qlinear.h"

namespace qlx {

__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    const u32x4 b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3] ^ c[0] ^ c[1] ^ c[2] ^ c[3] ^ d[0] ^ d[1] ^
           d[2] ^ d[3];
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  acc = (uint32_t)__shfl_xor((int)acc, 1, 64) ^ acc;
  if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace qlx

extern "C" int qlx_stream_read(const void* p, long long bytes, void* sink, int blocks, void* stream) {
  QLX_REQUIRE(bytes > 0 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
  QLX_REQUIRE(blocks > 0, "blocks must be positive");
  qlx::stream_read_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const qlx::u32x4*>(p), (size_t)bytes / 16, reinterpret_cast<uint32_t*>(sink));
  QLX_LAUNCH_CHECK("stream_read");
}
