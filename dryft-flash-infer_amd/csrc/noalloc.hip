// The skinny GEMM (qlx_linear_skinny) for callers that cannot allocate: its split-K planes and
// ticket counters live in this file's static device array instead of caller-passed memory.
//
// Each GPU the library runs on holds its own copy of `scratch` (kNoallocPlaneBytes of fp32
// planes + kNoallocTickets counters) until the process ends. Host code never passes the
// array's name to a kernel (in host code it is a stand-in, not a device address): the address
// on each device comes from hipGetSymbolAddress, taken once per device on the first call with
// that device current, and only that pointer is used. Every call on one GPU shares the array,
// so calls that overlap on one GPU (concurrent streams, or threads) race.
#include <mutex>

#include "gemm_launch.h"

namespace qlx {
namespace {

constexpr long long kNoallocPlaneBytes = 8ll << 20;  // fp32 K-slice planes [splits][m][n]
constexpr int kNoallocTickets = 16384;               // one per 16-row group: n <= 262144
constexpr int kMaxDevices = 64;

}  // namespace
}  // namespace qlx

static __device__ __align__(256) unsigned char scratch[qlx::kNoallocPlaneBytes + qlx::kNoallocTickets * 4];

namespace qlx {
namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, looked up once per device.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "linear_skinny_noalloc");
  QLX_REQUIRE(dev >= 0 && dev < kMaxDevices, "linear_skinny_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "linear_skinny_noalloc: hipGetSymbolAddress");
    QLX_REQUIRE(p != nullptr, "linear_skinny_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return QLX_OK;
}

// Ticket counters start each call at zero (a fill kernel, not a memset: graph-capture safe).
__global__ void __launch_bounds__(256) zero_ints(int* p, int count) {
  for (int i = threadIdx.x + blockIdx.x * 256; i < count; i += 256 * gridDim.x) p[i] = 0;
}

}  // namespace
}  // namespace qlx

extern "C" int qlx_linear_skinny_noalloc(int fmt, const void* w, const void* w_scale, const void* x, void* y, int m,
                                         int n, int k, int mode, void* stream) {
  QLX_REQUIRE(w && w_scale && x && y, "linear_skinny_noalloc: NULL pointer");
  // The formats qlx_linear_skinny serves; checked before the shared array is touched, so a
  // rejected call enqueues nothing.
  QLX_REQUIRE(fmt == QLX_FMT_W4A16 || fmt == QLX_FMT_W8A16,
              "linear_skinny_noalloc serves W4A16 and W8A16 (format %d)", fmt);
  qlx_plan plan = {};
  int rc = qlx_plan_skinny(fmt, mode, m, n, k, &plan);
  if (rc != QLX_OK) return rc;
  const long long plane_bytes = plan.splits > 1 ? 4ll * plan.splits * m * n : 0;
  QLX_REQUIRE(plane_bytes <= qlx::kNoallocPlaneBytes,
              "linear_skinny_noalloc: %d planes of %d x %d floats (%lld bytes) exceed the %lld-byte scratch",
              plan.splits, m, n, plane_bytes, qlx::kNoallocPlaneBytes);
  QLX_REQUIRE(n / 16 <= qlx::kNoallocTickets, "linear_skinny_noalloc: n=%d exceeds %d rows", n,
              qlx::kNoallocTickets * 16);
  void* base = nullptr;
  if ((rc = qlx::scratch_ptr(&base)) != QLX_OK) return rc;
  if (plan.splits > 1) {
    plan.workspace = static_cast<float*>(base);
    // Up to 32 tokens the row group's last workgroup reduces the planes (tickets); 33..64
    // token blocks share planes across blocks and reduce them in a second launch.
    if (m <= 32) {
      int* tickets = reinterpret_cast<int*>(static_cast<char*>(base) + qlx::kNoallocPlaneBytes);
      const int count = n / 16;
      qlx::zero_ints<<<(count + 255) / 256, 256, 0, (hipStream_t)stream>>>(tickets, count);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return qlx::hip_status(e, "linear_skinny_noalloc");
      plan.tickets = tickets;
    }
  }
  return qlx_linear_skinny(fmt, w, w_scale, x, y, m, n, k, &plan, stream);
}
