// Advantage normalisation with no device allocation, for callers that cannot allocate (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Same kernels and the same fixed-order reduction as ph_adv_normalize, with the per-chunk partials
// and the statistics in a file-scope device array instead of library scratch. Each device holds its
// own copy of the array (kNoAllocBytes) until the process ends. The array's name is a host-side
// stand-in: host code uses only the device address hipGetSymbolAddress returns for it, looked up
// once per device on the device's first call.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace {

// 2 x 4096 double partials (one per 4096-element chunk and pass) and 2 double statistics.
constexpr size_t kNoAllocMaxChunks = 4096;
constexpr size_t kNoAllocStatsOff = 2 * kNoAllocMaxChunks * 8;
constexpr size_t kNoAllocBytes = kNoAllocStatsOff + 256;
constexpr size_t kNoAllocMaxN = kNoAllocMaxChunks * ph::kMomentsChunk;  // 16,777,216 elements

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDev = 16;
void* g_ptr[kMaxDev] = {};
std::mutex g_mu;

// Device address of this device's array (nullptr and an error message on failure).
void* device_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    ph::set_error("ph_adv_normalize_noalloc: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      ph::set_error("ph_adv_normalize_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return nullptr;
    }
    g_ptr[dev] = p;
  }
  return g_ptr[dev];
}

}  // namespace

extern "C" int ph_adv_normalize_noalloc(int dtype, const void* adv, size_t n, void* out, void* stats,
                                        void* stream) {
  PH_REQUIRE(dtype == PH_F32 || dtype == PH_F64, "ph_adv_normalize_noalloc: dtype must be F32 or F64");
  PH_REQUIRE(n == 0 || (adv && out), "ph_adv_normalize_noalloc: null pointer");
  PH_REQUIRE(n <= kNoAllocMaxN,
             "ph_adv_normalize_noalloc: n=%zu exceeds the fixed workspace's maximum of %zu elements "
             "(ph_adv_normalize has no such limit)", n, kNoAllocMaxN);
  if (n == 0) return PH_OK;
  unsigned char* ws = (unsigned char*)device_scratch();
  if (!ws) return PH_ERR_HIP;
  return ph::moments_normalize_ws(dtype, adv, n, out, stats ? stats : ws + kNoAllocStatsOff, ws,
                                  ph::as_stream(stream));
}
