// Library runtime: error channel, per-device growable buffers, device query.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <set>

#include "common.hpp"
#include "kernels.hpp"
#include "slot_table.hpp"

namespace ph {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

namespace {
constexpr int kMaxDev = 16;
constexpr int kSlots = 128;
SlotTable<kSlots> g_tables[kMaxDev];
std::mutex g_mu;
std::set<void*> g_zeroed;  // word blocks ensure_zeroed_words has cleared (by address)

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return -1;
  return dev;
}
}  // namespace

// Buffers only grow. A grown slot's old buffer is retired, not freed (a captured graph may still use
// it), so growth needs no device synchronisation and is legal between captures; ph_release_scratch()
// frees the retired buffers.
void* scratch(int slot, size_t bytes) {
  const int dev = current_device();
  if (dev < 0) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  void* p = g_tables[dev].get(slot, bytes, [&](size_t n) -> void* {
    void* q = nullptr;
    if (hipMalloc(&q, n) != hipSuccess) {
      (void)hipGetLastError();
      set_error("device allocation of %zu bytes failed (slot %d)", n, slot);
      return nullptr;
    }
    return q;
  });
  if (!p && (slot < 0 || slot >= kSlots)) set_error("scratch: slot %d out of range", slot);
  return p;
}

void* scratch_peek(int slot) {
  const int dev = current_device();
  if (dev < 0) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  return g_tables[dev].peek(slot);
}

namespace {
__global__ void k_zero_words(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}
}  // namespace

int ensure_zeroed_words(unsigned* words, int n, hipStream_t st) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_zeroed.count(words)) return PH_OK;
    g_zeroed.insert(words);
  }
  k_zero_words<<<1, 256, 0, st>>>(words, n);
  PH_LAUNCH_CHECK();
  return PH_OK;
}


namespace {
__global__ void k_zero_words_grid(unsigned* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = 0u;
}
}  // namespace

void* scratch_zeroed(int slot, size_t bytes, hipStream_t st) {
  void* p = scratch(slot, bytes);
  if (!p) return nullptr;
  const int dev = current_device();
  if (dev < 0) return nullptr;
  size_t sz = 0;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    SlotTable<kSlots>& tb = g_tables[dev];
    if (tb.zgen[slot] != tb.gen[slot]) {
      tb.zgen[slot] = tb.gen[slot];
      sz = tb.bytes[slot];
    }
  }
  if (sz) {
    const long words = (long)(sz / 4);
    const unsigned g = (unsigned)((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024);
    k_zero_words_grid<<<g, 256, 0, st>>>((unsigned*)p, words);
    if (hipGetLastError() != hipSuccess) {
      set_error("scratch_zeroed: fill launch failed (slot %d)", slot);
      return nullptr;
    }
  }
  return p;
}

namespace {
struct LaneTable {
  hipStream_t s[kLanes] = {};
  hipEvent_t fork = nullptr;
  hipEvent_t join[kLanes] = {};
};
LaneTable g_lanes[kMaxDev];

LaneTable* lane_table() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return nullptr;
  return &g_lanes[dev];
}

hipEvent_t make_event(hipEvent_t& e) {
  if (!e && hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    e = nullptr;
  }
  return e;
}
}  // namespace

hipStream_t lane_stream(int lane) {
  if (lane < 0 || lane >= kLanes) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  LaneTable* t = lane_table();
  if (!t) return nullptr;
  if (!t->s[lane] && hipStreamCreateWithFlags(&t->s[lane], hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    t->s[lane] = nullptr;
  }
  return t->s[lane];
}

int fork_lanes(hipStream_t main, int n) {
  PH_REQUIRE(n >= 0 && n <= kLanes, "fork_lanes: %d lanes", n);
  hipEvent_t ev = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    LaneTable* t = lane_table();
    if (t) ev = make_event(t->fork);
  }
  if (!ev) {
    set_error("fork_lanes: event creation failed");
    return PH_ERR_HIP;
  }
  PH_CHECK_HIP(hipEventRecord(ev, main));
  for (int i = 0; i < n; i++) {
    hipStream_t s = lane_stream(i);
    if (!s) {
      set_error("fork_lanes: stream creation failed");
      return PH_ERR_HIP;
    }
    PH_CHECK_HIP(hipStreamWaitEvent(s, ev, 0));
  }
  return PH_OK;
}

int join_lanes(hipStream_t main, int n) {
  PH_REQUIRE(n >= 0 && n <= kLanes, "join_lanes: %d lanes", n);
  for (int i = 0; i < n; i++) {
    hipEvent_t ev = nullptr;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      LaneTable* t = lane_table();
      if (t) ev = make_event(t->join[i]);
    }
    hipStream_t s = lane_stream(i);
    if (!ev || !s) {
      set_error("join_lanes: event or stream creation failed");
      return PH_ERR_HIP;
    }
    PH_CHECK_HIP(hipEventRecord(ev, s));
    PH_CHECK_HIP(hipStreamWaitEvent(main, ev, 0));
  }
  return PH_OK;
}

void join_lanes_on_exit(hipStream_t main, int n) {
  char saved[sizeof(g_err)];
  snprintf(saved, sizeof(saved), "%s", g_err);
  if (join_lanes(main, n) != PH_OK) set_error("%s", saved);
}

}  // namespace ph

extern "C" const char* ph_last_error(void) { return ph::g_err; }

extern "C" int ph_version(void) { return PH_VERSION; }

extern "C" int ph_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

extern "C" int ph_release_scratch(void) {
  const int dev = ph::current_device();
  if (dev < 0) {
    ph::set_error("ph_release_scratch: no current device");
    return PH_ERR_HIP;
  }
  PH_CHECK_HIP(hipDeviceSynchronize());
  std::lock_guard<std::mutex> lk(ph::g_mu);
  hipError_t err = hipSuccess;
  ph::g_tables[dev].release([&](void* p) {
    ph::g_zeroed.erase(p);
    const hipError_t e = hipFree(p);
    if (e != hipSuccess && err == hipSuccess) err = e;
  });
  if (err != hipSuccess) {
    ph::set_error("ph_release_scratch: hipFree failed: %s", hipGetErrorString(err));
    return PH_ERR_HIP;
  }
  return PH_OK;
}

extern "C" int ph_scratch_retired(size_t* count, size_t* bytes) {
  const int dev = ph::current_device();
  if (dev < 0) {
    ph::set_error("ph_scratch_retired: no current device");
    return PH_ERR_HIP;
  }
  std::lock_guard<std::mutex> lk(ph::g_mu);
  if (count) *count = ph::g_tables[dev].retired.size();
  if (bytes) *bytes = ph::g_tables[dev].retired_bytes;
  return PH_OK;
}

extern "C" int ph_synchronize(void* stream) {
  PH_CHECK_HIP(hipStreamSynchronize(ph::as_stream(stream)));
  return PH_OK;
}
