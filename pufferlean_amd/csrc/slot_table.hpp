// Bookkeeping of the library's growable scratch slots, free of HIP so the host can test it alone.
//
// A slot holds one buffer that only grows. A request larger than the buffer allocates a new one and
// RETIRES the old one instead of freeing it: a HIP graph captured by an earlier call may still hold
// the old address in its kernel arguments, and replaying that graph must not touch freed memory.
// Retired buffers are freed only by release(), which the caller invokes when no such graph will be
// replayed again (ph_release_scratch). A slot that has never grown costs nothing extra.
#pragma once
#include <cstddef>
#include <vector>

namespace ph {

template <int NSLOT>
struct SlotTable {
  void* ptr[NSLOT] = {};
  size_t bytes[NSLOT] = {};
  unsigned gen[NSLOT] = {};   // allocations made for the slot so far
  unsigned zgen[NSLOT] = {};  // the allocation a zero-fill last cleared
  std::vector<void*> retired;
  size_t retired_bytes = 0;

  // Buffer of at least `bytes` for `slot` (rounded up to 256 bytes); nullptr if alloc fails, in which
  // case the slot keeps its old buffer. alloc(size) -> void* (nullptr on failure).
  template <typename Alloc>
  void* get(int slot, size_t bytes, Alloc&& alloc) {
    if (slot < 0 || slot >= NSLOT) return nullptr;
    if (bytes == 0) bytes = 1;
    if (this->bytes[slot] >= bytes) return ptr[slot];
    const size_t rounded = (bytes + 255) & ~(size_t)255;
    void* p = alloc(rounded);
    if (!p) return nullptr;
    if (ptr[slot]) {
      retired.push_back(ptr[slot]);
      retired_bytes += this->bytes[slot];
    }
    ptr[slot] = p;
    this->bytes[slot] = rounded;
    gen[slot]++;
    return p;
  }

  // Current buffer of a slot without allocating (nullptr if it has none).
  void* peek(int slot) const { return slot >= 0 && slot < NSLOT ? ptr[slot] : nullptr; }

  // Frees every retired buffer through free_fn(void*); returns how many.
  template <typename Free>
  size_t release(Free&& free_fn) {
    const size_t n = retired.size();
    for (void* p : retired) free_fn(p);
    retired.clear();
    retired_bytes = 0;
    return n;
  }
};

}  // namespace ph
