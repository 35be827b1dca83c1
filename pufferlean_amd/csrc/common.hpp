// Shared helpers for the pufferhip library (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/pufferhip.h"

namespace ph {

// Last-error text of the calling thread (read through ph_last_error()).
void set_error(const char* fmt, ...);

#define PH_CHECK_HIP(expr)                                                                  \
  do {                                                                                      \
    hipError_t e_ = (expr);                                                                 \
    if (e_ != hipSuccess) {                                                                 \
      ::ph::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__,      \
                      __LINE__);                                                            \
      return PH_ERR_HIP;                                                                    \
    }                                                                                       \
  } while (0)

#define PH_REQUIRE(cond, ...)                                                               \
  do {                                                                                      \
    if (!(cond)) {                                                                          \
      ::ph::set_error(__VA_ARGS__);                                                         \
      return PH_ERR_ARG;                                                                    \
    }                                                                                       \
  } while (0)

#define PH_TRY(expr)                                                                        \
  do {                                                                                      \
    int s_ = (expr);                                                                        \
    if (s_ != PH_OK) return s_;                                                             \
  } while (0)

// Launch-error check right after a <<<>>> launch.
#define PH_LAUNCH_CHECK() PH_CHECK_HIP(hipGetLastError())

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// LDS budget of every kernel in the library, per workgroup. Each kernel with a sizeable static LDS
// footprint asserts against it, and dynamic LDS is checked on the host before the launch. Larger
// footprints (a single workgroup may hold up to 160 KB on gfx950) stay out until a form using them
// has been shown sound.
constexpr int kMaxLdsBytes = 80 * 1024;

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Growable per-slot device buffers owned by the library (allocated on first use, reused across
// calls). A slot that must grow retires its old buffer instead of freeing it, since a captured graph
// may still use it; ph_release_scratch() frees retired buffers. Slot ids: kernels.hpp.
void* scratch(int slot, size_t bytes);
// The slot's current buffer, or nullptr if it has none (never allocates).
void* scratch_peek(int slot);
// scratch() whose memory is zero-filled (a fill kernel on st) whenever the slot is newly allocated;
// the caller keeps it zero between uses.
void* scratch_zeroed(int slot, size_t bytes, hipStream_t st);

// bf16 <-> f32 with round-to-nearest-even (IEEE bit trick; NaN kept quiet).
__host__ __device__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Device conversions on the gfx950 hardware converter (v_cvt_pk_bf16_f32, round-to-nearest-even).
typedef __bf16 ph_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ph_floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
  ph_floatx2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, ph_bf16x2));
}
__device__ __forceinline__ uint16_t bf16_rne(float a) { return (uint16_t)(bf16x2_rne(a, 0.f) & 0xffffu); }

// Logistic function on the hardware exp2 / reciprocal instructions (a few ulp). exp(-x) overflowing
// to +inf gives exactly 0. Shared by the MinGRU scans and the GEMM epilogue that applies a gate, so
// both see the same gate value.
__device__ __forceinline__ float sigm(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// Gradient of the (optionally clipped) value loss 0.5 (v - ret)^2 with respect to v: with vfClip > 0
// and an old value, the loss is max((v - ret)^2, (clip(v - vold) + vold - ret)^2) / 2
// (d_vloss_grad, puffercuda.cu:692-700).
__device__ inline float vloss_grad(float vnew, float ret, float vold, bool has_old, float vfClip) {
  if (vfClip <= 0.f || !has_old) return vnew - ret;
  const float dd = vnew - vold;
  const float vc = vold + (dd < -vfClip ? -vfClip : (dd > vfClip ? vfClip : dd));
  const float du = (vnew - ret) * (vnew - ret), cc = (vc - ret) * (vc - ret);
  if (du >= cc) return vnew - ret;
  if (dd > -vfClip && dd < vfClip) return vnew - ret;
  return 0.f;
}

}  // namespace ph
