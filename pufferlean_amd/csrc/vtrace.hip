// V-trace / GAE reverse scan (bandwidth-bound: no MFMA).
//
// One lane per segment walks t backwards; the recurrence runs in registers with the done mask
// applied there. Loads are issued a chunk of CH steps ahead of the dependent arithmetic so a lane
// keeps 4*CH loads in flight. Time-major [T][B] puts consecutive segments on consecutive lanes, so
// every load and store is a fully coalesced 256 B row per wavefront. Segment-major [B][T] rows are
// read with 16 B vector loads along t.
//
// Arithmetic follows the reference's sequential op order with contraction disabled, so the f64
// kernel is bit-identical to the reference CPU scans (puffercuda.cu:120-132, 200-211) and the f32
// kernel is bit-identical to an f32 evaluation of the same expressions.
#include "common.hpp"
#include "kernels.hpp"

namespace ph {
namespace {

template <typename R>
__device__ inline R clamp_unit(R r) {
  return r > R(1) ? R(1) : (r < R(-1) ? R(-1) : r);
}

template <typename R>
__device__ inline R ratio_of(R x, int is_log) {
  if (!is_log) return x;
  if constexpr (sizeof(R) == 8) return exp(x);
  else return expf(x);
}

// VARIANT 0: vec form (adv[T-1] = 0, delta = rho*(r + g*V'*nnt - V), done := term != 0).
// VARIANT 1: bootstrapped form (delta = rho*r + g*V'*nnt - V, V' at T-1 = boot, done := term > .5).
// rho == nullptr means ratio 1 (plain GAE).
template <typename R, int VARIANT, bool TIME_MAJOR, int CH>
__global__ void __launch_bounds__(256) k_vtrace(const R* __restrict__ rew, const R* __restrict__ val,
                                                const R* __restrict__ term, const R* __restrict__ rho,
                                                const R* __restrict__ boot, R* __restrict__ adv,
                                                R* __restrict__ tgt, int B, int T, int rho_is_log,
                                                int clamp, R gamma, R lam, R rhoClip, R cClip) {
#pragma clang fp contract(off)
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  auto at = [&](int t) -> size_t {
    return TIME_MAJOR ? (size_t)t * (size_t)B + (size_t)b : (size_t)b * (size_t)T + (size_t)t;
  };
  const R gl = gamma * lam;
  R last = R(0);
  R vnext;
  int tEnd;  // scan covers t = tEnd-1 .. 0
  if (VARIANT == 0) {
    if (T <= 0) return;
    const size_t il = at(T - 1);
    const R vl = val[il];
    adv[il] = R(0);
    if (tgt) tgt[il] = R(0) + vl;
    vnext = vl;
    tEnd = T - 1;
  } else {
    vnext = boot[b];
    tEnd = T;
  }
  // Two register buffers of CH steps: chunk k+1 is loaded while chunk k is computed. Every load is
  // unconditional (a step before t = 0 re-reads row 0, a few L2-resident bytes), so the loads of a
  // chunk issue together and the compiler waits for exactly the older buffer.
  R ra[CH], va[CH], da[CH], wa[CH], rb[CH], vb[CH], db[CH], wb[CH];
  auto ld = [&](R (&rr)[CH], R (&vv)[CH], R (&dd)[CH], R (&ww)[CH], int t0) {
#pragma unroll
    for (int c = 0; c < CH; c++) {
      const int tc = t0 - c >= 0 ? t0 - c : 0;
      const size_t i = at(tc);
      rr[c] = rew[i];
      vv[c] = val[i];
      dd[c] = term[i];
      ww[c] = rho ? rho[i] : R(1);
    }
  };
  auto step = [&](R r0, R v0, R d0, R w0, int tc) {
    const R w = ratio_of(w0, rho_is_log);
    const R rh = w < rhoClip ? w : rhoClip;
    const R cc = w < cClip ? w : cClip;
    const R r = clamp ? clamp_unit(r0) : r0;
    R nnt, delta;
    if (VARIANT == 0) {
      nnt = (d0 != R(0)) ? R(0) : R(1);
      delta = rh * (r + gamma * vnext * nnt - v0);
    } else {
      nnt = (d0 > R(0.5)) ? R(0) : R(1);
      delta = rh * r + gamma * vnext * nnt - v0;
    }
    last = delta + gl * cc * last * nnt;
    const size_t i = at(tc);
    adv[i] = last;
    if (tgt) tgt[i] = last + v0;
    vnext = v0;
  };
  // steps t0, t0-1, ..., t0-CH+1 (the tail chunk stops at t = 0)
  auto run = [&](const R (&rr)[CH], const R (&vv)[CH], const R (&dd)[CH], const R (&ww)[CH], int t0) {
    if (t0 >= CH - 1) {
#pragma unroll
      for (int c = 0; c < CH; c++) step(rr[c], vv[c], dd[c], ww[c], t0 - c);
    } else {
#pragma unroll
      for (int c = 0; c < CH; c++)
        if (t0 - c >= 0) step(rr[c], vv[c], dd[c], ww[c], t0 - c);
    }
  };
  int t = tEnd - 1;
  if (t < 0) return;
  ld(ra, va, da, wa, t);
  while (true) {
    ld(rb, vb, db, wb, t - CH);
    run(ra, va, da, wa, t);
    t -= CH;
    if (t < 0) break;
    ld(ra, va, da, wa, t - CH);
    run(rb, vb, db, wb, t);
    t -= CH;
    if (t < 0) break;
  }
}

template <typename R>
int launch_vtrace(const R* rew, const R* val, const R* term, const R* rho, const R* boot, size_t B,
                  size_t T, int variant, int time_major, int rho_is_log, int clamp, double gamma,
                  double lam, double rhoClip, double cClip, R* adv, R* tgt, hipStream_t st) {
  if (B == 0 || T == 0) return PH_OK;
  const unsigned grid = ceil_div(B, 256);
  constexpr int CH = sizeof(R) == 8 ? 4 : 8;
#define PH_VT(V, TM)                                                                        \
  k_vtrace<R, V, TM, CH><<<grid, 256, 0, st>>>(rew, val, term, rho, boot, adv, tgt, (int)B,     \
                                               (int)T, rho_is_log, clamp, (R)gamma, (R)lam,     \
                                               (R)rhoClip, (R)cClip)
  if (variant == 0) {
    if (time_major) PH_VT(0, true); else PH_VT(0, false);
  } else {
    if (time_major) PH_VT(1, true); else PH_VT(1, false);
  }
#undef PH_VT
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace

int vtrace_f32(const float* rew, const float* val, const float* term, const float* rho,
               const float* boot, size_t B, size_t T, int variant, int time_major, int rho_is_log,
               int clamp, double gamma, double lam, double rhoClip, double cClip, float* adv,
               float* tgt, hipStream_t st) {
  return launch_vtrace<float>(rew, val, term, rho, boot, B, T, variant, time_major, rho_is_log, clamp,
                              gamma, lam, rhoClip, cClip, adv, tgt, st);
}

}  // namespace ph

using namespace ph;

extern "C" int ph_vtrace(int dtype, const void* rew, const void* val, const void* term,
                         const void* rho, const void* boot, size_t B, size_t T, int variant,
                         int time_major, int rho_is_log, int clamp, double gamma, double lam,
                         double rhoClip, double cClip, void* adv, void* tgt, void* stream) {
  PH_REQUIRE(variant == 0 || variant == 1, "ph_vtrace: variant must be 0 or 1");
  PH_REQUIRE(variant == 0 || boot != nullptr || B == 0, "ph_vtrace: variant 1 needs boot values");
  PH_REQUIRE(B <= (size_t)INT32_MAX && T <= (size_t)INT32_MAX, "ph_vtrace: extents exceed int32");
  PH_REQUIRE(B * T == 0 || (rew && val && term && adv), "ph_vtrace: null input");
  if (dtype == PH_F32)
    return launch_vtrace<float>((const float*)rew, (const float*)val, (const float*)term,
                                (const float*)rho, (const float*)boot, B, T, variant, time_major,
                                rho_is_log, clamp, gamma, lam, rhoClip, cClip, (float*)adv,
                                (float*)tgt, as_stream(stream));
  if (dtype == PH_F64)
    return launch_vtrace<double>((const double*)rew, (const double*)val, (const double*)term,
                                 (const double*)rho, (const double*)boot, B, T, variant,
                                 time_major, rho_is_log, clamp, gamma, lam, rhoClip, cClip,
                                 (double*)adv, (double*)tgt, as_stream(stream));
  set_error("ph_vtrace: dtype must be PH_F32 or PH_F64");
  return PH_ERR_ARG;
}
