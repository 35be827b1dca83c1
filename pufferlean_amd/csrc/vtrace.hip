// V-trace / GAE reverse scan (bandwidth-bound: no MFMA).
//
// One lane per segment (two for large fp32 time-major batches) walks t backwards; the recurrence
// runs in registers with the done mask applied there. Loads are issued a chunk of CH steps ahead of the dependent arithmetic so a lane
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

// V consecutive segments per lane (V = 2: 8-byte vector accesses along b, time-major fp32 only).
// NT: nontemporal loads and stores (the scan streams every element exactly once).
template <typename R, int V> struct Lanes { R v[V]; };
template <typename R, int V, bool NT>
__device__ __forceinline__ Lanes<R, V> ldl(const R* p) {
  Lanes<R, V> o;
  if constexpr (V == 1) {
    o.v[0] = NT ? __builtin_nontemporal_load(p) : *p;
  } else {
    typedef R VT __attribute__((ext_vector_type(V)));
    const VT x = NT ? __builtin_nontemporal_load(reinterpret_cast<const VT*>(p)) : *reinterpret_cast<const VT*>(p);
#pragma unroll
    for (int q = 0; q < V; q++) o.v[q] = x[q];
  }
  return o;
}
template <typename R, int V, bool NT>
__device__ __forceinline__ void stl(R* p, const Lanes<R, V>& o) {
  if constexpr (V == 1) {
    if constexpr (NT) __builtin_nontemporal_store(o.v[0], p);
    else *p = o.v[0];
  } else {
    typedef R VT __attribute__((ext_vector_type(V)));
    VT x;
#pragma unroll
    for (int q = 0; q < V; q++) x[q] = o.v[q];
    if constexpr (NT) __builtin_nontemporal_store(x, reinterpret_cast<VT*>(p));
    else *reinterpret_cast<VT*>(p) = x;
  }
}

// VARIANT 0: vec form (adv[T-1] = 0, delta = rho*(r + g*V'*nnt - V), done := term != 0).
// VARIANT 1: bootstrapped form (delta = rho*r + g*V'*nnt - V, V' at T-1 = boot, done := term > .5).
// rho == nullptr means ratio 1 (plain GAE). Each lane runs the recurrence of V segments side by
// side, each in the reference's op order.
template <typename R, int VARIANT, bool TIME_MAJOR, int CH, int V, bool NT>
__global__ void __launch_bounds__(256) k_vtrace(const R* __restrict__ rew, const R* __restrict__ val,
                                                const R* __restrict__ term, const R* __restrict__ rho,
                                                const R* __restrict__ boot, R* __restrict__ adv,
                                                R* __restrict__ tgt, int B, int T, int rho_is_log,
                                                int clamp, R gamma, R lam, R rhoClip, R cClip) {
#pragma clang fp contract(off)
  static_assert(V == 1 || TIME_MAJOR, "vector lanes run along b (time-major rows)");
  const int b = (blockIdx.x * blockDim.x + threadIdx.x) * V;
  if (b >= B) return;
  auto at = [&](int t) -> size_t {
    return TIME_MAJOR ? (size_t)t * (size_t)B + (size_t)b : (size_t)b * (size_t)T + (size_t)t;
  };
  typedef Lanes<R, V> P;
  const R gl = gamma * lam;
  R last[V], vnext[V];
  int tEnd;  // scan covers t = tEnd-1 .. 0
  if (VARIANT == 0) {
    if (T <= 0) return;
    const size_t il = at(T - 1);
    const P vl = ldl<R, V, NT>(val + il);
    P z, tl;
#pragma unroll
    for (int q = 0; q < V; q++) {
      z.v[q] = R(0);
      tl.v[q] = R(0) + vl.v[q];
      vnext[q] = vl.v[q];
      last[q] = R(0);
    }
    stl<R, V, NT>(adv + il, z);
    if (tgt) stl<R, V, NT>(tgt + il, tl);
    tEnd = T - 1;
  } else {
    const P bv = ldl<R, V, false>(boot + b);
#pragma unroll
    for (int q = 0; q < V; q++) {
      vnext[q] = bv.v[q];
      last[q] = R(0);
    }
    tEnd = T;
  }
  // Two register buffers of CH steps: chunk k+1 is loaded while chunk k is computed. Every load is
  // unconditional (a step before t = 0 re-reads row 0, a few L2-resident bytes), so the loads of a
  // chunk issue together and the compiler waits for exactly the older buffer.
  P ra[CH], va[CH], da[CH], wa[CH], rb[CH], vb[CH], db[CH], wb[CH];
  auto ld = [&](P (&rr)[CH], P (&vv)[CH], P (&dd)[CH], P (&ww)[CH], int t0) {
#pragma unroll
    for (int c = 0; c < CH; c++) {
      const int tc = t0 - c >= 0 ? t0 - c : 0;
      const size_t i = at(tc);
      rr[c] = ldl<R, V, NT>(rew + i);
      vv[c] = ldl<R, V, NT>(val + i);
      dd[c] = ldl<R, V, NT>(term + i);
      if (rho) {
        ww[c] = ldl<R, V, NT>(rho + i);
      } else {
#pragma unroll
        for (int q = 0; q < V; q++) ww[c].v[q] = R(1);
      }
    }
  };
  auto step = [&](const P& r0, const P& v0, const P& d0, const P& w0, int tc) {
    P oa, ot;
#pragma unroll
    for (int q = 0; q < V; q++) {
      const R w = ratio_of(w0.v[q], rho_is_log);
      const R rh = w < rhoClip ? w : rhoClip;
      const R cc = w < cClip ? w : cClip;
      const R r = clamp ? clamp_unit(r0.v[q]) : r0.v[q];
      R nnt, delta;
      if (VARIANT == 0) {
        nnt = (d0.v[q] != R(0)) ? R(0) : R(1);
        delta = rh * (r + gamma * vnext[q] * nnt - v0.v[q]);
      } else {
        nnt = (d0.v[q] > R(0.5)) ? R(0) : R(1);
        delta = rh * r + gamma * vnext[q] * nnt - v0.v[q];
      }
      last[q] = delta + gl * cc * last[q] * nnt;
      oa.v[q] = last[q];
      ot.v[q] = last[q] + v0.v[q];
      vnext[q] = v0.v[q];
    }
    const size_t i = at(tc);
    stl<R, V, NT>(adv + i, oa);
    if (tgt) stl<R, V, NT>(tgt + i, ot);
  };
  // steps t0, t0-1, ..., t0-CH+1 (the tail chunk stops at t = 0)
  auto run = [&](const P (&rr)[CH], const P (&vv)[CH], const P (&dd)[CH], const P (&ww)[CH], int t0) {
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
  constexpr int CH = sizeof(R) == 8 ? 4 : 8;
  // Streaming form for large fp32 time-major batches: two segments per lane (8-byte accesses) and
  // nontemporal loads/stores, once there are >= 256 blocks of lanes (measured 5.86 vs 5.16 TB/s
  // over 262144 x 64); smaller batches keep one segment per lane for parallelism.
  const auto aligned8 = [](const void* p) { return p == nullptr || ((uintptr_t)p & 7) == 0; };
  const bool wide = sizeof(R) == 4 && time_major && B % 2 == 0 && B >= 2 * 256 * 256 &&
                    aligned8(rew) && aligned8(val) && aligned8(term) && aligned8(rho) &&
                    aligned8(boot) && aligned8(adv) && aligned8(tgt);
#define PH_VT(VAR, TM, VV, NT)                                                                     \
  k_vtrace<R, VAR, TM, CH, VV, NT><<<ceil_div(B / VV, 256), 256, 0, st>>>(                           \
      rew, val, term, rho, boot, adv, tgt, (int)B, (int)T, rho_is_log, clamp, (R)gamma, (R)lam,     \
      (R)rhoClip, (R)cClip)
  if constexpr (sizeof(R) == 4) {
    if (wide) {
      if (variant == 0) PH_VT(0, true, 2, true);
      else PH_VT(1, true, 2, true);
      PH_LAUNCH_CHECK();
      return PH_OK;
    }
  }
  if (variant == 0) {
    if (time_major) PH_VT(0, true, 1, false); else PH_VT(0, false, 1, false);
  } else {
    if (time_major) PH_VT(1, true, 1, false); else PH_VT(1, false, 1, false);
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
