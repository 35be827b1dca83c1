// Fused PPO loss gradient (one lane per row; bandwidth-bound, exp/log in registers).
//
// Per row: log-sum-exp over the A policy logits (optionally max-shifted), p_k, log p(a), the
// importance ratio against the behaviour log-prob, the clipped-surrogate subgradient, the entropy
// gradient, and PufferLib's clipped value-loss gradient; ascent sign (puffercuda.cu:692-744,
// 4910-4930; pufferblas.c:726-736). Optionally the 7 dashboard losses are reduced deterministically
// (per-block partials in f64, folded in block order by a one-block kernel).
#include "common.hpp"
#include "kernels.hpp"
#include "losses.hpp"

namespace ph {
namespace {

constexpr int kMaxA = 64;

// VEC: logit and gradient rows are 16-byte aligned with a pitch that covers A rounded up to 4, so each
// row moves as float4s (a quarter of the memory instructions of the scalar form; same arithmetic).
template <int AMAX, bool VEC>
__global__ void __launch_bounds__(256) k_ppo_grad(
    const float* __restrict__ logits, int ldl, const float* __restrict__ values, int ldv,
    const int* __restrict__ act, const float* __restrict__ adv, const float* __restrict__ ret,
    const float* __restrict__ old, const float* __restrict__ ov, int N, int A, float vfCoef,
    float entCoef, float clipEps, float vfClip, int max_shift, float* __restrict__ dlogits, int ldd,
    float* __restrict__ dvalues, int lddv, float* __restrict__ newlp, float* __restrict__ newval,
    double* __restrict__ part, double* __restrict__ losses) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  double lsum[6] = {0, 0, 0, 0, 0, 0};  // pg, v, ent, old_kl, kl, nclip
  if (n < N) {
    const float* lg = logits + (size_t)n * ldl;
    // All AMAX loads are issued unconditionally (columns past A re-read column A-1, in bounds) so
    // they are in flight together; the values past A are masked where they are used.
    float x[AMAX];
    if constexpr (VEC && AMAX % 4 == 0) {
#pragma unroll
      for (int k4 = 0; k4 < AMAX; k4 += 4) {
        const float4 v = *reinterpret_cast<const float4*>(lg + (k4 < A ? k4 : 0));
        x[k4] = v.x;
        x[k4 + 1] = v.y;
        x[k4 + 2] = v.z;
        x[k4 + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int k = 0; k < AMAX; k++) x[k] = lg[k < A ? k : A - 1];
    }
    float lse;
    if (max_shift) {
      float mx = x[0];
#pragma unroll
      for (int k = 1; k < AMAX; k++) if (k < A && x[k] > mx) mx = x[k];
      float se = 0.f;
#pragma unroll
      for (int k = 0; k < AMAX; k++) if (k < A) se += expf(x[k] - mx);
      lse = mx + logf(se);
    } else {
      float se = 0.f;
#pragma unroll
      for (int k = 0; k < AMAX; k++) if (k < A) se += expf(x[k]);
      lse = logf(se);
    }
    float pk[AMAX];
    float pout = 0.f;
#pragma unroll
    for (int k = 0; k < AMAX; k++) {
      pk[k] = k < A ? expf(x[k] - lse) : 0.f;
      if (k < A) pout += pk[k] * x[k];
    }
    const int a = act[n];
    const float av = adv[n], rv = ret[n], ol = old[n];
    float xa = 0.f;
#pragma unroll
    for (int k = 0; k < AMAX; k++) if (k == a) xa = x[k];
    const float logpA = xa - lse;
    const float ratio = expf(logpA - ol);
    const float lo = 1.f - clipEps, hi = 1.f + clipEps;
    const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const float s1 = av * ratio, s2 = av * rc;
    float dpol;
    if (s1 <= s2) dpol = av * ratio;
    else dpol = av * ((lo < ratio && ratio < hi) ? 1.f : 0.f) * ratio;
    float* dl = dlogits + (size_t)n * ldd;
    auto dlk = [&](int k) { return dpol * ((k == a ? 1.f : 0.f) - pk[k]) + entCoef * pk[k] * (pout - x[k]); };
    if constexpr (VEC && AMAX % 4 == 0) {
#pragma unroll
      for (int k4 = 0; k4 < AMAX; k4 += 4) {
        if (k4 + 4 <= A) {
          *reinterpret_cast<float4*>(dl + k4) = make_float4(dlk(k4), dlk(k4 + 1), dlk(k4 + 2), dlk(k4 + 3));
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++)
            if (k4 + q < A) dl[k4 + q] = dlk(k4 + q);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < AMAX; k++)
        if (k < A) dl[k] = dlk(k);
    }
    const float vnew = values[(size_t)n * ldv];
    const float vold = ov ? ov[n] : 0.f;
    dvalues[(size_t)n * lddv] = -vfCoef * vloss_grad(vnew, rv, vold, ov != nullptr, vfClip);
    if (newlp) newlp[n] = logpA;
    if (newval) newval[n] = vnew;
    if (losses) {
      // entropy from the fp32 probabilities of the gradient path (one fp64 exp per row in row_losses
      // is for the ratio terms; 16 more per row made this kernel fp64-bound)
      float ent = 0.f;
#pragma unroll
      for (int k = 0; k < AMAX; k++)
        if (k < A) ent -= pk[k] * (x[k] - lse);
      row_losses(logpA, ol, av, vnew, rv, vold, vfClip > 0.f && ov, vfClip, clipEps, ent, lsum);
    }
  }
  if (losses) block_losses(lsum, part);
}

}  // namespace

int ppo_grad(const float* logits, size_t ldl, const float* values, size_t ldv, const int* act,
             const float* adv, const float* ret, const float* old, const float* ov, size_t N,
             size_t A, float vfCoef, float entCoef, float clipEps, float vfClip, int max_shift,
             float* dlogits, size_t ldd, float* dvalues, size_t lddv, float* newlp, float* newval,
             double* losses, hipStream_t st) {
  if (N == 0) return PH_OK;
  PH_REQUIRE(A >= 1 && A <= (size_t)kMaxA, "ppo_grad: action count %zu outside [1,%d]", A, kMaxA);
  const unsigned grid = ceil_div(N, 256);
  double* part = nullptr;
  if (losses) {
    part = (double*)scratch(kSlotPpoPart, (size_t)grid * 6 * 8);
    if (!part) return PH_ERR_NOMEM;
  }
  const size_t A4 = (A + 3) / 4 * 4;
  const bool vec = ldl % 4 == 0 && ldl >= A4 && ((uintptr_t)logits & 15) == 0 && ldd % 4 == 0 &&
                   ((uintptr_t)dlogits & 15) == 0;
#define PH_PPO(AM)                                                                                  \
  do {                                                                                              \
    if (vec)                                                                                        \
      k_ppo_grad<AM, true><<<grid, 256, 0, st>>>(logits, (int)ldl, values, (int)ldv, act, adv, ret, \
                                                 old, ov, (int)N, (int)A, vfCoef, entCoef, clipEps, \
                                                 vfClip, max_shift, dlogits, (int)ldd, dvalues,     \
                                                 (int)lddv, newlp, newval, part, losses);           \
    else                                                                                            \
      k_ppo_grad<AM, false><<<grid, 256, 0, st>>>(logits, (int)ldl, values, (int)ldv, act, adv,    \
                                                  ret, old, ov, (int)N, (int)A, vfCoef, entCoef,   \
                                                  clipEps, vfClip, max_shift, dlogits, (int)ldd,   \
                                                  dvalues, (int)lddv, newlp, newval, part, losses); \
  } while (0)
  if (A <= 2) PH_PPO(2);
  else if (A <= 4) PH_PPO(4);
  else if (A <= 8) PH_PPO(8);
  else if (A <= 16) PH_PPO(16);
  else if (A <= 32) PH_PPO(32);
  else PH_PPO(64);
#undef PH_PPO
  PH_LAUNCH_CHECK();
  if (losses) {
    k_fold_losses<<<1, 256, 0, st>>>(part, (int)grid, (long)N, vfCoef, entCoef, losses);
    PH_LAUNCH_CHECK();
  }
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_ppo_grad(const float* logits, size_t ldl, const float* values, size_t ldv,
                           const int* act, const float* adv, const float* ret, const float* old,
                           const float* ov, size_t N, size_t A, float vfCoef, float entCoef,
                           float clipEps, float vfClip, int max_shift, float* dlogits, size_t ldd,
                           float* dvalues, size_t lddv, float* newlp, float* newval,
                           double* losses, void* stream) {
  PH_REQUIRE(N <= (size_t)INT32_MAX, "ph_ppo_grad: N exceeds int32");
  PH_REQUIRE(N == 0 || (logits && values && act && adv && ret && old && dlogits && dvalues),
             "ph_ppo_grad: null pointer");
  return ppo_grad(logits, ldl, values, ldv, act, adv, ret, old, ov, N, A, vfCoef, entCoef, clipEps,
                  vfClip, max_shift, dlogits, ldd, dvalues, lddv, newlp, newval, losses,
                  as_stream(stream));
}
