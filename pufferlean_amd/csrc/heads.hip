// Multi-discrete and continuous policy heads: the fused PPO loss gradient and the samplers for K
// categorical heads and for a diagonal Gaussian.
//
//   ph_ppo_grad_md / ph_sample_actions_md      k_ppo_dout_md, puffercuda.cu:702-727; k_sample_md 1538-1551
//   ph_ppo_grad_cont / ph_sample_actions_cont  k_ppo_dout_cont 1767-1790; k_sample_cont 1652-1668;
//                                              CPU twin of the Gaussian gradient pufferffi.c:223-330
//
// One lane per row, as the heads are a few dozen columns wide; each row's head outputs are read once
// and its gradient row written once.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"
#include "losses.hpp"

#pragma clang fp contract(off)

namespace ph {
namespace {

constexpr double kHalfLog2Pi = 0.9189385332046727;  // log(2 pi) / 2

__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
constexpr unsigned long long kGold = 0x9E3779B97F4A7C15ULL, kGold2 = 0xD1B54A32D192ED03ULL;
__device__ __forceinline__ double unit53(unsigned long long w) { return (double)(w >> 11) / 9007199254740992.0; }
__device__ __forceinline__ float ex(float x) { return expf(x); }
__device__ __forceinline__ double ex(double x) { return exp(x); }
__device__ __forceinline__ float lg(float x) { return logf(x); }
__device__ __forceinline__ double lg(double x) { return log(x); }

// ---- multi-discrete -------------------------------------------------------------------------------
// Row n: head h owns logits [off_h, off_h + size_h) (off = running sum of sizes), the value is at
// column W = sum of sizes; act[n*K + h] is head h's action. joint = sum_h log softmax_h[a_h]
// (max-shifted log-sum-exp); one clipped surrogate on exp(joint - old); per head
//   dlogit_k = dPol (onehot(a_h)_k - p_k) + ent p_k (sum_j p_j l_j - l_k)
// (the entropy term is d/dl_k of the head's entropy), dvalue = -vf dvloss. With losses, the dashboard
// losses of the rows (entropy summed over the heads) are folded into losses[7].
__global__ void __launch_bounds__(256) k_ppo_grad_md(const float* __restrict__ out, long ldo,
                                                     const int* __restrict__ act, const float* __restrict__ adv,
                                                     const float* __restrict__ ret, const float* __restrict__ old,
                                                     const float* __restrict__ ov, long N, HeadSizes hs, int W,
                                                     float vf, float ent, float clip, float vfClip,
                                                     float* __restrict__ dout, long ldd, float* __restrict__ newlp,
                                                     float* __restrict__ newval, double* __restrict__ part,
                                                     double* __restrict__ losses) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  double lsum[6] = {0, 0, 0, 0, 0, 0};
  if (n < N) {
    const float* o = out + n * ldo;
    float* d = dout + n * ldd;
    const int* a = act + n * hs.K;
    float joint = 0.f;
    bool inRange = true;
    int off = 0;
    for (int h = 0; h < hs.K; h++) {
      const int sz = hs.n[h], ah = a[h];
      float m = o[off];
      for (int k = 1; k < sz; k++) m = fmaxf(m, o[off + k]);
      float se = 0.f;
      for (int k = 0; k < sz; k++) se += expf(o[off + k] - m);
      if (ah >= 0 && ah < sz) joint += o[off + ah] - (m + logf(se));
      else inRange = false;  // never read outside the head's logits
      off += sz;
    }
    if (!inRange) joint = __builtin_nanf("");
    const float ratio = expf(joint - old[n]), lo = 1.f - clip, hi = 1.f + clip;
    const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const float A = adv[n];
    const float dPol = !inRange ? __builtin_nanf("")
                     : (A * ratio <= A * rc) ? A * ratio : ((lo < ratio && ratio < hi) ? A * ratio : 0.f);
    float entropy = 0.f;
    off = 0;
    for (int h = 0; h < hs.K; h++) {
      const int sz = hs.n[h];
      float m = o[off];
      for (int k = 1; k < sz; k++) m = fmaxf(m, o[off + k]);
      float se = 0.f;
      for (int k = 0; k < sz; k++) se += expf(o[off + k] - m);
      const float lse = m + logf(se);
      float pout = 0.f;
      for (int k = 0; k < sz; k++) pout += expf(o[off + k] - lse) * o[off + k];
      for (int k = 0; k < sz; k++) {
        const float p = expf(o[off + k] - lse);
        d[off + k] = dPol * ((k == a[h] ? 1.f : 0.f) - p) + ent * p * (pout - o[off + k]);
        entropy -= p * (o[off + k] - lse);
      }
      off += sz;
    }
    const float vold = ov ? ov[n] : 0.f;
    d[W] = -vf * vloss_grad(o[W], ret[n], vold, ov != nullptr, vfClip);
    if (newlp) newlp[n] = joint;
    if (newval) newval[n] = o[W];
    if (losses) row_losses(joint, old[n], A, o[W], ret[n], vold, vfClip > 0.f && ov, vfClip, clip, entropy, lsum);
  }
  if (losses) block_losses(lsum, part);
}

// ---- LDS-staged forms for rows up to kTileW wide ---------------------------------------------------
// A workgroup's 256 rows of head outputs arrive through LDS with coalesced loads (columns past the
// row width, if the stride has any, are skipped), each lane then holds its row in
// registers, and the gradient rows leave through the same tile with coalesced stores. The pitch is
// odd, so the lanes reading one column of their rows hit distinct banks. Head boundaries are the
// same for every lane, so the per-head loops below branch uniformly.
constexpr int kTileW = 32;
constexpr int kTileP = 33;

// Lane t walks the (row, column) pairs t, t + 256, ... of the R x O block in row-major order; the
// pair advances by 256 / O rows and 256 % O columns with a carry, so no division runs per element.
__device__ __forceinline__ void tile_load(const float* __restrict__ src, long ld, int O, long n0, int R,
                                          float* __restrict__ tile) {
  // a lane's share is at most kTileW elements (R * O <= 256 * kTileW): every load is issued before
  // the first LDS store waits on one
  constexpr int kPer = kTileW;
  const int q = (int)blockDim.x / O, rm = (int)blockDim.x % O;
  int r = (int)threadIdx.x / O, c = (int)threadIdx.x % O;
  const float* s = src + n0 * ld;
  float v[kPer];
  int dst[kPer];
#pragma unroll
  for (int it = 0; it < kPer; it++) {
    dst[it] = -1;
    if (r < R) {
      v[it] = s[(long)r * ld + c];
      dst[it] = r * kTileP + c;
    }
    r += q;
    c += rm;
    if (c >= O) {
      c -= O;
      r++;
    }
  }
#pragma unroll
  for (int it = 0; it < kPer; it++)
    if (dst[it] >= 0) tile[dst[it]] = v[it];
}
__device__ __forceinline__ void tile_store(float* __restrict__ dst, long ld, int O, long n0, int R,
                                           const float* __restrict__ tile) {
  const int q = (int)blockDim.x / O, rm = (int)blockDim.x % O;
  int r = (int)threadIdx.x / O, c = (int)threadIdx.x % O;
  float* d = dst + n0 * ld;
  while (r < R) {
    d[(long)r * ld + c] = tile[r * kTileP + c];
    r += q;
    c += rm;
    if (c >= O) {
      c -= O;
      r++;
    }
  }
}

// k_ppo_grad_md for W + 1 <= kTileW and K <= kTileHeads: each probability is computed once and kept
// with its head's expected logit for the gradient pass; the actions and the row's scalars are loaded
// before the staging barrier, so their latency overlaps the tile's.
constexpr int kTileHeads = 8;
__global__ void __launch_bounds__(256) k_ppo_grad_md_tile(const float* __restrict__ out, long ldo,
                                                          const int* __restrict__ act, const float* __restrict__ adv,
                                                          const float* __restrict__ ret, const float* __restrict__ old,
                                                          const float* __restrict__ ov, long N, HeadSizes hs, int W,
                                                          float vf, float ent, float clip, float vfClip,
                                                          float* __restrict__ dout, long ldd, float* __restrict__ newlp,
                                                          float* __restrict__ newval, double* __restrict__ part,
                                                          double* __restrict__ losses) {
  __shared__ float tile[256 * kTileP];
  static_assert(256 * kTileP * 4 <= kMaxLdsBytes, "LDS budget");
  const long n0 = (long)blockIdx.x * 256;
  const int R = (int)(N - n0 < 256 ? N - n0 : 256);
  const int t = threadIdx.x, O = W + 1, K = hs.K;
  const long n = n0 + t;
  const bool live = t < R;
  int av[kTileHeads];
  float A = 0.f, rv = 0.f, ol = 0.f, vold = 0.f;
  if (live) {
#pragma unroll
    for (int h = 0; h < kTileHeads; h++) av[h] = h < K ? act[n * K + h] : 0;
    A = adv[n];
    rv = ret[n];
    ol = old[n];
    vold = ov ? ov[n] : 0.f;
  }
  tile_load(out, ldo, O, n0, R, tile);
  __syncthreads();
  double lsum[6] = {0, 0, 0, 0, 0, 0};
  if (live) {
    float x[kTileW], p[kTileW], pouth[kTileHeads];
#pragma unroll
    for (int k = 0; k < kTileW; k++) x[k] = k < O ? tile[t * kTileP + k] : 0.f;
    float joint = 0.f, entropy = 0.f;
    unsigned hit = 0u;
    bool inRange = true;
    int off = 0;
#pragma unroll
    for (int h = 0; h < kTileHeads; h++) {
      pouth[h] = 0.f;
      if (h >= K) break;
      const int end = off + hs.n[h], ah = av[h];
      float m = -INFINITY;
#pragma unroll
      for (int k = 0; k < kTileW; k++)
        if (k >= off && k < end) m = fmaxf(m, x[k]);
      float se = 0.f;
#pragma unroll
      for (int k = 0; k < kTileW; k++)
        if (k >= off && k < end) se += expf(x[k] - m);
      const float lse = m + logf(se);
      float po = 0.f, xa = 0.f;
#pragma unroll
      for (int k = 0; k < kTileW; k++)
        if (k >= off && k < end) {
          p[k] = expf(x[k] - lse);
          po += p[k] * x[k];
          entropy -= p[k] * (x[k] - lse);
          if (k == off + ah) xa = x[k];
        }
      pouth[h] = po;
      if (ah >= 0 && ah < end - off) {
        joint += xa - lse;
        hit |= 1u << (off + ah);
      } else {
        inRange = false;
      }
      off = end;
    }
    if (!inRange) joint = __builtin_nanf("");
    const float ratio = expf(joint - ol), lo = 1.f - clip, hi = 1.f + clip;
    const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const float dPol = !inRange ? __builtin_nanf("")
                     : (A * ratio <= A * rc) ? A * ratio : ((lo < ratio && ratio < hi) ? A * ratio : 0.f);
    // the gradient pass walks the heads again: each head's expected logit stays one register
    off = 0;
#pragma unroll
    for (int h = 0; h < kTileHeads; h++) {
      if (h >= K) break;
      const int end = off + hs.n[h];
#pragma unroll
      for (int k = 0; k < kTileW; k++)
        if (k >= off && k < end)
          tile[t * kTileP + k] = dPol * ((float)((hit >> k) & 1u) - p[k]) + ent * p[k] * (pouth[h] - x[k]);
      off = end;
    }
    float vnew = 0.f;
#pragma unroll
    for (int k = 0; k < kTileW; k++)
      if (k == W) vnew = x[k];
    tile[t * kTileP + W] = -vf * vloss_grad(vnew, rv, vold, ov != nullptr, vfClip);
    if (newlp) newlp[n] = joint;
    if (newval) newval[n] = vnew;
    if (losses) row_losses(joint, ol, A, vnew, rv, vold, vfClip > 0.f && ov, vfClip, clip, entropy, lsum);
  }
  __syncthreads();
  tile_store(dout, ldd, O, n0, R, tile);
  if (losses) block_losses(lsum, part);
}

// k_ppo_grad_cont for 2d + 1 <= kTileW.
__global__ void __launch_bounds__(256) k_ppo_grad_cont_tile(const float* __restrict__ out, long ldo,
                                                            const float* __restrict__ act, const float* __restrict__ adv,
                                                            const float* __restrict__ ret, const float* __restrict__ old,
                                                            const float* __restrict__ ov, long N, int d, float vf,
                                                            float ent, float clip, float vfClip, float lslo, float lshi,
                                                            float* __restrict__ dout, long ldd,
                                                            float* __restrict__ newlp, float* __restrict__ newval,
                                                            double* __restrict__ part,
                                                            double* __restrict__ losses) {
  __shared__ float tile[256 * kTileP];
  static_assert(256 * kTileP * 4 <= kMaxLdsBytes, "LDS budget");
  const long n0 = (long)blockIdx.x * 256;
  const int R = (int)(N - n0 < 256 ? N - n0 : 256);
  const int t = threadIdx.x, W = 2 * d, O = W + 1;
  tile_load(out, ldo, O, n0, R, tile);
  __syncthreads();
  double lsum[6] = {0, 0, 0, 0, 0, 0};
  if (t < R) {
    const long n = n0 + t;
    constexpr int DM = kTileW / 2;
    float mu[DM], lsr[DM], z[DM];
#pragma unroll
    for (int i = 0; i < DM; i++) {
      mu[i] = i < d ? tile[t * kTileP + i] : 0.f;
      lsr[i] = i < d ? tile[t * kTileP + d + i] : 0.f;
    }
    const float vnew = tile[t * kTileP + W];
    const float* a = act + n * d;
    const float hl = (float)kHalfLog2Pi;
    float logp = 0.f, entropy = 0.f;
#pragma unroll
    for (int i = 0; i < DM; i++)
      if (i < d) {
        const float ls = lsr[i] < lslo ? lslo : (lsr[i] > lshi ? lshi : lsr[i]);
        z[i] = (a[i] - mu[i]) * expf(-ls);
        logp += -0.5f * z[i] * z[i] - ls - hl;
        entropy += ls + (0.5f + hl);
      }
    const float ratio = expf(logp - old[n]), lo = 1.f - clip, hi = 1.f + clip;
    const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const float A = adv[n];
    const float dPol = (A * ratio <= A * rc) ? A * ratio : ((lo < ratio && ratio < hi) ? A * ratio : 0.f);
#pragma unroll
    for (int i = 0; i < DM; i++)
      if (i < d) {
        const float ls = lsr[i] < lslo ? lslo : (lsr[i] > lshi ? lshi : lsr[i]);
        tile[t * kTileP + i] = dPol * z[i] * expf(-ls);
        tile[t * kTileP + d + i] = (lslo < lsr[i] && lsr[i] < lshi) ? dPol * (z[i] * z[i] - 1.f) + ent : 0.f;
      }
    const float vold = ov ? ov[n] : 0.f;
    tile[t * kTileP + W] = -vf * vloss_grad(vnew, ret[n], vold, ov != nullptr, vfClip);
    if (newlp) newlp[n] = logp;
    if (newval) newval[n] = vnew;
    if (losses) row_losses(logp, old[n], A, vnew, ret[n], vold, vfClip > 0.f && ov, vfClip, clip, entropy, lsum);
  }
  __syncthreads();
  tile_store(dout, ldd, O, n0, R, tile);
  if (losses) block_losses(lsum, part);
}

// Draws per head: word of rng + (n+1) GOLD + (h+1) GOLD2; out = [actions (head h at h*N + n); joint
// logp (N); value (N)] as f64. R is the logit type.
template <typename R>
__global__ void __launch_bounds__(256) k_sample_md(const R* __restrict__ Y, long ldy, long N, HeadSizes hs, int W,
                                                   unsigned long long rng, double* __restrict__ out) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const R* row = Y + n * ldy;
  R joint = 0;
  int off = 0;
  for (int h = 0; h < hs.K; h++) {
    const int sz = hs.n[h];
    R m = row[off];
    for (int k = 1; k < sz; k++)
      if (row[off + k] > m) m = row[off + k];
    R z = 0;
    for (int k = 0; k < sz; k++) z += ex(row[off + k] - m);
    const double u =
        unit53(mix64(rng + (unsigned long long)(n + 1) * kGold + (unsigned long long)(h + 1) * kGold2));
    R acc = 0;
    int a = sz - 1;
    for (int k = 0; k < sz; k++) {
      acc += ex(row[off + k] - m) / z;
      if (u < (double)acc) {
        a = k;
        break;
      }
    }
    out[(long)h * N + n] = (double)a;
    joint += lg(ex(row[off + a] - m) / z);
    off += sz;
  }
  out[(long)hs.K * N + n] = (double)joint;
  out[(long)(hs.K + 1) * N + n] = (double)row[W];
}

// ---- continuous (diagonal Gaussian) ---------------------------------------------------------------
// Row n: means [0, d), raw log-stds [d, 2d) clamped to [lslo, lshi], the value at 2d; act[n*d + i].
//   z_i = (a_i - mu_i) exp(-ls_i),  logp = sum_i (-z_i^2 / 2 - ls_i - log(2 pi) / 2)
//   dmu_i = dPol z_i exp(-ls_i),  dls_i = (dPol (z_i^2 - 1) + ent) [lslo < raw ls < lshi]
// With losses, the dashboard losses (entropy sum_i (ls_i + (1 + log(2 pi)) / 2)) go into losses[7].
__global__ void __launch_bounds__(256) k_ppo_grad_cont(const float* __restrict__ out, long ldo,
                                                       const float* __restrict__ act, const float* __restrict__ adv,
                                                       const float* __restrict__ ret, const float* __restrict__ old,
                                                       const float* __restrict__ ov, long N, int d, float vf, float ent,
                                                       float clip, float vfClip, float lslo, float lshi,
                                                       float* __restrict__ dout, long ldd, float* __restrict__ newlp,
                                                       float* __restrict__ newval, double* __restrict__ part,
                                                       double* __restrict__ losses) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  double lsum[6] = {0, 0, 0, 0, 0, 0};
  if (n < N) {
    const float* o = out + n * ldo;
    float* g = dout + n * ldd;
    const float* a = act + n * d;
    const float hl = (float)kHalfLog2Pi;
    float logp = 0.f, entropy = 0.f;
    for (int i = 0; i < d; i++) {
      const float lsr = o[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
      const float z = (a[i] - o[i]) * expf(-ls);
      logp += -0.5f * z * z - ls - hl;
      entropy += ls + (0.5f + hl);  // differential entropy of the dim: ls + (1 + log(2 pi)) / 2
    }
    const float ratio = expf(logp - old[n]), lo = 1.f - clip, hi = 1.f + clip;
    const float rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const float A = adv[n];
    const float dPol = (A * ratio <= A * rc) ? A * ratio : ((lo < ratio && ratio < hi) ? A * ratio : 0.f);
    for (int i = 0; i < d; i++) {
      const float lsr = o[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
      const float inv = expf(-ls), z = (a[i] - o[i]) * inv;
      g[i] = dPol * z * inv;
      g[d + i] = (lslo < lsr && lsr < lshi) ? dPol * (z * z - 1.f) + ent : 0.f;
    }
    const int W = 2 * d;
    const float vold = ov ? ov[n] : 0.f;
    g[W] = -vf * vloss_grad(o[W], ret[n], vold, ov != nullptr, vfClip);
    if (newlp) newlp[n] = logp;
    if (newval) newval[n] = o[W];
    if (losses) row_losses(logp, old[n], A, o[W], ret[n], vold, vfClip > 0.f && ov, vfClip, clip, entropy, lsum);
  }
  if (losses) block_losses(lsum, part);
}

// Box-Muller per dim from two words, rng + (n+1) GOLD + (2i+1) GOLD2 and (2i+2) GOLD2 (u1 floored at
// 1e-7): z = sqrt(-2 log u1) cos(2 pi u2); a = mu + exp(ls) z; logp = sum(-z^2/2 - ls - log(2 pi)/2).
// out = [actions (dim i at i*N + n); logp (N); value (N)] as f64. f64 rows compute in f64; f32 rows
// compute z in f64 and the rest in f32, as the reference's two forms do.
template <typename R>
__global__ void __launch_bounds__(256) k_sample_cont(const R* __restrict__ Y, long ldy, long N, int d,
                                                     unsigned long long rng, R lslo, R lshi, double* __restrict__ out) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const R* row = Y + n * ldy;
  R logp = 0;
  for (int i = 0; i < d; i++) {
    const R lsr = row[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
    const unsigned long long base = rng + (unsigned long long)(n + 1) * kGold;
    double u1 = unit53(mix64(base + (unsigned long long)(2 * i + 1) * kGold2));
    if (u1 < 1.0e-7) u1 = 1.0e-7;
    const double u2 = unit53(mix64(base + (unsigned long long)(2 * i + 2) * kGold2));
    const R z = (R)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    const R a = row[i] + ex(ls) * z;
    out[(long)i * N + n] = (double)a;
    logp += (R)(-0.5) * z * z - ls - (R)kHalfLog2Pi;
  }
  out[(long)d * N + n] = (double)logp;
  out[(long)(d + 1) * N + n] = (double)row[2 * d];
}

int head_sizes(const int* sizes, size_t K, HeadSizes& hs, int& W, const char* who) {
  PH_REQUIRE(sizes && K >= 1 && K <= (size_t)kMaxHeads, "%s: K=%zu heads (1..%d)", who, K, kMaxHeads);
  hs.K = (int)K;
  W = 0;
  for (size_t h = 0; h < K; h++) {
    PH_REQUIRE(sizes[h] >= 1 && sizes[h] <= 4096, "%s: head %zu has %d actions", who, h, sizes[h]);
    hs.n[h] = sizes[h];
    W += sizes[h];
  }
  return PH_OK;
}

}  // namespace

// Block partials of the dashboard losses for a grid of `grid` blocks (none without losses), and their
// fold after the kernel.
static int loss_part(double* losses, unsigned grid, double*& part) {
  part = nullptr;
  if (!losses) return PH_OK;
  part = (double*)scratch(kSlotHeadsPart, (size_t)grid * 6 * 8);
  return part ? PH_OK : PH_ERR_NOMEM;
}
static int loss_fold(double* losses, const double* part, unsigned grid, size_t N, float vf, float ent, hipStream_t st) {
  if (!losses) return PH_OK;
  k_fold_losses<<<1, 256, 0, st>>>(part, (int)grid, (long)N, vf, ent, losses);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int ppo_grad_md(const float* out, size_t ldo, const int* act, const float* adv, const float* ret, const float* old,
                const float* ov, size_t N, const int* sizes, size_t K, float vf, float ent, float clip, float vfClip,
                float* dout, size_t ldd, float* newlp, float* newval, double* losses, hipStream_t st) {
  HeadSizes hs;
  int W;
  PH_TRY(head_sizes(sizes, K, hs, W, "ppo_grad_md"));
  PH_REQUIRE(ldo >= (size_t)W + 1 && ldd >= (size_t)W + 1, "ppo_grad_md: row stride below %d", W + 1);
  if (N == 0) return PH_OK;
  const unsigned grid = ceil_div(N, 256);
  double* part;
  PH_TRY(loss_part(losses, grid, part));
  if (W + 1 <= kTileW && K <= (size_t)kTileHeads)
    k_ppo_grad_md_tile<<<grid, 256, 0, st>>>(out, (long)ldo, act, adv, ret, old, ov, (long)N, hs, W, vf, ent, clip,
                                             vfClip, dout, (long)ldd, newlp, newval, part, losses);
  else
    k_ppo_grad_md<<<grid, 256, 0, st>>>(out, (long)ldo, act, adv, ret, old, ov, (long)N, hs, W, vf, ent, clip, vfClip,
                                        dout, (long)ldd, newlp, newval, part, losses);
  PH_LAUNCH_CHECK();
  return loss_fold(losses, part, grid, N, vf, ent, st);
}

int ppo_grad_cont(const float* out, size_t ldo, const float* act, const float* adv, const float* ret,
                  const float* old, const float* ov, size_t N, size_t d, float vf, float ent, float clip, float vfClip,
                  float lslo, float lshi, float* dout, size_t ldd, float* newlp, float* newval, double* losses,
                  hipStream_t st) {
  PH_REQUIRE(d >= 1 && ldo >= 2 * d + 1 && ldd >= 2 * d + 1, "ppo_grad_cont: d=%zu ldo=%zu ldd=%zu", d, ldo, ldd);
  if (N == 0) return PH_OK;
  const unsigned grid = ceil_div(N, 256);
  double* part;
  PH_TRY(loss_part(losses, grid, part));
  if (2 * d + 1 <= (size_t)kTileW)
    k_ppo_grad_cont_tile<<<grid, 256, 0, st>>>(out, (long)ldo, act, adv, ret, old, ov, (long)N, (int)d, vf, ent, clip,
                                               vfClip, lslo, lshi, dout, (long)ldd, newlp, newval, part, losses);
  else
    k_ppo_grad_cont<<<grid, 256, 0, st>>>(out, (long)ldo, act, adv, ret, old, ov, (long)N, (int)d, vf, ent, clip,
                                          vfClip, lslo, lshi, dout, (long)ldd, newlp, newval, part, losses);
  PH_LAUNCH_CHECK();
  return loss_fold(losses, part, grid, N, vf, ent, st);
}

int sample_actions_md(int dtype, const void* Y, size_t ldy, size_t N, const int* sizes, size_t K, uint64_t rng,
                      double* out, hipStream_t st) {
  HeadSizes hs;
  int W;
  PH_TRY(head_sizes(sizes, K, hs, W, "sample_actions_md"));
  PH_REQUIRE(ldy >= (size_t)W + 1, "sample_actions_md: row stride below %d", W + 1);
  if (N == 0) return PH_OK;
  if (dtype == PH_F64)
    k_sample_md<double><<<ceil_div(N, 256), 256, 0, st>>>((const double*)Y, (long)ldy, (long)N, hs, W, rng, out);
  else
    k_sample_md<float><<<ceil_div(N, 256), 256, 0, st>>>((const float*)Y, (long)ldy, (long)N, hs, W, rng, out);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int sample_actions_cont(int dtype, const void* Y, size_t ldy, size_t N, size_t d, uint64_t rng, double lslo,
                        double lshi, double* out, hipStream_t st) {
  PH_REQUIRE(d >= 1 && ldy >= 2 * d + 1, "sample_actions_cont: d=%zu ldy=%zu", d, ldy);
  if (N == 0) return PH_OK;
  if (dtype == PH_F64)
    k_sample_cont<double><<<ceil_div(N, 256), 256, 0, st>>>((const double*)Y, (long)ldy, (long)N, (int)d, rng, lslo,
                                                            lshi, out);
  else
    k_sample_cont<float><<<ceil_div(N, 256), 256, 0, st>>>((const float*)Y, (long)ldy, (long)N, (int)d, rng,
                                                           (float)lslo, (float)lshi, out);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_ppo_grad_md(const float* logits, size_t ldl, const int* act, const float* adv, const float* ret,
                              const float* old, const float* ov, size_t N, const int* head_sizes, size_t K,
                              float vfCoef, float entCoef, float clipEps, float vfClip, float* dlogits, size_t ldd,
                              float* newlp, float* newval, double* losses, void* stream) {
  PH_REQUIRE(N <= 0x7fffffffUL, "ph_ppo_grad_md: N=%zu", N);
  if (N > 0)
    PH_REQUIRE(logits && act && adv && ret && old && dlogits, "ph_ppo_grad_md: null buffer");
  return ppo_grad_md(logits, ldl, act, adv, ret, old, ov, N, head_sizes, K, vfCoef, entCoef, clipEps, vfClip, dlogits,
                     ldd, newlp, newval, losses, (hipStream_t)stream);
}

extern "C" int ph_ppo_grad_cont(const float* out, size_t ldo, const float* act, const float* adv, const float* ret,
                                const float* old, const float* ov, size_t N, size_t d, float vfCoef, float entCoef,
                                float clipEps, float vfClip, float ls_lo, float ls_hi, float* dout, size_t ldd,
                                float* newlp, float* newval, double* losses, void* stream) {
  PH_REQUIRE(N <= 0x7fffffffUL && ls_lo < ls_hi, "ph_ppo_grad_cont: N=%zu log-std range [%g, %g]", N, ls_lo, ls_hi);
  if (N > 0)
    PH_REQUIRE(out && act && adv && ret && old && dout, "ph_ppo_grad_cont: null buffer");
  return ppo_grad_cont(out, ldo, act, adv, ret, old, ov, N, d, vfCoef, entCoef, clipEps, vfClip, ls_lo, ls_hi, dout,
                       ldd, newlp, newval, losses, (hipStream_t)stream);
}

extern "C" int ph_sample_actions_md(int dtype, const void* Y, size_t ldy, size_t N, const int* head_sizes, size_t K,
                                    uint64_t rng, double* out, void* stream) {
  PH_REQUIRE(dtype == PH_F32 || dtype == PH_F64, "ph_sample_actions_md: dtype must be PH_F32 or PH_F64");
  PH_REQUIRE(N <= 0x7fffffffUL, "ph_sample_actions_md: N=%zu", N);
  if (N > 0) PH_REQUIRE(Y && out, "ph_sample_actions_md: null buffer");
  return sample_actions_md(dtype, Y, ldy, N, head_sizes, K, rng, out, (hipStream_t)stream);
}

extern "C" int ph_sample_actions_cont(int dtype, const void* Y, size_t ldy, size_t N, size_t d, uint64_t rng,
                                      double ls_lo, double ls_hi, double* out, void* stream) {
  PH_REQUIRE(dtype == PH_F32 || dtype == PH_F64, "ph_sample_actions_cont: dtype must be PH_F32 or PH_F64");
  PH_REQUIRE(N <= 0x7fffffffUL && ls_lo < ls_hi, "ph_sample_actions_cont: N=%zu", N);
  if (N > 0) PH_REQUIRE(Y && out, "ph_sample_actions_cont: null buffer");
  return sample_actions_cont(dtype, Y, ldy, N, d, rng, ls_lo, ls_hi, out, (hipStream_t)stream);
}
