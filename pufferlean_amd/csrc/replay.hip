// Prioritised replay on the device: the step between V-trace and the MinGRU BPTT.
//
//   ph_seg_l1       sum_t |adv(e,t)| per segment                         (k_adv_l1, puffercuda.cu:311-312)
//   ph_prio_sample  prioritised segment draws + importance weights       (puffercuda.cu:400-470; CPU twin
//                                                                          pufferffi.c:1094-1125)
//   ph_mb_gather    minibatch columns, timestep-major, adv normalised    (puffercuda.cu:472-502; CPU twin
//                                                                          pufferffi.c:1126-1200)
//   ph_mb_iterate   value/ratio of the sampled segments from the BPTT    (puffercuda.cu:503-511)
//
// Design: the reference chains seven launches for the sampler (weights, a one-block sum, a 64-chunk
// single-thread scan, its combine and add, the draws). Here the sampler is one 1024-thread workgroup
// launch: segment weights, a fixed-tree sum, a chunked scan with a fixed-tree carry and the draws all
// run in one kernel, with the cumulative table in LDS when it fits. The gather is one pass that also
// produces per-block (count, mean, M2) partials; the last block merges them in block order (Chan et
// al.'s pairwise update), so mean and std cost no extra pass over the columns, and a second small
// kernel applies the normalisation. The iterate is two launches (last-writer table, then one
// wavefront per sampled row over its T steps); the table is left zeroed by the second launch, so it
// never needs clearing.
//
// Every reduction here has a fixed order, so results are reproducible run to run. They are not
// bit-identical to the CPU twins, whose sums are sequential: mean, std, the probability normaliser
// and the cumulative table agree to rounding, and device exp/log agree with the host's to an ulp. A
// draw whose uniform lies within that rounding of a cumulative boundary can therefore pick the
// neighbouring segment; the reference's own device sampler has the same property.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

// The formulas below execute in the order written (no fused multiply-add), as in the CPU twins.
#pragma clang fp contract(off)

namespace ph {
namespace {

constexpr int kPsThreads = 1024;
constexpr long kPsLdsCum = 6144;  // cumulative table held in LDS up to this many segments (48 KiB)
constexpr int kGaThreads = 256;
constexpr int kGaPer = 4;         // minibatch elements per gather thread (256 blocks at 4096 x 64)
constexpr int kGaBlock = kGaThreads * kGaPer;

// ---- per-segment |adv| sums ------------------------------------------------------------------------
// One thread per segment, t ascending, f64 accumulation (the reference's order). Time-major columns
// give coalesced loads across the segment threads.
template <typename R, bool TM>
__global__ void __launch_bounds__(256) k_seg_l1(const R* __restrict__ adv, long N, int T,
                                                double* __restrict__ L1) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N) return;
  double s = 0.0;
  if constexpr (TM) {
#pragma unroll 8
    for (int t = 0; t < T; t++) s += fabs((double)adv[(long)t * N + e]);
  } else {
    const R* a = adv + e * T;
#pragma unroll 8
    for (int t = 0; t < T; t++) s += fabs((double)a[t]);
  }
  L1[e] = s;
}

// ---- prioritised sampler ---------------------------------------------------------------------------
// One workgroup. Thread i owns the contiguous segment chunk [i*R, min(N, (i+1)*R)).
//   w[e]   = exp(alpha * log(L1[e] + 1e-12))
//   p[e]   = (w[e] + 1e-6) / (sum w + 1e-6)            (sum: per-chunk sequential, then a fixed tree)
//   cum[e] = chunk-local running sum of p + the sum of the earlier chunks (fixed-tree scan)
//   draw i: z = splitmix64 finaliser of rng + (i+1)*GOLD; u = (z >> 11) / 2^53 * total;
//           idx = first e with cum[e] >= u (N-1 if none); mp[i] = exp(-beta * log(N * p[idx] + 1e-12))
// prob holds w, then p; cumg is the cumulative table when N exceeds the LDS copy.
__global__ void __launch_bounds__(kPsThreads) k_prio_sample(const double* __restrict__ L1, long N, long B,
                                                            double alpha, double beta,
                                                            unsigned long long rng, double* prob,
                                                            double* cumg, int* __restrict__ seg,
                                                            double* __restrict__ mp) {
  __shared__ double red[kPsThreads];
  __shared__ double cumL[kPsLdsCum];
  static_assert((kPsThreads + kPsLdsCum) * 8 <= kMaxLdsBytes, "LDS budget");
  const int tid = threadIdx.x;
  const long R = (N + kPsThreads - 1) / kPsThreads;
  const long lo = (long)tid * R < N ? (long)tid * R : N;
  const long hi = lo + R < N ? lo + R : N;
  double s = 0.0;
  for (long e = lo; e < hi; e++) {
    const double w = exp(alpha * log(L1[e] + 1e-12));
    prob[e] = w;
    s += w;
  }
  red[tid] = s;
  __syncthreads();
  for (int st = kPsThreads / 2; st > 0; st >>= 1) {
    if (tid < st) red[tid] += red[tid + st];
    __syncthreads();
  }
  const double denom = red[0] + 1e-6;
  __syncthreads();
  double* cum = N <= kPsLdsCum ? cumL : cumg;
  double c = 0.0;
  for (long e = lo; e < hi; e++) {
    const double p = (prob[e] + 1e-6) / denom;
    prob[e] = p;
    c += p;
    cum[e] = c;
  }
  // inclusive scan of the chunk totals (Hillis-Steele, fixed order)
  red[tid] = c;
  __syncthreads();
  for (int off = 1; off < kPsThreads; off <<= 1) {
    const double v = tid >= off ? red[tid - off] : 0.0;
    __syncthreads();
    if (tid >= off) red[tid] += v;
    __syncthreads();
  }
  const double carry = tid > 0 ? red[tid - 1] : 0.0;
  const double total = red[kPsThreads - 1];
  if (tid > 0)
    for (long e = lo; e < hi; e++) cum[e] += carry;
  __syncthreads();
  for (long i = tid; i < B; i += kPsThreads) {
    unsigned long long z = rng + (unsigned long long)(i + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z = z ^ (z >> 31);
    const double u = (double)(z >> 11) / 9007199254740992.0 * total;
    long L = 0, Rb = N;
    while (L < Rb) {
      const long mid = (L + Rb) >> 1;
      if (cum[mid] >= u) Rb = mid;
      else L = mid + 1;
    }
    const long idx = L < N ? L : N - 1;
    seg[i] = (int)idx;
    mp[i] = exp((-beta) * log((double)N * prob[idx] + 1e-12));
  }
}

// ---- minibatch gather ------------------------------------------------------------------------------
// Chan et al.'s pairwise merge of (count, mean, M2) summaries.
__device__ inline void chan_merge(double& n, double& m, double& M2, double nb, double mb, double M2b) {
  if (nb == 0.0) return;
  if (n == 0.0) {
    n = nb; m = mb; M2 = M2b;
    return;
  }
  const double nn = n + nb, d = mb - m;
  m = m + d * (nb / nn);
  M2 = M2 + M2b + d * d * (n * nb / nn);
  n = nn;
}

// Output element j = t*B + bi (timestep-major) reads source row e = seg[bi] at step t:
//   act (K wide, truncated to an integer) | adv (raw here) | ret = adv + value | old = logp |
//   term = term > 0.5 ? 1 : 0 | ov = value
// An index outside [0, N) yields NaN columns for that row (the sampler never produces one).
// Each block also reduces its raw adv values to (count, mean, M2) in part; k_mb_stats merges the
// blocks in index order into stats = [mean, std] (population std).
template <typename R, bool TM>
__global__ void __launch_bounds__(kGaThreads) k_mb_gather(
    const R* __restrict__ adv, const R* __restrict__ value, const R* __restrict__ act,
    const R* __restrict__ logp, const R* __restrict__ term, long N, int T, int K,
    const int* __restrict__ seg, long B, R* __restrict__ out, double* __restrict__ part) {
  __shared__ double sh[3][kGaThreads];
  const long n = B * T;
  const int tid = threadIdx.x;
  R* oact = out;
  R* oadv = out + (long)K * n;
  R* oret = oadv + n;
  R* oold = oret + n;
  R* oterm = oold + n;
  R* oov = oterm + n;
  const R qnan = (R)__builtin_nan("");
  // Workgroups are dispatched round-robin over the 8 XCDs; XCD x takes the contiguous run of
  // logical blocks [start_x, start_x + count_x), i.e. a contiguous range of steps t, so its L2 holds
  // about an eighth of the source rows instead of all of them.
  const unsigned q8 = gridDim.x / 8, r8 = gridDim.x % 8, x8 = blockIdx.x % 8;
  const unsigned lb = x8 * q8 + (x8 < r8 ? x8 : r8) + blockIdx.x / 8;
  double av[kGaPer];
  int cnt = 0;
  double s = 0.0;
#pragma unroll
  for (int k = 0; k < kGaPer; k++) {
    const long j = (long)lb * kGaBlock + (long)k * kGaThreads + tid;
    av[k] = 0.0;
    if (j < n) {
      const long t = j / B, bi = j - t * B;
      const long e = seg[bi];
      if (e >= 0 && e < N) {
        const long si = TM ? t * N + e : e * T + t;
        const R a = adv[si], v = value[si];
        for (int h = 0; h < K; h++) oact[j * K + h] = (R)trunc((double)act[si * K + h]);
        oadv[j] = a;
        oret[j] = a + v;
        oold[j] = logp[si];
        oterm[j] = term[si] > (R)0.5 ? (R)1 : (R)0;
        oov[j] = v;
        av[k] = (double)a;
        s += av[k];
      } else {
        for (int h = 0; h < K; h++) oact[j * K + h] = qnan;
        oadv[j] = qnan; oret[j] = qnan; oold[j] = qnan; oterm[j] = qnan; oov[j] = qnan;
        av[k] = (double)qnan;
        s += av[k];
      }
      cnt++;
    }
  }
  // block (count, mean, M2): fixed-tree sums
  sh[0][tid] = s;
  sh[1][tid] = (double)cnt;
  __syncthreads();
  for (int st = kGaThreads / 2; st > 0; st >>= 1) {
    if (tid < st) {
      sh[0][tid] += sh[0][tid + st];
      sh[1][tid] += sh[1][tid + st];
    }
    __syncthreads();
  }
  const double bn = sh[1][0];
  const double bm = bn > 0.0 ? sh[0][0] / bn : 0.0;
  __syncthreads();
  double q = 0.0;
#pragma unroll
  for (int k = 0; k < kGaPer; k++)
    if (k < cnt) {
      const double d = av[k] - bm;
      q += d * d;
    }
  sh[2][tid] = q;
  __syncthreads();
  for (int st = kGaThreads / 2; st > 0; st >>= 1) {
    if (tid < st) sh[2][tid] += sh[2][tid + st];
    __syncthreads();
  }
  if (tid == 0) {
    part[3 * lb] = bn;
    part[3 * lb + 1] = bm;
    part[3 * lb + 2] = sh[2][0];
  }
}

// One block: thread i folds the gather blocks i, i+256, ... in order, then a fixed tree over the
// threads; stats = [mean, std]. Launched after the gather, whose partials the launch boundary orders.
__global__ void __launch_bounds__(kGaThreads) k_mb_stats(const double* __restrict__ part, unsigned G,
                                                         double* __restrict__ stats) {
  __shared__ double sh[3][kGaThreads];
  const int tid = threadIdx.x;
  double mn = 0.0, mm = 0.0, mq = 0.0;
  for (unsigned b = tid; b < G; b += kGaThreads) chan_merge(mn, mm, mq, part[3 * b], part[3 * b + 1], part[3 * b + 2]);
  sh[0][tid] = mn;
  sh[1][tid] = mm;
  sh[2][tid] = mq;
  __syncthreads();
  for (int st = kGaThreads / 2; st > 0; st >>= 1) {
    if (tid < st) {
      double a0 = sh[0][tid], a1 = sh[1][tid], a2 = sh[2][tid];
      chan_merge(a0, a1, a2, sh[0][tid + st], sh[1][tid + st], sh[2][tid + st]);
      sh[0][tid] = a0;
      sh[1][tid] = a1;
      sh[2][tid] = a2;
    }
    __syncthreads();
  }
  if (tid == 0) {
    const double nt = sh[0][0] > 0.0 ? sh[0][0] : 1.0;
    stats[0] = sh[1][0];
    stats[1] = sqrt(sh[2][0] / nt);
  }
}

// adv[j] = mp[bi] * (adv[j] - mean) / (std + 1e-8), j = t*B + bi (mp NULL: weight 1).
template <typename R>
__global__ void __launch_bounds__(256) k_mb_normalize(R* __restrict__ adv, long B, long n,
                                                      const double* __restrict__ mp,
                                                      const double* __restrict__ stats) {
  const long j = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n) return;
  const long bi = j % B;
  const double w = mp ? mp[bi] : 1.0;
  adv[j] = (R)(w * ((double)adv[j] - stats[0]) / (stats[1] + 1e-8));
}

// ---- value / ratio iterate -------------------------------------------------------------------------
// Pass 1: lw[e] = max over the draws bi of segment e of (bi + 1). The table is all zero between
// calls: pass 2 clears every entry pass 1 set.
__global__ void __launch_bounds__(256) k_mb_lastw(const int* __restrict__ seg, long B, long N, int* lw) {
  const long bi = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (bi >= B) return;
  const int e = seg[bi];
  if (e >= 0 && e < N) atomicMax(&lw[e], (int)(bi + 1));
}

// Pass 2: one wavefront per draw bi, lanes over t. Only the last draw of a segment (the writer an
// in-order loop over bi leaves in place) stores ratio = exp(newlp - logp) and value = newval, then
// clears the table entry. A draw that reads the entry after the clear sees 0, which matches no draw.
template <typename R, bool TM>
__global__ void __launch_bounds__(256) k_mb_iterate(R* __restrict__ value, R* __restrict__ ratio,
                                                    const R* __restrict__ logp,
                                                    const float* __restrict__ newlp,
                                                    const float* __restrict__ newval,
                                                    const int* __restrict__ seg, long B, long N, int T,
                                                    int* lw) {
  const long bi = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (bi >= B) return;
  const int e = seg[bi];
  if (e < 0 || e >= N) return;
  if (lw[e] != (int)(bi + 1)) return;
  for (int t = lane; t < T; t += 64) {
    const long si = TM ? (long)t * N + e : (long)e * T + t;
    const long os = (long)t * B + bi;
    ratio[si] = (R)exp((double)newlp[os] - (double)logp[si]);
    value[si] = (R)newval[os];
  }
  if (lane == 0) lw[e] = 0;
}

int check_cols(const ph_replay_cols* c, const char* who) {
  PH_REQUIRE(c, "%s: null column descriptor", who);
  PH_REQUIRE(c->dtype == PH_F32 || c->dtype == PH_F64, "%s: dtype must be PH_F32 or PH_F64", who);
  PH_REQUIRE(c->N > 0 && c->N <= 0x7fffffffL && c->T > 0 && c->T <= 0x7fffffffL,
             "%s: N=%zu T=%zu out of range", who, c->N, c->T);
  return PH_OK;
}

}  // namespace

int seg_l1(const ph_replay_cols& c, double* L1, hipStream_t st) {
  const long N = (long)c.N;
  const int T = (int)c.T;
  const unsigned g = ceil_div(c.N, 256);
  if (c.dtype == PH_F64) {
    if (c.time_major) k_seg_l1<double, true><<<g, 256, 0, st>>>((const double*)c.adv, N, T, L1);
    else k_seg_l1<double, false><<<g, 256, 0, st>>>((const double*)c.adv, N, T, L1);
  } else {
    if (c.time_major) k_seg_l1<float, true><<<g, 256, 0, st>>>((const float*)c.adv, N, T, L1);
    else k_seg_l1<float, false><<<g, 256, 0, st>>>((const float*)c.adv, N, T, L1);
  }
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int prio_sample(const double* L1, size_t N, size_t B, double alpha, double beta, uint64_t rng, int* seg,
                double* mp, hipStream_t st) {
  PH_REQUIRE(N > 0 && N <= 0x7fffffffUL, "prio_sample: N=%zu out of range", N);
  PH_REQUIRE(B <= 0x7fffffffUL, "prio_sample: %zu draws out of range", B);
  if (B == 0) return PH_OK;
  PH_REQUIRE(L1 && seg && mp, "prio_sample: null buffer");
  const size_t tab = (N + 31) & ~(size_t)31;
  double* w = (double*)scratch(kSlotPrio, (N > (size_t)kPsLdsCum ? 2 : 1) * tab * 8);
  if (!w) return PH_ERR_NOMEM;
  k_prio_sample<<<1, kPsThreads, 0, st>>>(L1, (long)N, (long)B, alpha, beta, (unsigned long long)rng, w,
                                          w + tab, seg, mp);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int mb_gather(const ph_replay_cols& c, const int* seg, const double* mp, size_t B, void* out, double* stats,
              hipStream_t st) {
  const long n = (long)(B * c.T);
  if (n == 0) return PH_OK;
  const int K = c.K ? (int)c.K : 1;
  const unsigned nb = ceil_div((size_t)n, kGaBlock);
  double* part = (double*)scratch(kSlotReplayPart, (size_t)nb * 3 * 8 + 64);
  if (!part) return PH_ERR_NOMEM;
  if (!stats) {
    stats = (double*)scratch(kSlotReplayStats, 64);
    if (!stats) return PH_ERR_NOMEM;
  }
  const long N = (long)c.N;
  const int T = (int)c.T;
#define PH_GATHER(R, TM)                                                                                \
  do {                                                                                                  \
    k_mb_gather<R, TM><<<nb, kGaThreads, 0, st>>>((const R*)c.adv, (const R*)c.value, (const R*)c.act,  \
                                                  (const R*)c.logp, (const R*)c.term, N, T, K, seg,      \
                                                  (long)B, (R*)out, part);                               \
    k_mb_stats<<<1, kGaThreads, 0, st>>>(part, nb, stats);                                              \
  } while (0)
  if (c.dtype == PH_F64) {
    if (c.time_major) PH_GATHER(double, true);
    else PH_GATHER(double, false);
    k_mb_normalize<double><<<ceil_div((size_t)n, 256), 256, 0, st>>>((double*)out + (long)K * n, (long)B,
                                                                     n, mp, stats);
  } else {
    if (c.time_major) PH_GATHER(float, true);
    else PH_GATHER(float, false);
    k_mb_normalize<float><<<ceil_div((size_t)n, 256), 256, 0, st>>>((float*)out + (long)K * n, (long)B,
                                                                    n, mp, stats);
  }
#undef PH_GATHER
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int mb_iterate(const ph_replay_cols& c, const int* seg, size_t B, const float* newlp, const float* newval,
               hipStream_t st) {
  if (B == 0) return PH_OK;
  int* lw = (int*)scratch_zeroed(kSlotReplayLastw, c.N * 4, st);
  if (!lw) return PH_ERR_NOMEM;
  const long N = (long)c.N;
  const int T = (int)c.T;
  k_mb_lastw<<<ceil_div(B, 256), 256, 0, st>>>(seg, (long)B, N, lw);
  const unsigned g = ceil_div(B, 4);
  if (c.dtype == PH_F64) {
    if (c.time_major)
      k_mb_iterate<double, true><<<g, 256, 0, st>>>((double*)c.value, (double*)c.ratio, (const double*)c.logp,
                                                     newlp, newval, seg, (long)B, N, T, lw);
    else
      k_mb_iterate<double, false><<<g, 256, 0, st>>>((double*)c.value, (double*)c.ratio,
                                                      (const double*)c.logp, newlp, newval, seg, (long)B, N,
                                                      T, lw);
  } else {
    if (c.time_major)
      k_mb_iterate<float, true><<<g, 256, 0, st>>>((float*)c.value, (float*)c.ratio, (const float*)c.logp,
                                                    newlp, newval, seg, (long)B, N, T, lw);
    else
      k_mb_iterate<float, false><<<g, 256, 0, st>>>((float*)c.value, (float*)c.ratio, (const float*)c.logp,
                                                     newlp, newval, seg, (long)B, N, T, lw);
  }
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_seg_l1(const ph_replay_cols* c, double* L1, void* stream) {
  PH_TRY(check_cols(c, "ph_seg_l1"));
  PH_REQUIRE(c->adv && L1, "ph_seg_l1: null buffer");
  return seg_l1(*c, L1, (hipStream_t)stream);
}

extern "C" int ph_prio_sample(const double* L1, size_t N, size_t Bmb, double alpha, double beta, uint64_t rng,
                              int* seg, double* mbprio, void* stream) {
  return prio_sample(L1, N, Bmb, alpha, beta, rng, seg, mbprio, (hipStream_t)stream);
}

extern "C" int ph_mb_gather(const ph_replay_cols* c, const int* seg, const double* mbprio, size_t Bmb, void* out,
                            double* stats, void* stream) {
  PH_TRY(check_cols(c, "ph_mb_gather"));
  PH_REQUIRE(c->K <= 256, "ph_mb_gather: K=%zu action components", c->K);
  PH_REQUIRE(Bmb <= 0x7fffffffUL && Bmb * c->T <= ((size_t)1 << 40), "ph_mb_gather: Bmb=%zu too large", Bmb);
  if (Bmb == 0) return PH_OK;
  PH_REQUIRE(c->adv && c->value && c->act && c->logp && c->term && seg && out,
             "ph_mb_gather: null buffer");
  return mb_gather(*c, seg, mbprio, Bmb, out, stats, (hipStream_t)stream);
}

extern "C" int ph_mb_iterate(const ph_replay_cols* c, const int* seg, size_t Bmb, const float* newlp,
                             const float* newval, void* stream) {
  PH_TRY(check_cols(c, "ph_mb_iterate"));
  PH_REQUIRE(Bmb <= 0x7fffffffUL, "ph_mb_iterate: Bmb=%zu too large", Bmb);
  if (Bmb == 0) return PH_OK;
  PH_REQUIRE(c->value && c->ratio && c->logp && seg && newlp && newval, "ph_mb_iterate: null buffer");
  return mb_iterate(*c, seg, Bmb, newlp, newval, (hipStream_t)stream);
}
