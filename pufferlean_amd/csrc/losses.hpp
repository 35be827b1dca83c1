// The 7 dashboard losses of the PPO objective, [pg, v, ent, total, old_kl, kl, clipfrac] as means over
// the rows (PufferLib's decomposition, puffercuda.cu:1798-1870 for every head kind), reduced
// deterministically: six f64 sums per row, a fixed tree per block, per-block partials, and the last
// block to finish folding the partials in block order.
#pragma once
#include <hip/hip_runtime.h>

namespace ph {

// Per-row sums {pg, v, ent, old_kl, kl, nclip} from the row's new log-prob, behaviour log-prob,
// advantage, new value, return and entropy. clipV applies PufferLib's clipped value loss against vold.
__device__ inline void row_losses(float logp, float old, float adv, float vnew, float ret, float vold, bool clipV,
                                  float vfClip, float clipEps, float ent, double lsum[6]) {
  const double lr = (double)logp - (double)old;
  const double r = exp(lr);
  const double dlo = 1.0 - (double)clipEps, dhi = 1.0 + (double)clipEps;
  const double rcd = r < dlo ? dlo : (r > dhi ? dhi : r);
  const double p1 = -(double)adv * r, p2 = -(double)adv * rcd;
  lsum[0] = p1 > p2 ? p1 : p2;
  const double rv = (double)ret;
  const double du = ((double)vnew - rv) * ((double)vnew - rv);
  double vl = du;
  if (clipV) {
    const double dd = (double)vnew - (double)vold;
    const double c = (double)vfClip;
    const double vc = (double)vold + (dd < -c ? -c : (dd > c ? c : dd));
    const double cc = (vc - rv) * (vc - rv);
    if (cc > du) vl = cc;
  }
  lsum[1] = 0.5 * vl;
  lsum[2] = (double)ent;
  lsum[3] = -lr;
  lsum[4] = (r - 1.0) - lr;
  lsum[5] = (r < dlo || r > dhi) ? 1.0 : 0.0;
}

// Every thread of a 256-thread block calls this once with its row's sums (zeros for rows past N).
// part holds 6 doubles per block; counter starts at 0 and is left at 0.
__device__ inline void fold_losses(const double lsum[6], double* __restrict__ part, unsigned* counter,
                                   double* __restrict__ losses, long N, float vfCoef, float entCoef) {
  __shared__ double sh[6][256];
  __shared__ bool last;
#pragma unroll
  for (int q = 0; q < 6; q++) sh[q][threadIdx.x] = lsum[q];
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s)
#pragma unroll
      for (int q = 0; q < 6; q++) sh[q][threadIdx.x] += sh[q][threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
#pragma unroll
    for (int q = 0; q < 6; q++) part[(size_t)blockIdx.x * 6 + q] = sh[q][0];
    __threadfence();
    last = atomicAdd(counter, 1u) == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  // thread t adds blocks t, t+256, ... in sequence; the same tree then combines the 256 thread sums
#pragma unroll
  for (int q = 0; q < 6; q++) {
    double s = 0.0;
    for (unsigned b = threadIdx.x; b < gridDim.x; b += blockDim.x)
      s += __hip_atomic_load(&part[(size_t)b * 6 + q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh[q][threadIdx.x] = s;
  }
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s)
#pragma unroll
      for (int q = 0; q < 6; q++) sh[q][threadIdx.x] += sh[q][threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double dn = (double)(N > 0 ? N : 1);
    const double pg = sh[0][0] / dn, vl = sh[1][0] / dn, en = sh[2][0] / dn;
    losses[0] = pg;
    losses[1] = vl;
    losses[2] = en;
    losses[3] = pg + (double)vfCoef * vl - (double)entCoef * en;
    losses[4] = sh[3][0] / dn;
    losses[5] = sh[4][0] / dn;
    losses[6] = sh[5][0] / dn;
    *counter = 0u;
  }
}

}  // namespace ph
