// The 7 dashboard losses of the PPO objective, [pg, v, ent, total, old_kl, kl, clipfrac] as means over
// the rows (PufferLib's decomposition, puffercuda.cu:1798-1870 for every head kind), reduced
// deterministically: six f64 sums per row, fixed-order wavefront butterflies per block, per-block
// partials, and a one-block kernel folding the partials in block order.
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

// Sum over the 64 lanes of a wavefront by an xor butterfly: each step adds the partner's partial, so
// both partners hold the same value and, after six steps, every lane holds the same total, formed in
// the same order on every run.
__device__ inline double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Every thread of a 256-thread block calls this once with its row's sums (zeros for rows past N):
// the block's six sums go to part[6 * blockIdx.x ..]. k_fold_losses, launched after the kernel on
// the same stream, folds the blocks. (A last-block fold inside the kernel needs a device-scope
// release per block, which on this part writes back the XCD's L2 mid-kernel; the launch boundary
// orders the partials at no such cost.)
__device__ inline void block_losses(const double lsum[6], double* __restrict__ part) {
  __shared__ double sh[6][4];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  double v[6];
#pragma unroll
  for (int q = 0; q < 6; q++) v[q] = wave_sum(lsum[q]);
  if (lane == 0)
#pragma unroll
    for (int q = 0; q < 6; q++) sh[q][w] = v[q];
  __syncthreads();
  if (threadIdx.x < 6) {
    const int q = threadIdx.x;
    part[(size_t)blockIdx.x * 6 + q] = ((sh[q][0] + sh[q][1]) + sh[q][2]) + sh[q][3];
  }
}

// One 256-thread block: thread t adds blocks t, t + 256, ... in sequence, the wavefront butterflies
// and the wavefront order combine them, and the means over N rows form the 7 losses. (Internal
// linkage: each source file that launches it has its own copy.)
static __global__ void __launch_bounds__(256) k_fold_losses(const double* __restrict__ part, int G, long N, float vfCoef,
                                                     float entCoef, double* __restrict__ losses) {
  __shared__ double sh[6][4];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // each sum runs over blocks t, t + 256, ... in order; four blocks' loads are in flight at a time
  double acc[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  const int bd = blockDim.x;
  int b = threadIdx.x;
  for (; b + 3 * bd < G; b += 4 * bd) {
    double pv[4][6];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int q = 0; q < 6; q++) pv[k][q] = part[(size_t)(b + k * bd) * 6 + q];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int q = 0; q < 6; q++) acc[q] += pv[k][q];
  }
  for (; b < G; b += bd)
#pragma unroll
    for (int q = 0; q < 6; q++) acc[q] += part[(size_t)b * 6 + q];
  double v[6];
#pragma unroll
  for (int q = 0; q < 6; q++) v[q] = wave_sum(acc[q]);
  if (lane == 0)
#pragma unroll
    for (int q = 0; q < 6; q++) sh[q][w] = v[q];
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot[6];
#pragma unroll
    for (int q = 0; q < 6; q++) tot[q] = ((sh[q][0] + sh[q][1]) + sh[q][2]) + sh[q][3];
    const double dn = (double)(N > 0 ? N : 1);
    const double pg = tot[0] / dn, vl = tot[1] / dn, en = tot[2] / dn;
    losses[0] = pg;
    losses[1] = vl;
    losses[2] = en;
    losses[3] = pg + (double)vfCoef * vl - (double)entCoef * en;
    losses[4] = tot[3] / dn;
    losses[5] = tot[4] / dn;
    losses[6] = tot[5] / dn;
  }
}

}  // namespace ph
