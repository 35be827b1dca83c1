// Muon optimizer step: Nesterov momentum -> Newton-Schulz orthogonalisation -> decoupled weight
// decay (ascent form), plus the bias step and the global grad-norm clip.
//
// Two tiers:
//  * exact (f64): naive matmuls that sum over the shared index in ascending order, the two-level
//    Frobenius fold (rows in parallel, then rows summed in order by one lane) and contraction
//    disabled, so every value matches the reference CPU step (pufferblas.c:1369-1406) bit for bit.
//  * fast, bf16 MFMA: the whole batch's quintic in one fused launch (ns.hip).
//  * fast, fp32 MFMA: the quintic iterate as a chain of GEMMs (fp32 state), wide form
//    X <- aX + (bA + cA^2)X with A = XX^T; A and A^2 are symmetric, so A^2 = A A^T is computed by
//    the same NT kernel as XX^T, and the b/c/a combinations are fused into the GEMM epilogues.
//    Tall matrices are transposed to wide on the way in and back on the way out.
#include "common.hpp"
#include "kernels.hpp"

namespace ph {
namespace {

// ---- exact tier ---------------------------------------------------------------------------------
__global__ void k_nesterov_f64(const double* __restrict__ G, const double* __restrict__ M,
                               double* __restrict__ nM, double* __restrict__ U, long n, double gscale,
                               double mu) {
#pragma clang fp contract(off)
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double gi = G[i] * gscale;
  const double m = mu * M[i] + gi;
  nM[i] = m;
  U[i] = gi + mu * m;
}

// per-row sum of squares, ascending column order
__global__ void k_rowsq_f64(const double* __restrict__ U, double* __restrict__ rs, int rows, int cols) {
#pragma clang fp contract(off)
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const double* u = U + (long)r * cols;
  double s = 0.0;
  for (int j = 0; j < cols; j++) {
    const double v = u[j];
    s = s + v * v;
  }
  rs[r] = s;
}

// rows summed in order by one lane; inv = 1/(sqrt(s)+eps)
__global__ void k_frob_inv_f64(const double* __restrict__ rs, int rows, double eps, double* __restrict__ inv) {
#pragma clang fp contract(off)
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  double s = 0.0;
  for (int r = 0; r < rows; r++) s = s + rs[r];
  inv[0] = 1.0 / (sqrt(s) + eps);
}

__global__ void k_scale_f64(const double* __restrict__ U, const double* __restrict__ inv,
                            double* __restrict__ X, long n) {
#pragma clang fp contract(off)
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) X[i] = inv[0] * U[i];
}

__global__ void k_transpose_f64(const double* __restrict__ X, double* __restrict__ Xt, int rows, int cols) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * cols) return;
  int i = (int)(idx / cols), j = (int)(idx % cols);
  Xt[(long)j * rows + i] = X[idx];
}

// C[m x n] = A[m x k] B[k x n], one lane per output, ascending l, no contraction
__global__ void k_matmul_f64(const double* __restrict__ A, const double* __restrict__ B,
                             double* __restrict__ C, int m, int k, int n) {
#pragma clang fp contract(off)
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)m * n) return;
  int i = (int)(idx / n), j = (int)(idx % n);
  double t = 0.0;
  for (int l = 0; l < k; l++) t = t + A[(long)i * k + l] * B[(long)l * n + j];
  C[idx] = t;
}

__global__ void k_lincomb3_f64(double* __restrict__ X, double a, const double* __restrict__ P, double b,
                               const double* __restrict__ Q, double c, long n) {
#pragma clang fp contract(off)
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) X[i] = a * X[i] + b * P[i] + c * Q[i];
}

__global__ void k_finalize_f64(const double* __restrict__ W, const double* __restrict__ X,
                               double* __restrict__ nW, double c1, double c2, long n) {
#pragma clang fp contract(off)
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) nW[i] = c1 * W[i] + c2 * X[i];
}

__global__ void k_stepvec_f64(const double* __restrict__ b, const double* __restrict__ g,
                              const double* __restrict__ m, double* __restrict__ nb,
                              double* __restrict__ nm, long n, double gscale, double lr, double wd,
                              double mu) {
#pragma clang fp contract(off)
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double gi = g[i] * gscale;
  const double newm = mu * m[i] + gi;
  const double upd = gi + mu * newm;
  nb[i] = b[i] * (1.0 - lr * wd) + lr * upd;
  nm[i] = newm;
}

// ---- fast tier helpers --------------------------------------------------------------------------
// sum of squares of an fp32 matrix into part[blockIdx.x] (fixed chunks), then a one-block fold
__global__ void __launch_bounds__(256) k_sumsq_part(const float* __restrict__ x, long n, long chunk,
                                                    float* __restrict__ part) {
  __shared__ float sh[256];
  const long lo = (long)blockIdx.x * chunk, hi = lo + chunk < n ? lo + chunk : n;
  // eight loads in flight at a time, added in index order
  float s = 0.f;
  long i = lo + threadIdx.x;
  for (; i + 7 * 256 < hi; i += 8 * 256) {
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = x[i + q * 256];
#pragma unroll
    for (int q = 0; q < 8; q++) s += v[q] * v[q];
  }
  for (; i < hi; i += 256) s += x[i] * x[i];
  sh[threadIdx.x] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) sh[threadIdx.x] += sh[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = sh[0];
}

__global__ void k_norm_inv(const float* __restrict__ part, int G, float eps, float* __restrict__ inv) {
  __shared__ float sh[256];
  float s = 0.f;
  for (int i = threadIdx.x; i < G; i += 256) s += part[i];
  sh[threadIdx.x] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st) sh[threadIdx.x] += sh[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) inv[0] = 1.f / (sqrtf(sh[0]) + eps);
}

// Load the normalised iterate in wide form: Xf (fp32, m x w), Xb (bf16, m x w), Xt (bf16, w x m).
// src is rows x cols; tall (rows > cols) sources are transposed.
__global__ void k_ns_load(const float* __restrict__ src, int rows, int cols, const float* __restrict__ inv,
                          float* __restrict__ Xf, uint16_t* __restrict__ Xb, uint16_t* __restrict__ Xt) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * cols) return;
  const int i = (int)(idx / cols), j = (int)(idx % cols);
  const bool tall = rows > cols;
  const int m = tall ? cols : rows, w = tall ? rows : cols;
  const int wi = tall ? j : i, wj = tall ? i : j;  // wide coordinates
  const float v = inv[0] * src[idx];
  Xf[(long)wi * w + wj] = v;
  const uint16_t b = bf16_rne(v);
  Xb[(long)wi * w + wj] = b;
  Xt[(long)wj * m + wi] = b;
}

__global__ void k_ns_load_f32(const float* __restrict__ src, int rows, int cols,
                              const float* __restrict__ inv, float* __restrict__ Xf) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * cols) return;
  const int i = (int)(idx / cols), j = (int)(idx % cols);
  const bool tall = rows > cols;
  const int w = tall ? rows : cols;
  const int wi = tall ? j : i, wj = tall ? i : j;
  Xf[(long)wi * w + wj] = inv[0] * src[idx];
}

__global__ void k_ns_store(const float* __restrict__ Xf, int rows, int cols, float* __restrict__ dst) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * cols) return;
  const int i = (int)(idx / cols), j = (int)(idx % cols);
  const bool tall = rows > cols;
  const int w = tall ? rows : cols;
  const int wi = tall ? j : i, wj = tall ? i : j;
  dst[idx] = Xf[(long)wi * w + wj];
}

// Nesterov on fp32 state: nM = mu*M + g*gscale; U = g*gscale + mu*nM
__global__ void k_nesterov_f32(const float* __restrict__ G, float* __restrict__ M, float* __restrict__ U,
                               long n, float gscale, float mu) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = G[i] * gscale;
  const float m = mu * M[i] + gi;
  M[i] = m;
  U[i] = gi + mu * m;
}

__global__ void k_finalize_f32(float* __restrict__ W, const float* __restrict__ X, long n, float c1, float c2) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) W[i] = c1 * W[i] + c2 * X[i];
}

__global__ void k_stepvec_f32(float* __restrict__ b, const float* __restrict__ g, float* __restrict__ m,
                              long n, float gscale, float lr, float wd, float mu) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = g[i] * gscale;
  const float newm = mu * m[i] + gi;
  const float upd = gi + mu * newm;
  b[i] = b[i] * (1.f - lr * wd) + lr * upd;
  m[i] = newm;
}

// The same elementwise updates over up to kNsMaxMats arrays in one launch: the arrays are laid end to
// end in one index space (start[k] is the first index of array k), so the many small launches of an
// optimizer step become one. Each element gets exactly the single-array kernel's arithmetic.
struct EwBatch {
  int n;
  long start[kNsMaxMats + 1];
  float* p[kNsMaxMats];        // nesterov: G; finalize: W; stepvec: b
  float* q[kNsMaxMats];        // nesterov: M; stepvec: g
  float* r[kNsMaxMats];        // nesterov: U; finalize: X; stepvec: m
  float s[kNsMaxMats];         // finalize: the array's update scale
};
__device__ __forceinline__ int ew_array(const EwBatch& B, long i) {
  int k = 0;
  while (k + 1 < B.n && i >= B.start[k + 1]) k++;
  return k;
}
__global__ void k_nesterov_batch(EwBatch B, float gscale, float mu) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B.start[B.n]) return;
  const int k = ew_array(B, i);
  const long j = i - B.start[k];
  const float gi = B.p[k][j] * gscale;
  const float m = mu * B.q[k][j] + gi;
  B.q[k][j] = m;
  B.r[k][j] = gi + mu * m;
}
__global__ void k_finalize_batch(EwBatch B, float c1) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B.start[B.n]) return;
  const int k = ew_array(B, i);
  const long j = i - B.start[k];
  B.p[k][j] = c1 * B.p[k][j] + B.s[k] * B.r[k][j];
}
__global__ void k_stepvec_batch(EwBatch B, float gscale, float lr, float wd, float mu) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B.start[B.n]) return;
  const int k = ew_array(B, i);
  const long j = i - B.start[k];
  const float gi = B.q[k][j] * gscale;
  const float newm = mu * B.r[k][j] + gi;
  const float upd = gi + mu * newm;
  B.p[k][j] = B.p[k][j] * (1.f - lr * wd) + lr * upd;
  B.r[k][j] = newm;
}

// Global grad-norm clip over a flat fp32 gradient: sumsq in fixed-chunk partials, then scale.
__global__ void k_gclip_scale(float* __restrict__ g, long n, const float* __restrict__ part, int G,
                              float sc, float maxNorm) {
  // the partials are summed by one thread in order; the block first stages them in LDS so their loads
  // are one round trip instead of G dependent ones
  __shared__ float sp[1024];
  __shared__ float tot;
  float s = 0.f;
  for (int b0 = 0; b0 < G; b0 += 1024) {
    const int nb = G - b0 < 1024 ? G - b0 : 1024;
    __syncthreads();  // the previous slice has been summed
    for (int i = threadIdx.x; i < nb; i += blockDim.x) sp[i] = part[b0 + i];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int i = 0; i < nb; i++) s += sp[i];
  }
  if (threadIdx.x == 0) tot = s;
  __syncthreads();
  const float gn = sqrtf(tot) * fabsf(sc);
  const float cc = ((maxNorm > 0.f && gn > maxNorm) ? maxNorm / gn : 1.f) * sc;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    g[i] = g[i] * cc;
}

constexpr unsigned kB = 256;

// The whole exact-tier step of one small matrix in one workgroup: X, P and the Gram matrix A live in
// LDS (2 n + min(rows, cols)^2 doubles), so the Newton-Schulz steps need no launches between them.
// Every value is computed with the chain's operations in the chain's order (ascending sums, no
// contraction), so the result is bit-identical to the multi-launch form. The Q = A P (or P A)
// product is consumed where it is made: the thread computing Q(i, j) updates X(i, j) in place, as
// that phase reads only A and P (X is then read by no other thread of the phase). W/nW and M/nM may alias (each element is read and written by one
// thread).
// Four running sums s[2r + c] = s[2r + c] + u_r(l) * v_c(l) for l ascending, with
// u_r(l) = U[ur + l * us] and v_c(l) = V[vc + l * vs]. Loads are issued four steps at a time, so a step
// waits on LDS once per four; each sum still adds its products one at a time in ascending l.
__device__ __forceinline__ void dot2x2(const double* U, int u0, int u1, int us, const double* V, int v0, int v1,
                                       int vs, int L, double s[4]) {
#pragma clang fp contract(off)
  int l = 0;
  for (; l + 4 <= L; l += 4) {
    double a0[4], a1[4], b0[4], b1[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      a0[k] = U[u0 + (l + k) * us];
      a1[k] = U[u1 + (l + k) * us];
      b0[k] = V[v0 + (l + k) * vs];
      b1[k] = V[v1 + (l + k) * vs];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      s[0] = s[0] + a0[k] * b0[k];
      s[1] = s[1] + a0[k] * b1[k];
      s[2] = s[2] + a1[k] * b0[k];
      s[3] = s[3] + a1[k] * b1[k];
    }
  }
  for (; l < L; l++) {
    const double a0 = U[u0 + l * us], a1 = U[u1 + l * us], b0 = V[v0 + l * vs], b1 = V[v1 + l * vs];
    s[0] = s[0] + a0 * b0;
    s[1] = s[1] + a0 * b1;
    s[2] = s[2] + a1 * b0;
    s[3] = s[3] + a1 * b1;
  }
}

constexpr int kExactFusedMaxSteps = 8;
constexpr long kExactFusedLds = 8192;  // doubles: 64 KB
static_assert(kExactFusedLds * 8 + 64 <= kMaxLdsBytes, "LDS budget of the fused exact Muon");
struct ExactCoeffs {
  double v[3 * kExactFusedMaxSteps];
};

struct ExactBatch {
  ExactMat m[kExactBatchMax];
  ExactVec v[kExactBatchMax];
  int nm;
};

// One workgroup per matrix of the batch (they are independent, so they run side by side), then one
// per bias vector, which takes the f64 bias step (k_stepvec_f64's arithmetic) in place.
__global__ void __launch_bounds__(1024) k_muon_exact_fused(ExactBatch bt, double gscale, double lr, double mu,
                                                           double eps, ExactCoeffs cf, int nsteps, double c1) {
#pragma clang fp contract(off)
  if ((int)blockIdx.x >= bt.nm) {  // uniform per workgroup: the matrix path's barriers are not reached
    const ExactVec& vt = bt.v[blockIdx.x - bt.nm];
    for (long i = threadIdx.x; i < vt.n; i += blockDim.x) {
      const double gi = vt.g[i] * gscale;
      const double newm = mu * vt.m[i] + gi;
      const double upd = gi + mu * newm;
      vt.b[i] = vt.b[i] * c1 + lr * upd;
      vt.m[i] = newm;
    }
    return;
  }
  const ExactMat& mt = bt.m[blockIdx.x];
  const double* W = mt.W;
  const double* G = mt.G;
  const double* M = mt.M;
  double* nW = mt.nW;
  double* nM = mt.nM;
  const int rows = mt.rows, cols = mt.cols;
  const double c2 = mt.c2;
  extern __shared__ double lds[];
  const int n = rows * cols, T = blockDim.x, tid = threadIdx.x;
  const bool wide = rows <= cols;
  const int mn = wide ? rows : cols;
  double* X = lds;
  double* P = lds + n;
  double* A = lds + 2 * n;
  __shared__ double inv;
  // Nesterov: U (kept in X) and the new momentum
  for (int i = tid; i < n; i += T) {
    const double gi = G[i] * gscale;
    const double m = mu * M[i] + gi;
    nM[i] = m;
    X[i] = gi + mu * m;
  }
  __syncthreads();
  // Frobenius norm: row sums of squares in ascending column order, then the rows in order
  for (int r = tid; r < rows; r += T) {
    double sq = 0.0;
#pragma unroll 8
    for (int j = 0; j < cols; j++) {
      const double v = X[r * cols + j];
      sq = sq + v * v;
    }
    P[r] = sq;
  }
  __syncthreads();
  if (tid == 0) {
    double sq = 0.0;
#pragma unroll 8
    for (int r = 0; r < rows; r++) sq = sq + P[r];
    inv = 1.0 / (sqrt(sq) + eps);
  }
  __syncthreads();
  for (int i = tid; i < n; i += T) X[i] = inv * X[i];
  __syncthreads();
  // 2 x 2 output tiles per thread: four independent sums, each operand load serving two outputs.
  // Every output keeps its own ascending sum. A(i, j) and A(j, i) are the same products in the same
  // order, so only tiles on or above the diagonal are formed and the other half is mirrored.
  const int tm = (mn + 1) / 2, tr = (rows + 1) / 2, tc = (cols + 1) / 2;
  for (int it = 0; it < nsteps; it++) {
    const double a = cf.v[3 * it], b = cf.v[3 * it + 1], c = cf.v[3 * it + 2];
    for (int e = tid; e < tm * tm; e += T) {  // A = X X^T (wide) or X^T X (tall)
      const int ti = e / tm, tj = e % tm;
      if (tj < ti) continue;
      const int i0 = 2 * ti, j0 = 2 * tj;
      const int i1 = i0 + 1 < mn ? i0 + 1 : i0, j1 = j0 + 1 < mn ? j0 + 1 : j0;  // clamped loads
      double sv[4] = {0.0, 0.0, 0.0, 0.0};
      if (wide)
        dot2x2(X, i0 * cols, i1 * cols, 1, X, j0 * cols, j1 * cols, 1, cols, sv);
      else
        dot2x2(X, i0, i1, cols, X, j0, j1, cols, rows, sv);
      const double s00 = sv[0], s01 = sv[1], s10 = sv[2], s11 = sv[3];
      A[i0 * mn + j0] = s00;
      A[j0 * mn + i0] = s00;
      if (j0 + 1 < mn) {
        A[i0 * mn + j0 + 1] = s01;
        A[(j0 + 1) * mn + i0] = s01;
      }
      if (i0 + 1 < mn) {
        A[(i0 + 1) * mn + j0] = s10;
        A[j0 * mn + i0 + 1] = s10;
      }
      if (i0 + 1 < mn && j0 + 1 < mn) {
        A[(i0 + 1) * mn + j0 + 1] = s11;
        A[(j0 + 1) * mn + i0 + 1] = s11;
      }
    }
    __syncthreads();
    // P = A X (wide) or X A (tall), then Q = A P (wide) or P A (tall) with X = a X + b P + c Q
    for (int pass = 0; pass < 2; pass++) {
      const double* Y = pass == 0 ? X : P;  // right (wide) or left (tall) operand
      for (int e = tid; e < tr * tc; e += T) {
        const int i0 = 2 * (e / tc), j0 = 2 * (e % tc);
        const int i1 = i0 + 1 < rows ? i0 + 1 : i0, j1 = j0 + 1 < cols ? j0 + 1 : j0;
        double sv[4] = {0.0, 0.0, 0.0, 0.0};
        if (wide)
          dot2x2(A, i0 * rows, i1 * rows, 1, Y, j0, j1, cols, rows, sv);
        else
          dot2x2(Y, i0 * cols, i1 * cols, 1, A, j0, j1, cols, cols, sv);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int i = i0 + (q >> 1), j = j0 + (q & 1);
          if (i >= rows || j >= cols) continue;
          const int o = i * cols + j;
          if (pass == 0) P[o] = sv[q];
          else X[o] = a * X[o] + b * P[o] + c * sv[q];
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < n; i += T) nW[i] = c1 * W[i] + c2 * X[i];
}

}  // namespace

// ---- exact tier host drivers: device f64 buffers --------------------------------------------------
// Matrices whose iterate, product and Gram matrix fit the LDS budget, in one launch of one workgroup
// each; PH_ERR_UNSUPPORTED (nothing launched) when one does not fit or the batch is too large.
int muon_mat_exact_batch(const ExactMat* mats, int n, const ExactVec* vecs, int nv, double gscale, double lr,
                         double wd, double mu, double eps, const double* coeffs, int nsteps, hipStream_t st) {
  if (n < 1 || n > kExactBatchMax || nv < 0 || nv > kExactBatchMax || nsteps > kExactFusedMaxSteps)
    return PH_ERR_UNSUPPORTED;
  ExactBatch bt{};
  bt.nm = n;
  for (int i = 0; i < nv; i++) bt.v[i] = vecs[i];
  long lds = 0;
  for (int i = 0; i < n; i++) {
    const ExactMat& m = mats[i];
    const long e = (long)m.rows * m.cols, mn = m.rows < m.cols ? m.rows : m.cols;
    if (e == 0 || 2 * e + mn * mn > kExactFusedLds) return PH_ERR_UNSUPPORTED;
    if (2 * e + mn * mn > lds) lds = 2 * e + mn * mn;
    bt.m[i] = m;
    bt.m[i].c2 = lr * sqrt(fmax(1.0, (double)m.rows / (double)m.cols));
  }
  ExactCoeffs cf{};
  for (int i = 0; i < 3 * nsteps; i++) cf.v[i] = coeffs[i];
  k_muon_exact_fused<<<n + nv, 1024, (size_t)lds * 8, st>>>(bt, gscale, lr, mu, eps, cf, nsteps, 1.0 - lr * wd);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int muon_mat_exact(int rows, int cols, const double* W, const double* G, const double* M, double* nW,
                   double* nM, double gscale, double lr, double wd, double mu, double eps,
                   const double* coeffs, int nsteps, hipStream_t st) {
  const long n = (long)rows * cols;
  if (n == 0) return PH_OK;
  const int mn = rows < cols ? rows : cols;
  const double scale = sqrt(fmax(1.0, (double)rows / (double)cols));
  {
    const ExactMat one{W, G, M, nW, nM, rows, cols, 0.0};
    const int r = muon_mat_exact_batch(&one, 1, nullptr, 0, gscale, lr, wd, mu, eps, coeffs, nsteps, st);
    if (r != PH_ERR_UNSUPPORTED) return r;
  }
  double* ws = (double*)scratch(kSlotMuonExact, (size_t)(6 * n + (long)mn * mn + rows + 8) * 8);
  if (!ws) return PH_ERR_NOMEM;
  double *U = ws, *X = U + n, *Xt = X + n, *P = Xt + n, *Q = P + n, *A = Q + n, *rs = A + (long)mn * mn,
         *inv = rs + rows;
  const unsigned gN = ceil_div(n, kB);
  k_nesterov_f64<<<gN, kB, 0, st>>>(G, M, nM, U, n, gscale, mu);
  k_rowsq_f64<<<ceil_div(rows, kB), kB, 0, st>>>(U, rs, rows, cols);
  k_frob_inv_f64<<<1, 1, 0, st>>>(rs, rows, eps, inv);
  k_scale_f64<<<gN, kB, 0, st>>>(U, inv, X, n);
  for (int it = 0; it < nsteps; it++) {
    const double a = coeffs[3 * it], b = coeffs[3 * it + 1], c = coeffs[3 * it + 2];
    k_transpose_f64<<<gN, kB, 0, st>>>(X, Xt, rows, cols);
    if (rows <= cols) {
      k_matmul_f64<<<ceil_div((long)rows * rows, kB), kB, 0, st>>>(X, Xt, A, rows, cols, rows);
      k_matmul_f64<<<gN, kB, 0, st>>>(A, X, P, rows, rows, cols);
      k_matmul_f64<<<gN, kB, 0, st>>>(A, P, Q, rows, rows, cols);
    } else {
      k_matmul_f64<<<ceil_div((long)cols * cols, kB), kB, 0, st>>>(Xt, X, A, cols, rows, cols);
      k_matmul_f64<<<gN, kB, 0, st>>>(X, A, P, rows, cols, cols);
      k_matmul_f64<<<gN, kB, 0, st>>>(P, A, Q, rows, cols, cols);
    }
    k_lincomb3_f64<<<gN, kB, 0, st>>>(X, a, P, b, Q, c, n);
  }
  k_finalize_f64<<<gN, kB, 0, st>>>(W, X, nW, 1.0 - lr * wd, lr * scale, n);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int stepvec_exact(long n, const double* b, const double* g, const double* m, double* nb, double* nm,
                  double gscale, double lr, double wd, double mu, hipStream_t st) {
  if (n == 0) return PH_OK;
  k_stepvec_f64<<<ceil_div(n, kB), kB, 0, st>>>(b, g, m, nb, nm, n, gscale, lr, wd, mu);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

// ---- fast tier as a GEMM chain: in-place NS of one fp32 matrix -------------------------------------
// Used for fp32 MFMA math and for zero steps (normalisation only); bf16 runs fused (ns.hip).
// Per step, all operands read straight from fp32 buffers:
//   A  = X X^T                 (bf16 MFMA; math == PH_MATH_F32: fp32 MFMA)
//   B  = b A + c A A^T         (split-bf16 MFMA, epilogue b*A + c*acc)
//   X' = a X + B X             (split-bf16 MFMA, epilogue a*X + acc, into the other X buffer)
// The split products keep the quintic within 1e-2 of the f64 iterate, which plain bf16 operands for
// A^2 and BX do not (about 2% at 512 x 1024 with the constant coefficients).
int newton_schulz_fast(float* X, int rows, int cols, const float* coeffs, int nsteps, float eps,
                       int math, int ns_slot, int ws_slot, hipStream_t st) {
  const long n = (long)rows * cols;
  if (n == 0) return PH_OK;
  const int m = rows < cols ? rows : cols, w = rows < cols ? cols : rows;
  const long mm = (long)m * m;
  const long chunk = 4096;
  const int G = (int)((n + chunk - 1) / chunk);
  if (G > 4000) {
    set_error("newton_schulz: matrix too large (%ld elements)", n);
    return PH_ERR_UNSUPPORTED;
  }
  const size_t bytes = (size_t)(2 * n + 2 * mm) * 4 + 4096 * 4 + 256;
  float* ws = (float*)scratch(ns_slot, bytes);
  if (!ws) return PH_ERR_NOMEM;
  float* Xs[2] = {ws, ws + n};
  float* Af = ws + 2 * n;
  float* Bf = Af + mm;
  float* part = Bf + mm;
  float* inv = part + 4000;
  k_sumsq_part<<<G, 256, 0, st>>>(X, n, chunk, part);
  k_norm_inv<<<1, 256, 0, st>>>(part, G, eps, inv);
  k_ns_load_f32<<<ceil_div(n, kB), kB, 0, st>>>(X, rows, cols, inv, Xs[0]);
  PH_LAUNCH_CHECK();
  const int m1 = math == PH_MATH_F32 ? PH_MATH_F32 : PH_MATH_BF16;
  const int m23 = math == PH_MATH_F32 ? PH_MATH_F32 : PH_MATH_BF16X3;
  for (int it = 0; it < nsteps; it++) {
    const float a = coeffs[3 * it], b = coeffs[3 * it + 1], c = coeffs[3 * it + 2];
    float* Xi = Xs[it & 1];
    float* Xo = Xs[(it + 1) & 1];
    PhGemmDesc d{};
    d.trans_a = 0; d.trans_b = 1; d.M = m; d.N = m; d.K = w;
    d.a_dtype = PH_F32; d.A = Xi; d.lda = w; d.b_dtype = PH_F32; d.B = Xi; d.ldb = w;
    d.c_dtype = PH_F32; d.C = Af; d.ldc = m; d.math = m1; d.epi = PH_EPI_NONE; d.alpha = 1.f;
    d.ws_slot = ws_slot;
    PH_TRY(gemm(d, st));
    d = PhGemmDesc{};
    d.trans_a = 0; d.trans_b = 1; d.M = m; d.N = m; d.K = m;
    d.a_dtype = PH_F32; d.A = Af; d.lda = m; d.b_dtype = PH_F32; d.B = Af; d.ldb = m;
    d.c_dtype = PH_F32; d.C = Bf; d.ldc = m; d.math = m23;
    d.epi = PH_EPI_AXPBY; d.alpha = c; d.beta = b; d.aux = Af; d.ldaux = m;
    d.ws_slot = ws_slot;
    PH_TRY(gemm(d, st));
    d = PhGemmDesc{};
    d.trans_a = 0; d.trans_b = 0; d.M = m; d.N = w; d.K = m;
    d.a_dtype = PH_F32; d.A = Bf; d.lda = m; d.b_dtype = PH_F32; d.B = Xi; d.ldb = w;
    d.c_dtype = PH_F32; d.C = Xo; d.ldc = w; d.math = m23;
    d.epi = PH_EPI_AXPBY; d.alpha = 1.f; d.beta = a; d.aux = Xi; d.ldaux = w;
    d.ws_slot = ws_slot;
    PH_TRY(gemm(d, st));
  }
  k_ns_store<<<ceil_div(n, kB), kB, 0, st>>>(Xs[nsteps & 1], rows, cols, X);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int muon_fast(float* W, const float* G, float* M, int rows, int cols, float gscale, float lr,
              float wd, float mu, float eps, const float* coeffs, int nsteps, int math,
              const LaneSlots& slots, hipStream_t st) {
  const long n = (long)rows * cols;
  if (n == 0) return PH_OK;
  float* U = (float*)scratch(slots.u, (size_t)n * 4);
  if (!U) return PH_ERR_NOMEM;
  k_nesterov_f32<<<ceil_div(n, kB), kB, 0, st>>>(G, M, U, n, gscale, mu);
  PH_LAUNCH_CHECK();
  PH_TRY(newton_schulz_fast(U, rows, cols, coeffs, nsteps, eps, math, slots.ns, slots.gemm_ws, st));
  const float scale = sqrtf(fmaxf(1.f, (float)rows / (float)cols));
  k_finalize_f32<<<ceil_div(n, kB), kB, 0, st>>>(W, U, n, 1.f - lr * wd, lr * scale);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int muon_fast_batch(const MuonMat* mats, int n, float gscale, float lr, float wd, float mu, float eps,
                    const float* coeffs, int nsteps, int math, hipStream_t st) {
  if (n <= 0) return PH_OK;
  if (n > kNsMaxMats) {
    set_error("muon: at most %d matrices per batch", kNsMaxMats);
    return PH_ERR_UNSUPPORTED;
  }
  size_t tot = 0;
  long off[kNsMaxMats];
  for (int i = 0; i < n; i++) {
    off[i] = (long)tot;
    tot += ((size_t)mats[i].rows * mats[i].cols + 63) & ~(size_t)63;  // 256-byte aligned updates
  }
  float* U = (float*)scratch(kSlotMuonU, tot * 4 + 4);
  if (!U) return PH_ERR_NOMEM;
  float* X[kNsMaxMats];
  int rows[kNsMaxMats], cols[kNsMaxMats];
  EwBatch nb{}, fb{};
  nb.n = fb.n = n;
  for (int i = 0; i < n; i++) {
    const long e = (long)mats[i].rows * mats[i].cols;
    X[i] = U + off[i];
    rows[i] = mats[i].rows;
    cols[i] = mats[i].cols;
    nb.start[i + 1] = fb.start[i + 1] = nb.start[i] + e;
    nb.p[i] = const_cast<float*>(mats[i].G);
    nb.q[i] = mats[i].M;
    nb.r[i] = X[i];
    fb.p[i] = mats[i].W;
    fb.r[i] = X[i];
    fb.s[i] = lr * sqrtf(fmaxf(1.f, (float)rows[i] / (float)cols[i]));
  }
  const long total = nb.start[n];
  if (total > 0) {
    k_nesterov_batch<<<ceil_div(total, kB), kB, 0, st>>>(nb, gscale, mu);
    PH_LAUNCH_CHECK();
  }
  if (math == PH_MATH_F32 || nsteps == 0) {
    for (int i = 0; i < n; i++)
      PH_TRY(newton_schulz_fast(X[i], rows[i], cols[i], coeffs, nsteps, eps, math, kSlotNs, 0, st));
  } else {
    PH_TRY(ns_fused(X, rows, cols, n, coeffs, nsteps, eps, kSlotNs, kSlotNsCtl, st));
  }
  if (total > 0) {
    k_finalize_batch<<<ceil_div(total, kB), kB, 0, st>>>(fb, 1.f - lr * wd);
    PH_LAUNCH_CHECK();
  }
  return PH_OK;
}

int stepvec_f32_batch(const StepVec* v, int n, float gscale, float lr, float wd, float mu, hipStream_t st) {
  PH_REQUIRE(n >= 0 && n <= kNsMaxMats, "stepvec: at most %d vectors per batch", kNsMaxMats);
  EwBatch b{};
  b.n = n;
  for (int i = 0; i < n; i++) {
    b.start[i + 1] = b.start[i] + v[i].n;
    b.p[i] = v[i].b;
    b.q[i] = const_cast<float*>(v[i].g);
    b.r[i] = v[i].m;
  }
  const long total = n > 0 ? b.start[n] : 0;
  if (total == 0) return PH_OK;
  k_stepvec_batch<<<ceil_div(total, kB), kB, 0, st>>>(b, gscale, lr, wd, mu);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int stepvec_f32(float* b, const float* g, float* m, long n, float gscale, float lr, float wd, float mu,
                hipStream_t st) {
  if (n == 0) return PH_OK;
  k_stepvec_f32<<<ceil_div(n, kB), kB, 0, st>>>(b, g, m, n, gscale, lr, wd, mu);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int gclip_f32(float* g, long n, float sc, float maxNorm, hipStream_t st) {
  if (n == 0) return PH_OK;
  const long chunk = 8192;
  const int G = (int)((n + chunk - 1) / chunk);
  float* part = (float*)scratch(kSlotGclip, (size_t)G * 4);
  if (!part) return PH_ERR_NOMEM;
  k_sumsq_part<<<G, 256, 0, st>>>(g, n, chunk, part);
  unsigned grid = ceil_div(n, 256);
  if (grid > 2048) grid = 2048;
  k_gclip_scale<<<grid, 256, 0, st>>>(g, n, part, G, sc, maxNorm);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_muon_mat_f64(int rows, int cols, const double* W, const double* G, const double* M,
                               double* nW, double* nM, double gscale, double lr, double wd, double mu,
                               double eps, const double* coeffs, int nsteps, void* stream) {
  PH_REQUIRE(rows >= 0 && cols >= 0 && nsteps >= 0 && nsteps <= 64, "ph_muon_mat_f64: bad shape");
  PH_REQUIRE(coeffs != nullptr || nsteps == 0, "ph_muon_mat_f64: coefficient table missing");
  return muon_mat_exact(rows, cols, W, G, M, nW, nM, gscale, lr, wd, mu, eps, coeffs, nsteps,
                        as_stream(stream));
}

extern "C" int ph_stepvec_f64(size_t n, const double* b, const double* g, const double* m, double* nb,
                              double* nm, double gscale, double lr, double wd, double mu, void* stream) {
  return stepvec_exact((long)n, b, g, m, nb, nm, gscale, lr, wd, mu, as_stream(stream));
}

extern "C" int ph_newton_schulz(float* X, int rows, int cols, const float* coeffs, int nsteps,
                                float eps, int math, void* stream) {
  PH_REQUIRE(rows >= 0 && cols >= 0 && nsteps >= 0 && nsteps <= 64, "ph_newton_schulz: bad shape");
  PH_REQUIRE(math == PH_MATH_BF16 || math == PH_MATH_F32 || math == PH_MATH_BF16X3,
             "ph_newton_schulz: unknown math");
  PH_REQUIRE(coeffs != nullptr || nsteps == 0, "ph_newton_schulz: coefficient table missing");
  if (math == PH_MATH_F32 || nsteps == 0)
    return newton_schulz_fast(X, rows, cols, coeffs, nsteps, eps, math, kSlotNs, 0, as_stream(stream));
  return ns_fused(&X, &rows, &cols, 1, coeffs, nsteps, eps, kSlotNs, kSlotNsCtl, as_stream(stream));
}

extern "C" int ph_newton_schulz_batch(float* const* X, const int* rows, const int* cols, int n,
                                      const float* coeffs, int nsteps, float eps, int math, void* stream) {
  PH_REQUIRE(n >= 0 && (n == 0 || (X && rows && cols)), "ph_newton_schulz_batch: bad arguments");
  PH_REQUIRE(nsteps >= 0 && nsteps <= 64 && (coeffs != nullptr || nsteps == 0),
             "ph_newton_schulz_batch: bad coefficient table");
  PH_REQUIRE(math == PH_MATH_BF16 || math == PH_MATH_F32 || math == PH_MATH_BF16X3,
             "ph_newton_schulz_batch: unknown math");
  for (int i = 0; i < n; i++) PH_REQUIRE(rows[i] >= 0 && cols[i] >= 0, "ph_newton_schulz_batch: bad shape");
  if (n == 0) return PH_OK;
  hipStream_t st = as_stream(stream);
  // bf16: the whole batch in fused launches on `stream`
  if (math != PH_MATH_F32 && nsteps > 0)
    return ns_fused(X, rows, cols, n, coeffs, nsteps, eps, kSlotNs, kSlotNsCtl, st);
  // fp32 MFMA: matrix i runs on stream lane i % kLanes with that lane's scratch; the lanes fork
  // from and join back into `stream`.
  const int nl = n < kLanes ? n : kLanes;
  LaneJoin lanes(st);
  PH_TRY(lanes.fork(nl));
  for (int i = 0; i < n; i++) {
    const LaneSlots sl = lane_slots(i % kLanes);
    PH_TRY(newton_schulz_fast(X[i], rows[i], cols[i], coeffs, nsteps, eps, math, sl.ns, sl.gemm_ws,
                              lane_stream(i % kLanes)));
  }
  return lanes.join();
}

extern "C" int ph_muon_mat(float* W, const float* G, float* M, int rows, int cols, float gscale,
                           float lr, float wd, float mu, float eps, const float* coeffs, int nsteps,
                           int math, void* stream) {
  PH_REQUIRE(rows >= 0 && cols >= 0 && nsteps >= 0 && nsteps <= 64, "ph_muon_mat: bad shape");
  PH_REQUIRE(coeffs != nullptr || nsteps == 0, "ph_muon_mat: coefficient table missing");
  PH_REQUIRE(math == PH_MATH_BF16 || math == PH_MATH_F32 || math == PH_MATH_BF16X3,
             "ph_muon_mat: unknown math");
  const MuonMat mm{W, G, M, rows, cols};
  return muon_fast_batch(&mm, 1, gscale, lr, wd, mu, eps, coeffs, nsteps, math, as_stream(stream));
}

extern "C" int ph_stepvec(float* b, const float* g, float* m, size_t n, float gscale, float lr,
                          float wd, float mu, void* stream) {
  return stepvec_f32(b, g, m, (long)n, gscale, lr, wd, mu, as_stream(stream));
}

extern "C" int ph_gclip(float* g, size_t n, float sc, float maxNorm, void* stream) {
  return gclip_f32(g, (long)n, sc, maxNorm, as_stream(stream));
}
