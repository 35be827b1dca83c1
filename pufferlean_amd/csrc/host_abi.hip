// Host-buffer entry points: one per GPU symbol the reference's Lean side binds with @[extern]
// (Puffer/Float/CUDA.lean, Puffer/Float/BLAS.lean; C bodies in ffi/puffercuda.cu, ffi/pufferblas.c).
//
// Each takes the reference symbol's arguments with every Lean FloatArray turned into a host
// `const double*` (input) or a caller-allocated `double*` (output of the documented size), uploads,
// runs the device kernels of this library on the default stream, downloads and synchronises, as the
// reference entries do. Differences from the reference, by design:
//   - no CPU fallback and no zero-filled result: a failure returns a ph_status and sets
//     ph_last_error(), and the outputs are unspecified;
//   - device buffers are library-owned scratch reused across calls (the reference's ts_buf / bg / rb2
//     caches play the same role).
#include <cmath>
#include <cstdlib>

#include <cstring>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

// The shared dashboard-loss channel (policy, value, entropy, total, old_kl, kl, clipfrac): defined
// here with external linkage because the reference's pufferblas.c declares it extern
// (pufferblas.c:38-39; defined at puffercuda.cu:261-262).
extern "C" {
int g_mgLossOn = 0;
double g_mgLoss[7] = {0, 0, 0, 0, 0, 0, 0};
}

namespace ph {
namespace {

constexpr unsigned kT = 256;

// The reference's Newton-Schulz coefficient schedule, one triple per step (pufferblas.c:1362-1364,
// puffercuda.cu:520-525).
const double kRefCoeffs[15] = {4.0848, -6.8946, 2.9270, 3.9505, -6.3029, 2.6377, 3.7418, -5.5913,
                               2.3037, 2.8769, -3.1427, 1.2046, 2.8366, -3.0525, 1.2012};
const float kRefCoeffsF[15] = {4.0848f, -6.8946f, 2.9270f, 3.9505f, -6.3029f, 2.6377f, 3.7418f, -5.5913f,
                               2.3037f, 2.8769f, -3.1427f, 1.2046f, 2.8366f, -3.0525f, 1.2012f};

enum : int {
  kHsVtrace = kSlotHost,
  kHsMlp = kSlotHost + 1,     // MLP minibatch working set
  kHsState = kSlotHost + 2,   // f64 parameter / momentum / gradient state of the non-resident steps
  kHsCols = kSlotHost + 3,    // whole-update columns + permutation
  kHsMuonU = kSlotHost + 4,   // f32 Newton-Schulz input of the mixed-precision Muon
  kHsMg = kSlotHost + 5,      // MinGRU host-mode staging
  kHsDense = kSlotHost + 6,
  kHsLoss = kSlotHost + 7,
  kHsClip = kSlotHost + 8,
  kHsGrad = kSlotHost + 9,    // uploaded f64 gradient of the resident Muon entries
  kHsMgOut = kSlotHost + 10,  // MinGRU host-mode result staging
  kHsDc = kSlotHost + 11,     // resident rollout columns of the MinGRU minibatch chain
  kHsPrio = kSlotHost + 12,   // resident sampler draws (segment indices, importance weights)
  kHsPrioHost = kSlotHost + 13,
  kHsGather = kSlotHost + 14,
  kHsRoll = kSlotHost + 15,   // MinGRU rollout step staging
  kHsSample = kSlotHost + 16, // sampler staging
  kHsObsTraj = kSlotHost + 17,  // resident obs trajectory of the MinGRU chain (f32)
  kHsHeads = kSlotHost + 18,    // multi-discrete / continuous head staging
  kHsGradRes = kSlotHost + 19,  // the MinGRU gradient left on the device for the resident Muon (f64)
};

// The resident hand-off between the MinGRU gradient and the resident Muon (the reference's bg 70 with
// its g_mgg_fresh stamp, and the g_mgw stamp of the weights the Muon leaves for the next gradient,
// puffercuda.cu:5237-5248, 5560-5580, 5727-5768, 5950-5968). The gradient stamp is consumed by one Muon
// step; the weights stamp names the policy handle whose weights the next gradient may take when the
// caller passes no parameters.
struct ResGrad {
  bool fresh = false;
  int dev = -1;
  long P = 0;
};
ResGrad g_mgg;
struct ResWeights {
  bool valid = false;
  int dev = -1;
  long P = 0;
  size_t handle = 0;
};
ResWeights g_mgw;

// Carves typed sub-buffers from one scratch slot: run the layout once to size it, allocate, run it
// again to assign.
struct Carve {
  uint8_t* base = nullptr;
  size_t off = 0;
  template <typename T>
  T* take(size_t n) {
    const size_t o = off;
    off += (n * sizeof(T) + 255) & ~(size_t)255;
    return base ? reinterpret_cast<T*>(base + o) : nullptr;
  }
};
template <typename F>
int carve(int slot, F&& layout) {
  Carve c0;
  layout(c0);
  void* p = scratch(slot, c0.off);
  if (!p) return PH_ERR_NOMEM;
  Carve c1;
  c1.base = (uint8_t*)p;
  layout(c1);
  return PH_OK;
}

int up(void* d, const void* h, size_t bytes) {
  if (bytes) PH_CHECK_HIP(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice));
  return PH_OK;
}
int down(void* h, const void* d, size_t bytes) {
  if (bytes) PH_CHECK_HIP(hipMemcpy(h, d, bytes, hipMemcpyDeviceToHost));
  return PH_OK;
}
int finish() {
  PH_CHECK_HIP(hipDeviceSynchronize());
  return PH_OK;
}

// ---- element kernels ---------------------------------------------------------------------------
__global__ void k_f64_f32(const double* __restrict__ x, float* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (float)x[i];
}
__global__ void k_f32_f64(const float* __restrict__ x, double* __restrict__ y, long n, double scale) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (double)x[i] * scale;
}
__global__ void k_f64_i32(const double* __restrict__ x, int* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (int)x[i];
}
// dst row k = src row idx[k] (the permutation holds row indices as doubles, read as (int)).
__global__ void k_gather_rows(const float* __restrict__ src, const double* __restrict__ idx,
                              float* __restrict__ dst, long n, int cols) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * cols) return;
  const long k = t / cols;
  const int j = (int)(t % cols);
  dst[t] = src[(long)(int)idx[k] * cols + j];
}
// Minibatch columns: actions as int, the rest as the f32 the loss kernel computes in.
__global__ void k_gather_cols(const double* __restrict__ idx, long n, const double* __restrict__ act,
                              const double* __restrict__ adv, const double* __restrict__ ret,
                              const double* __restrict__ old, const double* __restrict__ ov,
                              int* __restrict__ gact, double* __restrict__ gadv, float* __restrict__ gret,
                              float* __restrict__ gold, float* __restrict__ gov) {
  const long k = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n) return;
  const long r = idx ? (long)(int)idx[k] : k;
  if (gact) gact[k] = (int)act[r];
  gadv[k] = adv[r];
  gret[k] = (float)ret[r];
  gold[k] = (float)old[r];
  if (ov) gov[k] = (float)ov[r];
}
// Wide action rows: the Wd f64 action columns of row idx[k] (row k without idx) as int32
// (multi-discrete heads) into gi, or as f32 (Gaussian dims) into gf.
__global__ void k_gather_wide(const double* __restrict__ idx, long n, int Wd, const double* __restrict__ act,
                              int* __restrict__ gi, float* __restrict__ gf) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * Wd) return;
  const long k = t / Wd;
  const int j = (int)(t % Wd);
  const long r = idx ? (long)(int)idx[k] : k;
  const double v = act[r * Wd + j];
  if (gi) gi[t] = (int)v;
  else gf[t] = (float)v;
}
__global__ void k_bias_relu_f64(double* __restrict__ Y, const double* __restrict__ b, long N, int H,
                                int relu) {
#pragma clang fp contract(off)
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * H) return;
  const double v = Y[i] + b[i % H];
  Y[i] = relu ? (v > 0.0 ? v : 0.0) : v;
}
// Y[N x H] = relu(X W^T + b) in f64, each dot product an ascending fold over d (the reference's
// left-folded scalar order, pufferblas.c:65-80).
__global__ void k_dense_f64(const double* __restrict__ X, const double* __restrict__ W,
                            const double* __restrict__ b, double* __restrict__ Y, long N, int D, int H) {
#pragma clang fp contract(off)
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * H) return;
  const long i = t / H;
  const int j = (int)(t % H);
  const double* xr = X + i * D;
  const double* wr = W + (long)j * D;
  double acc = 0.0;
  for (int d = 0; d < D; d++) acc += xr[d] * wr[d];
  const double v = acc + b[j];
  Y[t] = v > 0.0 ? v : 0.0;
}
__global__ void k_f64_bf16(const double* __restrict__ x, uint16_t* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = bf16_rne((float)x[i]);
}

// Mixed-precision Muon pieces: f64 momentum and weights, f32 orthogonalisation input.
__global__ void k_nesterov_mixed(const double* __restrict__ G, double* __restrict__ M,
                                 float* __restrict__ U, long n, double gscale, double mu) {
#pragma clang fp contract(off)
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double gi = G[i] * gscale;
  const double m = mu * M[i] + gi;
  M[i] = m;
  U[i] = (float)(gi + mu * m);
}
__global__ void k_finalize_mixed(double* __restrict__ W, const float* __restrict__ X, long n, double c1,
                                 double c2) {
#pragma clang fp contract(off)
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) W[i] = c1 * W[i] + c2 * (double)X[i];
}

// Gradient-norm clip on an f64 vector (PufferLib clip_grad_norm_ over all parameters; the
// reference's k_gclip_norm/k_gclip_scale, puffercuda.cu:5122-5131): s = sum (g*sc)^2 in fixed
// chunks, folded in chunk order; cc = (maxNorm > 0 and sqrt(s) > maxNorm ? maxNorm/sqrt(s) : 1)*sc.
__global__ void __launch_bounds__(256) k_sq_part_f64(const double* __restrict__ g, long n, long chunk,
                                                     double sc, double* __restrict__ part) {
  __shared__ double sh[256];
  const long lo = (long)blockIdx.x * chunk;
  const long hi = lo + chunk < n ? lo + chunk : n;
  // eight loads in flight at a time, added in index order
  double s = 0.0;
  long i = lo + threadIdx.x;
  for (; i + 7 * 256 < hi; i += 8 * 256) {
    double v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) v[q] = g[i + q * 256];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const double x = v[q] * sc;
      s += x * x;
    }
  }
  for (; i < hi; i += 256) {
    const double x = g[i] * sc;
    s += x * x;
  }
  sh[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = sh[0];
}
__global__ void k_clip_scale_f64(double* __restrict__ g, long n, const double* __restrict__ part, int G,
                                 double maxNorm, double sc) {
  // one thread sums the partials in order, from LDS: their loads are one round trip per 512
  __shared__ double sp[512];
  __shared__ double cc;
  double s = 0.0;
  for (int b0 = 0; b0 < G; b0 += 512) {
    const int nb = G - b0 < 512 ? G - b0 : 512;
    __syncthreads();  // the previous slice has been summed
    for (int q = threadIdx.x; q < nb; q += blockDim.x) sp[q] = part[b0 + q];
    __syncthreads();
    if (threadIdx.x == 0)
      for (int q = 0; q < nb; q++) s += sp[q];
  }
  if (threadIdx.x == 0) {
    const double gn = sqrt(s);
    cc = ((maxNorm > 0.0 && gn > maxNorm) ? maxNorm / gn : 1.0) * sc;
  }
  __syncthreads();
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    g[i] = g[i] * cc;
}
__global__ void k_scale_f64v(double* __restrict__ g, long n, double sc) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) g[i] = sc * g[i];
}

int to_f32(const double* d, float* f, long n, hipStream_t st) {
  if (n <= 0) return PH_OK;
  k_f64_f32<<<ceil_div(n, kT), kT, 0, st>>>(d, f, n);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

// ---- one-hidden-layer MLP policy (flattenMLP: W1[H*D] | b1[H] | W2[O*H] | b2[O], O = A + 1) --------
struct MlpShape {
  long N;
  int H, D, A, O;
  long P, oW1, ob1, oW2, ob2;
};
MlpShape mlp_shape(size_t N, size_t H, size_t D, size_t A) {
  MlpShape s;
  s.N = (long)N; s.H = (int)H; s.D = (int)D; s.A = (int)A; s.O = (int)A + 1;
  s.oW1 = 0; s.ob1 = (long)H * D; s.oW2 = s.ob1 + (long)H; s.ob2 = s.oW2 + (long)s.O * H;
  s.P = s.ob2 + s.O;
  return s;
}

struct MlpWork {
  float *X, *Wf, *H1, *Out, *dOut, *dZ, *gf, *ret, *old, *ov;
  int* act;
  double *adv, *advn, *stats, *losses;
};
int mlp_work(const MlpShape& s, long Nmax, MlpWork& w) {
  return carve(kHsMlp, [&](Carve& c) {
    w.X = c.take<float>((size_t)Nmax * s.D);
    w.Wf = c.take<float>(s.P);
    w.H1 = c.take<float>((size_t)Nmax * s.H);
    w.Out = c.take<float>((size_t)Nmax * s.O);
    w.dOut = c.take<float>((size_t)Nmax * s.O);
    w.dZ = c.take<float>((size_t)Nmax * s.H);
    w.gf = c.take<float>(s.P);
    w.ret = c.take<float>(Nmax);
    w.old = c.take<float>(Nmax);
    w.ov = c.take<float>(Nmax);
    w.act = c.take<int>(Nmax);
    w.adv = c.take<double>(Nmax);
    w.advn = c.take<double>(Nmax);
    w.stats = c.take<double>(8);
    w.losses = c.take<double>(8);
  });
}

PhGemmDesc f32desc(int ta, int tb, long M, long N, long K, const float* A, long lda, const float* B, long ldb,
                   float* C, long ldc, int math) {
  PhGemmDesc d{};
  d.trans_a = ta; d.trans_b = tb; d.M = (int)M; d.N = (int)N; d.K = (int)K;
  d.a_dtype = PH_F32; d.A = A; d.lda = lda; d.b_dtype = PH_F32; d.B = B; d.ldb = ldb;
  d.c_dtype = PH_F32; d.C = C; d.ldc = ldc; d.math = math; d.alpha = 1.f;
  return d;
}

// Summed PPO gradient of one minibatch into w.gf (f32, flattenMLP layout). Inputs in w: X [N][D],
// Wf [P], act, adv (f64, already normalised if the caller wants), ret, old, ov (or use_ov = 0).
// Follows lean_cuda_mlp_ppo_grad (puffercuda.cu:748-820): H1 = relu(X W1^T + b1); Out = H1 W2^T + b2;
// dOut by the fused PPO loss (no max shift, as k_ppo_dout); gb2 = colsum dOut; gW2 = dOut^T H1;
// dZ = (dOut W2) masked by H1 > 0; gb1 = colsum dZ; gW1 = dZ^T X. `bf`: bf16 MFMA on the fp32
// operands (the reference's FAST_16BF), else fp32 MFMA.
// MLP forward (relu hidden, linear head) -> head(): the loss gradient of Out into dOut -> backward into
// the f32 gradient gf. head() may use dZ's first N floats as staging: dZ is written only by the dgrad
// GEMM that follows it.
template <typename HeadFn>
int mlp_grad_head(const MlpShape& s, long N, const MlpWork& w, int bf, HeadFn&& head, hipStream_t st) {
  const int math = bf ? PH_MATH_BF16 : PH_MATH_F32;
  const float* W1 = w.Wf + s.oW1;
  const float* b1 = w.Wf + s.ob1;
  const float* W2 = w.Wf + s.oW2;
  const float* b2 = w.Wf + s.ob2;
  PhGemmDesc g = f32desc(0, 1, N, s.H, s.D, w.X, s.D, W1, s.D, w.H1, s.H, math);
  g.epi = PH_EPI_BIAS_RELU; g.bias = b1;
  PH_TRY(gemm(g, st));
  g = f32desc(0, 1, N, s.O, s.H, w.H1, s.H, W2, s.H, w.Out, s.O, math);
  g.epi = PH_EPI_BIAS; g.bias = b2;
  PH_TRY(gemm(g, st));
  PH_TRY(head());
  PH_TRY(colsum_f32(w.dOut, N, s.O, s.O, w.gf + s.ob2, 1.f, 0, st));
  PH_TRY(gemm(f32desc(1, 0, s.O, s.H, N, w.dOut, s.O, w.H1, s.H, w.gf + s.oW2, s.H, math), st));
  g = f32desc(0, 0, N, s.H, s.O, w.dOut, s.O, W2, s.H, w.dZ, s.H, math);
  g.epi = PH_EPI_RELU_MASK; g.aux = w.H1; g.ldaux = s.H;
  PH_TRY(gemm(g, st));
  PH_TRY(colsum_f32(w.dZ, N, s.H, s.H, w.gf + s.ob1, 1.f, 0, st));
  PH_TRY(gemm(f32desc(1, 0, s.H, s.D, N, w.dZ, s.H, w.X, s.D, w.gf + s.oW1, s.D, math), st));
  return PH_OK;
}

int mlp_grad_dev(const MlpShape& s, long N, const MlpWork& w, int bf, double vf, double ent, double clip,
                 double vfClip, bool use_ov, double* losses, hipStream_t st) {
  return mlp_grad_head(s, N, w, bf, [&]() {
    // advantages as the f32 the loss computes in, staged in dZ
    float* advf = w.dZ;
    PH_TRY(to_f32(w.advn, advf, N, st));
    return ppo_grad(w.Out, s.O, w.Out + s.A, s.O, w.act, advf, w.ret, w.old, use_ov ? w.ov : nullptr, N, s.A,
                    (float)vf, (float)ent, (float)clip, (float)vfClip, 0, w.dOut, s.O, w.dOut + s.A, s.O, nullptr,
                    nullptr, losses, st);
  }, st);
}

// Muon on an f64 [rows x cols] matrix in place: exact tier (f64 Newton-Schulz, the reference's op
// order) or mixed tier (f64 momentum and weights, f32-MFMA Newton-Schulz, as muon_mat_dev_bf,
// puffercuda.cu:942-966).
int muon_f64(int rows, int cols, double* W, const double* G, double* M, double gscale, double lr,
             double wd, double mu, double eps, bool mixed, hipStream_t st) {
  const long n = (long)rows * cols;
  if (n == 0) return PH_OK;
  if (!mixed)
    return muon_mat_exact(rows, cols, W, G, M, W, M, gscale, lr, wd, mu, eps, kRefCoeffs, 5, st);
  float* U = (float*)scratch(kHsMuonU, (size_t)n * 4);
  if (!U) return PH_ERR_NOMEM;
  k_nesterov_mixed<<<ceil_div(n, kT), kT, 0, st>>>(G, M, U, n, gscale, mu);
  PH_LAUNCH_CHECK();
  PH_TRY(newton_schulz_fast(U, rows, cols, kRefCoeffsF, 5, (float)eps, PH_MATH_F32, kSlotNs, 0, st));
  const double scale = sqrt(fmax(1.0, (double)rows / (double)cols));
  k_finalize_mixed<<<ceil_div(n, kT), kT, 0, st>>>(W, U, n, 1.0 - lr * wd, lr * scale);
  PH_LAUNCH_CHECK();
  return PH_OK;
}
int stepvec_f64(long n, double* b, const double* g, double* m, double gscale, double lr, double wd,
                double mu, hipStream_t st) {
  return stepvec_exact(n, b, g, m, b, m, gscale, lr, wd, mu, st);
}
// Whole-MLP Muon over [params | mom] in place (W1, W2 orthogonalised; b1, b2 by stepvec).
int mlp_muon(const MlpShape& s, double* par, double* mom, const double* G, double gscale, double lr,
             double wd, double mu, double eps, bool mixed, hipStream_t st) {
  if (!mixed) {  // both matrices and both bias steps in one launch when the matrices fit a workgroup each
    const ExactMat mats[2] = {{par + s.oW1, G + s.oW1, mom + s.oW1, par + s.oW1, mom + s.oW1, s.H, s.D, 0.0},
                              {par + s.oW2, G + s.oW2, mom + s.oW2, par + s.oW2, mom + s.oW2, s.O, s.H, 0.0}};
    const ExactVec vecs[2] = {{par + s.ob1, G + s.ob1, mom + s.ob1, (long)s.H},
                              {par + s.ob2, G + s.ob2, mom + s.ob2, (long)s.O}};
    const int r = muon_mat_exact_batch(mats, 2, vecs, 2, gscale, lr, wd, mu, eps, kRefCoeffs, 5, st);
    if (r != PH_ERR_UNSUPPORTED) return r;
  }
  PH_TRY(muon_f64(s.H, s.D, par + s.oW1, G + s.oW1, mom + s.oW1, gscale, lr, wd, mu, eps, mixed, st));
  PH_TRY(stepvec_f64(s.H, par + s.ob1, G + s.ob1, mom + s.ob1, gscale, lr, wd, mu, st));
  PH_TRY(muon_f64(s.O, s.H, par + s.oW2, G + s.oW2, mom + s.oW2, gscale, lr, wd, mu, eps, mixed, st));
  PH_TRY(stepvec_f64(s.O, par + s.ob2, G + s.ob2, mom + s.ob2, gscale, lr, wd, mu, st));
  return PH_OK;
}

int gclip_f64(double* g, long n, double sc, double maxNorm, hipStream_t st) {
  if (n == 0) return PH_OK;
  const long chunk = 16384;
  const int G = (int)((n + chunk - 1) / chunk);
  double* part = (double*)scratch(kHsClip, (size_t)G * 8);
  if (!part) return PH_ERR_NOMEM;
  k_sq_part_f64<<<G, 256, 0, st>>>(g, n, chunk, sc, part);
  unsigned grid = ceil_div(n, 256);
  if (grid > 2048) grid = 2048;
  k_clip_scale_f64<<<grid, 256, 0, st>>>(g, n, part, G, maxNorm, sc);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

// Minibatch-sized f64 state of a non-resident step: params | mom | G.
struct State {
  double *par, *mom, *G;
};
int state_bufs(long P, State& t) {
  return carve(kHsState, [&](Carve& c) {
    t.par = c.take<double>(2 * P);
    t.mom = t.par ? t.par + P : nullptr;
    t.G = c.take<double>(P);
  });
}

// One minibatch of the PPO+Muon update on device-resident state: gather (idx may be null: rows 0..N-1
// of the columns), normalise the advantages, gradient, mean (and optional clip), Muon in place.
struct Cols {
  float* obs;  // [NT][D]
  const double *act, *adv, *ret, *old, *ov;  // act: [NT][Wd] (Wd = 1 for the categorical head)
};
// The action head of an update: one categorical head over the O - 1 logits (mode 0), K categorical
// heads of the given sizes (mode 1), or a Gaussian of Wd dims (mode 2). actI / actF hold the gathered
// minibatch actions of modes 1 and 2.
struct HeadSpec {
  int mode = 0;
  int Wd = 1;
  int sizes[kMaxHeads] = {};
  int* actI = nullptr;
  float* actF = nullptr;
};
constexpr double kContLsLo = -20.0, kContLsHi = 2.0;  // the reference's GPU clamp (puffercuda.cu:1646-1647)
int mlp_minibatch(const MlpShape& s, const HeadSpec& head, const Cols& cols, const double* idx, long Nmb,
                  MlpWork& w, double* par, double* mom, double* G, int bf, bool mixed, double lr, double wd,
                  double mu, double eps, double vf, double ent, double clip, double vfClip, double maxGradNorm,
                  bool want_losses, hipStream_t st) {
  const bool use_ov = cols.ov != nullptr && vfClip > 0.0;
  const bool cat = head.mode == 0;
  if (idx) {
    k_gather_rows<<<ceil_div(Nmb * s.D, kT), kT, 0, st>>>(cols.obs, idx, w.X, Nmb, s.D);
  } else {
    PH_CHECK_HIP(hipMemcpyAsync(w.X, cols.obs, (size_t)Nmb * s.D * 4, hipMemcpyDeviceToDevice, st));
  }
  k_gather_cols<<<ceil_div(Nmb, kT), kT, 0, st>>>(idx, Nmb, cat ? cols.act : nullptr, cols.adv, cols.ret, cols.old,
                                                 use_ov ? cols.ov : nullptr, cat ? w.act : nullptr, w.adv, w.ret,
                                                 w.old, w.ov);
  PH_LAUNCH_CHECK();
  if (!cat) {
    k_gather_wide<<<ceil_div(Nmb * head.Wd, kT), kT, 0, st>>>(idx, Nmb, head.Wd, cols.act, head.actI, head.actF);
    PH_LAUNCH_CHECK();
  }
  PH_TRY(moments_normalize(PH_F64, w.adv, Nmb, w.advn, w.stats, st));
  PH_TRY(to_f32(par, w.Wf, s.P, st));
  double* losses = want_losses ? w.losses : nullptr;
  if (cat) {
    PH_TRY(mlp_grad_dev(s, Nmb, w, bf, vf, ent, clip, vfClip, use_ov, losses, st));
  } else {
    PH_TRY(mlp_grad_head(s, Nmb, w, bf, [&]() {
      PH_TRY(to_f32(w.advn, w.dZ, Nmb, st));  // advantages as the f32 the loss computes in, staged in dZ
      const float* ov = use_ov ? w.ov : nullptr;
      if (head.mode == 1)
        return ppo_grad_md(w.Out, s.O, head.actI, w.dZ, w.ret, w.old, ov, Nmb, head.sizes, head.Wd, (float)vf,
                           (float)ent, (float)clip, (float)vfClip, w.dOut, s.O, nullptr, nullptr, losses, st);
      return ppo_grad_cont(w.Out, s.O, head.actF, w.dZ, w.ret, w.old, ov, Nmb, head.Wd, (float)vf, (float)ent,
                           (float)clip, (float)vfClip, (float)kContLsLo, (float)kContLsHi, w.dOut, s.O, nullptr,
                           nullptr, losses, st);
    }, st));
  }
  k_f32_f64<<<ceil_div(s.P, kT), kT, 0, st>>>(w.gf, G, s.P, 1.0);
  PH_LAUNCH_CHECK();
  double gscale = 1.0 / (double)Nmb;
  if (maxGradNorm > 0.0) {
    PH_TRY(gclip_f64(G, s.P, gscale, maxGradNorm, st));
    gscale = 1.0;
  }
  PH_TRY(mlp_muon(s, par, mom, G, gscale, lr, wd, mu, eps, mixed, st));
  if (want_losses) PH_TRY(down(g_mgLoss, w.losses, 7 * 8));
  return PH_OK;
}

bool env_is(const char* name, const char* val) {
  const char* e = getenv(name);
  return e && strcmp(e, val) == 0;
}

}  // namespace
}  // namespace ph

using namespace ph;

// ---- V-trace / advantage normalisation --------------------------------------------------------
extern "C" int ph_cuda_vtrace(const double* rew, const double* val, const double* term, const double* imp,
                              size_t B, size_t T, double gamma, double lam, double rhoClip, double cClip,
                              double* adv) {
  PH_REQUIRE(B * T == 0 || (rew && val && term && imp && adv), "ph_cuda_vtrace: null buffer");
  if (B * T == 0) return PH_OK;
  const size_t n = B * T;
  double *dR, *dV, *dT, *dI, *dA;
  PH_TRY(carve(kHsVtrace, [&](Carve& c) {
    dR = c.take<double>(n); dV = c.take<double>(n); dT = c.take<double>(n); dI = c.take<double>(n);
    dA = c.take<double>(n);
  }));
  PH_TRY(up(dR, rew, n * 8)); PH_TRY(up(dV, val, n * 8)); PH_TRY(up(dT, term, n * 8)); PH_TRY(up(dI, imp, n * 8));
  PH_TRY(ph_vtrace(PH_F64, dR, dV, dT, dI, nullptr, B, T, 0, 0, 0, 1, gamma, lam, rhoClip, cClip, dA,
                   nullptr, nullptr));
  PH_TRY(finish());
  return down(adv, dA, n * 8);
}

extern "C" int ph_cuda_vtrace_mingru(const double* rew, const double* val, const double* term,
                                     const double* imp, const double* bootv, size_t B, size_t T,
                                     double gamma, double lam, double rhoClip, double cClip, double* adv) {
  PH_REQUIRE(B * T == 0 || (rew && val && term && imp && bootv && adv), "ph_cuda_vtrace_mingru: null buffer");
  if (B * T == 0) return PH_OK;
  const size_t n = B * T;
  double *dR, *dV, *dT, *dI, *dB, *dA;
  PH_TRY(carve(kHsVtrace, [&](Carve& c) {
    dR = c.take<double>(n); dV = c.take<double>(n); dT = c.take<double>(n); dI = c.take<double>(n);
    dB = c.take<double>(B); dA = c.take<double>(n);
  }));
  PH_TRY(up(dR, rew, n * 8)); PH_TRY(up(dV, val, n * 8)); PH_TRY(up(dT, term, n * 8));
  PH_TRY(up(dI, imp, n * 8)); PH_TRY(up(dB, bootv, B * 8));
  PH_TRY(ph_vtrace(PH_F64, dR, dV, dT, dI, dB, B, T, 1, 0, 0, 1, gamma, lam, rhoClip, cClip, dA, nullptr,
                   nullptr));
  PH_TRY(finish());
  return down(adv, dA, n * 8);
}

extern "C" int ph_cuda_adv_normalize(const double* adv, size_t n, double* out) {
  PH_REQUIRE(n == 0 || (adv && out), "ph_cuda_adv_normalize: null buffer");
  if (n == 0) return PH_OK;
  double *dA, *dO, *dS;
  PH_TRY(carve(kHsVtrace, [&](Carve& c) {
    dA = c.take<double>(n); dO = c.take<double>(n); dS = c.take<double>(8);
  }));
  PH_TRY(up(dA, adv, n * 8));
  PH_TRY(moments_normalize(PH_F64, dA, n, dO, dS, nullptr));
  PH_TRY(finish());
  return down(out, dO, n * 8);
}

// ---- MLP PPO gradient and whole steps -----------------------------------------------------------
extern "C" int ph_cuda_mlp_ppo_grad(const double* params, const double* obs, const double* acts,
                                    const double* advs, const double* rets, const double* oldlps, size_t N,
                                    size_t H, size_t D, size_t A, double vfCoef, double entCoef,
                                    double clipEps, uint8_t bf16, double* g) {
  PH_REQUIRE(N > 0 && H > 0 && D > 0 && A >= 1 && A <= 64, "ph_cuda_mlp_ppo_grad: bad shape");
  PH_REQUIRE(params && obs && acts && advs && rets && oldlps && g, "ph_cuda_mlp_ppo_grad: null buffer");
  const MlpShape s = mlp_shape(N, H, D, A);
  MlpWork w;
  PH_TRY(mlp_work(s, s.N, w));
  double *dp, *dx, *dc, *dg;
  PH_TRY(carve(kHsCols, [&](Carve& c) {
    dp = c.take<double>(s.P); dx = c.take<double>((size_t)N * D); dc = c.take<double>(4 * N);
    dg = c.take<double>(s.P);
  }));
  PH_TRY(up(dp, params, s.P * 8)); PH_TRY(up(dx, obs, N * D * 8));
  PH_TRY(up(dc, acts, N * 8)); PH_TRY(up(dc + N, advs, N * 8));
  PH_TRY(up(dc + 2 * N, rets, N * 8)); PH_TRY(up(dc + 3 * N, oldlps, N * 8));
  PH_TRY(to_f32(dp, w.Wf, s.P, nullptr));
  PH_TRY(to_f32(dx, w.X, (long)N * D, nullptr));
  k_gather_cols<<<ceil_div(N, kT), kT>>>(nullptr, (long)N, dc, dc + N, dc + 2 * N, dc + 3 * N, nullptr, w.act,
                                         w.advn, w.ret, w.old, nullptr);
  PH_LAUNCH_CHECK();
  PH_TRY(mlp_grad_dev(s, s.N, w, bf16, vfCoef, entCoef, clipEps, 0.0, false, nullptr, nullptr));
  k_f32_f64<<<ceil_div(s.P, kT), kT>>>(w.gf, dg, s.P, 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(g, dg, s.P * 8);
}

namespace {
// Shared set-up of the multi-discrete / continuous MLP gradients: params, obs, adv, ret, old on the
// device in the f32/f64 forms mlp_grad_head's head kernel reads.
int mlp_head_inputs(const MlpShape& s, const double* params, const double* obs, const double* advs,
                    const double* rets, const double* oldlps, MlpWork& w, double*& dg) {
  PH_TRY(mlp_work(s, s.N, w));
  double *dp, *dx, *dc;
  PH_TRY(carve(kHsCols, [&](Carve& c) {
    dp = c.take<double>(s.P); dx = c.take<double>((size_t)s.N * s.D); dc = c.take<double>(3 * s.N);
    dg = c.take<double>(s.P);
  }));
  PH_TRY(up(dp, params, s.P * 8)); PH_TRY(up(dx, obs, (size_t)s.N * s.D * 8));
  PH_TRY(up(w.advn, advs, s.N * 8)); PH_TRY(up(dc, rets, s.N * 8)); PH_TRY(up(dc + s.N, oldlps, s.N * 8));
  PH_TRY(to_f32(dp, w.Wf, s.P, nullptr));
  PH_TRY(to_f32(dx, w.X, s.N * s.D, nullptr));
  PH_TRY(to_f32(dc, w.ret, s.N, nullptr));
  PH_TRY(to_f32(dc + s.N, w.old, s.N, nullptr));
  return PH_OK;
}
int mlp_head_finish(const MlpShape& s, const MlpWork& w, double* dg, double* g) {
  k_f32_f64<<<ceil_div(s.P, kT), kT>>>(w.gf, dg, s.P, 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(g, dg, s.P * 8);
}
int sizes_from(const double* hs, size_t K, int* sizes, size_t& W, const char* who) {
  PH_REQUIRE(hs && K >= 1 && K <= (size_t)kMaxHeads, "%s: K=%zu heads (1..%d)", who, K, kMaxHeads);
  W = 0;
  for (size_t h = 0; h < K; h++) {
    PH_REQUIRE(hs[h] >= 1.0 && hs[h] <= 4096.0, "%s: head %zu size %g", who, h, hs[h]);
    sizes[h] = (int)hs[h];
    W += (size_t)sizes[h];
  }
  return PH_OK;
}
}  // namespace

extern "C" int ph_cuda_mlp_ppo_grad_md(const double* params, const double* obs, const double* acts,
                                       const double* advs, const double* rets, const double* oldlps,
                                       const double* hs, size_t N, size_t H, size_t D, size_t K, double vfCoef,
                                       double entCoef, double clipEps, uint8_t bf16, double* g) {
  int sizes[kMaxHeads];
  size_t W = 0;
  PH_TRY(sizes_from(hs, K, sizes, W, "ph_cuda_mlp_ppo_grad_md"));
  PH_REQUIRE(N > 0 && H > 0 && D > 0 && N <= 0x7fffffffUL, "ph_cuda_mlp_ppo_grad_md: bad shape");
  PH_REQUIRE(params && obs && acts && advs && rets && oldlps && g, "ph_cuda_mlp_ppo_grad_md: null buffer");
  const MlpShape s = mlp_shape(N, H, D, W);
  MlpWork w;
  double* dg;
  PH_TRY(mlp_head_inputs(s, params, obs, advs, rets, oldlps, w, dg));
  double* da;
  int* ai;
  PH_TRY(carve(kHsHeads, [&](Carve& c) { da = c.take<double>(N * K); ai = c.take<int>(N * K); }));
  PH_TRY(up(da, acts, N * K * 8));
  k_f64_i32<<<ceil_div(N * K, kT), kT>>>(da, ai, (long)(N * K));
  PH_LAUNCH_CHECK();
  PH_TRY(mlp_grad_head(s, s.N, w, bf16, [&]() {
    PH_TRY(to_f32(w.advn, w.dZ, s.N, nullptr));
    return ppo_grad_md(w.Out, s.O, ai, w.dZ, w.ret, w.old, nullptr, N, sizes, K, (float)vfCoef, (float)entCoef,
                       (float)clipEps, 0.f, w.dOut, s.O, nullptr, nullptr, nullptr, nullptr);
  }, nullptr));
  return mlp_head_finish(s, w, dg, g);
}

extern "C" int ph_cuda_mlp_ppo_grad_cont(const double* params, const double* obs, const double* acts,
                                         const double* advs, const double* rets, const double* oldlps, size_t N,
                                         size_t H, size_t D, size_t d, double vfCoef, double entCoef, double clipEps,
                                         uint8_t bf16, double* g) {
  PH_REQUIRE(N > 0 && H > 0 && D > 0 && d >= 1 && N <= 0x7fffffffUL, "ph_cuda_mlp_ppo_grad_cont: bad shape");
  PH_REQUIRE(params && obs && acts && advs && rets && oldlps && g, "ph_cuda_mlp_ppo_grad_cont: null buffer");
  const MlpShape s = mlp_shape(N, H, D, 2 * d);
  MlpWork w;
  double* dg;
  PH_TRY(mlp_head_inputs(s, params, obs, advs, rets, oldlps, w, dg));
  double* da;
  float* af;
  PH_TRY(carve(kHsHeads, [&](Carve& c) { da = c.take<double>(N * d); af = c.take<float>(N * d); }));
  PH_TRY(up(da, acts, N * d * 8));
  PH_TRY(to_f32(da, af, (long)(N * d), nullptr));
  PH_TRY(mlp_grad_head(s, s.N, w, bf16, [&]() {
    PH_TRY(to_f32(w.advn, w.dZ, s.N, nullptr));
    return ppo_grad_cont(w.Out, s.O, af, w.dZ, w.ret, w.old, nullptr, N, d, (float)vfCoef, (float)entCoef,
                         (float)clipEps, 0.f, (float)kContLsLo, (float)kContLsHi, w.dOut, s.O, nullptr, nullptr,
                         nullptr, nullptr);
  }, nullptr));
  return mlp_head_finish(s, w, dg, g);
}

extern "C" int ph_cuda_sample_actions_md(const double* Y, const double* hs, size_t N, size_t K, size_t O,
                                         uint64_t rng, double* out) {
  int sizes[kMaxHeads];
  size_t W = 0;
  PH_TRY(sizes_from(hs, K, sizes, W, "ph_cuda_sample_actions_md"));
  PH_REQUIRE(O >= W + 1 && N <= 0x7fffffffUL, "ph_cuda_sample_actions_md: O=%zu below %zu", O, W + 1);
  if (N == 0) return PH_OK;
  PH_REQUIRE(Y && out, "ph_cuda_sample_actions_md: null buffer");
  double *dY, *dO;
  PH_TRY(carve(kHsSample, [&](Carve& c) { dY = c.take<double>(N * O); dO = c.take<double>((K + 2) * N); }));
  PH_TRY(up(dY, Y, N * O * 8));
  PH_TRY(sample_actions_md(PH_F64, dY, O, N, sizes, K, rng, dO, nullptr));
  PH_TRY(finish());
  return down(out, dO, (K + 2) * N * 8);
}

extern "C" int ph_cuda_sample_actions_cont(const double* Y, size_t N, size_t d, size_t O, uint64_t rng, double* out) {
  PH_REQUIRE(d >= 1 && O >= 2 * d + 1 && N <= 0x7fffffffUL, "ph_cuda_sample_actions_cont: d=%zu O=%zu", d, O);
  if (N == 0) return PH_OK;
  PH_REQUIRE(Y && out, "ph_cuda_sample_actions_cont: null buffer");
  double *dY, *dO;
  PH_TRY(carve(kHsSample, [&](Carve& c) { dY = c.take<double>(N * O); dO = c.take<double>((d + 2) * N); }));
  PH_TRY(up(dY, Y, N * O * 8));
  PH_TRY(sample_actions_cont(PH_F64, dY, O, N, d, rng, kContLsLo, kContLsHi, dO, nullptr));
  PH_TRY(finish());
  return down(out, dO, (d + 2) * N * 8);
}

extern "C" int ph_cuda_train_step(const double* pm, const double* obs, const double* acts,
                                  const double* advRaw, const double* rets, const double* oldlps, size_t N,
                                  size_t H, size_t D, size_t A, double lr, double wd, double mu, double eps,
                                  double vfCoef, double entCoef, double clipEps, uint8_t bf16, double* out) {
  PH_REQUIRE(N > 0 && H > 0 && D > 0 && A >= 1 && A <= 64, "ph_cuda_train_step: bad shape");
  PH_REQUIRE(pm && obs && acts && advRaw && rets && oldlps && out, "ph_cuda_train_step: null buffer");
  const MlpShape s = mlp_shape(N, H, D, A);
  MlpWork w;
  State t;
  PH_TRY(mlp_work(s, s.N, w));
  PH_TRY(state_bufs(s.P, t));
  double *dx, *dc;
  float* obsf;
  PH_TRY(carve(kHsCols, [&](Carve& c) {
    dx = c.take<double>((size_t)N * D); dc = c.take<double>(4 * N); obsf = c.take<float>((size_t)N * D);
  }));
  PH_TRY(up(t.par, pm, 2 * s.P * 8)); PH_TRY(up(dx, obs, N * D * 8));
  PH_TRY(up(dc, acts, N * 8)); PH_TRY(up(dc + N, advRaw, N * 8));
  PH_TRY(up(dc + 2 * N, rets, N * 8)); PH_TRY(up(dc + 3 * N, oldlps, N * 8));
  PH_TRY(to_f32(dx, obsf, (long)N * D, nullptr));
  const Cols cols{obsf, dc, dc + N, dc + 2 * N, dc + 3 * N, nullptr};
  // bf16 tier: bf16-MFMA gradient GEMMs and fp32-MFMA Newton-Schulz (the reference's bf16 Muon runs
  // fp32 Sgemm, puffercuda.cu:937-941); fp32 tier: fp32 GEMMs and the exact f64 Newton-Schulz.
  PH_TRY(mlp_minibatch(s, HeadSpec{}, cols, nullptr, s.N, w, t.par, t.mom, t.G, bf16, bf16 != 0, lr, wd, mu, eps,
                       vfCoef, entCoef, clipEps, 0.0, 0.0, false, nullptr));
  PH_TRY(finish());
  return down(out, t.par, 2 * s.P * 8);
}

namespace {
// Shared body of the whole-update entries: columns uploaded once, epochs x minibatches on device.
// acts holds head.Wd f64 columns per row. Every shuffle index must lie in [0, NT): the gathers read
// the row it names.
int train_update_impl(double* par, double* mom, const HeadSpec& head0, const double* obs, const double* acts,
                      const double* adv, const double* ret, const double* olp, const double* ov, const double* perm,
                      size_t NT, size_t D, size_t H, size_t O, size_t epochs, size_t numMB, double lr, double wd,
                      double mu, double eps, double vfCoef, double entCoef, double clipEps, double vfClip,
                      double maxGradNorm, int bf, bool mixed, bool losses, const char* who) {
  for (size_t i = 0; i < epochs * NT; i++)
    PH_REQUIRE(perm[i] >= 0.0 && perm[i] < (double)NT, "%s: shuffle index %g at %zu outside [0, %zu)", who, perm[i], i,
               NT);
  const MlpShape s = mlp_shape(NT, H, D, O - 1);
  const size_t mbSize = numMB > 0 && NT / numMB > 0 ? NT / numMB : 1;
  const size_t Wd = (size_t)head0.Wd;
  HeadSpec head = head0;
  MlpWork w;
  PH_TRY(mlp_work(s, s.N, w));
  double *dx, *dact, *dc, *dperm, *G;
  float* obsf;
  PH_TRY(carve(kHsCols, [&](Carve& c) {
    dx = c.take<double>(NT * D); dact = c.take<double>(NT * Wd); dc = c.take<double>(4 * NT);
    dperm = c.take<double>(epochs * NT); obsf = c.take<float>(NT * D); G = c.take<double>(s.P);
    head.actI = head.mode == 1 ? c.take<int>(NT * Wd) : nullptr;
    head.actF = head.mode == 2 ? c.take<float>(NT * Wd) : nullptr;
  }));
  PH_TRY(up(dx, obs, NT * D * 8));
  PH_TRY(up(dact, acts, NT * Wd * 8)); PH_TRY(up(dc, adv, NT * 8));
  PH_TRY(up(dc + NT, ret, NT * 8)); PH_TRY(up(dc + 2 * NT, olp, NT * 8));
  if (ov) PH_TRY(up(dc + 3 * NT, ov, NT * 8));
  PH_TRY(up(dperm, perm, epochs * NT * 8));
  PH_TRY(to_f32(dx, obsf, (long)(NT * D), nullptr));
  const Cols cols{obsf, dact, dc, dc + NT, dc + 2 * NT, ov ? dc + 3 * NT : nullptr};
  for (size_t e = 0; e < epochs; e++)
    for (size_t m = 0; m < numMB; m++) {
      const size_t lo = m * mbSize;
      size_t hi = (m + 1 == numMB) ? NT : (m + 1) * mbSize;
      if (hi > NT) hi = NT;
      if (hi <= lo) continue;
      const bool last = losses && e + 1 == epochs && m + 1 == numMB;
      PH_TRY(mlp_minibatch(s, head, cols, dperm + e * NT + lo, (long)(hi - lo), w, par, mom, G, bf, mixed, lr, wd,
                           mu, eps, vfCoef, entCoef, clipEps, vfClip, maxGradNorm, last, nullptr));
    }
  return PH_OK;
}
}  // namespace

extern "C" int ph_cuda_train_update(const double* pm, const double* obs, const double* acts, const double* adv,
                                    const double* ret, const double* olp, const double* perm, size_t NT,
                                    size_t D, size_t H, size_t A, size_t epochs, size_t numMB, double lr,
                                    double wd, double mu, double eps, double vfCoef, double entCoef,
                                    double clipEps, uint8_t bf16, double* out) {
  PH_REQUIRE(NT > 0 && H > 0 && D > 0 && A >= 1 && A <= 64 && numMB > 0, "ph_cuda_train_update: bad shape");
  PH_REQUIRE(pm && obs && acts && adv && ret && olp && perm && out, "ph_cuda_train_update: null buffer");
  const MlpShape s = mlp_shape(NT, H, D, A);
  State t;
  PH_TRY(state_bufs(s.P, t));
  PH_TRY(up(t.par, pm, 2 * s.P * 8));
  // the whole-update twin always orthogonalises in exact f64 (puffercuda.cu:1168-1171)
  PH_TRY(train_update_impl(t.par, t.mom, HeadSpec{}, obs, acts, adv, ret, olp, nullptr, perm, NT, D, H, A + 1,
                           epochs, numMB, lr, wd, mu, eps, vfCoef, entCoef, clipEps, 0.0, 0.0, bf16, false, false,
                           "ph_cuda_train_update"));
  PH_TRY(finish());
  return down(out, t.par, 2 * s.P * 8);
}

extern "C" int ph_cuda_train_update_resident(size_t policyH, const double* obs, const double* acts,
                                             const double* adv, const double* ret, const double* olp,
                                             const double* ov, size_t ovN, const double* perm, size_t NT,
                                             size_t D, size_t H, size_t A, size_t epochs, size_t numMB,
                                             double lr, double wd, double mu, double eps, double vfCoef,
                                             double entCoef, double clipEps, double vfClip,
                                             double maxGradNorm, uint8_t bf16, double* out1) {
  PH_REQUIRE(policyH != 0, "ph_cuda_train_update_resident: no policy handle");
  PH_REQUIRE(NT > 0 && H > 0 && D > 0 && A >= 1 && A <= 64 && numMB > 0,
             "ph_cuda_train_update_resident: bad shape");
  PH_REQUIRE(obs && acts && adv && ret && olp && perm && out1, "ph_cuda_train_update_resident: null buffer");
  const MlpShape s = mlp_shape(NT, H, D, A);
  double* par = (double*)policyH;
  const bool vclip = vfClip > 0.0 && ov && ovN >= NT;  // an empty old-value column turns the clip off
  PH_TRY(train_update_impl(par, par + s.P, HeadSpec{}, obs, acts, adv, ret, olp, vclip ? ov : nullptr, perm, NT, D,
                           H, A + 1, epochs, numMB, lr, wd, mu, eps, vfCoef, entCoef, clipEps, vclip ? vfClip : 0.0,
                           maxGradNorm, bf16, bf16 != 0, g_mgLossOn != 0, "ph_cuda_train_update_resident"));
  PH_TRY(finish());
  return down(out1, par, 8);  // params[0], the caller's divergence guard
}

extern "C" int ph_cuda_train_update_wide_resident(size_t policyH, const double* obs, const double* acts,
                                                  const double* adv, const double* ret, const double* olp,
                                                  const double* ov, size_t ovN, const double* perm, const double* hs,
                                                  size_t hsN, size_t NT, size_t D, size_t H, size_t O, size_t Wdim,
                                                  uint32_t mode, size_t epochs, size_t numMB, double lr, double wd,
                                                  double mu, double eps, double vfCoef, double entCoef,
                                                  double clipEps, double vfClip, double maxGradNorm, uint8_t bf16,
                                                  double* out1) {
  const char* who = "ph_cuda_train_update_wide_resident";
  PH_REQUIRE(policyH != 0, "%s: no policy handle", who);
  PH_REQUIRE(mode == 1 || mode == 2, "%s: mode %u (1 multi-discrete, 2 Gaussian)", who, mode);
  PH_REQUIRE(NT > 0 && H > 0 && D > 0 && Wdim >= 1 && numMB > 0 && NT <= 0x7fffffffUL, "%s: bad shape", who);
  PH_REQUIRE(obs && acts && adv && ret && olp && perm && out1, "%s: null buffer", who);
  HeadSpec head;
  head.mode = (int)mode;
  head.Wd = (int)Wdim;
  if (mode == 1) {
    PH_REQUIRE(hs && hsN >= Wdim, "%s: %zu head sizes for %zu heads", who, hsN, Wdim);
    size_t W = 0;
    PH_TRY(sizes_from(hs, Wdim, head.sizes, W, who));
    PH_REQUIRE(O == W + 1, "%s: O=%zu but the head sizes sum to %zu", who, O, W);
  } else {
    PH_REQUIRE(O == 2 * Wdim + 1, "%s: O=%zu for %zu Gaussian dims (2d+1)", who, O, Wdim);
  }
  const MlpShape s = mlp_shape(NT, H, D, O - 1);
  double* par = (double*)policyH;
  const bool vclip = vfClip > 0.0 && ov && ovN >= NT;  // an empty old-value column turns the clip off
  // the wide update orthogonalises in exact f64 whatever the GEMM precision (puffercuda.cu:1397-1400)
  PH_TRY(train_update_impl(par, par + s.P, head, obs, acts, adv, ret, olp, vclip ? ov : nullptr, perm, NT, D, H, O,
                           epochs, numMB, lr, wd, mu, eps, vfCoef, entCoef, clipEps, vclip ? vfClip : 0.0,
                           maxGradNorm, bf16, false, g_mgLossOn != 0, who));
  PH_TRY(finish());
  return down(out1, par, 8);  // params[0], the caller's divergence guard
}

// ---- Muon -----------------------------------------------------------------------------------------
extern "C" int ph_cuda_muon_stepmat(const double* W, const double* G, const double* M, size_t rows,
                                    size_t cols, double lr, double wd, double mu, double eps, double* out) {
  PH_REQUIRE(rows * cols == 0 || (W && G && M && out), "ph_cuda_muon_stepmat: null buffer");
  PH_REQUIRE(rows <= INT32_MAX && cols <= INT32_MAX, "ph_cuda_muon_stepmat: extents exceed int32");
  const size_t n = rows * cols;
  if (n == 0) return PH_OK;
  double *dW, *dG, *dM;
  PH_TRY(carve(kHsState, [&](Carve& c) { dW = c.take<double>(n); dG = c.take<double>(n); dM = c.take<double>(n); }));
  PH_TRY(up(dW, W, n * 8)); PH_TRY(up(dG, G, n * 8)); PH_TRY(up(dM, M, n * 8));
  PH_TRY(muon_f64((int)rows, (int)cols, dW, dG, dM, 1.0, lr, wd, mu, eps, false, nullptr));
  PH_TRY(finish());
  PH_TRY(down(out, dW, n * 8));
  return down(out + n, dM, n * 8);
}

extern "C" int ph_cuda_muon_step_mlp_resident(size_t policyH, const double* gRaw, size_t H, size_t D, size_t O,
                                              double gscale, double lr, double wd, double mu, double eps,
                                              double* newParams) {
  PH_REQUIRE(policyH != 0, "ph_cuda_muon_step_mlp_resident: no policy handle");
  PH_REQUIRE(O >= 2 && H > 0 && D > 0 && gRaw && newParams, "ph_cuda_muon_step_mlp_resident: bad arguments");
  const MlpShape s = mlp_shape(1, H, D, O - 1);
  double* par = (double*)policyH;
  double* G = (double*)scratch(kHsGrad, (size_t)s.P * 8);
  if (!G) return PH_ERR_NOMEM;
  PH_TRY(up(G, gRaw, s.P * 8));
  PH_TRY(mlp_muon(s, par, par + s.P, G, gscale, lr, wd, mu, eps, false, nullptr));
  PH_TRY(finish());
  return down(newParams, par, s.P * 8);
}

// ---- device-resident policy handle ([params(P); mom(P)] f64) ----------------------------------------
extern "C" int ph_cuda_policy_load(const double* pm, size_t P, size_t* handle) {
  PH_REQUIRE(pm && handle && P > 0, "ph_cuda_policy_load: bad arguments");
  double* d = nullptr;
  PH_CHECK_HIP(hipMalloc((void**)&d, 16 * P));
  if (hipMemcpy(d, pm, 16 * P, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(d);
    set_error("ph_cuda_policy_load: upload failed");
    return PH_ERR_HIP;
  }
  *handle = (size_t)d;
  return PH_OK;
}
extern "C" int ph_cuda_policy_download(size_t handle, size_t P, double* pm) {
  PH_REQUIRE(handle != 0 && pm, "ph_cuda_policy_download: bad arguments");
  PH_TRY(finish());
  return down(pm, (const void*)handle, 16 * P);
}
extern "C" int ph_cuda_policy_free(size_t handle) {
  if (handle && g_mgw.handle == handle) g_mgw = ResWeights{};
  if (handle) {
    PH_CHECK_HIP(hipDeviceSynchronize());
    PH_CHECK_HIP(hipFree((void*)handle));
  }
  return PH_OK;
}

// ---- checkpoint byte layout (FFITrain.lean:40-69): [P as u64 LE][P doubles as IEEE bits, LE] -------
namespace {
void put_u64le(uint8_t* b, uint64_t x) {
  for (int k = 0; k < 8; k++) b[k] = (uint8_t)(x >> (8 * k));
}
uint64_t get_u64le(const uint8_t* b) {
  uint64_t x = 0;
  for (int k = 0; k < 8; k++) x |= (uint64_t)b[k] << (8 * k);
  return x;
}
}  // namespace

extern "C" size_t ph_ckpt_bytes(size_t P) { return 8 * (P + 1); }

extern "C" int ph_ckpt_encode(const double* w, size_t P, uint8_t* out) {
  PH_REQUIRE(out && (P == 0 || w), "ph_ckpt_encode: null buffer");
  put_u64le(out, (uint64_t)P);
  for (size_t i = 0; i < P; i++) {
    uint64_t bits;
    memcpy(&bits, &w[i], 8);
    put_u64le(out + 8 * (i + 1), bits);
  }
  return PH_OK;
}

extern "C" int ph_ckpt_decode(const uint8_t* b, size_t nbytes, double* w, size_t cap, size_t* P_out) {
  PH_REQUIRE(P_out && (nbytes == 0 || b), "ph_ckpt_decode: null buffer");
  // bytesToCkpt: the header's count, bounded by the whole doubles the file holds
  const size_t avail = nbytes >= 8 ? (nbytes - 8) / 8 : 0;
  const size_t head = nbytes >= 8 ? (size_t)get_u64le(b) : 0;
  const size_t P = head < avail ? head : avail;
  *P_out = P;
  if (!w) return PH_OK;
  PH_REQUIRE(cap >= P, "ph_ckpt_decode: %zu doubles do not fit a buffer of %zu", P, cap);
  for (size_t i = 0; i < P; i++) {
    const uint64_t bits = get_u64le(b + 8 * (i + 1));
    memcpy(&w[i], &bits, 8);
  }
  return PH_OK;
}

extern "C" int ph_cuda_policy_save_ckpt(size_t handle, size_t P, uint8_t* out) {
  PH_REQUIRE(handle != 0 && out && P > 0, "ph_cuda_policy_save_ckpt: bad arguments");
  std::vector<double> w(P);
  PH_TRY(finish());
  PH_TRY(down(w.data(), (const void*)handle, 8 * P));  // the weights: the first P of [params; mom]
  return ph_ckpt_encode(w.data(), P, out);
}

extern "C" int ph_cuda_policy_load_ckpt(const uint8_t* b, size_t nbytes, size_t P, size_t* handle) {
  PH_REQUIRE(handle && P > 0, "ph_cuda_policy_load_ckpt: bad arguments");
  size_t Pf = 0;
  PH_TRY(ph_ckpt_decode(b, nbytes, nullptr, 0, &Pf));
  PH_REQUIRE(Pf == P, "ph_cuda_policy_load_ckpt: checkpoint has %zu params, this policy needs %zu", Pf, P);
  std::vector<double> pm(2 * P, 0.0);  // momentum starts at zero, as the trainers reload
  PH_TRY(ph_ckpt_decode(b, nbytes, pm.data(), P, &Pf));
  return ph_cuda_policy_load(pm.data(), P, handle);
}

// ---- dashboard-loss channel --------------------------------------------------------------------
extern "C" int ph_cuda_mg_loss_enable(uint8_t on) {
  g_mgLossOn = on ? 1 : 0;
  return PH_OK;
}
extern "C" int ph_cuda_mg_read_losses(double* out7) {
  PH_REQUIRE(out7, "ph_cuda_mg_read_losses: null buffer");
  for (int i = 0; i < 7; i++) out7[i] = g_mgLoss[i];
  return PH_OK;
}

// ---- dense forward entries of pufferblas.c -----------------------------------------------------------
extern "C" int ph_ffi_dense_forward_gpu(const double* X, const double* W, const double* b, size_t N, size_t D,
                                        size_t H, double* Y) {
  PH_REQUIRE(N * H == 0 || (X && W && b && Y), "ph_ffi_dense_forward_gpu: null buffer");
  if (N * H == 0) return PH_OK;
  double *dX, *dW, *db, *dY;
  PH_TRY(carve(kHsDense, [&](Carve& c) {
    dX = c.take<double>(N * D); dW = c.take<double>(H * D); db = c.take<double>(H); dY = c.take<double>(N * H);
  }));
  PH_TRY(up(dX, X, N * D * 8)); PH_TRY(up(dW, W, H * D * 8)); PH_TRY(up(db, b, H * 8));
  k_dense_f64<<<ceil_div(N * H, kT), kT>>>(dX, dW, db, dY, (long)N, (int)D, (int)H);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(Y, dY, N * H * 8);
}

extern "C" int ph_ffi_dense_forward_bf16(const double* X, const double* W, const double* b, size_t N, size_t D,
                                         size_t H, double* Y) {
  PH_REQUIRE(N * H == 0 || (X && W && b && Y), "ph_ffi_dense_forward_bf16: null buffer");
  if (N * H == 0) return PH_OK;
  double *dX, *dW, *db, *dY;
  uint16_t *xb, *wb;
  float* yf;
  PH_TRY(carve(kHsDense, [&](Carve& c) {
    dX = c.take<double>(N * D); dW = c.take<double>(H * D); db = c.take<double>(H); dY = c.take<double>(N * H);
    xb = c.take<uint16_t>(N * D); wb = c.take<uint16_t>(H * D); yf = c.take<float>(N * H);
  }));
  PH_TRY(up(dX, X, N * D * 8)); PH_TRY(up(dW, W, H * D * 8)); PH_TRY(up(db, b, H * 8));
  k_f64_bf16<<<ceil_div(N * D, kT), kT>>>(dX, xb, (long)(N * D));
  k_f64_bf16<<<ceil_div(H * D, kT), kT>>>(dW, wb, (long)(H * D));
  PH_LAUNCH_CHECK();
  PhGemmDesc g{};
  g.trans_a = 0; g.trans_b = 1; g.M = (int)N; g.N = (int)H; g.K = (int)D;
  g.a_dtype = PH_BF16; g.A = xb; g.lda = (long)D; g.b_dtype = PH_BF16; g.B = wb; g.ldb = (long)D;
  g.c_dtype = PH_F32; g.C = yf; g.ldc = (long)H; g.math = PH_MATH_BF16; g.alpha = 1.f;
  PH_TRY(gemm(g, nullptr));
  k_f32_f64<<<ceil_div(N * H, kT), kT>>>(yf, dY, (long)(N * H), 1.0);
  k_bias_relu_f64<<<ceil_div(N * H, kT), kT>>>(dY, db, (long)N, (int)H, 1);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(Y, dY, N * H * 8);
}

namespace {
// relu(X W1^T + b1) W2^T + b2 on the MFMA GEMMs, f64 in and out.
int mlp_forward_host(const double* p, const double* X, size_t N, size_t D, size_t H, size_t O, int math,
                     double* Y) {
  const size_t P = H * D + H + O * H + O;
  double *dp, *dX, *dY;
  float *pf, *xf, *h1, *of;
  PH_TRY(carve(kHsDense, [&](Carve& c) {
    dp = c.take<double>(P); dX = c.take<double>(N * D); dY = c.take<double>(N * O);
    pf = c.take<float>(P); xf = c.take<float>(N * D); h1 = c.take<float>(N * H); of = c.take<float>(N * O);
  }));
  PH_TRY(up(dp, p, P * 8)); PH_TRY(up(dX, X, N * D * 8));
  PH_TRY(to_f32(dp, pf, (long)P, nullptr));
  PH_TRY(to_f32(dX, xf, (long)(N * D), nullptr));
  PhGemmDesc g = f32desc(0, 1, (long)N, (long)H, (long)D, xf, (long)D, pf, (long)D, h1, (long)H, math);
  g.epi = PH_EPI_BIAS_RELU; g.bias = pf + H * D;
  PH_TRY(gemm(g, nullptr));
  g = f32desc(0, 1, (long)N, (long)O, (long)H, h1, (long)H, pf + H * D + H, (long)H, of, (long)O, math);
  g.epi = PH_EPI_BIAS; g.bias = pf + H * D + H + O * H;
  PH_TRY(gemm(g, nullptr));
  k_f32_f64<<<ceil_div(N * O, kT), kT>>>(of, dY, (long)(N * O), 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(Y, dY, N * O * 8);
}
}  // namespace

extern "C" int ph_ffi_mlp_forward_batch_bf16(const double* p, const double* X, size_t N, size_t D, size_t H,
                                             size_t O, double* Y) {
  PH_REQUIRE(N * O == 0 || (p && X && Y), "ph_ffi_mlp_forward_batch_bf16: null buffer");
  if (N * O == 0) return PH_OK;
  return mlp_forward_host(p, X, N, D, H, O, PH_MATH_BF16, Y);
}

// lean_cuda_mlp_forward (puffercuda.cu:6038-6060): the same forward with the reference's gemm32
// precision switch (bf16 products, or fp32).
extern "C" int ph_cuda_mlp_forward(const double* params, const double* obs, size_t N, size_t D, size_t H,
                                   size_t O, uint8_t bf16, double* out) {
  PH_REQUIRE(N * O == 0 || (params && obs && out), "ph_cuda_mlp_forward: null buffer");
  if (N * O == 0) return PH_OK;
  return mlp_forward_host(params, obs, N, D, H, O, bf16 ? PH_MATH_BF16 : PH_MATH_F32, out);
}

// lean_cuda_sample_actions (puffercuda.cu:1521-1536): f64 logits rows in, [act; logp; value] out.
extern "C" int ph_cuda_sample_actions(const double* Y, size_t N, size_t A, size_t O, uint64_t rng, double* out) {
  PH_REQUIRE(A >= 1 && O >= A + 1, "ph_cuda_sample_actions: A=%zu O=%zu (the value column is A)", A, O);
  PH_REQUIRE(N <= 0x7fffffffUL, "ph_cuda_sample_actions: N=%zu", N);
  if (N == 0) return PH_OK;
  PH_REQUIRE(Y && out, "ph_cuda_sample_actions: null buffer");
  double *dY, *dO;
  PH_TRY(carve(kHsSample, [&](Carve& c) { dY = c.take<double>(N * O); dO = c.take<double>(3 * N); }));
  PH_TRY(up(dY, Y, N * O * 8));
  PH_TRY(sample_actions(PH_F64, dY, O, N, A, 1, rng, nullptr, nullptr, nullptr, dO, nullptr));
  PH_TRY(finish());
  return down(out, dO, 3 * N * 8);
}

// lean_cuda_mingru_step (puffercuda.cu:2190-2265): one rollout timestep over N envs, state in and out
// as f64 [n][l][h].
extern "C" int ph_cuda_mingru_step(const double* params, const double* obs, const double* state, size_t N,
                                   size_t D, size_t H, size_t L, size_t A, uint8_t bf16, double* out) {
  PH_REQUIRE(N > 0 && D > 0 && H > 0 && L > 0 && A > 0 && A + 1 <= 32 && N <= 0x7fffffffUL,
             "ph_cuda_mingru_step: N=%zu D=%zu H=%zu L=%zu A=%zu (A + 1 <= 32)", N, D, H, L, A);
  PH_REQUIRE(params && obs && state && out, "ph_cuda_mingru_step: null buffer");
  const size_t O = A + 1, P = H * D + H + L * 3 * H * H + A * H + A + H + 1, ns = N * L * H;
  double *dp, *dx, *ds, *dout;
  float *pf, *xf, *sf, *of;
  PH_TRY(carve(kHsRoll, [&](Carve& c) {
    dp = c.take<double>(P); dx = c.take<double>(N * D); ds = c.take<double>(ns); dout = c.take<double>(N * O + ns);
    pf = c.take<float>(P); xf = c.take<float>(N * D); sf = c.take<float>(ns); of = c.take<float>(N * O);
  }));
  PH_TRY(up(dp, params, P * 8)); PH_TRY(up(dx, obs, N * D * 8)); PH_TRY(up(ds, state, ns * 8));
  PH_TRY(to_f32(dp, pf, (long)P, nullptr));
  PH_TRY(to_f32(dx, xf, (long)(N * D), nullptr));
  PH_TRY(to_f32(ds, sf, (long)ns, nullptr));
  ph_mingru_dims d{(int)N, 1, (int)D, (int)H, (int)L, (int)A, bf16 ? 0 : 1};
  PH_TRY(mingru_rollout_step(d, pf, xf, sf, of, nullptr));
  k_f32_f64<<<ceil_div(N * O, kT), kT>>>(of, dout, (long)(N * O), 1.0);
  k_f32_f64<<<ceil_div(ns, kT), kT>>>(sf, dout + N * O, (long)ns, 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  return down(out, dout, (N * O + ns) * 8);
}

// Device-resident bf16 dense-layer throughput in GFLOP/s (2*N*D*H per rep); -1 without a device.
extern "C" double ph_ffi_bench_bf16_resident(size_t N, size_t D, size_t H, size_t reps) {
  if (N * D * H == 0 || reps == 0) return -1.0;
  uint16_t *xb = nullptr, *wb = nullptr;
  float* yf = nullptr;
  if (carve(kHsDense, [&](Carve& c) {
        xb = c.take<uint16_t>(N * D); wb = c.take<uint16_t>(H * D); yf = c.take<float>(N * H);
      }) != PH_OK)
    return -1.0;
  PhGemmDesc g{};
  g.trans_a = 0; g.trans_b = 1; g.M = (int)N; g.N = (int)H; g.K = (int)D;
  g.a_dtype = PH_BF16; g.A = xb; g.lda = (long)D; g.b_dtype = PH_BF16; g.B = wb; g.ldb = (long)D;
  g.c_dtype = PH_F32; g.C = yf; g.ldc = (long)H; g.math = PH_MATH_BF16; g.alpha = 1.f;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
  if (gemm(g, nullptr) != PH_OK) return -1.0;
  (void)hipEventRecord(e0, nullptr);
  for (size_t r = 0; r < reps; r++)
    if (gemm(g, nullptr) != PH_OK) return -1.0;
  (void)hipEventRecord(e1, nullptr);
  (void)hipEventSynchronize(e1);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ms > 0.f ? 2.0 * (double)N * D * H * reps / (ms * 1e-3) / 1e9 : -1.0;
}

extern "C" uint8_t ph_ffi_cuda_available(void) { return ph_device_count() > 0 ? 1 : 0; }

// Link-time contract of pufferblas.c (pufferblas.c:46-50): the GPU LSTM BPTT is not part of this
// library, and returning 0 is the reference's documented "no usable device / unsupported shape" answer
// that makes the caller run its own CPU path.
extern "C" int cuda_lstm_ppo_grad_batch(const double*, const double*, const double*, const double*,
                                        const double*, const double*, const double*, const double*,
                                        const double*, size_t, size_t, size_t, size_t, size_t, double, double,
                                        double, double*, double*, int) {
  return 0;
}

// ---- prioritised replay: resident rollout columns ------------------------------------------------
namespace {
// The resident columns of the MinGRU minibatch chain (the reference's g_dc* buffers,
// puffercuda.cu:286-336), segment-major [N][T] f64, bound to the device current at prep; and the
// sampler's resident draws (the reference's bg 75/76 with the g_prio_fresh stamp).
struct DcState {
  bool valid = false;
  int dev = -1;
  long N = 0, T = 0, K = 1;
  double *rew = nullptr, *term = nullptr, *act = nullptr, *logp = nullptr, *value = nullptr,
         *ratio = nullptr, *boot = nullptr, *adv = nullptr, *L1 = nullptr;
  bool prio_fresh = false;
  long prioB = 0;
  int* seg = nullptr;
  double* mp = nullptr;
};
DcState g_dc;


// The resident obs trajectory [N*T][D] f32, row e*T+t (the reference's g_dMGObsTraj,
// puffercuda.cu:2136), bound to the device current when it was stored.
struct ObsTraj {
  bool valid = false;
  int dev = -1;
  long N = 0, T = 0, D = 0;
  float* obs = nullptr;
};
ObsTraj g_traj;

// Minibatch obs, time-major: x[(t*B + bi)*D + j] = traj[(seg[bi]*T + t)*D + j] (k_gather_mg_obs,
// puffercuda.cu:2146-2150).
__global__ void k_gather_obs_traj(const float* __restrict__ traj, const int* __restrict__ seg, long B, long T,
                                  long D, float* __restrict__ x) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * B * D) return;
  const long j = i % D, r = i / D, t = r / B, bi = r - t * B;
  x[i] = traj[((long)seg[bi] * T + t) * D + j];
}

__global__ void k_fill_f64(double* __restrict__ x, long n, double v) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = v;
}
__global__ void k_i32_f64(const int* __restrict__ x, double* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (double)x[i];
}

ph_replay_cols dc_cols() {
  ph_replay_cols c{};
  c.dtype = PH_F64;
  c.time_major = 0;
  c.N = (size_t)g_dc.N; c.T = (size_t)g_dc.T; c.K = (size_t)g_dc.K;
  c.adv = g_dc.adv; c.value = g_dc.value; c.ratio = g_dc.ratio;
  c.act = g_dc.act; c.logp = g_dc.logp; c.term = g_dc.term;
  return c;
}

int dc_check(size_t N, size_t T, const char* who) {
  int dev = -1;
  PH_CHECK_HIP(hipGetDevice(&dev));
  PH_REQUIRE(g_dc.valid && g_dc.N == (long)N && g_dc.T == (long)T && g_dc.dev == dev,
             "%s: no resident columns for N=%zu T=%zu on this device (call ph_cuda_mg_prep first)", who, N,
             T);
  return PH_OK;
}

// Segment indices arrive as doubles; every one must name a segment.
int check_seg_host(const double* seg, size_t B, size_t N, const char* who) {
  for (size_t i = 0; i < B; i++)
    PH_REQUIRE(seg[i] >= 0.0 && seg[i] < (double)N && seg[i] == (double)(long)seg[i],
               "%s: segIdx[%zu] = %g is not a segment index in [0, %zu)", who, i, seg[i], N);
  return PH_OK;
}
}  // namespace

extern "C" int ph_cuda_mg_prep(const double* rew, const double* term, const double* act, const double* logp,
                               const double* val, const double* boot, size_t N, size_t T, size_t K) {
  g_dc.valid = false;
  g_dc.prio_fresh = false;
  if (K < 1) K = 1;
  PH_REQUIRE(N > 0 && T > 0 && N <= 0x7fffffffUL && T <= 0x7fffffffUL, "ph_cuda_mg_prep: N=%zu T=%zu", N, T);
  PH_REQUIRE(rew && term && act && logp && val && boot, "ph_cuda_mg_prep: null buffer");
  const size_t n = N * T;
  DcState d;
  PH_TRY(carve(kHsDc, [&](Carve& c) {
    d.rew = c.take<double>(n); d.term = c.take<double>(n); d.act = c.take<double>(n * K);
    d.logp = c.take<double>(n); d.value = c.take<double>(n); d.ratio = c.take<double>(n);
    d.boot = c.take<double>(N); d.adv = c.take<double>(n); d.L1 = c.take<double>(N);
  }));
  PH_TRY(up(d.rew, rew, n * 8)); PH_TRY(up(d.term, term, n * 8)); PH_TRY(up(d.act, act, n * K * 8));
  PH_TRY(up(d.logp, logp, n * 8)); PH_TRY(up(d.value, val, n * 8)); PH_TRY(up(d.boot, boot, N * 8));
  k_fill_f64<<<ceil_div(n, kT), kT>>>(d.ratio, (long)n, 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  PH_CHECK_HIP(hipGetDevice(&d.dev));
  d.N = (long)N; d.T = (long)T; d.K = (long)K;
  d.valid = true;
  g_dc = d;
  return PH_OK;
}

extern "C" int ph_cuda_mg_cols_ready(size_t N, size_t T, uint8_t* ready) {
  (void)N;
  (void)T;
  PH_REQUIRE(ready, "ph_cuda_mg_cols_ready: null output");
  *ready = 0;
  return PH_OK;
}

extern "C" int ph_cuda_mg_obs_traj(const double* obs, size_t N, size_t T, size_t D) {
  g_traj.valid = false;
  PH_REQUIRE(N > 0 && T > 0 && D > 0 && N <= 0x7fffffffUL, "ph_cuda_mg_obs_traj: N=%zu T=%zu D=%zu", N, T, D);
  PH_REQUIRE(obs, "ph_cuda_mg_obs_traj: null buffer");
  const size_t n = N * T * D;
  double* d64;
  float* f;
  PH_TRY(carve(kHsObsTraj, [&](Carve& c) { d64 = c.take<double>(n); f = c.take<float>(n); }));
  PH_TRY(up(d64, obs, n * 8));
  PH_TRY(to_f32(d64, f, (long)n, nullptr));
  PH_TRY(finish());
  PH_CHECK_HIP(hipGetDevice(&g_traj.dev));
  g_traj.N = (long)N; g_traj.T = (long)T; g_traj.D = (long)D; g_traj.obs = f;
  g_traj.valid = true;
  return PH_OK;
}

namespace {
int dc_vtrace_l1(double gamma, double lam, double rhoClip, double cClip) {
  PH_TRY(ph_vtrace(PH_F64, g_dc.rew, g_dc.value, g_dc.term, g_dc.ratio, g_dc.boot, (size_t)g_dc.N,
                   (size_t)g_dc.T, 1, 0, 0, 1, gamma, lam, rhoClip, cClip, g_dc.adv, nullptr, nullptr));
  const ph_replay_cols c = dc_cols();
  return seg_l1(c, g_dc.L1, nullptr);
}
}  // namespace

extern "C" int ph_cuda_mg_vtrace(size_t N, size_t T, double gamma, double lam, double rhoClip, double cClip,
                                 double* L1out) {
  PH_TRY(dc_check(N, T, "ph_cuda_mg_vtrace"));
  PH_REQUIRE(L1out, "ph_cuda_mg_vtrace: null output");
  PH_TRY(dc_vtrace_l1(gamma, lam, rhoClip, cClip));
  PH_TRY(finish());
  return down(L1out, g_dc.L1, N * 8);
}

extern "C" int ph_cuda_mg_vtrace_prio(size_t N, size_t T, double gamma, double lam, double rhoClip,
                                      double cClip, size_t mbSegs, double prioAlpha, double annealBeta,
                                      uint64_t rng, uint8_t* used) {
  PH_REQUIRE(used, "ph_cuda_mg_vtrace_prio: null output");
  *used = 0;
  g_dc.prio_fresh = false;
  if (env_is("PUFFER_MG_DEVPRIO", "0")) return PH_OK;
  PH_TRY(dc_check(N, T, "ph_cuda_mg_vtrace_prio"));
  PH_REQUIRE(mbSegs > 0 && mbSegs <= 0x7fffffffUL, "ph_cuda_mg_vtrace_prio: mbSegs=%zu", mbSegs);
  int* seg;
  double* mp;
  PH_TRY(carve(kHsPrio, [&](Carve& c) { seg = c.take<int>(mbSegs); mp = c.take<double>(mbSegs); }));
  PH_TRY(dc_vtrace_l1(gamma, lam, rhoClip, cClip));
  PH_TRY(prio_sample(g_dc.L1, N, mbSegs, prioAlpha, annealBeta, rng, seg, mp, nullptr));
  g_dc.seg = seg;
  g_dc.mp = mp;
  g_dc.prioB = (long)mbSegs;
  g_dc.prio_fresh = true;
  *used = 1;
  return PH_OK;
}

extern "C" int ph_ffi_prio_sample(const double* advL1, size_t N, size_t T, size_t mbSegs, double prioAlpha,
                                  double annealBeta, uint64_t rng, double* idx, double* mbPrio) {
  (void)T;
  PH_REQUIRE(N > 0, "ph_ffi_prio_sample: N=0");
  if (mbSegs == 0) return PH_OK;
  PH_REQUIRE(advL1 && idx && mbPrio, "ph_ffi_prio_sample: null buffer");
  double *dL, *dI, *dM;
  int* dS;
  PH_TRY(carve(kHsPrioHost, [&](Carve& c) {
    dL = c.take<double>(N); dI = c.take<double>(mbSegs); dM = c.take<double>(mbSegs); dS = c.take<int>(mbSegs);
  }));
  PH_TRY(up(dL, advL1, N * 8));
  PH_TRY(prio_sample(dL, N, mbSegs, prioAlpha, annealBeta, rng, dS, dM, nullptr));
  k_i32_f64<<<ceil_div(mbSegs, kT), kT>>>(dS, dI, (long)mbSegs);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  PH_TRY(down(idx, dI, mbSegs * 8));
  return down(mbPrio, dM, mbSegs * 8);
}

extern "C" int ph_ffi_gather_seq_minibatch(const double* obsCol, const double* actCol, const double* logpCol,
                                           const double* termCol, const double* advFlat, const double* valueBuf,
                                           const double* segIdx, const double* mbPrio, size_t T, size_t Bmb,
                                           size_t D, size_t N, double* out) {
  (void)obsCol;
  (void)D;
  if (T * Bmb == 0) return PH_OK;
  PH_REQUIRE(N > 0 && N <= 0x7fffffffUL && Bmb <= 0x7fffffffUL, "ph_ffi_gather_seq_minibatch: N=%zu Bmb=%zu",
             N, Bmb);
  PH_REQUIRE(actCol && logpCol && termCol && advFlat && valueBuf && segIdx && mbPrio && out,
             "ph_ffi_gather_seq_minibatch: null buffer");
  PH_TRY(check_seg_host(segIdx, Bmb, N, "ph_ffi_gather_seq_minibatch"));
  const size_t n = N * T, nb = T * Bmb;
  double *dAct, *dLogp, *dTerm, *dAdv, *dVal, *dSegD, *dMp, *dOut;
  int* dSeg;
  PH_TRY(carve(kHsGather, [&](Carve& c) {
    dAct = c.take<double>(n); dLogp = c.take<double>(n); dTerm = c.take<double>(n); dAdv = c.take<double>(n);
    dVal = c.take<double>(n); dSegD = c.take<double>(Bmb); dMp = c.take<double>(Bmb);
    dOut = c.take<double>(6 * nb); dSeg = c.take<int>(Bmb);
  }));
  PH_TRY(up(dAct, actCol, n * 8)); PH_TRY(up(dLogp, logpCol, n * 8)); PH_TRY(up(dTerm, termCol, n * 8));
  PH_TRY(up(dAdv, advFlat, n * 8)); PH_TRY(up(dVal, valueBuf, n * 8)); PH_TRY(up(dSegD, segIdx, Bmb * 8));
  PH_TRY(up(dMp, mbPrio, Bmb * 8));
  k_f64_i32<<<ceil_div(Bmb, kT), kT>>>(dSegD, dSeg, (long)Bmb);
  PH_LAUNCH_CHECK();
  ph_replay_cols c{};
  c.dtype = PH_F64; c.time_major = 0; c.N = N; c.T = T; c.K = 1;
  c.adv = dAdv; c.value = dVal; c.act = dAct; c.logp = dLogp; c.term = dTerm;
  PH_TRY(mb_gather(c, dSeg, dMp, Bmb, dOut, nullptr, nullptr));
  PH_TRY(finish());
  return down(out, dOut, 6 * nb * 8);
}

// ---- MinGRU ---------------------------------------------------------------------------------------
// lean_cuda_mingru_ppo_grad (puffercuda.cu:5206) with the reference's two scalar sources: host scal,
// or the device-column mode (puffercuda.cu:5226-5240 mode choice; 5366-5383 gather; 5554-5558
// iterate). obs is always the host array: the resident obs trajectory belongs to a rollout, which
// this library does not run. Writes out[P + 2*T*B] = [summed gradient | new_logp | new_value].
extern "C" int ph_cuda_mingru_ppo_grad(const double* params, size_t nparams, const double* obs, size_t nobs,
                                       const double* scal, size_t nscal, size_t B, size_t T, size_t H, size_t D,
                                       size_t L, size_t A, size_t K, const double* hs, size_t nhs, double vfCoef,
                                       double entCoef, double clipEps, double vfClip, const double* segIdx,
                                       size_t nseg, const double* mbPrio, size_t nprio, double* out,
                                       size_t* out_len) {
  // K > 1: A is the logits width (the sum of the K head sizes in hs) and the action column is K wide
  // (puffercuda.cu:5202-5205, 5216-5220)
  const size_t Kh = K < 1 ? 1 : K;
  HeadSizes heads{};
  if (Kh > 1) {
    PH_REQUIRE(hs && nhs >= Kh, "ph_cuda_mingru_ppo_grad: %zu head sizes for K=%zu heads", nhs, Kh);
    size_t W = 0;
    PH_TRY(sizes_from(hs, Kh, heads.n, W, "ph_cuda_mingru_ppo_grad"));
    heads.K = (int)Kh;
    PH_REQUIRE(W == A, "ph_cuda_mingru_ppo_grad: head sizes sum to %zu, A=%zu", W, A);
  }
  const size_t TB = T * B, NS = (Kh + 5) * TB;  // scal: [act (K per row) | adv | ret | old | term | ov]
  int dev = -1;
  const bool prioRes = nseg == 0 && nprio == 0 && g_dc.prio_fresh && g_dc.prioB == (long)B;
  g_dc.prio_fresh = false;
  if (prioRes || (nseg > 0 && nprio > 0)) PH_CHECK_HIP(hipGetDevice(&dev));
  // a K-wide action column is gathered only from resident columns of the same width
  const bool devCol = (prioRes || (nseg > 0 && nprio > 0)) && g_dc.valid && g_dc.T == (long)T &&
                      g_dc.K == (long)Kh && g_dc.dev == dev;
  PH_REQUIRE(devCol || nscal >= NS,
             "ph_cuda_mingru_ppo_grad: no scalar source: scal holds %zu of %zu values and the device-column "
             "mode is off (needs segIdx+mbPrio or a fresh ph_cuda_mg_vtrace_prio draw, and resident columns "
             "for T=%zu, K=%zu)", nscal, NS, T, Kh);
  // empty obs: gather the minibatch from the resident obs trajectory by the drawn segments
  // (puffercuda.cu:5226-5230, 5362-5363), which needs segment indices and a trajectory of these shapes
  const bool useTraj = nobs == 0 && devCol && g_traj.valid && g_traj.dev == dev && g_traj.N == g_dc.N &&
                       g_traj.T == (long)T && g_traj.D == (long)D;
  PH_REQUIRE(useTraj || nobs >= TB * D,
             "ph_cuda_mingru_ppo_grad: obs holds %zu of %zu values and no resident obs trajectory matches "
             "(the device-column mode with a ph_cuda_mg_obs_traj trajectory of N=%ld segments, T=%zu, D=%zu)",
             nobs, TB * D, g_dc.N, T, D);
  PH_REQUIRE((useTraj || obs) && out && out_len && (devCol || scal), "ph_cuda_mingru_ppo_grad: null buffer");
  if (devCol && !prioRes) {
    PH_REQUIRE(nseg >= B && nprio >= B && segIdx && mbPrio,
               "ph_cuda_mingru_ppo_grad: segIdx/mbPrio hold %zu/%zu of %zu draws", nseg, nprio, B);
    PH_TRY(check_seg_host(segIdx, B, (size_t)g_dc.N, "ph_cuda_mingru_ppo_grad"));
  }
  ph_mingru_dims d{(int)B, (int)T, (int)D, (int)H, (int)L, (int)A, env_is("PUFFER_MG_PREC", "bf16") ? 0 : 1};
  const long P = mingru_param_count(d);
  // empty params: the weights the last resident Muon step left on the device (its policy handle)
  if (nparams == 0) {
    if (dev < 0) PH_CHECK_HIP(hipGetDevice(&dev));
    PH_REQUIRE(g_mgw.valid && g_mgw.P == P && g_mgw.dev == dev,
               "ph_cuda_mingru_ppo_grad: empty params but no resident weights of P=%ld on this device (the "
               "resident Muon leaves them; a policy handle freed since then drops them)", P);
  } else {
    PH_REQUIRE(params && nparams >= (size_t)P, "ph_cuda_mingru_ppo_grad: params hold %zu of P=%ld values",
               nparams, P);
  }
  ph_ppo_coefs c{};
  c.vf_coef = vfCoef; c.ent_coef = entCoef; c.clip_eps = clipEps; c.vf_clip = vfClip;
  double *dp, *dx, *ds, *losses, *segd, *mpd;
  float *pf, *xf, *sf, *G, *nlp, *nv;
  int *act, *segi;
  PH_TRY(carve(kHsMg, [&](Carve& cv) {
    dp = cv.take<double>(P); dx = cv.take<double>(TB * D); ds = cv.take<double>(NS);
    losses = cv.take<double>(8); pf = cv.take<float>(P); xf = cv.take<float>(TB * D);
    sf = cv.take<float>(NS); G = cv.take<float>(P); nlp = cv.take<float>(TB); nv = cv.take<float>(TB);
    act = cv.take<int>(Kh * TB); segd = cv.take<double>(B); mpd = cv.take<double>(B); segi = cv.take<int>(B);
  }));
  if (nparams) PH_TRY(up(dp, params, P * 8));
  if (!useTraj) PH_TRY(up(dx, obs, TB * D * 8));
  const int* seg = nullptr;
  if (devCol) {
    const double* mp = nullptr;
    if (prioRes) {
      seg = g_dc.seg;
      mp = g_dc.mp;
    } else {
      PH_TRY(up(segd, segIdx, B * 8)); PH_TRY(up(mpd, mbPrio, B * 8));
      k_f64_i32<<<ceil_div(B, kT), kT>>>(segd, segi, (long)B);
      PH_LAUNCH_CHECK();
      seg = segi;
      mp = mpd;
    }
    const ph_replay_cols cols = dc_cols();
    PH_TRY(mb_gather(cols, seg, mp, B, ds, nullptr, nullptr));
  } else {
    PH_TRY(up(ds, scal, NS * 8));
  }
  PH_TRY(to_f32(nparams ? dp : (const double*)g_mgw.handle, pf, P, nullptr));
  if (useTraj) {
    k_gather_obs_traj<<<ceil_div(TB * D, kT), kT>>>(g_traj.obs, seg, (long)B, (long)T, (long)D, xf);
    PH_LAUNCH_CHECK();
  } else {
    PH_TRY(to_f32(dx, xf, (long)(TB * D), nullptr));
  }
  PH_TRY(to_f32(ds, sf, (long)NS, nullptr));
  k_f64_i32<<<ceil_div(Kh * TB, kT), kT>>>(ds, act, (long)(Kh * TB));
  PH_LAUNCH_CHECK();
  const float* sc = sf + Kh * TB;  // adv | ret | old | term | ov
  if (Kh > 1)
    PH_TRY(ph_mingru_ppo_grad_md(&d, &c, heads.n, Kh, pf, xf, act, sc, sc + TB, sc + 2 * TB, sc + 4 * TB,
                                 sc + 3 * TB, G, nlp, nv, g_mgLossOn ? losses : nullptr, nullptr));
  else
    PH_TRY(ph_mingru_ppo_grad(&d, &c, pf, xf, act, sc, sc + TB, sc + 2 * TB, sc + 4 * TB, sc + 3 * TB, G, nlp, nv,
                              g_mgLossOn ? losses : nullptr, nullptr));
  if (devCol) {
    const ph_replay_cols cols = dc_cols();
    PH_TRY(mb_iterate(cols, seg, B, nlp, nv, nullptr));
    // resident mode (the reference's size-0 return): the summed gradient stays on the device for the
    // resident Muon, nothing is copied back and nothing waits; host mode only if that buffer cannot be had
    double* gres = (double*)scratch(kHsGradRes, P * 8);
    if (gres) {
      k_f32_f64<<<ceil_div(P, kT), kT>>>(G, gres, P, 1.0);
      PH_LAUNCH_CHECK();
      g_mgg.fresh = true;
      g_mgg.dev = dev;
      g_mgg.P = P;
      *out_len = 0;
      if (g_mgLossOn) {
        PH_TRY(finish());
        PH_TRY(down(g_mgLoss, losses, 7 * 8));
      }
      return PH_OK;
    }
    (void)hipGetLastError();
  }
  double* o = (double*)scratch(kHsMgOut, (P + 2 * TB) * 8);
  if (!o) return PH_ERR_NOMEM;
  k_f32_f64<<<ceil_div(P, kT), kT>>>(G, o, P, 1.0);
  k_f32_f64<<<ceil_div(TB, kT), kT>>>(nlp, o + P, (long)TB, 1.0);
  k_f32_f64<<<ceil_div(TB, kT), kT>>>(nv, o + P + TB, (long)TB, 1.0);
  PH_LAUNCH_CHECK();
  PH_TRY(finish());
  if (g_mgLossOn) PH_TRY(down(g_mgLoss, losses, 7 * 8));
  *out_len = (size_t)P + 2 * TB;
  return down(out, o, (P + 2 * TB) * 8);
}

extern "C" int ph_cuda_mg_resident_grad(size_t P, double* out) {
  int dev = -1;
  PH_CHECK_HIP(hipGetDevice(&dev));
  PH_REQUIRE(out && g_mgg.fresh && g_mgg.P == (long)P && g_mgg.dev == dev,
             "ph_cuda_mg_resident_grad: no unconsumed resident gradient of P=%zu", P);
  double* gres = (double*)scratch_peek(kHsGradRes);
  PH_REQUIRE(gres, "ph_cuda_mg_resident_grad: resident gradient buffer missing");
  PH_TRY(finish());
  return down(out, gres, P * 8);
}

// Host-gradient mode of lean_cuda_mingru_muon_resident (puffercuda.cu:5727): the clipped gradient
// gClip[P] is uploaded and every flattenMG matrix takes a Muon step on the resident [weights; mom]
// (fp32-MFMA Newton-Schulz with f64 state; PUFFER_MUON_EXACT=1 selects the exact f64 tier), every
// bias a Nesterov stepvec; writes the new weights (P). The resident-gradient mode (empty gClip) is
// not provided.
extern "C" int ph_cuda_mingru_muon_resident(size_t policyH, const double* gClip, size_t nG, size_t H, size_t D,
                                            size_t L, size_t A, double lr, double wd, double mu, double eps,
                                            double maxGradNorm, double gscale, double* wOut, size_t* wOut_len) {
  PH_REQUIRE(policyH != 0, "ph_cuda_mingru_muon_resident: no policy handle");
  const size_t szE = H * D, szL = 3 * H * H;
  const size_t P = szE + H + L * szL + A * H + A + H + 1;
  PH_REQUIRE(wOut_len, "ph_cuda_mingru_muon_resident: null output length");
  int dev = -1;
  PH_CHECK_HIP(hipGetDevice(&dev));
  // empty gClip: consume the gradient the last MinGRU gradient call left on the device, clipped here
  // (k_gclip_norm / k_gclip_scale, puffercuda.cu:5122-5131); the stamp is consumed by this step
  const bool gres = nG == 0 && g_mgg.fresh && g_mgg.P == (long)P && g_mgg.dev == dev;
  if (nG == 0) g_mgg.fresh = false;
  PH_REQUIRE(nG > 0 || gres,
             "ph_cuda_mingru_muon_resident: empty gClip but no resident gradient of P=%zu is present (the "
             "MinGRU gradient leaves one only in its device-column mode)", P);
  PH_REQUIRE(gres || (gClip && nG >= P), "ph_cuda_mingru_muon_resident: gClip holds %zu of P=%zu values", nG,
             P);
  PH_REQUIRE(gres || wOut, "ph_cuda_mingru_muon_resident: null output");
  const bool mixed = !env_is("PUFFER_MUON_EXACT", "1");
  double* W = (double*)policyH;
  double* M = W + P;
  double* G;
  if (gres) {
    G = (double*)scratch_peek(kHsGradRes);
    PH_REQUIRE(G, "ph_cuda_mingru_muon_resident: resident gradient buffer missing");
    PH_TRY(gclip_f64(G, (long)P, gscale, maxGradNorm, nullptr));
  } else {
    G = (double*)scratch(kHsGrad, P * 8);
    if (!G) return PH_ERR_NOMEM;
    PH_TRY(up(G, gClip, P * 8));
  }
  const size_t offW = szE + H, offDec = offW + L * szL, offBDec = offDec + A * H, offVal = offBDec + A,
               offBVal = offVal + H;
  PH_TRY(muon_f64((int)H, (int)D, W, G, M, 1.0, lr, wd, mu, eps, mixed, nullptr));
  PH_TRY(stepvec_f64((long)H, W + szE, G + szE, M + szE, 1.0, lr, wd, mu, nullptr));
  for (size_t l = 0; l < L; l++)
    PH_TRY(muon_f64((int)(3 * H), (int)H, W + offW + l * szL, G + offW + l * szL, M + offW + l * szL, 1.0, lr,
                    wd, mu, eps, mixed, nullptr));
  PH_TRY(muon_f64((int)A, (int)H, W + offDec, G + offDec, M + offDec, 1.0, lr, wd, mu, eps, mixed, nullptr));
  PH_TRY(stepvec_f64((long)A, W + offBDec, G + offBDec, M + offBDec, 1.0, lr, wd, mu, nullptr));
  PH_TRY(muon_f64(1, (int)H, W + offVal, G + offVal, M + offVal, 1.0, lr, wd, mu, eps, mixed, nullptr));
  PH_TRY(stepvec_f64(1, W + offBVal, G + offBVal, M + offBVal, 1.0, lr, wd, mu, nullptr));
  // the next gradient may take these weights from the handle (empty params)
  g_mgw.valid = true;
  g_mgw.dev = dev;
  g_mgw.P = (long)P;
  g_mgw.handle = policyH;
  if (gres) {  // resident form: nothing copied back, nothing waited for (the reference's empty return)
    PH_LAUNCH_CHECK();
    *wOut_len = 0;
    return PH_OK;
  }
  PH_TRY(finish());
  *wOut_len = P;
  return down(wOut, W, P * 8);
}
