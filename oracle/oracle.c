/* CPU oracle for the pufferlean training-step hot path — TEST INFRASTRUCTURE, not product code.
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as the
 * checker or the timed CPU baseline. Built with -ffp-contract=off so every expression below executes
 * in the order written (the reference builds its CPU path the same way, lakefile.lean:138-160).
 *
 * Each function restates a reference CPU routine and cites it. Where the op order must be identical
 * for a bit-exact comparison (V-trace scans, GAE, the naive NS matmuls, the two-level Frobenius fold)
 * the order is kept; everything else is written from the formulas.
 *
 * Pinning (the checks in tests/test_oracle.py that each function must pass):
 *   orc_rng_next / orc_randf     known-answer splitmix64 words (published test vectors of splitmix64 for
 *                                seed 0; Train.lean:18-28 is that algorithm)
 *   orc_vtrace_vec               GAE identity at imp=1 vs orc_gae_soa (bit-exact); all-done closed form;
 *                                gamma=0 closed form; brute-force sum-of-discounted-deltas on tiny B,T
 *   orc_vtrace_mingru            same invariants with bootstrap; rho=c=1 no-clamp reduces to
 *                                orc_gae_boot_norm's pre-normalisation recurrence
 *   orc_vtrace_f64 / _f32        equals the two functions above on their layouts; f32 twin within
 *                                1e-5 of f64; time-major == transposed segment-major
 *   orc_gae_soa / gae_boot_norm  closed-form per-step expansion on tiny inputs
 *   orc_adv_normalize            mean 0 / pop-std 1 closed form
 *   orc_ppo_grad                 central finite differences of the PPO objective (orc_ppo_objective
 *                                below, a separate forward-only function); uniform-logit special case
 *   orc_ppo_losses               hand-computed two-row case
 *   orc_gemm                     numpy matmul on all four transpose forms
 *   orc_mlp_ppo_grad             finite differences of the summed objective through the MLP
 *   orc_mlp_deep_ppo_grad        L = 1 equals orc_mlp_ppo_grad bit for bit; L = 2, 3 (with and without
 *                                the value clip) against central finite differences of an
 *                                independently written numpy objective
 *   orc_newton_schulz            scaled-orthogonal input closed form (scalar quintic); diagonal input
 *                                closed form; form 0 vs form 1 within roundoff; tall/wide transpose
 *   orc_muon_mat / stepvec       closed form on diagonal inputs; mlp wrapper == per-tensor calls
 *   orc_gclip                    closed form
 *   orc_mingru_ppo_grad_seq      finite differences of its own forward objective (orc_mingru_objective)
 *   orc_mingru_ppo_grad_seq_md   two heads equal one categorical head over the product space (decoder
 *                                rows W1[i] + W2[j]): identical shared-layer gradients, head gradients
 *                                the product's summed over the other head; K = 1 equals the categorical
 *   orc_mingru_heinsen           equals the sequential recurrence within roundoff
 *   orc_seg_l1                   exact on dyadic inputs (every summation order gives the same bits);
 *                                numpy row sums of |adv| within roundoff
 *   orc_prio_sample              draws equal numpy searchsorted (side left, the Python reference's
 *                                tools/puffer_ref.py:157) and the first-hit linear scan of
 *                                weightedSampleReplace (VecTrain.lean:147-165) on the pinned splitmix64
 *                                words; probabilities and weights equal the numpy power forms
 *                                (tools/puffer_ref.py:151-159) within roundoff; uniform-L1 closed form
 *                                idx = floor(u*N); empirical draw frequencies match the probabilities
 *   orc_gather_seq_minibatch     numpy fancy-index construction of the six columns (exact), numpy mean
 *                                and population std; exact mean/std closed form on dyadic inputs
 *   orc_mb_iterate               a dictionary of last assignments per segment (exact)
 *   orc_sample_actions           numpy softmax + inverse-CDF on the pinned splitmix64 words; uniform-logit
 *                                closed form a = floor(u*A); draw frequencies against the softmax
 *   orc_mingru_step              T chained steps from a zero state equal orc_mingru_ppo_grad_seq's
 *                                new values and new log-probs (a separately pinned function)
 *   orc_ppo_grad_md / _cont      central finite differences of independently written numpy objectives
 *                                (joint clipped surrogate, value loss, entropy); K = 1 equals
 *                                orc_ppo_grad; the clamp mask zeroes saturated log-stds
 *   orc_sample_md / _cont        numpy inverse-CDF / Box-Muller on the pinned splitmix64 words; Gaussian
 *                                draw moments; K = 1 logp equals log softmax
 *   timed CPU baselines          orc_vtrace_f32_mt equals orc_vtrace_f32 bit for bit; orc_gemm_blocked
 *                                equals numpy matmul within roundoff; orc_mingru_ppo_grad_batch equals
 *                                the sum of orc_mingru_ppo_grad_seq over its segments; threaded
 *                                Newton-Schulz (orc_set_threads) equals the serial one bit for bit
 *   orc_wide_losses              mode 1 with K = 1 equals orc_ppo_losses; two heads equal one head over
 *                                the product space; mode 2 logp and entropy against scipy's normal
 *                                logpdf / entropy; special cases (adv 0, ratio 1, no value clip)
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define M_PI_ORACLE 3.14159265358979323846
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ */
/* splitmix64 (Puffer/RL/Train.lean:18-28): the state advances by the golden gamma, the word is the
 * finaliser of the advanced state. uniform01 keeps the top 53 bits (Train.lean:27-28). */
uint64_t orc_rng_next(uint64_t* state) {
  uint64_t s = *state + 0x9E3779B97F4A7C15ULL;
  *state = s;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

double orc_uniform01(uint64_t word) { return (double)(word >> 11) / 9007199254740992.0; }

/* randF (Exe/Puffer.lean:65-67): lo + (hi-lo)*u. */
void orc_randf(double* out, size_t n, double lo, double hi, uint64_t* state) {
  for (size_t i = 0; i < n; i++) out[i] = lo + (hi - lo) * orc_uniform01(orc_rng_next(state));
}

/* ------------------------------------------------------------------------------------------------ */
static inline double clamp1(double r) { return r > 1.0 ? 1.0 : (r < -1.0 ? -1.0 : r); }
static inline float clamp1f(float r) { return r > 1.0f ? 1.0f : (r < -1.0f ? -1.0f : r); }

/* vec-form V-trace (puffercuda.cu:120-132, VecTrain.lean:98-114). Per segment the last step keeps
 * advantage 0; for t = T-2 .. 0 the TD error is scaled by the clipped ratio as a whole. */
void orc_vtrace_vec(const double* rew, const double* val, const double* term, const double* imp,
                    size_t B, size_t T, double gamma, double lam, double rhoClip, double cClip,
                    double* adv) {
  for (size_t b = 0; b < B; b++) {
    const double* r_ = rew + b * T; const double* v_ = val + b * T;
    const double* d_ = term + b * T; const double* i_ = imp + b * T;
    double* a_ = adv + b * T;
    if (T == 0) continue;
    a_[T - 1] = 0.0;
    double last = 0.0;
    for (size_t k = 1; k < T; k++) {
      size_t t = T - 1 - k;
      double nnt = (d_[t] != 0.0) ? 0.0 : 1.0;
      double w = i_[t];
      double rho = w < rhoClip ? w : rhoClip;
      double c = w < cClip ? w : cClip;
      double r = clamp1(r_[t]);
      double delta = rho * (r + gamma * v_[t + 1] * nnt - v_[t]);
      last = delta + gamma * lam * c * last * nnt;
      a_[t] = last;
    }
  }
}

/* bootstrapped MinGRU-form V-trace (puffercuda.cu:200-211, VecTrain.lean:122-139): the clipped
 * ratio scales the reward only, V(s_T) comes from bootv, terminal means term > 0.5. */
void orc_vtrace_mingru(const double* rew, const double* val, const double* term, const double* imp,
                       const double* bootv, size_t B, size_t T, double gamma, double lam,
                       double rhoClip, double cClip, double* adv) {
  for (size_t b = 0; b < B; b++) {
    const double* r_ = rew + b * T; const double* v_ = val + b * T;
    const double* d_ = term + b * T; const double* i_ = imp + b * T;
    double* a_ = adv + b * T;
    double last = 0.0;
    for (size_t k = 0; k < T; k++) {
      size_t t = T - 1 - k;
      double nnt = (d_[t] > 0.5) ? 0.0 : 1.0;
      double vnext = (t + 1 < T) ? v_[t + 1] : bootv[b];
      double w = i_[t];
      double rho = w < rhoClip ? w : rhoClip;
      double c = w < cClip ? w : cClip;
      double r = clamp1(r_[t]);
      double delta = rho * r + gamma * vnext * nnt - v_[t];
      last = delta + gamma * lam * c * last * nnt;
      a_[t] = last;
    }
  }
}

/* GAE without bootstrap (pufferffi.c:946-971). */
void orc_gae_soa(const double* vals, const double* rews, const double* terms, size_t N, size_t T,
                 double gamma, double lam, double* out) {
  size_t NT = N * T;
  double* adv = out; double* ret = out + NT;
  for (size_t e = 0; e < N; e++) {
    size_t base = e * T;
    if (T >= 1) adv[base + T - 1] = 0.0;
    double last = 0.0;
    for (size_t k = 1; k < T; k++) {
      size_t t = base + T - 1 - k;
      double nnt = (terms[t] != 0.0) ? 0.0 : 1.0;
      double r = clamp1(rews[t]);
      double delta = r + gamma * vals[t + 1] * nnt - vals[t];
      last = delta + gamma * lam * last * nnt;
      adv[t] = last;
    }
  }
  for (size_t i = 0; i < NT; i++) ret[i] = adv[i] + vals[i];
}

/* GAE with bootstrap, time-major, then global advantage normalisation (pufferffi.c:980-1010). */
void orc_gae_boot_norm(const double* vals, const double* rews, const double* terms,
                       const double* bootv, size_t N, size_t T, double gamma, double lam,
                       double* out) {
  size_t NT = N * T;
  double* adv = out; double* ret = out + NT;
  for (size_t n = 0; n < N; n++) {
    double last = 0.0;
    for (size_t k = 0; k < T; k++) {
      size_t t = T - 1 - k, idx = t * N + n;
      double nnt = (terms[idx] > 0.5) ? 0.0 : 1.0;
      double vnext = (t + 1 < T) ? vals[(t + 1) * N + n] : bootv[n];
      double delta = rews[idx] + gamma * vnext * nnt - vals[idx];
      last = delta + gamma * lam * nnt * last;
      adv[idx] = last;
      ret[idx] = last + vals[idx];
    }
  }
  size_t den = NT > 0 ? NT : 1;
  double sum = 0.0;
  for (size_t i = 0; i < NT; i++) sum += adv[i];
  double mean = sum / (double)den;
  double vs = 0.0;
  for (size_t i = 0; i < NT; i++) { double d = adv[i] - mean; vs += d * d; }
  double inv = 1.0 / (sqrt(vs / (double)den) + 1e-8);
  for (size_t i = 0; i < NT; i++) adv[i] = (adv[i] - mean) * inv;
}

/* General form: one body per precision, identical op order to the two reference variants above. */
#define VTRACE_BODY(REAL, CLAMP, EXP)                                                              \
  for (size_t b = 0; b < B; b++) {                                                                 \
    REAL last = 0;                                                                                 \
    size_t t0;                                                                                     \
    if (variant == 0) {                                                                            \
      if (T == 0) continue;                                                                        \
      size_t il = time_major ? (T - 1) * B + b : b * T + T - 1;                                    \
      adv[il] = 0;                                                                                 \
      if (tgt) tgt[il] = adv[il] + val[il];                                                        \
      t0 = T - 1;                                                                                  \
    } else {                                                                                       \
      t0 = T;                                                                                      \
    }                                                                                              \
    for (size_t k = 0; k < t0; k++) {                                                              \
      size_t t = t0 - 1 - k;                                                                       \
      size_t i = time_major ? t * B + b : b * T + t;                                               \
      size_t in = time_major ? (t + 1) * B + b : b * T + t + 1;                                    \
      REAL w = rho_is_log ? EXP(rho[i]) : rho[i];                                                  \
      REAL rh = w < rhoClip ? w : rhoClip;                                                         \
      REAL c = w < cClip ? w : cClip;                                                              \
      REAL r = clamp ? CLAMP(rew[i]) : rew[i];                                                     \
      REAL delta;                                                                                  \
      REAL nnt;                                                                                    \
      if (variant == 0) {                                                                          \
        nnt = (term[i] != 0) ? (REAL)0 : (REAL)1;                                                  \
        delta = rh * (r + gamma * val[in] * nnt - val[i]);                                         \
      } else {                                                                                     \
        nnt = (term[i] > (REAL)0.5) ? (REAL)0 : (REAL)1;                                           \
        REAL vnext = (t + 1 < T) ? val[in] : boot[b];                                              \
        delta = rh * r + gamma * vnext * nnt - val[i];                                             \
      }                                                                                            \
      last = delta + gamma * lam * c * last * nnt;                                                 \
      adv[i] = last;                                                                               \
      if (tgt) tgt[i] = last + val[i];                                                             \
    }                                                                                              \
  }

void orc_vtrace_f64(const double* rew, const double* val, const double* term, const double* rho,
                    const double* boot, size_t B, size_t T, int variant, int time_major,
                    int rho_is_log, int clamp, double gamma, double lam, double rhoClip,
                    double cClip, double* adv, double* tgt) {
  VTRACE_BODY(double, clamp1, exp)
}

void orc_vtrace_f32(const float* rew, const float* val, const float* term, const float* rho,
                    const float* boot, size_t B, size_t T, int variant, int time_major,
                    int rho_is_log, int clamp, float gamma, float lam, float rhoClip, float cClip,
                    float* adv, float* tgt) {
  VTRACE_BODY(float, clamp1f, expf)
}

/* ------------------------------------------------------------------------------------------------ */
/* normalizeAdv (NNTrain.lean:274-279): sequential folds for mean and population variance, epsilon
 * added to the standard deviation. */
void orc_adv_normalize(const double* adv, size_t n, double* out) {
  double s = 0.0;
  for (size_t i = 0; i < n; i++) s = s + adv[i];
  double mean = s / (double)n;
  double v = 0.0;
  for (size_t i = 0; i < n; i++) { double d = adv[i] - mean; v = v + d * d; }
  double den = sqrt(v / (double)n) + 1e-8;
  for (size_t i = 0; i < n; i++) out[i] = (adv[i] - mean) / den;
}

/* ------------------------------------------------------------------------------------------------ */
/* d(value loss)/dv for PufferLib's clipped value loss (puffercuda.cu:692-700; pufferffi.c:853). */
static double vloss_grad(double vnew, double ret, const double* ov, size_t i, double vfClip) {
  if (vfClip <= 0.0 || !ov) return vnew - ret;
  double vold = ov[i], dd = vnew - vold;
  double vc = vold + (dd < -vfClip ? -vfClip : (dd > vfClip ? vfClip : dd));
  double du = (vnew - ret) * (vnew - ret), cc = (vc - ret) * (vc - ret);
  if (du >= cc) return vnew - ret;
  if (dd > -vfClip && dd < vfClip) return vnew - ret;
  return 0.0;
}

/* Per-row PPO objective gradient (pufferblas.c:726-736 with the value clip of puffercuda.cu:692-700;
 * max-shifted log-sum-exp as in puffercuda.cu:4914-4916 when max_shift). */
void orc_ppo_grad(const double* logits, size_t ldl, const double* values, size_t ldv,
                  const double* act, const double* adv, const double* ret, const double* old,
                  const double* ov, size_t N, size_t A, double vfCoef, double entCoef,
                  double clipEps, double vfClip, int max_shift, double* dlogits, size_t ldd,
                  double* dvalues, size_t lddv, double* newlp, double* newval) {
  double* pk = (double*)malloc(sizeof(double) * (A ? A : 1));
  for (size_t n = 0; n < N; n++) {
    const double* lg = logits + n * ldl;
    double lse;
    if (max_shift) {
      double mx = lg[0];
      for (size_t k = 1; k < A; k++) if (lg[k] > mx) mx = lg[k];
      double se = 0.0;
      for (size_t k = 0; k < A; k++) se += exp(lg[k] - mx);
      lse = mx + log(se);
    } else {
      double se = 0.0;
      for (size_t k = 0; k < A; k++) se += exp(lg[k]);
      lse = log(se);
    }
    double pout = 0.0;
    for (size_t k = 0; k < A; k++) { pk[k] = exp(lg[k] - lse); pout += pk[k] * lg[k]; }
    size_t a = (size_t)act[n];
    double logpA = lg[a] - lse;
    double ratio = exp(logpA - old[n]);
    double lo = 1.0 - clipEps, hi = 1.0 + clipEps;
    double rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    double s1 = adv[n] * ratio, s2 = adv[n] * rc;
    double dpol;
    if (s1 <= s2) dpol = adv[n] * ratio;
    else dpol = adv[n] * ((lo < ratio && ratio < hi) ? 1.0 : 0.0) * ratio;
    double* dl = dlogits + n * ldd;
    for (size_t k = 0; k < A; k++)
      dl[k] = dpol * ((k == a ? 1.0 : 0.0) - pk[k]) + entCoef * pk[k] * (pout - lg[k]);
    double v = values[n * ldv];
    dvalues[n * lddv] = -vfCoef * vloss_grad(v, ret[n], ov, n, vfClip);
    if (newlp) newlp[n] = logpA;
    if (newval) newval[n] = v;
  }
  free(pk);
}

/* Dashboard losses (puffercuda.cu:5453-5478): pg = mean max(-adv*r, -adv*clip(r)); v = mean
 * 0.5*max-branch value loss; ent = mean entropy; total = pg + vf*v - ent_coef*ent; old_kl =
 * mean(-logratio); kl = mean((r-1) - logratio); clipfrac = mean(r outside [1-eps, 1+eps]). */
void orc_ppo_losses(const double* logits, size_t ldl, const double* values, size_t ldv,
                    const double* act, const double* adv, const double* ret, const double* old,
                    const double* ov, size_t N, size_t A, double vfCoef, double entCoef,
                    double clipEps, double vfClip, double* L) {
  double lo = 1.0 - clipEps, hi = 1.0 + clipEps;
  double sPg = 0, sV = 0, sEnt = 0, sKL = 0, sOld = 0;
  size_t nclip = 0;
  for (size_t n = 0; n < N; n++) {
    const double* lg = logits + n * ldl;
    double mx = lg[0];
    for (size_t k = 1; k < A; k++) if (lg[k] > mx) mx = lg[k];
    double se = 0;
    for (size_t k = 0; k < A; k++) se += exp(lg[k] - mx);
    double lse = mx + log(se);
    double lr = (lg[(size_t)act[n]] - lse) - old[n];
    double ratio = exp(lr), rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    double p1 = -adv[n] * ratio, p2 = -adv[n] * rc;
    sPg += p1 > p2 ? p1 : p2;
    if (ratio < lo || ratio > hi) nclip++;
    sKL += (ratio - 1.0) - lr;
    sOld += -lr;
    double vnew = values[n * ldv];
    double du = (vnew - ret[n]) * (vnew - ret[n]);
    double vl = du;
    if (vfClip > 0.0 && ov) {
      double dd = vnew - ov[n];
      double vc = ov[n] + (dd < -vfClip ? -vfClip : (dd > vfClip ? vfClip : dd));
      double cc = (vc - ret[n]) * (vc - ret[n]);
      if (cc > du) vl = cc;
    }
    sV += 0.5 * vl;
    for (size_t k = 0; k < A; k++) { double lp = lg[k] - lse; sEnt -= exp(lp) * lp; }
  }
  double dn = (double)N;
  L[0] = sPg / dn; L[1] = sV / dn; L[2] = sEnt / dn;
  L[3] = L[0] + vfCoef * L[1] - entCoef * L[2];
  L[4] = sOld / dn; L[5] = sKL / dn; L[6] = (double)nclip / dn;
}

/* ------------------------------------------------------------------------------------------------ */
/* Row-major GEMM with cblas semantics. Inner loop over j with op(B) rows contiguous when possible;
 * OpenMP over output rows (the reference's CPU GEMMs are multithreaded OpenBLAS). */
void orc_gemm(int transA, int transB, size_t M, size_t N, size_t K, double alpha, const double* A,
              size_t lda, const double* B, size_t ldb, double beta, double* C, size_t ldc,
              int threads) {
#ifdef _OPENMP
  int nt = threads > 1 ? threads : 1;
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
  for (long i = 0; i < (long)M; i++) {
    double* c = C + (size_t)i * ldc;
    double* acc = (double*)calloc(N ? N : 1, sizeof(double));
    for (size_t k = 0; k < K; k++) {
      double a = transA ? A[k * lda + (size_t)i] : A[(size_t)i * lda + k];
      if (a == 0.0) continue;
      if (!transB) {
        const double* br = B + k * ldb;
        for (size_t j = 0; j < N; j++) acc[j] += a * br[j];
      } else {
        for (size_t j = 0; j < N; j++) acc[j] += a * B[j * ldb + k];
      }
    }
    for (size_t j = 0; j < N; j++) c[j] = (beta == 0.0 ? 0.0 : beta * c[j]) + alpha * acc[j];
    free(acc);
  }
  (void)threads;
}

/* ------------------------------------------------------------------------------------------------ */
/* relu(X W^T + b) (pufferblas.c:65-97). */
void orc_dense_forward(const double* X, const double* W, const double* b, size_t N, size_t D,
                       size_t H, double* Y) {
  orc_gemm(0, 1, N, H, D, 1.0, X, D, W, D, 0.0, Y, H, 1);
  for (size_t i = 0; i < N; i++)
    for (size_t j = 0; j < H; j++) { double v = Y[i * H + j] + b[j]; Y[i * H + j] = v > 0.0 ? v : 0.0; }
}

/* Two-layer MLP forward over [W1|b1|W2|b2] (pufferblas.c:670-690). */
void orc_mlp_forward(const double* p, const double* X, size_t N, size_t D, size_t H, size_t O,
                     double* Y) {
  const double* W1 = p; const double* b1 = W1 + H * D; const double* W2 = b1 + H; const double* b2 = W2 + O * H;
  double* Z = (double*)malloc(sizeof(double) * N * H);
  orc_dense_forward(X, W1, b1, N, D, H, Z);
  orc_gemm(0, 1, N, O, H, 1.0, Z, H, W2, H, 0.0, Y, O, 1);
  for (size_t n = 0; n < N; n++) for (size_t k = 0; k < O; k++) Y[n * O + k] += b2[k];
  free(Z);
}

/* Summed PPO gradient of the one-hidden-layer MLP over the minibatch (pufferblas.c:699-747).
 * g = [gW1(H*D) | gb1(H) | gW2(O*H) | gb2(O)], O = A+1, value in output column A. */
void orc_mlp_ppo_grad(const double* p, const double* obs, const double* act, const double* adv,
                      const double* ret, const double* old, size_t N, size_t H, size_t D, size_t A,
                      double vfCoef, double entCoef, double clipEps, double* g, int threads) {
  size_t O = A + 1, P = H * D + H + O * H + O;
  const double* W1 = p; const double* b1 = W1 + H * D; const double* W2 = b1 + H; const double* b2 = W2 + O * H;
  for (size_t i = 0; i < P; i++) g[i] = 0.0;
  double* gW1 = g; double* gb1 = gW1 + H * D; double* gW2 = gb1 + H; double* gb2 = gW2 + O * H;
  double* H1 = (double*)malloc(sizeof(double) * N * H);
  double* Out = (double*)malloc(sizeof(double) * N * O);
  double* dOut = (double*)malloc(sizeof(double) * N * O);
  double* dH1 = (double*)malloc(sizeof(double) * N * H);
  orc_gemm(0, 1, N, H, D, 1.0, obs, D, W1, D, 0.0, H1, H, threads);
  for (size_t n = 0; n < N; n++)
    for (size_t j = 0; j < H; j++) { double v = H1[n * H + j] + b1[j]; H1[n * H + j] = v > 0.0 ? v : 0.0; }
  orc_gemm(0, 1, N, O, H, 1.0, H1, H, W2, H, 0.0, Out, O, threads);
  for (size_t n = 0; n < N; n++) for (size_t k = 0; k < O; k++) Out[n * O + k] += b2[k];
  orc_ppo_grad(Out, O, Out + A, O, act, adv, ret, old, NULL, N, A, vfCoef, entCoef, clipEps, 0.0, 0,
               dOut, O, dOut + A, O, NULL, NULL);
  for (size_t n = 0; n < N; n++) for (size_t k = 0; k < O; k++) gb2[k] += dOut[n * O + k];
  orc_gemm(1, 0, O, H, N, 1.0, dOut, O, H1, H, 0.0, gW2, H, threads);
  orc_gemm(0, 0, N, H, O, 1.0, dOut, O, W2, H, 0.0, dH1, H, threads);
  for (size_t n = 0; n < N; n++)
    for (size_t j = 0; j < H; j++) if (!(H1[n * H + j] > 0.0)) dH1[n * H + j] = 0.0;
  for (size_t n = 0; n < N; n++) for (size_t j = 0; j < H; j++) gb1[j] += dH1[n * H + j];
  orc_gemm(1, 0, H, D, N, 1.0, dH1, H, obs, D, 0.0, gW1, D, threads);
  free(H1); free(Out); free(dOut); free(dH1);
}

/* The same gradient for L >= 1 hidden ReLU layers of width H and the combined head (pufferblas.c:699-747
 * with its one hidden layer repeated): p = [W1(H*D) | b1(H) | W2(H*H) | b2(H) | ... | WL | bL |
 * Wo(O*H) | bo(O)], O = A+1, value in output column A. ov (may be NULL) and vfClip select the clipped
 * value loss. newlp/newval (may be NULL) receive the per-row log-prob of the action and the value.
 * With L = 1, ov = NULL the operations are those of orc_mlp_ppo_grad in the same order. */
void orc_mlp_deep_ppo_grad(const double* p, const double* obs, const double* act, const double* adv,
                           const double* ret, const double* old, const double* ov, size_t N, size_t D,
                           size_t H, size_t L, size_t A, double vfCoef, double entCoef, double clipEps,
                           double vfClip, double* g, double* newlp, double* newval, int threads) {
  size_t O = A + 1;
  size_t P = H * D + H + (L - 1) * (H * H + H) + O * H + O;
  for (size_t i = 0; i < P; i++) g[i] = 0.0;
  /* offsets of layer l's weight and bias (l = 0..L-1), then the head */
  size_t* oW = (size_t*)malloc(sizeof(size_t) * (L + 1));
  size_t* ob = (size_t*)malloc(sizeof(size_t) * (L + 1));
  size_t off = 0;
  for (size_t l = 0; l < L; l++) {
    size_t in = l == 0 ? D : H;
    oW[l] = off; off += H * in;
    ob[l] = off; off += H;
  }
  oW[L] = off; off += O * H;
  ob[L] = off;
  double** Hs = (double**)malloc(sizeof(double*) * L);
  for (size_t l = 0; l < L; l++) Hs[l] = (double*)malloc(sizeof(double) * N * H);
  double* Out = (double*)malloc(sizeof(double) * N * O);
  double* dOut = (double*)malloc(sizeof(double) * N * O);
  double* dA = (double*)malloc(sizeof(double) * N * H);
  double* dB = (double*)malloc(sizeof(double) * N * H);
  for (size_t l = 0; l < L; l++) {
    const double* X = l == 0 ? obs : Hs[l - 1];
    size_t in = l == 0 ? D : H;
    orc_gemm(0, 1, N, H, in, 1.0, X, in, p + oW[l], in, 0.0, Hs[l], H, threads);
    const double* b = p + ob[l];
    for (size_t n = 0; n < N; n++)
      for (size_t j = 0; j < H; j++) { double v = Hs[l][n * H + j] + b[j]; Hs[l][n * H + j] = v > 0.0 ? v : 0.0; }
  }
  orc_gemm(0, 1, N, O, H, 1.0, Hs[L - 1], H, p + oW[L], H, 0.0, Out, O, threads);
  for (size_t n = 0; n < N; n++) for (size_t k = 0; k < O; k++) Out[n * O + k] += p[ob[L] + k];
  orc_ppo_grad(Out, O, Out + A, O, act, adv, ret, old, ov, N, A, vfCoef, entCoef, clipEps, vfClip, 0,
               dOut, O, dOut + A, O, newlp, newval);
  for (size_t n = 0; n < N; n++) for (size_t k = 0; k < O; k++) g[ob[L] + k] += dOut[n * O + k];
  orc_gemm(1, 0, O, H, N, 1.0, dOut, O, Hs[L - 1], H, 0.0, g + oW[L], H, threads);
  orc_gemm(0, 0, N, H, O, 1.0, dOut, O, p + oW[L], H, 0.0, dA, H, threads);
  for (size_t l = L; l-- > 0;) {
    /* dA = gradient at layer l's output; mask by its activation */
    for (size_t n = 0; n < N; n++)
      for (size_t j = 0; j < H; j++) if (!(Hs[l][n * H + j] > 0.0)) dA[n * H + j] = 0.0;
    for (size_t n = 0; n < N; n++) for (size_t j = 0; j < H; j++) g[ob[l] + j] += dA[n * H + j];
    const double* X = l == 0 ? obs : Hs[l - 1];
    size_t in = l == 0 ? D : H;
    orc_gemm(1, 0, H, in, N, 1.0, dA, H, X, in, 0.0, g + oW[l], in, threads);
    if (l > 0) {
      orc_gemm(0, 0, N, H, H, 1.0, dA, H, p + oW[l], H, 0.0, dB, H, threads);
      double* t = dA; dA = dB; dB = t;
    }
  }
  for (size_t l = 0; l < L; l++) free(Hs[l]);
  free(Hs); free(Out); free(dOut); free(dA); free(dB); free(oW); free(ob);
}

/* ------------------------------------------------------------------------------------------------ */
const double ORC_MUON_COEFFS[5][3] = {
    {4.0848, -6.8946, 2.9270}, {3.9505, -6.3029, 2.6377}, {3.7418, -5.5913, 2.3037},
    {2.8769, -3.1427, 1.2046}, {2.8366, -3.0525, 1.2012}};

/* Threads of the naive Newton-Schulz products (orc_set_threads; 1 unless a timed CPU baseline sets it).
 * Each output row is one thread's, so the results do not depend on the count. */
static int g_ns_threads = 1;
int orc_set_threads(int n) {
  int old = g_ns_threads;
  g_ns_threads = n > 1 ? n : 1;
  return old;
}

/* C[m x n] = A[m x k] B[k x n], naive, accumulation over l in ascending order (Muon.lean:19-32). */
static void mm_naive(const double* A, const double* B, double* C, int m, int k, int n) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(g_ns_threads) if (g_ns_threads > 1)
#endif
  for (int i = 0; i < m; i++)
    for (int j = 0; j < n; j++) {
      double t = 0.0;
      for (int l = 0; l < k; l++) t = t + A[(long)i * k + l] * B[(long)l * n + j];
      C[(long)i * n + j] = t;
    }
}

static void transpose_d(const double* X, double* Xt, int rows, int cols) {
  for (int i = 0; i < rows; i++)
    for (int j = 0; j < cols; j++) Xt[(long)j * rows + i] = X[(long)i * cols + j];
}

/* Frobenius norm as the two-level row fold of pufferblas.c:1380-1381. */
static double frob_fold(const double* u, int rows, int cols) {
  double s = 0.0;
  for (int i = 0; i < rows; i++) {
    double rs = 0.0;
    for (int j = 0; j < cols; j++) { double v = u[(long)i * cols + j]; rs = rs + v * v; }
    s = s + rs;
  }
  return sqrt(s);
}

/* NS on an already-normalised X (rows x cols), in place. */
static void ns_iterate(double* X, int rows, int cols, const double* coeffs, int nsteps, int form) {
  long n = (long)rows * cols;
  if (form == 0) {
    int mn = rows < cols ? rows : cols;
    double* Xt = (double*)malloc(sizeof(double) * n);
    double* A = (double*)malloc(sizeof(double) * mn * mn);
    double* P = (double*)malloc(sizeof(double) * n);
    double* Q = (double*)malloc(sizeof(double) * n);
    for (int it = 0; it < nsteps; it++) {
      double a = coeffs[3 * it], b = coeffs[3 * it + 1], c = coeffs[3 * it + 2];
      transpose_d(X, Xt, rows, cols);
      if (rows <= cols) {
        mm_naive(X, Xt, A, rows, cols, rows);
        mm_naive(A, X, P, rows, rows, cols);
        mm_naive(A, P, Q, rows, rows, cols);
      } else {
        mm_naive(Xt, X, A, cols, rows, cols);
        mm_naive(X, A, P, rows, cols, cols);
        mm_naive(P, A, Q, rows, cols, cols);
      }
      for (long i = 0; i < n; i++) X[i] = a * X[i] + b * P[i] + c * Q[i];
    }
    free(Xt); free(A); free(P); free(Q);
  } else {
    /* wide form: Y = X (rows<=cols) or X^T; A = Y Y^T (m x m); Bm = bA + cA^2; Y <- aY + Bm Y */
    int tall = rows > cols;
    int m = tall ? cols : rows, w = tall ? rows : cols;
    double* Y = (double*)malloc(sizeof(double) * n);
    if (tall) transpose_d(X, Y, rows, cols); else memcpy(Y, X, sizeof(double) * n);
    double* Yt = (double*)malloc(sizeof(double) * n);
    double* A = (double*)malloc(sizeof(double) * m * m);
    double* A2 = (double*)malloc(sizeof(double) * m * m);
    double* BY = (double*)malloc(sizeof(double) * n);
    for (int it = 0; it < nsteps; it++) {
      double a = coeffs[3 * it], b = coeffs[3 * it + 1], c = coeffs[3 * it + 2];
      transpose_d(Y, Yt, m, w);
      mm_naive(Y, Yt, A, m, w, m);
      mm_naive(A, A, A2, m, m, m);
      for (long i = 0; i < (long)m * m; i++) A2[i] = b * A[i] + c * A2[i];
      mm_naive(A2, Y, BY, m, m, w);
      for (long i = 0; i < n; i++) Y[i] = a * Y[i] + BY[i];
    }
    if (tall) transpose_d(Y, X, m, w); else memcpy(X, Y, sizeof(double) * n);
    free(Y); free(Yt); free(A); free(A2); free(BY);
  }
}

void orc_newton_schulz(const double* X0, int rows, int cols, const double* coeffs, int nsteps,
                       double eps, int form, double* out) {
  long n = (long)rows * cols;
  double inv = 1.0 / (frob_fold(X0, rows, cols) + eps);
  for (long i = 0; i < n; i++) out[i] = inv * X0[i];
  ns_iterate(out, rows, cols, coeffs, nsteps, form);
}

/* One Muon matrix step (pufferblas.c:1369-1400; Muon.lean:93-102). */
void orc_muon_mat(int rows, int cols, const double* W, const double* G, const double* M, double* nW,
                  double* nM, double gscale, double lr, double wd, double mu, double eps,
                  const double* coeffs, int nsteps, int form) {
  long n = (long)rows * cols;
  double* u = (double*)malloc(sizeof(double) * n);
  double* X = (double*)malloc(sizeof(double) * n);
  for (long i = 0; i < n; i++) {
    double gi = G[i] * gscale;
    nM[i] = mu * M[i] + gi;
    u[i] = gi + mu * nM[i];
  }
  orc_newton_schulz(u, rows, cols, coeffs ? coeffs : &ORC_MUON_COEFFS[0][0], nsteps, eps, form, X);
  double scale = sqrt(fmax(1.0, (double)rows / (double)cols));
  double c1 = 1.0 - lr * wd, c2 = lr * scale;
  for (long i = 0; i < n; i++) nW[i] = c1 * W[i] + c2 * X[i];
  free(u); free(X);
}

void orc_stepvec(int n, const double* b, const double* g, const double* m, double* nb, double* nm,
                 double gscale, double lr, double wd, double mu) {
  for (int i = 0; i < n; i++) {
    double gi = g[i] * gscale;
    double newm = mu * m[i] + gi;
    double upd = gi + mu * newm;
    nb[i] = b[i] * (1.0 - lr * wd) + lr * upd;
    nm[i] = newm;
  }
}

void orc_muon_step_mlp(const double* pm, const double* g, size_t H, size_t D, size_t O,
                       double gscale, double lr, double wd, double mu, double eps, double* out) {
  size_t P = H * D + H + O * H + O;
  size_t oW1 = 0, ob1 = H * D, oW2 = H * D + H, ob2 = H * D + H + O * H;
  const double* mm = pm + P;
  double* nmo = out + P;
  const double* C = &ORC_MUON_COEFFS[0][0];
  orc_muon_mat((int)H, (int)D, pm + oW1, g + oW1, mm + oW1, out + oW1, nmo + oW1, gscale, lr, wd, mu, eps, C, 5, 0);
  orc_stepvec((int)H, pm + ob1, g + ob1, mm + ob1, out + ob1, nmo + ob1, gscale, lr, wd, mu);
  orc_muon_mat((int)O, (int)H, pm + oW2, g + oW2, mm + oW2, out + oW2, nmo + oW2, gscale, lr, wd, mu, eps, C, 5, 0);
  orc_stepvec((int)O, pm + ob2, g + ob2, mm + ob2, out + ob2, nmo + ob2, gscale, lr, wd, mu);
}

double orc_gclip(double* g, size_t P, double sc, double maxNorm) {
  double s = 0.0;
  for (size_t i = 0; i < P; i++) { double x = g[i] * sc; s += x * x; }
  double gn = sqrt(s);
  double cc = ((maxNorm > 0.0 && gn > maxNorm) ? maxNorm / gn : 1.0) * sc;
  for (size_t i = 0; i < P; i++) g[i] = g[i] * cc;
  return gn;
}

/* ------------------------------------------------------------------------------------------------ */
static inline double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }
static inline double gact(double x) { return x >= 0.0 ? x + 0.5 : sigm(x); }

/* K == 0: one categorical head over the A logits, acts[t]; K >= 1: K heads of sizes[K] summing to A,
 * acts[t*K + h] (MinGRUTrain.lean:130-200, the multi-discrete head on the same MinGRU core). */
static void mingru_seq(const double* p, const double* obsSeq, const double* acts, const double* advs,
                       const double* rets, const double* oldlps, const double* terms, const double* oldvals,
                       size_t T, size_t H, size_t D, size_t L, size_t A, size_t K, const int* sizes,
                       double vfCoef, double entCoef, double clipEps, double vfClip, double* out) {
  size_t szE = H * D, szL = 3 * H * H;
  size_t P = szE + H + L * szL + A * H + A + H + 1;
  const double* wEnc = p; const double* bEnc = p + szE; const double* Wl0 = p + szE + H;
  const double* wDec = Wl0 + L * szL; const double* bDec = wDec + A * H;
  const double* wVal = bDec + A; const double* bVal = wVal + H;
  for (size_t i = 0; i < P + 2 * T; i++) out[i] = 0.0;
  double* gEnc = out; double* gbEnc = out + szE; double* gL0 = out + szE + H;
  double* gDec = gL0 + L * szL; double* gbDec = gDec + A * H; double* gVal = gbDec + A; double* gbVal = gVal + H;
  size_t TLH = T * L * H;
  double* hin = (double*)calloc(TLH, sizeof(double));
  double* prv = (double*)calloc(TLH, sizeof(double));
  double* yh = (double*)calloc(TLH, sizeof(double));
  double* yg = (double*)calloc(TLH, sizeof(double));
  double* yp = (double*)calloc(TLH, sizeof(double));
  double* oo = (double*)calloc(TLH, sizeof(double));
  double* hf = (double*)calloc(T * H, sizeof(double));
  double* lg = (double*)calloc(T * A, sizeof(double));
  double* vv = (double*)calloc(T, sizeof(double));
  double* st = (double*)calloc(L * H, sizeof(double));
  double* h = (double*)calloc(H, sizeof(double));
  double* y = (double*)calloc(3 * H, sizeof(double));
  double* hn = (double*)calloc(H, sizeof(double));
  for (size_t t = 0; t < T; t++) {
    const double* x = obsSeq + t * D;
    for (size_t i = 0; i < H; i++) {
      double acc = 0.0;
      for (size_t k = 0; k < D; k++) acc += wEnc[i * D + k] * x[k];
      h[i] = bEnc[i] + acc;
    }
    for (size_t l = 0; l < L; l++) {
      const double* W = Wl0 + l * szL;
      size_t base = (t * L + l) * H;
      for (size_t j = 0; j < H; j++) { hin[base + j] = h[j]; prv[base + j] = st[l * H + j]; }
      for (size_t r = 0; r < 3 * H; r++) {
        double acc = 0.0;
        for (size_t j = 0; j < H; j++) acc += W[r * H + j] * h[j];
        y[r] = acc;
      }
      for (size_t j = 0; j < H; j++) {
        double z = sigm(y[H + j]);
        double gg = gact(y[j]);
        double o = (1.0 - z) * st[l * H + j] + z * gg;
        double hg = sigm(y[2 * H + j]);
        hn[j] = hg * o + (1.0 - hg) * h[j];
        yh[base + j] = y[j]; yg[base + j] = y[H + j]; yp[base + j] = y[2 * H + j]; oo[base + j] = o;
        st[l * H + j] = o;
      }
      memcpy(h, hn, sizeof(double) * H);
    }
    memcpy(hf + t * H, h, sizeof(double) * H);
    for (size_t k = 0; k < A; k++) {
      double acc = 0.0;
      for (size_t j = 0; j < H; j++) acc += wDec[k * H + j] * h[j];
      lg[t * A + k] = bDec[k] + acc;
    }
    { double acc = 0.0; for (size_t j = 0; j < H; j++) acc += wVal[j] * h[j]; vv[t] = bVal[0] + acc; }
    if (terms[t] != 0.0) memset(st, 0, sizeof(double) * L * H);
  }
  double* dOn = (double*)calloc(L * H, sizeof(double));
  double* dpv = (double*)calloc(L * H, sizeof(double));
  double* dh = (double*)calloc(H, sizeof(double));
  double* dhi = (double*)calloc(H, sizeof(double));
  double* dyh = (double*)calloc(H, sizeof(double));
  double* dyg = (double*)calloc(H, sizeof(double));
  double* dyp = (double*)calloc(H, sizeof(double));
  double* dl = (double*)calloc(A ? A : 1, sizeof(double));
  double* row = (double*)calloc(A + 1, sizeof(double));
  double* drow = (double*)calloc(A + 1, sizeof(double));
  double dv;
  for (size_t k1 = 0; k1 < T; k1++) {
    size_t t = T - 1 - k1;
    const double* x = obsSeq + t * D;
    double nlp, nv;
    if (K == 0) {
      orc_ppo_grad(lg + t * A, A, vv + t, 1, acts + t, advs + t, rets + t, oldlps + t,
                   oldvals ? oldvals + t : NULL, 1, A, vfCoef, entCoef, clipEps, vfClip, 0, dl, A,
                   &dv, 1, &nlp, &nv);
    } else {
      for (size_t k = 0; k < A; k++) row[k] = lg[t * A + k];
      row[A] = vv[t];
      orc_ppo_grad_md(row, A + 1, acts + t * K, advs + t, rets + t, oldlps + t, oldvals ? oldvals + t : NULL, 1,
                      sizes, K, vfCoef, entCoef, clipEps, vfClip, drow, A + 1, &nlp, &nv);
      for (size_t k = 0; k < A; k++) dl[k] = drow[k];
      dv = drow[A];
    }
    out[P + t] = nlp; out[P + T + t] = nv;
    const double* hft = hf + t * H;
    for (size_t j = 0; j < H; j++) dh[j] = 0.0;
    for (size_t k = 0; k < A; k++) {
      for (size_t j = 0; j < H; j++) { gDec[k * H + j] += dl[k] * hft[j]; dh[j] += dl[k] * wDec[k * H + j]; }
      gbDec[k] += dl[k];
    }
    for (size_t j = 0; j < H; j++) { gVal[j] += dv * hft[j]; dh[j] += dv * wVal[j]; }
    gbVal[0] += dv;
    for (size_t l1 = 0; l1 < L; l1++) {
      size_t l = L - 1 - l1;
      size_t base = (t * L + l) * H;
      const double* W = Wl0 + l * szL; double* gW = gL0 + l * szL;
      for (size_t j = 0; j < H; j++) dhi[j] = 0.0;
      for (size_t j = 0; j < H; j++) {
        double z = sigm(yg[base + j]), hg = sigm(yp[base + j]), gg = gact(yh[base + j]);
        double dhg = dh[j] * (oo[base + j] - hin[base + j]);
        double dox = dh[j] * hg + dOn[l * H + j];
        dhi[j] += dh[j] * (1.0 - hg);
        double dz = dox * (gg - prv[base + j]);
        dpv[l * H + j] = dox * (1.0 - z);
        double dg = dox * z;
        double sg;
        if (yh[base + j] >= 0.0) sg = 1.0; else { double s = sigm(yh[base + j]); sg = s * (1.0 - s); }
        dyh[j] = dg * sg; dyg[j] = dz * z * (1.0 - z); dyp[j] = dhg * hg * (1.0 - hg);
      }
      for (size_t j = 0; j < H; j++) {
        for (size_t k = 0; k < H; k++) { gW[j * H + k] += dyh[j] * hin[base + k]; dhi[k] += dyh[j] * W[j * H + k]; }
        for (size_t k = 0; k < H; k++) { gW[(H + j) * H + k] += dyg[j] * hin[base + k]; dhi[k] += dyg[j] * W[(H + j) * H + k]; }
        for (size_t k = 0; k < H; k++) { gW[(2 * H + j) * H + k] += dyp[j] * hin[base + k]; dhi[k] += dyp[j] * W[(2 * H + j) * H + k]; }
      }
      memcpy(dh, dhi, sizeof(double) * H);
    }
    for (size_t i = 0; i < H; i++) {
      gbEnc[i] += dh[i];
      for (size_t k = 0; k < D; k++) gEnc[i * D + k] += dh[i] * x[k];
    }
    if (t > 0) {
      double keep = (terms[t - 1] == 0.0) ? 1.0 : 0.0;
      for (size_t q = 0; q < L * H; q++) dOn[q] = dpv[q] * keep;
    }
  }
  free(hin); free(prv); free(yh); free(yg); free(yp); free(oo); free(hf); free(lg); free(vv);
  free(st); free(h); free(y); free(hn); free(dOn); free(dpv); free(dh); free(dhi); free(dyh);
  free(dyg); free(dyp); free(dl); free(row); free(drow);
}

/* Single-sequence MinGRU PPO BPTT (pufferffi.c:763-876). Layout [wEnc(H*D)|bEnc(H)|L x W(3H*H)|
 * wDec(A*H)|bDec(A)|wVal(H)|bVal(1)]; W rows [0,H) hid, [H,2H) gate, [2H,3H) proj. Zero initial state,
 * state reset after a terminal, no gradient across a terminal. */
void orc_mingru_ppo_grad_seq(const double* p, const double* obsSeq, const double* acts,
                             const double* advs, const double* rets, const double* oldlps,
                             const double* terms, const double* oldvals, size_t T, size_t H,
                             size_t D, size_t L, size_t A, double vfCoef, double entCoef,
                             double clipEps, double vfClip, double* out) {
  mingru_seq(p, obsSeq, acts, advs, rets, oldlps, terms, oldvals, T, H, D, L, A, 0, NULL, vfCoef, entCoef, clipEps,
             vfClip, out);
}

/* The multi-discrete form (mingruGradSeqMD, MinGRUTrain.lean:140-230; the device's k_mg_ppo_b_md,
 * puffercuda.cu:4940-4975): A = sum of sizes[K] decoder rows, acts [T][K], new_logp the joint. */
void orc_mingru_ppo_grad_seq_md(const double* p, const double* obsSeq, const double* acts, const double* advs,
                                const double* rets, const double* oldlps, const double* terms,
                                const double* oldvals, size_t T, size_t H, size_t D, size_t L, size_t A,
                                const int* sizes, size_t K, double vfCoef, double entCoef, double clipEps,
                                double vfClip, double* out) {
  mingru_seq(p, obsSeq, acts, advs, rets, oldlps, terms, oldvals, T, H, D, L, A, K, sizes, vfCoef, entCoef, clipEps,
             vfClip, out);
}

/* Heinsen log-space scan (MinGRU.lean:116-168; tools/mingru_ref.py:113-131): with log a_t = log(1-z_t),
 * log b_t = log z_t + log g_t, o_t = exp(a*_t + logcumsumexp_{s<=t}(log b_s - a*_s)), a*_t = sum log a.
 * Online logcumsumexp with running max. softplus / log g as in the reference's restatement. */
static double softplus(double x) { return x > 0.0 ? x + log(1.0 + exp(-x)) : log(1.0 + exp(x)); }
static double log_g(double x) { return x >= 0.0 ? log(x + 0.5) : -softplus(-x); }

void orc_mingru_heinsen(const double* gate, const double* hid, size_t T, size_t H, double* o) {
  for (size_t j = 0; j < H; j++) {
    double astar = 0.0, m = -1e308, s = 0.0;
    for (size_t t = 0; t < T; t++) {
      double g = gate[t * H + j], hv = hid[t * H + j];
      astar += -softplus(g);
      double x = (-softplus(-g) + log_g(hv)) - astar;
      if (x > m) { s = s * exp(m - x) + 1.0; m = x; }
      else s = s + exp(x - m);
      o[t * H + j] = exp(astar + m + log(s));
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* Prioritised replay. */

/* k_adv_l1 (puffercuda.cu:311-312): one segment at a time, t ascending. */
void orc_seg_l1(const double* adv, size_t N, size_t T, double* L1) {
  for (size_t e = 0; e < N; e++) {
    const double* a = adv + e * T;
    double s = 0.0;
    for (size_t t = 0; t < T; t++) s += fabs(a[t]);
    L1[e] = s;
  }
}

/* lean_ffi_prio_sample (pufferffi.c:1094-1125): weights, sequential normaliser and running sum, then
 * each draw takes the splitmix64 word of rng + (i+1)*GOLD, scales its top 53 bits by the total, and
 * takes the first segment whose running sum reaches it (binary search; the running sum is strictly
 * increasing because every probability is positive). */
void orc_prio_sample(const double* L1, size_t N, size_t mbSegs, double alpha, double beta, uint64_t rng,
                     double* idx, double* mbPrio, double* probs, double* cum) {
  double* w = (double*)malloc(N * sizeof(double));
  double* p = (double*)malloc(N * sizeof(double));
  double* c = (double*)malloc(N * sizeof(double));
  double sumW = 0.0;
  for (size_t e = 0; e < N; e++) {
    w[e] = exp(alpha * log(L1[e] + 1e-12));
    sumW += w[e];
  }
  const double denom = sumW + 1e-6;
  double acc = 0.0;
  for (size_t e = 0; e < N; e++) {
    p[e] = (w[e] + 1e-6) / denom;
    acc += p[e];
    c[e] = acc;
  }
  const double total = acc;
  for (size_t i = 0; i < mbSegs; i++) {
    uint64_t s = rng + (uint64_t)i * 0x9E3779B97F4A7C15ULL;
    const double u = orc_uniform01(orc_rng_next(&s)) * total;
    size_t lo = 0, hi = N;
    while (lo < hi) {
      const size_t mid = (lo + hi) >> 1;
      if (c[mid] >= u) hi = mid;
      else lo = mid + 1;
    }
    const size_t k = lo < N ? lo : N - 1;
    idx[i] = (double)k;
    mbPrio[i] = exp((-beta) * log((double)N * p[k] + 1e-12));
  }
  if (probs) memcpy(probs, p, N * sizeof(double));
  if (cum) memcpy(cum, c, N * sizeof(double));
  free(w);
  free(p);
  free(c);
}

/* lean_ffi_gather_seq_minibatch (pufferffi.c:1126-1200): mean and population std over the sampled
 * rows in (bi outer, t inner) order, then the six columns. */
void orc_gather_seq_minibatch(const double* act, const double* logp, const double* term,
                              const double* adv, const double* value, const double* segIdx,
                              const double* mbPrio, size_t T, size_t Bmb, double* out, double* stats2) {
  const size_t nb = T * Bmb;
  const double navd = (double)(nb > 0 ? nb : 1);
  double sum = 0.0;
  for (size_t bi = 0; bi < Bmb; bi++) {
    const double* a = adv + (size_t)segIdx[bi] * T;
    for (size_t t = 0; t < T; t++) sum += a[t];
  }
  const double mean = sum / navd;
  double sq = 0.0;
  for (size_t bi = 0; bi < Bmb; bi++) {
    const double* a = adv + (size_t)segIdx[bi] * T;
    for (size_t t = 0; t < T; t++) {
      const double d = a[t] - mean;
      sq += d * d;
    }
  }
  const double sd = sqrt(sq / navd), stde = sd + 1e-8;
  double *oact = out, *oadv = out + nb, *oret = out + 2 * nb, *oold = out + 3 * nb, *oterm = out + 4 * nb,
         *oov = out + 5 * nb;
  for (size_t bi = 0; bi < Bmb; bi++) {
    const size_t e = (size_t)segIdx[bi];
    for (size_t t = 0; t < T; t++) {
      const size_t si = e * T + t, os = t * Bmb + bi;
      const double a = adv[si], v = value[si];
      oact[os] = (double)(unsigned long long)act[si];
      oadv[os] = mbPrio[bi] * (a - mean) / stde;
      oret[os] = a + v;
      oold[os] = logp[si];
      oov[os] = v;
      oterm[os] = term[si] > 0.5 ? 1.0 : 0.0;
    }
  }
  if (stats2) {
    stats2[0] = mean;
    stats2[1] = sd;
  }
}

void orc_mb_iterate(double* value, double* ratio, const double* logp, const float* newlp,
                    const float* newval, const double* seg, size_t Bmb, size_t T) {
  for (size_t bi = 0; bi < Bmb; bi++) {
    const size_t e = (size_t)seg[bi];
    for (size_t t = 0; t < T; t++) {
      const size_t si = e * T + t, os = t * Bmb + bi;
      ratio[si] = exp((double)newlp[os] - logp[si]);
      value[si] = (double)newval[os];
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* Rollout policy forward and categorical sampler. */

/* lean_ffi_sample_actions_batch (pufferffi.c:896-918): max-shifted softmax, the first k whose running
 * probability exceeds u (else the last action), log of the chosen probability, the value column. */
void orc_sample_actions(const double* Y, size_t N, size_t A, size_t O, uint64_t rng, double* out) {
  for (size_t n = 0; n < N; n++) {
    const double* row = Y + n * O;
    double m = row[0];
    for (size_t k = 1; k < A; k++)
      if (row[k] > m) m = row[k];
    double z = 0.0;
    for (size_t k = 0; k < A; k++) z += exp(row[k] - m);
    uint64_t s = rng + (uint64_t)n * 0x9E3779B97F4A7C15ULL;
    const double u = orc_uniform01(orc_rng_next(&s));
    double acc = 0.0;
    size_t a = A - 1;
    for (size_t k = 0; k < A; k++) {
      acc += exp(row[k] - m) / z;
      if (u < acc) {
        a = k;
        break;
      }
    }
    out[n] = (double)a;
    out[N + n] = log(exp(row[a] - m) / z);
    out[2 * N + n] = row[A];
  }
}

/* lean_cuda_mingru_step (puffercuda.cu:2190-2265) in f64: encoder, then per layer the 3H x H product
 * (hid | gate | proj) and the cell o = (1-z) prev + z gact(hid), h = hg o + (1-hg) h_in; then the
 * action and value heads. */
void orc_mingru_step(const double* p, const double* obs, const double* state, size_t N, size_t D,
                     size_t H, size_t L, size_t A, double* out) {
  const size_t szE = H * D, szL = 3 * H * H, O = A + 1;
  const double* wEnc = p; const double* bEnc = p + szE; const double* Wl0 = p + szE + H;
  const double* wDec = Wl0 + L * szL; const double* bDec = wDec + A * H;
  const double* wVal = bDec + A; const double* bVal = wVal + H;
  double* h = (double*)malloc(H * sizeof(double));
  double* hn = (double*)malloc(H * sizeof(double));
  double* y = (double*)malloc(3 * H * sizeof(double));
  double* ns = out + N * O;
  for (size_t n = 0; n < N; n++) {
    const double* x = obs + n * D;
    for (size_t i = 0; i < H; i++) {
      double acc = 0.0;
      for (size_t k = 0; k < D; k++) acc += wEnc[i * D + k] * x[k];
      h[i] = bEnc[i] + acc;
    }
    for (size_t l = 0; l < L; l++) {
      const double* W = Wl0 + l * szL;
      const double* prev = state + (n * L + l) * H;
      for (size_t r = 0; r < 3 * H; r++) {
        double acc = 0.0;
        for (size_t j = 0; j < H; j++) acc += W[r * H + j] * h[j];
        y[r] = acc;
      }
      for (size_t j = 0; j < H; j++) {
        const double z = sigm(y[H + j]), gg = gact(y[j]), hg = sigm(y[2 * H + j]);
        const double o = (1.0 - z) * prev[j] + z * gg;
        hn[j] = hg * o + (1.0 - hg) * h[j];
        ns[(n * L + l) * H + j] = o;
      }
      memcpy(h, hn, H * sizeof(double));
    }
    for (size_t k = 0; k < A; k++) {
      double acc = 0.0;
      for (size_t j = 0; j < H; j++) acc += wDec[k * H + j] * h[j];
      out[n * O + k] = bDec[k] + acc;
    }
    double acc = 0.0;
    for (size_t j = 0; j < H; j++) acc += wVal[j] * h[j];
    out[n * O + A] = bVal[0] + acc;
  }
  free(h);
  free(hn);
  free(y);
}

/* ------------------------------------------------------------------------------------------------ */
/* Multi-discrete and continuous heads. */

static double vloss_grad_d(double v, double ret, const double* ov, size_t n, double vfClip) {
  if (vfClip <= 0.0 || !ov) return v - ret;
  const double dd = v - ov[n];
  const double vc = ov[n] + (dd < -vfClip ? -vfClip : (dd > vfClip ? vfClip : dd));
  if ((v - ret) * (v - ret) >= (vc - ret) * (vc - ret)) return v - ret;
  if (dd > -vfClip && dd < vfClip) return v - ret;
  return 0.0;
}

static double dpol_of(double ratio, double adv, double clip) {
  const double lo = 1.0 - clip, hi = 1.0 + clip;
  const double rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
  if (adv * ratio <= adv * rc) return adv * ratio;
  return (lo < ratio && ratio < hi) ? adv * ratio : 0.0;
}

/* k_ppo_dout_md (puffercuda.cu:702-727): joint log-prob over the heads, one clip, per-head softmax and
 * entropy gradients. A row with an action outside [0, size) of its head gets NaN logit gradients and
 * NaN log-prob (its value gradient stands). */
void orc_ppo_grad_md(const double* out, size_t ldo, const double* act, const double* adv, const double* ret,
                     const double* old, const double* ov, size_t N, const int* sizes, size_t K, double vf,
                     double ent, double clip, double vfClip, double* dout, size_t ldd, double* newlp,
                     double* newval) {
  size_t W = 0;
  for (size_t h = 0; h < K; h++) W += (size_t)sizes[h];
  for (size_t n = 0; n < N; n++) {
    const double* o = out + n * ldo;
    double* d = dout + n * ldd;
    double joint = 0.0;
    int inRange = 1;
    size_t off = 0;
    for (size_t h = 0; h < K; h++) {
      const double ah = act[n * K + h];
      double se = 0.0;
      for (int k = 0; k < sizes[h]; k++) se += exp(o[off + k]);
      if (ah >= 0.0 && ah < (double)sizes[h]) joint += o[off + (size_t)ah] - log(se);
      else inRange = 0;
      off += (size_t)sizes[h];
    }
    if (!inRange) joint = NAN;
    const double dPol = inRange ? dpol_of(exp(joint - old[n]), adv[n], clip) : NAN;
    off = 0;
    for (size_t h = 0; h < K; h++) {
      const int a = (int)act[n * K + h];
      double se = 0.0;
      for (int k = 0; k < sizes[h]; k++) se += exp(o[off + k]);
      const double lse = log(se);
      double pout = 0.0;
      for (int k = 0; k < sizes[h]; k++) pout += exp(o[off + k] - lse) * o[off + k];
      for (int k = 0; k < sizes[h]; k++) {
        const double p = exp(o[off + k] - lse);
        d[off + k] = dPol * ((k == a ? 1.0 : 0.0) - p) + ent * p * (pout - o[off + k]);
      }
      off += (size_t)sizes[h];
    }
    d[W] = -vf * vloss_grad_d(o[W], ret[n], ov, n, vfClip);
    if (newlp) newlp[n] = joint;
    if (newval) newval[n] = o[W];
  }
}

/* k_ppo_dout_cont (puffercuda.cu:1767-1790); the CPU twin pufferffi.c:264-307 is this with a [-5, 2]
 * clamp and no value clip. */
void orc_ppo_grad_cont(const double* out, size_t ldo, const double* act, const double* adv, const double* ret,
                       const double* old, const double* ov, size_t N, size_t d, double vf, double ent,
                       double clip, double vfClip, double lslo, double lshi, double* dout, size_t ldd,
                       double* newlp, double* newval) {
  const double hl = 0.5 * log(2.0 * M_PI_ORACLE);
  for (size_t n = 0; n < N; n++) {
    const double* o = out + n * ldo;
    double* g = dout + n * ldd;
    const double* a = act + n * d;
    double logp = 0.0;
    for (size_t i = 0; i < d; i++) {
      const double lsr = o[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
      const double z = (a[i] - o[i]) * exp(-ls);
      logp += -0.5 * z * z - ls - hl;
    }
    const double dPol = dpol_of(exp(logp - old[n]), adv[n], clip);
    for (size_t i = 0; i < d; i++) {
      const double lsr = o[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
      const double inv = exp(-ls), z = (a[i] - o[i]) * inv;
      g[i] = dPol * z * inv;
      g[d + i] = (lslo < lsr && lsr < lshi) ? dPol * (z * z - 1.0) + ent : 0.0;
    }
    g[2 * d] = -vf * vloss_grad_d(o[2 * d], ret[n], ov, n, vfClip);
    if (newlp) newlp[n] = logp;
    if (newval) newval[n] = o[2 * d];
  }
}

static const uint64_t ORC_GOLD2 = 0xD1B54A32D192ED03ULL;
static double orc_word_unit(uint64_t state) {
  uint64_t s = state - 0x9E3779B97F4A7C15ULL; /* orc_rng_next advances before mixing */
  return orc_uniform01(orc_rng_next(&s));
}

/* ff_surface_losses modes 1 and 2 (puffercuda.cu:1798-1870): the 7 dashboard losses [pg, v, ent, total,
 * old_kl, kl, clipfrac] as means over N rows of head outputs. mode 1: K categorical heads of sizes[K]
 * (max-shifted log-sum-exp per head, entropy summed over the heads); mode 2: d Gaussian dims with the
 * log-std clamped to [lslo, lshi], entropy sum(ls + (1 + log 2 pi)/2). The value is at column ldo-wide
 * row index W (sum of sizes, or 2d). ov NULL or vfClip <= 0: unclipped value loss. */
void orc_wide_losses(int mode, const double* out, size_t ldo, const double* act, const double* adv,
                     const double* ret, const double* old, const double* ov, size_t N, const int* sizes, size_t K,
                     size_t d, double vfCoef, double entCoef, double clipEps, double vfClip, double lslo,
                     double lshi, double* L) {
  const double lo = 1.0 - clipEps, hi = 1.0 + clipEps, hl = 0.5 * log(2.0 * M_PI_ORACLE);
  const int clipV = ov != NULL && vfClip > 0.0;
  double sPg = 0, sV = 0, sEnt = 0, sKL = 0, sOld = 0;
  size_t nclip = 0;
  for (size_t n = 0; n < N; n++) {
    const double* o = out + n * ldo;
    double newlp = 0.0, ent = 0.0, newval;
    if (mode == 2) {
      for (size_t i = 0; i < d; i++) {
        const double lsr = o[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
        const double z = (act[n * d + i] - o[i]) * exp(-ls);
        newlp += -0.5 * z * z - ls - hl;
        ent += ls + (0.5 + hl);
      }
      newval = o[2 * d];
    } else {
      size_t off = 0;
      for (size_t h = 0; h < K; h++) {
        const int sz = sizes[h];
        const size_t a = (size_t)act[n * K + h];
        double mx = o[off];
        for (int k = 1; k < sz; k++) if (o[off + k] > mx) mx = o[off + k];
        double se = 0.0;
        for (int k = 0; k < sz; k++) se += exp(o[off + k] - mx);
        const double lse = mx + log(se);
        newlp += o[off + a] - lse;
        for (int k = 0; k < sz; k++) { const double lp = o[off + k] - lse; ent -= exp(lp) * lp; }
        off += (size_t)sz;
      }
      newval = o[off];
    }
    sEnt += ent;
    const double lr = newlp - old[n], ratio = exp(lr);
    const double rc = ratio < lo ? lo : (ratio > hi ? hi : ratio);
    const double p1 = -adv[n] * ratio, p2 = -adv[n] * rc;
    sPg += p1 > p2 ? p1 : p2;
    if (ratio < lo || ratio > hi) nclip++;
    sKL += (ratio - 1.0) - lr;
    sOld += -lr;
    const double du = (newval - ret[n]) * (newval - ret[n]);
    double vl = du;
    if (clipV) {
      const double dd = newval - ov[n];
      const double vc = ov[n] + (dd < -vfClip ? -vfClip : (dd > vfClip ? vfClip : dd));
      const double cc = (vc - ret[n]) * (vc - ret[n]);
      if (cc > du) vl = cc;
    }
    sV += 0.5 * vl;
  }
  const double dn = (double)N;
  L[0] = sPg / dn; L[1] = sV / dn; L[2] = sEnt / dn;
  L[3] = L[0] + vfCoef * L[1] - entCoef * L[2];
  L[4] = sOld / dn; L[5] = sKL / dn; L[6] = (double)nclip / dn;
}

/* k_sample_md (puffercuda.cu:1538-1551). */
void orc_sample_md(const double* Y, size_t ldy, size_t N, const int* sizes, size_t K, uint64_t rng,
                   double* out) {
  size_t W = 0;
  for (size_t h = 0; h < K; h++) W += (size_t)sizes[h];
  for (size_t n = 0; n < N; n++) {
    const double* row = Y + n * ldy;
    double joint = 0.0;
    size_t off = 0;
    for (size_t h = 0; h < K; h++) {
      const int sz = sizes[h];
      double m = row[off];
      for (int k = 1; k < sz; k++)
        if (row[off + k] > m) m = row[off + k];
      double z = 0.0;
      for (int k = 0; k < sz; k++) z += exp(row[off + k] - m);
      const double u = orc_word_unit(rng + (uint64_t)(n + 1) * 0x9E3779B97F4A7C15ULL + (uint64_t)(h + 1) * ORC_GOLD2);
      double acc = 0.0;
      int a = sz - 1;
      for (int k = 0; k < sz; k++) {
        acc += exp(row[off + k] - m) / z;
        if (u < acc) {
          a = k;
          break;
        }
      }
      out[h * N + n] = (double)a;
      joint += log(exp(row[off + a] - m) / z);
      off += (size_t)sz;
    }
    out[K * N + n] = joint;
    out[(K + 1) * N + n] = row[W];
  }
}

/* k_sample_cont (puffercuda.cu:1652-1668). */
void orc_sample_cont(const double* Y, size_t ldy, size_t N, size_t d, uint64_t rng, double lslo, double lshi,
                     double* out) {
  const double hl = 0.5 * log(2.0 * M_PI_ORACLE);
  for (size_t n = 0; n < N; n++) {
    const double* row = Y + n * ldy;
    double logp = 0.0;
    for (size_t i = 0; i < d; i++) {
      const double lsr = row[d + i], ls = lsr < lslo ? lslo : (lsr > lshi ? lshi : lsr);
      const uint64_t base = rng + (uint64_t)(n + 1) * 0x9E3779B97F4A7C15ULL;
      double u1 = orc_word_unit(base + (uint64_t)(2 * i + 1) * ORC_GOLD2);
      if (u1 < 1.0e-7) u1 = 1.0e-7;
      const double u2 = orc_word_unit(base + (uint64_t)(2 * i + 2) * ORC_GOLD2);
      const double z = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI_ORACLE * u2);
      out[i * N + n] = row[i] + exp(ls) * z;
      logp += -0.5 * z * z - ls - hl;
    }
    out[d * N + n] = logp;
    out[(d + 1) * N + n] = row[2 * d];
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* Timed CPU baselines (bench.py's cpu_baseline legs). Same arithmetic as the functions above, spread
 * over threads. */

/* V-trace over segments in parallel (each segment's scan is orc_vtrace_f32's, unchanged). */
void orc_vtrace_f32_mt(const float* rew, const float* val, const float* term, const float* rho,
                       const float* boot, size_t B, size_t T, int variant, int time_major, int rho_is_log,
                       int clamp, float gamma, float lam, float rhoClip, float cClip, float* adv, float* tgt,
                       int threads) {
  int nt = threads > 1 ? threads : 1;
  size_t chunk = (B + (size_t)nt - 1) / (size_t)nt;
  {
    /* thread w scans segments [b0, b1) in either layout */
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
    for (int w = 0; w < nt; w++) {
      size_t b0 = (size_t)w * chunk, b1 = b0 + chunk < B ? b0 + chunk : B;
      for (size_t b = b0; b < b1; b++) {
        float last = 0;
        size_t t0;
        if (variant == 0) {
          if (T == 0) continue;
          size_t il = time_major ? (T - 1) * B + b : b * T + T - 1;
          adv[il] = 0;
          if (tgt) tgt[il] = adv[il] + val[il];
          t0 = T - 1;
        } else {
          t0 = T;
        }
        for (size_t k = 0; k < t0; k++) {
          size_t t = t0 - 1 - k;
          size_t i = time_major ? t * B + b : b * T + t;
          size_t in = time_major ? (t + 1) * B + b : b * T + t + 1;
          float wgt = rho_is_log ? expf(rho[i]) : rho[i];
          float rh = wgt < rhoClip ? wgt : rhoClip;
          float c = wgt < cClip ? wgt : cClip;
          float r = clamp ? clamp1f(rew[i]) : rew[i];
          float delta, nnt;
          if (variant == 0) {
            nnt = (term[i] != 0) ? 0.0f : 1.0f;
            delta = rh * (r + gamma * val[in] * nnt - val[i]);
          } else {
            nnt = (term[i] > 0.5f) ? 0.0f : 1.0f;
            float vnext = (t + 1 < T) ? val[in] : boot[b];
            delta = rh * r + gamma * vnext * nnt - val[i];
          }
          last = delta + gamma * lam * c * last * nnt;
          adv[i] = last;
          if (tgt) tgt[i] = last + val[i];
        }
      }
    }
  }
}

/* C = op(A) op(B) (row-major, f64) with cache blocking: threads take 64-row blocks of C; for each
 * 256-deep k block the op(B) panel is packed contiguous per thread and every C row block is updated
 * in 4 x 8 register tiles. A timing baseline for the policy GEMMs (the reference runs them through
 * OpenBLAS cblas_dgemm, pufferblas.c:720-743). */
void orc_gemm_blocked(int transA, int transB, size_t M, size_t N, size_t K, const double* A, size_t lda,
                      const double* B, size_t ldb, double* C, size_t ldc, int threads) {
  enum { MB = 64, KB = 256 };
  int nt = threads > 1 ? threads : 1;
  long nblk = (long)((M + MB - 1) / MB);
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
  {
    double* Bp = (double*)malloc(sizeof(double) * KB * (N ? N : 1));
    double* Ap = (double*)malloc(sizeof(double) * MB * KB);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (long blk = 0; blk < nblk; blk++) {
      size_t i0 = (size_t)blk * MB, mb = i0 + MB <= M ? MB : M - i0;
      for (size_t i = 0; i < mb; i++) for (size_t j = 0; j < N; j++) C[(i0 + i) * ldc + j] = 0.0;
      for (size_t k0 = 0; k0 < K; k0 += KB) {
        size_t kb = k0 + KB <= K ? KB : K - k0;
        /* pack op(B)[k0..k0+kb) x N as kb rows of N, op(A) block as mb rows of kb */
        for (size_t k = 0; k < kb; k++)
          for (size_t j = 0; j < N; j++) Bp[k * N + j] = transB ? B[j * ldb + k0 + k] : B[(k0 + k) * ldb + j];
        for (size_t i = 0; i < mb; i++)
          for (size_t k = 0; k < kb; k++) Ap[i * kb + k] = transA ? A[(k0 + k) * lda + i0 + i] : A[(i0 + i) * lda + k0 + k];
        size_t i = 0;
        for (; i + 4 <= mb; i += 4) {
          size_t j = 0;
          for (; j + 8 <= N; j += 8) {
            double acc[4][8] = {{0}};
            for (size_t k = 0; k < kb; k++) {
              const double* br = Bp + k * N + j;
              for (int r = 0; r < 4; r++) {
                double a = Ap[(i + r) * kb + k];
                for (int q = 0; q < 8; q++) acc[r][q] += a * br[q];
              }
            }
            for (int r = 0; r < 4; r++) for (int q = 0; q < 8; q++) C[(i0 + i + r) * ldc + j + q] += acc[r][q];
          }
          for (; j < N; j++)
            for (int r = 0; r < 4; r++) {
              double t = 0.0;
              for (size_t k = 0; k < kb; k++) t += Ap[(i + r) * kb + k] * Bp[k * N + j];
              C[(i0 + i + r) * ldc + j] += t;
            }
        }
        for (; i < mb; i++)
          for (size_t j = 0; j < N; j++) {
            double t = 0.0;
            for (size_t k = 0; k < kb; k++) t += Ap[i * kb + k] * Bp[k * N + j];
            C[(i0 + i) * ldc + j] += t;
          }
      }
    }
    free(Bp); free(Ap);
  }
}

/* Summed single-sequence MinGRU gradients over B segments of time-major columns (obs [T][B][D], the
 * rest [T][B]), segments spread over threads; each thread sums its segments in order, then the thread
 * sums are added in thread order. out = [G (P) | newlp [T][B] | newval [T][B]]. */
void orc_mingru_ppo_grad_batch(const double* p, const double* obs, const double* act, const double* adv,
                               const double* ret, const double* old, const double* term, const double* ov,
                               size_t B, size_t T, size_t H, size_t D, size_t L, size_t A, double vfCoef,
                               double entCoef, double clipEps, double vfClip, double* out, int threads) {
  int nt = threads > 1 ? threads : 1;
  size_t P = H * D + H + L * 3 * H * H + A * H + A + H + 1;
  double* part = (double*)calloc((size_t)nt * P, sizeof(double));
  size_t chunk = (B + (size_t)nt - 1) / (size_t)nt;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
  for (int w = 0; w < nt; w++) {
    double* seq = (double*)malloc(sizeof(double) * T * (D + 7));
    double* res = (double*)malloc(sizeof(double) * (P + 2 * T));
    double* ob = seq; double* ac = ob + T * D; double* ad = ac + T; double* re = ad + T; double* ol = re + T;
    double* te = ol + T; double* ovs = te + T;
    size_t b0 = (size_t)w * chunk, b1 = b0 + chunk < B ? b0 + chunk : B;
    for (size_t b = b0; b < b1; b++) {
      for (size_t t = 0; t < T; t++) {
        size_t r = t * B + b;
        memcpy(ob + t * D, obs + r * D, sizeof(double) * D);
        ac[t] = act[r]; ad[t] = adv[r]; re[t] = ret[r]; ol[t] = old[r]; te[t] = term[r];
        ovs[t] = ov ? ov[r] : 0.0;
      }
      mingru_seq(p, ob, ac, ad, re, ol, te, ovs, T, H, D, L, A, 0, NULL, vfCoef, entCoef, clipEps, vfClip, res);
      for (size_t i = 0; i < P; i++) part[(size_t)w * P + i] += res[i];
      for (size_t t = 0; t < T; t++) {
        out[P + t * B + b] = res[P + t];
        out[P + T * B + t * B + b] = res[P + T + t];
      }
    }
    free(seq); free(res);
  }
  for (size_t i = 0; i < P; i++) {
    double s = 0.0;
    for (int w = 0; w < nt; w++) s += part[(size_t)w * P + i];
    out[i] = s;
  }
  free(part);
}

