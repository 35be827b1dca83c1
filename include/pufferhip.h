/* pufferhip — MI355X (gfx950) native library for the pufferlean training-step hot path.
 *
 * Plain C ABI: raw pointers, sizes and scalars; no Lean, torch or HIP types in any signature.
 * Every function returns a ph_status (0 = success); ph_last_error() describes the last failure on
 * the calling thread. There is no CPU fallback: without a usable device the calls fail.
 *
 * Two layers:
 *   1. Stream-ordered device entry points (ph_*): device pointers in and out, an opaque stream
 *      handle (a hipStream_t, or NULL for the default stream), no implicit synchronisation.
 *   2. Host-buffer entry points (ph_cuda_* / ph_ffi_*): one per GPU symbol the reference's Lean
 *      side binds with @[extern] (Puffer/Float/CUDA.lean, Puffer/Float/BLAS.lean). Each takes the
 *      same arguments as the reference symbol it replaces, with every FloatArray turned into a
 *      host `const double*` (input) or `double*` (caller-allocated output of the documented size).
 *      They copy in, run, copy out and synchronise, like the reference entries. The Lean glue that
 *      maps lean_cuda_X(lean_obj_arg ...) onto ph_cuda_X(const double* ...) is a few lines each.
 */
#ifndef PUFFERHIP_H
#define PUFFERHIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define PH_VERSION 100

typedef enum {
  PH_OK = 0,
  PH_ERR_ARG = -1,         /* invalid argument (shape, pointer, enum) */
  PH_ERR_HIP = -2,         /* HIP runtime error (no device, launch failure, ...) */
  PH_ERR_NOMEM = -3,       /* device allocation failed */
  PH_ERR_UNSUPPORTED = -4  /* combination not implemented */
} ph_status;

typedef enum { PH_F32 = 0, PH_F64 = 1, PH_BF16 = 2, PH_I32 = 3 } ph_dtype;
/* PH_MATH_BF16X3: fp32 operands split into bf16 hi + lo, three MFMA products per k (hi*hi + hi*lo
 * + lo*hi), close to fp32 accuracy on the bf16 matrix cores. */
typedef enum { PH_MATH_BF16 = 0, PH_MATH_F32 = 1, PH_MATH_BF16X3 = 2 } ph_math;
typedef enum {
  PH_EPI_NONE = 0,       /* C = acc */
  PH_EPI_BIAS = 1,       /* C = acc + bias[col] */
  PH_EPI_BIAS_RELU = 2,  /* C = max(acc + bias[col], 0) */
  PH_EPI_RELU_MASK = 3,  /* C = aux[row,col] > 0 ? acc : 0 */
  PH_EPI_AXPBY = 4       /* C = alpha*acc + beta*aux[row,col] (aux may be NULL: beta term 0) */
} ph_epilogue;

/* ---------------------------------------------------------------------------------------------- */
/* Runtime */
const char* ph_last_error(void);
int ph_version(void);
/* Number of visible devices (0 if none). Replaces lean_ffi_cuda_available (pufferblas.c:1348). */
int ph_device_count(void);
int ph_synchronize(void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* V-trace / GAE reverse scan. Replaces k_vtrace / k_vtrace_mingru (puffercuda.cu:69-90, 146-167)
 * and generalises them:
 *   dtype      PH_F32 or PH_F64 (all float arrays share it)
 *   variant    0: vec form, adv[T-1]=0, delta = rho*(r + g*V[t+1]*nnt - V[t]), done := term != 0
 *              1: bootstrapped form, delta = rho*r + g*V'*nnt - V[t], V' at T-1 = boot[b],
 *                 done := term > 0.5
 *   time_major element (b,t) at t*B+b; otherwise b*T+t (the reference's segment-major rows)
 *   rho        importance ratios (or log ratios if rho_is_log); NULL means ratio 1 (GAE)
 *   clamp      clamp rewards to [-1,1] (the reference always does)
 *   adv        advantages out; tgt = adv + V out (may be NULL) */
int ph_vtrace(int dtype, const void* rew, const void* val, const void* term, const void* rho,
              const void* boot, size_t B, size_t T, int variant, int time_major, int rho_is_log,
              int clamp, double gamma, double lam, double rhoClip, double cClip, void* adv,
              void* tgt, void* stream);

/* Advantage normalisation out = (adv - mean)/(pop_std + 1e-8) (puffercuda.cu:824-855,
 * NNTrain.lean:274-279). Deterministic reduction. stats (device, 2 elements of dtype: mean,
 * std+eps) may be NULL. */
int ph_adv_normalize(int dtype, const void* adv, size_t n, void* out, void* stats, void* stream);

/* Column sums out[j] (+)= scale * sum_n X[n*ld + j] (k_colsum, puffercuda.cu:676-683). */
int ph_colsum(const float* X, size_t N, size_t J, size_t ld, float* out, float scale,
              int accumulate, void* stream);

/* Elementwise dtype conversion (f64->f32, f32->f64, f64->i32, f32->bf16 RNE). */
int ph_convert(int src_dtype, const void* x, int dst_dtype, void* y, size_t n, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Fused PPO loss gradient, one row per sample (k_ppo_dout + d_vloss_grad, puffercuda.cu:692-744;
 * k_mg_ppo_b, 4910-4930). Row n: logits[n*ldl + 0..A), value values[n*ldv]; act int32; adv, ret,
 * old (behaviour log-prob), ov (old value, NULL disables the value clip) fp32. Writes
 * dlogits[n*ldd + k], dvalues[n*lddv] (ascent sign), optional newlp/newval, and optionally the 7
 * dashboard losses [pg, v, ent, total, old_kl, kl, clipfrac] into device doubles `losses`
 * (puffercuda.cu:5437-5481). max_shift subtracts the row max inside the log-sum-exp. A <= 64. */
int ph_ppo_grad(const float* logits, size_t ldl, const float* values, size_t ldv, const int* act,
                const float* adv, const float* ret, const float* old, const float* ov, size_t N,
                size_t A, float vfCoef, float entCoef, float clipEps, float vfClip, int max_shift,
                float* dlogits, size_t ldd, float* dvalues, size_t lddv, float* newlp,
                float* newval, double* losses, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* GEMM on MFMA. C[MxN] = op(A)[MxK] op(B)[KxN] with a fused epilogue, row-major. Replaces gemm32
 * (cublasGemmEx, puffercuda.cu:661-667) and the cuBLASLt dense layers (pufferblas.c:302-365).
 *   trans_a  A stored [K][M] (lda >= M), else [M][K] (lda >= K)
 *   trans_b  B stored [N][K] (ldb >= K), else [K][N] (ldb >= N)
 *   a/b/c_dtype PH_F32 or PH_BF16; math PH_MATH_BF16 (fp32 accumulate; fp32 inputs rounded to
 *            bf16 RNE) or PH_MATH_F32 (fp32 inputs only)
 *   epilogue ph_epilogue; aux has C's dtype, leading dimension ldaux (0: ldc)
 *   C2       optional bf16 copy of the result, transposed when c2_trans
 *   splits   split-K count (<= 0: chosen from the shape); the fold is deterministic */
int ph_gemm(int trans_a, int trans_b, int M, int N, int K, int a_dtype, const void* A, long lda,
            int b_dtype, const void* B, long ldb, int c_dtype, void* C, long ldc, int math,
            int epilogue, const float* bias, const void* aux, long ldaux, float alpha, float beta,
            void* C2, long ldc2, int c2_trans, int splits, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Muon / Newton-Schulz.
 * Exact tier (f64, device buffers): one Muon matrix step with the reference's op order, bit-exact
 * with the CPU path (muon_mat_cpu, pufferblas.c:1369-1400; muon_mat_dev, puffercuda.cu:892-912).
 * nW/nM may alias W/M. coeffs: nsteps rows of (a, b, c), host memory. */
int ph_muon_mat_f64(int rows, int cols, const double* W, const double* G, const double* M,
                    double* nW, double* nM, double gscale, double lr, double wd, double mu,
                    double eps, const double* coeffs, int nsteps, void* stream);
/* Bias step (stepvec_cpu, pufferblas.c:1403-1406; k_stepvec, puffercuda.cu:880-889). */
int ph_stepvec_f64(size_t n, const double* b, const double* g, const double* m, double* nb,
                   double* nm, double gscale, double lr, double wd, double mu, void* stream);
/* Fast tier (fp32 state, bf16 or fp32 MFMA): in-place NS orthogonalisation of X (rows x cols),
 * X <- NS(X/(|X|_F+eps)) with X <- aX + (bA + cA^2)X, A = XX^T, tall matrices transposed to wide
 * (newtonSchulzWith, Puffer/Float/Muon.lean:73-89, on MFMA; replaces muon_mat_dev_bf,
 * puffercuda.cu:942-966). coeffs: host float[nsteps][3]. */
int ph_newton_schulz(float* X, int rows, int cols, const float* coeffs, int nsteps, float eps,
                     int math, void* stream);
/* In-place Muon matrix step on fp32 state: M <- mu*M + gscale*G; U = gscale*G + mu*M;
 * W <- (1-lr*wd)*W + lr*sqrt(max(1,rows/cols))*NS(U). */
int ph_muon_mat(float* W, const float* G, float* M, int rows, int cols, float gscale, float lr,
                float wd, float mu, float eps, const float* coeffs, int nsteps, int math,
                void* stream);
/* In-place bias step on fp32 state. */
int ph_stepvec(float* b, const float* g, float* m, size_t n, float gscale, float lr, float wd,
               float mu, void* stream);
/* Global grad-norm clip, in place: g <- g*sc*min(1, maxNorm/|g*sc|) (maxNorm <= 0: g*sc)
 * (k_gclip_norm/k_gclip_scale, puffercuda.cu:5122-5131). */
int ph_gclip(float* g, size_t n, float sc, float maxNorm, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* MinGRU policy PPO+Muon minibatch step (the reference's MinGRU trainer chain: cudaMgVtracePrioFFI ->
 * cudaMinGRUPpoGradFFI -> cudaMinGRUMuonResidentFFI, Puffer/RL/MinGRUTrain.lean:814-849;
 * lean_cuda_mingru_ppo_grad puffercuda.cu:5206, lean_cuda_mingru_muon_resident puffercuda.cu:5727).
 * Policy: obs D -> encoder H -> L MinGRU layers of H -> A-way categorical head + value head; params
 * and momentum are fp32 [P] in the reference's flattenMG order [wEnc(H*D) | bEnc(H) | L x W(3H*H) |
 * wDec(A*H) | bDec(A) | wVal(H) | bVal(1)]. All columns are time-major [T][B] (obs [T][B][D]); act is
 * int32; done is 0/1. GEMMs run bf16 MFMA with fp32 accumulate; activations are stored bf16. */
/* precision 0: bf16 activations and weight copies, bf16 MFMA (fp32 accumulate, fp32 master weights
 * and gradient); 1: fp32 throughout on fp32 MFMA (the tight cross-check tier). */
typedef struct { int B, T, D, H, L, A, precision; } ph_mingru_dims;
typedef struct {
  float gamma, lam, rho_clip, c_clip;        /* V-trace */
  float clip_eps, vf_coef, ent_coef, vf_clip; /* PPO loss (vf_clip <= 0: unclipped value loss) */
} ph_ppo_coefs;
typedef struct {
  float lr, wd, mu, eps;     /* Muon */
  float max_grad_norm;       /* global grad-norm clip (<= 0: none) */
  float gscale;              /* gradient scale applied with the clip (1/rows for a mean) */
  int nsteps, math;          /* NS steps, PH_MATH_BF16 or PH_MATH_F32 */
  const float* coeffs;       /* host float[nsteps][3] */
} ph_muon_coefs;
long ph_mingru_param_count(const ph_mingru_dims* d);
/* Forward + backward over one minibatch: G (fp32 [P]) receives the summed gradient of the PPO
 * objective (ascent sign, reference convention), newlp/newval the new log-prob of the taken action
 * and the new value per row, losses (optional, device double[7]) the dashboard losses. adv is the
 * normalised advantage, ret the value target. */
int ph_mingru_ppo_grad(const ph_mingru_dims* d, const ph_ppo_coefs* c, const float* params,
                       const float* obs, const int* act, const float* adv, const float* ret,
                       const float* oldlp, const float* oldval, const float* done, float* G,
                       float* newlp, float* newval, double* losses, void* stream);
/* Grad-norm clip of G (scaled by gscale) then Muon on every matrix, stepvec on every bias, in place
 * on params/mom (the matrices: wEnc, each W_l, wDec, wVal). */
int ph_mingru_muon(const ph_mingru_dims* d, const ph_muon_coefs* m, float* params, float* mom,
                   float* G, void* stream);
/* The whole minibatch step: V-trace (bootstrapped variant on oldval with boot[B]; logrho may be NULL
 * for ratio 1) -> advantage normalisation -> ph_mingru_ppo_grad -> ph_mingru_muon. G is caller
 * scratch of P floats (holds the clipped gradient afterwards). */
int ph_mingru_step(const ph_mingru_dims* d, const ph_ppo_coefs* c, const ph_muon_coefs* m,
                   float* params, float* mom, const float* obs, const int* act, const float* oldlp,
                   const float* oldval, const float* rew, const float* done, const float* logrho,
                   const float* boot, float* G, double* losses, void* stream);

#ifdef __cplusplus
}
#endif
#endif
