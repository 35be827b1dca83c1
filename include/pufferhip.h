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
 *
 * Concurrency. Intermediate buffers (GEMM padding and split-K partials, the MinGRU activations, loss
 * and reduction partials, the Newton-Schulz work items and control words) live in library-owned
 * scratch, one buffer per purpose per device. Two calls in flight at once on different streams of
 * one device race on that scratch: order them on one stream, or make the later stream wait for the
 * earlier. (The library's own concurrent Muon lanes use per-lane scratch.)
 *
 * Graph capture. Every ph_* device entry can be captured into a HIP graph: it launches kernels
 * only (no memset nodes, no host synchronisation). Run each shape once before capturing it, so its
 * scratch already has full size. When a later call needs a larger buffer, the old one is retired,
 * not freed, so a graph captured earlier keeps valid memory; ph_release_scratch() frees retired
 * buffers and must only be called once no graph captured before it will be replayed.
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
/* Free the scratch buffers retired by growth (see "Graph capture" above) after a device
 * synchronisation. Graphs captured before this call must not be replayed after it. */
int ph_release_scratch(void);
/* Number and total bytes of retired scratch buffers on the current device. */
int ph_scratch_retired(size_t* count, size_t* bytes);

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
/* ph_adv_normalize without any device allocation. No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same kernels and fixed-order reduction, so the results are bit-identical to
 * ph_adv_normalize's. The partials (and the statistics when stats is NULL) live in a fixed 64 KB
 * device array per GPU, held until the process ends, so n is limited to 4096 * 4096 = 16,777,216
 * elements (PH_ERR_ARG beyond). Calls on one GPU share that array: calls that overlap in time on one
 * GPU (different streams) race. */
int ph_adv_normalize_noalloc(int dtype, const void* adv, size_t n, void* out, void* stats, void* stream);

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

/* Multi-discrete heads (k_ppo_dout_md, puffercuda.cu:702-727): K categorical heads of head_sizes[K]
 * actions (host array, K <= 32); row n holds the heads' logits back to back, then the value at
 * column W = sum of sizes (stride ldl >= W + 1). act int32 [N][K]. One clipped surrogate on the joint
 * ratio exp(sum_h log softmax_h[a_h] - old); each head's logits get dPol (onehot - p) plus the entropy
 * gradient; dvalue as ph_ppo_grad. Writes dlogits rows (W + 1 columns, stride ldd) and optional
 * newlp (joint) / newval. Log-sum-exp is max-shifted (the reference's is not; equal to rounding).
 * A row with an action outside [0, head_sizes[h]) gets NaN logit gradients and NaN newlp (its value
 * gradient stands); no logit outside the row is read. losses (device doubles, may be NULL): the 7
 * dashboard losses as ph_ppo_grad, the entropy summed over the heads (ff_surface_losses mode 1,
 * puffercuda.cu:1798-1870). */
int ph_ppo_grad_md(const float* logits, size_t ldl, const int* act, const float* adv, const float* ret,
                   const float* old, const float* ov, size_t N, const int* head_sizes, size_t K,
                   float vfCoef, float entCoef, float clipEps, float vfClip, float* dlogits, size_t ldd,
                   float* newlp, float* newval, double* losses, void* stream);
/* Diagonal Gaussian head (k_ppo_dout_cont, puffercuda.cu:1767-1790; CPU twin pufferffi.c:223-330): row n
 * holds d means, d raw log-stds (clamped to [ls_lo, ls_hi]; the reference's GPU path uses [-20, 2], its
 * CPU twin [-5, 2]), the value at 2d. act f32 [N][d]. z = (a - mu) exp(-ls), logp = sum(-z^2/2 - ls -
 * log(2 pi)/2); dmu = dPol z exp(-ls), dls = dPol (z^2 - 1) + ent inside the clamp range, else 0.
 * losses (device doubles, may be NULL): the 7 dashboard losses, entropy sum(ls + (1 + log(2 pi))/2)
 * (ff_surface_losses mode 2, puffercuda.cu:1798-1870). */
int ph_ppo_grad_cont(const float* out, size_t ldo, const float* act, const float* adv, const float* ret,
                     const float* old, const float* ov, size_t N, size_t d, float vfCoef, float entCoef,
                     float clipEps, float vfClip, float ls_lo, float ls_hi, float* dout, size_t ldd,
                     float* newlp, float* newval, double* losses, void* stream);
/* Multi-discrete draw (k_sample_md, puffercuda.cu:1538-1551): head h of row n draws the splitmix64 word of
 * rng + (n+1)*GOLD + (h+1)*0xD1B54A32D192ED03. out (device f64, (K+2)*N) = [actions (head h at
 * h*N + n); joint logp; value]. Y: PH_F32 or PH_F64 rows as for ph_ppo_grad_md. */
int ph_sample_actions_md(int dtype, const void* Y, size_t ldy, size_t N, const int* head_sizes, size_t K,
                         uint64_t rng, double* out, void* stream);
/* Gaussian draw (k_sample_cont, puffercuda.cu:1652-1668): Box-Muller from the words of rng + (n+1)*GOLD +
 * (2i+1)*G2 and (2i+2)*G2 (u1 floored at 1e-7); a = mu + exp(ls) z. out (device f64, (d+2)*N) =
 * [actions (dim i at i*N + n); logp; value]. */
int ph_sample_actions_cont(int dtype, const void* Y, size_t ldy, size_t N, size_t d, uint64_t rng,
                           double ls_lo, double ls_hi, double* out, void* stream);

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
/* The same for a batch of independent matrices X[i] (rows[i] x cols[i]), run concurrently on the
 * library's stream lanes (forked from and joined back into `stream`); results equal n calls of
 * ph_newton_schulz. No counterpart in the reference (its NS walks the matrices in sequence). */
int ph_newton_schulz_batch(float* const* X, const int* rows, const int* cols, int n,
                           const float* coeffs, int nsteps, float eps, int math, void* stream);
/* The bf16 Newton-Schulz launches (ph_newton_schulz, _batch, ph_muon_mat, ph_mingru_muon and
 * ph_mingru_step in bf16 math) run every matrix in one persistent launch whose work items wait, with
 * a bounded spin, for the tiles of earlier phases computed by other workgroups. A wait that reaches
 * its bound lets the launch finish with invalid matrices and records the failure on the device.
 * ph_ns_status synchronises `stream`, reads and clears that record, and returns PH_ERR_HIP (with a
 * message) when a launch since the last check gave up; PH_OK otherwise. Callers of the entries above
 * in bf16 math poll it, e.g. once per update (the weights of an update whose launch gave up are
 * invalid, though usually still finite). These launches share one set of control words per device:
 * two of them must not overlap in time on different streams of one device (order them on one
 * stream). */
int ph_ns_status(void* stream);
/* Spin bound of those waits, in polls of about a microsecond (0 restores the default, 2^20). A tiny
 * bound makes the waits give up; it exists so that the failure report can be tested. */
int ph_ns_set_spin_limit(unsigned polls);
/* Work placement of that launch. Per-XCD queues (on a device of 8 XCDs of 32 CUs, MI355X): each matrix
 * runs on the CUs of one XCD, with its signals and intermediate data in that XCD's L2; faster for small
 * matrices, slower for large ones (32 CUs per matrix). The device-wide queue: signals and data go
 * through memory. 0 (default): per-XCD queues when every Newton-Schulz phase of every matrix has at
 * most 32 output tiles of 64x64 (min(rows, cols) <= 256 or so), the device-wide queue otherwise;
 * 1: always device-wide; 2: per XCD whenever the device has them. All give bit-identical matrices. A
 * queue with work but no workgroups on its XCD is recorded, and ph_ns_status reports it. No
 * counterpart in the reference. */
int ph_ns_set_queues(int mode);
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
/* Prioritised replay: the step between V-trace and the MinGRU BPTT in the reference's trainer
 * (MinGRUTrain.lean:814-834). The rollout columns of N segments x T steps, as the library reads them:
 *   dtype       PH_F64 (the reference's resident columns) or PH_F32, for every column below
 *   time_major  element (e,t) at t*N+e, else e*T+t (the reference's segment-major rows)
 *   K           action components per row (act row holds K values; 0 means 1)
 *   adv         advantages (the V-trace output); value, ratio: the columns the iterate rewrites;
 *   act, logp, term: actions, behaviour log-probs, terminal flags.
 * Unused members may be NULL. */
typedef struct {
  int dtype, time_major;
  size_t N, T, K;
  const void* adv;
  void* value;
  void* ratio;
  const void* act;
  const void* logp;
  const void* term;
} ph_replay_cols;
/* L1[e] = sum_t |adv(e,t)|, t ascending, f64 (k_adv_l1, puffercuda.cu:311-312). Bit-identical to
 * the reference's per-segment sum. L1: device double[N]. */
int ph_seg_l1(const ph_replay_cols* c, double* L1, void* stream);
/* Prioritised draws of Bmb segments with replacement (k_prio_w/sum/scan/draw, puffercuda.cu:400-446;
 * CPU twin lean_ffi_prio_sample, pufferffi.c:1094-1125): w = exp(alpha*log(L1+1e-12)),
 * p = (w+1e-6)/(sum w+1e-6), draw i takes the splitmix64 word of rng+(i+1)*GOLD, u = word>>11 / 2^53
 * * sum p, seg[i] = first e with cum p >= u (N-1 if none), mbprio[i] = exp(-beta*log(N*p[seg]+1e-12)).
 * The caller advances rng by Bmb*GOLD afterwards. One workgroup launch. Sums use a fixed tree
 * order: reproducible, equal to the sequential CPU twin to rounding (a draw within rounding of a
 * cumulative boundary may take the neighbouring segment, as the reference's device sampler may).
 * L1 device double[N]; seg device int[Bmb]; mbprio device double[Bmb]. */
int ph_prio_sample(const double* L1, size_t N, size_t Bmb, double alpha, double beta, uint64_t rng,
                   int* seg, double* mbprio, void* stream);
/* Minibatch gather of the Bmb sampled segments (k_mg_advpart/k_mg_ms_fin/k_mg_gather_scal,
 * puffercuda.cu:472-502; CPU twin lean_ffi_gather_seq_minibatch, pufferffi.c:1126-1200). out (device,
 * the columns' dtype) is the packed [(K+5)*T*Bmb] = [act (K wide) | adv | ret | old | term | ov],
 * timestep-major (row t*Bmb+bi reads segment seg[bi] at step t): act truncated to an integer,
 * adv = mbprio[bi]*(a-mean)/(std+1e-8) with mean and population std of the gathered raw adv,
 * ret = a + value, old = logp, term = term > 0.5, ov = value. mbprio NULL: weight 1. stats (device
 * double[2], may be NULL) receives [mean, std]. A seg entry outside [0,N) gives NaN for its rows.
 * Every column but adv is bit-identical to the CPU twin; mean and std are merged per block in a fixed
 * order (equal to the twin's sequential sums to rounding). */
int ph_mb_gather(const ph_replay_cols* c, const int* seg, const double* mbprio, size_t Bmb, void* out,
                 double* stats, void* stream);
/* Value/ratio iterate from the BPTT outputs (k_mg_lastw/k_mg_iterate, puffercuda.cu:503-511): for every
 * segment drawn, the last draw bi that took it (the writer of an in-order loop over bi) stores
 * ratio(e,t) = exp(newlp[t*Bmb+bi] - logp(e,t)) and value(e,t) = newval[t*Bmb+bi] for all t. newlp and
 * newval are device float[T*Bmb]. seg entries outside [0,N) are ignored. Calls on one device share a
 * last-writer table: calls that overlap in time on different streams race. */
int ph_mb_iterate(const ph_replay_cols* c, const int* seg, size_t Bmb, const float* newlp,
                  const float* newval, void* stream);

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
/* The same with K categorical heads (k_mg_ppo_b_md, puffercuda.cu:4940-4975): d->A is the logits
 * width, the sum of head_sizes[K] (host array); act is int32 [T*B][K]; newlp is the joint log-prob.
 * The loss on the head rows is ph_ppo_grad_md's; the rest of the BPTT is the categorical one. */
int ph_mingru_ppo_grad_md(const ph_mingru_dims* d, const ph_ppo_coefs* c, const int* head_sizes, size_t K,
                          const float* params, const float* obs, const int* act, const float* adv,
                          const float* ret, const float* oldlp, const float* oldval, const float* done,
                          float* G, float* newlp, float* newval, double* losses, void* stream);
/* Grad-norm clip of G (scaled by gscale) then Muon on every matrix, stepvec on every bias, in place
 * on params/mom (the matrices: wEnc, each W_l, wDec, wVal). */
int ph_mingru_muon(const ph_mingru_dims* d, const ph_muon_coefs* m, float* params, float* mom,
                   float* G, void* stream);
/* ---------------------------------------------------------------------------------------------- */
/* MLP policy update on the device. The reference's MLP policy is D -> H (ReLU) -> A+1 (A logits and
 * the value in one head matrix; flattenMLP [W1|b1|W2|b2], pufferblas.c:699-747, puffercuda.cu:748-820);
 * these entries take L >= 1 hidden layers of width H (at most 8) and repeat the hidden layer:
 * params = [W1(H*D) | b1(H) | W2(H*H) | b2(H) | ... | WL | bL | Wo((A+1)*H) | bo(A+1)], fp32. With
 * L = 1 this is flattenMLP. Rows are [N][D] observations; math is PH_MATH_F32 (fp32 MFMA) or
 * PH_MATH_BF16 (bf16 MFMA on the fp32 operands, the reference's FAST_16BF). */
typedef struct { int N, D, H, L, A; } ph_mlp_dims;
long ph_mlp_param_count(const ph_mlp_dims* d);
/* out[N][A+1] = the forward's head outputs (logits, value). */
int ph_mlp_forward(const ph_mlp_dims* d, int math, const float* params, const float* obs, float* out,
                   void* stream);
/* Summed PPO gradient over the N rows into G (fp32 [P], overwritten): the fused loss of ph_ppo_grad
 * without the max shift (as k_ppo_dout), then the backward (lean_cuda_mlp_ppo_grad,
 * puffercuda.cu:748-820, for any L). adv is the (normalised) advantage, ret the value target, old the
 * behaviour log-prob, ov the old value (NULL: no value clip); newlp/newval/losses may be NULL. */
int ph_mlp_ppo_grad(const ph_mlp_dims* d, const ph_ppo_coefs* c, int math, const float* params,
                    const float* obs, const int* act, const float* adv, const float* ret, const float* old,
                    const float* ov, float* G, float* newlp, float* newval, double* losses, void* stream);
/* One whole PPO+Muon update over N = T*B time-major rows (row t*B + b): the forward; per row the
 * log-prob of the taken action and the value; vec-form V-trace (variant 0) with the ratio
 * exp(logp - behav_logp); advantage normalisation; the PPO gradient with old = behav_logp and the
 * V-trace targets as returns; then G scaled by m->gscale and clipped (m->max_grad_norm), Muon on every
 * matrix and stepvec on every bias, in place on params/mom (fp32). The reference runs this chain as
 * computePuffAdvantageV -> normalizeAdv -> lean_cuda_train_step (VecTrain.lean:98-114, NNTrain.lean:
 * 274-279, puffercuda.cu:988-1092). G receives the scaled, clipped gradient. */
int ph_mlp_update(const ph_mlp_dims* d, int T, const ph_ppo_coefs* c, const ph_muon_coefs* m, int math,
                  float* params, float* mom, const float* obs, const int* act, const float* behav_logp,
                  const float* rew, const float* done, float* G, double* losses, void* stream);

/* ---------------------------------------------------------------------------------------------- */
/* Rollout policy forward and categorical sampler: the producers of the behaviour log-prob and value
 * columns the update consumes. */
/* Categorical draw per row (k_sample / k_sample_f32, puffercuda.cu:1429-1460; CPU twin
 * lean_ffi_sample_actions_batch, pufferffi.c:896-918). Y: N rows of logits (dtype PH_F32 or PH_F64,
 * row stride ldy >= A + has_value), the value at column A when has_value. Row n draws the splitmix64
 * word of rng + (n+1)*GOLD, u = word>>11 / 2^53; the action is the first k whose running softmax sum
 * exceeds u (A-1 if none), logp = log(softmax[a]) (max-shifted). act (int32), logp and value (Y's dtype)
 * are device arrays of N, each may be NULL. The caller advances rng by N*GOLD. f64 rows match the CPU
 * twin to an ulp of exp/log: a draw within that of a boundary may take the neighbouring action (as
 * the reference's device sampler may). */
int ph_sample_actions(int dtype, const void* Y, size_t ldy, size_t N, size_t A, int has_value,
                      uint64_t rng, int* act, void* logp, void* value, void* stream);
/* One rollout timestep of the MinGRU policy over N = d->B envs (lean_cuda_mingru_step,
 * puffercuda.cu:2190-2265): params fp32 flattenMG [P], obs [N][D] fp32, state [N][L][H] fp32 updated
 * in place, out [N][A+1] fp32 (A logits, then the value). The cell is the reference's
 * (k_mingru_gate, puffercuda.cu:1949-1959). d->precision 0: bf16 MFMA products (fp32 operands
 * rounded), 1: fp32 MFMA. A + 1 <= 32; d->T is not used. */
int ph_mingru_rollout_step(const ph_mingru_dims* d, const float* params, const float* obs, float* state,
                           float* out, void* stream);

/* The whole minibatch step: V-trace (bootstrapped variant on oldval with boot[B]; logrho may be NULL
 * for ratio 1) -> advantage normalisation -> ph_mingru_ppo_grad -> ph_mingru_muon. G is caller
 * scratch of P floats (holds the clipped gradient afterwards). */
int ph_mingru_step(const ph_mingru_dims* d, const ph_ppo_coefs* c, const ph_muon_coefs* m,
                   float* params, float* mom, const float* obs, const int* act, const float* oldlp,
                   const float* oldval, const float* rew, const float* done, const float* logrho,
                   const float* boot, float* G, double* losses, void* stream);

/* ============================================================================================== */
/* Host-buffer entry points (layer 2). Each replaces the reference GPU symbol named beside it, with
 * the same argument order and meaning; FloatArray inputs become host `const double*`, the returned
 * FloatArray a caller-allocated `double*` of the stated length. All synchronise before returning.
 * Where the reference falls back to its CPU path or returns zeros, these return an error status.
 * Policy handles are device addresses of a [params(P); mom(P)] f64 buffer, as in the reference. */

/* lean_cuda_vtrace (puffercuda.cu:94-136): vec-form V-trace over segment-major [B][T] f64 arrays;
 * imp is the importance ratio, rewards clamped to [-1,1]. adv: B*T. */
int ph_cuda_vtrace(const double* rew, const double* val, const double* term, const double* imp,
                   size_t B, size_t T, double gamma, double lam, double rhoClip, double cClip,
                   double* adv);
/* lean_cuda_vtrace_mingru (puffercuda.cu:168-216): bootstrapped form with bootv[B]. adv: B*T. */
int ph_cuda_vtrace_mingru(const double* rew, const double* val, const double* term, const double* imp,
                          const double* bootv, size_t B, size_t T, double gamma, double lam,
                          double rhoClip, double cClip, double* adv);
/* lean_cuda_adv_normalize (puffercuda.cu:836-855): (adv - mean) / (pop-std + 1e-8). out: n. */
int ph_cuda_adv_normalize(const double* adv, size_t n, double* out);
/* lean_cuda_mlp_ppo_grad (puffercuda.cu:748-820): summed PPO gradient of the one-hidden-layer MLP
 * (flattenMLP params W1[H*D] | b1[H] | W2[O*H] | b2[O], O = A+1). bf16: bf16-MFMA GEMMs on fp32
 * operands, else fp32 MFMA. g: P = H*D + H + O*H + O. */
int ph_cuda_mlp_ppo_grad(const double* params, const double* obs, const double* acts,
                         const double* advs, const double* rets, const double* oldlps, size_t N,
                         size_t H, size_t D, size_t A, double vfCoef, double entCoef, double clipEps,
                         uint8_t bf16, double* g);
/* lean_cuda_train_step (puffercuda.cu:988-1090): pm = [params; mom] (2P); adv-normalise, gradient,
 * mean over N, Muon (the reference's 5-triple schedule; bf16: fp32-MFMA Newton-Schulz with f64
 * state, else the exact f64 tier) on W1, W2, stepvec on b1, b2. out: [newParams; newMom] (2P). */
int ph_cuda_train_step(const double* pm, const double* obs, const double* acts, const double* advRaw,
                       const double* rets, const double* oldlps, size_t N, size_t H, size_t D,
                       size_t A, double lr, double wd, double mu, double eps, double vfCoef,
                       double entCoef, double clipEps, uint8_t bf16, double* out);
/* lean_cuda_train_update (puffercuda.cu:1094-1172): epochs x numMB minibatches (perm: epochs*NT row
 * indices as doubles), exact f64 Muon. out: [params; mom] (2P). */
int ph_cuda_train_update(const double* pm, const double* obs, const double* acts, const double* adv,
                         const double* ret, const double* olp, const double* perm, size_t NT,
                         size_t D, size_t H, size_t A, size_t epochs, size_t numMB, double lr,
                         double wd, double mu, double eps, double vfCoef, double entCoef,
                         double clipEps, uint8_t bf16, double* out);
/* lean_cuda_train_update_resident (puffercuda.cu:1187-1290): as above on a policy handle, in place,
 * with the value-loss clip (when vfClip > 0 and ovN >= NT) and the global grad-norm clip
 * (maxGradNorm > 0); bf16 also selects the fp32-MFMA Newton-Schulz. Fills the dashboard-loss channel
 * on the last minibatch when enabled. out1: params[0]. */
int ph_cuda_train_update_resident(size_t policyH, const double* obs, const double* acts,
                                  const double* adv, const double* ret, const double* olp,
                                  const double* ov, size_t ovN, const double* perm, size_t NT, size_t D,
                                  size_t H, size_t A, size_t epochs, size_t numMB, double lr, double wd,
                                  double mu, double eps, double vfCoef, double entCoef, double clipEps,
                                  double vfClip, double maxGradNorm, uint8_t bf16, double* out1);
/* lean_cuda_train_update_wide_resident (puffercuda.cu:1307-1411): the whole resident update for
 * multi-discrete (mode 1: Wdim heads of sizes hs[0..Wdim), O = sum + 1) and Gaussian (mode 2: Wdim
 * dims, O = 2 Wdim + 1) policies. acts: NT x Wdim row-major. hs/hsN: the head sizes as doubles (read
 * in mode 1 only). Otherwise as ph_cuda_train_update_resident, except that Newton-Schulz is always
 * the exact f64 one, as in the reference. Every perm entry must lie in [0, NT) (all whole-update
 * entries check this on the host; the reference would read out of bounds). out1: params[0]. */
int ph_cuda_train_update_wide_resident(size_t policyH, const double* obs, const double* acts,
                                       const double* adv, const double* ret, const double* olp,
                                       const double* ov, size_t ovN, const double* perm, const double* hs,
                                       size_t hsN, size_t NT, size_t D, size_t H, size_t O, size_t Wdim,
                                       uint32_t mode, size_t epochs, size_t numMB, double lr, double wd,
                                       double mu, double eps, double vfCoef, double entCoef,
                                       double clipEps, double vfClip, double maxGradNorm, uint8_t bf16,
                                       double* out1);
/* lean_cuda_muon_stepmat (puffercuda.cu:557-631): exact f64 Muon of one matrix. out: [newW; newMom]. */
int ph_cuda_muon_stepmat(const double* W, const double* G, const double* M, size_t rows, size_t cols,
                         double lr, double wd, double mu, double eps, double* out);
/* lean_cuda_muon_step_mlp_resident (puffercuda.cu:5985-6011): gRaw (P) scaled by gscale, exact f64
 * Muon on the handle in place. newParams: P. */
int ph_cuda_muon_step_mlp_resident(size_t policyH, const double* gRaw, size_t H, size_t D, size_t O,
                                   double gscale, double lr, double wd, double mu, double eps,
                                   double* newParams);
/* lean_cuda_policy_load / _download / _free (puffercuda.cu:6100-6116). */
int ph_cuda_policy_load(const double* pm, size_t P, size_t* handle);
int ph_cuda_policy_download(size_t handle, size_t P, double* pm);
int ph_cuda_policy_free(size_t handle);
/* Checkpoint byte layout of the trainers (ckptToBytes / bytesToCkpt, Puffer/RL/FFITrain.lean:40-69):
 * [P as u64 little-endian][P doubles as their IEEE bits, little-endian], 8 (P + 1) bytes.
 * ph_ckpt_decode reports P = min(header, whole doubles present), as bytesToCkpt does for a short
 * file; with w NULL it only reports P. Host-only: no device needed. */
size_t ph_ckpt_bytes(size_t P);
int ph_ckpt_encode(const double* w, size_t P, uint8_t* out);
int ph_ckpt_decode(const uint8_t* b, size_t nbytes, double* w, size_t cap, size_t* P_out);
/* The same layout straight from / into a resident policy handle (savePolicyCheckpoint after
 * policyDownloadFFI, MinGRUTrain.lean:866-873; the load path 680-692): save writes the handle's P
 * weights (not the momentum) to out (ph_ckpt_bytes(P) bytes); load makes a new handle of
 * [weights; zero momentum] and rejects a checkpoint whose parameter count differs from P. */
int ph_cuda_policy_save_ckpt(size_t handle, size_t P, uint8_t* out);
int ph_cuda_policy_load_ckpt(const uint8_t* b, size_t nbytes, size_t P, size_t* handle);
/* lean_cuda_mg_loss_enable / lean_cuda_mg_read_losses (puffercuda.cu:336-352): the 7 dashboard
 * losses (policy, value, entropy, total, old_kl, kl, clipfrac) of the last surfaced minibatch. */
int ph_cuda_mg_loss_enable(uint8_t on);
int ph_cuda_mg_read_losses(double* out7);
extern int g_mgLossOn;      /* link-time contract of pufferblas.c:38-39 */
extern double g_mgLoss[7];
/* pufferblas.c:46-50 link-time contract: always 0 here (the GPU LSTM BPTT is not in this library),
 * which makes pufferblas.c take its CPU path. */
int cuda_lstm_ppo_grad_batch(const double* pp, const double* obsB, const double* actA,
                             const double* advA, const double* retA, const double* oldA,
                             const double* termA, const double* h0s, const double* c0s, size_t B,
                             size_t T, size_t H, size_t D, size_t A, double vfCoef, double entCoef,
                             double clipEps, double* gOut, double* outHostOrNull, int tier);
/* lean_ffi_dense_forward_cublas (pufferblas.c:111-147): Y = relu(X W^T + b), f64 (each dot product
 * an ascending fold, the order of lean_ffi_dense_forward_ref). Y: N*H. */
int ph_ffi_dense_forward_gpu(const double* X, const double* W, const double* b, size_t N, size_t D,
                             size_t H, double* Y);
/* lean_ffi_dense_forward_cublaslt_bf16 (pufferblas.c:190-249): bf16 (RNE) operands, fp32 MFMA
 * accumulate, bias and ReLU in f64. Y: N*H. */
int ph_ffi_dense_forward_bf16(const double* X, const double* W, const double* b, size_t N, size_t D,
                              size_t H, double* Y);
/* lean_ffi_mlp_forward_batch_cublaslt_bf16 (pufferblas.c:373-416): flattenMLP forward, bf16 MFMA on
 * fp32 operands, fused bias+ReLU / bias. Y: N*O. */
int ph_ffi_mlp_forward_batch_bf16(const double* p, const double* X, size_t N, size_t D, size_t H,
                                  size_t O, double* Y);
/* lean_ffi_bench_cublaslt_bf16_resident (pufferblas.c:256-292): device-resident bf16 dense-layer
 * GFLOP/s over reps launches; -1 without a device. */
double ph_ffi_bench_bf16_resident(size_t N, size_t D, size_t H, size_t reps);
/* lean_ffi_cuda_available (pufferblas.c:1348-1352). */
uint8_t ph_ffi_cuda_available(void);
/* The persistent resident MLP policy of the rollout (lean_ffi_mlp_policy_load / _update / _forward /
 * _free, pufferblas.c:460-592): flattenMLP weights [W1(H*D) | b1(H) | W2(O*H) | b2(O)] uploaded once
 * (W1 as bf16 RNE of its fp32 value, the rest fp32) into an opaque handle on the current device; the
 * forward sends the N x D observations up as bf16, runs relu(X W1^T + b1) (bf16 products, fp32 out,
 * kept on the device) then (. W2^T + b2) (bf16 MFMA on fp32), and returns Y[N*O] f64. update re-uploads
 * the weights (dims unchanged); free releases the handle. Where the reference falls back to its host
 * weights or returns 0, these return an error status. */
int ph_ffi_mlp_policy_load(const double* params, size_t D, size_t H, size_t O, size_t* handle);
int ph_ffi_mlp_policy_update(size_t handle, const double* params);
int ph_ffi_mlp_policy_forward(size_t handle, const double* X, size_t N, double* Y);
int ph_ffi_mlp_policy_free(size_t handle);
/* The handle's output width O (0 for a null handle): the forward returns N*O values. */
size_t ph_ffi_mlp_policy_outputs(size_t handle);
/* lean_ffi_bench_mlp2_bf16_resident (pufferblas.c:421-452): GF/s (2ND*H + 2NHO per forward) of `reps`
 * device-resident two-layer forwards (after 5 warm-up passes); lean_ffi_bench_mlp2_bf16_wres
 * (pufferblas.c:598-636): the same with the bf16 observations uploaded and the outputs downloaded
 * (pinned staging) every forward. -1 without a device. */
double ph_ffi_bench_mlp2_bf16_resident(size_t N, size_t D, size_t H, size_t O, size_t reps);
double ph_ffi_bench_mlp2_bf16_wres(size_t N, size_t D, size_t H, size_t O, size_t reps);
/* lean_cuda_selftest (puffercuda.cu:41-60): out[i] = 2i + 1 computed on the device (n values). */
int ph_cuda_selftest(size_t n, double* out);
/* lean_cuda_mingru_ppo_grad (puffercuda.cu:5206): params (flattenMG, P), obs (nobs >= T*B*D, host,
 * time-major; or nobs = 0 in the device-column mode, which gathers the minibatch from the resident obs
 * trajectory of ph_cuda_mg_obs_traj by the drawn segments, as the reference gathers its rollout's),
 * K heads (K <= 1: one categorical head over A logits; K > 1: hs[K] (nhs >= K) holds the head sizes as
 * doubles, summing to A, and every action field below is K wide). Two scalar sources, chosen as the
 * reference chooses them:
 *   device-column mode: (nseg > 0 and nprio > 0: host segIdx[B] as doubles and mbPrio[B]) or (both 0
 *     and a fresh sampler result of B draws from ph_cuda_mg_vtrace_prio, consumed here), with the
 *     resident columns of ph_cuda_mg_prep for this T and K: the scalars are gathered on the device
 *     (ph_mb_gather) and, after the BPTT, value/ratio of the drawn segments are iterated in place
 *     (ph_mb_iterate), exactly the reference's order;
 *   host mode: scal = [act (K per row)|adv|ret|old|term|ov] (nscal >= (K+5)*T*B).
 * The returned length is the mode, as the reference's return size (Puffer/Float/CUDA.lean:138-148,
 * puffercuda.cu:5237-5248, 5560-5580):
 *   *out_len = 0 (resident): the device-column mode leaves the summed gradient on the device for the
 *     next ph_cuda_mingru_muon_resident with an empty gClip, copies nothing back and does not wait;
 *   *out_len = P + 2*T*B (host): out receives [g (P); new_logp (T*B); new_value (T*B)]; the host mode
 *     always, the device-column mode only if the resident gradient buffer cannot be allocated.
 * out must hold P + 2*T*B. params: nparams >= P host weights, or nparams = 0 to take the weights the
 * last resident Muon step left in its policy handle (the reference's g_mgw hand-off).
 * Precision: bf16 activations and MFMA when PUFFER_MG_PREC=bf16, else fp32. */
int ph_cuda_mingru_ppo_grad(const double* params, size_t nparams, const double* obs, size_t nobs,
                            const double* scal, size_t nscal, size_t B, size_t T, size_t H, size_t D, size_t L,
                            size_t A, size_t K, const double* hs, size_t nhs, double vfCoef, double entCoef,
                            double clipEps, double vfClip, const double* segIdx, size_t nseg,
                            const double* mbPrio, size_t nprio, double* out, size_t* out_len);
/* No counterpart in the reference (a test and debugging aid): copies the unconsumed resident gradient
 * (P values) to out without consuming it. */
int ph_cuda_mg_resident_grad(size_t P, double* out);
/* Prioritised replay, host-buffer forms. The resident columns are library-owned, one set per
 * process (the reference's g_dc* buffers), bound to the device current at ph_cuda_mg_prep. */
/* lean_cuda_mg_prep (puffercuda.cu:316-336): upload the rollout columns rew, term, logp, val (N*T
 * each, segment-major), act (N*T*K) and boot (N); value := val, ratio := 1. K = 0 means 1. */
int ph_cuda_mg_prep(const double* rew, const double* term, const double* act, const double* logp,
                    const double* val, const double* boot, size_t N, size_t T, size_t K);
/* lean_cuda_mg_cols_ready (puffercuda.cu:305-309): *ready = 1 when a rollout stamped the resident
 * columns for (N, T). This library has no rollout, so it is always 0 and ph_cuda_mg_prep is needed. */
int ph_cuda_mg_cols_ready(size_t N, size_t T, uint8_t* ready);
/* No counterpart in the reference: its rollout entries store the obs trajectory the device-column
 * gradient reads (g_dMGObsTraj, puffercuda.cu:2136, written at 4116-4403 and 4598-4843) while they step
 * the env plugins, which this library does not run. A caller whose rollout runs elsewhere stores it
 * here: obs N*T*D f64, row e*T+t (segment-major), kept as f32 on the current device. */
int ph_cuda_mg_obs_traj(const double* obs, size_t N, size_t T, size_t D);
/* lean_cuda_mg_vtrace (puffercuda.cu:386-399): bootstrapped V-trace on the resident columns (ratio,
 * value) into the resident advantages, and L1out[N] = sum_t |adv| per segment. */
int ph_cuda_mg_vtrace(size_t N, size_t T, double gamma, double lam, double rhoClip, double cClip,
                      double* L1out);
/* lean_cuda_mg_vtrace_prio (puffercuda.cu:447-470): V-trace, L1 and the prioritised sampler of
 * mbSegs draws, all on the device; the draws stay resident for the next ph_cuda_mingru_ppo_grad.
 * *used = 1, or 0 when PUFFER_MG_DEVPRIO=0 (the caller then takes the two-call path: ph_cuda_mg_vtrace
 * + ph_ffi_prio_sample). Fails when ph_cuda_mg_prep was not called for (N, T). Does not synchronise. */
int ph_cuda_mg_vtrace_prio(size_t N, size_t T, double gamma, double lam, double rhoClip, double cClip,
                           size_t mbSegs, double prioAlpha, double annealBeta, uint64_t rng,
                           uint8_t* used);
/* lean_ffi_prio_sample (pufferffi.c:1094-1125) on the device: advL1[N] in, idx[mbSegs] (segment
 * indices as doubles) and mbPrio[mbSegs] out. Same formulas and tolerance as ph_prio_sample. */
int ph_ffi_prio_sample(const double* advL1, size_t N, size_t T, size_t mbSegs, double prioAlpha,
                       double annealBeta, uint64_t rng, double* idx, double* mbPrio);
/* lean_ffi_gather_seq_minibatch (pufferffi.c:1126-1200) on the device: the N*T segment-major columns
 * act, logp, term, advFlat, valueBuf and segIdx/mbPrio[Bmb] in; out[6*T*Bmb] = [act|adv|ret|old|
 * term|ov] timestep-major. obsCol is not read (the reference ignores it too; may be NULL). */
int ph_ffi_gather_seq_minibatch(const double* obsCol, const double* actCol, const double* logpCol,
                                const double* termCol, const double* advFlat, const double* valueBuf,
                                const double* segIdx, const double* mbPrio, size_t T, size_t Bmb,
                                size_t D, size_t N, double* out);
/* lean_cuda_sample_actions (puffercuda.cu:1521-1536): Y N*O f64 (A logits, the value at column A),
 * out[3N] = [act; logp; value]. Same draw as ph_sample_actions on f64 rows. */
int ph_cuda_sample_actions(const double* Y, size_t N, size_t A, size_t O, uint64_t rng, double* out);
/* lean_cuda_mingru_step (puffercuda.cu:2190-2265): params (flattenMG, P), obs N*D, state N*L*H
 * ([n][l][h]); out[N*O + N*L*H] = [logits and value per env (O = A+1); new state]. bf16 selects bf16
 * MFMA products, else fp32. */
int ph_cuda_mingru_step(const double* params, const double* obs, const double* state, size_t N, size_t D,
                        size_t H, size_t L, size_t A, uint8_t bf16, double* out);
/* lean_cuda_mlp_forward (puffercuda.cu:6038-6060): flattenMLP params, obs N*D; out[N*O] =
 * relu(obs W1^T + b1) W2^T + b2. bf16 selects bf16 MFMA products, else fp32. */
int ph_cuda_mlp_forward(const double* params, const double* obs, size_t N, size_t D, size_t H, size_t O,
                        uint8_t bf16, double* out);
/* lean_cuda_sample_actions_md (puffercuda.cu:1553-1568): Y N*O f64, hs K head sizes as doubles;
 * out[(K+2)*N] = [actions (head-major); joint logp; value]. */
int ph_cuda_sample_actions_md(const double* Y, const double* hs, size_t N, size_t K, size_t O, uint64_t rng,
                              double* out);
/* lean_cuda_sample_actions_cont (puffercuda.cu:1670-1684): Y N*O f64 (O = 2d+1), log-std clamp [-20, 2];
 * out[(d+2)*N] = [actions (dim-major); logp; value]. */
int ph_cuda_sample_actions_cont(const double* Y, size_t N, size_t d, size_t O, uint64_t rng, double* out);
/* lean_cuda_mlp_ppo_grad_md (puffercuda.cu:1570-1650): flattenMLP with O = sum(hs) + 1 outputs, acts N*K,
 * the multi-discrete head loss; g: P summed gradient. */
int ph_cuda_mlp_ppo_grad_md(const double* params, const double* obs, const double* acts, const double* advs,
                            const double* rets, const double* oldlps, const double* hs, size_t N, size_t H,
                            size_t D, size_t K, double vfCoef, double entCoef, double clipEps, uint8_t bf16,
                            double* g);
/* lean_cuda_mlp_ppo_grad_cont (puffercuda.cu:1873-1940): flattenMLP with O = 2d+1 outputs, acts N*d,
 * the Gaussian head loss (log-std clamp [-20, 2]); g: P summed gradient. */
int ph_cuda_mlp_ppo_grad_cont(const double* params, const double* obs, const double* acts, const double* advs,
                              const double* rets, const double* oldlps, size_t N, size_t H, size_t D, size_t d,
                              double vfCoef, double entCoef, double clipEps, uint8_t bf16, double* g);
/* lean_cuda_mingru_muon_resident (puffercuda.cu:5727-5976): Muon on every flattenMG matrix of the
 * handle (fp32-MFMA Newton-Schulz on f64 state; PUFFER_MUON_EXACT=1: exact f64), stepvec on the
 * biases, in place. Two gradient forms, as the reference's:
 *   nG >= P (host): gClip is the gradient, already clipped by the caller; wOut (P) receives the new
 *     weights, *wOut_len = P;
 *   nG = 0 (resident): consumes the gradient the last device-column ph_cuda_mingru_ppo_grad left on the
 *     device, clips it there (s = sum (g*gscale)^2; cc = (maxGradNorm > 0 and sqrt(s) > maxGradNorm ?
 *     maxGradNorm/sqrt(s) : 1)*gscale, k_gclip_norm/k_gclip_scale, puffercuda.cu:5122-5131), copies
 *     nothing back and does not wait, *wOut_len = 0; an error if no such gradient is present.
 * Either way the next ph_cuda_mingru_ppo_grad may pass nparams = 0 to use the new weights. */
int ph_cuda_mingru_muon_resident(size_t policyH, const double* gClip, size_t nG, size_t H, size_t D,
                                 size_t L, size_t A, double lr, double wd, double mu, double eps,
                                 double maxGradNorm, double gscale, double* wOut, size_t* wOut_len);

#ifdef __cplusplus
}
#endif
#endif
