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
typedef enum { PH_MATH_BF16 = 0, PH_MATH_F32 = 1 } ph_math;
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

#ifdef __cplusplus
}
#endif
#endif
