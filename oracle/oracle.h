/* CPU oracle for the pufferlean training-step hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: only the tests, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py load it. The product (libpufferhip.so)
 * never links, loads or calls it, and has no CPU fallback.
 *
 * Every function restates the reference's own CPU path in f64 (built with -ffp-contract=off so the
 * op order below is the op order executed). Each cites the reference file:line it follows.
 * Pinning (what checks each function beyond retyping its formula) is listed in oracle.c's header.
 */
#ifndef PUFFER_ORACLE_H
#define PUFFER_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic generator: splitmix64 (Puffer/RL/Train.lean:18-28) ---- */
uint64_t orc_rng_next(uint64_t* state);
double orc_uniform01(uint64_t word);
/* randF lo hi, n times (Exe/Puffer.lean:65-67). */
void orc_randf(double* out, size_t n, double lo, double hi, uint64_t* state);

/* ---- V-trace / GAE ---- */
/* vec-form V-trace, segment-major [B][T] (puffercuda.cu:120-132; VecTrain.lean:98-114). */
void orc_vtrace_vec(const double* rew, const double* val, const double* term, const double* imp,
                    size_t B, size_t T, double gamma, double lam, double rhoClip, double cClip,
                    double* adv);
/* MinGRU-form V-trace with bootstrap, segment-major (puffercuda.cu:200-211; VecTrain.lean:122-139). */
void orc_vtrace_mingru(const double* rew, const double* val, const double* term, const double* imp,
                       const double* bootv, size_t B, size_t T, double gamma, double lam,
                       double rhoClip, double cClip, double* adv);
/* GAE SoA, no bootstrap: out = [adv(NT); ret(NT)] (pufferffi.c:946-971). */
void orc_gae_soa(const double* vals, const double* rews, const double* terms, size_t N, size_t T,
                 double gamma, double lam, double* out);
/* GAE with bootstrap + global adv normalisation, time-major: out = [adv; ret] (pufferffi.c:980-1010). */
void orc_gae_boot_norm(const double* vals, const double* rews, const double* terms,
                       const double* bootv, size_t N, size_t T, double gamma, double lam,
                       double* out);

/* General V-trace (layout / variant / log-ratio / clamp as parameters), in f64 and in an f32 twin with
 * the identical op order. variant 0 = vec form (a1), 1 = bootstrapped MinGRU form (a2).
 * time_major: element (b,t) at t*B+b, else b*T+t. rho_is_log: rho input is log ratio (ratio = exp).
 * clamp: clamp rewards to [-1,1]. boot may be NULL for variant 0. tgt = adv + V (may be NULL). */
void orc_vtrace_f64(const double* rew, const double* val, const double* term, const double* rho,
                    const double* boot, size_t B, size_t T, int variant, int time_major,
                    int rho_is_log, int clamp, double gamma, double lam, double rhoClip,
                    double cClip, double* adv, double* tgt);
void orc_vtrace_f32(const float* rew, const float* val, const float* term, const float* rho,
                    const float* boot, size_t B, size_t T, int variant, int time_major,
                    int rho_is_log, int clamp, float gamma, float lam, float rhoClip, float cClip,
                    float* adv, float* tgt);

/* ---- advantage normalisation (NNTrain.lean:274-279; puffercuda.cu:847-851) ---- */
void orc_adv_normalize(const double* adv, size_t n, double* out);

/* ---- PPO loss gradient per row (pufferblas.c:726-736; puffercuda.cu:692-700, 730-744, 4910-4930).
 * logits row n at logits[n*ldl], value at values[n*ldv]. act/adv/ret/old per row; ov (old values)
 * may be NULL (then no value clip). max_shift: subtract the row max inside the log-sum-exp (the MinGRU
 * form); 0 reproduces pufferblas.c exactly. Outputs dlogits[n*ldd+k], dvalues[n*lddv]; newlp/newval
 * may be NULL. Ascent sign. */
void orc_ppo_grad(const double* logits, size_t ldl, const double* values, size_t ldv,
                  const double* act, const double* adv, const double* ret, const double* old,
                  const double* ov, size_t N, size_t A, double vfCoef, double entCoef,
                  double clipEps, double vfClip, int max_shift, double* dlogits, size_t ldd,
                  double* dvalues, size_t lddv, double* newlp, double* newval);
/* The 7 dashboard losses [pg, v, ent, total, old_kl, kl, clipfrac] over N rows (means),
 * PufferLib's decomposition (puffercuda.cu:5437-5481). */
void orc_ppo_losses(const double* logits, size_t ldl, const double* values, size_t ldv,
                    const double* act, const double* adv, const double* ret, const double* old,
                    const double* ov, size_t N, size_t A, double vfCoef, double entCoef,
                    double clipEps, double vfClip, double* losses7);

/* ---- GEMM (row-major, f64). C = alpha*op(A)*op(B) + beta*C. op(A) is MxK, op(B) is KxN.
 * Follows cblas_dgemm(CblasRowMajor, ...) semantics (pufferblas.c:720-743). threads<=1: serial. */
void orc_gemm(int transA, int transB, size_t M, size_t N, size_t K, double alpha, const double* A,
              size_t lda, const double* B, size_t ldb, double beta, double* C, size_t ldc,
              int threads);

/* ---- MLP forward / PPO gradient (pufferblas.c:65-97, 644-690, 699-747) ---- */
void orc_dense_forward(const double* X, const double* W, const double* b, size_t N, size_t D,
                       size_t H, double* Y);
void orc_mlp_forward(const double* params, const double* X, size_t N, size_t D, size_t H, size_t O,
                     double* Y);
void orc_mlp_ppo_grad(const double* params, const double* obs, const double* act,
                      const double* adv, const double* ret, const double* old, size_t N, size_t H,
                      size_t D, size_t A, double vfCoef, double entCoef, double clipEps, double* g,
                      int threads);
void orc_mlp_deep_ppo_grad(const double* p, const double* obs, const double* act, const double* adv,
                           const double* ret, const double* old, const double* ov, size_t N, size_t D,
                           size_t H, size_t L, size_t A, double vfCoef, double entCoef, double clipEps,
                           double vfClip, double* g, double* newlp, double* newval, int threads);

/* ---- Muon / Newton-Schulz ---- */
/* The reference's 5-triple schedule (pufferblas.c:1362-1364). */
extern const double ORC_MUON_COEFFS[5][3];
/* NS orthogonalisation of X0 (rows x cols), nsteps with coeffs[nsteps][3].
 * form 0: the reference's order (pufferblas.c:1379-1398): X=X0/(|X0|+eps); rows<=cols: A=XX^T, P=AX,
 *         Q=AP, else A=X^TX, P=XA, Q=PA; X=aX+bP+cQ.
 * form 1: transpose-to-wide with X <- aX + (bA + cA^2)X, A=XX^T (tools/puffer_ref.py:31-40 order). */
void orc_newton_schulz(const double* X0, int rows, int cols, const double* coeffs, int nsteps,
                       double eps, int form, double* out);
/* One Muon matrix step (pufferblas.c:1369-1400): Nesterov, NS, decoupled wd. */
void orc_muon_mat(int rows, int cols, const double* W, const double* G, const double* M, double* nW,
                  double* nM, double gscale, double lr, double wd, double mu, double eps,
                  const double* coeffs, int nsteps, int form);
/* Bias step (pufferblas.c:1403-1406). */
void orc_stepvec(int n, const double* b, const double* g, const double* m, double* nb, double* nm,
                 double gscale, double lr, double wd, double mu);
/* Whole-MLP Muon over [params(P); mom(P)] (pufferblas.c:1411-1428): out = [newParams; newMom]. */
void orc_muon_step_mlp(const double* pm, const double* g, size_t H, size_t D, size_t O,
                       double gscale, double lr, double wd, double mu, double eps, double* out);
/* Global grad-norm clip, in place: g <- g * (gnorm>maxNorm ? maxNorm/gnorm : 1) * sc with
 * gnorm = |g*sc| (puffercuda.cu:5122-5131). Returns gnorm. */
double orc_gclip(double* g, size_t P, double sc, double maxNorm);

/* ---- MinGRU ---- */
/* Single-sequence MinGRU PPO BPTT (pufferffi.c:763-876). out = [grad(P); newlogp(T); newval(T)]. */
void orc_mingru_ppo_grad_seq(const double* params, const double* obsSeq, const double* acts,
                             const double* advs, const double* rets, const double* oldlps,
                             const double* terms, const double* oldvals, size_t T, size_t H,
                             size_t D, size_t L, size_t A, double vfCoef, double entCoef,
                             double clipEps, double vfClip, double* out);
/* The same with K heads of sizes[K] summing to A; acts [T][K]; new_logp is the joint log-prob. */
void orc_mingru_ppo_grad_seq_md(const double* p, const double* obsSeq, const double* acts, const double* advs,
                                const double* rets, const double* oldlps, const double* terms,
                                const double* oldvals, size_t T, size_t H, size_t D, size_t L, size_t A,
                                const int* sizes, size_t K, double vfCoef, double entCoef, double clipEps,
                                double vfClip, double* out);
/* Log-space (Heinsen) parallel-scan form of the MinGRU layer recurrence for one sequence with zero
 * initial state and no resets: given gate/hid pre-activations (T x H) returns o (T x H)
 * (Puffer/Net/MinGRU.lean:116-168; tools/mingru_ref.py:113-154). */
void orc_mingru_heinsen(const double* gate, const double* hid, size_t T, size_t H, double* o);

/* ---- prioritised replay (the MinGRU minibatch chain, MinGRUTrain.lean:814-834) ---- */
/* L1[e] = sum_t |adv[e*T+t]|, t ascending (k_adv_l1, puffercuda.cu:311-312). */
void orc_seg_l1(const double* adv, size_t N, size_t T, double* L1);
/* lean_ffi_prio_sample (pufferffi.c:1094-1125): idx[mbSegs] (as doubles) and mbPrio[mbSegs]; probs and
 * cum (N each, may be NULL) receive the normalised probabilities and their running sum. */
void orc_prio_sample(const double* L1, size_t N, size_t mbSegs, double alpha, double beta, uint64_t rng,
                     double* idx, double* mbPrio, double* probs, double* cum);
/* lean_ffi_gather_seq_minibatch (pufferffi.c:1126-1200): out[6*T*Bmb] = [act|adv|ret|old|term|ov],
 * timestep-major; stats2 (may be NULL) = [advMean, advStd]. Columns are N*T segment-major. */
void orc_gather_seq_minibatch(const double* act, const double* logp, const double* term,
                              const double* adv, const double* value, const double* segIdx,
                              const double* mbPrio, size_t T, size_t Bmb, double* out, double* stats2);
/* The value/ratio iterate as an in-order loop over the draws (puffercuda.cu:500-511: the device form
 * is defined as equal to this loop): for bi = 0..Bmb-1, t = 0..T-1 with e = seg[bi], si = e*T+t,
 * os = t*Bmb+bi: ratio[si] = exp((double)newlp[os] - logp[si]); value[si] = newval[os]. */
void orc_mb_iterate(double* value, double* ratio, const double* logp, const float* newlp,
                    const float* newval, const double* seg, size_t Bmb, size_t T);

/* ---- rollout policy forward and sampler ---- */
/* lean_ffi_sample_actions_batch (pufferffi.c:896-918): Y is N x O row-major (A logits, then the value
 * at column A); row n draws the splitmix64 word of rng + (n+1)*GOLD. out = [act(N); logp(N); value(N)]. */
void orc_sample_actions(const double* Y, size_t N, size_t A, size_t O, uint64_t rng, double* out);
/* One rollout timestep of the MinGRU policy for N envs (lean_cuda_mingru_step, puffercuda.cu:2190-2265,
 * the cell of k_mingru_gate 1949-1959): params in flattenMG order, obs N*D, state N*L*H ([n][l][h]).
 * out = [N*O (A logits, then the value, per env); new state N*L*H]. */
void orc_mingru_step(const double* p, const double* obs, const double* state, size_t N, size_t D,
                     size_t H, size_t L, size_t A, double* out);

/* ---- multi-discrete and continuous heads ---- */
/* k_ppo_dout_md (puffercuda.cu:702-727) in f64: row n of out (stride ldo) holds the K heads' logits
 * (sizes[h] each, W in all) then the value at W; act N x K. Writes dout (W+1 per row, stride ldd),
 * newlp (joint log-prob) and newval (may be NULL). Ascent sign. */
void orc_ppo_grad_md(const double* out, size_t ldo, const double* act, const double* adv, const double* ret,
                     const double* old, const double* ov, size_t N, const int* sizes, size_t K, double vf,
                     double ent, double clip, double vfClip, double* dout, size_t ldd, double* newlp,
                     double* newval);
/* k_ppo_dout_cont (puffercuda.cu:1767-1790; pufferffi.c:223-330) in f64: row n holds d means, d raw
 * log-stds (clamped to [lslo, lshi]) and the value at 2d; act N x d. */
void orc_ppo_grad_cont(const double* out, size_t ldo, const double* act, const double* adv, const double* ret,
                       const double* old, const double* ov, size_t N, size_t d, double vf, double ent,
                       double clip, double vfClip, double lslo, double lshi, double* dout, size_t ldd,
                       double* newlp, double* newval);
/* k_sample_md (puffercuda.cu:1538-1551): out[(K+2)N] = [actions (head-major); joint logp; value]. */
/* Dashboard losses of multi-discrete (mode 1) / Gaussian (mode 2) heads (ff_surface_losses). */
void orc_wide_losses(int mode, const double* out, size_t ldo, const double* act, const double* adv,
                     const double* ret, const double* old, const double* ov, size_t N, const int* sizes, size_t K,
                     size_t d, double vfCoef, double entCoef, double clipEps, double vfClip, double lslo,
                     double lshi, double* L);
void orc_sample_md(const double* Y, size_t ldy, size_t N, const int* sizes, size_t K, uint64_t rng,
                   double* out);
/* k_sample_cont (puffercuda.cu:1652-1668): out[(d+2)N] = [actions (dim-major); logp; value]. */
void orc_sample_cont(const double* Y, size_t ldy, size_t N, size_t d, uint64_t rng, double lslo, double lshi,
                     double* out);

/* timed CPU baselines */
int orc_set_threads(int n);
void orc_vtrace_f32_mt(const float* rew, const float* val, const float* term, const float* rho,
                       const float* boot, size_t B, size_t T, int variant, int time_major, int rho_is_log,
                       int clamp, float gamma, float lam, float rhoClip, float cClip, float* adv, float* tgt,
                       int threads);
void orc_gemm_blocked(int transA, int transB, size_t M, size_t N, size_t K, const double* A, size_t lda,
                      const double* B, size_t ldb, double* C, size_t ldc, int threads);
void orc_mingru_ppo_grad_batch(const double* p, const double* obs, const double* act, const double* adv,
                               const double* ret, const double* old, const double* term, const double* ov,
                               size_t B, size_t T, size_t H, size_t D, size_t L, size_t A, double vfCoef,
                               double entCoef, double clipEps, double vfClip, double* out, int threads);

#ifdef __cplusplus
}
#endif
#endif
