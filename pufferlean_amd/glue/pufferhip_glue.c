/* Lean @[extern] bodies over libpufferhip: the drop-in for ffi/puffercuda.cu and the GPU entries of
 * ffi/pufferblas.c. Every GPU symbol that Puffer/Float/CUDA.lean and Puffer/Float/BLAS.lean bind is
 * defined here with the reference's prototype; each unpacks its FloatArrays, calls the host-buffer
 * entry of include/pufferhip.h that mirrors it, and packs the result.
 *
 * Ownership follows the reference: FloatArray arguments are owned (lean_obj_arg) and released here;
 * USize/Float/UInt8/UInt32/UInt64 arrive unboxed; IO entries take the world token last and return
 * an IO result. lean_cuda_mg_prep and lean_cuda_mg_vtrace keep the reference's prototypes without the
 * world token (puffercuda.cu:316, 389).
 *
 * Errors. IO entries return the library's message as an IO user error. Pure entries have no error
 * channel: where the reference fell back to a CPU loop or zero-filled its result, a failure here
 * stops the program with the library's message, so a broken device path is never mistaken for a
 * result. Entry points of parts this library does not provide (the env-plugin rollout drivers, the
 * CNN forward, the sin/cos port) answer as the reference does without a device where it has such an
 * answer (a no-op, "not ready"), and otherwise fail the same way.
 *
 * Build: compiled with the Lean toolchain's C compiler like pufferblas.c, -I<pufferhip>/include,
 * linked with -lpufferhip -lamdhip64. */
#include <lean/lean.h>
#include <stdlib.h>
#include <string.h>

#include "pufferhip.h"

static inline double* fa(b_lean_obj_arg a) { return lean_float_array_cptr((lean_object*)a); }
static inline size_t fn(b_lean_obj_arg a) { return lean_sarray_size(a); }
static inline lean_object* fnew(size_t n) { return lean_alloc_sarray(sizeof(double), n, n); }
/* pointer to a possibly empty array's data, NULL when empty (the host entries read sizes, not data) */
static inline const double* fa0(b_lean_obj_arg a) { return fn(a) ? fa(a) : NULL; }

static void need(int s) {
  if (s != PH_OK) lean_internal_panic(ph_last_error());
}
static lean_obj_res io_fail(void) {
  return lean_io_result_mk_error(lean_mk_io_user_error(lean_mk_string(ph_last_error())));
}
static lean_obj_res io_unit(int s) { return s == PH_OK ? lean_io_result_mk_ok(lean_box(0)) : io_fail(); }
static lean_obj_res io_array(int s, lean_object* a) {
  if (s != PH_OK) {
    lean_dec(a);
    return io_fail();
  }
  return lean_io_result_mk_ok(a);
}
static lean_obj_res not_provided_io(const char* name) {
  char msg[256];
  strcpy(msg, name);
  strcat(msg, ": not provided by pufferhip (this library runs the training-step hot path only)");
  return lean_io_result_mk_error(lean_mk_io_user_error(lean_mk_string(msg)));
}
static size_t mlp_params(size_t H, size_t D, size_t O) { return H * D + H + O * H + O; }
static size_t mg_params(size_t H, size_t D, size_t L, size_t A) {
  return H * D + H + L * 3 * H * H + A * H + A + H + 1;
}
static size_t head_sum(b_lean_obj_arg hs, size_t K) {
  size_t s = 0;
  for (size_t i = 0; i < K && i < fn(hs); i++) s += (size_t)fa(hs)[i];
  return s;
}

/* ---- V-trace / advantage normalisation ----------------------------------------------------------- */
LEAN_EXPORT lean_obj_res lean_cuda_vtrace(lean_obj_arg rew, lean_obj_arg val, lean_obj_arg term, lean_obj_arg imp,
                                          size_t B, size_t T, double gamma, double lam, double rhoClip,
                                          double cClip) {
  lean_object* adv = fnew(B * T);
  need(ph_cuda_vtrace(fa(rew), fa(val), fa(term), fa(imp), B, T, gamma, lam, rhoClip, cClip, fa(adv)));
  lean_dec(rew); lean_dec(val); lean_dec(term); lean_dec(imp);
  return adv;
}

LEAN_EXPORT lean_obj_res lean_cuda_vtrace_mingru(lean_obj_arg rew, lean_obj_arg val, lean_obj_arg term,
                                                 lean_obj_arg imp, lean_obj_arg bv, size_t B, size_t T, double gamma,
                                                 double lam, double rhoClip, double cClip) {
  lean_object* adv = fnew(B * T);
  need(ph_cuda_vtrace_mingru(fa(rew), fa(val), fa(term), fa(imp), fa(bv), B, T, gamma, lam, rhoClip, cClip,
                             fa(adv)));
  lean_dec(rew); lean_dec(val); lean_dec(term); lean_dec(imp); lean_dec(bv);
  return adv;
}

LEAN_EXPORT lean_obj_res lean_cuda_adv_normalize(lean_obj_arg adv, size_t n) {
  lean_object* out = fnew(n);
  need(ph_cuda_adv_normalize(fa(adv), n, fa(out)));
  lean_dec(adv);
  return out;
}

/* ---- MLP gradient, steps and updates ------------------------------------------------------------- */
LEAN_EXPORT lean_obj_res lean_cuda_mlp_ppo_grad(lean_obj_arg p, lean_obj_arg obs, lean_obj_arg acts,
                                                lean_obj_arg advs, lean_obj_arg rets, lean_obj_arg oldlps, size_t N,
                                                size_t H, size_t D, size_t A, double vf, double ent, double clip,
                                                uint8_t bf16) {
  lean_object* g = fnew(mlp_params(H, D, A + 1));
  need(ph_cuda_mlp_ppo_grad(fa(p), fa(obs), fa(acts), fa(advs), fa(rets), fa(oldlps), N, H, D, A, vf, ent, clip,
                            bf16, fa(g)));
  lean_dec(p); lean_dec(obs); lean_dec(acts); lean_dec(advs); lean_dec(rets); lean_dec(oldlps);
  return g;
}

LEAN_EXPORT lean_obj_res lean_cuda_mlp_ppo_grad_md(lean_obj_arg p, lean_obj_arg obs, lean_obj_arg acts,
                                                   lean_obj_arg advs, lean_obj_arg rets, lean_obj_arg oldlps,
                                                   lean_obj_arg hs, size_t N, size_t H, size_t D, size_t K, double vf,
                                                   double ent, double clip, uint8_t bf16) {
  lean_object* g = fnew(mlp_params(H, D, head_sum(hs, K) + 1));
  need(ph_cuda_mlp_ppo_grad_md(fa(p), fa(obs), fa(acts), fa(advs), fa(rets), fa(oldlps), fa(hs), N, H, D, K, vf,
                               ent, clip, bf16, fa(g)));
  lean_dec(p); lean_dec(obs); lean_dec(acts); lean_dec(advs); lean_dec(rets); lean_dec(oldlps); lean_dec(hs);
  return g;
}

LEAN_EXPORT lean_obj_res lean_cuda_mlp_ppo_grad_cont(lean_obj_arg p, lean_obj_arg obs, lean_obj_arg acts,
                                                     lean_obj_arg advs, lean_obj_arg rets, lean_obj_arg oldlps,
                                                     size_t N, size_t H, size_t D, size_t d, double vf, double ent,
                                                     double clip, uint8_t bf16) {
  lean_object* g = fnew(mlp_params(H, D, 2 * d + 1));
  need(ph_cuda_mlp_ppo_grad_cont(fa(p), fa(obs), fa(acts), fa(advs), fa(rets), fa(oldlps), N, H, D, d, vf, ent,
                                 clip, bf16, fa(g)));
  lean_dec(p); lean_dec(obs); lean_dec(acts); lean_dec(advs); lean_dec(rets); lean_dec(oldlps);
  return g;
}

LEAN_EXPORT lean_obj_res lean_cuda_train_step(lean_obj_arg pm, lean_obj_arg obs, lean_obj_arg acts, lean_obj_arg adv,
                                              lean_obj_arg rets, lean_obj_arg olps, size_t N, size_t H, size_t D,
                                              size_t A, double lr, double wd, double mu, double eps, double vf,
                                              double ent, double clip, uint8_t bf16) {
  lean_object* out = fnew(2 * mlp_params(H, D, A + 1));
  need(ph_cuda_train_step(fa(pm), fa(obs), fa(acts), fa(adv), fa(rets), fa(olps), N, H, D, A, lr, wd, mu, eps, vf,
                          ent, clip, bf16, fa(out)));
  lean_dec(pm); lean_dec(obs); lean_dec(acts); lean_dec(adv); lean_dec(rets); lean_dec(olps);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_train_update(lean_obj_arg pm, lean_obj_arg obs, lean_obj_arg acts,
                                                lean_obj_arg adv, lean_obj_arg ret, lean_obj_arg olp, lean_obj_arg perm,
                                                size_t NT, size_t D, size_t H, size_t A, size_t epochs, size_t numMB,
                                                double lr, double wd, double mu, double eps, double vf, double ent,
                                                double clip, uint8_t bf16) {
  lean_object* out = fnew(2 * mlp_params(H, D, A + 1));
  need(ph_cuda_train_update(fa(pm), fa(obs), fa(acts), fa(adv), fa(ret), fa(olp), fa(perm), NT, D, H, A, epochs,
                            numMB, lr, wd, mu, eps, vf, ent, clip, bf16, fa(out)));
  lean_dec(pm); lean_dec(obs); lean_dec(acts); lean_dec(adv); lean_dec(ret); lean_dec(olp); lean_dec(perm);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_train_update_resident(size_t h, lean_obj_arg obs, lean_obj_arg acts,
                                                         lean_obj_arg adv, lean_obj_arg ret, lean_obj_arg olp,
                                                         lean_obj_arg ov, lean_obj_arg perm, size_t NT, size_t D,
                                                         size_t H, size_t A, size_t epochs, size_t numMB, double lr,
                                                         double wd, double mu, double eps, double vf, double ent,
                                                         double clip, double vfClip, double maxGradNorm, uint8_t bf16,
                                                         lean_obj_arg w) {
  (void)w;
  lean_object* out = fnew(1);
  int s = ph_cuda_train_update_resident(h, fa(obs), fa(acts), fa(adv), fa(ret), fa(olp), fa0(ov), fn(ov), fa(perm),
                                        NT, D, H, A, epochs, numMB, lr, wd, mu, eps, vf, ent, clip, vfClip,
                                        maxGradNorm, bf16, fa(out));
  lean_dec(obs); lean_dec(acts); lean_dec(adv); lean_dec(ret); lean_dec(olp); lean_dec(ov); lean_dec(perm);
  return io_array(s, out);
}

LEAN_EXPORT lean_obj_res lean_cuda_train_update_wide_resident(
    size_t h, lean_obj_arg obs, lean_obj_arg acts, lean_obj_arg adv, lean_obj_arg ret, lean_obj_arg olp,
    lean_obj_arg ov, lean_obj_arg perm, lean_obj_arg hs, size_t NT, size_t D, size_t H, size_t O, size_t Wdim,
    uint32_t mode, size_t epochs, size_t numMB, double lr, double wd, double mu, double eps, double vf, double ent,
    double clip, double vfClip, double maxGradNorm, uint8_t bf16, lean_obj_arg w) {
  (void)w;
  lean_object* out = fnew(1);
  int s = ph_cuda_train_update_wide_resident(h, fa(obs), fa(acts), fa(adv), fa(ret), fa(olp), fa0(ov), fn(ov),
                                             fa(perm), fa0(hs), fn(hs), NT, D, H, O, Wdim, mode, epochs, numMB, lr,
                                             wd, mu, eps, vf, ent, clip, vfClip, maxGradNorm, bf16, fa(out));
  lean_dec(obs); lean_dec(acts); lean_dec(adv); lean_dec(ret); lean_dec(olp); lean_dec(ov); lean_dec(perm);
  lean_dec(hs);
  return io_array(s, out);
}

/* ---- Muon ---------------------------------------------------------------------------------------- */
LEAN_EXPORT lean_obj_res lean_cuda_muon_stepmat(lean_obj_arg W, lean_obj_arg G, lean_obj_arg M, size_t rows,
                                                size_t cols, double lr, double wd, double mu, double eps) {
  lean_object* out = fnew(2 * rows * cols);
  need(ph_cuda_muon_stepmat(fa(W), fa(G), fa(M), rows, cols, lr, wd, mu, eps, fa(out)));
  lean_dec(W); lean_dec(G); lean_dec(M);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_muon_step_mlp_resident(size_t h, lean_obj_arg gRaw, size_t H, size_t D, size_t O,
                                                          double gscale, double lr, double wd, double mu, double eps,
                                                          lean_obj_arg w) {
  (void)w;
  lean_object* out = fnew(mlp_params(H, D, O));
  int s = ph_cuda_muon_step_mlp_resident(h, fa(gRaw), H, D, O, gscale, lr, wd, mu, eps, fa(out));
  lean_dec(gRaw);
  return io_array(s, out);
}

/* Empty gClip: the resident gradient of the last device-column gradient call is clipped and consumed
 * on the device, and the result is empty (the weights stay in the handle for the next gradient). */
LEAN_EXPORT lean_obj_res lean_cuda_mingru_muon_resident(size_t h, lean_obj_arg gClip, size_t H, size_t D, size_t L,
                                                        size_t A, double lr, double wd, double mu, double eps,
                                                        double maxGradNorm, double gscale, lean_obj_arg w) {
  (void)w;
  size_t P = mg_params(H, D, L, A), len = 0;
  lean_object* out = fnew(P);
  int s = ph_cuda_mingru_muon_resident(h, fa0(gClip), fn(gClip), H, D, L, A, lr, wd, mu, eps, maxGradNorm, gscale,
                                       fa(out), &len);
  lean_dec(gClip);
  if (s == PH_OK && len == 0) {
    lean_dec(out);
    out = fnew(0);
  }
  return io_array(s, out);
}

/* ---- resident policy handle and the loss channel ------------------------------------------------- */
LEAN_EXPORT lean_obj_res lean_cuda_policy_load(lean_obj_arg pm, size_t P, lean_obj_arg w) {
  (void)w;
  size_t h = 0;
  int s = ph_cuda_policy_load(fa(pm), P, &h);
  lean_dec(pm);
  return s == PH_OK ? lean_io_result_mk_ok(lean_box_usize(h)) : io_fail();
}

LEAN_EXPORT lean_obj_res lean_cuda_policy_download(size_t h, size_t P, lean_obj_arg w) {
  (void)w;
  lean_object* out = fnew(2 * P);
  return io_array(ph_cuda_policy_download(h, P, fa(out)), out);
}

LEAN_EXPORT lean_obj_res lean_cuda_policy_free(size_t h, lean_obj_arg w) {
  (void)w;
  return io_unit(ph_cuda_policy_free(h));
}

LEAN_EXPORT lean_obj_res lean_cuda_mg_loss_enable(uint8_t on, lean_obj_arg w) {
  (void)w;
  return io_unit(ph_cuda_mg_loss_enable(on));
}

LEAN_EXPORT lean_obj_res lean_cuda_mg_read_losses(lean_obj_arg w) {
  (void)w;
  lean_object* out = fnew(7);
  return io_array(ph_cuda_mg_read_losses(fa(out)), out);
}

/* ---- MinGRU minibatch chain ------------------------------------------------------------------------ */
LEAN_EXPORT lean_obj_res lean_cuda_mg_prep(lean_obj_arg rew, lean_obj_arg term, lean_obj_arg act, lean_obj_arg logp,
                                           lean_obj_arg val, lean_obj_arg boot, size_t N, size_t T, size_t K) {
  int s = ph_cuda_mg_prep(fa(rew), fa(term), fa(act), fa(logp), fa(val), fa(boot), N, T, K);
  lean_dec(rew); lean_dec(term); lean_dec(act); lean_dec(logp); lean_dec(val); lean_dec(boot);
  return io_unit(s);
}

LEAN_EXPORT lean_obj_res lean_cuda_mg_cols_ready(size_t N, size_t T, lean_obj_arg w) {
  (void)w;
  uint8_t r = 0;
  int s = ph_cuda_mg_cols_ready(N, T, &r);
  return s == PH_OK ? lean_io_result_mk_ok(lean_box(r)) : io_fail();
}

LEAN_EXPORT lean_obj_res lean_cuda_mg_vtrace(size_t N, size_t T, double gamma, double lam, double rhoClip,
                                             double cClip) {
  lean_object* out = fnew(N);
  return io_array(ph_cuda_mg_vtrace(N, T, gamma, lam, rhoClip, cClip, fa(out)), out);
}

LEAN_EXPORT lean_obj_res lean_cuda_mg_vtrace_prio(size_t N, size_t T, double gamma, double lam, double rhoClip,
                                                  double cClip, size_t mbSegs, double prioAlpha, double annealBeta,
                                                  uint64_t rng, lean_obj_arg w) {
  (void)w;
  uint8_t used = 0;
  int s = ph_cuda_mg_vtrace_prio(N, T, gamma, lam, rhoClip, cClip, mbSegs, prioAlpha, annealBeta, rng, &used);
  return s == PH_OK ? lean_io_result_mk_ok(lean_box(used)) : io_fail();
}

/* The result length is the gradient mode (Puffer/Float/CUDA.lean:138-148): empty when the gradient was
 * left on the device (device-column mode), P + 2*T*B in the host form. An empty `p` takes the weights
 * the last resident Muon step left in its handle. */
LEAN_EXPORT lean_obj_res lean_cuda_mingru_ppo_grad(lean_obj_arg p, lean_obj_arg obs, lean_obj_arg scal, size_t B,
                                                   size_t T, size_t H, size_t D, size_t L, size_t A, size_t K,
                                                   lean_obj_arg hs, double vf, double ent, double clip, double vfClip,
                                                   lean_obj_arg segIdx, lean_obj_arg mbPrio, lean_obj_arg w) {
  (void)w;
  size_t P = mg_params(H, D, L, A), len = 0;
  lean_object* out = fnew(P + 2 * T * B);
  int s = ph_cuda_mingru_ppo_grad(fa0(p), fn(p), fa0(obs), fn(obs), fa0(scal), fn(scal), B, T, H, D, L, A, K,
                                  fa0(hs), fn(hs), vf, ent, clip, vfClip, fa0(segIdx), fn(segIdx), fa0(mbPrio),
                                  fn(mbPrio), fa(out), &len);
  lean_dec(p); lean_dec(obs); lean_dec(scal); lean_dec(hs); lean_dec(segIdx); lean_dec(mbPrio);
  if (s == PH_OK && len == 0) {
    lean_dec(out);
    out = fnew(0);
  }
  return io_array(s, out);
}

/* ---- rollout forward and samplers ------------------------------------------------------------------ */
LEAN_EXPORT lean_obj_res lean_cuda_sample_actions(lean_obj_arg Y, size_t N, size_t A, size_t O, uint64_t rng) {
  lean_object* out = fnew(3 * N);
  need(ph_cuda_sample_actions(fa(Y), N, A, O, rng, fa(out)));
  lean_dec(Y);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_sample_actions_md(lean_obj_arg Y, lean_obj_arg hs, size_t N, size_t K, size_t O,
                                                     uint64_t rng) {
  lean_object* out = fnew((K + 2) * N);
  need(ph_cuda_sample_actions_md(fa(Y), fa(hs), N, K, O, rng, fa(out)));
  lean_dec(Y); lean_dec(hs);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_sample_actions_cont(lean_obj_arg Y, size_t N, size_t d, size_t O, uint64_t rng) {
  lean_object* out = fnew((d + 2) * N);
  need(ph_cuda_sample_actions_cont(fa(Y), N, d, O, rng, fa(out)));
  lean_dec(Y);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_mingru_step(lean_obj_arg p, lean_obj_arg obs, lean_obj_arg state, size_t N,
                                               size_t D, size_t H, size_t L, size_t A, uint8_t bf16) {
  lean_object* out = fnew(N * (A + 1) + N * L * H);
  need(ph_cuda_mingru_step(fa(p), fa(obs), fa(state), N, D, H, L, A, bf16, fa(out)));
  lean_dec(p); lean_dec(obs); lean_dec(state);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_mlp_forward(lean_obj_arg p, lean_obj_arg obs, size_t N, size_t D, size_t H,
                                               size_t O, uint8_t bf16) {
  lean_object* out = fnew(N * O);
  need(ph_cuda_mlp_forward(fa(p), fa(obs), N, D, H, O, bf16, fa(out)));
  lean_dec(p); lean_dec(obs);
  return out;
}

LEAN_EXPORT lean_obj_res lean_cuda_selftest(size_t n) {
  lean_object* out = fnew(n);
  need(ph_cuda_selftest(n, fa(out)));
  return out;
}

/* ---- GPU entries of pufferblas.c ---------------------------------------------------------------- */
LEAN_EXPORT lean_obj_res lean_ffi_dense_forward_cublas(lean_obj_arg X, lean_obj_arg W, lean_obj_arg b, size_t N,
                                                       size_t D, size_t H) {
  lean_object* Y = fnew(N * H);
  need(ph_ffi_dense_forward_gpu(fa(X), fa(W), fa(b), N, D, H, fa(Y)));
  lean_dec(X); lean_dec(W); lean_dec(b);
  return Y;
}

LEAN_EXPORT lean_obj_res lean_ffi_dense_forward_cublaslt_bf16(lean_obj_arg X, lean_obj_arg W, lean_obj_arg b,
                                                              size_t N, size_t D, size_t H) {
  lean_object* Y = fnew(N * H);
  need(ph_ffi_dense_forward_bf16(fa(X), fa(W), fa(b), N, D, H, fa(Y)));
  lean_dec(X); lean_dec(W); lean_dec(b);
  return Y;
}

LEAN_EXPORT double lean_ffi_bench_cublaslt_bf16_resident(size_t N, size_t D, size_t H, size_t reps) {
  return ph_ffi_bench_bf16_resident(N, D, H, reps);
}

LEAN_EXPORT lean_obj_res lean_ffi_mlp_forward_batch_cublaslt_bf16(lean_obj_arg p, lean_obj_arg X, size_t N,
                                                                  size_t D, size_t H, size_t O) {
  lean_object* Y = fnew(N * O);
  need(ph_ffi_mlp_forward_batch_bf16(fa(p), fa(X), N, D, H, O, fa(Y)));
  lean_dec(p); lean_dec(X);
  return Y;
}

LEAN_EXPORT double lean_ffi_bench_mlp2_bf16_resident(size_t N, size_t D, size_t H, size_t O, size_t reps) {
  return ph_ffi_bench_mlp2_bf16_resident(N, D, H, O, reps);
}

LEAN_EXPORT double lean_ffi_bench_mlp2_bf16_wres(size_t N, size_t D, size_t H, size_t O, size_t reps) {
  return ph_ffi_bench_mlp2_bf16_wres(N, D, H, O, reps);
}

/* 0 without a usable device, as the reference's handle-less answer */
LEAN_EXPORT size_t lean_ffi_mlp_policy_load(lean_obj_arg p, size_t D, size_t H, size_t O) {
  size_t h = 0;
  if (ph_ffi_mlp_policy_load(fa(p), D, H, O, &h) != PH_OK) h = 0;
  lean_dec(p);
  return h;
}

LEAN_EXPORT uint8_t lean_ffi_mlp_policy_update(size_t h, lean_obj_arg p) {
  uint8_t ok = h != 0 && ph_ffi_mlp_policy_update(h, fa(p)) == PH_OK;
  lean_dec(p);
  return ok;
}

LEAN_EXPORT lean_obj_res lean_ffi_mlp_policy_forward(size_t h, lean_obj_arg X, size_t N) {
  /* the output width is the handle's O: N*O values */
  size_t O = ph_ffi_mlp_policy_outputs(h);
  lean_object* Y = fnew(N * O);
  need(ph_ffi_mlp_policy_forward(h, fa(X), N, fa(Y)));
  lean_dec(X);
  return Y;
}

LEAN_EXPORT uint8_t lean_ffi_mlp_policy_free(size_t h) { return h != 0 && ph_ffi_mlp_policy_free(h) == PH_OK; }

LEAN_EXPORT uint8_t lean_ffi_cuda_available(lean_obj_arg unit) {
  lean_dec(unit);
  return ph_ffi_cuda_available();
}

/* ---- parts of the reference this library does not provide ---------------------------------------- */
/* a hint for the LSTM trainer's input reuse: nothing to do without the LSTM path */
LEAN_EXPORT lean_obj_res lean_cuda_lstm_reuse_inputs(uint8_t on, lean_obj_arg w) {
  (void)on; (void)w;
  return lean_io_result_mk_ok(lean_box(0));
}

/* no rollout leaves a fused chain behind: never ready (the trainer then passes its host columns) */
LEAN_EXPORT lean_obj_res lean_cuda_mg_chain_ready(size_t N, size_t D, size_t LH, lean_obj_arg w) {
  (void)N; (void)D; (void)LH; (void)w;
  return lean_io_result_mk_ok(lean_box(0));
}

/* the rollout double-buffer count: a setting of the rollout drivers, which are not here */
LEAN_EXPORT lean_obj_res lean_cuda_set_roll_buffers(size_t nbuf, uint8_t graphOn, lean_obj_arg w) {
  (void)nbuf; (void)graphOn; (void)w;
  return lean_io_result_mk_ok(lean_box(0));
}

LEAN_EXPORT lean_obj_res lean_cuda_plugin_rollout(size_t hh, size_t policyH, lean_obj_arg obs0, size_t N, size_t D,
                                                  size_t H, size_t A, size_t T, uint8_t bf16, uint64_t rolloutRng,
                                                  lean_obj_arg w) {
  (void)hh; (void)policyH; (void)N; (void)D; (void)H; (void)A; (void)T; (void)bf16; (void)rolloutRng; (void)w;
  lean_dec(obs0);
  return not_provided_io("lean_cuda_plugin_rollout");
}

LEAN_EXPORT lean_obj_res lean_cuda_plugin_rollout_lstm(size_t hh, lean_obj_arg params, lean_obj_arg obs0,
                                                       lean_obj_arg h0, lean_obj_arg c0, size_t N, size_t D, size_t H,
                                                       size_t A, size_t T, uint64_t rolloutRng, lean_obj_arg w) {
  (void)hh; (void)N; (void)D; (void)H; (void)A; (void)T; (void)rolloutRng; (void)w;
  lean_dec(params); lean_dec(obs0); lean_dec(h0); lean_dec(c0);
  return not_provided_io("lean_cuda_plugin_rollout_lstm");
}

LEAN_EXPORT lean_obj_res lean_cuda_plugin_rollout_multi(size_t hh, size_t policyH, lean_obj_arg obs0, lean_obj_arg hs,
                                                        size_t N, size_t D, size_t H, size_t O, size_t Wdim, size_t T,
                                                        uint32_t mode, uint8_t bf16, uint64_t rolloutRng,
                                                        lean_obj_arg w) {
  (void)hh; (void)policyH; (void)N; (void)D; (void)H; (void)O; (void)Wdim; (void)T; (void)mode; (void)bf16;
  (void)rolloutRng; (void)w;
  lean_dec(obs0); lean_dec(hs);
  return not_provided_io("lean_cuda_plugin_rollout_multi");
}

LEAN_EXPORT lean_obj_res lean_cuda_plugin_rollout_mingru(size_t hh, size_t policyH, lean_obj_arg obs0,
                                                         lean_obj_arg state0, size_t N, size_t D, size_t H, size_t L,
                                                         size_t A, size_t T, uint8_t wantLog, uint64_t rolloutRng,
                                                         lean_obj_arg w) {
  (void)hh; (void)policyH; (void)N; (void)D; (void)H; (void)L; (void)A; (void)T; (void)wantLog; (void)rolloutRng;
  (void)w;
  lean_dec(obs0); lean_dec(state0);
  return not_provided_io("lean_cuda_plugin_rollout_mingru");
}

LEAN_EXPORT lean_obj_res lean_cuda_plugin_rollout_mingru_md(size_t hh, size_t policyH, lean_obj_arg obs0,
                                                            lean_obj_arg state0, lean_obj_arg hs, size_t N, size_t D,
                                                            size_t H, size_t L, size_t W, size_t K, size_t T,
                                                            uint64_t rolloutRng, lean_obj_arg w) {
  (void)hh; (void)policyH; (void)N; (void)D; (void)H; (void)L; (void)W; (void)K; (void)T; (void)rolloutRng; (void)w;
  lean_dec(obs0); lean_dec(state0); lean_dec(hs);
  return not_provided_io("lean_cuda_plugin_rollout_mingru_md");
}

LEAN_EXPORT lean_obj_res lean_cuda_cnn_forward(lean_obj_arg p, lean_obj_arg obs, size_t N, size_t C, size_t inH,
                                               size_t inW, size_t nF, size_t k, size_t s, size_t hidden, size_t O,
                                               uint8_t bf16) {
  (void)p; (void)obs; (void)N; (void)C; (void)inH; (void)inW; (void)nF; (void)k; (void)s; (void)hidden; (void)O;
  (void)bf16;
  lean_internal_panic("lean_cuda_cnn_forward: not provided by pufferhip (the CNN trainer is not on its path)");
  return fnew(0);
}

LEAN_EXPORT lean_obj_res lean_cuda_sincosf(lean_obj_arg angles, size_t N, uint8_t isCos) {
  (void)angles; (void)N; (void)isCos;
  lean_internal_panic("lean_cuda_sincosf: not provided by pufferhip (an env-physics helper, not on its path)");
  return fnew(0);
}
