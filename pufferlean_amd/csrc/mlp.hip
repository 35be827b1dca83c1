// The MLP policy's PPO update on the device, for L >= 1 hidden ReLU layers of width H and the
// combined head (A logits and the value in one (A+1) x H matrix).
//
// The reference's MLP policy has one hidden layer (flattenMLP [W1|b1|W2|b2], pufferblas.c:699-747,
// puffercuda.cu:748-820); with L = 1 the parameter layout and every product here are that policy's,
// and deeper policies repeat the hidden layer: [W1 | b1 | W2 | b2 | ... | WL | bL | Wo | bo].
//
// One update (ph_mlp_update) over N = T x B time-major rows (row t*B + b):
//   forward (kept for the backward) -> per-row log-prob of the taken action and value ->
//   V-trace (vec form) with ratio exp(logp - behaviour logp) -> advantage normalisation ->
//   fused PPO loss gradient -> backward -> grad clip / mean -> Muon on every matrix, stepvec on
//   every bias.
// The forward is run once: its activations serve both the log-probs V-trace needs and the backward.
// Activations and gradients are fp32 in HBM; `math` picks fp32 MFMA or bf16 MFMA on the fp32
// operands (the reference's FAST_16BF).
#include "common.hpp"
#include "kernels.hpp"

namespace ph {
namespace {

constexpr int kB = 256;

struct MlpGeo {
  long N;
  int D, H, L, A, O;
  long P;
  long oW[kMlpMaxLayers + 1], ob[kMlpMaxLayers + 1];  // layer l's weight / bias; [L] = the head
};

MlpGeo mlp_geo(const ph_mlp_dims& d) {
  MlpGeo g{};
  g.N = d.N; g.D = d.D; g.H = d.H; g.L = d.L; g.A = d.A; g.O = d.A + 1;
  long off = 0;
  for (int l = 0; l < d.L; l++) {
    const long in = l == 0 ? d.D : d.H;
    g.oW[l] = off; off += (long)d.H * in;
    g.ob[l] = off; off += d.H;
  }
  g.oW[d.L] = off; off += (long)g.O * d.H;
  g.ob[d.L] = off; off += g.O;
  g.P = off;
  return g;
}

struct MlpBufs {
  float* Hs;    // [L][N][H] hidden activations
  float* Out;   // [N][O]
  float* dOut;  // [N][O]
  float *dA, *dB;  // [N][H] gradients at a layer's output
  float *logrho, *val, *adv, *advn, *tgt, *stats;
};

int mlp_bufs(const MlpGeo& g, MlpBufs& b) {
  const long N = g.N;
  size_t off = 0;
  auto take = [&](size_t n) { size_t o = off; off += (n * 4 + 255) & ~(size_t)255; return o; };
  const size_t oHs = take((size_t)g.L * N * g.H), oOut = take((size_t)N * g.O), odOut = take((size_t)N * g.O),
               odA = take((size_t)N * g.H), odB = take((size_t)N * g.H), olr = take(N), oval = take(N),
               oadv = take(N), oadvn = take(N), otgt = take(N), ost = take(16);
  uint8_t* base = (uint8_t*)scratch(kSlotMlpBufs, off);
  if (!base) return PH_ERR_NOMEM;
  b.Hs = (float*)(base + oHs); b.Out = (float*)(base + oOut); b.dOut = (float*)(base + odOut);
  b.dA = (float*)(base + odA); b.dB = (float*)(base + odB); b.logrho = (float*)(base + olr);
  b.val = (float*)(base + oval); b.adv = (float*)(base + oadv); b.advn = (float*)(base + oadvn);
  b.tgt = (float*)(base + otgt); b.stats = (float*)(base + ost);
  return PH_OK;
}

PhGemmDesc f32g(int ta, int tb, long M, long N, long K, const float* A, long lda, const float* B, long ldb,
                float* C, long ldc, int math) {
  PhGemmDesc d{};
  d.trans_a = ta; d.trans_b = tb; d.M = (int)M; d.N = (int)N; d.K = (int)K;
  d.a_dtype = PH_F32; d.A = A; d.lda = lda; d.b_dtype = PH_F32; d.B = B; d.ldb = ldb;
  d.c_dtype = PH_F32; d.C = C; d.ldc = ldc; d.math = math; d.alpha = 1.f;
  return d;
}

// H_l = relu(X_l W_l^T + b_l), Out = H_L Wo^T + bo.
int forward(const MlpGeo& g, const float* p, const float* obs, const MlpBufs& b, int math, hipStream_t st) {
  for (int l = 0; l < g.L; l++) {
    const float* X = l == 0 ? obs : b.Hs + (long)(l - 1) * g.N * g.H;
    const long in = l == 0 ? g.D : g.H;
    PhGemmDesc d = f32g(0, 1, g.N, g.H, in, X, in, p + g.oW[l], in, b.Hs + (long)l * g.N * g.H, g.H, math);
    d.epi = PH_EPI_BIAS_RELU; d.bias = p + g.ob[l];
    PH_TRY(gemm(d, st));
  }
  PhGemmDesc d = f32g(0, 1, g.N, g.O, g.H, b.Hs + (long)(g.L - 1) * g.N * g.H, g.H, p + g.oW[g.L], g.H, b.Out,
                      g.O, math);
  d.epi = PH_EPI_BIAS; d.bias = p + g.ob[g.L];
  return gemm(d, st);
}

// Gradient of the loss from dOut back to every parameter (G, flat layout; overwritten). The mask of a
// layer's ReLU is applied where its output gradient is formed, as the reference's k_dz1_mask.
int backward(const MlpGeo& g, const float* p, const float* obs, const MlpBufs& b, float* G, int math,
             hipStream_t st) {
  const float* HL = b.Hs + (long)(g.L - 1) * g.N * g.H;
  PH_TRY(colsum_f32(b.dOut, g.N, g.O, g.O, G + g.ob[g.L], 1.f, 0, st));
  PH_TRY(gemm(f32g(1, 0, g.O, g.H, g.N, b.dOut, g.O, HL, g.H, G + g.oW[g.L], g.H, math), st));
  PhGemmDesc d = f32g(0, 0, g.N, g.H, g.O, b.dOut, g.O, p + g.oW[g.L], g.H, b.dA, g.H, math);
  d.epi = PH_EPI_RELU_MASK; d.aux = HL; d.ldaux = g.H;
  PH_TRY(gemm(d, st));
  float* dA = b.dA;
  float* dB = b.dB;
  for (int l = g.L - 1; l >= 0; l--) {
    const float* X = l == 0 ? obs : b.Hs + (long)(l - 1) * g.N * g.H;
    const long in = l == 0 ? g.D : g.H;
    PH_TRY(colsum_f32(dA, g.N, g.H, g.H, G + g.ob[l], 1.f, 0, st));
    PH_TRY(gemm(f32g(1, 0, g.H, in, g.N, dA, g.H, X, in, G + g.oW[l], in, math), st));
    if (l > 0) {
      PhGemmDesc e = f32g(0, 0, g.N, g.H, g.H, dA, g.H, p + g.oW[l], g.H, dB, g.H, math);
      e.epi = PH_EPI_RELU_MASK; e.aux = X; e.ldaux = g.H;
      PH_TRY(gemm(e, st));
      float* t = dA; dA = dB; dB = t;
    }
  }
  return PH_OK;
}

// Per row: log-prob of the taken action (log-sum-exp without the max shift, as the MLP loss kernel
// k_ppo_dout computes it, puffercuda.cu:736-738), the log importance ratio against the behaviour
// log-prob, and the value (column A).
__global__ void k_logp_value(const float* __restrict__ out, int O, int A, const int* __restrict__ act,
                             const float* __restrict__ behav, long N, float* __restrict__ logrho,
                             float* __restrict__ val) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float* r = out + n * O;
  float se = 0.f;
  for (int k = 0; k < A; k++) se += expf(r[k]);
  const int a = act[n];
  const float lp = (a >= 0 && a < A) ? r[a] - logf(se) : __builtin_nanf("");
  logrho[n] = lp - behav[n];
  val[n] = r[A];
}

int check_dims(const ph_mlp_dims& d, const char* who) {
  PH_REQUIRE(d.N > 0 && d.D > 0 && d.H > 0 && d.A > 0, "%s: empty dims", who);
  PH_REQUIRE(d.L >= 1 && d.L <= kMlpMaxLayers, "%s: L=%d hidden layers (1..%d)", who, d.L, kMlpMaxLayers);
  return PH_OK;
}

int muon_all(const MlpGeo& g, const ph_muon_coefs& m, float* params, float* mom, float* G, hipStream_t st) {
  PH_TRY(gclip_f32(G, g.P, m.gscale, m.max_grad_norm, st));
  MuonMat mats[kMlpMaxLayers + 1];
  StepVec vecs[kMlpMaxLayers + 1];
  for (int l = 0; l <= g.L; l++) {
    const int rows = l == g.L ? g.O : g.H, cols = l == 0 ? g.D : g.H;
    mats[l] = MuonMat{params + g.oW[l], G + g.oW[l], mom + g.oW[l], rows, cols};
    const long nb = l == g.L ? g.O : g.H;
    vecs[l] = StepVec{params + g.ob[l], G + g.ob[l], mom + g.ob[l], nb};
  }
  PH_TRY(stepvec_f32_batch(vecs, g.L + 1, 1.f, m.lr, m.wd, m.mu, st));
  return muon_fast_batch(mats, g.L + 1, 1.f, m.lr, m.wd, m.mu, m.eps, m.coeffs, m.nsteps, m.math, st);
}

}  // namespace

long mlp_param_count(const ph_mlp_dims& d) { return mlp_geo(d).P; }

}  // namespace ph

using namespace ph;

extern "C" long ph_mlp_param_count(const ph_mlp_dims* d) {
  if (!d || d->L < 1 || d->L > kMlpMaxLayers) return -1;
  return mlp_param_count(*d);
}

extern "C" int ph_mlp_forward(const ph_mlp_dims* d, int math, const float* params, const float* obs, float* out,
                              void* stream) {
  PH_REQUIRE(d, "ph_mlp_forward: null dims");
  PH_TRY(check_dims(*d, "ph_mlp_forward"));
  PH_REQUIRE(params && obs && out, "ph_mlp_forward: null pointer");
  PH_REQUIRE(math == PH_MATH_F32 || math == PH_MATH_BF16, "ph_mlp_forward: math must be F32 or BF16");
  const hipStream_t st = as_stream(stream);
  const MlpGeo g = mlp_geo(*d);
  MlpBufs b;
  PH_TRY(mlp_bufs(g, b));
  PH_TRY(forward(g, params, obs, b, math, st));
  PH_CHECK_HIP(hipMemcpyAsync(out, b.Out, (size_t)g.N * g.O * 4, hipMemcpyDeviceToDevice, st));
  return PH_OK;
}

extern "C" int ph_mlp_ppo_grad(const ph_mlp_dims* d, const ph_ppo_coefs* c, int math, const float* params,
                               const float* obs, const int* act, const float* adv, const float* ret,
                               const float* old, const float* ov, float* G, float* newlp, float* newval,
                               double* losses, void* stream) {
  PH_REQUIRE(d && c, "ph_mlp_ppo_grad: null config");
  PH_TRY(check_dims(*d, "ph_mlp_ppo_grad"));
  PH_REQUIRE(params && obs && act && adv && ret && old && G, "ph_mlp_ppo_grad: null pointer");
  PH_REQUIRE(math == PH_MATH_F32 || math == PH_MATH_BF16, "ph_mlp_ppo_grad: math must be F32 or BF16");
  const hipStream_t st = as_stream(stream);
  const MlpGeo g = mlp_geo(*d);
  MlpBufs b;
  PH_TRY(mlp_bufs(g, b));
  PH_TRY(forward(g, params, obs, b, math, st));
  PH_TRY(ppo_grad(b.Out, g.O, b.Out + g.A, g.O, act, adv, ret, old, ov, g.N, g.A, c->vf_coef, c->ent_coef,
                  c->clip_eps, c->vf_clip, 0, b.dOut, g.O, b.dOut + g.A, g.O, newlp, newval, losses, st));
  return backward(g, params, obs, b, G, math, st);
}

extern "C" int ph_mlp_update(const ph_mlp_dims* d, int T, const ph_ppo_coefs* c, const ph_muon_coefs* m,
                             int math, float* params, float* mom, const float* obs, const int* act,
                             const float* behav_logp, const float* rew, const float* done, float* G,
                             double* losses, void* stream) {
  PH_REQUIRE(d && c && m, "ph_mlp_update: null config");
  PH_TRY(check_dims(*d, "ph_mlp_update"));
  PH_REQUIRE(T > 0 && d->N % T == 0, "ph_mlp_update: N=%d rows are not whole segments of T=%d steps", d->N, T);
  PH_REQUIRE(params && mom && obs && act && behav_logp && rew && done && G, "ph_mlp_update: null pointer");
  PH_REQUIRE(math == PH_MATH_F32 || math == PH_MATH_BF16, "ph_mlp_update: math must be F32 or BF16");
  PH_REQUIRE(m->nsteps >= 0 && (m->coeffs || m->nsteps == 0), "ph_mlp_update: coefficient table missing");
  const hipStream_t st = as_stream(stream);
  const MlpGeo g = mlp_geo(*d);
  const long B = g.N / T;
  MlpBufs b;
  PH_TRY(mlp_bufs(g, b));
  PH_TRY(forward(g, params, obs, b, math, st));
  k_logp_value<<<ceil_div(g.N, kB), kB, 0, st>>>(b.Out, g.O, g.A, act, behav_logp, g.N, b.logrho, b.val);
  PH_LAUNCH_CHECK();
  PH_TRY(vtrace_f32(rew, b.val, done, b.logrho, nullptr, (size_t)B, (size_t)T, 0, 1, 1, 1, c->gamma, c->lam,
                    c->rho_clip, c->c_clip, b.adv, b.tgt, st));
  PH_TRY(moments_normalize(PH_F32, b.adv, g.N, b.advn, b.stats, st));
  PH_TRY(ppo_grad(b.Out, g.O, b.Out + g.A, g.O, act, b.advn, b.tgt, behav_logp, nullptr, g.N, g.A, c->vf_coef,
                  c->ent_coef, c->clip_eps, c->vf_clip, 0, b.dOut, g.O, b.dOut + g.A, g.O, nullptr, nullptr,
                  losses, st));
  PH_TRY(backward(g, params, obs, b, G, math, st));
  return muon_all(g, *m, params, mom, G, st);
}
