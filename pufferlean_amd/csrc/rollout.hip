// Rollout policy forward and categorical sampler: what produces the behaviour log-prob and value
// columns the update consumes.
//
//   ph_sample_actions       categorical draw per row of logits      (k_sample / k_sample_f32,
//                                                                     puffercuda.cu:1429-1460; CPU twin
//                                                                     pufferffi.c:896-918)
//   ph_mingru_rollout_step  one timestep of the MinGRU policy       (lean_cuda_mingru_step,
//                           over N envs, state carried in place      puffercuda.cu:2190-2265)
//
// The step runs the policy's products on the MFMA GEMMs (encoder with its bias fused, one 3H x H
// product per layer, one padded head whose first A + 1 rows are the action logits and the value, bias
// fused, written straight into the [N][A+1] output) and one elementwise kernel per layer for the cell.
// Its launches are plain stream work, so a caller can capture a whole horizon in one HIP graph.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

// The sampler's formulas execute in the order written (no fused multiply-add), as in the CPU twin.
#pragma clang fp contract(off)

namespace ph {
namespace {

constexpr int HP = 32;  // padded head rows: A logits, the value, zeros

__device__ __forceinline__ unsigned long long sm64_mix(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float ex(float x) { return expf(x); }
__device__ __forceinline__ double ex(double x) { return exp(x); }
__device__ __forceinline__ float lg(float x) { return logf(x); }
__device__ __forceinline__ double lg(double x) { return log(x); }

// Row n (stride ldy): m = max of the A logits, z = sum exp(l - m); the draw u is the top 53 bits of
// the splitmix64 word of rng + (n+1)*GOLD over 2^53; the action is the first k whose running sum of
// exp(l_k - m)/z exceeds u (A-1 if none); logp = log(exp(l_a - m)/z); the value is column A. R is the
// logit type (the running sum and logp are in R; u is always f64, as in the reference's f32 form).
template <typename R, bool OUT3>
__global__ void __launch_bounds__(256) k_sample_cat(const R* __restrict__ Y, long ldy, long N, int A,
                                                    int has_value, unsigned long long rng, int* __restrict__ act,
                                                    R* __restrict__ logp, R* __restrict__ val,
                                                    double* __restrict__ out3) {
  const long n = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const R* row = Y + n * ldy;
  R m = row[0];
  for (int k = 1; k < A; k++)
    if (row[k] > m) m = row[k];
  R z = 0;
  for (int k = 0; k < A; k++) z += ex(row[k] - m);
  const unsigned long long w = sm64_mix(rng + (unsigned long long)(n + 1) * 0x9E3779B97F4A7C15ULL);
  const double u = (double)(w >> 11) / 9007199254740992.0;
  R acc = 0;
  int a = A - 1;
  for (int k = 0; k < A; k++) {
    acc += ex(row[k] - m) / z;
    if (u < (double)acc) {
      a = k;
      break;
    }
  }
  const R lp = lg(ex(row[a] - m) / z);
  const R v = has_value ? row[A] : R(0);
  if (act) act[n] = a;
  if (logp) logp[n] = lp;
  if (val) val[n] = v;
  if constexpr (OUT3) {
    out3[n] = (double)a;
    out3[N + n] = (double)lp;
    out3[2 * N + n] = (double)v;
  }
}

// The MinGRU cell of layer l for one step (the reference's k_mingru_gate, puffercuda.cu:1949-1959):
// cmb [N][3H] = hid | gate | proj of this layer's product, xin [N][H] the layer input, state [N][L][H].
//   o = (1 - sigmoid(gate)) * prev + sigmoid(gate) * gact(hid),  gact(x) = x >= 0 ? x + 1/2 : sigmoid(x)
//   xout = sigmoid(proj) * o + (1 - sigmoid(proj)) * xin,  state <- o
__device__ __forceinline__ float sig_ieee(float x) { return 1.0f / (1.0f + expf(-x)); }
__global__ void __launch_bounds__(256) k_rollout_cell(const float* __restrict__ cmb, const float* __restrict__ xin,
                                                      float* __restrict__ state, float* __restrict__ xout, long N,
                                                      int L, int H, int l) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * H) return;
  const long n = idx / H;
  const int j = (int)(idx - n * H);
  const float* y = cmb + n * 3 * H;
  const float hid = y[j], gate = y[H + j], proj = y[2 * H + j];
  const float zg = sig_ieee(gate), g = hid >= 0.f ? hid + 0.5f : sig_ieee(hid), hg = sig_ieee(proj);
  float* s = state + (n * L + l) * H + j;
  const float o = (1.0f - zg) * *s + zg * g;
  xout[idx] = hg * o + (1.0f - hg) * xin[idx];
  *s = o;
}

// Padded head [HP][H] (rows: wDec, wVal, zeros) and its bias [HP] from the flat parameters.
__global__ void k_rollout_head(const float* __restrict__ p, int D, int H, int L, int A, float* __restrict__ wh,
                               float* __restrict__ bh) {
  const long offDec = (long)H * D + H + (long)L * 3 * H * H, offBDec = offDec + (long)A * H,
             offVal = offBDec + A, offBVal = offVal + H;
  const long n = (long)HP * H + HP;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    if (i < (long)HP * H) {
      const int row = (int)(i / H), col = (int)(i % H);
      wh[i] = row < A ? p[offDec + (long)row * H + col] : (row == A ? p[offVal + col] : 0.f);
    } else {
      const int k = (int)(i - (long)HP * H);
      bh[k] = k < A ? p[offBDec + k] : (k == A ? p[offBVal] : 0.f);
    }
  }
}

PhGemmDesc nt_f32(int M, int N, int K, const float* A, long lda, const float* B, long ldb, float* C, long ldc,
                  int math) {
  PhGemmDesc d{};
  d.trans_a = 0; d.trans_b = 1; d.M = M; d.N = N; d.K = K;
  d.a_dtype = PH_F32; d.A = A; d.lda = lda; d.b_dtype = PH_F32; d.B = B; d.ldb = ldb;
  d.c_dtype = PH_F32; d.C = C; d.ldc = ldc; d.math = math; d.alpha = 1.f;
  return d;
}

}  // namespace

int sample_actions(int dtype, const void* Y, size_t ldy, size_t N, size_t A, int has_value, uint64_t rng, int* act,
                   void* logp, void* val, double* out3, hipStream_t st) {
  if (N == 0) return PH_OK;
  const unsigned g = ceil_div(N, 256);
  if (dtype == PH_F64) {
    if (out3)
      k_sample_cat<double, true><<<g, 256, 0, st>>>((const double*)Y, (long)ldy, (long)N, (int)A, has_value, rng, act,
                                                     (double*)logp, (double*)val, out3);
    else
      k_sample_cat<double, false><<<g, 256, 0, st>>>((const double*)Y, (long)ldy, (long)N, (int)A, has_value, rng,
                                                      act, (double*)logp, (double*)val, nullptr);
  } else {
    if (out3)
      k_sample_cat<float, true><<<g, 256, 0, st>>>((const float*)Y, (long)ldy, (long)N, (int)A, has_value, rng, act,
                                                    (float*)logp, (float*)val, out3);
    else
      k_sample_cat<float, false><<<g, 256, 0, st>>>((const float*)Y, (long)ldy, (long)N, (int)A, has_value, rng, act,
                                                     (float*)logp, (float*)val, nullptr);
  }
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int mingru_rollout_step(const ph_mingru_dims& d, const float* params, const float* obs, float* state, float* out,
                        hipStream_t st) {
  const long N = d.B;
  const int D = d.D, H = d.H, L = d.L, A = d.A;
  const int math = d.precision ? PH_MATH_F32 : PH_MATH_BF16;
  const size_t nx = (size_t)N * H;
  float* base = (float*)scratch(kSlotRollout, (2 * nx + (size_t)N * 3 * H + (size_t)HP * H + HP) * 4);
  if (!base) return PH_ERR_NOMEM;
  float* x[2] = {base, base + nx};
  float* cmb = base + 2 * nx;
  float* wh = cmb + (size_t)N * 3 * H;
  float* bh = wh + (size_t)HP * H;
  k_rollout_head<<<ceil_div((size_t)HP * H + HP, 256), 256, 0, st>>>(params, D, H, L, A, wh, bh);
  PH_LAUNCH_CHECK();
  PhGemmDesc g = nt_f32((int)N, H, D, obs, D, params, D, x[0], H, math);
  g.epi = PH_EPI_BIAS;
  g.bias = params + (long)H * D;
  PH_TRY(gemm(g, st));
  const float* wl = params + (long)H * D + H;
  for (int l = 0; l < L; l++) {
    g = nt_f32((int)N, 3 * H, H, x[l & 1], H, wl + (long)l * 3 * H * H, H, cmb, 3 * H, math);
    PH_TRY(gemm(g, st));
    k_rollout_cell<<<ceil_div(nx, 256), 256, 0, st>>>(cmb, x[l & 1], state, x[(l + 1) & 1], N, L, H, l);
    PH_LAUNCH_CHECK();
  }
  g = nt_f32((int)N, A + 1, H, x[L & 1], H, wh, H, out, A + 1, math);
  g.epi = PH_EPI_BIAS;
  g.bias = bh;
  return gemm(g, st);
}

}  // namespace ph

using namespace ph;

extern "C" int ph_sample_actions(int dtype, const void* Y, size_t ldy, size_t N, size_t A, int has_value,
                                 uint64_t rng, int* act, void* logp, void* value, void* stream) {
  PH_REQUIRE(dtype == PH_F32 || dtype == PH_F64, "ph_sample_actions: dtype must be PH_F32 or PH_F64");
  PH_REQUIRE(A >= 1 && ldy >= A + (has_value ? 1 : 0), "ph_sample_actions: A=%zu ldy=%zu", A, ldy);
  PH_REQUIRE(N <= 0x7fffffffUL, "ph_sample_actions: N=%zu", N);
  if (N == 0) return PH_OK;
  PH_REQUIRE(Y, "ph_sample_actions: null logits");
  return sample_actions(dtype, Y, ldy, N, A, has_value, rng, act, logp, value, nullptr, (hipStream_t)stream);
}

extern "C" int ph_mingru_rollout_step(const ph_mingru_dims* d, const float* params, const float* obs, float* state,
                                      float* out, void* stream) {
  PH_REQUIRE(d && params && obs && state && out, "ph_mingru_rollout_step: null argument");
  PH_REQUIRE(d->B > 0 && d->D > 0 && d->H > 0 && d->L > 0 && d->A > 0 && d->A + 1 <= HP,
             "ph_mingru_rollout_step: envs=%d D=%d H=%d L=%d A=%d (A + 1 <= %d)", d->B, d->D, d->H, d->L, d->A, HP);
  return mingru_rollout_step(*d, params, obs, state, out, (hipStream_t)stream);
}
