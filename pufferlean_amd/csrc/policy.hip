// The persistent resident MLP policy of the rollout (lean_ffi_mlp_policy_load / _update / _forward /
// _free, pufferblas.c:460-592) and the two-layer forward throughput entries (lean_ffi_bench_mlp2_bf16_
// resident, pufferblas.c:421-452; lean_ffi_bench_mlp2_bf16_wres, 598-636), plus lean_cuda_selftest
// (puffercuda.cu:41-60).
//
// A policy handle owns the weights on the device in the forms the forward reads: W1 as bf16 (the
// observations travel as bf16, halving the per-step upload), b1, W2 and b2 as fp32. The forward is
//   H1 = relu(Xb W1b^T + b1)   bf16 x bf16 products, fp32 accumulate and output
//   Y  = H1 W2^T + b2          fp32 storage, bf16 MFMA (the reference's FAST_16BF)
// with H1 kept on the device, as the reference's. Observations and outputs pass through pinned host
// staging that grows with N.
#include "common.hpp"
#include "kernels.hpp"

namespace ph {
namespace {

constexpr unsigned kB = 256;

struct MlpPolicy {
  int dev = -1;
  size_t D = 0, H = 0, O = 0, capN = 0;
  uint16_t* w1b = nullptr;  // device bf16 [H][D]
  float *b1 = nullptr, *w2 = nullptr, *b2 = nullptr;
  uint16_t* xb = nullptr;   // device bf16 [capN][D]
  float *h1 = nullptr, *out = nullptr;
  uint16_t* hx = nullptr;   // pinned host bf16 obs staging
  float* hy = nullptr;      // pinned host fp32 output staging
};

void release_rows(MlpPolicy* p) {
  if (p->xb) (void)hipFree(p->xb);
  if (p->h1) (void)hipFree(p->h1);
  if (p->out) (void)hipFree(p->out);
  if (p->hx) (void)hipHostFree(p->hx);
  if (p->hy) (void)hipHostFree(p->hy);
  p->xb = nullptr; p->h1 = p->out = nullptr; p->hx = nullptr; p->hy = nullptr;
  p->capN = 0;
}

void release(MlpPolicy* p) {
  release_rows(p);
  if (p->w1b) (void)hipFree(p->w1b);
  if (p->b1) (void)hipFree(p->b1);
  if (p->w2) (void)hipFree(p->w2);
  if (p->b2) (void)hipFree(p->b2);
  delete p;
}

// Grow the per-row buffers (device and pinned host) to N rows.
int ensure_rows(MlpPolicy* p, size_t N) {
  if (p->capN >= N) return PH_OK;
  release_rows(p);
  if (hipMalloc((void**)&p->xb, 2 * N * p->D) != hipSuccess || hipMalloc((void**)&p->h1, 4 * N * p->H) != hipSuccess ||
      hipMalloc((void**)&p->out, 4 * N * p->O) != hipSuccess ||
      hipHostMalloc((void**)&p->hx, 2 * N * p->D, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&p->hy, 4 * N * p->O, hipHostMallocDefault) != hipSuccess) {
    (void)hipGetLastError();
    release_rows(p);
    set_error("mlp policy: allocation of %zu rows failed", N);
    return PH_ERR_NOMEM;
  }
  p->capN = N;
  return PH_OK;
}

// Host f64 weights [W1 | b1 | W2 | b2] -> the handle's device forms (W1 through fp32 to bf16 RNE).
int upload_weights(MlpPolicy* p, const double* w) {
  const size_t D = p->D, H = p->H, O = p->O;
  std::string buf;
  buf.resize(2 * H * D + 4 * (H + O * H + O));
  uint16_t* w1 = reinterpret_cast<uint16_t*>(&buf[0]);
  float* rest = reinterpret_cast<float*>(&buf[2 * H * D]);
  for (size_t i = 0; i < H * D; i++) w1[i] = f32_to_bf16_rne((float)w[i]);
  for (size_t i = 0; i < H + O * H + O; i++) rest[i] = (float)w[H * D + i];
  PH_CHECK_HIP(hipMemcpy(p->w1b, w1, 2 * H * D, hipMemcpyHostToDevice));
  PH_CHECK_HIP(hipMemcpy(p->b1, rest, 4 * H, hipMemcpyHostToDevice));
  PH_CHECK_HIP(hipMemcpy(p->w2, rest + H, 4 * O * H, hipMemcpyHostToDevice));
  PH_CHECK_HIP(hipMemcpy(p->b2, rest + H + O * H, 4 * O, hipMemcpyHostToDevice));
  return PH_OK;
}

int check_handle(size_t handle, const char* who, MlpPolicy*& p) {
  p = reinterpret_cast<MlpPolicy*>(handle);
  PH_REQUIRE(p, "%s: null policy handle", who);
  int dev = -1;
  PH_CHECK_HIP(hipGetDevice(&dev));
  PH_REQUIRE(p->dev == dev, "%s: the handle belongs to device %d, the current device is %d", who, p->dev, dev);
  return PH_OK;
}

// The two products of the forward on the handle's device buffers, rows already in p->xb.
int forward_rows(const MlpPolicy* p, size_t N, hipStream_t st) {
  PhGemmDesc g{};
  g.trans_a = 0; g.trans_b = 1; g.M = (int)N; g.N = (int)p->H; g.K = (int)p->D;
  g.a_dtype = PH_BF16; g.A = p->xb; g.lda = (long)p->D; g.b_dtype = PH_BF16; g.B = p->w1b; g.ldb = (long)p->D;
  g.c_dtype = PH_F32; g.C = p->h1; g.ldc = (long)p->H; g.math = PH_MATH_BF16; g.alpha = 1.f;
  g.epi = PH_EPI_BIAS_RELU; g.bias = p->b1;
  PH_TRY(gemm(g, st));
  PhGemmDesc h{};
  h.trans_a = 0; h.trans_b = 1; h.M = (int)N; h.N = (int)p->O; h.K = (int)p->H;
  h.a_dtype = PH_F32; h.A = p->h1; h.lda = (long)p->H; h.b_dtype = PH_F32; h.B = p->w2; h.ldb = (long)p->H;
  h.c_dtype = PH_F32; h.C = p->out; h.ldc = (long)p->O; h.math = PH_MATH_BF16; h.alpha = 1.f;
  h.epi = PH_EPI_BIAS; h.bias = p->b2;
  return gemm(h, st);
}

int load(const double* w, size_t D, size_t H, size_t O, MlpPolicy*& out) {
  out = nullptr;
  PH_REQUIRE(w && D > 0 && H > 0 && O > 0, "ph_ffi_mlp_policy_load: bad arguments");
  MlpPolicy* p = new MlpPolicy();
  p->D = D; p->H = H; p->O = O;
  if (hipGetDevice(&p->dev) != hipSuccess || hipMalloc((void**)&p->w1b, 2 * H * D) != hipSuccess ||
      hipMalloc((void**)&p->b1, 4 * H) != hipSuccess || hipMalloc((void**)&p->w2, 4 * O * H) != hipSuccess ||
      hipMalloc((void**)&p->b2, 4 * O) != hipSuccess) {
    (void)hipGetLastError();
    release(p);
    set_error("ph_ffi_mlp_policy_load: device allocation failed");
    return PH_ERR_NOMEM;
  }
  const int s = upload_weights(p, w);
  if (s != PH_OK) {
    release(p);
    return s;
  }
  out = p;
  return PH_OK;
}

__global__ void k_selftest(double* out, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 2.0 * (double)i + 1.0;
}

template <typename F>
double timed_gflops(double flops_per_rep, size_t reps, const F& body) {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1.0;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return -1.0;
  }
  double r = -1.0;
  bool ok = true;
  for (int i = 0; i < 5 && ok; i++) ok = body() == PH_OK;  // warm-up, as the reference's 5 passes
  if (ok && hipDeviceSynchronize() == hipSuccess && hipEventRecord(e0, nullptr) == hipSuccess) {
    for (size_t i = 0; i < reps && ok; i++) ok = body() == PH_OK;
    float ms = 0.f;
    if (ok && hipEventRecord(e1, nullptr) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
        hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.f)
      r = flops_per_rep * (double)reps / (ms * 1e-3) / 1e9;
  }
  (void)hipGetLastError();
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return r;
}

}  // namespace
}  // namespace ph

using namespace ph;

extern "C" int ph_ffi_mlp_policy_load(const double* params, size_t D, size_t H, size_t O, size_t* handle) {
  PH_REQUIRE(handle, "ph_ffi_mlp_policy_load: null handle output");
  *handle = 0;
  MlpPolicy* p = nullptr;
  PH_TRY(load(params, D, H, O, p));
  *handle = reinterpret_cast<size_t>(p);
  return PH_OK;
}

extern "C" int ph_ffi_mlp_policy_update(size_t handle, const double* params) {
  MlpPolicy* p = nullptr;
  PH_TRY(check_handle(handle, "ph_ffi_mlp_policy_update", p));
  PH_REQUIRE(params, "ph_ffi_mlp_policy_update: null params");
  return upload_weights(p, params);
}

extern "C" int ph_ffi_mlp_policy_forward(size_t handle, const double* X, size_t N, double* Y) {
  MlpPolicy* p = nullptr;
  PH_TRY(check_handle(handle, "ph_ffi_mlp_policy_forward", p));
  if (N == 0) return PH_OK;
  PH_REQUIRE(X && Y, "ph_ffi_mlp_policy_forward: null buffer");
  PH_REQUIRE(N <= (size_t)INT32_MAX, "ph_ffi_mlp_policy_forward: N=%zu rows", N);
  PH_TRY(ensure_rows(p, N));
  const size_t nx = N * p->D, ny = N * p->O;
  for (size_t i = 0; i < nx; i++) p->hx[i] = f32_to_bf16_rne((float)X[i]);
  PH_CHECK_HIP(hipMemcpy(p->xb, p->hx, 2 * nx, hipMemcpyHostToDevice));
  PH_TRY(forward_rows(p, N, nullptr));
  PH_CHECK_HIP(hipMemcpy(p->hy, p->out, 4 * ny, hipMemcpyDeviceToHost));
  for (size_t i = 0; i < ny; i++) Y[i] = (double)p->hy[i];
  return PH_OK;
}

extern "C" size_t ph_ffi_mlp_policy_outputs(size_t handle) {
  const MlpPolicy* p = reinterpret_cast<const MlpPolicy*>(handle);
  return p ? p->O : 0;
}

extern "C" int ph_ffi_mlp_policy_free(size_t handle) {
  MlpPolicy* p = reinterpret_cast<MlpPolicy*>(handle);
  PH_REQUIRE(p, "ph_ffi_mlp_policy_free: null policy handle");
  PH_CHECK_HIP(hipDeviceSynchronize());
  release(p);
  return PH_OK;
}

// GF/s (2 N D H + 2 N H O per forward) of `reps` device-resident two-layer forwards on zero weights and
// inputs: the weights-resident ceiling of the rollout forward. -1 without a device.
extern "C" double ph_ffi_bench_mlp2_bf16_resident(size_t N, size_t D, size_t H, size_t O, size_t reps) {
  if (N * D * H * O == 0 || reps == 0 || N > (size_t)INT32_MAX) return -1.0;
  std::string zeros;
  zeros.assign(8 * (H * D + H + O * H + O), '\0');
  MlpPolicy* p = nullptr;
  if (load(reinterpret_cast<const double*>(zeros.data()), D, H, O, p) != PH_OK) return -1.0;
  double r = -1.0;
  if (ensure_rows(p, N) == PH_OK && hipMemset(p->xb, 0, 2 * N * D) == hipSuccess)
    r = timed_gflops(2.0 * (double)N * D * H + 2.0 * (double)N * H * O, reps,
                     [&]() -> int { return forward_rows(p, N, nullptr); });
  (void)hipDeviceSynchronize();
  release(p);
  return r;
}

// GF/s of the persistent-policy pattern: per forward the bf16 observations go up and the outputs come
// down (pinned staging), the weights stay resident. -1 without a device.
extern "C" double ph_ffi_bench_mlp2_bf16_wres(size_t N, size_t D, size_t H, size_t O, size_t reps) {
  if (N * D * H * O == 0 || reps == 0 || N > (size_t)INT32_MAX) return -1.0;
  std::string zeros;
  zeros.assign(8 * (H * D + H + O * H + O), '\0');
  MlpPolicy* p = nullptr;
  if (load(reinterpret_cast<const double*>(zeros.data()), D, H, O, p) != PH_OK) return -1.0;
  double r = -1.0;
  if (ensure_rows(p, N) == PH_OK) {
    memset(p->hx, 0, 2 * N * D);
    r = timed_gflops(2.0 * (double)N * D * H + 2.0 * (double)N * H * O, reps, [&]() -> int {
      if (hipMemcpyAsync(p->xb, p->hx, 2 * N * D, hipMemcpyHostToDevice, nullptr) != hipSuccess) return PH_ERR_HIP;
      PH_TRY(forward_rows(p, N, nullptr));
      if (hipMemcpyAsync(p->hy, p->out, 4 * N * O, hipMemcpyDeviceToHost, nullptr) != hipSuccess) return PH_ERR_HIP;
      return PH_OK;
    });
  }
  (void)hipDeviceSynchronize();
  release(p);
  return r;
}

extern "C" int ph_cuda_selftest(size_t n, double* out) {
  if (n == 0) return PH_OK;
  PH_REQUIRE(out, "ph_cuda_selftest: null output");
  double* d = nullptr;
  PH_CHECK_HIP(hipMalloc((void**)&d, 8 * n));
  k_selftest<<<ceil_div(n, kB), kB>>>(d, (long)n);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpy(out, d, 8 * n, hipMemcpyDeviceToHost);
  (void)hipFree(d);
  if (e != hipSuccess) {
    set_error("ph_cuda_selftest: %s", hipGetErrorString(e));
    return PH_ERR_HIP;
  }
  return PH_OK;
}
