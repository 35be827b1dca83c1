// Deterministic reductions and small elementwise kernels: advantage normalisation, column sums,
// dtype conversion, minibatch gathers. Every reduction uses a fixed partition and a fixed tree, so
// results are reproducible run to run (no float atomics).
#include "common.hpp"
#include "kernels.hpp"

namespace ph {

// Block-wide sum of one value per thread (256 threads) in a fixed tree; result valid in thread 0.
template <typename R>
__device__ inline R block_sum_256(R v, R* sh) {
  sh[threadIdx.x] = v;
  __syncthreads();
#pragma unroll
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) sh[threadIdx.x] += sh[threadIdx.x + s];
    __syncthreads();
  }
  return sh[0];
}

namespace {

// Two-pass mean/std over x[0..n) in fixed 4096-element chunks. Pass 0 stores each chunk's sum of x in
// part0, pass 1 each chunk's sum of (x - mean)^2 in part1. The passes and the normalisation form the
// mean and the std from the partials themselves (every block the same way: a strided sum per lane and
// the fixed tree), so no block waits on another inside a kernel; block 0 of pass 1 stores
// stats[0] = mean and block 0 of the normalisation (or of k_moments_std) stats[1] = sqrt(var) + eps.
template <typename R>
__device__ inline R fold_parts(const R* __restrict__ part, unsigned G, R* sh) {
  R a2 = 0;
  for (unsigned i = threadIdx.x; i < G; i += 256) a2 += part[i];
  const R tot = block_sum_256(a2, sh);
  __syncthreads();  // sh is reused by the caller
  return tot;
}

template <typename R>
__global__ void __launch_bounds__(256) k_moments(const R* __restrict__ x, size_t n, size_t chunk,
                                                 const R* __restrict__ part0, R* __restrict__ part,
                                                 R* __restrict__ stats, int mode) {
  __shared__ R sh[256];
  const size_t lo = (size_t)blockIdx.x * chunk;
  const size_t hi = lo + chunk < n ? lo + chunk : n;
  const R dn = (R)(n > 0 ? n : 1);
  R mean = R(0);
  if (mode) {
    mean = fold_parts(part0, gridDim.x, sh) / dn;
    if (blockIdx.x == 0 && threadIdx.x == 0) stats[0] = mean;
  }
  R acc = 0;
  for (size_t i = lo + threadIdx.x; i < hi; i += 256) {
    R v = x[i];
    if (mode) {
      R d = v - mean;
      acc += d * d;
    } else {
      acc += v;
    }
  }
  R s = block_sum_256(acc, sh);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

template <typename R>
__global__ void __launch_bounds__(256) k_normalize(const R* __restrict__ x, R* __restrict__ y, size_t n,
                                                   const R* __restrict__ part0, const R* __restrict__ part1,
                                                   unsigned G, R* __restrict__ stats, R eps) {
  __shared__ R sh[256];
  const R dn = (R)(n > 0 ? n : 1);
  const R mean = fold_parts(part0, G, sh) / dn;
  const R sd = sqrt(fold_parts(part1, G, sh) / dn) + eps;
  if (blockIdx.x == 0 && threadIdx.x == 0) stats[1] = sd;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (x[i] - mean) / sd;
}

template <typename R>
__global__ void __launch_bounds__(256) k_moments_std(size_t n, const R* __restrict__ part1, unsigned G,
                                                     R* __restrict__ stats, R eps) {
  __shared__ R sh[256];
  const R dn = (R)(n > 0 ? n : 1);
  const R sd = sqrt(fold_parts(part1, G, sh) / dn) + eps;
  if (threadIdx.x == 0) stats[1] = sd;
}

// Column sums of a row-major [N x J] matrix (fp32 or bf16 elements), deterministic.
// Pass 1: grid (column blocks, G row chunks). A block is CT column threads x (256/CT) row lanes;
// each thread owns V consecutive columns (one 16-byte fp32 / 8-byte bf16 load per row when V = 4)
// and walks its lane's rows of the chunk; the row lanes are then added in lane order into
// partials [G][J]. CT is sized to the matrix width so narrow matrices keep all lanes busy.
// Pass 2: 64 columns per block, 4 lanes per column each adding every 4th partial in order, then
// ((l0 + l1) + l2) + l3.
__device__ inline float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ inline float4 load4(const uint16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(bf16_to_f32((uint16_t)(u.x & 0xffffu)), bf16_to_f32((uint16_t)(u.x >> 16)),
                     bf16_to_f32((uint16_t)(u.y & 0xffffu)), bf16_to_f32((uint16_t)(u.y >> 16)));
}
__device__ inline float load1(const float* p) { return *p; }
__device__ inline float load1(const uint16_t* p) { return bf16_to_f32(*p); }

template <typename T, int V>
__global__ void __launch_bounds__(256) k_colsum_part(const T* __restrict__ X, long N, int J, long ld,
                                                     long rows_per, int ct, float* __restrict__ part) {
  __shared__ float4 sh[256];
  const int cg = threadIdx.x % ct, rl = threadIdx.x / ct, nrl = 256 / ct;
  const int c = (blockIdx.x * ct + cg) * V;
  const long lo = (long)blockIdx.y * rows_per;
  const long hi = lo + rows_per < N ? lo + rows_per : N;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c < J && rl < nrl) {
    if constexpr (V == 4) {
#pragma unroll 4
      for (long r = lo + rl; r < hi; r += nrl) {
        const float4 v = load4(X + r * ld + c);
        acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
      }
    } else {
#pragma unroll 4
      for (long r = lo + rl; r < hi; r += nrl) acc.x += load1(X + r * ld + c);
    }
  }
  sh[threadIdx.x] = acc;
  __syncthreads();
  if (rl == 0 && c < J) {
    float4 s4 = sh[cg];
    for (int q = 1; q < nrl; q++) {
      const float4 v = sh[q * ct + cg];
      s4.x += v.x; s4.y += v.y; s4.z += v.z; s4.w += v.w;
    }
    float* o = part + (long)blockIdx.y * J + c;
    o[0] = s4.x;
    if constexpr (V == 4) { o[1] = s4.y; o[2] = s4.z; o[3] = s4.w; }
  }
}

// out[c] (+)= scale * sum of the G partials of column c: 16 lanes per column each add every 16th
// partial in order, then a fixed tree combines the 16 lane sums.
__global__ void __launch_bounds__(256) k_colsum_finish(const float* __restrict__ part, int G, int J,
                                                       float* __restrict__ out, float scale,
                                                       int accumulate) {
  __shared__ float sh[16][17];
  const int lc = threadIdx.x & 15, ln = threadIdx.x >> 4;
  const int c = blockIdx.x * 16 + lc;
  float s = 0.f;
  if (c < J) {
    // eight loads in flight at a time, added in partial order
    int g = ln;
    for (; g + 7 * 16 < G; g += 8 * 16) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; q++) v[q] = part[(long)(g + 16 * q) * J + c];
#pragma unroll
      for (int q = 0; q < 8; q++) s += v[q];
    }
    for (; g < G; g += 16) s += part[(long)g * J + c];
  }
  sh[ln][lc] = s;
  __syncthreads();
  for (int w = 8; w > 0; w >>= 1) {
    if (ln < w) sh[ln][lc] += sh[ln + w][lc];
    __syncthreads();
  }
  if (ln == 0 && c < J) {
    const float t = sh[0][lc] * scale;
    out[c] = accumulate ? out[c] + t : t;
  }
}

template <typename T>
int colsum_t(const T* X, long N, int J, long ld, float* out, float scale, int accumulate,
             hipStream_t st) {
  if (J <= 0) return PH_OK;
  const bool vec = J % 4 == 0 && ld % 4 == 0 && ((uintptr_t)X % (4 * sizeof(T))) == 0;
  const int V = vec ? 4 : 1;
  const int groups = (J + V - 1) / V;           // column threads needed
  int ct = 64;
  while (ct > 1 && ct / 2 >= groups) ct /= 2;   // narrow matrices: more row lanes per block
  const unsigned gx = (unsigned)((groups + ct - 1) / ct);
  // row slices of >= 128 rows, as many as keep the grid within about 1024 workgroups (a minibatch of
  // 32768 rows then spreads over 256 workgroups instead of 16); the slicing depends only on N and J
  long G = (N + 127) / 128;
  const long gmax = 1024 / (long)gx > 0 ? 1024 / (long)gx : 1;
  if (G > gmax) G = gmax;
  if (G < 1) G = 1;
  const long rows_per = (N + G - 1) / G;
  float* part = (float*)scratch(kSlotColsumPart, (size_t)G * J * 4);
  if (!part) return PH_ERR_NOMEM;
  dim3 grid(gx, (unsigned)G);
  if (vec) k_colsum_part<T, 4><<<grid, 256, 0, st>>>(X, N, J, ld, rows_per, ct, part);
  else k_colsum_part<T, 1><<<grid, 256, 0, st>>>(X, N, J, ld, rows_per, ct, part);
  k_colsum_finish<<<ceil_div(J, 16), 256, 0, st>>>(part, (int)G, J, out, scale, accumulate);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

template <typename S, typename D>
__global__ void k_convert(const S* __restrict__ x, D* __restrict__ y, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (D)x[i];
}

__global__ void k_f32_to_bf16(const float* __restrict__ x, uint16_t* __restrict__ y, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = bf16_rne(x[i]);
}

// 32x32 tiles through LDS (+1 column of padding against bank conflicts)
__global__ void k_transpose_u16(const uint16_t* __restrict__ X, uint16_t* __restrict__ Xt, int rows,
                                int cols) {
  __shared__ uint16_t t[32][33];
  const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 8 rows per pass
  for (int r = ty; r < 32; r += 8) {
    const int i = by + r, j = bx + tx;
    if (i < rows && j < cols) t[r][tx] = X[(long)i * cols + j];
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int j = bx + r, i = by + tx;
    if (i < rows && j < cols) Xt[(long)j * rows + i] = t[tx][r];
  }
}

}  // namespace

int transpose_bf16(const uint16_t* X, uint16_t* Xt, int rows, int cols, hipStream_t st) {
  if (rows == 0 || cols == 0) return PH_OK;
  dim3 grid(ceil_div(cols, 32), ceil_div(rows, 32));
  k_transpose_u16<<<grid, 256, 0, st>>>(X, Xt, rows, cols);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int moments_normalize(int dtype, const void* x, size_t n, void* y, void* stats, hipStream_t st) {
  if (n == 0) return PH_OK;
  const size_t G = moments_chunks(n);
  const size_t es = dtype == PH_F64 ? 8 : 4;
  uint8_t* part = (uint8_t*)scratch(kSlotMomentsPart, 2 * G * es);
  if (!part) return PH_ERR_NOMEM;
  if (!stats) {
    stats = scratch(kSlotMomentsStats, 16);
    if (!stats) return PH_ERR_NOMEM;
  }
  return moments_normalize_ws(dtype, x, n, y, stats, part, st);
}

// The same with the caller's workspace: part holds 2 * moments_chunks(n) elements of dtype, stats
// 2 elements. Every partial is written before it is read, so neither needs clearing.
int moments_normalize_ws(int dtype, const void* x, size_t n, void* y, void* stats, void* part_ws,
                         hipStream_t st) {
  if (n == 0) return PH_OK;
  const size_t chunk = kMomentsChunk;
  const size_t G = moments_chunks(n);
  uint8_t* part = (uint8_t*)part_ws;
  const unsigned g = (unsigned)G;
  if (dtype == PH_F64) {
    using R = double;
    R *p0 = (R*)part, *p1 = p0 + G;
    k_moments<R><<<g, 256, 0, st>>>((const R*)x, n, chunk, nullptr, p0, (R*)stats, 0);
    k_moments<R><<<g, 256, 0, st>>>((const R*)x, n, chunk, p0, p1, (R*)stats, 1);
    if (y) k_normalize<R><<<ceil_div(n, 256), 256, 0, st>>>((const R*)x, (R*)y, n, p0, p1, g, (R*)stats, 1e-8);
    else k_moments_std<R><<<1, 256, 0, st>>>(n, p1, g, (R*)stats, 1e-8);
  } else {
    using R = float;
    R *p0 = (R*)part, *p1 = p0 + G;
    k_moments<R><<<g, 256, 0, st>>>((const R*)x, n, chunk, nullptr, p0, (R*)stats, 0);
    k_moments<R><<<g, 256, 0, st>>>((const R*)x, n, chunk, p0, p1, (R*)stats, 1);
    if (y) k_normalize<R><<<ceil_div(n, 256), 256, 0, st>>>((const R*)x, (R*)y, n, p0, p1, g, (R*)stats, 1e-8f);
    else k_moments_std<R><<<1, 256, 0, st>>>(n, p1, g, (R*)stats, 1e-8f);
  }
  PH_LAUNCH_CHECK();
  return PH_OK;
}

int colsum_f32(const float* X, size_t N, int J, size_t ld, float* out, float scale, int accumulate,
               hipStream_t st) {
  return colsum_t<float>(X, (long)N, J, (long)ld, out, scale, accumulate, st);
}

int colsum_bf16(const uint16_t* X, long N, int J, long ld, float* out, float scale, int accumulate,
                hipStream_t st) {
  return colsum_t<uint16_t>(X, N, J, ld, out, scale, accumulate, st);
}

int convert(int src_dtype, const void* x, int dst_dtype, void* y, size_t n, hipStream_t st) {
  if (n == 0) return PH_OK;
  const unsigned g = ceil_div(n, 256);
  if (src_dtype == PH_F64 && dst_dtype == PH_F32)
    k_convert<double, float><<<g, 256, 0, st>>>((const double*)x, (float*)y, n);
  else if (src_dtype == PH_F32 && dst_dtype == PH_F64)
    k_convert<float, double><<<g, 256, 0, st>>>((const float*)x, (double*)y, n);
  else if (src_dtype == PH_F64 && dst_dtype == PH_I32)
    k_convert<double, int><<<g, 256, 0, st>>>((const double*)x, (int*)y, n);
  else if (src_dtype == PH_F32 && dst_dtype == PH_BF16)
    k_f32_to_bf16<<<g, 256, 0, st>>>((const float*)x, (uint16_t*)y, n);
  else {
    set_error("convert: unsupported dtype pair %d -> %d", src_dtype, dst_dtype);
    return PH_ERR_ARG;
  }
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_adv_normalize(int dtype, const void* adv, size_t n, void* out, void* stats,
                                void* stream) {
  PH_REQUIRE(dtype == PH_F32 || dtype == PH_F64, "ph_adv_normalize: dtype must be F32 or F64");
  PH_REQUIRE(n == 0 || (adv && out), "ph_adv_normalize: null pointer");
  return moments_normalize(dtype, adv, n, out, stats, as_stream(stream));
}

extern "C" int ph_colsum(const float* X, size_t N, size_t J, size_t ld, float* out, float scale,
                         int accumulate, void* stream) {
  PH_REQUIRE(J <= (size_t)INT32_MAX, "ph_colsum: too many columns");
  PH_REQUIRE(N * J == 0 || (X && out), "ph_colsum: null pointer");
  return colsum_f32(X, N, (int)J, ld ? ld : J, out, scale, accumulate, as_stream(stream));
}

extern "C" int ph_convert(int src_dtype, const void* x, int dst_dtype, void* y, size_t n,
                          void* stream) {
  return convert(src_dtype, x, dst_dtype, y, n, as_stream(stream));
}
