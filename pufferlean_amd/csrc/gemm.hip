// Policy GEMMs on CDNA4 matrix cores.
//
// C[MxN] = op(A)[MxK] * op(B)[KxN], row-major storage; op(A) is A or A^T (A stored [K][M]),
// op(B) is B or B^T (B stored [N][K]). Math is either bf16 MFMA (v_mfma_f32_32x32x16_bf16, fp32
// accumulate; fp32 inputs are rounded to bf16 RNE on their way into LDS, i.e. the reference's
// FAST_16BF semantics) or fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Block = 4 wavefronts in a 2x2 grid over a BM x BN tile; each wavefront owns (BM/2) x (BN/2) as
// 32x32 MFMA sub-tiles. Operand tiles are staged through double-buffered LDS in a k-contiguous
// [row][BK+pad] layout so every MFMA operand fetch is one 16-byte LDS read per lane. Sources that
// are k-contiguous (X in the forward, W^T) are copied with 16-byte vector moves; m/n-contiguous
// sources (the dgrad weight, both wgrad operands) are transposed while being written to LDS.
// The reduction over k is evaluated in a lane-permuted order (each lane reads 2x8 (bf16) or 4 (f32)
// consecutive k and the MFMAs cover them in pairs), which is a permutation of the same sum.
//
// Epilogues are fused: bias, bias+ReLU, ReLU-mask by an aux tensor, alpha*acc+beta*aux, plus an
// optional second bf16 output (plain or transposed). Split-K writes fp32 partials per split and a
// second kernel adds them in split order (deterministic).
#include "common.hpp"
#include "kernels.hpp"

namespace ph {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
  int M, N, K;
  const void* A;
  long lda;
  const void* B;
  long ldb;
  void* C;
  long ldc;
  int c_bf16;
  int epi;
  const float* bias;
  const void* aux;  // same dtype as C
  long ldaux;
  float alpha, beta;
  uint16_t* C2;  // optional bf16 copy of the result
  long ldc2;
  int c2_trans;
  int kps;       // k per split
  float* ws;     // split-K partials [splits][M][N]
  int remap;     // XCD-aware tile order
};

__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
}

// 8 consecutive source elements -> 8 bf16 (raw bits in a uint4).
__device__ inline uint4 load8_bf16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ inline uint4 load8_bf16(const float* p) {
  const float4 x = reinterpret_cast<const float4*>(p)[0];
  const float4 y = reinterpret_cast<const float4*>(p)[1];
  uint4 r;
  r.x = pack_bf16x2(x.x, x.y);
  r.y = pack_bf16x2(x.z, x.w);
  r.z = pack_bf16x2(y.x, y.y);
  r.w = pack_bf16x2(y.z, y.w);
  return r;
}

__device__ inline float to_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ inline float to_f32(float v) { return v; }

// Thread-block tile id -> (tile_m, tile_n). With remap, the blocks that land on one XCD (blocks are
// dispatched round-robin over the 8 XCDs) get a contiguous run of tiles sharing the same A rows.
__device__ inline void tile_coords(int tm, int tn, int remap, int& bm, int& bn) {
  int id = blockIdx.x;
  const int total = tm * tn;
  if (remap && (total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  bm = id / tn;
  bn = id % tn;
}

template <typename TOut>
__device__ inline void store_out(TOut* p, float v);
template <>
__device__ inline void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ inline void store_out<uint16_t>(uint16_t* p, float v) { *p = f32_to_bf16_rne(v); }

template <typename TC>
__device__ inline void epilogue_store(const GemmArgs& g, int row, int col, float acc) {
  if (row >= g.M || col >= g.N) return;
  float v = acc;
  switch (g.epi) {
    case PH_EPI_BIAS: v = acc + g.bias[col]; break;
    case PH_EPI_BIAS_RELU: v = fmaxf(acc + g.bias[col], 0.f); break;
    case PH_EPI_RELU_MASK: {
      const float h = to_f32(reinterpret_cast<const TC*>(g.aux)[(long)row * g.ldaux + col]);
      v = h > 0.f ? acc : 0.f;
      break;
    }
    case PH_EPI_AXPBY: {
      const float x = g.aux ? to_f32(reinterpret_cast<const TC*>(g.aux)[(long)row * g.ldaux + col]) : 0.f;
      v = g.alpha * acc + g.beta * x;
      break;
    }
    default: break;
  }
  store_out<TC>(reinterpret_cast<TC*>(g.C) + (long)row * g.ldc + col, v);
  if (g.C2) {
    const long o = g.c2_trans ? (long)col * g.ldc2 + row : (long)row * g.ldc2 + col;
    g.C2[o] = f32_to_bf16_rne(v);
  }
}

// ------------------------------------------------------------------------------------------------
// bf16-math kernel.
template <int BM, int BN, int BK, bool TA, bool TB, typename TIA, typename TIB, typename TC>
__global__ void __launch_bounds__(256) k_gemm_bf16(GemmArgs g) {
  constexpr int PAD = 8;
  constexpr int LDK = BK + PAD;             // LDS row pitch in bf16 elements
  constexpr int WM = BM / 2, WN = BN / 2;   // per-wave tile
  constexpr int SM = WM / 32, SN = WN / 32; // 32x32 sub-tiles per wave
  constexpr int CA = BM * BK / 8 / 256;     // 8-element chunks per thread (A)
  constexpr int CB = BN * BK / 8 / 256;
  static_assert(CA >= 1 && CB >= 1, "tile too small for 256 threads");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32");

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(tm, tn, g.remap, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int kbeg = blockIdx.z * g.kps;
  const int kend = min(g.K, kbeg + g.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const TIA* A = reinterpret_cast<const TIA*>(g.A);
  const TIB* B = reinterpret_cast<const TIB*>(g.B);

  uint4 ra[CA], rb[CB];

  // Global -> registers for k-tile starting at k0. Out-of-range elements read as zero.
  auto gload = [&](int k0) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int id = tid + c * 256;
      int r, k;
      if (!TA) { r = id / (BK / 8); k = (id % (BK / 8)) * 8; }
      else { k = id / (BM / 8); r = (id % (BM / 8)) * 8; }
      const int gm = m0 + r, gk = k0 + k;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (!TA) {
        if (gm < g.M && gk < kend) v = load8_bf16(A + (long)gm * g.lda + gk);
      } else {
        if (gk < kend && gm < g.M) v = load8_bf16(A + (long)gk * g.lda + gm);
      }
      ra[c] = v;
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int id = tid + c * 256;
      int r, k;
      if (TB) { r = id / (BK / 8); k = (id % (BK / 8)) * 8; }
      else { k = id / (BN / 8); r = (id % (BN / 8)) * 8; }
      const int gn = n0 + r, gk = k0 + k;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (TB) {
        if (gn < g.N && gk < kend) v = load8_bf16(B + (long)gn * g.ldb + gk);
      } else {
        if (gk < kend && gn < g.N) v = load8_bf16(B + (long)gk * g.ldb + gn);
      }
      rb[c] = v;
    }
  };
  // Registers -> LDS buffer `s` (transposing m/n-contiguous chunks).
  auto sstore = [&](int s) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int id = tid + c * 256;
      if (!TA) {
        const int r = id / (BK / 8), k = (id % (BK / 8)) * 8;
        *reinterpret_cast<uint4*>(&sA[s][r * LDK + k]) = ra[c];
      } else {
        const int k = id / (BM / 8), r = (id % (BM / 8)) * 8;
        const uint32_t w[4] = {ra[c].x, ra[c].y, ra[c].z, ra[c].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          sA[s][(r + 2 * q) * LDK + k] = (uint16_t)(w[q] & 0xffffu);
          sA[s][(r + 2 * q + 1) * LDK + k] = (uint16_t)(w[q] >> 16);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int id = tid + c * 256;
      if (TB) {
        const int r = id / (BK / 8), k = (id % (BK / 8)) * 8;
        *reinterpret_cast<uint4*>(&sB[s][r * LDK + k]) = rb[c];
      } else {
        const int k = id / (BN / 8), r = (id % (BN / 8)) * 8;
        const uint32_t w[4] = {rb[c].x, rb[c].y, rb[c].z, rb[c].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          sB[s][(r + 2 * q) * LDK + k] = (uint16_t)(w[q] & 0xffffu);
          sB[s][(r + 2 * q + 1) * LDK + k] = (uint16_t)(w[q] >> 16);
        }
      }
    }
  };

  floatx16 acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int lr = lane & 31;         // row (A) / column (B) inside a 32x32 sub-tile
  const int lk = (lane >> 5) * 16;  // this lane's 16-wide k slice inside each 32-wide k block

  if (nk > 0) {
    gload(kbeg);
    sstore(0);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; kt++) {
    const int s = kt & 1;
    if (kt + 1 < nk) gload(kbeg + (kt + 1) * BK);
#pragma unroll
    for (int kb = 0; kb < BK; kb += 32) {
      uint4 a0[SM], a1[SM], b0[SN], b1[SN];
#pragma unroll
      for (int i = 0; i < SM; i++) {
        const uint16_t* p = &sA[s][(wm0 + i * 32 + lr) * LDK + kb + lk];
        a0[i] = *reinterpret_cast<const uint4*>(p);
        a1[i] = *reinterpret_cast<const uint4*>(p + 8);
      }
#pragma unroll
      for (int j = 0; j < SN; j++) {
        const uint16_t* p = &sB[s][(wn0 + j * 32 + lr) * LDK + kb + lk];
        b0[j] = *reinterpret_cast<const uint4*>(p);
        b1[j] = *reinterpret_cast<const uint4*>(p + 8);
      }
#pragma unroll
      for (int i = 0; i < SM; i++)
#pragma unroll
        for (int j = 0; j < SN; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a0[i]), __builtin_bit_cast(bf16x8_t, b0[j]), acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8_t, a1[i]), __builtin_bit_cast(bf16x8_t, b1[j]), acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < nk) sstore(s ^ 1);
    __syncthreads();
  }

  // Accumulator layout of a 32x32 MFMA: lane holds column (lane & 31); element r sits in row
  // 8*(r/4) + 4*(lane/32) + (r%4).
  const int hrow = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm0 + i * 32 + 8 * (r >> 2) + hrow + (r & 3);
        const int col = n0 + wn0 + j * 32 + lr;
        if (g.ws) {
          if (row < g.M && col < g.N) g.ws[((long)blockIdx.z * g.M + row) * g.N + col] = acc[i][j][r];
        } else {
          epilogue_store<TC>(g, row, col, acc[i][j][r]);
        }
      }
}

// ------------------------------------------------------------------------------------------------
// fp32-math kernel (fp32 inputs only).
template <int BM, int BN, int BK, bool TA, bool TB, typename TC>
__global__ void __launch_bounds__(256) k_gemm_f32(GemmArgs g) {
  constexpr int PAD = 4;
  constexpr int LDK = BK + PAD;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int SM = WM / 32, SN = WN / 32;
  constexpr int CA = BM * BK / 4 / 256;  // 4-element chunks per thread
  constexpr int CB = BN * BK / 4 / 256;
  static_assert(CA >= 1 && CB >= 1, "tile too small");
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");

  __shared__ __attribute__((aligned(16))) float sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) float sB[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(tm, tn, g.remap, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int kbeg = blockIdx.z * g.kps;
  const int kend = min(g.K, kbeg + g.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;
  const float* A = reinterpret_cast<const float*>(g.A);
  const float* B = reinterpret_cast<const float*>(g.B);
  float4 ra[CA], rb[CB];

  auto gload = [&](int k0) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int id = tid + c * 256;
      int r, k;
      if (!TA) { r = id / (BK / 4); k = (id % (BK / 4)) * 4; }
      else { k = id / (BM / 4); r = (id % (BM / 4)) * 4; }
      const int gm = m0 + r, gk = k0 + k;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (gm < g.M && gk < kend)
        v = !TA ? *reinterpret_cast<const float4*>(A + (long)gm * g.lda + gk)
                : *reinterpret_cast<const float4*>(A + (long)gk * g.lda + gm);
      ra[c] = v;
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int id = tid + c * 256;
      int r, k;
      if (TB) { r = id / (BK / 4); k = (id % (BK / 4)) * 4; }
      else { k = id / (BN / 4); r = (id % (BN / 4)) * 4; }
      const int gn = n0 + r, gk = k0 + k;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (gn < g.N && gk < kend)
        v = TB ? *reinterpret_cast<const float4*>(B + (long)gn * g.ldb + gk)
               : *reinterpret_cast<const float4*>(B + (long)gk * g.ldb + gn);
      rb[c] = v;
    }
  };
  auto sstore = [&](int s) {
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const int id = tid + c * 256;
      if (!TA) {
        const int r = id / (BK / 4), k = (id % (BK / 4)) * 4;
        *reinterpret_cast<float4*>(&sA[s][r * LDK + k]) = ra[c];
      } else {
        const int k = id / (BM / 4), r = (id % (BM / 4)) * 4;
        sA[s][(r + 0) * LDK + k] = ra[c].x;
        sA[s][(r + 1) * LDK + k] = ra[c].y;
        sA[s][(r + 2) * LDK + k] = ra[c].z;
        sA[s][(r + 3) * LDK + k] = ra[c].w;
      }
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const int id = tid + c * 256;
      if (TB) {
        const int r = id / (BK / 4), k = (id % (BK / 4)) * 4;
        *reinterpret_cast<float4*>(&sB[s][r * LDK + k]) = rb[c];
      } else {
        const int k = id / (BN / 4), r = (id % (BN / 4)) * 4;
        sB[s][(r + 0) * LDK + k] = rb[c].x;
        sB[s][(r + 1) * LDK + k] = rb[c].y;
        sB[s][(r + 2) * LDK + k] = rb[c].z;
        sB[s][(r + 3) * LDK + k] = rb[c].w;
      }
    }
  };

  floatx16 acc[SM][SN];
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  const int lr = lane & 31;
  const int lk = (lane >> 5) * 4;  // 4-wide k slice in each 8-wide k block

  if (nk > 0) {
    gload(kbeg);
    sstore(0);
    __syncthreads();
  }
  for (int kt = 0; kt < nk; kt++) {
    const int s = kt & 1;
    if (kt + 1 < nk) gload(kbeg + (kt + 1) * BK);
#pragma unroll
    for (int kb = 0; kb < BK; kb += 8) {
      float4 a[SM], b[SN];
#pragma unroll
      for (int i = 0; i < SM; i++) a[i] = *reinterpret_cast<const float4*>(&sA[s][(wm0 + i * 32 + lr) * LDK + kb + lk]);
#pragma unroll
      for (int j = 0; j < SN; j++) b[j] = *reinterpret_cast<const float4*>(&sB[s][(wn0 + j * 32 + lr) * LDK + kb + lk]);
#pragma unroll
      for (int i = 0; i < SM; i++)
#pragma unroll
        for (int j = 0; j < SN; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
        }
    }
    if (kt + 1 < nk) sstore(s ^ 1);
    __syncthreads();
  }
  const int hrow = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm0 + i * 32 + 8 * (r >> 2) + hrow + (r & 3);
        const int col = n0 + wn0 + j * 32 + lr;
        if (g.ws) {
          if (row < g.M && col < g.N) g.ws[((long)blockIdx.z * g.M + row) * g.N + col] = acc[i][j][r];
        } else {
          epilogue_store<TC>(g, row, col, acc[i][j][r]);
        }
      }
}

// Split-K fold: C = epilogue(sum over splits in order).
template <typename TC>
__global__ void k_splitk_reduce(GemmArgs g, int splits) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long MN = (long)g.M * g.N;
  if (idx >= MN) return;
  float s = 0.f;
  for (int z = 0; z < splits; z++) s += g.ws[(long)z * MN + idx];
  epilogue_store<TC>(g, (int)(idx / g.N), (int)(idx % g.N), s);
}

// ------------------------------------------------------------------------------------------------
template <int BM, int BN, int BK, bool TA, bool TB, typename TIA, typename TIB>
void launch_bf16(const GemmArgs& g, dim3 grid, hipStream_t st) {
  if (g.c_bf16) k_gemm_bf16<BM, BN, BK, TA, TB, TIA, TIB, uint16_t><<<grid, 256, 0, st>>>(g);
  else k_gemm_bf16<BM, BN, BK, TA, TB, TIA, TIB, float><<<grid, 256, 0, st>>>(g);
}

template <int BM, int BN, int BK, typename TIA, typename TIB>
void dispatch_bf16_t(const GemmArgs& g, int ta, int tb, dim3 grid, hipStream_t st) {
  if (!ta && !tb) launch_bf16<BM, BN, BK, false, false, TIA, TIB>(g, grid, st);
  else if (!ta && tb) launch_bf16<BM, BN, BK, false, true, TIA, TIB>(g, grid, st);
  else if (ta && !tb) launch_bf16<BM, BN, BK, true, false, TIA, TIB>(g, grid, st);
  else launch_bf16<BM, BN, BK, true, true, TIA, TIB>(g, grid, st);
}

template <int BM, int BN, int BK>
void dispatch_bf16(const GemmArgs& g, int a_dt, int b_dt, int ta, int tb, dim3 grid, hipStream_t st) {
  if (a_dt == PH_BF16 && b_dt == PH_BF16) dispatch_bf16_t<BM, BN, BK, uint16_t, uint16_t>(g, ta, tb, grid, st);
  else if (a_dt == PH_F32 && b_dt == PH_F32) dispatch_bf16_t<BM, BN, BK, float, float>(g, ta, tb, grid, st);
  else if (a_dt == PH_BF16 && b_dt == PH_F32) dispatch_bf16_t<BM, BN, BK, uint16_t, float>(g, ta, tb, grid, st);
  else dispatch_bf16_t<BM, BN, BK, float, uint16_t>(g, ta, tb, grid, st);
}

template <int BM, int BN, int BK>
void dispatch_f32(const GemmArgs& g, int ta, int tb, dim3 grid, hipStream_t st) {
#define PH_F32K(TA_, TB_)                                                                  \
  do {                                                                                     \
    if (g.c_bf16) k_gemm_f32<BM, BN, BK, TA_, TB_, uint16_t><<<grid, 256, 0, st>>>(g);      \
    else k_gemm_f32<BM, BN, BK, TA_, TB_, float><<<grid, 256, 0, st>>>(g);                  \
  } while (0)
  if (!ta && !tb) PH_F32K(false, false);
  else if (!ta && tb) PH_F32K(false, true);
  else if (ta && !tb) PH_F32K(true, false);
  else PH_F32K(true, true);
#undef PH_F32K
}

// Scalar fallback for shapes the MFMA kernels do not take: one lane per output element, fp32
// accumulation in ascending k; with bf16 math each operand is rounded to bf16 first.
template <typename TIA, typename TIB, typename TC>
__global__ void __launch_bounds__(256) k_gemm_scalar(GemmArgs g, int ta, int tb, int bf) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)g.M * g.N) return;
  const int row = (int)(idx / g.N), col = (int)(idx % g.N);
  const TIA* A = reinterpret_cast<const TIA*>(g.A);
  const TIB* B = reinterpret_cast<const TIB*>(g.B);
  float acc = 0.f;
  for (int k = 0; k < g.K; k++) {
    float a = to_f32(ta ? A[(long)k * g.lda + row] : A[(long)row * g.lda + k]);
    float b = to_f32(tb ? B[(long)col * g.ldb + k] : B[(long)k * g.ldb + col]);
    if (bf) {
      a = bf16_to_f32(f32_to_bf16_rne(a));
      b = bf16_to_f32(f32_to_bf16_rne(b));
    }
    acc += a * b;
  }
  epilogue_store<TC>(g, row, col, acc);
}

template <typename TIA, typename TIB>
void launch_scalar_t(const GemmArgs& g, int ta, int tb, int bf, hipStream_t st) {
  const unsigned grid = ceil_div((size_t)g.M * g.N, 256);
  if (g.c_bf16) k_gemm_scalar<TIA, TIB, uint16_t><<<grid, 256, 0, st>>>(g, ta, tb, bf);
  else k_gemm_scalar<TIA, TIB, float><<<grid, 256, 0, st>>>(g, ta, tb, bf);
}

int gemm_scalar(const GemmArgs& g, const PhGemmDesc& d, hipStream_t st) {
  const int bf = d.math == PH_MATH_BF16;
  if (d.a_dtype == PH_BF16 && d.b_dtype == PH_BF16) launch_scalar_t<uint16_t, uint16_t>(g, d.trans_a, d.trans_b, bf, st);
  else if (d.a_dtype == PH_F32 && d.b_dtype == PH_F32) launch_scalar_t<float, float>(g, d.trans_a, d.trans_b, bf, st);
  else if (d.a_dtype == PH_BF16) launch_scalar_t<uint16_t, float>(g, d.trans_a, d.trans_b, bf, st);
  else launch_scalar_t<float, uint16_t>(g, d.trans_a, d.trans_b, bf, st);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

}  // namespace

int gemm(const PhGemmDesc& d, hipStream_t st) {
  PH_REQUIRE(d.M >= 0 && d.N >= 0 && d.K >= 0, "gemm: negative extent");
  if (d.M == 0 || d.N == 0) return PH_OK;
  PH_REQUIRE(d.a_dtype == PH_F32 || d.a_dtype == PH_BF16, "gemm: A dtype must be F32 or BF16");
  PH_REQUIRE(d.b_dtype == PH_F32 || d.b_dtype == PH_BF16, "gemm: B dtype must be F32 or BF16");
  PH_REQUIRE(d.c_dtype == PH_F32 || d.c_dtype == PH_BF16, "gemm: C dtype must be F32 or BF16");
  PH_REQUIRE(d.math == PH_MATH_BF16 || (d.a_dtype == PH_F32 && d.b_dtype == PH_F32),
             "gemm: fp32 math needs fp32 inputs");
  PH_REQUIRE(d.epi == PH_EPI_NONE || d.epi == PH_EPI_BIAS || d.epi == PH_EPI_BIAS_RELU ||
                 d.epi == PH_EPI_RELU_MASK || d.epi == PH_EPI_AXPBY,
             "gemm: unknown epilogue %d", d.epi);
  PH_REQUIRE(!(d.epi == PH_EPI_BIAS || d.epi == PH_EPI_BIAS_RELU) || d.bias, "gemm: bias missing");
  PH_REQUIRE(d.epi != PH_EPI_RELU_MASK || d.aux, "gemm: mask tensor missing");

  GemmArgs g{};
  g.M = d.M; g.N = d.N; g.K = d.K;
  g.A = d.A; g.lda = d.lda; g.B = d.B; g.ldb = d.ldb;
  g.C = d.C; g.ldc = d.ldc; g.c_bf16 = d.c_dtype == PH_BF16;
  g.epi = d.epi; g.bias = d.bias; g.aux = d.aux; g.ldaux = d.ldaux ? d.ldaux : d.ldc;
  g.alpha = d.alpha; g.beta = d.beta;
  g.C2 = (uint16_t*)d.C2; g.ldc2 = d.ldc2; g.c2_trans = d.c2_trans;
  g.remap = 1;

  // Vector-load preconditions of the MFMA kernels: every 8 (bf16 math) or 4 (fp32 math) consecutive
  // elements along each operand's contiguous dimension, and along K, start on a multiple of that
  // count. Shapes that miss them (e.g. a 4-wide observation layer) take the scalar kernel.
  const int vec = d.math == PH_MATH_BF16 ? 8 : 4;
  const long a_contig = d.trans_a ? d.M : d.K, b_contig = d.trans_b ? d.K : d.N;
  const bool aligned = a_contig % vec == 0 && d.lda % vec == 0 && b_contig % vec == 0 &&
                       d.ldb % vec == 0 && d.K % vec == 0 && ((uintptr_t)d.A % 16) == 0 &&
                       ((uintptr_t)d.B % 16) == 0;
  if (!aligned) return gemm_scalar(g, d, st);

  // Tile choice: 128x128 when that gives >= 128 tiles; else 64x64 tiles when those reach 128;
  // else 128x128 with split-K up to 256 blocks, keeping >= 256 of k per split.
  int splits = d.splits > 0 ? d.splits : 1;
  const long tiles128 = (long)((d.M + 127) / 128) * ((d.N + 127) / 128);
  const long tiles64 = (long)((d.M + 63) / 64) * ((d.N + 63) / 64);
  bool small = false;
  if (d.splits <= 0 && tiles128 < 128) {
    if (tiles64 >= 128 || d.K < 512) {
      small = true;
    } else {
      const long want = 256 / (tiles128 > 0 ? tiles128 : 1);
      const long maxs = d.K / 256;
      splits = (int)(want < maxs ? want : maxs);
      if (splits < 1) splits = 1;
    }
  }
  const int BK = d.math == PH_MATH_BF16 ? 64 : 32;
  int kps = (d.K + splits - 1) / splits;
  kps = (kps + BK - 1) / BK * BK;
  splits = kps > 0 ? (d.K + kps - 1) / kps : 1;
  if (splits < 1) splits = 1;
  g.kps = kps > 0 ? kps : BK;
  if (splits > 1) {
    g.ws = (float*)scratch(kSlotGemmWs, (size_t)splits * d.M * d.N * 4);
    if (!g.ws) return PH_ERR_NOMEM;
  }
  const int bm = small ? 64 : 128, bn = small ? 64 : 128;
  const unsigned tiles = (unsigned)(((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn));
  dim3 grid(tiles, 1, splits);
  if (d.math == PH_MATH_BF16) {
    if (small) dispatch_bf16<64, 64, 64>(g, d.a_dtype, d.b_dtype, d.trans_a, d.trans_b, grid, st);
    else dispatch_bf16<128, 128, 64>(g, d.a_dtype, d.b_dtype, d.trans_a, d.trans_b, grid, st);
  } else {
    if (small) dispatch_f32<64, 64, 32>(g, d.trans_a, d.trans_b, grid, st);
    else dispatch_f32<128, 128, 32>(g, d.trans_a, d.trans_b, grid, st);
  }
  PH_LAUNCH_CHECK();
  if (splits > 1) {
    const long MN = (long)d.M * d.N;
    if (g.c_bf16) k_splitk_reduce<uint16_t><<<ceil_div(MN, 256), 256, 0, st>>>(g, splits);
    else k_splitk_reduce<float><<<ceil_div(MN, 256), 256, 0, st>>>(g, splits);
    PH_LAUNCH_CHECK();
  }
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_gemm(int trans_a, int trans_b, int M, int N, int K, int a_dtype, const void* A,
                       long lda, int b_dtype, const void* B, long ldb, int c_dtype, void* C,
                       long ldc, int math, int epilogue, const float* bias, const void* aux,
                       long ldaux, float alpha, float beta, void* C2, long ldc2, int c2_trans,
                       int splits, void* stream) {
  PhGemmDesc d{};
  d.trans_a = trans_a; d.trans_b = trans_b; d.M = M; d.N = N; d.K = K;
  d.a_dtype = a_dtype; d.A = A; d.lda = lda; d.b_dtype = b_dtype; d.B = B; d.ldb = ldb;
  d.c_dtype = c_dtype; d.C = C; d.ldc = ldc; d.math = math; d.epi = epilogue; d.bias = bias;
  d.aux = aux; d.ldaux = ldaux; d.alpha = alpha; d.beta = beta; d.C2 = C2; d.ldc2 = ldc2;
  d.c2_trans = c2_trans; d.splits = splits;
  return gemm(d, as_stream(stream));
}
