// Policy GEMMs on CDNA4 matrix cores.
//
// C[MxN] = op(A)[MxK] * op(B)[KxN], row-major storage; op(A) is A or A^T (A stored [K][M]),
// op(B) is B or B^T (B stored [N][K]). Math is either bf16 MFMA (v_mfma_f32_32x32x16_bf16, fp32
// accumulate; fp32 inputs are rounded to bf16 RNE on their way into LDS, i.e. the reference's
// FAST_16BF semantics) or fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Block = 4 wavefronts in a 2x2 grid over a BM x BN tile; each wavefront owns (BM/2) x (BN/2) as
// 32x32 MFMA sub-tiles (the load-to-LDS NT kernel also runs 256x256 tiles on a 4x4 grid of 16
// wavefronts, one block per CU). Operand tiles are staged through double-buffered LDS in a k-contiguous
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

#include <type_traits>
#include <utility>

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
  const void* aux2;  // same dtype as C (kEpiGateSkip)
  long ldaux2;
  float alpha, beta;
  uint16_t* C2;  // optional bf16 copy of the result
  long ldc2;
  int c2_trans;
  int kps;       // k per split
  float* ws;     // split-K partials [splits][M][N] (inside a kernel: this block's split)
  int remap;     // XCD-aware tile order
  int split_xcd; // the tiles of one k-split on one XCD
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) { return bf16x2_rne(a, b); }

__device__ inline float to_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ inline float to_f32(float v) { return v; }

// Raw 8-element chunk as loaded (no conversion, so a prefetched load is not waited on until the
// chunk is written to LDS).
template <typename T> struct Raw8;
template <> struct Raw8<uint16_t> { uint4 v; };
template <> struct Raw8<float> { float4 a, b; };
// Operand pointers are used in the global address space explicitly, so a select between a source
// address and the zero page below still compiles to global (not flat) loads.
#define PH_GLOBAL __attribute__((address_space(1)))
template <typename T> using gptr = const PH_GLOBAL T*;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ inline Raw8<uint16_t> load_raw8(gptr<uint16_t> p) {
  const u32x4_t v = *reinterpret_cast<gptr<u32x4_t>>(p);
  return {make_uint4(v.x, v.y, v.z, v.w)};
}
__device__ inline Raw8<float> load_raw8(gptr<float> p) {
  const f32x4_t a = reinterpret_cast<gptr<f32x4_t>>(p)[0], b = reinterpret_cast<gptr<f32x4_t>>(p)[1];
  return {make_float4(a.x, a.y, a.z, a.w), make_float4(b.x, b.y, b.z, b.w)};
}
// Out-of-range chunks (rows past M, k past the split's end) are loaded from this zero page instead
// of being masked after the load, so no work touches a prefetched register before its LDS store.
__device__ const float4 kZeroPage[2] = {};
template <typename T>
__device__ __forceinline__ gptr<T> zero_page() { return (gptr<T>)(&kZeroPage[0]); }
__device__ inline uint4 to_bf16x8(const Raw8<uint16_t>& r) { return r.v; }
__device__ inline uint4 to_bf16x8(const Raw8<float>& r) {
  uint4 o;
  o.x = pack_bf16x2(r.a.x, r.a.y);
  o.y = pack_bf16x2(r.a.z, r.a.w);
  o.z = pack_bf16x2(r.b.x, r.b.y);
  o.w = pack_bf16x2(r.b.z, r.b.w);
  return o;
}

// Low half of the split x = hi + lo: lo = bf16(x - hi) for the 8 elements of a chunk.
__device__ inline uint4 lo_bf16x8(const Raw8<float>& r, const uint4& hi) {
  auto h = [](uint32_t w, int q) { return bf16_to_f32((uint16_t)(q ? (w >> 16) : (w & 0xffffu))); };
  uint4 o;
  o.x = pack_bf16x2(r.a.x - h(hi.x, 0), r.a.y - h(hi.x, 1));
  o.y = pack_bf16x2(r.a.z - h(hi.y, 0), r.a.w - h(hi.y, 1));
  o.z = pack_bf16x2(r.b.x - h(hi.z, 0), r.b.y - h(hi.z, 1));
  o.w = pack_bf16x2(r.b.z - h(hi.w, 0), r.b.w - h(hi.w, 1));
  return o;
}
__device__ inline uint4 lo_bf16x8(const Raw8<uint16_t>&, const uint4&) { return make_uint4(0, 0, 0, 0); }

// Workgroup barrier that orders LDS only: global loads still in flight (the prefetched k-tiles)
// are not drained, unlike __syncthreads(), whose fence waits for every outstanding memory access.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Position (row r, k) of a thread's chunk c inside an R x BK operand tile (8 consecutive elements
// along the source's contiguous dimension per chunk, CH chunks per thread, NT threads).
//  - k-contiguous source: chunks walk a row's k first, so each chunk is one 16-byte LDS row piece.
//  - m/n-contiguous source, CH >= 2: the thread owns CH consecutive k rows of one 8-wide column
//    group and transposes them in registers into 8 LDS row pieces of CH elements. Consecutive
//    threads take consecutive k groups: with the padded pitch this puts the 8/4-byte LDS writes of a
//    wavefront on distinct banks, and a wavefront's loads cover whole 64-byte row segments.
//  - m/n-contiguous source, CH == 1: consecutive threads walk the column groups of a k row and
//    write their 8 elements one at a time.
template <bool TRANS, int R, int BK, int CH, int NT>
__device__ __forceinline__ void chunk_rk(int tid, int c, int& r, int& k) {
  if constexpr (!TRANS) {
    const int id = tid + c * NT;
    r = id / (BK / 8);
    k = (id % (BK / 8)) * 8;
  } else if constexpr (CH >= 2) {
    constexpr int KG = BK / CH;
    static_assert((R / 8) * KG == NT, "transposed chunk mapping");
    r = (tid / KG) * 8;
    k = (tid % KG) * CH + c;
  } else {
    const int id = tid + c * NT;
    k = id / (R / 8);
    r = (id % (R / 8)) * 8;
  }
}

// LDS placement of operand element (row, k) inside one k-tile buffer.
//  BK == 32: unpadded 64-byte rows. The four 16-byte k-chunks of a row are XOR-swizzled by row bits
//    2-3, and the rows of each aligned group of four are permuted by row bits 3-4. Both MFMA operand
//    reads (16 rows x one chunk per 16 lanes), 16-byte tile stores (4 rows x 4 chunks) and the
//    transposed 8/4-byte stores (rows 8 apart in one instruction) then hit distinct banks.
//  otherwise: rows padded by 8 elements (a 144-byte pitch at BK = 64 is already conflict-free).
template <int BK>
struct LdsLayout {
  static constexpr bool kSwz = BK == 32;
  static constexpr int kPitch = kSwz ? BK : BK + 8;  // elements per row
  __device__ static __forceinline__ int off(int row, int k) {
    if constexpr (kSwz) {
      const int pr = row ^ ((row >> 3) & 3);
      return pr * 32 + ((((k >> 3) ^ (row >> 2)) & 3) << 3) + (k & 7);
    } else {
      return row * kPitch + k;
    }
  }
};

__device__ __forceinline__ uint32_t word_of(const uint4& v, int j) {
  return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}

// v[c] holds the 8 bf16 of source k row (k + c) at columns r..r+7. Writes LDS rows r..r+7, each
// the CH elements k..k+CH-1 (one 8-byte or 4-byte store per row).
template <int CH, typename Lay>
__device__ __forceinline__ void put_trans(uint16_t* dst, int r, int k, const uint4 (&v)[CH]) {
  static_assert(CH == 2 || CH == 4, "transposed store width");
#pragma unroll
  for (int q = 0; q < 8; q++) {
    const int j = q >> 1;
    uint32_t w[CH / 2];
#pragma unroll
    for (int p = 0; p < CH / 2; p++) {
      const uint32_t lo = word_of(v[2 * p], j), hi = word_of(v[2 * p + 1], j);
      // column r+q of rows k+2p (low half) and k+2p+1 (high half)
      w[p] = (q & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
    uint16_t* p = &dst[Lay::off(r + q, k)];  // CH elements stay inside one 8-element chunk
    if constexpr (CH == 4) *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(p) = w[0];
  }
}

// Runs f(kt + i, set i % NS, LDS buffer i % 2) for i = 0..U-1 with compile-time set and buffer ids.
template <int NS, typename F, int... I>
__device__ __forceinline__ void unroll_steps(F& f, int kt, std::integer_sequence<int, I...>) {
  (f(kt + I, std::integral_constant<int, I % NS>{}, std::integral_constant<int, I % 2>{}), ...);
}

// Runs f(integral_constant<int, i>) for each i of the sequence.
template <typename F, int... I>
__device__ __forceinline__ void static_for(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

// Blocks are dispatched round-robin over the 8 XCDs (each with its own L2), so blocks whose linear
// ids differ by a multiple of 8 run on one XCD, whatever XCD a launch starts on. The tiles of one
// k-split all read the same k rows of the operands. With split_xcd each XCD takes a contiguous range
// of (split, tile) ids, so a split's tiles run on one XCD (two where a range boundary cuts the split)
// and its rows are fetched into one L2 instead of several. Only long splits (>= 2048 of k) are
// placed: where the tiles of a split read the same rows at once through one L2, short splits got
// slower (512x128x16384 at 32 splits: 17 -> 22 us). 512x128x262144 at 128 splits: 94 -> 82 us
// standalone, 103 -> 99 us inside the MinGRU step; 1536x512x262144 at 21 splits of 12 tiles: ~1 %
// inside the step.
__device__ __forceinline__ bool split_remap(const GemmArgs& g) { return g.split_xcd && gridDim.z > 1; }
// (k-split, tile id) of this block
__device__ __forceinline__ void block_split_tile(const GemmArgs& g, int& z, int& t) {
  z = blockIdx.z;
  t = blockIdx.x;
  if (split_remap(g)) {
    const int nt = gridDim.x, nb = nt * (int)gridDim.z;
    const int L = t + nt * z, x = L & 7;
    // XCD x holds ids [x * (nb / 8) + min(x, nb % 8), ...) in dispatch order
    const int v = x * (nb >> 3) + min(x, nb & 7) + (L >> 3);
    z = v / nt;
    t = v % nt;
  }
}
__device__ __forceinline__ int split_of(const GemmArgs& g) {
  int z, t;
  block_split_tile(g, z, t);
  return z;
}
// Thread-block tile id -> (tile_m, tile_n). With remap (and no split placement), the blocks that land
// on one XCD get a contiguous run of tiles sharing the same A rows.
__device__ inline void tile_coords(const GemmArgs& g, int tm, int tn, int& bm, int& bn) {
  int z, id;
  block_split_tile(g, z, id);
  const int total = tm * tn;
  if (g.remap && (total & 7) == 0 && !split_remap(g)) id = (id & 7) * (total >> 3) + (id >> 3);
  bm = id / tn;
  bn = id % tn;
}

template <typename TOut>
__device__ inline void store_out(TOut* p, float v);
template <>
__device__ inline void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ inline void store_out<uint16_t>(uint16_t* p, float v) { *p = bf16_rne(v); }

template <int EPI, typename TC>
__device__ __forceinline__ void epilogue_store_t(const GemmArgs& g, int row, int col, float acc) {
  if (row >= g.M || col >= g.N) return;
  float v = acc;
  if constexpr (EPI == PH_EPI_BIAS) v = acc + g.bias[col];
  if constexpr (EPI == PH_EPI_BIAS_RELU) v = fmaxf(acc + g.bias[col], 0.f);
  if constexpr (EPI == PH_EPI_RELU_MASK) {
    const float h = to_f32(reinterpret_cast<const TC*>(g.aux)[(long)row * g.ldaux + col]);
    v = h > 0.f ? acc : 0.f;
  }
  if constexpr (EPI == PH_EPI_AXPBY) {
    const float x = g.aux ? to_f32(reinterpret_cast<const TC*>(g.aux)[(long)row * g.ldaux + col]) : 0.f;
    v = g.alpha * acc + g.beta * x;
  }
  if constexpr (EPI == kEpiGateSkip) {
    const float dh = to_f32(reinterpret_cast<const TC*>(g.aux)[(long)row * g.ldaux + col]);
    const float p = to_f32(reinterpret_cast<const TC*>(g.aux2)[(long)row * g.ldaux2 + col]);
    v = acc + dh * (1.f - sigm(p));
  }
  store_out<TC>(reinterpret_cast<TC*>(g.C) + (long)row * g.ldc + col, v);
  if (g.C2) {
    const long o = g.c2_trans ? (long)col * g.ldc2 + row : (long)row * g.ldc2 + col;
    g.C2[o] = bf16_rne(v);
  }
}

template <typename TC>
__device__ __forceinline__ void epilogue_store(const GemmArgs& g, int row, int col, float acc) {
  switch (g.epi) {
    case PH_EPI_BIAS: epilogue_store_t<PH_EPI_BIAS, TC>(g, row, col, acc); break;
    case PH_EPI_BIAS_RELU: epilogue_store_t<PH_EPI_BIAS_RELU, TC>(g, row, col, acc); break;
    case PH_EPI_RELU_MASK: epilogue_store_t<PH_EPI_RELU_MASK, TC>(g, row, col, acc); break;
    case PH_EPI_AXPBY: epilogue_store_t<PH_EPI_AXPBY, TC>(g, row, col, acc); break;
    case kEpiGateSkip: epilogue_store_t<kEpiGateSkip, TC>(g, row, col, acc); break;
    default: epilogue_store_t<PH_EPI_NONE, TC>(g, row, col, acc); break;
  }
}

// Writes a wave's SM x SN block of 32x32 accumulators (or the split-K partial). The epilogue
// switch sits outside the element loops. Accumulator layout of a 32x32 MFMA: lane holds column
// (lane & 31); element r sits in row 8*(r/4) + 4*(lane/32) + (r%4).
template <int EPI, typename TC, int SM, int SN>
__device__ __forceinline__ void write_tile_t(const GemmArgs& g, const floatx16 (&acc)[SM][SN], int r0, int c0,
                                    int lane) {
  const int hrow = (lane >> 5) * 4, lr = lane & 31;
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = r0 + i * 32 + 8 * (r >> 2) + hrow + (r & 3);
        const int col = c0 + j * 32 + lr;
        if constexpr (EPI < 0) {
          if (row < g.M && col < g.N) g.ws[(long)row * g.N + col] = acc[i][j][r];
        } else {
          epilogue_store_t<EPI, TC>(g, row, col, acc[i][j][r]);
        }
      }
}

template <typename TC, int SM, int SN>
__device__ __forceinline__ void write_tile(const GemmArgs& g, const floatx16 (&acc)[SM][SN], int r0, int c0,
                                  int lane) {
  if (g.ws) { write_tile_t<-1, TC>(g, acc, r0, c0, lane); return; }
  switch (g.epi) {
    case PH_EPI_BIAS: write_tile_t<PH_EPI_BIAS, TC>(g, acc, r0, c0, lane); break;
    case PH_EPI_BIAS_RELU: write_tile_t<PH_EPI_BIAS_RELU, TC>(g, acc, r0, c0, lane); break;
    case PH_EPI_RELU_MASK: write_tile_t<PH_EPI_RELU_MASK, TC>(g, acc, r0, c0, lane); break;
    case PH_EPI_AXPBY: write_tile_t<PH_EPI_AXPBY, TC>(g, acc, r0, c0, lane); break;
    case kEpiGateSkip: write_tile_t<kEpiGateSkip, TC>(g, acc, r0, c0, lane); break;
    default: write_tile_t<PH_EPI_NONE, TC>(g, acc, r0, c0, lane); break;
  }
}

// LDS-staged epilogue. The block's fp32 accumulators are first written to an LDS tile
// [BM][BN+4]; the whole block then walks it in 4-column chunks, applies the epilogue with vector
// loads of bias/aux, and writes each chunk with one 16-byte (fp32) or 8-byte (bf16) store, so a
// wavefront's stores cover whole contiguous row segments.
template <int SM, int SN, int LDC>
__device__ __forceinline__ void stage_acc(float* sC, const floatx16 (&acc)[SM][SN], int wm0, int wn0,
                                          int lane) {
  const int hrow = (lane >> 5) * 4, lr = lane & 31;
#pragma unroll
  for (int i = 0; i < SM; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        sC[(wm0 + i * 32 + 8 * (r >> 2) + hrow + (r & 3)) * LDC + wn0 + j * 32 + lr] = acc[i][j][r];
}

// Sub-tiles i of a wave whose 32 rows (relative row wr0 + 32 i) fall inside [0, rows) of the
// current staging pass; the others belong to another pass.
template <int SM, int SN, int LDC>
__device__ __forceinline__ void stage_acc_rows(float* sC, const floatx16 (&acc)[SM][SN], int wr0, int wn0,
                                               int lane, int rows) {
  const int hrow = (lane >> 5) * 4, lr = lane & 31;
#pragma unroll
  for (int i = 0; i < SM; i++) {
    const int r0 = wr0 + i * 32;
    if (r0 < 0 || r0 >= rows) continue;
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        sC[(r0 + 8 * (r >> 2) + hrow + (r & 3)) * LDC + wn0 + j * 32 + lr] = acc[i][j][r];
  }
}

// Stages sub-tiles i in [I0, I0 + NI) of a wave's accumulators into rows r0 + 32 (i - I0) of sC.
template <int I0, int NI, int SM, int SN, int LDC>
__device__ __forceinline__ void stage_acc_part(float* sC, const floatx16 (&acc)[SM][SN], int r0, int wn0, int lane) {
  const int hrow = (lane >> 5) * 4, lr = lane & 31;
#pragma unroll
  for (int i = I0; i < I0 + NI; i++)
#pragma unroll
    for (int j = 0; j < SN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++)
        sC[(r0 + (i - I0) * 32 + 8 * (r >> 2) + hrow + (r & 3)) * LDC + wn0 + j * 32 + lr] = acc[i][j][r];
}

constexpr int epilogue_rows(int bm, int row_bytes, int budget) {
  int r = bm;
  while (r > 32 && (r * row_bytes > budget || bm % r != 0)) r -= 32;
  return r;
}

__device__ __forceinline__ float4 load4_f32(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4_f32(const uint16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return make_float4(bf16_to_f32(u.x & 0xffffu), bf16_to_f32(u.x >> 16), bf16_to_f32(u.y & 0xffffu),
                     bf16_to_f32(u.y >> 16));
}
__device__ __forceinline__ void store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
// bf16 results are written once and read by a later kernel, not by this one: nontemporal stores keep
// them from displacing the operand rows that other tiles of the launch still re-read from L2
// (measured: the MinGRU step 1.5 % faster, its layer-forward GEMM 4 %).
__device__ __forceinline__ void store4(uint16_t* p, float4 v) {
  __builtin_nontemporal_store(pack_bf16x2(v.x, v.y), reinterpret_cast<uint32_t*>(p));
  __builtin_nontemporal_store(pack_bf16x2(v.z, v.w), reinterpret_cast<uint32_t*>(p) + 1);
}

// 8 bf16 results as one 16-byte nontemporal store (half the store instructions of two store4 calls;
// measured: the 262144x1536x512 layer-forward GEMM 19 % faster, its 262144x512x1536 data-gradient 6 %).
__device__ __forceinline__ void store8(uint16_t* p, float4 a, float4 b) {
  const u32x4_t w = {pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y), pack_bf16x2(b.z, b.w)};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}

// The epilogue operands of one 4-column chunk, as loaded (bf16 operands stay packed until used).
// The flush issues them ahead of the arithmetic and stores (the 8-column path all of a pass's chunks,
// the 4-column path a group of four), so the loads are in flight together instead of costing one load
// latency per chunk (measured: the 262144x512x1536 GEMM with an aux operand 561 -> 534 us, against 497
// without one). C may alias aux, as in the in-place AXPBY: each element's operand is still read
// before that element is written, and the loads touch only the elements of the pass or group.
template <typename TC> struct EpiRaw4;
template <> struct EpiRaw4<uint16_t> { uint2 v; };
template <> struct EpiRaw4<float> { float4 v; };
__device__ __forceinline__ EpiRaw4<uint16_t> ld_raw4(const uint16_t* p) {
  return {*reinterpret_cast<const uint2*>(p)};
}
__device__ __forceinline__ EpiRaw4<float> ld_raw4(const float* p) {
  return {*reinterpret_cast<const float4*>(p)};
}
__device__ __forceinline__ float4 cvt4(const EpiRaw4<uint16_t>& r) {
  return make_float4(bf16_to_f32(r.v.x & 0xffffu), bf16_to_f32(r.v.x >> 16), bf16_to_f32(r.v.y & 0xffffu),
                     bf16_to_f32(r.v.y >> 16));
}
__device__ __forceinline__ float4 cvt4(const EpiRaw4<float>& r) { return r.v; }
template <typename TC>
struct EpiOps {
  float4 bias;
  EpiRaw4<TC> x, y;  // aux (mask, AXPBY term, gate-skip gradient) and aux2 (gate-skip pre-activation)
};

template <int EPI, typename TC>
__device__ __forceinline__ EpiOps<TC> epi_load4(const GemmArgs& g, int row, int col) {
  EpiOps<TC> o{};
  if constexpr (EPI == PH_EPI_BIAS || EPI == PH_EPI_BIAS_RELU) o.bias = load4_f32(g.bias + col);
  if constexpr (EPI == PH_EPI_RELU_MASK || EPI == kEpiGateSkip)
    o.x = ld_raw4(reinterpret_cast<const TC*>(g.aux) + (long)row * g.ldaux + col);
  if constexpr (EPI == PH_EPI_AXPBY) {
    if (g.aux) o.x = ld_raw4(reinterpret_cast<const TC*>(g.aux) + (long)row * g.ldaux + col);
  }
  if constexpr (EPI == kEpiGateSkip)
    o.y = ld_raw4(reinterpret_cast<const TC*>(g.aux2) + (long)row * g.ldaux2 + col);
  return o;
}

template <int EPI, typename TC>
__device__ __forceinline__ float4 epi_apply4(const GemmArgs& g, float4 v, const EpiOps<TC>& o) {
  if constexpr (EPI == PH_EPI_BIAS || EPI == PH_EPI_BIAS_RELU) {
    const float4 b = o.bias;
    v.x += b.x; v.y += b.y; v.z += b.z; v.w += b.w;
    if constexpr (EPI == PH_EPI_BIAS_RELU) {
      v.x = fmaxf(v.x, 0.f); v.y = fmaxf(v.y, 0.f); v.z = fmaxf(v.z, 0.f); v.w = fmaxf(v.w, 0.f);
    }
  }
  if constexpr (EPI == PH_EPI_RELU_MASK) {
    const float4 h = cvt4(o.x);
    v.x = h.x > 0.f ? v.x : 0.f; v.y = h.y > 0.f ? v.y : 0.f;
    v.z = h.z > 0.f ? v.z : 0.f; v.w = h.w > 0.f ? v.w : 0.f;
  }
  if constexpr (EPI == PH_EPI_AXPBY) {
    const float4 x = g.aux ? cvt4(o.x) : make_float4(0.f, 0.f, 0.f, 0.f);
    v.x = g.alpha * v.x + g.beta * x.x; v.y = g.alpha * v.y + g.beta * x.y;
    v.z = g.alpha * v.z + g.beta * x.z; v.w = g.alpha * v.w + g.beta * x.w;
  }
  if constexpr (EPI == kEpiGateSkip) {
    const float4 dh = cvt4(o.x), p = cvt4(o.y);
    v.x += dh.x * (1.f - sigm(p.x)); v.y += dh.y * (1.f - sigm(p.y));
    v.z += dh.z * (1.f - sigm(p.z)); v.w += dh.w * (1.f - sigm(p.w));
  }
  return v;
}

// Whether a BM x BN tile splits evenly into 8-column chunks over NT threads.
template <int BM, int BN, int NT>
constexpr bool kChunk8 = (BN % 8 == 0) && ((BM * (BN / 8)) % NT == 0);

// vec: 0 element stores, 4 four-column chunks, 8 eight-column chunks (bf16 C only). Staged rows
// [0, BM/2) are C rows m0.., rows [BM/2, BM) are C rows mhi.. (mhi = m0 + BM/2 for a contiguous tile).
// NT threads (tid = 0..NT-1) share the tile; WAVE: they are one wavefront flushing its own staging
// area, so LDS ordering needs no block barrier (a wave's LDS operations complete in issue order).
template <int EPI, typename TC, int BM, int BN, int NT, int LDC, bool WAVE = false>
__device__ __forceinline__ void flush_tile_t(const GemmArgs& g, float* sC, int m0, int mhi, int n0, int vec,
                                             int tid) {
  static_assert(!WAVE || NT == 64, "a wave-local flush runs on one wavefront");
  auto grow = [&](int lr) { return lr < BM / 2 ? m0 + lr : mhi + (lr - BM / 2); };
  constexpr int CPR = BN / 4;               // 4-column chunks per row
  constexpr int NCH = BM * CPR / NT;        // chunks per thread
  static_assert(NCH * NT == BM * CPR, "C tile / threads");
  constexpr bool kHas8 = EPI >= 0 && sizeof(TC) == 2 && kChunk8<BM, BN, NT>;
  if constexpr (!kHas8) {
    if (vec == 8) vec = 4;
  }
  if constexpr (kHas8) {
    if (vec == 8) {
      // G chunks in flight at a time: the LDS reads of a group are issued together (one wait), and
      // the group stays small enough that the registers of accumulators not yet staged are not spilled
      constexpr int CPR8 = BN / 8, NCH8 = BM * CPR8 / NT, G = NCH8 < 4 ? NCH8 : 4;
      static_assert(NCH8 % G == 0, "chunk groups");
      // The pass's aux operands first: one 16-byte load per chunk and operand, all in flight together
      // (one load latency per pass instead of one per group). They become their epilogue terms
      // before the first store: one counter covers both loads and stores here, so a wait for a load
      // issued before a store would also wait for that store, a store round trip before every chunk
      // (measured: the 262144x512x1536 GEMM with an aux operand 549 -> 544 us, 508 without one).
      constexpr bool kX = EPI == PH_EPI_RELU_MASK || EPI == PH_EPI_AXPBY || EPI == kEpiGateSkip;
      constexpr bool kY = EPI == kEpiGateSkip;
      constexpr bool kAdd = EPI == PH_EPI_AXPBY || EPI == kEpiGateSkip;
      constexpr bool kMask = EPI == PH_EPI_RELU_MASK;
      float4 ad[kAdd ? NCH8 : 1][2];  // AXPBY: beta * aux; gate skip: aux * (1 - sigm(aux2))
      uint32_t mk[kMask ? NCH8 : 1];  // RELU_MASK: bit e set where aux > 0
      if constexpr (kX) {
        uint4 xa[NCH8], xb[kY ? NCH8 : 1];
        const bool has = EPI != PH_EPI_AXPBY || g.aux;
#pragma unroll
        for (int q = 0; q < NCH8; q++) {
          const int c = tid + q * NT;
          const int row = grow(c / CPR8), col = n0 + (c % CPR8) * 8;
          const bool in = has && row < g.M && col < g.N;
          const uint16_t* pa = reinterpret_cast<const uint16_t*>(g.aux) + (long)row * g.ldaux + col;
          xa[q] = in ? *reinterpret_cast<const uint4*>(pa) : make_uint4(0u, 0u, 0u, 0u);
          if constexpr (kY) {
            const uint16_t* pb = reinterpret_cast<const uint16_t*>(g.aux2) + (long)row * g.ldaux2 + col;
            xb[q] = in ? *reinterpret_cast<const uint4*>(pb) : make_uint4(0u, 0u, 0u, 0u);
          }
        }
        // Wait for them here, before any store of the pass (the compiler would otherwise sink the
        // terms, and its waits, to the chunks' stores): s_waitcnt vmcnt(0), other counters unchanged.
        __builtin_amdgcn_s_waitcnt(0x0F70);
#pragma unroll
        for (int q = 0; q < NCH8; q++) {
          const float4 x[2] = {cvt4(EpiRaw4<uint16_t>{make_uint2(xa[q].x, xa[q].y)}),
                               cvt4(EpiRaw4<uint16_t>{make_uint2(xa[q].z, xa[q].w)})};
          if constexpr (kMask) {
            uint32_t m = 0u;
#pragma unroll
            for (int h = 0; h < 2; h++)
              m |= (x[h].x > 0.f ? 1u : 0u) << (4 * h) | (x[h].y > 0.f ? 2u : 0u) << (4 * h) |
                   (x[h].z > 0.f ? 4u : 0u) << (4 * h) | (x[h].w > 0.f ? 8u : 0u) << (4 * h);
            mk[q] = m;
          }
          if constexpr (EPI == PH_EPI_AXPBY) {
#pragma unroll
            for (int h = 0; h < 2; h++)
              ad[q][h] = make_float4(g.beta * x[h].x, g.beta * x[h].y, g.beta * x[h].z, g.beta * x[h].w);
          }
          if constexpr (kY) {
            const float4 pp[2] = {cvt4(EpiRaw4<uint16_t>{make_uint2(xb[q].x, xb[q].y)}),
                                  cvt4(EpiRaw4<uint16_t>{make_uint2(xb[q].z, xb[q].w)})};
#pragma unroll
            for (int h = 0; h < 2; h++)
              ad[q][h] = make_float4(x[h].x * (1.f - sigm(pp[h].x)), x[h].y * (1.f - sigm(pp[h].y)),
                                     x[h].z * (1.f - sigm(pp[h].z)), x[h].w * (1.f - sigm(pp[h].w)));
          }
        }
      }
      // The bias: when NT is a multiple of the chunks per row, all of a thread's chunks share one
      // column, so its 8 bias values are loaded once.
      constexpr bool kB = EPI == PH_EPI_BIAS || EPI == PH_EPI_BIAS_RELU;
      constexpr bool kB1 = kB && NT % CPR8 == 0;
      float4 bias1[2] = {};
      if constexpr (kB1) {
        const int col = n0 + (tid % CPR8) * 8;
        if (col < g.N) {
          bias1[0] = load4_f32(g.bias + col);
          bias1[1] = load4_f32(g.bias + col + 4);
        }
      }
#pragma unroll
      for (int q0 = 0; q0 < NCH8; q0 += G) {
        float4 v[G][2];
        EpiOps<TC> op[G][2];
#pragma unroll
        for (int q = 0; q < G; q++) {
          const int c = tid + (q0 + q) * NT;
          const int lr = c / CPR8, lc = (c % CPR8) * 8;
          const int row = grow(lr), col = n0 + lc;
          if constexpr (kB1) {
            op[q][0].bias = bias1[0];
            op[q][1].bias = bias1[1];
          } else if constexpr (kB) {
            if (row < g.M && col < g.N) {
              op[q][0] = epi_load4<EPI, TC>(g, row, col);
              op[q][1] = epi_load4<EPI, TC>(g, row, col + 4);
            }
          }
          const float* src = &sC[lr * LDC + lc];
          v[q][0] = *reinterpret_cast<const float4*>(src);
          v[q][1] = *reinterpret_cast<const float4*>(src + 4);
        }
#pragma unroll
        for (int q = 0; q < G; q++) {
          const int c = tid + (q0 + q) * NT;
          const int lr = c / CPR8, lc = (c % CPR8) * 8;
          const int row = grow(lr), col = n0 + lc;
          if (row >= g.M || col >= g.N) continue;
          float4 a, b;
          if constexpr (kAdd) {
            // AXPBY: alpha * acc + beta * aux; gate skip: acc + its term
            const float al = EPI == PH_EPI_AXPBY ? g.alpha : 1.f;
            const float4 u = v[q][0], w = v[q][1], t0 = ad[q0 + q][0], t1 = ad[q0 + q][1];
            a = make_float4(al * u.x + t0.x, al * u.y + t0.y, al * u.z + t0.z, al * u.w + t0.w);
            b = make_float4(al * w.x + t1.x, al * w.y + t1.y, al * w.z + t1.z, al * w.w + t1.w);
          } else if constexpr (kMask) {
            const uint32_t m = mk[q0 + q];
            const float4 u = v[q][0], w = v[q][1];
            a = make_float4(m & 1u ? u.x : 0.f, m & 2u ? u.y : 0.f, m & 4u ? u.z : 0.f, m & 8u ? u.w : 0.f);
            b = make_float4(m & 16u ? w.x : 0.f, m & 32u ? w.y : 0.f, m & 64u ? w.z : 0.f, m & 128u ? w.w : 0.f);
          } else {
            a = epi_apply4<EPI, TC>(g, v[q][0], op[q][0]);
            b = epi_apply4<EPI, TC>(g, v[q][1], op[q][1]);
          }
          store8(reinterpret_cast<uint16_t*>(g.C) + (long)row * g.ldc + col, a, b);
          if (g.C2 && !g.c2_trans) store8(g.C2 + (long)row * g.ldc2 + col, a, b);
          if (g.C2 && g.c2_trans) {
            *reinterpret_cast<float4*>(&sC[lr * LDC + lc]) = a;
            *reinterpret_cast<float4*>(&sC[lr * LDC + lc + 4]) = b;
          }
        }
      }
    }
  }
  if (vec == 4) {
    // all LDS reads first (one wait), then one vector store per chunk; the epilogue operands of a
    // group of G4 chunks are loaded before the group's stores
    constexpr int G4 = NCH < 4 ? NCH : 4;
    static_assert(NCH % G4 == 0, "chunk groups");
    float4 v[NCH];
#pragma unroll
    for (int q = 0; q < NCH; q++) {
      const int c = tid + q * NT;
      v[q] = *reinterpret_cast<const float4*>(&sC[(c / CPR) * LDC + (c % CPR) * 4]);
    }
    // bias: one load per thread when all of its chunks share a column (NT a multiple of CPR)
    constexpr bool kB1 = (EPI == PH_EPI_BIAS || EPI == PH_EPI_BIAS_RELU) && NT % CPR == 0;
    float4 bias1 = {};
    if constexpr (kB1) {
      const int col = n0 + (tid % CPR) * 4;
      if (col < g.N) bias1 = load4_f32(g.bias + col);
    }
#pragma unroll
    for (int q0 = 0; q0 < NCH; q0 += G4) {
      EpiOps<TC> op[G4];
      if constexpr (kB1) {
#pragma unroll
        for (int u = 0; u < G4; u++) op[u].bias = bias1;
      } else if constexpr (EPI >= 0) {
#pragma unroll
        for (int u = 0; u < G4; u++) {
          const int c = tid + (q0 + u) * NT;
          const int row = grow(c / CPR), col = n0 + (c % CPR) * 4;
          if (row < g.M && col < g.N) op[u] = epi_load4<EPI, TC>(g, row, col);
        }
      }
#pragma unroll
      for (int u = 0; u < G4; u++) {
        const int q = q0 + u;
        const int c = tid + q * NT;
        const int lr = c / CPR, lc = (c % CPR) * 4;
        const int row = grow(lr), col = n0 + lc;
        if (row >= g.M || col >= g.N) continue;
        if constexpr (EPI < 0) {
          store4(g.ws + (long)row * g.N + col, v[q]);
        } else {
          const float4 w = epi_apply4<EPI, TC>(g, v[q], op[u]);
          store4(reinterpret_cast<TC*>(g.C) + (long)row * g.ldc + col, w);
          if (g.C2 && !g.c2_trans) store4(g.C2 + (long)row * g.ldc2 + col, w);
          if (g.C2 && g.c2_trans) *reinterpret_cast<float4*>(&sC[lr * LDC + lc]) = w;
        }
      }
    }
  } else if (vec == 0) {
    // unaligned or ragged shapes: element stores
#pragma unroll 1
    for (int c = tid; c < BM * BN; c += NT) {
      const int lr = c / BN, lc = c % BN;
      const int row = grow(lr), col = n0 + lc;
      if (row >= g.M || col >= g.N) continue;
      const float e = sC[lr * LDC + lc];
      if constexpr (EPI < 0) g.ws[(long)row * g.N + col] = e;
      else epilogue_store_t<EPI, TC>(g, row, col, e);
    }
  }
  if constexpr (EPI >= 0) {
    if (vec != 0 && g.C2 && g.c2_trans) {
      // transposed bf16 copy: chunks of 4 consecutive rows of one column -> one 8-byte store
      if constexpr (WAVE) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      else lds_barrier();
      constexpr int CPC = BM / 4;
      for (int c = tid; c < BN * CPC; c += NT) {
        const int lc = c / CPC, lr = (c % CPC) * 4;  // 4 rows inside one half (BM/2 % 4 == 0)
        const int row = grow(lr), col = n0 + lc;
        if (row >= g.M || col >= g.N) continue;
        const float4 v = make_float4(sC[lr * LDC + lc], sC[(lr + 1) * LDC + lc],
                                     sC[(lr + 2) * LDC + lc], sC[(lr + 3) * LDC + lc]);
        store4(g.C2 + (long)col * g.ldc2 + row, v);
      }
    }
  }
}

// Chunk width of the flush: 8 (bf16 C, 8-column chunks), 4 (4-column chunks) or 0 (element stores).
template <typename TC>
__host__ __device__ __forceinline__ int flush_vec(const GemmArgs& g) {
  // vector path: every 4-column chunk is whole and 16-byte (fp32) / 8-byte (bf16) aligned
  const bool vec4 = (g.N % 4 == 0) && (g.ws ? true : (g.ldc % 4 == 0 && ((uintptr_t)g.C % 16) == 0)) &&
                    (!g.aux || (g.ldaux % 4 == 0 && ((uintptr_t)g.aux % 16) == 0)) &&
                    (!g.aux2 || (g.ldaux2 % 4 == 0 && ((uintptr_t)g.aux2 % 16) == 0)) &&
                    (!g.C2 || ((g.c2_trans ? g.M % 4 : g.ldc2 % 4) == 0 && ((uintptr_t)g.C2 % 8) == 0 &&
                               (g.c2_trans ? g.ldc2 % 4 == 0 : true))) &&
                    (!g.bias || ((uintptr_t)g.bias % 16) == 0);
  // 8-column chunks (bf16 C): every chunk whole and its 16-byte C (and row-major C2) store aligned
  const bool vec8 = vec4 && !g.ws && sizeof(TC) == 2 && g.N % 8 == 0 && g.ldc % 8 == 0 &&
                    (!g.aux || g.ldaux % 8 == 0) && (!g.aux2 || g.ldaux2 % 8 == 0) &&
                    (!g.C2 || g.c2_trans || (g.ldc2 % 8 == 0 && ((uintptr_t)g.C2 % 16) == 0));
  return vec8 ? 8 : (vec4 ? 4 : 0);
}

template <typename TC, int BM, int BN, int NT, int LDC, bool WAVE = false>
__device__ __forceinline__ void flush_tile(const GemmArgs& g, float* sC, int m0, int n0, int mhi = -1,
                                           int tid = -1) {
  static_assert(BM % 8 == 0, "two halves of whole 4-row chunks");
  if (mhi < 0) mhi = m0 + BM / 2;
  if (tid < 0) tid = threadIdx.x;
  const int vec = flush_vec<TC>(g);
  if (g.ws) { flush_tile_t<-1, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); return; }
  switch (g.epi) {
    case PH_EPI_BIAS: flush_tile_t<PH_EPI_BIAS, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
    case PH_EPI_BIAS_RELU: flush_tile_t<PH_EPI_BIAS_RELU, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
    case PH_EPI_RELU_MASK: flush_tile_t<PH_EPI_RELU_MASK, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
    case PH_EPI_AXPBY: flush_tile_t<PH_EPI_AXPBY, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
    case kEpiGateSkip: flush_tile_t<kEpiGateSkip, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
    default: flush_tile_t<PH_EPI_NONE, TC, BM, BN, NT, LDC, WAVE>(g, sC, m0, mhi, n0, vec, tid); break;
  }
}

// bf16 C with no aux operand (EPI NONE / BIAS / BIAS_RELU, no second output, no split-K partials, the
// 8-column path): the accumulators are rounded to bf16 in registers (bias and ReLU applied first, the
// same arithmetic as the fp32-staged flush) and the whole BM x BN tile is staged once, as bf16: half
// the LDS bytes of the fp32 staging passes, which share the LDS with the other block's k loop.
// Adjacent lanes hold adjacent columns: for each pair of rows they swap one value (DPP), so each lane
// writes two columns of one row as one 4-byte store. Rows are 2 BN bytes with no padding; the 16-byte
// chunks are XOR-swizzled by row (sbf_word) so the four rows one store instruction writes use
// different banks.
__host__ __device__ __forceinline__ bool stage_bf16_ok(const GemmArgs& g, int vec) {
  return g.c_bf16 && !g.ws && !g.C2 && vec == 8 &&
         (g.epi == PH_EPI_NONE || g.epi == PH_EPI_BIAS || g.epi == PH_EPI_BIAS_RELU);
}
// One staging store instruction writes rows R, R + 1 (half-wavefront 0) and R + 4, R + 5 (half 1),
// 32 columns (4 chunks) each; the 64 LDS banks see each row's chunks at a different 16-bank offset.
// 16 chunks per row (BN 128, rows 64 words): chunk ^ 4 (row bit 0) ^ 8 (row bit 2). 8 chunks per row
// (rows 32 words, so odd rows already sit 32 banks on): chunk ^ 4 when row bits 0 and 2 differ.
__device__ __forceinline__ int sbf_word(int row, int col, int BN) {
  const int sw = BN >= 128 ? ((row & 1) << 2) | (((row >> 2) & 1) << 3) : (((row ^ (row >> 2)) & 1) << 2);
  const int ch = (col >> 3) ^ sw;
  return row * (BN / 2) + ch * 4 + ((col & 7) >> 1);
}
template <int EPI, int BN, int SM, int SN>
__device__ __forceinline__ void stage_bf16(const GemmArgs& g, uint32_t* sT, const floatx16 (&acc)[SM][SN],
                                           int wm0, int wn0, int n0, int lane) {
  const bool odd = lane & 1;
  const int hrow = (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < SN; j++) {
    const int c = wn0 + j * 32 + (lane & 31);
    float bj = 0.f;
    if constexpr (EPI != PH_EPI_NONE) bj = n0 + c < g.N ? g.bias[n0 + c] : 0.f;
    const int ce = c & ~1;
#pragma unroll
    for (int i = 0; i < SM; i++)
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const int r0 = 2 * k, r1 = r0 + 1;
        float v0 = acc[i][j][r0], v1 = acc[i][j][r1];
        if constexpr (EPI != PH_EPI_NONE) {
          v0 += bj;
          v1 += bj;
        }
        if constexpr (EPI == PH_EPI_BIAS_RELU) {
          v0 = fmaxf(v0, 0.f);
          v1 = fmaxf(v1, 0.f);
        }
        // even lane: (own r0, odd neighbour's r0) at row r0; odd lane: (even neighbour's r1, own r1) at row r1
        const float x = odd ? v0 : v1;
        const int xi = __builtin_bit_cast(int, x);
        // the value of lane ^ 1 (DPP quad permutation 1, 0, 3, 2)
        const float y = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(xi, 0xB1, 0xF, 0xF, false));
        const uint32_t w = odd ? pack_bf16x2(y, v1) : pack_bf16x2(v0, y);
        const int row = wm0 + i * 32 + 8 * (r0 >> 2) + hrow + (r0 & 3) + (odd ? 1 : 0);
        sT[sbf_word(row, ce, BN)] = w;
      }
  }
}
// Writes the staged bf16 tile: one 16-byte LDS read and one 16-byte nontemporal store per chunk.
template <int BM, int BN, int NT>
__device__ __forceinline__ void flush_bf16(const GemmArgs& g, const uint32_t* sT, int m0, int n0, int tid) {
  constexpr int CPR = BN / 8, NCH = BM * CPR / NT, G = 8;
  static_assert(NCH * NT == BM * CPR && NCH % G == 0, "bf16 flush chunks");
#pragma unroll
  for (int q0 = 0; q0 < NCH; q0 += G) {
    u32x4_t v[G];
#pragma unroll
    for (int q = 0; q < G; q++) {
      const int c = tid + (q0 + q) * NT, row = c / CPR, ch = c % CPR;
      v[q] = *reinterpret_cast<const u32x4_t*>(&sT[sbf_word(row, ch * 8, BN)]);
    }
#pragma unroll
    for (int q = 0; q < G; q++) {
      const int c = tid + (q0 + q) * NT, row = m0 + c / CPR, col = n0 + (c % CPR) * 8;
      if (row < g.M && col < g.N) {
        uint16_t* dst = reinterpret_cast<uint16_t*>(g.C) + (long)row * g.ldc + col;
        __builtin_nontemporal_store(v[q], reinterpret_cast<u32x4_t*>(dst));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// bf16-math kernel. WGM x WGN wavefronts; prefetch distance 2: while k-tile kt is multiplied out of
// LDS, tile kt+1 sits in registers and tile kt+2 is in flight from memory. The two register sets
// alternate, so the k loop is unrolled by two to keep every register index static.
template <int BM, int BN, int BK, int WGM, int WGN, bool TA, bool TB, typename TIA, typename TIB,
          typename TC, bool X3 = false>
__global__ void __launch_bounds__(WGM * WGN * 64) k_gemm_bf16(GemmArgs g) {
  // X3: fp32 operands split as x = hi + lo (both bf16); acc += hi*hi + hi*lo + lo*hi
  static_assert(!X3 || (sizeof(TIA) == 4 && sizeof(TIB) == 4), "split-bf16 needs fp32 operands");
  constexpr int NSPLIT = X3 ? 2 : 1;
  constexpr int NT = WGM * WGN * 64;
  using Lay = LdsLayout<BK>;
  constexpr int LDK = Lay::kPitch;          // LDS row pitch in bf16 elements
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int SM = WM / 32, SN = WN / 32; // 32x32 sub-tiles per wave
  constexpr int CA = BM * BK / 8 / NT;      // 8-element chunks per thread (A)
  constexpr int CB = BN * BK / 8 / NT;
  static_assert(CA >= 1 && CB >= 1 && CA * NT * 8 == BM * BK && CB * NT * 8 == BN * BK, "tile/threads");
  static_assert(BK % 32 == 0 && SM >= 1 && SN >= 1, "tile shape");

  constexpr int LDC = BN + 4;  // fp32 C staging pitch
  constexpr int PIPE_BYTES = 2 * NSPLIT * (BM + BN) * LDK * 2;
  // The C tile is staged through the pipeline's LDS in passes of EPR rows (all BM rows at once
  // when they fit, else the largest multiple of 32 rows dividing BM that fits).
  constexpr int EPR = epilogue_rows(BM, LDC * 4, PIPE_BYTES);
  static_assert(EPR >= 32 && BM % EPR == 0, "epilogue staging rows");
  constexpr int C_BYTES = EPR * LDC * 4;
  static_assert((PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES) <= kMaxLdsBytes, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t smem[PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES];
  uint16_t (*sA)[BM * LDK] = reinterpret_cast<uint16_t (*)[BM * LDK]>(smem);
  uint16_t (*sB)[BN * LDK] = reinterpret_cast<uint16_t (*)[BN * LDK]>(smem + 2 * BM * LDK * 2);
  // low halves of the split operands (X3 only)
  uint16_t (*sAl)[BM * LDK] = reinterpret_cast<uint16_t (*)[BM * LDK]>(smem + 2 * (BM + BN) * LDK * 2);
  uint16_t (*sBl)[BN * LDK] =
      reinterpret_cast<uint16_t (*)[BN * LDK]>(smem + 2 * (BM + BN) * LDK * 2 + 2 * BM * LDK * 2);
  float* sC = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(g, tm, tn, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int zs = split_of(g);
  const int kbeg = zs * g.kps;
  if (g.ws) g.ws += (long)zs * g.M * g.N;  // this split's partials
  const int kend = min(g.K, kbeg + g.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const gptr<TIA> A = (gptr<TIA>)g.A;
  const gptr<TIB> B = (gptr<TIB>)g.B;

  // Prefetch depth: NSETS register sets of k-tiles in flight. Two measured best on the policy shapes
  // (a depth of four made the 256x128 forward 37 % slower: the longer unrolled body costs more than
  // the added latency cover; three or four made the split-K weight gradients 512x128x262144 and
  // 32x512x262144 at 128x128 tiles 4-14 % slower).
  constexpr int NSETS = 2;
  Raw8<TIA> ra[NSETS][CA];
  Raw8<TIB> rb[NSETS][CB];

  // Global -> register set for the k-tile starting at k0. Every load is issued unconditionally (an
  // out-of-range chunk reads the zero page), so no branch separates the loads and the compiler can
  // wait for exactly the set it needs.
  // Per-chunk source offsets split into a per-thread part fixed for the whole k loop and the
  // uniform k0-dependent part (k0 or k0*ld, a scalar), so a k step adds one scalar per chunk.
  long offA[CA], offB[CB];
  int kA[CA], kB[CB];
  uint32_t rowA = 0u, rowB = 0u;  // bit c: chunk c's row is inside the matrix
#pragma unroll
  for (int c = 0; c < CA; c++) {
    int r, k;
    chunk_rk<TA, BM, BK, CA, NT>(tid, c, r, k);
    const int gm = m0 + r;
    offA[c] = !TA ? (long)gm * g.lda + k : (long)k * g.lda + gm;
    kA[c] = k;
    rowA |= (gm < g.M ? 1u : 0u) << c;
  }
#pragma unroll
  for (int c = 0; c < CB; c++) {
    int r, k;
    chunk_rk<!TB, BN, BK, CB, NT>(tid, c, r, k);
    const int gn = n0 + r;
    offB[c] = TB ? (long)gn * g.ldb + k : (long)k * g.ldb + gn;
    kB[c] = k;
    rowB |= (gn < g.N ? 1u : 0u) << c;
  }
  auto gload = [&](Raw8<TIA> (&xa)[CA], Raw8<TIB> (&xb)[CB], int k0) {
    const long da = !TA ? (long)k0 : (long)k0 * g.lda;
    const long db = TB ? (long)k0 : (long)k0 * g.ldb;
#pragma unroll
    for (int c = 0; c < CA; c++) {
      const bool ok = ((rowA >> c) & 1u) && k0 + kA[c] < kend;
      xa[c] = load_raw8(ok ? A + (offA[c] + da) : zero_page<TIA>());
    }
#pragma unroll
    for (int c = 0; c < CB; c++) {
      const bool ok = ((rowB >> c) & 1u) && k0 + kB[c] < kend;
      xb[c] = load_raw8(ok ? B + (offB[c] + db) : zero_page<TIB>());
    }
  };
  // Register set -> LDS buffer `s` (transposing m/n-contiguous chunks).
  auto put = [&](uint16_t* dst, int r, int k, uint4 v, bool trans) {
    if (!trans) {
      *reinterpret_cast<uint4*>(&dst[Lay::off(r, k)]) = v;
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        dst[Lay::off(r + 2 * q, k)] = (uint16_t)(w[q] & 0xffffu);
        dst[Lay::off(r + 2 * q + 1, k)] = (uint16_t)(w[q] >> 16);
      }
    }
  };
  // One operand's register set -> LDS (hi part, and the lo part of the split for X3).
  auto sstore_op = [&](auto trans_c, auto rows_c, const auto& x, uint16_t* dst, uint16_t* dstl) {
    constexpr bool TR = decltype(trans_c)::value;
    constexpr int R = decltype(rows_c)::value;
    constexpr int CH = sizeof(x) / sizeof(x[0]);
    if constexpr (TR && CH >= 2) {
      uint4 v[CH], l[CH];
#pragma unroll
      for (int c = 0; c < CH; c++) {
        v[c] = to_bf16x8(x[c]);
        if constexpr (X3) l[c] = lo_bf16x8(x[c], v[c]);
      }
      int r, k;
      chunk_rk<TR, R, BK, CH, NT>(tid, 0, r, k);
      put_trans<CH, Lay>(dst, r, k, v);
      if constexpr (X3) put_trans<CH, Lay>(dstl, r, k, l);
    } else {
#pragma unroll
      for (int c = 0; c < CH; c++) {
        int r, k;
        chunk_rk<TR, R, BK, CH, NT>(tid, c, r, k);
        const uint4 v = to_bf16x8(x[c]);
        put(dst, r, k, v, TR);
        if constexpr (X3) put(dstl, r, k, lo_bf16x8(x[c], v), TR);
      }
    }
  };
  auto sstore = [&](const Raw8<TIA> (&xa)[CA], const Raw8<TIB> (&xb)[CB], int s) {
    sstore_op(std::integral_constant<bool, TA>{}, std::integral_constant<int, BM>{}, xa, sA[s], sAl[s]);
    sstore_op(std::integral_constant<bool, !TB>{}, std::integral_constant<int, BN>{}, xb, sB[s], sBl[s]);
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

  auto mfma = [&](floatx16& c, const uint4& a, const uint4& b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  };
  auto compute = [&](int s) {
#pragma unroll
    for (int kb = 0; kb < BK; kb += 32) {
      uint4 a0[SM], a1[SM], b0[SN], b1[SN];
#pragma unroll
      for (int i = 0; i < SM; i++) {
        const int row = wm0 + i * 32 + lr;
        a0[i] = *reinterpret_cast<const uint4*>(&sA[s][Lay::off(row, kb + lk)]);
        a1[i] = *reinterpret_cast<const uint4*>(&sA[s][Lay::off(row, kb + lk + 8)]);
      }
#pragma unroll
      for (int j = 0; j < SN; j++) {
        const int row = wn0 + j * 32 + lr;
        b0[j] = *reinterpret_cast<const uint4*>(&sB[s][Lay::off(row, kb + lk)]);
        b1[j] = *reinterpret_cast<const uint4*>(&sB[s][Lay::off(row, kb + lk + 8)]);
      }
      // all accumulators once with the first k half, then once with the second: consecutive
      // MFMAs never depend on each other
#pragma unroll
      for (int i = 0; i < SM; i++)
#pragma unroll
        for (int j = 0; j < SN; j++) mfma(acc[i][j], a0[i], b0[j]);
#pragma unroll
      for (int i = 0; i < SM; i++)
#pragma unroll
        for (int j = 0; j < SN; j++) mfma(acc[i][j], a1[i], b1[j]);
      if constexpr (X3) {
        uint4 l0[SM > SN ? SM : SN], l1[SM > SN ? SM : SN];
        // hi(A) * lo(B)
#pragma unroll
        for (int j = 0; j < SN; j++) {
          const int row = wn0 + j * 32 + lr;
          l0[j] = *reinterpret_cast<const uint4*>(&sBl[s][Lay::off(row, kb + lk)]);
          l1[j] = *reinterpret_cast<const uint4*>(&sBl[s][Lay::off(row, kb + lk + 8)]);
        }
#pragma unroll
        for (int i = 0; i < SM; i++)
#pragma unroll
          for (int j = 0; j < SN; j++) { mfma(acc[i][j], a0[i], l0[j]); }
#pragma unroll
        for (int i = 0; i < SM; i++)
#pragma unroll
          for (int j = 0; j < SN; j++) { mfma(acc[i][j], a1[i], l1[j]); }
        // lo(A) * hi(B)
#pragma unroll
        for (int i = 0; i < SM; i++) {
          const int row = wm0 + i * 32 + lr;
          l0[i] = *reinterpret_cast<const uint4*>(&sAl[s][Lay::off(row, kb + lk)]);
          l1[i] = *reinterpret_cast<const uint4*>(&sAl[s][Lay::off(row, kb + lk + 8)]);
        }
#pragma unroll
        for (int i = 0; i < SM; i++)
#pragma unroll
          for (int j = 0; j < SN; j++) { mfma(acc[i][j], l0[i], b0[j]); }
#pragma unroll
        for (int i = 0; i < SM; i++)
#pragma unroll
          for (int j = 0; j < SN; j++) { mfma(acc[i][j], l1[i], b1[j]); }
      }
    }
  };

  // The k loop runs over a multiple of U = lcm(NSETS, 2) tiles with no conditional work inside: a
  // tile at or past kend is loaded from the zero page and written to LDS as zeros (so the padding
  // tiles add nothing), and the prefetches past the end are issued the same way. Every load is
  // therefore issued on every path, which lets the compiler wait for exactly the register set a
  // store needs and keep the accumulators in place across iterations.
  constexpr int U = NSETS % 2 == 0 ? NSETS : 2 * NSETS;
  const int nkU = (nk + U - 1) / U * U;
  // Prologue: tiles 0..NSETS-1 into register sets 0..NSETS-1, tile 0 -> LDS buffer 0.
  if (nkU > 0) {
#pragma unroll
    for (int q = 0; q < NSETS; q++) gload(ra[q], rb[q], kbeg + q * BK);
    sstore(ra[0], rb[0], 0);
    lds_barrier();
  }
  // Step for tile kt held in LDS buffer P = kt % 2: register set S = kt % NSETS receives tile
  // kt + NSETS, set (S + 1) % NSETS (tile kt + 1) goes to the other LDS buffer. The phases are fenced
  // against the instruction scheduler: the prefetch is issued first and the LDS store of the older
  // set comes after the MFMAs, so each set has NSETS - 1 full steps to arrive.
  auto step = [&](int kt, auto Sc, auto Pc) {
    constexpr int S = decltype(Sc)::value, P = decltype(Pc)::value;
    constexpr int S1 = (S + 1) % NSETS;
    gload(ra[S], rb[S], kbeg + (kt + NSETS) * BK);
    __builtin_amdgcn_sched_barrier(0);
    compute(P);
    // 128x128 wavefront tiles run one wavefront per SIMD, with no second wavefront to cover a phase of
    // this one: their issue order interleaves the phases inside the wavefront. Per 32-wide k block the
    // first-half fragment reads, then the first-half MFMAs with the second-half reads between them,
    // then the second-half MFMAs; in the last k block the LDS stores of the next buffer go between the
    // second-half MFMAs (measured: the 1536x512x262144 weight gradient 7.5 % faster). Smaller
    // wavefront tiles keep the phases apart (two wavefronts per SIMD overlap them; the interleaved
    // order made the 256x128 NN form 14 % slower).
    constexpr bool kInterleave = !X3 && SM * SN >= 16;
    if constexpr (!kInterleave) __builtin_amdgcn_sched_barrier(0);
    sstore(ra[S1], rb[S1], P ^ 1);
    if constexpr (kInterleave) {
      constexpr int NR = SM + SN, NM = SM * SN;
      constexpr int NWA = TA ? (CA >= 2 ? 8 : 8 * CA) : CA;  // LDS stores of one register set
      constexpr int NWB = !TB ? (CB >= 2 ? 8 : 8 * CB) : CB;
      constexpr int NW = NWA + NWB < NM ? NWA + NWB : NM;
#pragma unroll
      for (int kb = 0; kb < BK / 32; kb++) {
        __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);  // LDS reads
#pragma unroll
        for (int q = 0; q < NR; q++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
        if (kb + 1 < BK / 32) {
          __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
        } else {
#pragma unroll
          for (int q = 0; q < NW; q++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // one LDS write
          }
          __builtin_amdgcn_sched_group_barrier(0x008, NM - NW, 0);
          __builtin_amdgcn_sched_group_barrier(0x200, 64, 0);
        }
      }
    }
    lds_barrier();
  };
  for (int kt = 0; kt < nkU; kt += U) unroll_steps<NSETS>(step, kt, std::make_integer_sequence<int, U>{});

  // the last loop iteration ended with a barrier: the pipeline buffers are free for the C tile
  if constexpr (EPR == BM) {
    stage_acc<SM, SN, LDC>(sC, acc, wm0, wn0, lane);
    lds_barrier();
    flush_tile<TC, BM, BN, NT, LDC>(g, sC, m0, n0);
  } else {
#pragma unroll 1
    for (int p = 0; p < BM / EPR; p++) {
      if (p > 0) lds_barrier();  // the previous pass's flush has read the staging area
      stage_acc_rows<SM, SN, LDC>(sC, acc, wm0 - p * EPR, wn0, lane, EPR);
      lds_barrier();
      flush_tile<TC, EPR, BN, NT, LDC>(g, sC, m0 + p * EPR, n0);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// NT bf16 GEMM (C = A B^T, both operands k-contiguous) with the operand tiles copied global -> LDS
// by the load-to-LDS path (global_load_lds_dwordx4): three LDS stages, two in flight while the third
// is multiplied, and no prefetch registers, so the deeper pipeline costs no occupancy.
//
// A DMA instruction writes 64 consecutive 16-byte LDS slots, lane l into slot l. Thread tid's slot
// in round i is p = i*256 + tid; it loads the source chunk (row, kc) that the swizzled BK = 32 layout
// places at slot p (the inverse of LdsLayout<32>::off), so the MFMA reads are the same as the
// register-staged kernel's. Rows past M and k past the end read the zero page.
//
// Ordering is explicit: each wave waits until only the next stage's copies are outstanding
// (vmcnt), then a barrier makes every wave's copies of this stage visible and guarantees that all
// waves are done reading the buffer the next copy overwrites. The barrier and waits are asm with a
// memory clobber: the compiler's own LDS fences would wait for every copy in flight.
// Wait until at most N of this wave's vector-memory operations are outstanding, and for all its LDS
// reads (so no read of a buffer is still in flight when the barrier lets a copy overwrite it).
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void barrier_mem() { asm volatile("s_barrier" ::: "memory"); }
// One 16-byte global -> LDS copy per lane into the wave's 1 KB window at lds (lane l -> +16 l). Issued
// as asm, like the waits: the compiler's own waits for the builtin form are vmcnt(0) before every LDS
// read, which would drain the copies in flight. M0 carries the window address; nothing else in the
// kernel uses M0 (the compiler needs it only for the builtin form).
__device__ __forceinline__ void copy_to_lds(gptr<uint16_t> src, const uint16_t* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(la) : "memory", "m0");
#pragma clang diagnostic pop
}

// S16: the launch takes the bf16-staged epilogue (stage_bf16_ok, decided on the host), so each
// instantiation carries one epilogue and its registers.
// The MFMA fragment of 32 columns c0.. (lane: column c0 + lane % 32) and 8 k-rows koff.. from a stage
// stored [k][LD] with XOR-permuted 16-byte chunks. ds_read_b64_tr_b16 exchanges data within each group
// of 16 lanes: lane j receives element j % 4 of the 8 bytes that lane 4q + j / 4 addressed, as its value
// q (measured lane layout). So lane s of a group addresses k-row koff + 4h + s / 4 at columns
// 4 (s % 4) .. + 3 of its 16, and lane j receives column j at k-rows koff + 4h + 0..3.
typedef short ph_v4i16 __attribute__((ext_vector_type(4)));
template <int LD>
__device__ __forceinline__ uint4 rd_tr(const uint16_t* s, int c0, int koff, int lane) {
  const int sl = lane & 15, cb = c0 + ((lane >> 4) & 1) * 16 + 4 * (sl & 3);
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int r = koff + 4 * h + (sl >> 2);
    const int e = r * LD + ((((cb >> 3) ^ ((r & 3) << 2))) << 3) + (cb & 7);
    const ph_v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) ph_v4i16*)(__attribute__((address_space(3))) void*)(s + e));
    w[2 * h] = (uint32_t)(uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16);
    w[2 * h + 1] = (uint32_t)(uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// WGM x WGN wavefronts (2 x 2: two blocks per CU; 4 x 4: one block of sixteen wavefronts per CU) and
// NSTG k-tile stages in LDS (NSTG - 1 in flight while one is read).
// TN: A stored [K][M] and B stored [K][N] (the weight-gradient form): each stage holds BK k-rows of the
// BM (BN) columns, the 16-byte chunks of a row XOR-permuted by the row's low two bits, and fragments are
// read with the LDS transpose read (ds_read_b64_tr_b16, two per fragment).
template <int BM, int BN, typename TC, bool S16 = false, int WGM = 2, int WGN = 2, int NSTG = 3, bool TN = false>
__global__ void __launch_bounds__(64 * WGM * WGN, WGM * WGN == 4 ? 2 : 1) k_gemm_nt_dma(GemmArgs g) {
  constexpr int BK = 32, NT = 64 * WGM * WGN;
  static_assert(!TN || (BM >= 128 && BN >= 128 && !S16), "transposed stages: 16+ chunks per row");
  static_assert(NSTG >= 3, "stages");
  static_assert(S16 || (WGM == 2 && WGN == 2) || WGM == 4, "fp32-staged epilogue layouts");
  using Lay = LdsLayout<BK>;
  static_assert(Lay::kSwz && Lay::kPitch == BK, "DMA slots follow the unpadded swizzled layout");
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int SM = WM / 32, SN = WN / 32;
  constexpr int IA = BM * BK / 8 / NT, IB = BN * BK / 8 / NT;  // DMA rounds per stage
  static_assert(IA * NT * 8 == BM * BK && IB * NT * 8 == BN * BK, "tile/threads");
  constexpr int A_EL = BM * BK, B_EL = BN * BK;  // elements per stage
  constexpr int STAGE_EL = A_EL + B_EL;
  constexpr int LDC = BN + 4;
  constexpr int PIPE_BYTES = NSTG * STAGE_EL * 2;
  constexpr int EPR = epilogue_rows(BM, LDC * 4, PIPE_BYTES);
  static_assert(EPR >= 32 && BM % EPR == 0, "epilogue staging rows");
  constexpr int C_BYTES = EPR * LDC * 4;
  constexpr int SMEM = PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES;
  static_assert(SMEM <= (WGM * WGN == 4 ? kMaxLdsBytes : 160 * 1024), "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
  uint16_t* const stages = reinterpret_cast<uint16_t*>(smem);  // stage s: A at s*STAGE_EL, B after
  float* sC = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(g, tm, tn, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int zs = split_of(g);
  const int kbeg = zs * g.kps;
  if (g.ws) g.ws += (long)zs * g.M * g.N;  // this split's partials
  const int kend = min(g.K, kbeg + g.kps);
  const int nk = (kend - kbeg + BK - 1) / BK;
  const gptr<uint16_t> A = (gptr<uint16_t>)g.A;
  const gptr<uint16_t> B = (gptr<uint16_t>)g.B;

  // this thread's source chunk in each DMA round
  auto slot_chunk = [](int p, int& row, int& kc) {
    const int pr = p >> 2;
    row = pr ^ ((pr >> 3) & 3);
    kc = (p & 3) ^ ((row >> 2) & 3);
  };
  // Per round: the chunk's offset from the tile's first row (32-bit: 256 rows of a row-major operand),
  // its k offset (2 bits, x8) and whether its row is inside the matrix (1 bit); kept compact so the
  // accumulators and fragments fit two wavefronts per SIMD without spilling.
  // TN: the chunk's k-row in the stage (5 bits) and whether its 8 columns are inside the matrix
  static_assert(!TN || (IA <= 6 && IB <= 6), "k-row fields");
  const gptr<uint16_t> Ablk = A + (TN ? (long)m0 : (long)m0 * g.lda), Bblk = B + (TN ? (long)n0 : (long)n0 * g.ldb);
  int offA[IA], offB[IB];
  uint32_t kcA = 0u, kcB = 0u, rowA = 0u, rowB = 0u;
#pragma unroll
  for (int i = 0; i < IA; i++) {
    int r, kc;
    if constexpr (TN) {
      const int p = i * NT + tid;
      r = p / (BM / 8);
      kc = (p % (BM / 8)) ^ ((r & 3) << 2);  // column chunk
      offA[i] = r * (int)g.lda + kc * 8;
      kcA |= (uint32_t)r << (5 * i);
      rowA |= (m0 + kc * 8 < g.M ? 1u : 0u) << i;
    } else {
      slot_chunk(i * NT + tid, r, kc);
      offA[i] = r * (int)g.lda + kc * 8;
      kcA |= (uint32_t)kc << (2 * i);
      rowA |= (m0 + r < g.M ? 1u : 0u) << i;
    }
  }
#pragma unroll
  for (int i = 0; i < IB; i++) {
    int r, kc;
    if constexpr (TN) {
      const int p = i * NT + tid;
      r = p / (BN / 8);
      kc = (p % (BN / 8)) ^ ((r & 3) << 2);
      offB[i] = r * (int)g.ldb + kc * 8;
      kcB |= (uint32_t)r << (5 * i);
      rowB |= (n0 + kc * 8 < g.N ? 1u : 0u) << i;
    } else {
      slot_chunk(i * NT + tid, r, kc);
      offB[i] = r * (int)g.ldb + kc * 8;
      kcB |= (uint32_t)kc << (2 * i);
      rowB |= (n0 + r < g.N ? 1u : 0u) << i;
    }
  }
  // copy the k-tile at k0 into stage st (a k-tile past the end copies zeros)
  auto issue = [&](int st, int k0) {
    uint16_t* base = stages + st * STAGE_EL;
#pragma unroll
    for (int i = 0; i < IA; i++) {
      if constexpr (TN) {
        const bool ok = ((rowA >> i) & 1u) && k0 + (int)((kcA >> (5 * i)) & 31u) < kend;
        copy_to_lds(ok ? Ablk + (offA[i] + (long)k0 * g.lda) : zero_page<uint16_t>(), base + (i * NT + wave * 64) * 8);
      } else {
        const bool ok = ((rowA >> i) & 1u) && k0 + (int)((kcA >> (2 * i)) & 3u) * 8 < kend;
        copy_to_lds(ok ? Ablk + (offA[i] + k0) : zero_page<uint16_t>(), base + (i * NT + wave * 64) * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < IB; i++) {
      if constexpr (TN) {
        const bool ok = ((rowB >> i) & 1u) && k0 + (int)((kcB >> (5 * i)) & 31u) < kend;
        copy_to_lds(ok ? Bblk + (offB[i] + (long)k0 * g.ldb) : zero_page<uint16_t>(),
                    base + A_EL + (i * NT + wave * 64) * 8);
      } else {
        const bool ok = ((rowB >> i) & 1u) && k0 + (int)((kcB >> (2 * i)) & 3u) * 8 < kend;
        copy_to_lds(ok ? Bblk + (offB[i] + k0) : zero_page<uint16_t>(), base + A_EL + (i * NT + wave * 64) * 8);
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
  const int lr = lane & 31, lk = (lane >> 5) * 16;
  // Fragments of one k sub-step (16 of the tile's 32 k; lanes 0-31 take k 0-7 of it, lanes 32-63 k 16-23,
  // and the second sub-step the k 8 above): A rows of the wave's SM sub-tiles, B rows of its SN.
  struct Frag { uint4 a[SM]; uint4 b[SN]; };
  auto rd = [&](Frag& f, int st, int koff) {
    const uint16_t* sa = stages + st * STAGE_EL;
    const uint16_t* sb = sa + A_EL;
    if constexpr (TN) {
#pragma unroll
      for (int i = 0; i < SM; i++) f.a[i] = rd_tr<BM>(sa, wm0 + i * 32, koff, lane);
#pragma unroll
      for (int j = 0; j < SN; j++) f.b[j] = rd_tr<BN>(sb, wn0 + j * 32, koff, lane);
    } else {
#pragma unroll
      for (int i = 0; i < SM; i++) f.a[i] = *reinterpret_cast<const uint4*>(&sa[Lay::off(wm0 + i * 32 + lr, koff)]);
#pragma unroll
      for (int j = 0; j < SN; j++) f.b[j] = *reinterpret_cast<const uint4*>(&sb[Lay::off(wn0 + j * 32 + lr, koff)]);
    }
  };
  auto mm = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < SM; i++)
#pragma unroll
      for (int j = 0; j < SN; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f.a[i]),
                                                            __builtin_bit_cast(bf16x8_t, f.b[j]), acc[i][j], 0, 0, 0);
  };

  // Software pipeline inside each wavefront: the LDS reads of the next sub-step are issued between the
  // MFMAs of the current one (one read after each product), so their latency and the LDS port time
  // overlap the matrix core instead of preceding it. The barrier sits between the two sub-steps of a
  // k-tile: the reads of kt's second half are done by then, and kt + 1's first half is read after it.
  if (nk > 0) {
#pragma unroll
    for (int s = 0; s < NSTG - 1; s++) issue(s, kbeg + s * BK);
    wait_vm<(NSTG - 2) * (IA + IB)>();  // k-tile 0 has landed (1 .. NSTG - 2 may be in flight)
    barrier_mem();
    issue(NSTG - 1, kbeg + (NSTG - 1) * BK);
    Frag X, Y;
    rd(X, 0, lk);
    int st = 0;  // stage of k-tile kt
#pragma unroll 1
    for (int kt = 0; kt < nk - 1; kt++) {
      rd(Y, st, lk + 8);   // second sub-step of kt, read while the first is multiplied
      mm(X);
      wait_vm<(NSTG - 2) * (IA + IB)>();  // this wave's copies of kt + 1 have landed, its reads of kt are done
      barrier_mem();       // ... every wave's: the stage of kt is free for kt + NSTG
      issue(st, kbeg + (kt + NSTG) * BK);
      st = st == NSTG - 1 ? 0 : st + 1;
      rd(X, st, lk);  // first sub-step of kt + 1, read while the second of kt is multiplied
      mm(Y);
      // issue order: products of X with the reads of Y between them, then (after the barrier) the
      // products of Y with the reads of the next X between them
      constexpr int NP = SM + SN < SM * SN ? SM + SN : SM * SN;  // MFMA / read pairs
#pragma unroll
      for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        }
        if constexpr (SM + SN > NP) __builtin_amdgcn_sched_group_barrier(0x100, SM + SN - NP, 0);
        if constexpr (SM * SN > NP) __builtin_amdgcn_sched_group_barrier(0x008, SM * SN - NP, 0);
      }
    }
    rd(Y, st, lk + 8);
    mm(X);
    mm(Y);
    wait_vm<0>();  // the copies issued past the end land before the LDS is reused
  }
  barrier_mem();
  if constexpr (S16) {
    static_assert(sizeof(TC) == 2 && BM * BN * 2 <= (PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES), "bf16 staging");
    uint32_t* sT = reinterpret_cast<uint32_t*>(smem);
    if (g.epi == PH_EPI_NONE) stage_bf16<PH_EPI_NONE, BN>(g, sT, acc, wm0, wn0, n0, lane);
    else if (g.epi == PH_EPI_BIAS) stage_bf16<PH_EPI_BIAS, BN>(g, sT, acc, wm0, wn0, n0, lane);
    else stage_bf16<PH_EPI_BIAS_RELU, BN>(g, sT, acc, wm0, wn0, n0, lane);
    lds_barrier();
    flush_bf16<BM, BN, NT>(g, sT, m0, n0, tid);
  } else if constexpr (WGM == 4) {
    // one wavefront row per pass: staged rows [0, WM) are C rows m0 + p WM ..
    static_assert(WM * LDC * 4 <= SMEM && WM % 8 == 0, "epilogue staging rows");
    auto pass = [&](auto P) {
      constexpr int p = decltype(P)::value;
      if (p > 0) lds_barrier();  // the previous pass's flush has read the staging area
      if (wave / WGN == p) stage_acc<SM, SN, LDC>(sC, acc, 0, wn0, lane);
      lds_barrier();
      flush_tile<TC, WM, BN, NT, LDC>(g, sC, m0 + p * WM, n0);
    };
    static_for(pass, std::make_integer_sequence<int, WGM>{});
  } else if constexpr (EPR == BM) {
    stage_acc<SM, SN, LDC>(sC, acc, wm0, wn0, lane);
    lds_barrier();
    flush_tile<TC, BM, BN, NT, LDC>(g, sC, m0, n0);
  } else {
    // Pass p stages sub-tiles [p SMP, (p + 1) SMP) of EVERY wave (staged rows [0, EPR/2) from the
    // upper wave row, [EPR/2, EPR) from the lower), so each pass retires part of every wave's
    // accumulators and the flush's registers do not compete with accumulators still to be staged.
    constexpr int SMP = SM * EPR / BM;
    static_assert(SMP * BM == SM * EPR && EPR == 2 * SMP * 32, "epilogue pass split");
    auto pass = [&](auto P) {
      constexpr int p = decltype(P)::value;
      if (p > 0) lds_barrier();  // the previous pass's flush has read the staging area
      stage_acc_part<p * SMP, SMP, SM, SN, LDC>(sC, acc, (wave / 2) * SMP * 32, wn0, lane);
      lds_barrier();
      flush_tile<TC, EPR, BN, NT, LDC>(g, sC, m0 + p * SMP * 32, n0, m0 + WM + p * SMP * 32);
    };
    static_for(pass, std::make_integer_sequence<int, BM / EPR>{});
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

  constexpr int LDC = BN + 4;
  constexpr int PIPE_BYTES = 2 * (BM + BN) * LDK * 4;
  constexpr int C_BYTES = BM * LDC * 4;
  static_assert((PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES) <= kMaxLdsBytes, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t smem[PIPE_BYTES > C_BYTES ? PIPE_BYTES : C_BYTES];
  float (*sA)[BM * LDK] = reinterpret_cast<float (*)[BM * LDK]>(smem);
  float (*sB)[BN * LDK] = reinterpret_cast<float (*)[BN * LDK]>(smem + 2 * BM * LDK * 4);
  float* sC = reinterpret_cast<float*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int tm = (g.M + BM - 1) / BM, tn = (g.N + BN - 1) / BN;
  int bm, bn;
  tile_coords(g, tm, tn, bm, bn);
  const int m0 = bm * BM, n0 = bn * BN;
  const int zs = split_of(g);
  const int kbeg = zs * g.kps;
  if (g.ws) g.ws += (long)zs * g.M * g.N;  // this split's partials
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
    lds_barrier();
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
    lds_barrier();
  }
  stage_acc<SM, SN, LDC>(sC, acc, wm0, wn0, lane);
  lds_barrier();
  flush_tile<TC, BM, BN, 256, LDC>(g, sC, m0, n0);
}

// Split-K fold: C = epilogue(sum over splits in order).
template <typename TC>
__global__ void k_splitk_reduce(GemmArgs g, int splits) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long MN = (long)g.M * g.N;
  if (idx >= MN) return;
  // sixteen splits' loads in flight at a time, added in split order
  float s = 0.f;
  int z = 0;
  for (; z + 16 <= splits; z += 16) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; q++) v[q] = g.ws[(long)(z + q) * MN + idx];
#pragma unroll
    for (int q = 0; q < 16; q++) s += v[q];
  }
  for (; z < splits; z++) s += g.ws[(long)z * MN + idx];
  epilogue_store<TC>(g, (int)(idx / g.N), (int)(idx % g.N), s);
}

// ------------------------------------------------------------------------------------------------
template <int BM, int BN, int BK, bool TA, bool TB>
void launch_x3(const GemmArgs& g, dim3 grid, hipStream_t st) {
  if (g.c_bf16) k_gemm_bf16<BM, BN, BK, 2, 2, TA, TB, float, float, uint16_t, true><<<grid, 256, 0, st>>>(g);
  else k_gemm_bf16<BM, BN, BK, 2, 2, TA, TB, float, float, float, true><<<grid, 256, 0, st>>>(g);
}

template <int BM, int BN>
void dispatch_x3(const GemmArgs& g, int ta, int tb, dim3 grid, hipStream_t st) {
  if (!ta && !tb) launch_x3<BM, BN, 32, false, false>(g, grid, st);
  else if (!ta && tb) launch_x3<BM, BN, 32, false, true>(g, grid, st);
  else if (ta && !tb) launch_x3<BM, BN, 32, true, false>(g, grid, st);
  else launch_x3<BM, BN, 32, true, true>(g, grid, st);
}

template <int BM, int BN, int BK, bool TA, bool TB, typename TIA, typename TIB>
void launch_bf16(const GemmArgs& g, dim3 grid, hipStream_t st) {
  if (g.c_bf16) k_gemm_bf16<BM, BN, BK, 2, 2, TA, TB, TIA, TIB, uint16_t><<<grid, 256, 0, st>>>(g);
  else k_gemm_bf16<BM, BN, BK, 2, 2, TA, TB, TIA, TIB, float><<<grid, 256, 0, st>>>(g);
}

template <int BM, int BN, int BK, typename TIA, typename TIB>
void dispatch_bf16_t(const GemmArgs& g, int ta, int tb, dim3 grid, hipStream_t st) {
  if (!ta && !tb) launch_bf16<BM, BN, BK, false, false, TIA, TIB>(g, grid, st);
  else if (!ta && tb) launch_bf16<BM, BN, BK, false, true, TIA, TIB>(g, grid, st);
  else if (ta && !tb) launch_bf16<BM, BN, BK, true, false, TIA, TIB>(g, grid, st);
  else launch_bf16<BM, BN, BK, true, true, TIA, TIB>(g, grid, st);
}

// Larger tiles for bf16 operands: 256x128 (four 128x64 wavefronts) for big outputs, 256x256 (four
// 128x128 wavefronts, one block per CU) for split-K over long reductions. Per MFMA they move 3/4
// and 1/2 of the 128x128 tile's LDS bytes.
// The NT form at 256x128 (both operands k-contiguous: the layer forward and the dgrad against the
// transposed weight copy) copies its tiles through the load-to-LDS path instead (bit-identical, about
// 5 % faster on the policy shapes).
void dispatch_big(const GemmArgs& g, int bn, int ta, int tb, dim3 grid, hipStream_t st) {
  const bool s16 = g.c_bf16 && stage_bf16_ok(g, flush_vec<uint16_t>(g));
  if (bn == 256 && ta && !tb) {
    // TN at 256x256 (the weight gradients): load-to-LDS copies of k-rows and transposing fragment reads,
    // no register transposes. The same MFMA sequence per element as the register-staged kernel
    // (bit-identical); the layer weight gradients 1536x512x262144 487 -> 364-373 us inside the step
    if (g.c_bf16) k_gemm_nt_dma<256, 256, uint16_t, false, 4, 4, 4, true><<<grid, 1024, 0, st>>>(g);
    else k_gemm_nt_dma<256, 256, float, false, 4, 4, 4, true><<<grid, 1024, 0, st>>>(g);
  } else if (bn == 256) {
    dispatch_bf16_t<256, 256, 32, uint16_t, uint16_t>(g, ta, tb, grid, st);
  } else if (!ta && tb && bn == 64) {
    if (s16) k_gemm_nt_dma<256, 64, uint16_t, true><<<grid, 256, 0, st>>>(g);
    else if (g.c_bf16) k_gemm_nt_dma<256, 64, uint16_t><<<grid, 256, 0, st>>>(g);
    else k_gemm_nt_dma<256, 64, float><<<grid, 256, 0, st>>>(g);
  } else if (!ta && tb) {
    if (s16) k_gemm_nt_dma<256, 128, uint16_t, true><<<grid, 256, 0, st>>>(g);
    else if (g.c_bf16) k_gemm_nt_dma<256, 128, uint16_t><<<grid, 256, 0, st>>>(g);
    else k_gemm_nt_dma<256, 128, float><<<grid, 256, 0, st>>>(g);
  } else {
    dispatch_bf16_t<256, 128, 32, uint16_t, uint16_t>(g, ta, tb, grid, st);
  }
}

// fp32 operands are kept raw (8 floats per chunk) in the two prefetch register sets, so they use
// half the k-tile of bf16 operands to stay within the register file.
template <int BM, int BN>
void dispatch_bf16(const GemmArgs& g, int a_dt, int b_dt, int ta, int tb, dim3 grid, hipStream_t st) {
  if (a_dt == PH_BF16 && b_dt == PH_BF16) dispatch_bf16_t<BM, BN, 64, uint16_t, uint16_t>(g, ta, tb, grid, st);
  else if (a_dt == PH_F32 && b_dt == PH_F32) dispatch_bf16_t<BM, BN, 32, float, float>(g, ta, tb, grid, st);
  else if (a_dt == PH_BF16 && b_dt == PH_F32) dispatch_bf16_t<BM, BN, 32, uint16_t, float>(g, ta, tb, grid, st);
  else dispatch_bf16_t<BM, BN, 32, float, uint16_t>(g, ta, tb, grid, st);
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
      a = bf16_to_f32(bf16_rne(a));
      b = bf16_to_f32(bf16_rne(b));
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

// dst [rows_p][cols_p] = src [rows][cols] (row stride ld) with zeros beyond it.
template <typename T>
__global__ void __launch_bounds__(256) k_pad2d(const T* __restrict__ src, long rows, long cols, long ld,
                                              T* __restrict__ dst, long rows_p, long cols_p) {
  const long n = rows_p * cols_p;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long r = i / cols_p, c = i % cols_p;
    dst[i] = (r < rows && c < cols) ? src[r * ld + c] : T(0);
  }
}

int pad2d(int dtype, const void* src, long rows, long cols, long ld, int slot, long rows_p, long cols_p, const void*& out,
          hipStream_t st) {
  const size_t esz = dtype == PH_BF16 ? 2 : 4;
  void* dst = scratch(slot, (size_t)rows_p * cols_p * esz);
  if (!dst) return PH_ERR_NOMEM;
  long blocks = (rows_p * cols_p + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (esz == 2)
    k_pad2d<uint16_t><<<(unsigned)blocks, 256, 0, st>>>((const uint16_t*)src, rows, cols, ld, (uint16_t*)dst, rows_p,
                                                        cols_p);
  else
    k_pad2d<float><<<(unsigned)blocks, 256, 0, st>>>((const float*)src, rows, cols, ld, (float*)dst, rows_p, cols_p);
  PH_LAUNCH_CHECK();
  out = dst;
  return PH_OK;
}

// Zero-padded copies of the operands whose contiguous extent, leading dimension, K or base address
// miss the MFMA kernels' vector preconditions: the contiguous extent and K round up to `vec`. K is
// padded in both operands (the zeros add nothing to the products); padded rows of A or columns of B
// feed only output rows and columns that are never stored.
int pad_operands(PhGemmDesc& d, int vec, hipStream_t st) {
  auto up = [vec](long x) { return (x + vec - 1) / vec * vec; };
  const long K8 = up(d.K);
  const bool padK = K8 != d.K;
  const long a_contig = d.trans_a ? d.M : d.K, b_contig = d.trans_b ? d.K : d.N;
  const bool padA = padK || a_contig % vec || d.lda % vec || ((uintptr_t)d.A % 16);
  const bool padB = padK || b_contig % vec || d.ldb % vec || ((uintptr_t)d.B % 16);
  if (padA) {
    // stored [M][K] (or [K][M] transposed)
    const long rows = d.trans_a ? d.K : d.M, cols = d.trans_a ? d.M : d.K;
    const long rows_p = d.trans_a ? K8 : d.M, cols_p = d.trans_a ? up(d.M) : K8;
    PH_TRY(pad2d(d.a_dtype, d.A, rows, cols, d.lda, kSlotGemmPadA, rows_p, cols_p, d.A, st));
    d.lda = cols_p;
  }
  if (padB) {
    // stored [K][N] (or [N][K] transposed)
    const long rows = d.trans_b ? d.N : d.K, cols = d.trans_b ? d.K : d.N;
    const long rows_p = d.trans_b ? d.N : K8, cols_p = d.trans_b ? K8 : up(d.N);
    PH_TRY(pad2d(d.b_dtype, d.B, rows, cols, d.ldb, kSlotGemmPadB, rows_p, cols_p, d.B, st));
    d.ldb = cols_p;
  }
  d.K = (int)K8;
  return PH_OK;
}

}  // namespace

int gemm(const PhGemmDesc& d_in, hipStream_t st) {
  PhGemmDesc d = d_in;
  PH_REQUIRE(d.M >= 0 && d.N >= 0 && d.K >= 0, "gemm: negative extent");
  if (d.M == 0 || d.N == 0) return PH_OK;
  PH_REQUIRE(d.a_dtype == PH_F32 || d.a_dtype == PH_BF16, "gemm: A dtype must be F32 or BF16");
  PH_REQUIRE(d.b_dtype == PH_F32 || d.b_dtype == PH_BF16, "gemm: B dtype must be F32 or BF16");
  PH_REQUIRE(d.c_dtype == PH_F32 || d.c_dtype == PH_BF16, "gemm: C dtype must be F32 or BF16");
  PH_REQUIRE(d.math == PH_MATH_BF16 || d.math == PH_MATH_F32 || d.math == PH_MATH_BF16X3,
             "gemm: unknown math %d", d.math);
  PH_REQUIRE(d.math == PH_MATH_BF16 || (d.a_dtype == PH_F32 && d.b_dtype == PH_F32),
             "gemm: fp32 and split-bf16 math need fp32 inputs");
  PH_REQUIRE(d.epi == PH_EPI_NONE || d.epi == PH_EPI_BIAS || d.epi == PH_EPI_BIAS_RELU ||
                 d.epi == PH_EPI_RELU_MASK || d.epi == PH_EPI_AXPBY || d.epi == kEpiGateSkip,
             "gemm: unknown epilogue %d", d.epi);
  PH_REQUIRE(d.epi != kEpiGateSkip || (d.aux && d.aux2), "gemm: gate-skip operands missing");
  PH_REQUIRE(!(d.epi == PH_EPI_BIAS || d.epi == PH_EPI_BIAS_RELU) || d.bias, "gemm: bias missing");
  PH_REQUIRE(d.epi != PH_EPI_RELU_MASK || d.aux, "gemm: mask tensor missing");

  // Vector-load preconditions of the MFMA kernels: every 8 (bf16 math) or 4 (fp32 math) consecutive
  // elements along each operand's contiguous dimension, and along K, start on a multiple of that
  // count. Shapes that miss them (a 28-wide observation, a 15-wide head) run on zero-padded copies
  // of the operands. A call with its own workspace slot (a concurrent update lane) takes the scalar
  // kernel instead, as the padded copies live in buffers shared by the calls of the default slot.
  const int vec = d.math == PH_MATH_F32 ? 4 : 8;
  const long a_contig = d.trans_a ? d.M : d.K, b_contig = d.trans_b ? d.K : d.N;
  bool aligned = a_contig % vec == 0 && d.lda % vec == 0 && b_contig % vec == 0 && d.ldb % vec == 0 &&
                 d.K % vec == 0 && ((uintptr_t)d.A % 16) == 0 && ((uintptr_t)d.B % 16) == 0;
  if (!aligned && d.ws_slot <= 0 && d.K > 0) {
    // the padded copies' rows (and K) are whole multiples of vec, whatever the logical M and N
    PH_TRY(pad_operands(d, vec, st));
    aligned = true;
  }

  GemmArgs g{};
  g.M = d.M; g.N = d.N; g.K = d.K;
  g.A = d.A; g.lda = d.lda; g.B = d.B; g.ldb = d.ldb;
  g.C = d.C; g.ldc = d.ldc; g.c_bf16 = d.c_dtype == PH_BF16;
  g.epi = d.epi; g.bias = d.bias; g.aux = d.aux; g.ldaux = d.ldaux ? d.ldaux : d.ldc;
  g.aux2 = d.epi == kEpiGateSkip ? d.aux2 : nullptr; g.ldaux2 = d.ldaux2;
  g.alpha = d.alpha; g.beta = d.beta;
  g.C2 = (uint16_t*)d.C2; g.ldc2 = d.ldc2; g.c2_trans = d.c2_trans;
  g.remap = 1;

  if (!aligned) return gemm_scalar(g, d, st);

  // Tile choice (measured on the policy shapes). bf16 x bf16 with >= 512 tiles of 256x128: the
  // 256x128 kernel. Otherwise 128x128 when that gives >= 128 tiles. Otherwise, for long reductions
  // (the wgrad forms, K = rows of the minibatch) split-K up to the resident block count (one 256x256
  // or two 128x128 blocks on each of the 256 CUs, so all splits run in one round); for short
  // reductions 64x64 tiles when those reach 128, else split-K with >= 256 of k each.
  int splits = d.splits > 0 ? d.splits : 1;
  const long tiles256 = (long)((d.M + 255) / 256) * ((d.N + 255) / 256);
  const long tiles256x128 = (long)((d.M + 255) / 256) * ((d.N + 127) / 128);
  const long tiles128 = (long)((d.M + 127) / 128) * ((d.N + 127) / 128);
  const long tiles64 = (long)((d.M + 63) / 64) * ((d.N + 63) / 64);
  const bool big_ok = d.math == PH_MATH_BF16 && d.a_dtype == PH_BF16 && d.b_dtype == PH_BF16;
  bool small = false, big = big_ok && tiles256x128 >= 512, wide_n = false;
  // NT outputs at most 64 wide (the policy heads): 256x64 tiles, half the wasted columns of 256x128
  int big_bn = !d.trans_a && d.trans_b && d.N <= 64 ? 64 : 128;
  if (!big && d.splits <= 0 && tiles128 < 128) {
    if (d.K >= 4096) {
      // 256x256 splits when the output fills the tile (TN products from 129 columns: their 256x256
      // kernel copies k-rows, so a narrow tile wastes MFMA work but no operand traffic; the encoder's
      // 512x136x262144 weight gradient 113 -> 70 us inside the step) and the reduction is long enough to
      // give every one of the 256 resident blocks >= 2048 of k; else 128x128 splits of >= 512
      big = big_ok && d.M >= 256 && (d.N >= 256 || (d.trans_a && !d.trans_b && d.N > 128)) &&
            d.K >= 2048L * (256 / (tiles256 > 0 ? tiles256 : 1));
      big_bn = 256;
      // TN bf16 products 129..256 wide that the 256x256 splits do not take (fewer than 256 rows or a
      // shorter reduction): 128x256 tiles, one block per CU, so each split reads its rows of A once
      wide_n = !big && d.trans_a && !d.trans_b && big_ok && d.N > 128 && d.N <= 256;
      // 128x128 splits: two resident blocks per CU (512 blocks) for small outputs, one (256 blocks)
      // once the output has >= 16 tiles (512x512x16384: 32 -> 16 splits, 31.8 -> 26.4 us: half the
      // fp32 partials to write and fold)
      const long tw = (long)((d.M + 127) / 128);
      const long want = big ? 256 / tiles256 : (wide_n ? 256 / tw : (tiles128 >= 16 ? 256 : 512) / tiles128);
      const long maxs = d.K / (big ? 2048 : 512);
      splits = (int)(want < maxs ? want : maxs);
      if (splits < 1) splits = 1;
    } else if (tiles64 >= 128 || d.K < 512) {
      small = true;
    } else {
      const long want = 256 / (tiles128 > 0 ? tiles128 : 1);
      const long maxs = d.K / 256;
      splits = (int)(want < maxs ? want : maxs);
      if (splits < 1) splits = 1;
    }
  }
  const int BK = 64;  // split granularity: a multiple of every k-tile in use
  int kps = (d.K + splits - 1) / splits;
  kps = (kps + BK - 1) / BK * BK;
  splits = kps > 0 ? (d.K + kps - 1) / kps : 1;
  if (splits < 1) splits = 1;
  g.kps = kps > 0 ? kps : BK;
  g.split_xcd = splits > 1 && g.kps >= 2048;
  if (splits > 1) {
    g.ws = (float*)scratch(d.ws_slot > 0 ? d.ws_slot : kSlotGemmWs, (size_t)splits * d.M * d.N * 4);
    if (!g.ws) return PH_ERR_NOMEM;
  }
  // Big NT bf16 products with 256-aligned N and no split: 256x256 tiles, sixteen 64x64 wavefronts in
  // one block per CU, four k-tile stages (128 KB). Half the operand re-reads of 256x128 tiles and twice
  // the wavefronts issuing copies per CU; the same MFMA sequence per element, so bit-identical to the
  // 256x128 kernel. Back to back over rotating operand sets the data gradient goes 528 -> 502 us; inside
  // the MinGRU step (kernel traces, alternated builds on one box) the data gradient 527 -> 523 us mean,
  // the layer forward 518 -> 515 and the encoder forward 114.5 -> 110 (five stages measured the same).
  const bool w16 = big && big_bn == 128 && !d.trans_a && d.trans_b && splits == 1 && d.N % 256 == 0;
  const int bm = big ? 256 : (small ? 64 : 128), bn = w16 ? 256 : (big ? big_bn : (wide_n ? 256 : bm));
  const unsigned tiles = (unsigned)(((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn));
  dim3 grid(tiles, 1, splits);
  if (w16) {
    if (g.c_bf16 && stage_bf16_ok(g, flush_vec<uint16_t>(g)))
      k_gemm_nt_dma<256, 256, uint16_t, true, 4, 4, 4><<<grid, 1024, 0, st>>>(g);
    else if (g.c_bf16) k_gemm_nt_dma<256, 256, uint16_t, false, 4, 4, 4><<<grid, 1024, 0, st>>>(g);
    else k_gemm_nt_dma<256, 256, float, false, 4, 4, 4><<<grid, 1024, 0, st>>>(g);
  } else if (big) {
    dispatch_big(g, bn, d.trans_a, d.trans_b, grid, st);
  } else if (wide_n) {
    launch_bf16<128, 256, 32, true, false, uint16_t, uint16_t>(g, grid, st);
  } else if (d.math == PH_MATH_BF16) {
    if (small) dispatch_bf16<64, 64>(g, d.a_dtype, d.b_dtype, d.trans_a, d.trans_b, grid, st);
    else dispatch_bf16<128, 128>(g, d.a_dtype, d.b_dtype, d.trans_a, d.trans_b, grid, st);
  } else if (d.math == PH_MATH_BF16X3) {
    if (small) dispatch_x3<64, 64>(g, d.trans_a, d.trans_b, grid, st);
    else dispatch_x3<128, 128>(g, d.trans_a, d.trans_b, grid, st);
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
  PH_REQUIRE(epilogue >= PH_EPI_NONE && epilogue <= PH_EPI_AXPBY, "gemm: unknown epilogue %d", epilogue);
  PhGemmDesc d{};
  d.trans_a = trans_a; d.trans_b = trans_b; d.M = M; d.N = N; d.K = K;
  d.a_dtype = a_dtype; d.A = A; d.lda = lda; d.b_dtype = b_dtype; d.B = B; d.ldb = ldb;
  d.c_dtype = c_dtype; d.C = C; d.ldc = ldc; d.math = math; d.epi = epilogue; d.bias = bias;
  d.aux = aux; d.ldaux = ldaux; d.alpha = alpha; d.beta = beta; d.C2 = C2; d.ldc2 = ldc2;
  d.c2_trans = c2_trans; d.splits = splits;
  return gemm(d, as_stream(stream));
}
