// Fused Newton-Schulz orthogonalisation of a batch of fp32 matrices on bf16 MFMA.
//
// One launch runs the whole quintic for every matrix of the batch: the Frobenius normalisation and
// all steps, with the iterate and its products resident in library scratch between phases (a few
// MB per matrix, so they stay in the L2 / Infinity Cache). Each matrix is taken in wide form
// (m = min(rows, cols) rows, w = max columns; tall inputs are transposed on the way in and out),
// zero-padded to multiples of 64, and each step
//   X' = aX + (bA + cA^2)X,   A = XX^T
// is evaluated in the shifted form, with E = A - I (so A^2 = I + 2E + E^2):
//   X' = (a+b+c)X + B'X,     B' = (b+2c)E + cE^2.
// It is the same polynomial, but the bf16 MFMA operands E and B' shrink as the singular values
// approach 1, so their rounding no longer cancels against the a*X term: at the same operand
// precision the shifted form roughly halves the error against an f64 iterate.
//
// Phases (each a list of 64x64 output tiles):
//   P0  raw input -> fp32, bf16 and transposed hi/lo bf16 wide copies; per-tile sums of squares
//   P1  E = s^2 XX^T - I       lower-triangle tiles (E is symmetric). Writes E in fp32 for the
//                              tile and its hi/lo bf16 halves (E = Eh + El) for the tile and its
//                              mirror, so later phases read whole rows
//   P2  B' = (b+2c)E + cE^2    lower-triangle tiles; E^2 = Eh Eh^T + Eh El^T + El Eh^T (three
//                              products, one k loop over the concatenated operands). Writes the
//                              hi/lo bf16 halves of B' (tile and mirror)
//   P3  X' = s((a+b+c)X + B'X) all tiles; B'X = Bh Xh + Bh Xl + Bl Xh with X = Xh + Xl its hi/lo
//                              bf16 halves (three products, one k loop). Writes fp32, bf16 and
//                              transposed hi/lo bf16 copies of X', or the caller's matrix after
//                              the last step
// The lo half of X matters on real gradients: B' is O(1) while small singular values are still
// growing, and 5 steps amplify an error along a small singular direction up to a^5 ~ 480-fold, so
// B' times the bf16 rounding of X alone left 1.4-2.5e-2 on the MinGRU step's 1536x512 and 16x512
// momenta (an emulation of this arithmetic reproduces the measured errors); with it, <= 3e-3.
// s = 1/(||X||_F + eps) at step 0 (the copies hold the raw input), 1 afterwards. Zero padding is
// exact: padded rows/columns of X stay zero, and E's padded diagonal (-1) only meets zeros of X.
//
// Memory: every step has its own output buffers, so within a launch each address is written once,
// and only read after its writer has signalled. Those writes are device-coherent (write-through)
// stores, so a reader on another XCD finds them in memory, and no cache can hold a stale copy of a
// line that is read: nothing needs writing back or invalidating between phases, and operand reads
// keep the L2.
//
// Scheduling: every tile of every phase of every matrix is one work item with a ticket number in
// its matrix's queue, ordered by (step, phase, matrix, tile). An item waits only for the items of
// its matrix in earlier phases, i.e. for smaller tickets of the same queue. A queue's blocks take its
// tickets from an atomic counter in increasing order, so every item waited on has been taken by a
// block that is already running: the launch completes for any grid size, without assuming that all
// blocks are co-resident. The launch's last block to leave resets the counters for the next launch.
//
// Queues: one device-wide queue, with device-coherent (write-through) stores, or, on a device of 8
// XCDs of 32 CUs (MI355X), one queue per XCD, served by the blocks that run on it (the XCC_ID
// hardware register): each matrix's items, iterates and products then stay on one XCD and its data
// moves through that XCD's L2 (plain stores, L2 hits; every line a block reads was written earlier in
// the launch by a block of the same XCD). Control words are device-scope in both (atomics, and
// relaxed device-scope loads for polling; many blocks poll one word, and polling with atomics
// serialises them behind the signal they wait for). A dependent phase costs about 6 us per-XCD
// against 8 us device-wide, but a matrix has 32 CUs instead of 256. Measured (5 steps): one 64x64 matrix 103 us per-XCD against 139 us
// device-wide, 128x128 119 against 164, but 512x512 425 against 260 and 1536x512 808 against 303.
// So per-XCD queues are used when every phase of every matrix fits one XCD (at most 32 tiles), the
// device-wide queue otherwise. Matrices go to queues by estimated work, largest first, each to the
// least loaded queue. The launch's last block checks that every queue with work had blocks on its
// XCD, else it raises a sticky flag that ph_ns_status reports.

#include "common.hpp"
#include "kernels.hpp"

#include <atomic>
#include <utility>

namespace ph {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 8 bf16 (native vector: stays in VGPRs)

constexpr int kT = 64;          // output tile edge and k chunk
constexpr int kPitch = kT + 8;  // LDS row pitch in bf16 elements (144 B: conflict-free MFMA reads)
constexpr int kGroups = 2;      // k-groups per block: each takes every other k chunk of a tile
constexpr int kThreads = 256 * kGroups;  // a k-group is 4 wavefronts, one per 32x32 quadrant
constexpr int kSets = 4;        // k chunks in flight per k-group (register prefetch depth)
constexpr unsigned kSpinLimit = 1u << 20;  // bounded wait (about a second); never reached in a valid run

struct NsMat {
  float* x;           // caller's matrix, rows x cols, normalised and orthogonalised in place
  unsigned char* ws;  // this matrix's scratch (ns_layout)
  int rows, cols;
};

constexpr int kNsQueues = 8;  // one work queue per XCD
constexpr int kXcdCus = 32;   // CUs per XCD

// Control words, each polled or updated on its own 128-byte line (32 words): the launch's blocks
// finished; the wait limit hit in this launch (kCtlFlag; +1: ever hit, +2: a queue with work had no
// blocks on its XCD, both never cleared by the kernel); the XCDs that had blocks in this launch (bit
// mask); per queue its next ticket; per matrix its items done.
constexpr int kCtlStride = 32;
constexpr int kCtlOut = 0;
constexpr int kCtlFlag = kCtlStride;
constexpr int kCtlSeen = 2 * kCtlStride;
constexpr int kCtlTicket = 3 * kCtlStride;                    // + kCtlStride * q
constexpr int kCtlDone = kCtlTicket + kCtlStride * kNsQueues;  // + kCtlStride * matrix
constexpr int kCtlWords = kCtlDone + kCtlStride * kNsMaxMats;

// One queue's share of a launch: its matrices in ticket order and their item counts per phase.
struct NsQueue {
  long n0, nt, n3;  // items of P0, of P1 (= P2) and of P3, summed over the queue's matrices
  int nmat;
  unsigned char mat[kNsMaxMats];
};
static_assert(kNsMaxMats <= 256, "queue slots are bytes");

struct NsLaunch {
  NsMat mat[kNsMaxMats];
  NsQueue q[kNsQueues];
  float coef[3 * kNsMaxSteps];
  unsigned* ctl;  // control words (kCtl*)
  int nmat, nsteps, nq;
  float eps;
  unsigned spin;   // wait bound (polls)
  unsigned qmask;  // queues with work (bit q)
};

// Buffers of step s start at base + s * stride (x*: the step's input iterate, e*/b*: its E and B').
struct Geo {
  int m, w, mp, wp, tm, tw;
  bool tall;
  long n0, nt, n3;
  long mw, mm;  // per-step strides (elements) of the wide and the square buffers
  float *xf, *ef, *part;
  uint16_t *xb, *xt, *xtl, *eh, *el, *bh, *bl;
};

// Geometry and scratch layout of one matrix for nsteps steps; returns the scratch bytes it needs.
__host__ __device__ inline size_t ns_layout(int rows, int cols, int nsteps, unsigned char* base, Geo& g) {
  g.tall = rows > cols;
  g.m = g.tall ? cols : rows;
  g.w = g.tall ? rows : cols;
  g.tm = (g.m + kT - 1) / kT;
  g.tw = (g.w + kT - 1) / kT;
  g.mp = g.tm * kT;
  g.wp = g.tw * kT;
  g.n0 = (long)g.tm * g.tw;
  g.nt = (long)g.tm * (g.tm + 1) / 2;
  g.n3 = g.n0;
  g.mw = (long)g.mp * g.wp;  // multiples of 64 * 64 elements: every step's buffer stays aligned
  g.mm = (long)g.mp * g.mp;
  const size_t ns = (size_t)nsteps, mw = (size_t)g.mw, mm = (size_t)g.mm;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (bytes + 255) & ~(size_t)255;
    return (void*)((uintptr_t)base + at);
  };
  g.xf = (float*)take(4 * mw * ns);
  g.ef = (float*)take(4 * mm * ns);
  g.xb = (uint16_t*)take(2 * mw * ns);
  g.xt = (uint16_t*)take(2 * mw * ns);
  g.xtl = (uint16_t*)take(2 * mw * ns);
  g.eh = (uint16_t*)take(2 * mm * ns);
  g.el = (uint16_t*)take(2 * mm * ns);
  g.bh = (uint16_t*)take(2 * mm * ns);
  g.bl = (uint16_t*)take(2 * mm * ns);
  g.part = (float*)take(4 * (size_t)g.n0);
  return off;
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Stores of every value another block reads in this launch. LOCAL (the reader runs on the same XCD):
// plain stores, which the write-through L1 passes to the XCD's L2. Otherwise device-coherent stores
// (relaxed agent-scope atomic stores: write-through to memory, sc1).
template <bool LOCAL, typename T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  if constexpr (LOCAL) *p = v;
  else __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Control-word atomics and polls, device scope (see the scheduling notes).
__device__ __forceinline__ unsigned ctl_add(unsigned* p, unsigned v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ctl_load(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ctl_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0 waits until `need` items of the matrix are done (relaxed polls: the data they guard is
// read for the first time after the wait, from the L2 it was written to, or from memory). The wait
// is bounded: past the limit it raises the launch's flag, and once the flag is up no further wait
// blocks, so the launch always drains quickly (with wrong results) instead of hanging.
__device__ void wait_done(unsigned* cnt, unsigned need, unsigned* flag, unsigned limit) {
  if (threadIdx.x == 0) {
    unsigned spins = 0;
    while (ctl_load(cnt) < need && ctl_load(flag) == 0u) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > limit) {
        ctl_store(flag, 1u);
        ctl_store(flag + 1, 1u);  // sticky record
        break;
      }
    }
  }
  __syncthreads();
}

// Every thread's stores have completed, then the item counts as done. A completed store has reached
// the XCD's L2 (LOCAL: where the readers look) or memory (device-coherent stores), so no L2
// write-back (an agent-scope release fence) is needed, and none is paid for (it measured 5-15 us
// per item). The asm's memory clobber keeps the compiler from moving stores past the wait.
__device__ void signal_done(unsigned* cnt) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) ctl_add(cnt, 1u);
}

// s = 1/(sqrt(sum of the P0 partials) + eps), summed in the same fixed order by every wavefront.
__device__ float norm_scale(const float* part, long n0, float eps) {
  const int lane = threadIdx.x & 63;
  float v = 0.f;
  for (long i = lane; i < n0; i += 64) v += part[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return 1.f / (sqrtf(v) + eps);
}

// Lower-triangle tile index -> (ti, tj), ti >= tj, row-major over the triangle.
__device__ inline void tri_coords(long r, int& ti, int& tj) {
  int i = (int)((sqrtf(8.f * (float)r + 1.f) - 1.f) * 0.5f);
  while ((long)i * (i + 1) / 2 > r) i--;
  while ((long)(i + 1) * (i + 2) / 2 <= r) i++;
  ti = i;
  tj = (int)(r - (long)i * (i + 1) / 2);
}

// acc0 + acc1 = this k-group's share of the sum over the nseg operand pairs of
// A_s[64 rows][K] . B_s[64 rows][K]^T, for this wavefront's 32x32 quadrant (wr, wc): k-group g
// takes chunks g, g + kGroups, ... of the concatenated k range. A_s / B_s point at the tile's first
// row; rows are ld apart; K is a multiple of 64. Chunks are loaded kSets - 1 steps ahead into
// registers, staged through the group's double-buffered LDS, and read as one 16-byte fragment per
// lane per MFMA. Both groups run the same number of steps (block barriers stay matched); a step
// whose chunk is past the end only skips its MFMAs.
struct TileOps {
  const uint16_t *a, *b;
  long da, db;
  int amask, bmask;
  int nseg;
  long ld;
  int K;
};

template <int... I>
__device__ __forceinline__ void mma_tile(const TileOps& op, uint16_t (*sA)[2][kT * kPitch],
                                         uint16_t (*sB)[2][kT * kPitch], floatx16& acc0, floatx16& acc1,
                                         std::integer_sequence<int, I...>) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave >> 2, gw = wave & 3;
  const int wr = gw >> 1, wc = gw & 1;
  const int lr = lane & 31, lk = (lane >> 5) * 16;
  const int kc = op.K / kT;
  const int nc = op.nseg * kc;
  const int nsteps = (nc + kGroups - 1) / kGroups;
  uint16_t (*gA)[kT * kPitch] = sA[grp];
  uint16_t (*gB)[kT * kPitch] = sB[grp];
  // this thread's two 16-byte pieces of each 64x64 operand chunk
  const int gt = tid & 255, prow = gt >> 3, pk = (gt & 7) * 8;
  u32x4 ra[kSets][2], rb[kSets][2];
  auto gload = [&](u32x4 (&xa)[2], u32x4 (&xb)[2], int i) __attribute__((always_inline)) {
    int c = i * kGroups + grp;
    c = c < nc ? c : nc - 1;  // past the end: reload the last chunk (never computed on)
    const int s = c / kc, k0 = (c - s * kc) * kT;
    const uint16_t* A = op.a + ((op.amask >> s) & 1) * op.da;
    const uint16_t* B = op.b + ((op.bmask >> s) & 1) * op.db;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      xa[h] = *reinterpret_cast<const u32x4*>(A + (long)(prow + 32 * h) * op.ld + k0 + pk);
      xb[h] = *reinterpret_cast<const u32x4*>(B + (long)(prow + 32 * h) * op.ld + k0 + pk);
    }
  };
  auto sstore = [&](const u32x4 (&xa)[2], const u32x4 (&xb)[2], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      *reinterpret_cast<u32x4*>(&gA[buf][(prow + 32 * h) * kPitch + pk]) = xa[h];
      *reinterpret_cast<u32x4*>(&gB[buf][(prow + 32 * h) * kPitch + pk]) = xb[h];
    }
  };
  auto mfma = [&](floatx16& c, const u32x4& a, const u32x4& b) __attribute__((always_inline)) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  };
  auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < kT; kb += 32) {
      const uint16_t* pa = &gA[buf][(wr * 32 + lr) * kPitch + kb + lk];
      const uint16_t* pb = &gB[buf][(wc * 32 + lr) * kPitch + kb + lk];
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(pa), a1 = *reinterpret_cast<const u32x4*>(pa + 8);
      const u32x4 b0 = *reinterpret_cast<const u32x4*>(pb), b1 = *reinterpret_cast<const u32x4*>(pb + 8);
      mfma(acc0, a0, b0);
      mfma(acc1, a1, b1);
    }
  };
  for (int r = 0; r < 16; r++) acc0[r] = acc1[r] = 0.f;
  // prologue: chunks 0..kSets-1 in flight, chunk 0 in LDS buffer 0
  (gload(ra[I], rb[I], I), ...);
  sstore(ra[0], rb[0], 0);
  lds_barrier();
  // step i (set S = i % kSets): refill set S with step i + kSets's chunk, compute step i's chunk,
  // stage step i + 1's
  auto step = [&](int i, auto Sc) __attribute__((always_inline)) {
    constexpr int S = decltype(Sc)::value, S1 = (S + 1) % kSets;
    if (i >= nsteps) return;
    gload(ra[S], rb[S], i + kSets);
    __builtin_amdgcn_sched_barrier(0);
    if (i * kGroups + grp < nc) compute(i & 1);
    __builtin_amdgcn_sched_barrier(0);
    sstore(ra[S1], rb[S1], (i + 1) & 1);
    lds_barrier();
  };
  for (int i = 0; i < nsteps; i += kSets) (step(i + I, std::integral_constant<int, I>{}), ...);
}

// Accumulator element e of this lane sits at tile row wr*32 + 8*(e/4) + 4*(lane/32) + e%4 and
// tile column wc*32 + lane%32.
__device__ __forceinline__ int acc_row(int e) {
  const int lane = threadIdx.x & 63, wr = ((threadIdx.x >> 6) & 3) >> 1;
  return wr * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
}
__device__ __forceinline__ int acc_col() {
  const int lane = threadIdx.x & 63, wc = ((threadIdx.x >> 6) & 3) & 1;
  return wc * 32 + (lane & 31);
}

// hi/lo bf16 halves of v (v = hi + lo to about 16 bits)
__device__ __forceinline__ void split_bf16(float v, uint16_t& h, uint16_t& l) {
  h = bf16_rne(v);
  l = bf16_rne(v - bf16_to_f32(h));
}

// Store the 4 consecutive-row values q*4..q*4+3 of this lane as 4 consecutive bf16 of the mirrored
// row (tile column -> row).
template <bool LOCAL>
__device__ __forceinline__ void store_mirror4(uint16_t* dst, const uint16_t (&v)[4]) {
  st_dev<LOCAL>(reinterpret_cast<uint64_t*>(dst), (uint64_t)v[0] | ((uint64_t)v[1] << 16) |
                                                      ((uint64_t)v[2] << 32) | ((uint64_t)v[3] << 48));
}

// P0: one 64x64 tile of the wide input into the fp32 / bf16 / transposed bf16 copies, plus the
// tile's sum of squares (fixed order).
template <bool LOCAL>
__device__ void p0_convert(const NsMat& mt, const Geo& g, long r, float* stage) {
  const int ti = (int)(r / g.tw), tj = (int)(r % g.tw);
  const int tid = threadIdx.x;
  // stage[a * 65 + b] = X_wide(ti*64 + a, tj*64 + b); loads run along the source's rows
  for (int it = 0; it < kT * kT / kThreads; it++) {
    const int id = it * kThreads + tid, a = id >> 6, b = id & 63;
    if (!g.tall) {
      const int wi = ti * kT + a, wj = tj * kT + b;
      stage[a * 65 + b] = (wi < g.m && wj < g.w) ? mt.x[(long)wi * mt.cols + wj] : 0.f;
    } else {
      const int wj = tj * kT + a, wi = ti * kT + b;  // source row wj, column wi
      stage[b * 65 + a] = (wi < g.m && wj < g.w) ? mt.x[(long)wj * mt.cols + wi] : 0.f;
    }
  }
  __syncthreads();
  float ss = 0.f;
  for (int it = 0; it < kT * kT / kThreads; it++) {
    const int id = it * kThreads + tid, a = id >> 6, b = id & 63;
    const float v = stage[a * 65 + b];
    ss += v * v;
    const long o = (long)(ti * kT + a) * g.wp + tj * kT + b;
    st_dev<LOCAL>(&g.xf[o], v);
    st_dev<LOCAL>(&g.xb[o], bf16_rne(v));
    uint16_t th, tl;
    split_bf16(stage[b * 65 + a], th, tl);
    const long ot = (long)(tj * kT + a) * g.mp + ti * kT + b;
    st_dev<LOCAL>(&g.xt[ot], th);
    st_dev<LOCAL>(&g.xtl[ot], tl);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  __syncthreads();
  if ((tid & 63) == 0) stage[tid >> 6] = ss;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int w = 0; w < kThreads / 64; w++) t += stage[w];
    st_dev<LOCAL>(&g.part[r], t);
  }
}

// LOCAL: one queue per XCD (block b serves queue b % kNsQueues); otherwise one device-wide queue.
template <bool LOCAL>
__global__ void __launch_bounds__(kThreads) k_ns_fused(const NsLaunch L) {
  __shared__ __align__(16) uint16_t sA[kGroups][2][kT * kPitch];
  __shared__ __align__(16) uint16_t sB[kGroups][2][kT * kPitch];
  __shared__ unsigned s_ticket;
  static_assert(2 * kGroups * 2 * kT * kPitch * 2 + 16 <= kMaxLdsBytes, "LDS budget");
  unsigned* ctl = L.ctl;
  const int tid = threadIdx.x;
  int qi = 0;
  if constexpr (LOCAL) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    qi = (int)(xcc & 0xfu);
  }
  if (tid == 0 && qi < kNsQueues)
    __hip_atomic_fetch_or(&ctl[kCtlSeen], 1u << qi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (qi >= kNsQueues) qi = -1;  // not a queue's XCD: no work (the last block checks coverage)
  // the queue's counts as values (binding a reference would move the kernel argument to scratch)
  const int qc = qi < 0 ? 0 : qi;
  const long qn0 = L.q[qc].n0, qnt = L.q[qc].nt, qn3 = L.q[qc].n3;
  const int qnmat = L.q[qc].nmat;
  const long per = 2 * qnt + qn3;
  const long total = qi < 0 ? 0 : qn0 + (long)L.nsteps * per;
  for (;;) {
    if (tid == 0) s_ticket = total > 0 ? ctl_add(&ctl[kCtlTicket + kCtlStride * qc], 1u) : 0u;
    __syncthreads();
    const long t = (long)s_ticket;
    __syncthreads();
    if (t >= total) break;
    // decode (phase p, step s, index r within the phase over the queue's matrices)
    int p, s = 0;
    long r;
    if (t < qn0) {
      p = 0;
      r = t;
    } else {
      const long u = t - qn0;
      s = (int)(u / per);
      r = u - (long)s * per;
      if (r < qnt) p = 1;
      else if (r < 2 * qnt) { p = 2; r -= qnt; }
      else { p = 3; r -= 2 * qnt; }
    }
    int gi = 0;
    Geo g;
    for (int k = 0;; k++) {
      gi = L.q[qc].mat[k];
      ns_layout(L.mat[gi].rows, L.mat[gi].cols, L.nsteps, L.mat[gi].ws, g);
      const long cnt = p == 0 ? g.n0 : (p == 3 ? g.n3 : g.nt);
      if (r < cnt || k == qnmat - 1) break;
      r -= cnt;
    }
    const NsMat mt = L.mat[gi];  // a copy: a reference would move the kernel argument to scratch
    unsigned* const done = &ctl[kCtlDone + kCtlStride * gi];
    if (p == 0) {
      p0_convert<LOCAL>(mt, g, r, reinterpret_cast<float*>(&sA[0][0][0]));
      signal_done(done);
      continue;
    }
    const long need = g.n0 + (long)s * (2 * g.nt + g.n3) + (p - 1) * g.nt;
    wait_done(done, (unsigned)need, &ctl[kCtlFlag], L.spin);
    const float a = L.coef[3 * s], b = L.coef[3 * s + 1], c = L.coef[3 * s + 2];
    const float sc = s == 0 ? norm_scale(g.part, g.n0, L.eps) : 1.f;
    const long xs = (long)s * g.mw, es = (long)s * g.mm;  // this step's buffers
    int ti, tj;
    TileOps op;
    if (p == 3) {
      ti = (int)(r / g.tw);
      tj = (int)(r % g.tw);
      op.nseg = 3;
      op.ld = g.mp;
      op.K = g.mp;
      // A segments (Bh, Bh, Bl) rows ti; B segments (Xh^T, Xl^T, Xh^T) rows tj
      op.a = g.bh + es + (long)ti * kT * g.mp;
      op.da = g.bl - g.bh;
      op.amask = 4;
      op.b = g.xt + xs + (long)tj * kT * g.mp;
      op.db = g.xtl - g.xt;
      op.bmask = 2;
    } else {
      tri_coords(r, ti, tj);
      if (p == 1) {
        op.nseg = 1;
        op.ld = g.wp;
        op.K = g.wp;
        op.a = g.xb + xs + (long)ti * kT * g.wp;
        op.b = g.xb + xs + (long)tj * kT * g.wp;
        op.da = op.db = 0;
        op.amask = op.bmask = 0;
      } else {
        op.nseg = 3;
        op.ld = g.mp;
        op.K = g.mp;
        const long oi = (long)ti * kT * g.mp, oj = (long)tj * kT * g.mp;
        // A segments (Eh, Eh, El) rows ti; B segments (Eh, El, Eh) rows tj
        op.a = g.eh + es + oi;
        op.b = g.eh + es + oj;
        op.da = op.db = g.el - g.eh;
        op.amask = 4;
        op.bmask = 2;
      }
    }
    // The epilogue's fp32 operand (E for P2, X for P3) in accumulator layout, loaded before the k loop
    // so that its memory latency overlaps the products (k-group 0 runs the epilogue).
    float pre[16];
    if (tid < 256 && p >= 2) {
      const float* src = p == 2 ? g.ef + es : g.xf + xs;
      const long ld = p == 2 ? g.mp : g.wp;
      const int c0 = tj * kT + acc_col(), r0 = ti * kT;
#pragma unroll
      for (int e = 0; e < 16; e++) pre[e] = src[(long)(r0 + acc_row(e)) * ld + c0];
    }
    floatx16 acc0, acc1;
    mma_tile(op, sA, sB, acc0, acc1, std::make_integer_sequence<int, kSets>{});
    // fold k-group 1's partial tile into group 0's (fixed order), through LDS
    float* red = reinterpret_cast<float*>(&sA[0][0][0]);
    if (tid >= 256) {
#pragma unroll
      for (int e = 0; e < 16; e++) red[e * 256 + (tid - 256)] = acc0[e] + acc1[e];
    }
    __syncthreads();
    if (tid < 256) {
#pragma unroll
      for (int e = 0; e < 16; e++) acc0[e] = (acc0[e] + acc1[e]) + red[e * 256 + tid];
    }
    const int col = tj * kT + acc_col();
    const int row0 = ti * kT;
    if (tid >= 256) {
      // k-group 1 is done with this item
    } else if (p == 1 || p == 2) {
      uint16_t* hi = (p == 1 ? g.eh : g.bh) + es;
      uint16_t* lo = (p == 1 ? g.el : g.bl) + es;
      float* ef = g.ef + es;
      const float cE = b + 2.f * c;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint16_t h4[4], l4[4];
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
          const int e = 4 * q + e4;
          const int row = row0 + acc_row(e);
          const long o = (long)row * g.mp + col;
          const float v = acc0[e];
          float val;
          if (p == 1) {
            val = sc * sc * v - (row == col ? 1.f : 0.f);
            st_dev<LOCAL>(&ef[o], val);
          } else {
            val = cE * pre[e] + c * v;
          }
          split_bf16(val, h4[e4], l4[e4]);
          st_dev<LOCAL>(&hi[o], h4[e4]);
          st_dev<LOCAL>(&lo[o], l4[e4]);
        }
        if (ti != tj) {
          const long om = (long)col * g.mp + row0 + acc_row(4 * q);
          store_mirror4<LOCAL>(hi + om, h4);
          store_mirror4<LOCAL>(lo + om, l4);
        }
      }
    } else {
      const bool last = s == L.nsteps - 1;
      const float abc = a + b + c;
      float* xfn = g.xf + xs + g.mw;  // next step's input (not touched after the last step)
      uint16_t* xbn = g.xb + xs + g.mw;
      uint16_t* xtn = g.xt + xs + g.mw;
      uint16_t* xtln = g.xtl + xs + g.mw;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint16_t x4[4], l4[4];
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
          const int e = 4 * q + e4;
          const int row = row0 + acc_row(e);
          const long o = (long)row * g.wp + col;
          const float v = sc * (abc * pre[e] + acc0[e]);
          if (last) {
            if (row < g.m && col < g.w) {
              if (g.tall) mt.x[(long)col * mt.cols + row] = v;
              else mt.x[(long)row * mt.cols + col] = v;
            }
          } else {
            st_dev<LOCAL>(&xfn[o], v);
            split_bf16(v, x4[e4], l4[e4]);
            st_dev<LOCAL>(&xbn[o], x4[e4]);
          }
        }
        if (!last) {
          const long om = (long)col * g.mp + row0 + acc_row(4 * q);
          store_mirror4<LOCAL>(xtn + om, x4);
          store_mirror4<LOCAL>(xtln + om, l4);
        }
      }
    }
    signal_done(done);
  }
  // Leave. The launch's last block out (every other block has taken its final ticket and finished
  // its items) checks that every queue with work had blocks on its XCD and resets the counters.
  if (tid == 0) {
    const unsigned out = __hip_atomic_fetch_add(&ctl[kCtlOut], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (out == gridDim.x - 1) {
      if ((L.qmask & ~ctl_load(&ctl[kCtlSeen])) != 0u) ctl_store(&ctl[kCtlFlag + 2], 1u);
      ctl_store(&ctl[kCtlSeen], 0u);
      ctl_store(&ctl[kCtlFlag], 0u);
      for (int q = 0; q < L.nq; q++) ctl_store(&ctl[kCtlTicket + kCtlStride * q], 0u);
      for (int i = 0; i < L.nmat; i++) ctl_store(&ctl[kCtlDone + kCtlStride * i], 0u);
      __hip_atomic_store(&ctl[kCtlOut], 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

std::atomic<unsigned> g_spin{kSpinLimit};
// 0: per-XCD queues where the device has 8 XCDs of 32 CUs and every phase of every matrix fits one
// XCD's CUs; 1: always one device-wide queue; 2: per-XCD queues whenever the device has them
std::atomic<int> g_queues{0};

__global__ void k_clear_word(unsigned* w) {
  if (threadIdx.x == 0) *w = 0u;
}

int cu_count() {
  static int n[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (n[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    n[dev] = v;
  }
  return n[dev];
}

}  // namespace

size_t ns_fused_ws_bytes(int rows, int cols, int nsteps) {
  Geo g;
  return ns_layout(rows, cols, nsteps, nullptr, g);
}

int ns_fused(float* const* X, const int* rows, const int* cols, int n, const float* coeffs, int nsteps,
             float eps, int ws_slot, int ctl_slot, hipStream_t st) {
  if (nsteps < 1 || nsteps > kNsMaxSteps) {
    set_error("newton_schulz (fused): steps must be in 1..%d", kNsMaxSteps);
    return PH_ERR_UNSUPPORTED;
  }
  unsigned* ctl = (unsigned*)scratch(ctl_slot, kCtlWords * 4);
  if (!ctl) return PH_ERR_NOMEM;
  PH_TRY(ensure_zeroed_words(ctl, kCtlWords, st));
  // per-XCD queues on a device of kNsQueues XCDs of kXcdCus CUs, for batches whose phases all fit one
  // XCD (one block per CU, so kXcdCus tiles at a time)
  const int cus = cu_count();
  const int mode = g_queues.load(std::memory_order_relaxed);
  bool local = mode != 1 && cus == kNsQueues * kXcdCus;
  if (local && mode == 0)
    for (int j = 0; j < n; j++) {
      Geo g;
      ns_layout(rows[j], cols[j], nsteps, nullptr, g);
      if (g.n3 > kXcdCus || g.nt > kXcdCus) local = false;
    }
  int i = 0;
  while (i < n) {
    // next group of at most kNsMaxMats non-empty matrices
    NsLaunch L{};
    size_t bytes = 0;
    long work[kNsMaxMats];
    long n0[kNsMaxMats], nt[kNsMaxMats], n3[kNsMaxMats];
    int j = i;
    for (; j < n && L.nmat < kNsMaxMats; j++) {
      if ((long)rows[j] * cols[j] == 0) continue;
      const int k = L.nmat++;
      NsMat& m = L.mat[k];
      m.x = X[j];
      m.rows = rows[j];
      m.cols = cols[j];
      Geo g;
      const size_t b = ns_layout(rows[j], cols[j], nsteps, nullptr, g);
      m.ws = (unsigned char*)(uintptr_t)bytes;  // offset for now
      bytes += b;
      n0[k] = g.n0;
      nt[k] = g.nt;
      n3[k] = g.n3;
      // tile-chunk products of a step: P1 over w, P2 three over m, P3 three over m
      const long cw = g.wp / kT, cm = g.mp / kT;
      work[k] = g.n0 + (long)nsteps * (g.nt * cw + 3 * g.nt * cm + 3 * g.n3 * cm);
    }
    i = j;
    if (L.nmat == 0) continue;
    unsigned char* ws = (unsigned char*)scratch(ws_slot, bytes);
    if (!ws) return PH_ERR_NOMEM;
    for (int k = 0; k < L.nmat; k++) L.mat[k].ws = ws + (uintptr_t)L.mat[k].ws;
    // matrices to queues: largest estimated work first, each to the least loaded queue (ties: the
    // lower index); a queue's matrices are ticketed in matrix order
    L.nq = local ? kNsQueues : 1;
    int qof[kNsMaxMats];
    {
      int order[kNsMaxMats];
      for (int k = 0; k < L.nmat; k++) order[k] = k;
      for (int a = 1; a < L.nmat; a++)  // stable insertion sort by work, descending
        for (int b = a; b > 0 && work[order[b]] > work[order[b - 1]]; b--) std::swap(order[b], order[b - 1]);
      long load[kNsQueues] = {};
      for (int a = 0; a < L.nmat; a++) {
        int best = 0;
        for (int q = 1; q < L.nq; q++)
          if (load[q] < load[best]) best = q;
        qof[order[a]] = best;
        load[best] += work[order[a]];
      }
    }
    long total = 0;
    for (int k = 0; k < L.nmat; k++) {
      NsQueue& Q = L.q[qof[k]];
      Q.mat[Q.nmat++] = (unsigned char)k;
      Q.n0 += n0[k];
      Q.nt += nt[k];
      Q.n3 += n3[k];
    }
    for (int q = 0; q < L.nq; q++) {
      const long tq = L.q[q].n0 + (long)nsteps * (2 * L.q[q].nt + L.q[q].n3);
      if (tq >= (1L << 31)) {
        set_error("newton_schulz (fused): batch too large");
        return PH_ERR_UNSUPPORTED;
      }
      total += tq;
    }
    for (int k = 0; k < 3 * nsteps; k++) L.coef[k] = coeffs[k];
    L.ctl = ctl;
    L.nsteps = nsteps;
    L.eps = eps;
    L.spin = g_spin.load(std::memory_order_relaxed);
    // one block per CU: measured faster than two (half as many blocks polling, and a CU's load
    // bandwidth goes to one tile at a time). Per-XCD queues take every CU (block b serves queue
    // b % kNsQueues; a queue with no items releases its blocks at once).
    const long cap = cus;
    const unsigned grid = local ? (unsigned)cap : (unsigned)(total < cap ? total : cap);
    L.qmask = 0u;
    for (int q = 0; q < L.nq; q++)
      if (L.q[q].nmat > 0) L.qmask |= 1u << q;
    if (local) k_ns_fused<true><<<grid, kThreads, 0, st>>>(L);
    else k_ns_fused<false><<<grid, kThreads, 0, st>>>(L);
    PH_LAUNCH_CHECK();
  }
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" int ph_ns_status(void* stream) {
  const hipStream_t st = as_stream(stream);
  PH_CHECK_HIP(hipStreamSynchronize(st));
  unsigned* ctl = (unsigned*)scratch_peek(kSlotNsCtl);
  if (!ctl) return PH_OK;  // no fused launch has run on this device
  unsigned rec[2] = {0u, 0u};
  PH_CHECK_HIP(hipMemcpy(rec, ctl + kCtlFlag + 1, sizeof(rec), hipMemcpyDeviceToHost));
  if (rec[0] == 0u && rec[1] == 0u) return PH_OK;
  if (rec[0]) k_clear_word<<<1, 64, 0, st>>>(ctl + kCtlFlag + 1);
  if (rec[1]) k_clear_word<<<1, 64, 0, st>>>(ctl + kCtlFlag + 2);
  PH_LAUNCH_CHECK();
  PH_CHECK_HIP(hipStreamSynchronize(st));
  if (rec[1])
    set_error("newton_schulz (fused): a workgroup ran on another XCD than its work queue's (the device does "
              "not dispatch workgroups to XCDs round-robin); the matrices written by the launches since the "
              "last status check are invalid; ph_ns_set_queues(1) selects the device-wide queue");
  else
    set_error("newton_schulz (fused): a bounded wait for another workgroup's tiles gave up; the matrices "
              "written by the launches since the last status check are invalid");
  return PH_ERR_HIP;
}

extern "C" int ph_ns_set_spin_limit(unsigned polls) {
  g_spin.store(polls ? polls : kSpinLimit, std::memory_order_relaxed);
  return PH_OK;
}

extern "C" int ph_ns_set_queues(int mode) {
  if (mode < 0 || mode > 2) {
    set_error("ph_ns_set_queues: mode must be 0 (by shape), 1 (device-wide) or 2 (per XCD)");
    return PH_ERR_ARG;
  }
  g_queues.store(mode, std::memory_order_relaxed);
  return PH_OK;
}
