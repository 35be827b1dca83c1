// Internal (non-exported) launch helpers shared between translation units.
#pragma once
#include "common.hpp"

namespace ph {

// Scratch slot ids (runtime.hip owns the table).
enum : int {
  kSlotMomentsPart = 0,
  kSlotMomentsStats = 2,
  kSlotColsumPart = 3,
  kSlotPpoPart = 4,
  kSlotGemmWs = 6,
  kSlotGemmPadA = 7,  // zero-padded copy of a GEMM's A operand (unaligned shapes)
  kSlotNs = 8,        // Newton-Schulz buffers of the stand-alone entry points
  kSlotNsCtl = 9,     // work-item counters of the fused Newton-Schulz launch (256 bytes)
  kSlotMuonU = 10,    // Nesterov updates of a batched Muon step
  kSlotPrio = 11,     // prioritised sampler: probabilities and (large N) the cumulative table
  kSlotReplayPart = 12,    // minibatch gather: per-block (count, mean, M2)
  kSlotReplayStats = 14,   // minibatch gather: [mean, std] when the caller passes none
  kSlotReplayLastw = 15,   // iterate: last-writer table, N ints, zero between calls
  kSlotMuonExact = 16,
  kSlotMuonFastU = 17,
  kSlotGclip = 18,
  kSlotRollout = 19,  // rollout step: layer inputs, layer products, padded head
  kSlotMgBufs = 20,
  kSlotHeadsPart = 21,     // multi-discrete / Gaussian heads: dashboard-loss block partials
  kSlotMlpBufs = 22,       // deep MLP update: activations, head outputs and their gradients
  kSlotGemmPadB = 23,      // zero-padded copy of a GEMM's B operand (unaligned shapes)
  kSlotLane = 24,     // 24..47: 8 concurrent update lanes x 3 slots (U, NS buffers, GEMM split-K)
  kSlotHost = 48,     // 48..127: host-buffer entry points
};
constexpr int kLanes = 8;

// Per-lane scratch for one Muon matrix update running on its own stream.
struct LaneSlots {
  int u, ns, gemm_ws;
};
inline LaneSlots lane_slots(int lane) {
  return {kSlotLane + 3 * lane, kSlotLane + 3 * lane + 1, kSlotLane + 3 * lane + 2};
}
// Library-owned side stream `lane` of the current device (created on first use, default priority)
// and fork/join events.
hipStream_t lane_stream(int lane);
int fork_lanes(hipStream_t main, int n);  // lanes 0..n-1 wait for work queued so far on main
int join_lanes(hipStream_t main, int n);  // main waits for everything queued on lanes 0..n-1
// join_lanes on an error path: the error message already set is kept whatever the join returns.
void join_lanes_on_exit(hipStream_t main, int n);

// Joins lanes 0..n-1 back into `main` on every exit of the scope that forked them, error returns
// included: an unjoined fork invalidates a stream capture, and in eager mode later work on `main`
// would not wait for the lanes' writes. join() joins now (its status is the caller's); the destructor
// joins whatever is still forked and keeps the error message already set.
struct LaneJoin {
  hipStream_t main;
  int n = 0;
  explicit LaneJoin(hipStream_t m) : main(m) {}
  int fork(int k) {
    if (k > n) n = k;  // lanes that waited before a failure are joined as well
    return fork_lanes(main, k);
  }
  int join() {
    const int k = n;
    n = 0;
    return join_lanes(main, k);
  }
  void joined() { n = 0; }  // a callee joined them
  ~LaneJoin() {
    if (n) join_lanes_on_exit(main, n);
  }
  LaneJoin(const LaneJoin&) = delete;
  LaneJoin& operator=(const LaneJoin&) = delete;
};

// Zero a block of n words once per pointer (fill kernel, no memset node; for a fixed-size scratch
// slot, whose pointer never changes).
int ensure_zeroed_words(unsigned* words, int n, hipStream_t st);

// Library-internal epilogue (not part of the public PH_EPI_* set): the MinGRU input-gradient skip term,
// C = acc + aux[row,col] * (1 - sigm(aux2[row,col])), with aux the gradient w.r.t. the layer output and
// aux2 the proj pre-activations (both of C's dtype).
constexpr int kEpiGateSkip = 0x100;

struct PhGemmDesc {
  int trans_a, trans_b, M, N, K;
  int a_dtype;
  const void* A;
  long lda;
  int b_dtype;
  const void* B;
  long ldb;
  int c_dtype;
  void* C;
  long ldc;
  int math, epi;
  const float* bias;
  const void* aux;
  long ldaux;
  float alpha, beta;
  void* C2;
  long ldc2;
  int c2_trans;
  int splits;   // <= 0: chosen by shape
  int ws_slot;  // scratch slot of the split-K partials (0: the shared default slot)
  const void* aux2;  // second epilogue operand (kEpiGateSkip)
  long ldaux2;
};
int gemm(const PhGemmDesc& d, hipStream_t st);

int ppo_grad(const float* logits, size_t ldl, const float* values, size_t ldv, const int* act,
             const float* adv, const float* ret, const float* old, const float* ov, size_t N,
             size_t A, float vfCoef, float entCoef, float clipEps, float vfClip, int max_shift,
             float* dlogits, size_t ldd, float* dvalues, size_t lddv, float* newlp, float* newval,
             double* losses, hipStream_t st);

int vtrace_f32(const float* rew, const float* val, const float* term, const float* rho,
               const float* boot, size_t B, size_t T, int variant, int time_major, int rho_is_log,
               int clamp, double gamma, double lam, double rhoClip, double cClip, float* adv,
               float* tgt, hipStream_t st);
int transpose_bf16(const uint16_t* X, uint16_t* Xt, int rows, int cols, hipStream_t st);
int muon_mat_exact(int rows, int cols, const double* W, const double* G, const double* M, double* nW,
                   double* nM, double gscale, double lr, double wd, double mu, double eps,
                   const double* coeffs, int nsteps, hipStream_t st);
// One matrix of a batched exact-tier step (nW/nM may alias W/M; c2 is set by the driver).
struct ExactMat {
  const double* W;
  const double* G;
  const double* M;
  double* nW;
  double* nM;
  int rows, cols;
  double c2;
};
// A bias vector stepped in the same launch (Nesterov + decay, as stepvec_exact; in place).
struct ExactVec {
  double* b;
  const double* g;
  double* m;
  long n;
};
constexpr int kExactBatchMax = 4;
int muon_mat_exact_batch(const ExactMat* mats, int n, const ExactVec* vecs, int nv, double gscale, double lr,
                         double wd, double mu, double eps, const double* coeffs, int nsteps, hipStream_t st);
int stepvec_exact(long n, const double* b, const double* g, const double* m, double* nb, double* nm,
                  double gscale, double lr, double wd, double mu, hipStream_t st);
int newton_schulz_fast(float* X, int rows, int cols, const float* coeffs, int nsteps, float eps,
                       int math, int ns_slot, int ws_slot, hipStream_t st);
int muon_fast(float* W, const float* G, float* M, int rows, int cols, float gscale, float lr,
              float wd, float mu, float eps, const float* coeffs, int nsteps, int math,
              const LaneSlots& slots, hipStream_t st);

// Fused bf16-MFMA Newton-Schulz of up to kNsMaxMats matrices per launch (more are run as further
// launches on `st`): X[i] (rows[i] x cols[i], fp32) is normalised and orthogonalised in place.
// ws_slot holds the per-matrix, per-step iterates and products (ns_fused_ws_bytes per matrix),
// ctl_slot the launch's work-item counters; two calls that overlap in time must not share either.
constexpr int kNsMaxMats = 16;
constexpr int kNsMaxSteps = 64;
int ns_fused(float* const* X, const int* rows, const int* cols, int n, const float* coeffs, int nsteps,
             float eps, int ws_slot, int ctl_slot, hipStream_t st);
size_t ns_fused_ws_bytes(int rows, int cols, int nsteps);

// Muon on several fp32 matrices: Nesterov into scratch, one Newton-Schulz batch, weight update.
struct MuonMat {
  float* W;
  const float* G;
  float* M;
  int rows, cols;
};
int muon_fast_batch(const MuonMat* mats, int n, float gscale, float lr, float wd, float mu, float eps,
                    const float* coeffs, int nsteps, int math, hipStream_t st);
int stepvec_f32(float* b, const float* g, float* m, long n, float gscale, float lr, float wd, float mu,
                hipStream_t st);
// stepvec over up to kNsMaxMats vectors in one launch (the same update per element).
struct StepVec {
  float* b;
  const float* g;
  float* m;
  long n;
};
int stepvec_f32_batch(const StepVec* v, int n, float gscale, float lr, float wd, float mu, hipStream_t st);
int gclip_f32(float* g, long n, float sc, float maxNorm, hipStream_t st);

int moments_normalize(int dtype, const void* x, size_t n, void* y, void* stats, hipStream_t st);
// Advantage moments over fixed chunks of kMomentsChunk elements: one partial per chunk and pass.
constexpr size_t kMomentsChunk = 4096;
inline size_t moments_chunks(size_t n) { return (n + kMomentsChunk - 1) / kMomentsChunk; }
int moments_normalize_ws(int dtype, const void* x, size_t n, void* y, void* stats, void* part,
                         hipStream_t st);
int colsum_f32(const float* X, size_t N, int J, size_t ld, float* out, float scale, int accumulate,
               hipStream_t st);
int colsum_bf16(const uint16_t* X, long N, int J, long ld, float* out, float scale, int accumulate,
                hipStream_t st);
int convert(int src_dtype, const void* x, int dst_dtype, void* y, size_t n, hipStream_t st);

long mingru_param_count(const ph_mingru_dims& d);
constexpr int kMlpMaxLayers = 8;  // hidden layers of the device MLP update
long mlp_param_count(const ph_mlp_dims& d);

// Prioritised replay (replay.hip). Column descriptor as in the C ABI.
int seg_l1(const ph_replay_cols& c, double* L1, hipStream_t st);
int prio_sample(const double* L1, size_t N, size_t B, double alpha, double beta, uint64_t rng, int* seg,
                double* mp, hipStream_t st);
int mb_gather(const ph_replay_cols& c, const int* seg, const double* mp, size_t B, void* out, double* stats,
              hipStream_t st);
int mb_iterate(const ph_replay_cols& c, const int* seg, size_t B, const float* newlp, const float* newval,
               hipStream_t st);

// Multi-discrete and continuous heads (heads.hip). Head sizes travel by value in the kernel arguments.
constexpr int kMaxHeads = 32;
struct HeadSizes {
  int K;
  int n[kMaxHeads];
};
int ppo_grad_md(const float* out, size_t ldo, const int* act, const float* adv, const float* ret, const float* old,
                const float* ov, size_t N, const int* sizes, size_t K, float vf, float ent, float clip, float vfClip,
                float* dout, size_t ldd, float* newlp, float* newval, double* losses, hipStream_t st);
int ppo_grad_cont(const float* out, size_t ldo, const float* act, const float* adv, const float* ret,
                  const float* old, const float* ov, size_t N, size_t d, float vf, float ent, float clip, float vfClip,
                  float lslo, float lshi, float* dout, size_t ldd, float* newlp, float* newval, double* losses,
                  hipStream_t st);
int sample_actions_md(int dtype, const void* Y, size_t ldy, size_t N, const int* sizes, size_t K, uint64_t rng,
                      double* out, hipStream_t st);
int sample_actions_cont(int dtype, const void* Y, size_t ldy, size_t N, size_t d, uint64_t rng, double lslo,
                        double lshi, double* out, hipStream_t st);

// Rollout forward and sampler (rollout.hip). out3 (may be NULL): [act; logp; value] as f64 [3N].
int sample_actions(int dtype, const void* Y, size_t ldy, size_t N, size_t A, int has_value, uint64_t rng, int* act,
                   void* logp, void* val, double* out3, hipStream_t st);
int mingru_rollout_step(const ph_mingru_dims& d, const float* params, const float* obs, float* state, float* out,
                        hipStream_t st);

}  // namespace ph
