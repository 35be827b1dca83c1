// Internal (non-exported) launch helpers shared between translation units.
#pragma once
#include "common.hpp"

namespace ph {

// Scratch slot ids (runtime.hip owns the table).
enum : int {
  kSlotMomentsPart = 0,
  kSlotMomentsCounter = 1,
  kSlotMomentsStats = 2,
  kSlotColsumPart = 3,
  kSlotPpoPart = 4,
  kSlotPpoCounter = 5,
  kSlotGemmWs = 6,
  kSlotGemmCounter = 7,
  kSlotNs = 8,        // 8..15 Newton-Schulz
  kSlotLean = 32,     // 32..95 host-buffer entry points
  kSlotMlp = 96,      // 96..127 resident MLP step
};

// Zero a 256-byte arrival-counter block once per pointer (fill kernel, no memset node).
int ensure_zeroed_counter(unsigned* counter, hipStream_t st);

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
  int splits;  // <= 0: chosen by shape
};
int gemm(const PhGemmDesc& d, hipStream_t st);

int ppo_grad(const float* logits, size_t ldl, const float* values, size_t ldv, const int* act,
             const float* adv, const float* ret, const float* old, const float* ov, size_t N,
             size_t A, float vfCoef, float entCoef, float clipEps, float vfClip, int max_shift,
             float* dlogits, size_t ldd, float* dvalues, size_t lddv, float* newlp, float* newval,
             double* losses, hipStream_t st);

int moments_normalize(int dtype, const void* x, size_t n, void* y, void* stats, hipStream_t st);
int colsum_f32(const float* X, size_t N, int J, size_t ld, float* out, float scale, int accumulate,
               hipStream_t st);
int convert(int src_dtype, const void* x, int dst_dtype, void* y, size_t n, hipStream_t st);

}  // namespace ph
