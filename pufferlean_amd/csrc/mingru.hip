// MinGRU policy PPO step (the reference's MinGRU trainer minibatch: V-trace -> advantage
// normalisation -> batched BPTT gradient -> grad-norm clip -> Muon; puffercuda.cu:443-466, 5206-5622,
// 5727-5976; CPU twin pufferffi.c:763-876).
//
// Layout (time-major, row r = t*B + b): obs [TB][D] fp32; activations bf16: x_l [TB][H] (layer
// inputs; x_L is the head input), cmb_l [TB][3H] (layer pre-activations, rows hid|gate|proj),
// o_l [TB][H] (recurrent state). One big MFMA GEMM per stage over all TB rows; the recurrence itself
// is a per-(b,j) scan over t with the state in registers (B*H independent chains), the done mask
// applied there (state reset after a terminal; no gradient across it).
//
// Parameters are fp32 master weights in the reference's flat order [wEnc(H*D) | bEnc(H) |
// L x W(3H*H) | wDec(A*H) | bDec(A) | wVal(H) | bVal(1)] (puffercuda.cu:5212). The policy and value
// heads run as one zero-padded head of HP = 32 rows (policy rows 0..A-1, value row A), so every
// head GEMM has an aligned reduction; padded rows stay zero.
#include "common.hpp"
#include "kernels.hpp"
#include <type_traits>

namespace ph {
namespace {

constexpr int HP = 32;  // padded head rows
constexpr unsigned kB = 256;

// sigm (common.hpp) uses the hardware exp2 / reciprocal instructions: the scans are VALU-bound with
// IEEE exp and division.
__device__ __forceinline__ float gact(float x) { return x >= 0.f ? x + 0.5f : sigm(x); }
__device__ __forceinline__ float ld(const uint16_t* p) { return bf16_to_f32(*p); }
__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ void st(uint16_t* p, float v) { *p = bf16_rne(v); }
__device__ __forceinline__ void st(float* p, float v) { *p = v; }

// 4 consecutive hidden units per thread: raw vector of 4 elements as loaded (8 bytes bf16,
// 16 bytes fp32), unpacked to fp32 only where the recurrence uses it. The scans stream each
// element once, so loads and stores are nontemporal (measured 5-10 % faster than cached ones).
template <typename TS> struct Raw4;
template <> struct Raw4<uint16_t> { uint2 v; };
template <> struct Raw4<float> { float4 v; };
typedef uint32_t ph_u32x2 __attribute__((ext_vector_type(2)));
typedef float ph_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ Raw4<uint16_t> ld4(const uint16_t* p) {
  const ph_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const ph_u32x2*>(p));
  return {make_uint2(v.x, v.y)};
}
__device__ __forceinline__ Raw4<float> ld4(const float* p) {
  const ph_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const ph_f32x4*>(p));
  return {make_float4(v.x, v.y, v.z, v.w)};
}
__device__ __forceinline__ float el(const Raw4<uint16_t>& r, int q) {
  const uint32_t w = q < 2 ? r.v.x : r.v.y;
  return bf16_to_f32((uint16_t)((q & 1) ? (w >> 16) : (w & 0xffffu)));
}
__device__ __forceinline__ float el(const Raw4<float>& r, int q) {
  return q == 0 ? r.v.x : (q == 1 ? r.v.y : (q == 2 ? r.v.z : r.v.w));
}
__device__ __forceinline__ void st4(uint16_t* p, const float (&v)[4]) {
  ph_u32x2 w;
  w.x = bf16x2_rne(v[0], v[1]);
  w.y = bf16x2_rne(v[2], v[3]);
  __builtin_nontemporal_store(w, reinterpret_cast<ph_u32x2*>(p));
}
__device__ __forceinline__ void st4(float* p, const float (&v)[4]) {
  ph_f32x4 w;
  w.x = v[0];
  w.y = v[1];
  w.z = v[2];
  w.w = v[3];
  __builtin_nontemporal_store(w, reinterpret_cast<ph_f32x4*>(p));
}

constexpr int kScanCh = 4;  // timesteps loaded ahead of the recurrence

// Forward scan of one layer. Thread = (b, 4 consecutive j); o = (1-z)*prev + z*g(hid),
// h = hg*o + (1-hg)*hin, state reset after a terminal step. The loads of kScanCh steps are issued
// before their arithmetic; per element the math is the sequential recurrence.
template <typename TS>
__global__ void __launch_bounds__(256) k_scan_fwd(const TS* __restrict__ cmb, const TS* __restrict__ hin,
                                                  TS* __restrict__ hout, TS* __restrict__ oS,
                                                  const float* __restrict__ done, int B, int H, int T) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int HV = H / 4;
  if (idx >= (long)B * HV) return;
  const int b = (int)(idx / HV), j = (int)(idx % HV) * 4;
  const long BH = (long)B * H, B3H = (long)B * 3 * H;
  const long xo = (long)b * H + j, yo = (long)b * 3 * H + j;
  float state[4] = {0.f, 0.f, 0.f, 0.f};
  // rolling prefetch: set c holds step t0 + c; after step t is computed its set is refilled with step
  // t + kScanCh, so kScanCh - 1 steps stay in flight while one is computed
  Raw4<TS> rh[kScanCh], rg[kScanCh], rp[kScanCh], rx[kScanCh];
  float rd[kScanCh];
  auto load = [&](int c, int t) __attribute__((always_inline)) {
    const TS* yt = cmb + (long)t * B3H + yo;
    rh[c] = ld4(yt);
    rg[c] = ld4(yt + H);
    rp[c] = ld4(yt + 2 * H);
    rx[c] = ld4(hin + (long)t * BH + xo);
    rd[c] = done[(long)t * B + b];
  };
#pragma unroll
  for (int c = 0; c < kScanCh; c++)
    if (c < T) load(c, c);
  for (int t0 = 0; t0 < T; t0 += kScanCh) {
#pragma unroll
    for (int c = 0; c < kScanCh; c++) {
      const int t = t0 + c;
      if (t >= T) break;
      float hv[4], ov[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float z = sigm(el(rg[c], q)), g = gact(el(rh[c], q)), hg = sigm(el(rp[c], q));
        const float o = (1.f - z) * state[q] + z * g;
        hv[q] = hg * o + (1.f - hg) * el(rx[c], q);
        ov[q] = o;
        state[q] = rd[c] != 0.f ? 0.f : o;
      }
      const long so = (long)t * BH + xo;
      st4(hout + so, hv);
      st4(oS + so, ov);
      if (t + kScanCh < T) load(c, t + kScanCh);  // t is uniform: no lane loads past the end
    }
  }
}

// Backward scan of one layer (adjoint of k_scan_fwd), t descending. dhn: gradient w.r.t. this
// layer's output; writes dy = d(hid,gate,proj) pre-activation gradients. The direct part of the
// gradient w.r.t. the layer input, dhn*(1-hg), is not written: the data-gradient GEMM dy.W adds it in
// its epilogue from dhn and the proj pre-activations. o_{t-1} is loaded once and carried as o_t of
// the next (earlier) step.
template <typename TS>
__global__ void __launch_bounds__(256) k_scan_bwd(const TS* __restrict__ cmb, const TS* __restrict__ oS,
                                                  const TS* __restrict__ hin, const TS* __restrict__ dhn,
                                                  TS* __restrict__ dy, const float* __restrict__ done, int B,
                                                  int H, int T) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int HV = H / 4;
  if (idx >= (long)B * HV || T <= 0) return;
  const int b = (int)(idx / HV), j = (int)(idx % HV) * 4;
  const long BH = (long)B * H, B3H = (long)B * 3 * H;
  const long xo = (long)b * H + j, yo = (long)b * 3 * H + j;
  float dOn[4] = {0.f, 0.f, 0.f, 0.f};
  Raw4<TS> ocur = ld4(oS + (long)(T - 1) * BH + xo);
  // rolling prefetch (t descending): set c holds step t0 - c and is refilled with step t - kScanCh
  // once step t is computed
  Raw4<TS> rh[kScanCh], rg[kScanCh], rp[kScanCh], rx[kScanCh], rdh[kScanCh], rpo[kScanCh];
  float rkeep[kScanCh];
  auto load = [&](int c, int t) __attribute__((always_inline)) {
    const int tp = t > 0 ? t - 1 : 0;
    const TS* yt = cmb + (long)t * B3H + yo;
    rh[c] = ld4(yt);
    rg[c] = ld4(yt + H);
    rp[c] = ld4(yt + 2 * H);
    rx[c] = ld4(hin + (long)t * BH + xo);
    rdh[c] = ld4(dhn + (long)t * BH + xo);
    rpo[c] = ld4(oS + (long)tp * BH + xo);
    rkeep[c] = (t > 0 && done[(long)tp * B + b] == 0.f) ? 1.f : 0.f;
  };
#pragma unroll
  for (int c = 0; c < kScanCh; c++)
    if (T - 1 - c >= 0) load(c, T - 1 - c);
  for (int t0 = T - 1; t0 >= 0; t0 -= kScanCh) {
#pragma unroll
    for (int c = 0; c < kScanCh; c++) {
      const int t = t0 - c;
      if (t < 0) break;
      const bool keep_prev = rkeep[c] != 0.f;
      float vdg[4], vdz[4], vdp[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float hid = el(rh[c], q), gate = el(rg[c], q), proj = el(rp[c], q);
        const float o = el(ocur, q), hi = el(rx[c], q), dh = el(rdh[c], q);
        const float prev = keep_prev ? el(rpo[c], q) : 0.f;
        const float z = sigm(gate), hg = sigm(proj), sh = sigm(hid);
        const float g = hid >= 0.f ? hid + 0.5f : sh;
        const float dhg = dh * (o - hi);
        const float dox = dh * hg + dOn[q];
        const float dz = dox * (g - prev);
        const float dprev = dox * (1.f - z);
        const float dg = dox * z;
        const float sg = hid >= 0.f ? 1.f : sh * (1.f - sh);
        vdg[q] = dg * sg;
        vdz[q] = dz * z * (1.f - z);
        vdp[q] = dhg * hg * (1.f - hg);
        dOn[q] = keep_prev ? dprev : 0.f;
      }
      const long yw = (long)t * B3H + yo;
      st4(dy + yw, vdg);
      st4(dy + yw + H, vdz);
      st4(dy + yw + 2 * H, vdp);
      ocur = rpo[c];
      if (t - kScanCh >= 0) load(c, t - kScanCh);  // t is uniform: no lane loads before step 0
    }
  }
}

// Backward scan of the top layer (bf16 tier) with the head's data gradient folded in. dh = dl[:, :nh] Wh
// is formed per step from the bf16 loss-gradient row of the segment (dlb [TB][HP]) and the head
// weights Wh [HP][H] (staged in LDS as row pairs; a thread's pairs stay in its registers across the
// steps) with packed bf16 dot products, instead of being read from a separate GEMM's output; besides dy the
// kernel writes the gate-skip term dh (1 - sigm(proj)), which the data-gradient GEMM adds with its
// AXPBY epilogue. H is a multiple of 256, so the H/4 lanes of a segment fill whole wavefronts and the
// loss-gradient row is read with wavefront-uniform (scalar) loads; NW is the number of its 32-bit words
// loaded per step (nh <= 2 NW) and CH the steps loaded ahead. The per-step arithmetic of the recurrence
// is that of k_scan_bwd.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int NW, int CH>
__global__ void __launch_bounds__(256) k_scan_bwd_top(const uint16_t* __restrict__ cmb, const uint16_t* __restrict__ oS,
                                                      const uint16_t* __restrict__ hin,
                                                      const uint16_t* __restrict__ dlb,
                                                      const uint16_t* __restrict__ wh, int nh,
                                                      uint16_t* __restrict__ dy, uint16_t* __restrict__ skip,
                                                      const float* __restrict__ done, int B, int H, int T) {
  // Wh row pairs: swp[p * H + j] = Wh[2p][j] | Wh[2p + 1][j] << 16 for p < NW (Wh has HP >= 2 NW rows,
  // zero past nh, as are dl's columns past nh, so pairs past nh add nothing)
  extern __shared__ uint32_t swp[];
  const int HV = H / 4;
  for (int i = threadIdx.x; i < NW * H; i += blockDim.x) {
    const int pr = i / H, jj = i - pr * H;
    swp[i] = (uint32_t)wh[(long)(2 * pr) * H + jj] | ((uint32_t)wh[(long)(2 * pr + 1) * H + jj] << 16);
  }
  __syncthreads();  // the only barrier: every thread reaches it before the bounds check
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)B * HV || T <= 0) return;
  const int b = __builtin_amdgcn_readfirstlane((int)(idx / HV));  // one segment per wavefront
  const int j = (int)(idx % HV) * 4;
  const long BH = (long)B * H, B3H = (long)B * 3 * H;
  const long xo = (long)b * H + j, yo = (long)b * 3 * H + j;
  const uint4* wj = reinterpret_cast<const uint4*>(swp + j);  // + p * H / 4 for pair p
  float dOn[4] = {0.f, 0.f, 0.f, 0.f};
  Raw4<uint16_t> ocur = ld4(oS + (long)(T - 1) * BH + xo);
  // rolling prefetch (t descending): set c holds step t0 - c and is refilled with step t - CH once
  // step t is computed
  Raw4<uint16_t> rh[CH], rg[CH], rp[CH], rx[CH], rpo[CH];
  uint32_t rl[CH][NW];
  float rkeep[CH];
  auto load = [&](int c, int t) __attribute__((always_inline)) {
    const int tp = t > 0 ? t - 1 : 0;
    const uint16_t* yt = cmb + (long)t * B3H + yo;
    rh[c] = ld4(yt);
    rg[c] = ld4(yt + H);
    rp[c] = ld4(yt + 2 * H);
    rx[c] = ld4(hin + (long)t * BH + xo);
    rpo[c] = ld4(oS + (long)tp * BH + xo);
    const uint32_t* lr = reinterpret_cast<const uint32_t*>(dlb + ((long)t * B + b) * HP);
#pragma unroll
    for (int w = 0; w < NW; w++) rl[c][w] = lr[w];
    rkeep[c] = (t > 0 && done[(long)tp * B + b] == 0.f) ? 1.f : 0.f;
  };
#pragma unroll
  for (int c = 0; c < CH; c++)
    if (T - 1 - c >= 0) load(c, T - 1 - c);
  for (int t0 = T - 1; t0 >= 0; t0 -= CH) {
#pragma unroll
    for (int c = 0; c < CH; c++) {
      const int t = t0 - c;
      if (t < 0) break;
      // dh = dl Wh[:, j..j+3]: packed bf16 pair products, pairs ascending
      float dhv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pr = 0; pr < NW; pr++) {
        const bf16x2_t dp = __builtin_bit_cast(bf16x2_t, rl[c][pr]);
        const uint4 w = wj[pr * HV];
        dhv[0] = __builtin_amdgcn_fdot2_f32_bf16(dp, __builtin_bit_cast(bf16x2_t, w.x), dhv[0], false);
        dhv[1] = __builtin_amdgcn_fdot2_f32_bf16(dp, __builtin_bit_cast(bf16x2_t, w.y), dhv[1], false);
        dhv[2] = __builtin_amdgcn_fdot2_f32_bf16(dp, __builtin_bit_cast(bf16x2_t, w.z), dhv[2], false);
        dhv[3] = __builtin_amdgcn_fdot2_f32_bf16(dp, __builtin_bit_cast(bf16x2_t, w.w), dhv[3], false);
      }
      const bool keep_prev = rkeep[c] != 0.f;
      float vdg[4], vdz[4], vdp[4], vsk[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float hid = el(rh[c], q), gate = el(rg[c], q), proj = el(rp[c], q);
        const float o = el(ocur, q), hi = el(rx[c], q), dh = dhv[q];
        const float prev = keep_prev ? el(rpo[c], q) : 0.f;
        const float z = sigm(gate), hg = sigm(proj), sh = sigm(hid);
        const float g = hid >= 0.f ? hid + 0.5f : sh;
        const float dhg = dh * (o - hi);
        const float dox = dh * hg + dOn[q];
        const float dz = dox * (g - prev);
        const float dprev = dox * (1.f - z);
        const float dg = dox * z;
        const float sg = hid >= 0.f ? 1.f : sh * (1.f - sh);
        vdg[q] = dg * sg;
        vdz[q] = dz * z * (1.f - z);
        vdp[q] = dhg * hg * (1.f - hg);
        vsk[q] = dh * (1.f - hg);
        dOn[q] = keep_prev ? dprev : 0.f;
      }
      const long yw = (long)t * B3H + yo;
      st4(dy + yw, vdg);
      st4(dy + yw + H, vdz);
      st4(dy + yw + 2 * H, vdp);
      st4(skip + (long)t * BH + xo, vsk);
      ocur = rpo[c];
      if (t - CH >= 0) load(c, t - CH);  // t is uniform: no lane loads before step 0
    }
  }
}

// bf16 copies of the weights for the GEMMs: WEnc [H][D]; W_l [3H][H] and W_l^T [H][3H];
// the padded head Wh [HP][H] (rows: wDec, wVal, zeros), its transpose WhT [H][HP] and bias bh [HP].
template <typename TW>
__global__ void k_prep_weights(const float* __restrict__ p, int D, int H, int L, int A,
                               TW* __restrict__ wenc, TW* __restrict__ wl, TW* __restrict__ wlt,
                               TW* __restrict__ wh, TW* __restrict__ wht, float* __restrict__ bh) {
  const long szE = (long)H * D, szL = 3L * H * H;
  const long nL = (long)L * szL, nH = (long)HP * H;
  const long total = szE + nL + nH + HP;
  const long offW = szE + H, offDec = offW + nL, offBDec = offDec + (long)A * H, offVal = offBDec + A,
             offBVal = offVal + H;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
    if (i < szE) {
      st(wenc + i, p[i]);
    } else if (i < szE + nL) {
      const long q = i - szE;
      const long l = q / szL, r = q % szL;
      const int row = (int)(r / H), col = (int)(r % H);  // W_l[row][col], row < 3H
      const float v = p[offW + q];
      st(wl + q, v);
      st(wlt + l * szL + (long)col * 3 * H + row, v);
    } else if (i < szE + nL + nH) {
      const long q = i - szE - nL;
      const int row = (int)(q / H), col = (int)(q % H);
      float v = 0.f;
      if (row < A) v = p[offDec + (long)row * H + col];
      else if (row == A) v = p[offVal + col];
      st(wh + q, v);
      st(wht + (long)col * HP + row, v);
    } else {
      const int k = (int)(i - szE - nL - nH);
      bh[k] = k < A ? p[offBDec + k] : (k == A ? p[offBVal] : 0.f);
    }
  }
}

// Head gradient scatter: gh [HP][H] and gbh [HP] into the flat gradient (wDec, bDec, wVal, bVal).
__global__ void k_head_scatter(const float* __restrict__ gh, const float* __restrict__ gbh, int H, int A,
                               float* __restrict__ gDec) {
  // gDec points at wDec's gradient; bDec follows it, then wVal, then bVal
  const long n = (long)(A + 1) * H + A + 1;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    if (i < (long)A * H) gDec[i] = gh[i];                                     // wDec rows
    else if (i < (long)A * H + A) gDec[i] = gbh[i - (long)A * H];              // bDec
    else if (i < (long)A * H + A + H) gDec[i] = gh[(long)A * H + (i - (long)A * H - A)];  // wVal
    else gDec[i] = gbh[A];                                                      // bVal
  }
}

// bf16 copy of the observations [rows][D] (D a multiple of 8, x 16-byte aligned) with row pitch
// D + 8: columns D..D+7 hold 1, 0, ..., 0. The encoder's weight-gradient product dh^T [obs | 1 | 0]
// then carries the bias gradient (the column sums of dh) in its column D.
__global__ void k_obs_bf16_ones(const float* __restrict__ x, uint16_t* __restrict__ y, long rows, int D) {
  const int cpr = D / 8 + 1;  // 8-element chunks per row of y
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cpr) return;
  const long r = i / cpr;
  const int c = (int)(i - r * cpr);
  uint4 v = make_uint4(0x3F80u, 0u, 0u, 0u);  // bf16 1.0, then zeros
  if (c < D / 8) {
    const float4 a = reinterpret_cast<const float4*>(x + r * D)[2 * c];
    const float4 b = reinterpret_cast<const float4*>(x + r * D)[2 * c + 1];
    v = make_uint4(bf16x2_rne(a.x, a.y), bf16x2_rne(a.z, a.w), bf16x2_rne(b.x, b.y), bf16x2_rne(b.z, b.w));
  }
  reinterpret_cast<uint4*>(y + r * (D + 8))[c] = v;
}

// [H][D + 8] product of the encoder backward -> gWEnc (H x D) and gbEnc (column D)
__global__ void k_enc_scatter(const float* __restrict__ ge, int H, int D, float* __restrict__ gW,
                              float* __restrict__ gb) {
  const long n = (long)H * (D + 1);
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const int h = (int)(i / (D + 1)), d = (int)(i - (long)h * (D + 1));
    const float v = ge[(long)h * (D + 8) + d];
    if (d < D) gW[(long)h * D + d] = v;
    else gb[h] = v;
  }
}

// V-trace outputs -> the minibatch columns the loss reads: ret = adv + V (already the target),
// advantage normalised with the minibatch mean/std (stats[0], stats[1] = std + 1e-8).
__global__ void k_norm_adv(const float* __restrict__ adv, const float* __restrict__ stats, long n,
                           float* __restrict__ advn) {
  long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) advn[i] = (adv[i] - stats[0]) / stats[1];
}

// fp32 -> bf16 (RNE), 8 elements per thread (n is a multiple of 8: the observation width is)
// y = bf16(x) over n elements (x 16-byte aligned): 8 per thread, the last partial group element-wise.
__global__ void k_f32_to_bf16_k(const float* __restrict__ x, uint16_t* __restrict__ y, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i * 8 >= n) return;
  if (i * 8 + 8 <= n) {
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    reinterpret_cast<uint4*>(y)[i] =
        make_uint4(bf16x2_rne(a.x, a.y), bf16x2_rne(a.z, a.w), bf16x2_rne(b.x, b.y), bf16x2_rne(b.z, b.w));
  } else {
    for (long e = i * 8; e < n; e++) y[e] = bf16_rne(x[e]);
  }
}

// Activation and weight-copy buffers hold bf16 (precision 0) or fp32 (precision 1) elements; they
// are sized for fp32 so one allocation serves both tiers.
struct Bufs {
  void *obsb, *x, *cmb, *o, *dy, *dh0, *dh1, *dlb;
  void *wenc, *wl, *wlt, *wh, *wht;
  float *bh, *logit, *dl, *gh, *gbh, *genc, *adv, *advn, *tgt, *newlp, *newval, *stats;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__global__ void k_zero_u32(uint32_t* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0u;
}

int fill_zero(void* p, size_t bytes, hipStream_t st) {
  const long n = (long)(bytes / 4);
  k_zero_u32<<<1024, 256, 0, st>>>((uint32_t*)p, n);
  PH_LAUNCH_CHECK();
  return PH_OK;
}

// Carves the step's device buffers from one library-owned allocation.
int get_bufs(const ph_mingru_dims& d, Bufs& b, hipStream_t st) {
  const long TB = (long)d.T * d.B, H = d.H, L = d.L;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align256(bytes); return o; };
  const size_t es = d.precision == 1 ? 4 : 2;
  const size_t o_obsb = take((size_t)TB * (d.D + 8) * 2);  // pitch D + 8 (a ones column)
  const size_t o_x = take((size_t)(L + 1) * TB * H * es);
  const size_t o_cmb = take((size_t)L * TB * 3 * H * es);
  const size_t o_o = take((size_t)L * TB * H * es);
  const size_t o_dy = take((size_t)TB * 3 * H * es);
  const size_t o_dh0 = take((size_t)TB * H * es);
  const size_t o_dh1 = take((size_t)TB * H * es);
  const size_t o_wenc = take((size_t)H * d.D * es);
  const size_t o_wl = take((size_t)L * 3 * H * H * es);
  const size_t o_wlt = take((size_t)L * 3 * H * H * es);
  const size_t o_wh = take((size_t)HP * H * es);
  const size_t o_wht = take((size_t)HP * H * es);
  const size_t o_bh = take(HP * 4);
  const size_t o_logit = take((size_t)TB * HP * 4);
  const size_t o_dl = take((size_t)TB * HP * 4);
  const size_t o_dlb = take((size_t)TB * HP * 2);
  const size_t o_gh = take((size_t)HP * H * 4);
  const size_t o_gbh = take(HP * 4);
  const size_t o_genc = take((size_t)H * (d.D + 8) * 4);
  const size_t o_adv = take((size_t)TB * 4);
  const size_t o_advn = take((size_t)TB * 4);
  const size_t o_tgt = take((size_t)TB * 4);
  const size_t o_newlp = take((size_t)TB * 4);
  const size_t o_newval = take((size_t)TB * 4);
  const size_t o_stats = take(64);
  uint8_t* base = (uint8_t*)scratch(kSlotMgBufs, off);
  if (!base) return PH_ERR_NOMEM;
  // The padded head columns of dl (past the A logits and the value) are never written by the loss
  // kernels and must read as zero: cleared with a fill kernel whenever this region moves (first use
  // or a new shape) or the head width changes (a wider head's columns would otherwise stay behind,
  // NaN rows of an out-of-range action included).
  static void* zeroed_at[16] = {};
  static size_t zeroed_len[16] = {};
  static int zeroed_a[16] = {};
  int dev = 0;
  PH_CHECK_HIP(hipGetDevice(&dev));
  const size_t dl_bytes = (size_t)TB * HP * 4;
  if (zeroed_at[dev & 15] != (void*)(base + o_dl) || zeroed_len[dev & 15] != dl_bytes ||
      zeroed_a[dev & 15] != d.A) {
    PH_TRY(fill_zero(base + o_dl, dl_bytes, st));
    zeroed_at[dev & 15] = base + o_dl;
    zeroed_len[dev & 15] = dl_bytes;
    zeroed_a[dev & 15] = d.A;
  }
  b.obsb = base + o_obsb; b.x = base + o_x; b.cmb = base + o_cmb; b.o = base + o_o; b.dy = base + o_dy;
  b.dh0 = base + o_dh0; b.dh1 = base + o_dh1; b.dlb = base + o_dlb; b.wenc = base + o_wenc; b.wl = base + o_wl;
  b.wlt = base + o_wlt; b.wh = base + o_wh; b.wht = base + o_wht;
  b.bh = (float*)(base + o_bh); b.logit = (float*)(base + o_logit); b.dl = (float*)(base + o_dl);
  b.gh = (float*)(base + o_gh); b.gbh = (float*)(base + o_gbh);
  b.genc = (float*)(base + o_genc); b.adv = (float*)(base + o_adv);
  b.advn = (float*)(base + o_advn); b.tgt = (float*)(base + o_tgt); b.newlp = (float*)(base + o_newlp);
  b.newval = (float*)(base + o_newval); b.stats = (float*)(base + o_stats);
  return PH_OK;
}

PhGemmDesc gd(int ta, int tb, int M, int N, int K, int adt, const void* A, long lda, int bdt,
              const void* B, long ldb, int cdt, void* C, long ldc, int math) {
  PhGemmDesc d{};
  d.trans_a = ta; d.trans_b = tb; d.M = M; d.N = N; d.K = K;
  d.a_dtype = adt; d.A = A; d.lda = lda; d.b_dtype = bdt; d.B = B; d.ldb = ldb;
  d.c_dtype = cdt; d.C = C; d.ldc = ldc; d.math = math; d.alpha = 1.f;
  return d;
}

// Forward + backward over one minibatch: writes the summed gradient G[P] and new_logp/new_value.
// TS: activation / weight-copy storage (uint16_t = bf16 with bf16 MFMA, float = fp32 MFMA).
// heads NULL: one categorical head over the A logits (act [TB]); otherwise K categorical heads whose
// sizes sum to A (act [TB][K]), the only difference being the loss kernel on the head rows
// (puffercuda.cu:5202-5205: the BPTT is generic in the logits width).
template <typename TS>
int mingru_ppo_grad_t(const ph_mingru_dims& d, const ph_ppo_coefs& c, const HeadSizes* heads, const float* params,
                      const float* obs, const int* act, const float* advn, const float* ret,
                      const float* oldlp, const float* oldval, const float* done, float* G,
                      float* newlp, float* newval, double* losses, hipStream_t st, bool join_lane0) {
  constexpr bool BF = sizeof(TS) == 2;
  constexpr int DT = BF ? PH_BF16 : PH_F32;
  constexpr int MATH = BF ? PH_MATH_BF16 : PH_MATH_F32;
  const long TB = (long)d.T * d.B;
  const int H = d.H, D = d.D, L = d.L, A = d.A;
  Bufs b;
  PH_TRY(get_bufs(d, b, st));
  LaneJoin lanes(st);  // lane 0 (head and fp32 encoder bias gradients) is joined on every exit
  TS* x = (TS*)b.x;
  TS* cmbs = (TS*)b.cmb;
  TS* os = (TS*)b.o;
  TS* dy = (TS*)b.dy;
  TS* wl = (TS*)b.wl;
  TS* wlt = (TS*)b.wlt;
  const long szE = (long)H * D, szL = 3L * H * H;
  const long offBEnc = szE, offW = szE + H, offDec = offW + (long)L * szL;

  // GEMM copies of the weights (and bf16 observations)
  k_prep_weights<TS><<<1024, kB, 0, st>>>(params, D, H, L, A, (TS*)b.wenc, wl, wlt, (TS*)b.wh,
                                          (TS*)b.wht, b.bh);
  const void* obsg = obs;
  if (BF) {
    PH_REQUIRE(((uintptr_t)obs % 16) == 0, "mingru: observations must be 16-byte aligned");
    k_obs_bf16_ones<<<ceil_div(TB * (D / 8 + 1), kB), kB, 0, st>>>(obs, (uint16_t*)b.obsb, TB, D);
    obsg = b.obsb;
  }
  const long ldo = BF ? D + 8 : D;  // row pitch of the observations the GEMMs read
  PH_LAUNCH_CHECK();

  // encoder: x0 = obs W_enc^T + b_enc
  {
    PhGemmDesc g = gd(0, 1, (int)TB, H, D, DT, obsg, ldo, DT, b.wenc, D, DT, x, H, MATH);
    g.epi = PH_EPI_BIAS; g.bias = params + offBEnc;
    PH_TRY(gemm(g, st));
  }
  // layers
  for (int l = 0; l < L; l++) {
    TS* xl = x + (long)l * TB * H;
    TS* cmb = cmbs + (long)l * TB * 3 * H;
    PhGemmDesc g = gd(0, 1, (int)TB, 3 * H, H, DT, xl, H, DT, wl + l * szL, H, DT, cmb, 3 * H, MATH);
    PH_TRY(gemm(g, st));
    k_scan_fwd<TS><<<ceil_div((long)d.B * H / 4, kB), kB, 0, st>>>(cmb, xl, xl + TB * H,
                                                                 os + (long)l * TB * H, done, d.B, H, d.T);
    PH_LAUNCH_CHECK();
  }
  TS* xL = x + (long)L * TB * H;
  // heads: logits|value = x_L Wh^T + bh  ([TB][HP] fp32)
  {
    PhGemmDesc g = gd(0, 1, (int)TB, HP, H, DT, xL, H, DT, b.wh, H, PH_F32, b.logit, HP, MATH);
    g.epi = PH_EPI_BIAS; g.bias = b.bh;
    PH_TRY(gemm(g, st));
  }
  // fused PPO loss: dlogits into dl[:, :A], dvalue into dl[:, A]; its advantages and returns may come
  // from work the caller queued on lane 0
  if (join_lane0) PH_TRY(join_lanes(st, 1));
  if (heads)
    PH_TRY(ppo_grad_md(b.logit, HP, act, advn, ret, oldlp, oldval, TB, heads->n, heads->K, c.vf_coef, c.ent_coef,
                       c.clip_eps, c.vf_clip, b.dl, HP, newlp, newval, losses, st));
  else
    PH_TRY(ppo_grad(b.logit, HP, b.logit + A, HP, act, advn, ret, oldlp, oldval, TB, A, c.vf_coef,
                    c.ent_coef, c.clip_eps, c.vf_clip, 1, b.dl, HP, b.dl + A, HP, newlp, newval, losses, st));
  // bf16 tier with H a multiple of 256: the top layer's backward scan forms dh_L = dl Wh itself from the
  // bf16 copy of dl and Wh in LDS (no dh_L GEMM and no dh_L round trip through memory) and writes the
  // gate-skip term, which its data-gradient GEMM adds as a plain AXPBY operand
  const int nh = A + 1;
  // (at most 18 head rows: the 9 words of a loss-gradient row per step, 4 steps ahead, fit the scalar
  // registers without spilling)
  const bool top_fused = BF && H % 256 == 0 && nh <= 18 && 9L * H * 4 <= 65536;
  // head backward: gh = dl^T x_L; gbh = colsum(dl); dh_L = dl Wh (by a GEMM, or inside the top layer's
  // backward scan). The bf16 tier rounds dl to bf16 on the way into these products; a bf16 copy made
  // once (the same rounding) lets them read half the bytes and the data-gradient GEMM take the
  // load-to-LDS kernel (86 -> 55 us at 262144 rows). The bias gradient sums fp32 dl.
  {
    const void* dlg = b.dl;
    int dlt = PH_F32;
    if (BF) {
      k_f32_to_bf16_k<<<ceil_div(ceil_div(TB * HP, 8), kB), kB, 0, st>>>(b.dl, (uint16_t*)b.dlb, TB * HP);
      PH_LAUNCH_CHECK();
      dlg = b.dlb;
      dlt = PH_BF16;
    }
    // The head's weight and bias gradients only fill G's head block, which nothing reads before the
    // join at the end of the backward: they run on library lane 0 (its own split-K slot) beside the
    // layer backward (and the head's data-gradient GEMM where it runs).
    PH_TRY(lanes.fork(1));
    const hipStream_t lane = lane_stream(0);
    PhGemmDesc g = gd(1, 0, HP, H, (int)TB, dlt, dlg, HP, DT, xL, H, PH_F32, b.gh, H, MATH);
    g.ws_slot = lane_slots(0).gemm_ws;
    PH_TRY(gemm(g, lane));
    PH_TRY(colsum_f32(b.dl, TB, HP, HP, b.gbh, 1.f, 0, lane));
    k_head_scatter<<<64, kB, 0, lane>>>(b.gh, b.gbh, H, A, G + offDec);
    PH_LAUNCH_CHECK();
    if (!top_fused) {
      PhGemmDesc g2 = gd(0, 1, (int)TB, H, HP, dlt, dlg, HP, DT, b.wht, HP, DT, b.dh0, H, MATH);
      PH_TRY(gemm(g2, st));
    }
  }
  // layers backward
  TS* dhn = (TS*)b.dh0;
  TS* dnext = (TS*)b.dh1;  // gradient w.r.t. the layer input, produced by the data-gradient GEMM
  for (int l = L - 1; l >= 0; l--) {
    TS* xl = x + (long)l * TB * H;
    TS* cmb = cmbs + (long)l * TB * 3 * H;
    const bool fused = top_fused && l == L - 1;  // dhn then receives the gate-skip term
    if constexpr (std::is_same_v<TS, uint16_t>) {
      if (fused) {
        const unsigned grid = ceil_div((long)d.B * H / 4, kB);
        const size_t lds = (size_t)(nh <= 16 ? 8 : 9) * H * 4;
        const uint16_t* os_l = os + (long)l * TB * H;
        if (nh <= 16)
          k_scan_bwd_top<8, kScanCh><<<grid, kB, lds, st>>>(cmb, os_l, xl, (const uint16_t*)b.dlb,
                                                            (const uint16_t*)b.wh, nh, dy, dhn, done, d.B, H, d.T);
        else
          k_scan_bwd_top<9, kScanCh><<<grid, kB, lds, st>>>(cmb, os_l, xl, (const uint16_t*)b.dlb,
                                                            (const uint16_t*)b.wh, nh, dy, dhn, done, d.B, H, d.T);
      }
    }
    if (!fused)
      k_scan_bwd<TS><<<ceil_div((long)d.B * H / 4, kB), kB, 0, st>>>(cmb, os + (long)l * TB * H, xl, dhn, dy, done,
                                                                   d.B, H, d.T);
    PH_LAUNCH_CHECK();
    // gW_l = dy^T x_l  -> G
    PhGemmDesc g = gd(1, 0, 3 * H, H, (int)TB, DT, dy, 3 * H, DT, xl, H, PH_F32,
                      G + offW + (long)l * szL, H, MATH);
    PH_TRY(gemm(g, st));
    // dh_in = dy W_l + dhn (1 - sigm(proj))   (W_l^T stored [H][3H]; proj = third block of cmb)
    PhGemmDesc g2 =
        gd(0, 1, (int)TB, H, 3 * H, DT, dy, 3 * H, DT, wlt + l * szL, 3 * H, DT, dnext, H, MATH);
    if (fused) {
      g2.epi = PH_EPI_AXPBY; g2.aux = dhn; g2.ldaux = H; g2.beta = 1.f;  // + dh (1 - sigm(proj)) from the scan
    } else {
      g2.epi = kEpiGateSkip; g2.aux = dhn; g2.ldaux = H; g2.aux2 = cmb + 2 * H; g2.ldaux2 = 3 * H;
    }
    PH_TRY(gemm(g2, st));
    TS* t = dhn; dhn = dnext; dnext = t;
  }
  // encoder backward. bf16: one product dh^T [obs | 1 | 0] gives gWEnc and, in its column D, gbEnc
  // (one pass over dh); then the main stream waits for the head's work on lane 0.
  if (BF) {
    PhGemmDesc g = gd(1, 0, H, D + 8, (int)TB, DT, dhn, H, DT, obsg, ldo, PH_F32, b.genc, D + 8, MATH);
    PH_TRY(gemm(g, st));
    k_enc_scatter<<<ceil_div((long)H * (D + 1), kB), kB, 0, st>>>(b.genc, H, D, G, G + offBEnc);
    PH_LAUNCH_CHECK();
    return lanes.join();
  }
  // fp32: gbEnc = colsum(dh) on lane 0 (after the head's work queued there) beside gWEnc = dh^T obs
  // on the main stream; then the main stream waits for the lane
  PH_TRY(lanes.fork(1));
  const hipStream_t lane = lane_stream(0);
  PH_TRY(colsum_f32((const float*)dhn, TB, H, H, G + offBEnc, 1.f, 0, lane));
  {
    PhGemmDesc g = gd(1, 0, H, D, (int)TB, DT, dhn, H, DT, obsg, ldo, PH_F32, G, D, MATH);
    PH_TRY(gemm(g, st));
  }
  return lanes.join();
}

}  // namespace

long mingru_param_count(const ph_mingru_dims& d) {
  return (long)d.H * d.D + d.H + (long)d.L * 3 * d.H * d.H + (long)d.A * d.H + d.A + d.H + 1;
}

int mingru_ppo_grad(const ph_mingru_dims& d, const ph_ppo_coefs& c, const HeadSizes* heads, const float* params,
                    const float* obs, const int* act, const float* advn, const float* ret,
                    const float* oldlp, const float* oldval, const float* done, float* G,
                    float* newlp, float* newval, double* losses, hipStream_t st, bool join_lane0) {
  PH_REQUIRE(d.B > 0 && d.T > 0 && d.D > 0 && d.H > 0 && d.L > 0 && d.A > 0, "mingru: empty dims");
  PH_REQUIRE(d.A + 1 <= HP, "mingru: at most %d actions", HP - 1);
  PH_REQUIRE(d.H % 8 == 0 && d.D % 8 == 0, "mingru: hidden and obs sizes must be multiples of 8");
  PH_REQUIRE(d.precision == 0 || d.precision == 1, "mingru: precision must be 0 (bf16) or 1 (fp32)");
  PH_REQUIRE(d.L <= kLanes - 3, "mingru: at most %d layers", kLanes - 3);
  PH_REQUIRE((long)d.T * d.B <= INT32_MAX, "mingru: T*B exceeds int32");
  if (heads) {
    int W = 0;
    for (int h = 0; h < heads->K; h++) W += heads->n[h];
    PH_REQUIRE(heads->K >= 1 && heads->K <= kMaxHeads && W == d.A,
               "mingru: %d head sizes summing to %d for %d logits", heads->K, W, d.A);
  }
  if (d.precision == 1)
    return mingru_ppo_grad_t<float>(d, c, heads, params, obs, act, advn, ret, oldlp, oldval, done, G, newlp,
                                    newval, losses, st, join_lane0);
  return mingru_ppo_grad_t<uint16_t>(d, c, heads, params, obs, act, advn, ret, oldlp, oldval, done, G, newlp,
                                     newval, losses, st, join_lane0);
}

// Clip the summed gradient and apply Muon to every matrix (fp32 master weights), stepvec to biases.
// The matrices' Newton-Schulz iterations run together in one fused launch.
int mingru_muon(const ph_mingru_dims& d, const ph_muon_coefs& m, float* params, float* mom, float* G,
                hipStream_t st) {
  const int H = d.H, D = d.D, L = d.L, A = d.A;
  const long P = mingru_param_count(d);
  PH_TRY(gclip_f32(G, P, m.gscale, m.max_grad_norm, st));
  const long szE = (long)H * D, szL = 3L * H * H;
  const long offBEnc = szE, offW = szE + H, offDec = offW + (long)L * szL, offBDec = offDec + (long)A * H,
             offVal = offBDec + A, offBVal = offVal + H;
  PH_REQUIRE(L + 3 <= kNsMaxMats, "mingru: at most %d layers", kNsMaxMats - 3);
  MuonMat mats[kNsMaxMats];
  int nm = 0;
  auto mat = [&](long off, int rows, int cols) {
    mats[nm++] = MuonMat{params + off, G + off, mom + off, rows, cols};
  };
  mat(0, H, D);
  for (int l = 0; l < L; l++) mat(offW + l * szL, 3 * H, H);
  mat(offDec, A, H);
  mat(offVal, 1, H);
  auto vec = [&](long off, long n) { return StepVec{params + off, G + off, mom + off, n}; };
  const StepVec vecs[3] = {vec(offBEnc, H), vec(offBDec, A), vec(offBVal, 1)};
  PH_TRY(stepvec_f32_batch(vecs, 3, 1.f, m.lr, m.wd, m.mu, st));
  return muon_fast_batch(mats, nm, 1.f, m.lr, m.wd, m.mu, m.eps, m.coeffs, m.nsteps, m.math, st);
}

int mingru_step(const ph_mingru_dims& d, const ph_ppo_coefs& c, const ph_muon_coefs& m,
                float* params, float* mom, const float* obs, const int* act, const float* oldlp,
                const float* oldval, const float* rew, const float* done, const float* logrho,
                const float* boot, float* G, double* losses, hipStream_t st) {
  const long TB = (long)d.T * d.B;
  Bufs b;
  PH_TRY(get_bufs(d, b, st));
  // V-trace (bootstrapped variant, time-major) on the behaviour values, targets = adv + V, and the
  // minibatch advantage normalisation: on lane 0 beside the forward pass, which does not need them
  // (the gradient joins the lane before its loss)
  LaneJoin lanes(st);
  PH_TRY(lanes.fork(1));
  const hipStream_t lane = lane_stream(0);
  PH_TRY(vtrace_f32(rew, oldval, done, logrho, boot, d.B, d.T, 1, 1, logrho != nullptr, 1, c.gamma,
                    c.lam, c.rho_clip, c.c_clip, b.adv, b.tgt, lane));
  PH_TRY(moments_normalize(PH_F32, b.adv, TB, b.advn, b.stats, lane));
  PH_TRY(mingru_ppo_grad(d, c, nullptr, params, obs, act, b.advn, b.tgt, oldlp, oldval, done, G, b.newlp,
                         b.newval, losses, st, true));
  lanes.joined();  // the gradient joined lane 0 before its loss
  PH_TRY(mingru_muon(d, m, params, mom, G, st));
  return PH_OK;
}

}  // namespace ph

using namespace ph;

extern "C" long ph_mingru_param_count(const ph_mingru_dims* d) { return d ? mingru_param_count(*d) : -1; }

extern "C" int ph_mingru_ppo_grad(const ph_mingru_dims* d, const ph_ppo_coefs* c, const float* params,
                                  const float* obs, const int* act, const float* adv, const float* ret,
                                  const float* oldlp, const float* oldval, const float* done, float* G,
                                  float* newlp, float* newval, double* losses, void* stream) {
  PH_REQUIRE(d && c, "ph_mingru_ppo_grad: null config");
  return mingru_ppo_grad(*d, *c, nullptr, params, obs, act, adv, ret, oldlp, oldval, done, G, newlp, newval,
                         losses, as_stream(stream), false);
}

extern "C" int ph_mingru_ppo_grad_md(const ph_mingru_dims* d, const ph_ppo_coefs* c, const int* head_sizes,
                                     size_t K, const float* params, const float* obs, const int* act,
                                     const float* adv, const float* ret, const float* oldlp, const float* oldval,
                                     const float* done, float* G, float* newlp, float* newval, double* losses,
                                     void* stream) {
  PH_REQUIRE(d && c && head_sizes, "ph_mingru_ppo_grad_md: null config");
  PH_REQUIRE(K >= 1 && K <= (size_t)kMaxHeads, "ph_mingru_ppo_grad_md: K=%zu heads (1..%d)", K, kMaxHeads);
  HeadSizes hs;
  hs.K = (int)K;
  for (size_t h = 0; h < K; h++) {
    PH_REQUIRE(head_sizes[h] >= 1, "ph_mingru_ppo_grad_md: head %zu has %d actions", h, head_sizes[h]);
    hs.n[h] = head_sizes[h];
  }
  return mingru_ppo_grad(*d, *c, &hs, params, obs, act, adv, ret, oldlp, oldval, done, G, newlp, newval, losses,
                         as_stream(stream), false);
}

extern "C" int ph_mingru_muon(const ph_mingru_dims* d, const ph_muon_coefs* m, float* params,
                              float* mom, float* G, void* stream) {
  PH_REQUIRE(d && m, "ph_mingru_muon: null config");
  return mingru_muon(*d, *m, params, mom, G, as_stream(stream));
}

extern "C" int ph_mingru_step(const ph_mingru_dims* d, const ph_ppo_coefs* c, const ph_muon_coefs* m,
                              float* params, float* mom, const float* obs, const int* act,
                              const float* oldlp, const float* oldval, const float* rew,
                              const float* done, const float* logrho, const float* boot, float* G,
                              double* losses, void* stream) {
  PH_REQUIRE(d && c && m, "ph_mingru_step: null config");
  return mingru_step(*d, *c, *m, params, mom, obs, act, oldlp, oldval, rew, done, logrho, boot, G,
                     losses, as_stream(stream));
}
