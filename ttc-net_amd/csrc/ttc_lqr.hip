// ttc_lqr.hip -- gfx950 kernels + C ABI for TTC-Net's batched receding-horizon LQR solve.
//
// Problem (one per token n and head h, P = N*H problems), restating
// ttc/solvers/torch_lqr.py:65-91 and ttc/solvers/lin_solver_lqr.py:113-212:
//   A_k  = diag(1 + a*exp(lgA*(k+1)))       B_k = B diag(exp(lgB*(k+1)))
//   Qc_k = diag(exp(lgQ*k)) Q diag(exp(lgQ*k)) (k >= 1)   R = diag(1/R_inv)
//   V_T = Q_f ;  for k = T-1..0:
//     W = V B_k,  Quu = R + B_k'W,  Qux = W'A_k,  K_k = -Quu^{-1} Qux,
//     V <- A_k V A_k + Qux' K_k + Qc_k
//   u0 = K_0 h0.
//
// Layout: one problem per D lanes of a wave (D = d = du in {16,32,64}); lane i owns
// row i of every D x D matrix (V, W, the augmented [Quu | Qux] row, gradient rows).
// Cross-lane traffic goes through wave-private LDS (write a row, read broadcast
// rows back) -- no workgroup barriers inside the time loop.  The token-shared B is
// staged once per block into LDS.  Gains are computed by Gauss-Jordan elimination
// with partial pivoting: Quu is SPD in exact arithmetic, but on long-horizon stress
// inputs fp32 rounding can make it indefinite, where Cholesky / unpivoted LDL' break
// down while pivoted elimination (what torch.linalg.solve does in the reference)
// stays accurate.
//
// Backward (gradients of sum(d_u * u0)): implicit differentiation of the KKT system
// (ttc/solvers/torch_lqr.py:34-63).  Primal and adjoint trajectories are rolled out
// with the stored gains, and costates are swept back with the closed-loop recursion
//   lambda_k = Qc_k h_k + A_k lambda_{k+1} + K_k'(R u_k + B_k' lambda_{k+1}),
// (the reference's open-loop recursion plus a term that is zero at the optimum),
// which is stable where the open-loop one amplifies rounding by prod(A_k).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ttc_lqr.h"

#define TTC_LQR_VERSION_STRING "ttc-lqr-gfx950 0.1.0"

namespace ttc {

constexpr int kPad = 4;  // LDS row padding (floats): keeps rows 16-byte aligned, staggers banks

template <int D>
struct Geo {
  static constexpr int PPB = (D == 16) ? 16 : (D == 32 ? 4 : 1);  // problems per block
  static constexpr int THREADS = PPB * D;
  static constexpr int LDM = D + kPad;                  // LDS row stride
  static constexpr int MAT = D * LDM;
  static constexpr int NVEC = 12;                       // D-float vector slots per problem
  static constexpr int PER_PROB = MAT + NVEC * D + 4;   // +4 floats: bank skew between problems
};

// Order LDS traffic between lanes of one wave: stores before this point are
// visible to loads after it (LDS executes one wave's requests in order).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int N>
__device__ __forceinline__ void ld_row(const float* s, float (&out)[N]) {
  static_assert(N % 4 == 0, "row length");
#pragma unroll
  for (int c = 0; c < N; c += 4) {
    const float4 v = *reinterpret_cast<const float4*>(s + c);
    out[c] = v.x; out[c + 1] = v.y; out[c + 2] = v.z; out[c + 3] = v.w;
  }
}

template <int N>
__device__ __forceinline__ void st_row(float* s, const float (&in)[N]) {
#pragma unroll
  for (int c = 0; c < N; c += 4)
    *reinterpret_cast<float4*>(s + c) = make_float4(in[c], in[c + 1], in[c + 2], in[c + 3]);
}

template <int N>
__device__ __forceinline__ void ld_global_row(const float* __restrict__ g, float (&out)[N]) {
#pragma unroll
  for (int c = 0; c < N; c += 4) {
    const float4 v = *reinterpret_cast<const float4*>(g + c);
    out[c] = v.x; out[c + 1] = v.y; out[c + 2] = v.z; out[c + 3] = v.w;
  }
}

template <int N>
__device__ __forceinline__ void st_global_row(float* __restrict__ g, const float (&in)[N]) {
#pragma unroll
  for (int c = 0; c < N; c += 4)
    *reinterpret_cast<float4*>(g + c) = make_float4(in[c], in[c + 1], in[c + 2], in[c + 3]);
}

// Max of a 32-bit key over the D lanes of a problem (all lanes get the result).
template <int N>
__device__ __forceinline__ unsigned ror16(unsigned v) {
  return __builtin_amdgcn_mov_dpp(v, 0x120 + N, 0xF, 0xF, false);  // row_ror:N
}
template <int D>
__device__ __forceinline__ unsigned group_max_u32(unsigned k) {
  k = max(k, ror16<8>(k));
  k = max(k, ror16<4>(k));
  k = max(k, ror16<2>(k));
  k = max(k, ror16<1>(k));
  if constexpr (D >= 32) k = max(k, (unsigned)__shfl_xor((int)k, 16, 64));
  if constexpr (D >= 64) k = max(k, (unsigned)__shfl_xor((int)k, 32, 64));
  return k;
}

template <int D>
__device__ __forceinline__ float group_sum(float v, float* scratch, int li) {
  // via LDS: every lane writes, everyone reads the D values
  wave_sync();
  scratch[li] = v;
  wave_sync();
  float vals[D];
  ld_row<D>(scratch, vals);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < D; ++c) s += vals[c];
  return s;
}

// In-place Gauss-Jordan elimination with partial pivoting on the D x D left block
// of the augmented rows `aug` (lane li owns row li, width W >= D).  On return the
// lane with pivot position `pos` holds row `pos` of (left^{-1} * right) scaled by
// `mypiv` (divide by it).  `prow` is W floats of this problem's LDS.
template <int D, int W>
__device__ __forceinline__ void gauss_jordan(float (&aug)[W], int li, float* prow, float& mypiv, int& pos) {
  constexpr unsigned kIdxBits = (D == 16) ? 4u : (D == 32 ? 5u : 6u);
  constexpr unsigned kIdxMask = (1u << kIdxBits) - 1u;
  bool done = false;
  mypiv = 1.f;
  pos = 0;
#pragma unroll
  for (int k = 0; k < D; ++k) {
    // pivot = largest |aug[k]| among rows not yet used; ties -> lowest lane.
    // Key = magnitude bits with the low mantissa bits replaced by (D-1-lane).
    const unsigned mag = __float_as_uint(fabsf(aug[k]));
    const unsigned key = done ? 0u : ((mag & ~kIdxMask) | (unsigned)(D - 1 - li));
    const unsigned best = group_max_u32<D>(key);
    const int who = D - 1 - (int)(best & kIdxMask);
    const bool me = (who == li);
    if (me) {
#pragma unroll
      for (int c = (k & ~3); c < W; c += 4)
        *reinterpret_cast<float4*>(prow + c) = make_float4(aug[c], aug[c + 1], aug[c + 2], aug[c + 3]);
    }
    wave_sync();
    float pr[W];
#pragma unroll
    for (int c = (k & ~3); c < W; c += 4) {
      const float4 v = *reinterpret_cast<const float4*>(prow + c);
      pr[c] = v.x; pr[c + 1] = v.y; pr[c + 2] = v.z; pr[c + 3] = v.w;
    }
    const float inv = 1.0f / pr[k];
    const float f = me ? 0.f : aug[k] * inv;
#pragma unroll
    for (int c = k + 1; c < W; ++c) aug[c] = fmaf(-f, pr[c], aug[c]);
    if (me) { mypiv = pr[k]; pos = k; done = true; }
    wave_sync();  // next pivot row may overwrite prow
  }
}

// ---------------------------------------------------------------------------
// Forward kernel: Riccati sweep, u0, optional gain stash.
// ---------------------------------------------------------------------------
template <int D, bool STASH, bool WRITE_U>
__global__ __launch_bounds__(Geo<D>::THREADS) void lqr_fwd_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, int ntok_lds, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status) {
  using G = Geo<D>;
  extern __shared__ float smem[];
  const int li = threadIdx.x % D;
  const int pb = threadIdx.x / D;
  const int64_t p0 = (int64_t)blockIdx.x * G::PPB;
  int64_t p = p0 + pb;
  const bool valid = p < P;
  if (!valid) p = P - 1;  // idle lanes recompute a real problem, never store
  const int64_t n = p / H;
  const int64_t n0 = p0 / H;

  // stage the block's token-shared B matrices in LDS
  {
    const int64_t plast = (p0 + G::PPB - 1 < P) ? (p0 + G::PPB - 1) : (P - 1);
    const int ntok = (int)(plast / H - n0 + 1);
    for (int e = threadIdx.x; e < ntok * D * D; e += G::THREADS) {
      const int tk = e / (D * D), rem = e % (D * D);
      smem[(tk * D + rem / D) * G::LDM + rem % D] = Bg[(n0 + tk) * D * D + rem];
    }
  }
  __syncthreads();
  const float* Bs = smem + (int)(n - n0) * G::MAT;
  float* S = smem + ntok_lds * G::MAT + pb * G::PER_PROB;
  float* mat = S;
  float* vb = S + G::MAT;
  float* va = vb + D;
  float* vx = va + D;
  float* prow = vx + D;  // 2D floats

  const float a_i = A_diag[p * D + li];
  const float rr_i = 1.0f / Rinv[p * D + li];
  const float lgB_i = lgB[p * D + li];
  const float lgQ_i = lgQ[p * D + li];
  const float lgA_p = lgA[p];

  float V[D], Bcol[D], Qrow[D];
  {
    const float* qf = Qf + p * D * D;
    const float* qg = Qg + n * D * D;
#pragma unroll
    for (int c = 0; c < D; ++c) {
      V[c] = 0.5f * (qf[li * D + c] + qf[c * D + li]);
      Qrow[c] = 0.5f * (qg[li * D + c] + qg[c * D + li]);
      Bcol[c] = Bs[c * G::LDM + li];
    }
  }
  for (int t = T - 1; t >= 0; --t) {
    const float tp1 = (float)(t + 1);
    const float eA = expf(lgA_p * tp1);
    const float beta_i = expf(lgB_i * tp1);
    const float alpha_i = fmaf(a_i, eA, 1.0f);
    const float q_i = (t > 0) ? expf(lgQ_i * (float)t) : 0.f;

    // W~ = V B (row li)
    float w[D];
#pragma unroll
    for (int k = 0; k < D; ++k) w[k] = 0.f;
#pragma unroll
    for (int m = 0; m < D; ++m) {
      float brow[D];
      ld_row<D>(Bs + m * G::LDM, brow);
#pragma unroll
      for (int k = 0; k < D; ++k) w[k] = fmaf(V[m], brow[k], w[k]);
    }
    wave_sync();
    vb[li] = beta_i;
    va[li] = alpha_i;
    wave_sync();
    float beta[D], alpha[D];
    ld_row<D>(vb, beta);
    ld_row<D>(va, alpha);
#pragma unroll
    for (int k = 0; k < D; ++k) w[k] *= beta[k];  // W = V B_k
    st_row<D>(mat + li * G::LDM, w);
    wave_sync();

    // augmented row li: [Quu_li | Qux_li],  Quu = B_k'W + R,  Qux_lc = W_cl * alpha_c
    float aug[2 * D];
#pragma unroll
    for (int k = 0; k < D; ++k) aug[k] = 0.f;
#pragma unroll
    for (int m = 0; m < D; ++m) {
      float wrow[D];
      ld_row<D>(mat + m * G::LDM, wrow);
#pragma unroll
      for (int k = 0; k < D; ++k) aug[k] = fmaf(Bcol[m], wrow[k], aug[k]);
    }
#pragma unroll
    for (int k = 0; k < D; ++k) aug[k] = aug[k] * beta_i + ((k == li) ? rr_i : 0.f);
#pragma unroll
    for (int c = 0; c < D; ++c) aug[D + c] = mat[c * G::LDM + li] * alpha[c];
    if (STASH && t == 0) {
      float qrow[D];
#pragma unroll
      for (int k = 0; k < D; ++k) qrow[k] = aug[k];
      if (valid) st_global_row<D>(q0stash + (p * D + li) * D, qrow);
    }

    float mypiv;
    int pos;
    gauss_jordan<D, 2 * D>(aug, li, prow, mypiv, pos);
    float x[D];  // row `pos` of X = Quu^{-1} Qux  (K = -X)
    const float ipiv = 1.0f / mypiv;
#pragma unroll
    for (int c = 0; c < D; ++c) x[c] = aug[D + c] * ipiv;
    if (STASH && valid) {
      float krow[D];
#pragma unroll
      for (int c = 0; c < D; ++c) krow[c] = -x[c];
      st_global_row<D>(kstash + (((int64_t)p * T + t) * D + pos) * D, krow);
    }
    if (t == 0) {
      // u0[pos] = K_0[pos,:] . h0
      float hv[D];
      wave_sync();
      vx[li] = h0[p * D + li];
      wave_sync();
      ld_row<D>(vx, hv);
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < D; ++c) s = fmaf(x[c], hv[c], s);
      const float u0 = -s;
      if (WRITE_U && valid) u_out[p * D + pos] = u0;
      if (status != nullptr && valid && !isfinite(u0)) atomicOr(status, TTC_LQR_STATUS_NONFINITE);
      break;  // V_0 is not needed
    }
    // all lanes finished reading W during the elimination; publish X rows by position
    st_row<D>(mat + pos * G::LDM, x);
    wave_sync();
    // V <- alpha_i (alpha_m V_im - sum_j W_ij X_jm) + q_i q_m Q_im
    float acc[D];
#pragma unroll
    for (int m = 0; m < D; ++m) acc[m] = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float xrow[D];
      ld_row<D>(mat + j * G::LDM, xrow);
#pragma unroll
      for (int m = 0; m < D; ++m) acc[m] = fmaf(w[j], xrow[m], acc[m]);
    }
    float qv[D];
    vx[li] = q_i;
    wave_sync();
    ld_row<D>(vx, qv);
#pragma unroll
    for (int m = 0; m < D; ++m)
      V[m] = fmaf(alpha_i, fmaf(alpha[m], V[m], -acc[m]), (q_i * qv[m]) * Qrow[m]);
    // symmetrise: V_im = (V_im + V_mi) / 2
    wave_sync();
    st_row<D>(mat + li * G::LDM, V);
    wave_sync();
#pragma unroll
    for (int m = 0; m < D; ++m) V[m] = 0.5f * (V[m] + mat[m * G::LDM + li]);
    wave_sync();
  }
}


// ---------------------------------------------------------------------------
// Backward kernel: adjoint feed-forward, closed-loop rollouts of the primal and
// adjoint trajectories (forward in time, into `traj`), then the reverse costate
// sweep with all gradient accumulations.  grad_B / grad_Q are written per problem
// into gBp / gQp and summed over heads by headsum_kernel.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void flag_value(float v, float limit, int& flags) {
  if (!isfinite(v)) flags |= TTC_LQR_STATUS_NONFINITE;
  else if (fabsf(v) >= limit) flags |= TTC_LQR_STATUS_LARGE;
}

template <int D>
__global__ __launch_bounds__(Geo<D>::THREADS) void lqr_bwd_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    const float* __restrict__ dU, const float* __restrict__ kstash, const float* __restrict__ q0stash,
    int64_t P, int H, int T, int ntok_lds, float4* __restrict__ traj, float* __restrict__ gA,
    float* __restrict__ gRinv, float* __restrict__ gQf, float* __restrict__ glgA,
    float* __restrict__ glgB, float* __restrict__ glgQ, float* __restrict__ gh0,
    float* __restrict__ gBp, float* __restrict__ gQp, float grad_limit, int* __restrict__ status) {
  using G = Geo<D>;
  extern __shared__ float smem[];
  const int li = threadIdx.x % D;
  const int pb = threadIdx.x / D;
  const int64_t p0 = (int64_t)blockIdx.x * G::PPB;
  int64_t p = p0 + pb;
  const bool valid = p < P;
  if (!valid) p = P - 1;
  const int64_t n = p / H;
  const int64_t n0 = p0 / H;
  {
    const int64_t plast = (p0 + G::PPB - 1 < P) ? (p0 + G::PPB - 1) : (P - 1);
    const int ntok = (int)(plast / H - n0 + 1);
    for (int e = threadIdx.x; e < ntok * D * D; e += G::THREADS) {
      const int tk = e / (D * D), rem = e % (D * D);
      smem[(tk * D + rem / D) * G::LDM + rem % D] = Bg[(n0 + tk) * D * D + rem];
    }
  }
  __syncthreads();
  const float* Bs = smem + (int)(n - n0) * G::MAT;
  float* S = smem + ntok_lds * G::MAT + pb * G::PER_PROB;
  float* v0 = S + G::MAT;     // 8 vectors of D floats
  float* v1 = v0 + D;
  float* v2 = v1 + D;
  float* v3 = v2 + D;
  float* v4 = v3 + D;
  float* v5 = v4 + D;
  float* v6 = v5 + D;
  float* v7 = v6 + D;
  float* prow = v7 + D;       // D + 4 floats

  const float a_i = A_diag[p * D + li];
  const float rr_i = 1.0f / Rinv[p * D + li];
  const float lgB_i = lgB[p * D + li];
  const float lgQ_i = lgQ[p * D + li];
  const float lgA_p = lgA[p];
  float Brow[D], Bcol[D], Qrow[D];
  {
    const float* qg = Qg + n * D * D;
#pragma unroll
    for (int c = 0; c < D; ++c) {
      Brow[c] = Bs[li * G::LDM + c];
      Bcol[c] = Bs[c * G::LDM + li];
      Qrow[c] = 0.5f * (qg[li * D + c] + qg[c * D + li]);
    }
  }

  // adjoint feed-forward at t = 0: w0 = -Quu_0^{-1} d_u
  float w0_i;
  {
    float aug[D + 4];
    ld_global_row<D>(q0stash + (p * D + li) * D, *reinterpret_cast<float(*)[D]>(aug));
    aug[D] = dU[p * D + li];
    aug[D + 1] = aug[D + 2] = aug[D + 3] = 0.f;
    float piv;
    int pos;
    gauss_jordan<D, D + 4>(aug, li, prow, piv, pos);
    v0[pos] = -aug[D] / piv;
    wave_sync();
    w0_i = v0[li];
    wave_sync();
  }

  // phase 1: rollouts, t = 0..T-1
  float h_i = h0[p * D + li];
  float hb_i = 0.f;
  for (int t = 0; t < T; ++t) {
    const float tp1 = (float)(t + 1);
    const float alpha_i = fmaf(a_i, expf(lgA_p * tp1), 1.0f);
    const float beta_i = expf(lgB_i * tp1);
    v0[li] = h_i;
    v1[li] = hb_i;
    wave_sync();
    float hv[D], hbv[D], krow[D];
    ld_row<D>(v0, hv);
    ld_row<D>(v1, hbv);
    ld_global_row<D>(kstash + (((int64_t)p * T + t) * D + li) * D, krow);
    float u_i = 0.f, w_i = (t == 0) ? w0_i : 0.f;
#pragma unroll
    for (int c = 0; c < D; ++c) {
      u_i = fmaf(krow[c], hv[c], u_i);
      w_i = fmaf(krow[c], hbv[c], w_i);
    }
    v2[li] = beta_i * u_i;
    v3[li] = beta_i * w_i;
    wave_sync();
    float bu[D], bw[D];
    ld_row<D>(v2, bu);
    ld_row<D>(v3, bw);
    float hn = alpha_i * h_i, hbn = alpha_i * hb_i;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      hn = fmaf(Brow[j], bu[j], hn);
      hbn = fmaf(Brow[j], bw[j], hbn);
    }
    if (valid) traj[((int64_t)p * T + t) * D + li] = make_float4(h_i, hb_i, u_i, w_i);
    h_i = hn;
    hb_i = hbn;
    wave_sync();
  }

  // phase 2: costates lambda_{t+1}, gradients, t = T-1..0
  int flags = 0;
  float lam_i, lamb_i;
  {
    v0[li] = h_i;
    v1[li] = hb_i;
    wave_sync();
    float hv[D], hbv[D], qf[D], gq[D];
    ld_row<D>(v0, hv);
    ld_row<D>(v1, hbv);
    const float* qfp = Qf + p * D * D;
    lam_i = 0.f;
    lamb_i = 0.f;
#pragma unroll
    for (int c = 0; c < D; ++c) {
      qf[c] = 0.5f * (qfp[li * D + c] + qfp[c * D + li]);
      lam_i = fmaf(qf[c], hv[c], lam_i);
      lamb_i = fmaf(qf[c], hbv[c], lamb_i);
      gq[c] = 0.5f * (h_i * hbv[c] + hb_i * hv[c]);
      flag_value<D>(gq[c], grad_limit, flags);
    }
    if (valid) st_global_row<D>(gQf + (p * D + li) * D, gq);
    wave_sync();
  }
  float gA_i = 0.f, glgA_part = 0.f, glgB_i = 0.f, gr_i = 0.f, glgQ_i = 0.f, gh0_i = 0.f;
  float gBrow[D], gQrow[D];
#pragma unroll
  for (int c = 0; c < D; ++c) { gBrow[c] = 0.f; gQrow[c] = 0.f; }

  for (int t = T - 1; t >= 0; --t) {
    const float4 tr = traj[((int64_t)p * T + t) * D + li];
    const float h_t = tr.x, hb_t = tr.y, u_i = tr.z, w_i = tr.w;
    const float tp1 = (float)(t + 1);
    const float eA = expf(lgA_p * tp1);
    const float alpha_i = fmaf(a_i, eA, 1.0f);
    const float beta_i = expf(lgB_i * tp1);
    // A: d/dA_t,i = h_t,i lamb_{t+1},i + hb_t,i lam_{t+1},i   (torch_lqr.py:51)
    const float gAt = fmaf(h_t, lamb_i, hb_t * lam_i);
    gA_i = fmaf(gAt, eA, gA_i);
    glgA_part = fmaf(gAt * a_i, tp1 * eA, glgA_part);
    v0[li] = lam_i;
    v1[li] = lamb_i;
    v2[li] = beta_i * u_i;
    v3[li] = beta_i * w_i;
    wave_sync();
    float lv[D], lbv[D], bu[D], bw[D];
    ld_row<D>(v0, lv);
    ld_row<D>(v1, lbv);
    ld_row<D>(v2, bu);
    ld_row<D>(v3, bw);
    // B: lamb u' + lam w' (torch_lqr.py:53), chained through B_t = B diag(beta_t)
    float btl = 0.f, btlb = 0.f;
#pragma unroll
    for (int c = 0; c < D; ++c) {
      gBrow[c] = fmaf(lamb_i, bu[c], fmaf(lam_i, bw[c], gBrow[c]));
      btl = fmaf(Bcol[c], lv[c], btl);
      btlb = fmaf(Bcol[c], lbv[c], btlb);
    }
    glgB_i = fmaf(tp1 * beta_i, fmaf(u_i, btlb, w_i * btl), glgB_i);
    // R = 1/R_inv:  d/dR_inv = -(u w) / R_inv^2   (torch_lqr.py:59)
    gr_i = fmaf(-u_i * w_i, rr_i * rr_i, gr_i);
    if (t >= 1) {
      const float q_i = expf(lgQ_i * (float)t);
      // closed-loop correction c = R u + B_t' lambda_{t+1}
      v4[li] = q_i * h_t;
      v5[li] = q_i * hb_t;
      v6[li] = fmaf(u_i, rr_i, beta_i * btl);
      v7[li] = fmaf(w_i, rr_i, beta_i * btlb);
      wave_sync();
      float qh[D], qhb[D], cu[D], cw[D];
      ld_row<D>(v4, qh);
      ld_row<D>(v5, qhb);
      ld_row<D>(v6, cu);
      ld_row<D>(v7, cw);
      float Qh = 0.f, Qhb = 0.f, kcu = 0.f, kcw = 0.f;
      const float* kp = kstash + (((int64_t)p * T + t) * D) * D + li;
#pragma unroll
      for (int c = 0; c < D; ++c) {
        Qh = fmaf(Qrow[c], qh[c], Qh);
        Qhb = fmaf(Qrow[c], qhb[c], Qhb);
        // Q_t = D_t Q D_t:  gradient D_t sym(h hb') D_t  (torch_lqr.py:55)
        gQrow[c] = fmaf(0.5f * q_i, fmaf(h_t, qhb[c], hb_t * qh[c]), gQrow[c]);
        const float kji = kp[c * D];  // K_t[c, li]
        kcu = fmaf(kji, cu[c], kcu);
        kcw = fmaf(kji, cw[c], kcw);
      }
      Qh *= q_i;
      Qhb *= q_i;
      glgQ_i = fmaf((float)t, fmaf(h_t, Qhb, hb_t * Qh), glgQ_i);
      lam_i = Qh + fmaf(alpha_i, lam_i, kcu);
      lamb_i = Qhb + fmaf(alpha_i, lamb_i, kcw);
    } else {
      gh0_i = alpha_i * lamb_i;  // torch_lqr.py:61 (lambda_0 = A_0' lambda_1)
    }
    wave_sync();
  }
  const float glgA_p = group_sum<D>(glgA_part, v0, li);
  flag_value<D>(gA_i, grad_limit, flags);
  flag_value<D>(glgB_i, grad_limit, flags);
  flag_value<D>(gr_i, grad_limit, flags);
  flag_value<D>(glgQ_i, grad_limit, flags);
  flag_value<D>(gh0_i, grad_limit, flags);
  flag_value<D>(glgA_p, grad_limit, flags);
  if (valid) {
    gA[p * D + li] = gA_i;
    gRinv[p * D + li] = gr_i;
    glgB[p * D + li] = glgB_i;
    glgQ[p * D + li] = glgQ_i;
    gh0[p * D + li] = gh0_i;
    if (li == 0) glgA[p] = glgA_p;
    st_global_row<D>(gBp + (p * D + li) * D, gBrow);
    st_global_row<D>(gQp + (p * D + li) * D, gQrow);
    if (flags && status != nullptr) atomicOr(status, flags);
  }
}

// grad_B / grad_Q: sum the per-problem partials over the H heads of each token.
__global__ void headsum_kernel(const float* __restrict__ part, int64_t N, int H, int DD,
                               float* __restrict__ out, float grad_limit, int* __restrict__ status) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * DD) return;
  const int64_t n = e / DD;
  const int r = (int)(e % DD);
  float s = 0.f;
  for (int h = 0; h < H; ++h) s += part[(n * H + h) * DD + r];
  out[e] = s;
  if (status != nullptr) {
    if (!isfinite(s)) atomicOr(status, TTC_LQR_STATUS_NONFINITE);
    else if (fabsf(s) >= grad_limit) atomicOr(status, TTC_LQR_STATUS_LARGE);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
template <int D>
static int ntok_lds_for(int H) {
  constexpr int PPB = Geo<D>::PPB;
  const int span = (PPB - 1) / H + 2;
  return span < PPB ? span : PPB;
}

template <int D>
static size_t lds_bytes(int H) {
  return sizeof(float) * ((size_t)ntok_lds_for<D>(H) * Geo<D>::MAT + (size_t)Geo<D>::PPB * Geo<D>::PER_PROB);
}

template <int D>
static int launch_fwd(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                      int T, float* u, float* kst, float* q0s, int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  const dim3 grid((unsigned)((P + Geo<D>::PPB - 1) / Geo<D>::PPB)), block(Geo<D>::THREADS);
  const size_t sh = lds_bytes<D>(H);
  const int nt = ntok_lds_for<D>(H);
  if (kst != nullptr) {
    if (u != nullptr)
      hipLaunchKernelGGL((lqr_fwd_kernel<D, true, true>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P, H,
                         T, nt, u, kst, q0s, status);
    else
      hipLaunchKernelGGL((lqr_fwd_kernel<D, true, false>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P,
                         H, T, nt, u, kst, q0s, status);
  } else {
    hipLaunchKernelGGL((lqr_fwd_kernel<D, false, true>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P, H,
                       T, nt, u, kst, q0s, status);
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

template <int D>
static int launch_bwd(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                      const float* kst, const float* q0s, int64_t P, int H, int T, float4* traj, float* gA,
                      float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                      float* gQp, float limit, int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  const dim3 grid((unsigned)((P + Geo<D>::PPB - 1) / Geo<D>::PPB)), block(Geo<D>::THREADS);
  hipLaunchKernelGGL((lqr_bwd_kernel<D>), grid, block, lds_bytes<D>(H), s, A, B, Q, R, Qf, lA, lB, lQ, h0, dU,
                     kst, q0s, P, H, T, ntok_lds_for<D>(H), traj, gA, gR, gQf, glA, glB, glQ, gh0, gBp, gQp,
                     limit, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

static int launch_headsum(const float* part, int64_t N, int H, int DD, float* out, float limit, int32_t* status,
                          hipStream_t s) {
  const int64_t total = N * DD;
  if (total <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(headsum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, N, H, DD, out,
                     limit, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct BwdLayout {
  size_t kst, q0s, traj, gBp, gQp, total;
};

static BwdLayout bwd_layout(int64_t chunk_tokens, int H, int d, int T, bool with_stash) {
  const size_t Pc = (size_t)chunk_tokens * (size_t)H;
  BwdLayout L{};
  size_t off = 0;
  L.kst = off;
  off += with_stash ? 0 : align256(Pc * (size_t)T * d * d * sizeof(float));
  L.q0s = off;
  off += with_stash ? 0 : align256(Pc * (size_t)d * d * sizeof(float));
  L.traj = off;
  off += align256(Pc * (size_t)T * d * 4 * sizeof(float));
  L.gBp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.gQp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.total = off;
  return L;
}

}  // namespace ttc

using namespace ttc;

extern "C" {

const char* ttc_lqr_version(void) { return TTC_LQR_VERSION_STRING; }

const char* ttc_lqr_strerror(int code) {
  switch (code) {
    case TTC_LQR_OK: return "ok";
    case TTC_LQR_EINVAL: return "invalid argument (sizes, null pointer or workspace too small)";
    case TTC_LQR_EUNSUPPORTED: return "unsupported (d, du): kernels exist for d == du in {16, 32, 64}";
    case TTC_LQR_ELAUNCH: return "HIP kernel launch failed";
    default: return "unknown error";
  }
}

int ttc_lqr_supported(int32_t d, int32_t du) { return (d == du && (d == 16 || d == 32 || d == 64)) ? 1 : 0; }

size_t ttc_lqr_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0 || T <= 0) return 0;
  const size_t P = (size_t)n_tokens * (size_t)heads;
  return sizeof(float) * P * ((size_t)T * du * d + (size_t)du * du);
}

size_t ttc_lqr_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                               int32_t with_stash) {
  if (chunk_tokens <= 0 || heads <= 0 || d <= 0 || du != d || T <= 0) return 0;
  return bwd_layout(chunk_tokens, heads, d, T, with_stash != 0).total;
}

int ttc_lqr_forward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                    const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                    int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, float* u, float* gain_stash,
                    float* quu0_stash, int32_t* status, void* stream) {
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported(d, du)) return TTC_LQR_EUNSUPPORTED;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !u)
    return TTC_LQR_EINVAL;
  if ((gain_stash == nullptr) != (quu0_stash == nullptr)) return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (d) {
    case 16: return launch_fwd<16>(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s);
    case 32: return launch_fwd<32>(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s);
    case 64: return launch_fwd<64>(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s);
  }
  return TTC_LQR_EUNSUPPORTED;
}

int ttc_lqr_backward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                     const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                     const float* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                     const float* gain_stash, const float* quu0_stash, float* grad_A_diag, float* grad_B,
                     float* grad_Q, float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                     float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, void* workspace,
                     size_t workspace_bytes, float grad_limit, int32_t* status, void* stream) {
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported(d, du)) return TTC_LQR_EUNSUPPORTED;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !d_u ||
      !grad_A_diag || !grad_B || !grad_Q || !grad_R_inv || !grad_Q_f || !grad_log_gamma_A || !grad_log_gamma_B ||
      !grad_log_gamma_Q || !grad_h0 || !workspace)
    return TTC_LQR_EINVAL;
  if ((gain_stash == nullptr) != (quu0_stash == nullptr)) return TTC_LQR_EINVAL;
  const bool with_stash = gain_stash != nullptr;
  const size_t per_token = bwd_layout(1, heads, d, T, with_stash).total;
  if (workspace_bytes < per_token) return TTC_LQR_EINVAL;
  // largest chunk whose layout fits (layout is monotone in the chunk size)
  int64_t chunk = (int64_t)(workspace_bytes / per_token);
  if (chunk > n_tokens) chunk = n_tokens;
  while (chunk > 1 && bwd_layout(chunk, heads, d, T, with_stash).total > workspace_bytes) --chunk;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t dd = (int64_t)d * d;
  for (int64_t n0 = 0; n0 < n_tokens; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * heads, Pc = nc * heads;
    const BwdLayout L = bwd_layout(nc, heads, d, T, with_stash);
    const float* a = A_diag + p0 * d;
    const float* b = B + n0 * dd;
    const float* q = Q + n0 * dd;
    const float* r = R_inv + p0 * du;
    const float* qf = Q_f + p0 * dd;
    const float* la = log_gamma_A + p0;
    const float* lb = log_gamma_B + p0 * du;
    const float* lq = log_gamma_Q + p0 * d;
    const float* hz = h0 + p0 * d;
    const float* dz = d_u + p0 * du;
    float* kst;
    float* q0s;
    int rc = TTC_LQR_OK;
    if (with_stash) {
      kst = const_cast<float*>(gain_stash) + p0 * (int64_t)T * dd;
      q0s = const_cast<float*>(quu0_stash) + p0 * dd;
    } else {
      kst = reinterpret_cast<float*>(ws + L.kst);
      q0s = reinterpret_cast<float*>(ws + L.q0s);
      switch (d) {
        case 16: rc = launch_fwd<16>(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s); break;
        case 32: rc = launch_fwd<32>(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s); break;
        case 64: rc = launch_fwd<64>(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s); break;
      }
      if (rc != TTC_LQR_OK) return rc;
    }
    float4* traj = reinterpret_cast<float4*>(ws + L.traj);
    float* gBp = reinterpret_cast<float*>(ws + L.gBp);
    float* gQp = reinterpret_cast<float*>(ws + L.gQp);
    float* gA = grad_A_diag + p0 * d;
    float* gR = grad_R_inv + p0 * du;
    float* gQf = grad_Q_f + p0 * dd;
    float* glA = grad_log_gamma_A + p0;
    float* glB = grad_log_gamma_B + p0 * du;
    float* glQ = grad_log_gamma_Q + p0 * d;
    float* gh = grad_h0 + p0 * d;
    switch (d) {
      case 16: rc = launch_bwd<16>(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
      case 32: rc = launch_bwd<32>(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
      case 64: rc = launch_bwd<64>(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
    }
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gBp, nc, heads, (int)dd, grad_B + n0 * dd, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gQp, nc, heads, (int)dd, grad_Q + n0 * dd, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
  }
  return TTC_LQR_OK;
}

}  // extern "C"
