// ttc_lqr_mfma16.hpp -- d = du = 16 forward kernel with the per-step products on
// the matrix cores (v_mfma_f32_16x16x4f32).
//
// One wave holds 4 LQR problems (q = 0..3).  The registers carry the negated value
// matrix N = -V (so that no step needs a separate negation).  Per Riccati step and
// problem:
//   B_k = B diag(beta_k)                  4 VALU multiplies (the MFMA operand, scaled)
//   -W = N B_k,  -Quu = B_k'(-W) - R      8 MFMA (-R enters as the accumulator)
//   Cholesky-scaled elimination of -Quu applied to the rows of [-Quu; -W; I]
//     (row layout, fused DPP updates)  ->  -M = -W L^{-T},  U = L^{-T}
//   N + M M' = -(V - W Quu^{-1} W')       4 MFMA (N enters as the accumulator)
//   N <- diag(a) (N + M M') diag(a) - diag(q) Q diag(q)
//   K = -Quu^{-1} Qux = U (-M)' diag(a)   4 MFMA (stored steps and t = 0 only)
// M M' is formed as a product of one operand with itself, so the value matrix stays
// exactly symmetric; an unsymmetric split such as (W L'^{-T} D^{-1})(W L'^{-T})'
// drifts and loses long-horizon stress problems.
//
// On gfx950 the fp32 matrix core and the vector ALU do not overlap (a measured
// property of this part: the time of a loop is the sum of both), so the design
// minimises vector instructions: the step scalings are folded into MFMA operands and
// accumulators and the elimination multiplies are DPP-fused (ttc_lqr_elim16.h).
//
// Matrix-core layout of a 16x16 tile X (the MFMA C/D layout): lane 16g + c holds
// X[4g + r][c], r = 0..3.  Each MFMA sums over k = 4g + s in lane group g (s = the
// instruction index), so the A operand of lane (g, c) is X[c][4g + s] and the B
// operand is Y[4g + s][c].  With N symmetric, N[c][4g + s] is the lane's own
// N[4g + s][c]; the MFMA result W[4g + s][c] is again the lane's own register, so
// N -> W -> Quu never leaves the registers.  The row layout (lane (g, c) owns row c
// of problem g) is reached through wave-private LDS.
//
// Breakdown guard: in exact arithmetic every pivot of Quu = R + B'VB is at least
// min_j 1/R_inv_j (Quu >= R).  A pivot below half of that, or not finite, means fp32
// rounding has made V indefinite; the wave then leaves the matrix-core loop and redoes
// this step and all remaining ones with the row-layout sweep (partially pivoted
// Gauss-Jordan on [Quu | Qux], rpl_sweep).
#pragma once
#include <utility>

#include "ttc_lqr_elim16.h"
#include "ttc_lqr_kernels.hpp"

namespace ttc {

typedef float v4f __attribute__((ext_vector_type(4)));

struct M16 {
  static constexpr int LD = 20;                 // LDS row stride of a 16x16 tile (floats)
  static constexpr int MAT = 16 * LD;           // 320 floats
  static constexpr int OFF_A = 0;               // -Quu
  static constexpr int OFF_B = MAT;             // -W, then -M
  static constexpr int OFF_U = 2 * MAT;         // U (steps that form the gains), else V for the fallback
  static constexpr int PER_PROB = 3 * MAT + 4;  // +4: bank skew between problems
  static constexpr int THREADS = 64;            // one wave per block
  // row-layout fallback: per problem B (Geo<16>::MAT) + rpl_sweep scratch (Geo<16>::PER_PROB)
  static constexpr int FB_PER_PROB = Geo<16>::MAT + Geo<16>::PER_PROB;
  static_assert(FB_PER_PROB <= PER_PROB, "fallback scratch must fit the tile region");
  // per-step vectors alpha, beta, q of the 4 problems, as [q][i] (row reads) and [i][q]
  // (column reads)
  static constexpr int OFF_VEC = 4 * PER_PROB;
  static constexpr int VEC = 64;
  static constexpr int LDS_FLOATS = OFF_VEC + 5 * VEC;
  static constexpr size_t LDS_BYTES = LDS_FLOATS * sizeof(float);
};

__device__ __forceinline__ v4f mfma16x16x4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ float ror16f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
// Lane K of each 16-lane row to the whole row (DPP row_newbcast).
template <int K>
__device__ __forceinline__ float bcast16(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + K, 0xF, 0xF, false));
}

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
// f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N-1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}


// lane K of each 16-lane row to the whole row (DPP row_newbcast:K).  Every lane has a valid
// source, so bound_ctrl lets the move fold into its consumer as that instruction's DPP operand.
template <int K>
__device__ __forceinline__ float rowbcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + K, 0xF, 0xF, true));
}

// Solve [M | b] (one system per lane: x, or two: x and y) by the row-layout Gauss-Jordan
// elimination without row exchanges of GjSpd (ttc_lqr_elim16.h), the pivot of step k
// broadcast from lane k.  For a symmetric positive definite M the pivots are those of its
// LDL' factorisation, all positive, and elimination in the natural order is stable; `bad`
// is set on the lanes of a system with a pivot that is not positive or not finite (M not
// positive definite in working precision), whose result must then be discarded.  On return
// the solution is x[16] / px on lane li (y[16] / py).
__device__ __forceinline__ void gj_spd16x1(float (&x)[17], int li, float& px, bool& bad) {
  px = 1.f;
  bad = false;
  static_for<16>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const float dx = rowbcast<k>(x[k]);  // the pivot, held by lane k
    bad |= !(dx > 0.f);                  // also catches NaN
    const bool own = li == k;
    const float nx = own ? 0.f : -x[k] * __builtin_amdgcn_rcpf(dx);
    if (own) px = dx;
    GjSpd<k>::upd(x, nx);
  });
}

__device__ __forceinline__ void gj_spd16x2(float (&x)[17], float (&y)[17], int li, float& px, float& py,
                                           bool& bad) {
  px = py = 1.f;
  bad = false;
  static_for<16>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    const float dx = rowbcast<k>(x[k]), dy = rowbcast<k>(y[k]);  // the pivots, held by lane k
    bad |= !(dx > 0.f) || !(dy > 0.f);                            // also catches NaN
    const bool own = li == k;
    const float nx = own ? 0.f : -x[k] * __builtin_amdgcn_rcpf(dx);
    const float ny = own ? 0.f : -y[k] * __builtin_amdgcn_rcpf(dy);
    if (own) {
      px = dx;
      py = dy;
    }
    GjSpd<k>::upd(x, y, nx, ny);
  });
}


__device__ __forceinline__ float row16_min(float v) {
  v = fminf(v, ror16f<8>(v));
  v = fminf(v, ror16f<4>(v));
  v = fminf(v, ror16f<2>(v));
  v = fminf(v, ror16f<1>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += ror16f<8>(v);
  v += ror16f<4>(v);
  v += ror16f<2>(v);
  v += ror16f<1>(v);
  return v;
}

__device__ __forceinline__ v4f ld4(const float* p) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  return v4f{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st4(float* p, v4f v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// The sweep of the 4 problems pbase .. pbase+3 (one wave).  RESCUE: only the problems a
// matrix-core forward marked with a NaN (u[p][0], or Quu_0[p][0][0] without u) are stored,
// and the wave returns at once when none of its 4 problems is marked.
template <int SM, bool WRITE_U, bool RESCUE>
__device__ __forceinline__ void fwd16_group(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status, const int64_t pbase) {
  extern __shared__ __align__(16) float sm[];
  constexpr float kLog2e = 1.4426950408889634f;
  const int lane = threadIdx.x;
  const int g = lane >> 4;  // lane group: MFMA row block, and "my problem" in the row layout
  const int c = lane & 15;  // MFMA column, and "my row" in the row layout

  int64_t pid[4];
  float* buf[4];
  bool pv[4];  // problem q exists (and, when rescuing, is marked): its results are stored
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    pid[q] = (pbase + q < P) ? (pbase + q) : (P - 1);  // idle problems recompute a real one, never store
    buf[q] = sm + q * M16::PER_PROB;
    pv[q] = pbase + q < P;
    if constexpr (RESCUE) pv[q] = pv[q] && isnan(WRITE_U ? u_out[pid[q] * 16] : q0stash[pid[q] * 256]);
  }
  if constexpr (RESCUE) {
    if (!(pv[0] || pv[1] || pv[2] || pv[3])) return;
  }
  const bool own_valid = pv[g];
  const int64_t po = pid[g];
  float* own = sm + g * M16::PER_PROB;  // (not buf[g]: a dynamically indexed pointer loses its LDS address space)
  float* vA = sm + M16::OFF_VEC;  // alpha [q][i]
  float* vQ = vA + M16::VEC;      // q     [q][i]
  float* vAT = vQ + M16::VEC;     // alpha [i][q]
  float* vBT = vAT + M16::VEC;    // beta  [i][q]
  float* vQT = vBT + M16::VEC;    // q     [i][q]

  // discount exponents in base 2: exp(l * n) = exp2(l * log2(e) * n)
  const float a_c = A_diag[po * 16 + c];
  const float lb2_c = lgB[po * 16 + c] * kLog2e;
  const float lq2_c = lgQ[po * 16 + c] * kLog2e;
  const float la2_o = lgA[po] * kLog2e;
  const float piv_floor = 0.5f * row16_min(1.0f / Rinv[po * 16 + c]);

  float Bop[4][4];  // B_q[4g+s][c]: B operand of N B, A operand (B') of B' W
  float Qn[4][4];   // -sym(Q_q)[4g+r][c]
  v4f Nc[4];        // N_q[4g+r][c] = -V_q[4g+r][c]
  v4f dR[4];        // -R_q = -diag(1/R_inv_q) in the tile layout (the -Quu accumulator)
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t n = pid[q] / H;
    const float* bq = Bg + n * 256;
    const float* qq = Qg + n * 256;
    const float* fq = Qf + pid[q] * 256;
    const float rr = 1.0f / Rinv[pid[q] * 16 + c];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g + s;
      Bop[q][s] = bq[i * 16 + c];
      Qn[q][s] = -0.5f * (qq[i * 16 + c] + qq[c * 16 + i]);
      Nc[q][s] = -0.5f * (fq[i * 16 + c] + fq[c * 16 + i]);
      dR[q][s] = (i == c) ? -rr : 0.0f;
    }
  }

  // One Riccati step; NEED_K: also form the gains K_t (stored steps, and t = 0 for u0).
  // Returns true when the breakdown guard fired.  V entering the step is then in tile U
  // for the row-layout sweep; the registers may hold garbage (steps without gains run to
  // their end regardless, which keeps their loop a single-exit loop).
  auto step = [&](auto need_k_c, const int t) -> bool {
    constexpr bool NEED_K = decltype(need_k_c)::value;
    const bool last = NEED_K && t == 0;
    const float tp1 = (float)(t + 1);
    {
      const float beta = __builtin_amdgcn_exp2f(lb2_c * tp1);
      const float alpha = fmaf(a_c, __builtin_amdgcn_exp2f(la2_o * tp1), 1.0f);
      const float qd = last ? 0.0f : __builtin_amdgcn_exp2f(lq2_c * (float)t);
      vA[g * 16 + c] = alpha;
      vQ[g * 16 + c] = qd;
      vAT[c * 4 + g] = alpha;
      vBT[c * 4 + g] = beta;
      vQT[c * 4 + g] = qd;
    }
    if (SM == STASH_V1 && last) {
      // compact stash: V_1 (the value entering step 0), rows 4g..4g+3 of column c
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (pv[q]) {
          float* vp = kstash + (pid[q] * 16 + 4 * g) * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) vp[r * 16] = -Nc[q][r];
        }
      }
    }
    if constexpr (!NEED_K) {
      // N entering the step, for the row-layout sweep should this step break down
      // (tile U is unused by steps that do not form the gains)
#pragma unroll
      for (int q = 0; q < 4; ++q) st4(buf[q] + M16::OFF_U + c * M16::LD + 4 * g, Nc[q]);
    }
    wave_sync();
    const v4f bcol = ld4(vBT + c * 4);  // beta_q[c], q = 0..3

    // ---- -W = N B_k -> tile B (row-major);  -Quu = B_k'(-W) - R -> tile A ----------------
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float bk[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) bk[s] = Bop[q][s] * bcol[q];
      v4f w = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) w = mfma16x16x4(Nc[q][s], bk[s], w);
#pragma unroll
      for (int r = 0; r < 4; ++r) buf[q][M16::OFF_B + (4 * g + r) * M16::LD + c] = w[r];
      v4f quu = dR[q];
#pragma unroll
      for (int s = 0; s < 4; ++s) quu = mfma16x16x4(bk[s], w[s], quu);
      st4(buf[q] + M16::OFF_A + c * M16::LD + 4 * g, quu);  // symmetric: column fragment = row fragment
    }
    wave_sync();

    // ---- row layout: elimination on the rows [-Quu; -W; I] -----------------------------
    // Pivot k of -Quu is -d_k (d_k > 0 the pivot of Quu); every row x is updated with the
    // multiplier x[k] / d_k, and column k of the -W rows is scaled by 1/sqrt(d_k) once final.
    float qr[16], wr[16], ir[16];
    ld_row<16>(own + M16::OFF_A + c * M16::LD, qr);
    ld_row<16>(own + M16::OFF_B + c * M16::LD, wr);
    if (SM != STASH_NONE && last && own_valid) {
      float quu_row[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) quu_row[k] = -qr[k];
      st_global_row<16>(q0stash + (po * 16 + c) * 16, quu_row);
    }
    if constexpr (NEED_K) {
#pragma unroll
      for (int k = 0; k < 16; ++k) ir[k] = (k == c) ? 1.0f : 0.0f;
    }
    bool bad = false;
    static_for<16>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      // pivot: diagonal entry k of the trailing matrix, held by lane (g, k)
      const float npiv = bcast16<k>(qr[k]);  // -d_k
      bad |= !(-npiv >= piv_floor);          // also catches NaN
      const float rs = __builtin_amdgcn_rsqf(-npiv);  // raw v_rsq_f32 (pivots are >= piv_floor, never denormal)
      const float ip = rs * rs;
      const float nw = wr[k] * ip;
      float ni = 0.f;
      if constexpr (NEED_K) ni = ir[k] * ip;
      if constexpr (k < 15) {
        const float nq = qr[k] * ip;
        if constexpr (NEED_K)
          Elim16<k>::qwi(qr, wr, ir, nq, nw, ni);
        else
          Elim16<k>::qw(qr, wr, nq, nw);
      }
      wr[k] *= rs;                        // -M[c][k]
      if constexpr (NEED_K) ir[k] *= rs;  // U[c][k]
    });
    const bool failed = __any(bad);
    if constexpr (NEED_K) {
      if (failed) {
        // hand N (unchanged by this step) to the row-layout sweep through tile U
        wave_sync();
#pragma unroll
        for (int q = 0; q < 4; ++q) st4(buf[q] + M16::OFF_U + c * M16::LD + 4 * g, Nc[q]);
        wave_sync();
        return true;
      }
    }
    st_row<16>(own + M16::OFF_B + c * M16::LD, wr);  // -M rows
    if constexpr (NEED_K) st_row<16>(own + M16::OFF_U + c * M16::LD, ir);  // U rows
    wave_sync();

    // ---- N + M M' (N as accumulator);  K = U (-M)' diag(a) -----------------------------
    const v4f acol = ld4(vAT + c * 4);  // alpha_q[c]
    const v4f qcol = ld4(vQT + c * 4);  // q_q[c]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const v4f m4 = ld4(buf[q] + M16::OFF_B + c * M16::LD + 4 * g);  // -M[c][4g+s]
      if constexpr (NEED_K) {
        const v4f u4 = ld4(buf[q] + M16::OFF_U + c * M16::LD + 4 * g);  // U[c][4g+s]
        v4f kt = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) kt = mfma16x16x4(u4[s], m4[s], kt);
        const bool qvalid = pv[q];
#pragma unroll
        for (int r = 0; r < 4; ++r) kt[r] *= acol[q];  // K[4g+r][c]
        if (SM == STASH_GAINS && qvalid) {
          float* kp = kstash + ((pid[q] * T + t) * 16 + 4 * g) * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) kp[r * 16] = kt[r];
        }
        if (last) {
          // u0[4g+r] = sum_c K[4g+r][c] h0[c]
          const float hc = h0[pid[q] * 16 + c];
          v4f u;
#pragma unroll
          for (int r = 0; r < 4; ++r) u[r] = row16_sum(kt[r] * hc);
          if (c == 0 && qvalid) {
            if (WRITE_U) st4(u_out + pid[q] * 16 + 4 * g, u);
            if (status != nullptr && !(isfinite(u[0]) && isfinite(u[1]) && isfinite(u[2]) && isfinite(u[3])))
              atomicOr(status, TTC_LQR_STATUS_NONFINITE);
          }
          continue;
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) Nc[q] = mfma16x16x4(m4[s], m4[s], Nc[q]);  // N + M M', in place
      const v4f arow = ld4(vA + q * 16 + 4 * g);
      const v4f qrow = ld4(vQ + q * 16 + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) Nc[q][r] = fmaf(arow[r] * acol[q], Nc[q][r], (qrow[r] * qcol[q]) * Qn[q][r]);
    }
    wave_sync();
    return failed;
  };

  // Row-layout sweep from step t_fb down to 0 after a breakdown at step t_fb: V rows (N in
  // tile U, stored by the failed step; N is symmetric, so the lane's column fragment is a
  // row fragment), then B of my problem, then rpl_sweep.
  auto row_sweep_from = [&](const int t_fb) {
    float V[16];
    ld_row<16>(own + M16::OFF_U + c * M16::LD, V);  // N rows
#pragma unroll
    for (int m = 0; m < 16; ++m) V[m] = -V[m];
    wave_sync();
    float* fb = own;
    const float* bn = Bg + (po / H) * 256;
#pragma unroll
    for (int m = 0; m < 16; ++m) fb[m * Geo<16>::LDM + c] = bn[m * 16 + c];
    wave_sync();
    rpl_sweep<16, float, SM, WRITE_U>(A_diag, Qg, Rinv, lgA, lgB, lgQ, h0, fb, fb + Geo<16>::MAT, c, po,
                                      own_valid, po / H, T, t_fb, V, u_out, kstash, q0stash, status);
  };

  if constexpr (SM == STASH_GAINS) {
    for (int t = T - 1; t >= 0; --t) {
      if (step(std::true_type{}, t)) {
        row_sweep_from(t);
        return;
      }
    }
  } else {
    // gains are formed only at t = 0: peel that step; the loop has a single exit
    int t = T - 1;
    bool failed = false;
    while (!failed && t >= 1) {
      failed = step(std::false_type{}, t);
      t -= failed ? 0 : 1;
    }
    if (failed || step(std::true_type{}, 0)) row_sweep_from(t);
  }
}

template <int SM, bool WRITE_U>
__global__ __launch_bounds__(M16::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void lqr_fwd16_mfma_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status) {
  fwd16_group<SM, WRITE_U, false>(A_diag, Bg, Qg, Rinv, Qf, lgA, lgB, lgQ, h0, P, H, T, u_out, kstash, q0stash,
                                  status, (int64_t)blockIdx.x * 4);
}

// Rescue pass after the d = 16 symplectic forward: the per-step Riccati sweep (with its own
// breakdown guard and row-layout finish) of every marked problem.  A small grid walks the
// 4-problem groups; it returns at once when `status` is given without
// TTC_LQR_STATUS_RESCUED (nothing was marked).
template <int SM, bool WRITE_U>
__global__ __launch_bounds__(M16::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void lqr_rescue16_mfma_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status) {
  if (status != nullptr && !(__atomic_load_n(status, __ATOMIC_RELAXED) & TTC_LQR_STATUS_RESCUED)) return;
  for (int64_t pb = (int64_t)blockIdx.x * 4; pb < P; pb += (int64_t)gridDim.x * 4) {
    fwd16_group<SM, WRITE_U, true>(A_diag, Bg, Qg, Rinv, Qf, lgA, lgB, lgQ, h0, P, H, T, u_out, kstash, q0stash,
                                   status, pb);
    wave_sync();  // the group's LDS is reused by the next one
  }
}

}  // namespace ttc
