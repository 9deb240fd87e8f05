// ttc_lqr_mfma16.cuh -- d = du = 16 forward kernel with the per-step products on
// the matrix cores (v_mfma_f32_16x16x4f32).
//
// One wave holds 4 LQR problems (q = 0..3).  Per Riccati step and problem:
//   W~ = V B,  G = B' W~                 8 MFMA, operands straight from registers
//   Quu = diag(b) G diag(b) + diag(1/r),  W = W~ diag(b)
//   right-looking Cholesky of Quu applied to the rows of [Quu; W; I]  (row layout)
//     -> M = W L^{-T} and U = L^{-T}
//   S = M M'                             4 MFMA
//   V <- diag(a) (V - S) diag(a) + diag(q) Q diag(q)
//   K = -Quu^{-1} Qux = -U M' diag(a)    4 MFMA (only when the gains are stored, and at t = 0)
//
// Matrix-core layout of a 16x16 tile X (the MFMA C/D layout): lane 16g + c holds
// X[4g + r][c], r = 0..3.  Each MFMA sums over k = 4g + s in lane group g (s = the
// instruction index), so the A operand of lane (g, c) is X[c][4g + s] and the B
// operand is Y[4g + s][c].  With V symmetric, V[c][4g + s] is the lane's own
// V[4g + s][c]; the MFMA result W~[4g + s][c] is again the lane's own register, so
// V -> W~ -> G never leaves the registers.  The row layout (lane (g, c) owns row c of
// problem g) is reached through wave-private LDS.
//
// Cholesky breakdown guard: in exact arithmetic every pivot of Quu = R + B'VB is at
// least min_j 1/R_inv_j (Quu >= R).  A pivot below half of that, or not finite, means
// fp32 rounding has made V indefinite; the wave then leaves the matrix-core loop and
// redoes this step and all remaining ones with the row-layout sweep (partially pivoted
// Gauss-Jordan on [Quu | Qux], rpl_sweep).  Keeping the two phases apart keeps their
// register footprints from adding up.
#pragma once
#include <utility>

#include "ttc_lqr_kernels.cuh"

namespace ttc {

typedef float v4f __attribute__((ext_vector_type(4)));

struct M16 {
  static constexpr int LD = 20;                      // LDS row stride of a 16x16 tile (floats)
  static constexpr int MAT = 16 * LD;                // 320 floats
  static constexpr int OFF_B = MAT;                  // tile A at 0, tile B at MAT
  static constexpr int OFF_VEC = 2 * MAT;            // beta, alpha, q (16 each), pivot row (32)
  static constexpr int PER_PROB = OFF_VEC + 80 + 4;  // +4: bank skew between problems
  static constexpr int THREADS = 64;                 // one wave per block
  // row-layout fallback: per problem B (Geo<16>::MAT) + rpl_sweep scratch (Geo<16>::PER_PROB)
  static constexpr int FB_PER_PROB = Geo<16>::MAT + Geo<16>::PER_PROB;
  static constexpr int LDS_FLOATS = 4 * (PER_PROB > FB_PER_PROB ? PER_PROB : FB_PER_PROB);
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

// Pin a row of registers at this program point.  Keeps the compiler from sinking the
// Cholesky updates of the W / I rows into the branch that consumes them, which would
// keep every broadcast pivot row alive at once.
template <int N>
__device__ __forceinline__ void pin_row(float (&r)[N]) {
#pragma unroll
  for (int i = 0; i < N; i += 4) asm volatile("" : "+v"(r[i]), "+v"(r[i + 1]), "+v"(r[i + 2]), "+v"(r[i + 3]));
}

__device__ __forceinline__ v4f ld4(const float* p) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  return v4f{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st4(float* p, v4f v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int SM, bool WRITE_U>
__global__ __launch_bounds__(M16::THREADS) void lqr_fwd16_mfma_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status) {
  extern __shared__ __align__(16) float sm[];
  const int lane = threadIdx.x;
  const int g = lane >> 4;  // lane group: MFMA row block, and "my problem" in the row layout
  const int c = lane & 15;  // MFMA column, and "my row" in the row layout
  const int64_t pbase = (int64_t)blockIdx.x * 4;

  int64_t pid[4];
  float* buf[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    pid[q] = (pbase + q < P) ? (pbase + q) : (P - 1);  // idle problems recompute a real one, never store
    buf[q] = sm + q * M16::PER_PROB;
  }
  const bool own_valid = pbase + g < P;
  const int64_t po = pid[g];
  float* own = sm + g * M16::PER_PROB;
  float* vbeta = own + M16::OFF_VEC;
  float* valpha = vbeta + 16;
  float* vq = valpha + 16;
  float* vpr = vq + 16;  // 32 floats

  const float a_c = A_diag[po * 16 + c];
  const float lgB_c = lgB[po * 16 + c];
  const float lgQ_c = lgQ[po * 16 + c];
  const float lgA_o = lgA[po];
  const float piv_floor = 0.5f * row16_min(1.0f / Rinv[po * 16 + c]);

  float Bop[4][4];  // B_q[4g+s][c]: B operand of V B, A operand (B') of B' W~
  float Qc[4][4];   // sym(Q_q)[4g+r][c]
  v4f Vc[4];        // V_q[4g+r][c]
  float rrc[4];     // 1/R_inv_q[c]
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t n = pid[q] / H;
    const float* bq = Bg + n * 256;
    const float* qq = Qg + n * 256;
    const float* fq = Qf + pid[q] * 256;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int i = 4 * g + s;
      Bop[q][s] = bq[i * 16 + c];
      Qc[q][s] = 0.5f * (qq[i * 16 + c] + qq[c * 16 + i]);
      Vc[q][s] = 0.5f * (fq[i * 16 + c] + fq[c * 16 + i]);
    }
    rrc[q] = 1.0f / Rinv[pid[q] * 16 + c];
  }

  // One Riccati step; NEED_K: also form the gains K_t (stored steps, and t = 0 for u0).
  // Returns false when the Cholesky guard fired (nothing of the step was kept).
  auto step = [&](auto need_k_c, const int t) -> bool {
    constexpr bool NEED_K = decltype(need_k_c)::value;
    const bool last = NEED_K && t == 0;
    const float tp1 = (float)(t + 1);
    const float my_beta = expf(lgB_c * tp1);
    const float my_alpha = fmaf(a_c, expf(lgA_o * tp1), 1.0f);
    const float my_q = last ? 0.0f : expf(lgQ_c * (float)t);
    if (SM == STASH_V1 && last) {
      // compact stash: V_1 (the value entering step 0), rows 4g..4g+3 of column c
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (pbase + q < P) {
          float* vp = kstash + (pid[q] * 16 + 4 * g) * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) vp[r * 16] = Vc[q][r];
        }
      }
    }
    vbeta[c] = my_beta;
    valpha[c] = my_alpha;
    vq[c] = my_q;

    // ---- W~ = V B -> tile B (row-major);  G = B' W~ ---------------------------------
    v4f Gq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4f w = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) w = mfma16x16x4(Vc[q][s], Bop[q][s], w);
#pragma unroll
      for (int r = 0; r < 4; ++r) buf[q][M16::OFF_B + (4 * g + r) * M16::LD + c] = w[r];
      v4f gg = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) gg = mfma16x16x4(Bop[q][s], w[s], gg);
      Gq[q] = gg;
    }
    wave_sync();
    // ---- Quu = diag(b) G diag(b) + diag(1/r): column fragment = row fragment -> tile A
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float* bv = buf[q] + M16::OFF_VEC;
      const v4f brow = ld4(bv + 4 * g);
      const float bcol = bv[c];
      v4f quu;
#pragma unroll
      for (int r = 0; r < 4; ++r) quu[r] = fmaf(brow[r] * bcol, Gq[q][r], (4 * g + r == c) ? rrc[q] : 0.f);
      st4(buf[q] + c * M16::LD + 4 * g, quu);
    }
    wave_sync();

    // ---- row layout: Cholesky of Quu on the rows [Quu; W; I] ---------------------------
    float qr[16], wr[16], ir[16];
    {
      float be[16];
      ld_row<16>(own + c * M16::LD, qr);
      ld_row<16>(own + M16::OFF_B + c * M16::LD, wr);
      ld_row<16>(vbeta, be);
#pragma unroll
      for (int k = 0; k < 16; ++k) wr[k] *= be[k];
    }
    if (SM != STASH_NONE && last && own_valid) st_global_row<16>(q0stash + (po * 16 + c) * 16, qr);
    if constexpr (NEED_K) {
#pragma unroll
      for (int k = 0; k < 16; ++k) ir[k] = (k == c) ? 1.0f : 0.0f;
    }
    bool bad = false;
    static_for<16>([&](auto kc) {
      constexpr int k = decltype(kc)::value;
      // row k of my problem's trailing matrix, broadcast from lane (g, k) by DPP
      const float piv = bcast16<k>(qr[k]);
      bad |= !(piv >= piv_floor);  // also catches NaN
      const float rs = rsqrtf(fmaxf(piv, 1e-30f));
      const float ip = rs * rs;
      const float fq = qr[k] * ip;
      const float fw = wr[k] * ip;
      const float fi = NEED_K ? ir[k] * ip : 0.f;
      wr[k] *= rs;  // M[c][k]
      if constexpr (NEED_K) ir[k] *= rs;  // U[c][k]
#pragma unroll
      for (int m = k + 1; m < 16; ++m) {
        const float pm = bcast16<k>(qr[m]);
        qr[m] = fmaf(-fq, pm, qr[m]);
        wr[m] = fmaf(-fw, pm, wr[m]);
        if constexpr (NEED_K) ir[m] = fmaf(-fi, pm, ir[m]);
      }
      pin_row(wr);
      if constexpr (NEED_K) pin_row(ir);
    });
    if (__any(bad)) return false;
    {
      // ---- M rows -> tile A, U rows -> tile B; S = M M', K = -U M' diag(a) -------------
      st_row<16>(own + c * M16::LD, wr);
      if constexpr (NEED_K) st_row<16>(own + M16::OFF_B + c * M16::LD, ir);
      wave_sync();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4f m4 = ld4(buf[q] + c * M16::LD + 4 * g);  // M[c][4g+s]
        const float* av = buf[q] + M16::OFF_VEC + 16;
        const float acol = av[c];
        if constexpr (NEED_K) {
          const v4f u4 = ld4(buf[q] + M16::OFF_B + c * M16::LD + 4 * g);  // U[c][4g+s]
          v4f kt = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) kt = mfma16x16x4(u4[s], m4[s], kt);
          const bool qvalid = pbase + q < P;
#pragma unroll
          for (int r = 0; r < 4; ++r) kt[r] *= -acol;  // K[4g+r][c]
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
        v4f S = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) S = mfma16x16x4(m4[s], m4[s], S);
        const float* qvv = buf[q] + M16::OFF_VEC + 32;
        const v4f arow = ld4(av + 4 * g);
        const v4f qrow4 = ld4(qvv + 4 * g);
        const float qcol = qvv[c];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          Vc[q][r] = fmaf(arow[r] * acol, Vc[q][r] - S[r], (qrow4[r] * qcol) * Qc[q][r]);
      }
      wave_sync();
    }
    return true;
  };

  int t_fb = -1;  // step at which the wave switched to the row-layout sweep
  for (int t = T - 1; t >= 0; --t) {
    const bool ok = (SM == STASH_GAINS || t == 0) ? step(std::true_type{}, t) : step(std::false_type{}, t);
    if (!ok) {
      t_fb = t;
      break;
    }
  }

  if (t_fb >= 0) {
    // ---- row-layout fallback from step t_fb: V rows (V symmetric, so the lane's column
    // fragment is a row fragment), then B of my problem, then rpl_sweep -------------------
#pragma unroll
    for (int q = 0; q < 4; ++q) st4(buf[q] + c * M16::LD + 4 * g, Vc[q]);
    wave_sync();
    float V[16];
    ld_row<16>(own + c * M16::LD, V);
    wave_sync();
    float* fb = sm + g * M16::FB_PER_PROB;
    const float* bn = Bg + (po / H) * 256;
#pragma unroll
    for (int m = 0; m < 16; ++m) fb[m * Geo<16>::LDM + c] = bn[m * 16 + c];
    wave_sync();
    rpl_sweep<16, float, SM, WRITE_U>(A_diag, Qg, Rinv, lgA, lgB, lgQ, h0, fb, fb + Geo<16>::MAT, c, po,
                                         own_valid, po / H, T, t_fb, V, u_out, kstash, q0stash, status);
  }
}

}  // namespace ttc
