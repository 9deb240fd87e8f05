// ttc_lqr_mfma_blk.cuh -- d = du in {32, 64} forward kernel: the Riccati sweep as 16x16
// tiles on the matrix cores (v_mfma_f32_16x16x4f32), with a blocked Cholesky.
//
// One wave holds PPW = 64 / D problems; every D x D matrix is NB x NB tiles (NB = D/16),
// each tile in the MFMA C/D layout: lane 16g + c holds X[4g + r][c], r = 0..3.  For a
// product C = X Y the A operand of lane (g, c) is X[c][4g + s] and the B operand
// Y[4g + s][c] (instruction s of 4 covers k = 4g + s), so a C-layout tile serves directly
// as a B operand, and as an A operand when X is the transpose of a tile we hold
// (X_IK = T_KI').  Per Riccati step t >= 1 and problem:
//   B_k = B diag(beta)                      NB*NB*4 VALU (the MFMA operand, scaled)
//   -W = N B_k           (N = -V)           NB^3 * 4 MFMA
//   -Quu = B_k'(-W) - R, upper tiles        NB(NB+1)/2 * NB * 4 MFMA
//   -W' from -W through LDS (tile transpose)
//   blocked Cholesky of S' = [Quu | W'] by 16-row panels j:
//     -L_jj^{-T} from a 16x16 DPP elimination of [-Quu_jj; -I] (row layout),
//     panel   P'_ji = L_jj^{-1} S'_ji       4 MFMA per tile
//     trailing -S'_Ji += P'_jJ' P'_ji      4 MFMA per tile
//   so that the W' tiles end as M' = L^{-1} W' (M = W L^{-T}, W Quu^{-1} W' = M M');
//   N + M M' = -(V - W Quu^{-1} W'), upper tiles, one operand -> exactly symmetric
//   N <- diag(a)(N + M M')diag(a) - diag(q) Q diag(q), lower tiles mirrored via LDS.
// Step 0 forms W and Quu the same way and solves Quu_0 z = W_0' A_0 h0 (u0 = -z) by
// partially pivoted Gauss-Jordan in the row layout (lane li owns row li); it also writes
// the compact stash V_1 / Quu_0.
//
// Breakdown guard: in exact arithmetic every Cholesky pivot of Quu = R + B'VB is at least
// min_j 1/R_inv_j (Quu >= R); a pivot below half of that, or not finite, means rounding
// made V indefinite.  The wave then stops and marks its problems with a NaN (u[p][0], or
// Quu_0[p][0][0] when u is not written); lqr_rescue_kernel recomputes every marked problem
// with the row-layout sweep (pivoted Gauss-Jordan at every step).
#pragma once
#include "ttc_lqr_mfma16.cuh"

namespace ttc {

template <int D>
struct MB {
  static constexpr int NB = D / 16;                 // tiles per dimension
  static constexpr int PPW = 64 / D;                // problems per wave
  static constexpr int NT = NB * (NB + 1) / 2;      // upper tiles (I <= J)
  static constexpr int LDX = D + kPad;              // LDS row stride of D-wide rows
  static constexpr int LDG = 20;                    // LDS row stride of a 16 x 16 tile
  // d = 64 keeps B and -sym(Q) in LDS (registers hold N and the step's products);
  // d = 32 keeps them in registers.
  static constexpr bool BQ_LDS = D == 64;
  static constexpr int CH = BQ_LDS ? 2 : NB;        // block-rows per transpose round
  // per-problem LDS region: [B' (column-major B) | -sym(Q) fragments | transpose buffer]
  static constexpr int OFF_Q = BQ_LDS ? D * LDX : 0;
  static constexpr int OFF_X = BQ_LDS ? OFF_Q + NT * 256 : 0;
  static constexpr int XROWS = CH * 16;
  static constexpr int REG0 = OFF_X + XROWS * LDX;
  static constexpr int QB_CAP = REG0 - OFF_Q;       // step 0: the full Quu_0 rows (from OFF_Q)
  static_assert(QB_CAP >= D * LDX, "step 0 needs D rows of Quu_0");
  static_assert(XROWS * LDX >= 16 * LDG, "the 16x16 tile buffer aliases the transpose buffer");
  static constexpr int REG = (REG0 + 3) & ~3;       // 16-byte multiple
  static constexpr int VEC = 3 * D;                 // alpha, q (step 0: alpha*h0), beta
  static constexpr int THREADS = 64;
  static constexpr int WAVES = D == 64 ? 1 : 2;     // waves per SIMD the registers allow
  static constexpr size_t LDS_BYTES = sizeof(float) * (size_t)PPW * (REG + VEC);
};

// upper tile (I, J), I <= J, in row-major order of the upper triangle
template <int NB>
__host__ __device__ constexpr int utile(int I, int J) {
  return I * NB - I * (I - 1) / 2 + (J - I);
}

template <int D, int SM, bool WRITE_U>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, MB<D>::WAVES))) void lqr_fwd_blk_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    int64_t P, int H, int T, float* __restrict__ u_out, float* __restrict__ kstash,
    float* __restrict__ q0stash, int* __restrict__ status) {
  using G = MB<D>;
  constexpr int NB = G::NB, PPW = G::PPW, NT = G::NT, LDX = G::LDX, LDG = G::LDG;
  constexpr bool BQL = G::BQ_LDS;
  extern __shared__ __align__(16) float sm[];
  constexpr float kLog2e = 1.4426950408889634f;
  const int lane = threadIdx.x;
  const int g = lane >> 4;   // lane group: MFMA row block
  const int c = lane & 15;   // MFMA column; row of the 16x16 elimination
  const int qo = lane / D;   // my problem in the row layout
  const int li = lane % D;   // my row (of D) in the row layout
  const int64_t pbase = (int64_t)blockIdx.x * PPW;

  int64_t pid[PPW];
#pragma unroll
  for (int q = 0; q < PPW; ++q) pid[q] = (pbase + q < P) ? (pbase + q) : (P - 1);  // idle: recompute, never store
  const int64_t po = (pbase + qo < P) ? (pbase + qo) : (P - 1);
  const bool own_valid = pbase + qo < P;
  auto region = [&](int q) { return sm + q * G::REG; };
  float* vecs = sm + PPW * G::REG;  // [q][alpha D | q D | beta D]

  // row-layout scalars of my problem (lane li of problem qo)
  const float a_l = A_diag[po * D + li];
  const float lb2_l = lgB[po * D + li] * kLog2e;
  const float lq2_l = lgQ[po * D + li] * kLog2e;
  const float la2_o = lgA[po] * kLog2e;
  float piv_floor = 1.0f / Rinv[po * D + li];
  piv_floor = row16_min(piv_floor);
  if constexpr (D >= 32) piv_floor = fminf(piv_floor, __shfl_xor(piv_floor, 16, 64));
  if constexpr (D >= 64) piv_floor = fminf(piv_floor, __shfl_xor(piv_floor, 32, 64));
  piv_floor *= 0.5f;

  // C-layout state: N = -V (all tiles); B and -sym(Q) (registers, or LDS for d = 64)
  v4f NV[PPW][NB][NB];
  float Bm[BQL ? 1 : PPW][NB][NB][4];
  v4f Qn[BQL ? 1 : PPW][NT];
  float rr[PPW][NB];  // 1 / R_inv[16I + c]
#pragma unroll
  for (int q = 0; q < PPW; ++q) {
    const int64_t n = pid[q] / H;
    const float* bq = Bg + n * D * D;
    const float* qq = Qg + n * D * D;
    const float* fq = Qf + pid[q] * D * D;
    float* rg = region(q);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      rr[q][I] = 1.0f / Rinv[pid[q] * D + 16 * I + c];
#pragma unroll
      for (int J = 0; J < NB; ++J) {
        v4f qn;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * g + r, j = 16 * J + c;
          NV[q][I][J][r] = -0.5f * (fq[i * D + j] + fq[j * D + i]);
          const float b = bq[i * D + j];
          if constexpr (BQL) rg[j * LDX + i] = b;  // column-major: a tile's operand is one float4
          else Bm[q][I][J][r] = b;
          qn[r] = -0.5f * (qq[i * D + j] + qq[j * D + i]);
        }
        if (I <= J) {
          if constexpr (BQL) st4(rg + G::OFF_Q + (utile<NB>(I, J) * 64 + lane) * 4, qn);
          else Qn[q][utile<NB>(I, J)] = qn;
        }
      }
    }
  }
  wave_sync();

  // B_k = B diag(beta) operand tiles of problem q (beta read from the vector buffer)
  auto load_bk = [&](int q, float (&Bk)[NB][NB][4]) {
    const float* v = vecs + q * G::VEC;
    const float* rg = region(q);
#pragma unroll
    for (int J = 0; J < NB; ++J) {
      const float bj = v[2 * D + 16 * J + c];
#pragma unroll
      for (int K = 0; K < NB; ++K) {
        if constexpr (BQL) {
          const v4f b4 = ld4(rg + (16 * J + c) * LDX + 16 * K + 4 * g);
#pragma unroll
          for (int s = 0; s < 4; ++s) Bk[K][J][s] = b4[s] * bj;
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) Bk[K][J][s] = Bm[q][K][J][s] * bj;
        }
      }
    }
  };
  // -W = N B_k and the upper tiles of -Quu = B_k'(-W) - R
  auto w_quu = [&](int q, const float (&Bk)[NB][NB][4], v4f (&nW)[NB][NB], v4f (&nQ)[NT]) {
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int J = 0; J < NB; ++J) nW[I][J] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int K = 0; K < NB; ++K)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
          for (int J = 0; J < NB; ++J) nW[I][J] = mfma16x16x4(NV[q][K][I][s], Bk[K][J][s], nW[I][J]);
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int J = I; J < NB; ++J) {
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
        if (I == J) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] = (4 * g + r == c) ? -rr[q][I] : 0.0f;
        }
        nQ[utile<NB>(I, J)] = acc;
      }
#pragma unroll
    for (int K = 0; K < NB; ++K)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
          for (int J = I; J < NB; ++J)
            nQ[utile<NB>(I, J)] = mfma16x16x4(Bk[K][I][s], nW[K][J][s], nQ[utile<NB>(I, J)]);
  };

  // One matrix-core Riccati step t >= 1.  Returns true when the breakdown guard fired
  // (N is then unchanged: the guard is evaluated before N is touched).
  auto step = [&](const int t) -> bool {
    const float tp1 = (float)(t + 1);
    {
      float* v = vecs + qo * G::VEC;
      v[li] = fmaf(a_l, __builtin_amdgcn_exp2f(la2_o * tp1), 1.0f);  // alpha
      v[D + li] = __builtin_amdgcn_exp2f(lq2_l * (float)t);          // q
      v[2 * D + li] = __builtin_amdgcn_exp2f(lb2_l * tp1);           // beta
    }
    wave_sync();

    v4f nWt[PPW][NB][NB];  // -W' tiles (C layout), later M'
    v4f nQ[PPW][NT];       // -Quu upper tiles, later the L' panels
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      v4f nW[NB][NB];
      {
        float Bk[NB][NB][4];
        load_bk(q, Bk);
        w_quu(q, Bk, nW, nQ[q]);
      }
      // -W -> LDS row-major, read back as -W' (CH block-rows per round)
      float* xb = region(q) + G::OFF_X;
#pragma unroll
      for (int h = 0; h < NB; h += G::CH) {
#pragma unroll
        for (int I = h; I < h + G::CH; ++I)
#pragma unroll
          for (int J = 0; J < NB; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) xb[(16 * (I - h) + 4 * g + r) * LDX + 16 * J + c] = nW[I][J][r];
        wave_sync();
#pragma unroll
        for (int I = h; I < h + G::CH; ++I)
#pragma unroll
          for (int J = 0; J < NB; ++J) nWt[q][J][I] = ld4(xb + (16 * (I - h) + c) * LDX + 16 * J + 4 * g);
        wave_sync();
      }
    }

    // ---- blocked Cholesky of S' = [Quu | W'] by 16-row panels --------------------------
    bool bad = false;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      // diagonal tile -Quu_jj (symmetric: the column fragment is a row fragment)
#pragma unroll
      for (int q = 0; q < PPW; ++q) st4(region(q) + G::OFF_X + c * LDG + 4 * g, nQ[q][utile<NB>(j, j)]);
      wave_sync();
      float* tb = region(qo) + G::OFF_X;
      float qr[16], ir[16];
      ld_row<16>(tb + c * LDG, qr);
#pragma unroll
      for (int k = 0; k < 16; ++k) ir[k] = (k == c) ? -1.0f : 0.0f;
      // elimination of the rows [-Quu_jj; -I]: the -I rows end as -L_jj^{-T}
      static_for<16>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const float npiv = bcast16<k>(qr[k]);  // -d_k
        bad |= !(-npiv >= piv_floor);          // also catches NaN
        const float rs = __builtin_amdgcn_rsqf(-npiv);
        const float ip = rs * rs;
        const float ni = ir[k] * ip;
        if constexpr (k < 15) {
          const float nq = qr[k] * ip;
          Elim16<k>::qw(qr, ir, nq, ni);
        }
        ir[k] *= rs;
      });
      wave_sync();
      st_row<16>(tb + c * LDG, ir);  // rows of -L_jj^{-T} (groups of one problem write equal values)
      wave_sync();
#pragma unroll
      for (int q = 0; q < PPW; ++q) {
        const float* ub = region(q) + G::OFF_X;
        float nU[4];  // A operand of -L_jj^{-1}: -L^{-T}[4g + s][c]
#pragma unroll
        for (int s = 0; s < 4; ++s) nU[s] = ub[(4 * g + s) * LDG + c];
        // panel: P'_ji = (-L^{-1})(-S'_ji)
#pragma unroll
        for (int i = j + 1; i < NB; ++i) {
          v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = mfma16x16x4(nU[s], nQ[q][utile<NB>(j, i)][s], acc);
          nQ[q][utile<NB>(j, i)] = acc;
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) acc = mfma16x16x4(nU[s], nWt[q][j][i][s], acc);
          nWt[q][j][i] = acc;
        }
        // trailing: -S'_Ji += P'_jJ' P'_ji
#pragma unroll
        for (int J = j + 1; J < NB; ++J) {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int i = J; i < NB; ++i)
              nQ[q][utile<NB>(J, i)] =
                  mfma16x16x4(nQ[q][utile<NB>(j, J)][s], nQ[q][utile<NB>(j, i)][s], nQ[q][utile<NB>(J, i)]);
#pragma unroll
            for (int i = 0; i < NB; ++i)
              nWt[q][J][i] = mfma16x16x4(nQ[q][utile<NB>(j, J)][s], nWt[q][j][i][s], nWt[q][J][i]);
          }
        }
      }
      wave_sync();  // the tile buffer is rewritten by the next panel
    }
    if (__any(bad)) return true;

    // ---- N + M M' (upper tiles), scaling, mirror ----------------------------------------
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
#pragma unroll
      for (int kb = 0; kb < NB; ++kb)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int I = 0; I < NB; ++I)
#pragma unroll
            for (int J = I; J < NB; ++J) NV[q][I][J] = mfma16x16x4(nWt[q][kb][I][s], nWt[q][kb][J][s], NV[q][I][J]);
      const float* v = vecs + q * G::VEC;
      float* rg = region(q);
#pragma unroll
      for (int I = 0; I < NB; ++I) {
        const v4f arow = ld4(v + 16 * I + 4 * g);
        const v4f qrow = ld4(v + D + 16 * I + 4 * g);
#pragma unroll
        for (int J = I; J < NB; ++J) {
          const float acol = v[16 * J + c];
          const float qcol = v[D + 16 * J + c];
          v4f qn;
          if constexpr (BQL) qn = ld4(rg + G::OFF_Q + (utile<NB>(I, J) * 64 + lane) * 4);
          else qn = Qn[q][utile<NB>(I, J)];
#pragma unroll
          for (int r = 0; r < 4; ++r) NV[q][I][J][r] = fmaf(arow[r] * acol, NV[q][I][J][r], (qrow[r] * qcol) * qn[r]);
        }
      }
      // lower tiles from the upper ones (CH block-rows per round)
      float* xb = rg + G::OFF_X;
#pragma unroll
      for (int h = 0; h < NB - 1; h += G::CH) {
#pragma unroll
        for (int I = h; I < h + G::CH && I < NB - 1; ++I)
#pragma unroll
          for (int J = I + 1; J < NB; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) xb[(16 * (I - h) + 4 * g + r) * LDX + 16 * J + c] = NV[q][I][J][r];
        wave_sync();
#pragma unroll
        for (int I = h; I < h + G::CH && I < NB - 1; ++I)
#pragma unroll
          for (int J = I + 1; J < NB; ++J) NV[q][J][I] = ld4(xb + (16 * (I - h) + c) * LDX + 16 * J + 4 * g);
        wave_sync();
      }
    }
    return false;
  };

  // Step 0: stash V_1, form W_0 and Quu_0, u0 = -Quu_0^{-1} W_0' (alpha_0 * h0).
  auto step0 = [&]() {
    {
      float* v = vecs + qo * G::VEC;
      const float alpha = fmaf(a_l, __builtin_amdgcn_exp2f(la2_o), 1.0f);
      v[li] = alpha;
      v[D + li] = alpha * h0[po * D + li];          // (A_0 h0)_li
      v[2 * D + li] = __builtin_amdgcn_exp2f(lb2_l);  // beta_0
    }
    wave_sync();
#pragma unroll
    for (int q = 0; q < PPW; ++q) {
      if (SM == STASH_V1 && pbase + q < P) {
        float* vp = kstash + pid[q] * D * D;
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
          for (int J = 0; J < NB; ++J)
#pragma unroll
            for (int r = 0; r < 4; ++r) vp[(16 * I + 4 * g + r) * D + 16 * J + c] = -NV[q][I][J][r];
      }
      v4f nW[NB][NB];
      v4f nQ[NT];
      {
        float Bk[NB][NB][4];
        load_bk(q, Bk);
        w_quu(q, Bk, nW, nQ);
      }
      // -y = -W' A_0 h0: -y[16J + c] = sum_{I,r} (-W)[16I+4g+r][16J+c] ah[16I+4g+r]
      const float* v = vecs + q * G::VEC;
      float ny[NB];
#pragma unroll
      for (int J = 0; J < NB; ++J) ny[J] = 0.f;
#pragma unroll
      for (int I = 0; I < NB; ++I) {
        const v4f ah = ld4(v + D + 16 * I + 4 * g);
#pragma unroll
        for (int J = 0; J < NB; ++J)
#pragma unroll
          for (int r = 0; r < 4; ++r) ny[J] = fmaf(nW[I][J][r], ah[r], ny[J]);
      }
#pragma unroll
      for (int J = 0; J < NB; ++J) {
        ny[J] += __shfl_xor(ny[J], 16, 64);
        ny[J] += __shfl_xor(ny[J], 32, 64);
      }
      // Quu_0 rows (upper tiles and their mirror) into the LDS row buffer
      float* qb = region(q) + G::OFF_Q;
#pragma unroll
      for (int I = 0; I < NB; ++I)
#pragma unroll
        for (int J = I; J < NB; ++J)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = -nQ[utile<NB>(I, J)][r];
            qb[(16 * I + 4 * g + r) * LDX + 16 * J + c] = x;
            if (J > I) qb[(16 * J + c) * LDX + 16 * I + 4 * g + r] = x;
          }
      wave_sync();  // every lane has read alpha*h0 before the rhs overwrites the beta slot
      if (g == 0) {
#pragma unroll
        for (int J = 0; J < NB; ++J) vecs[q * G::VEC + 2 * D + 16 * J + c] = -ny[J];  // y
      }
    }
    wave_sync();
    float aug[D + 4];
    float* qb = region(qo) + G::OFF_Q;
    ld_row<D>(qb + li * LDX, *reinterpret_cast<float(*)[D]>(aug));
    aug[D] = vecs[qo * G::VEC + 2 * D + li];
    aug[D + 1] = aug[D + 2] = aug[D + 3] = 0.f;
    if (SM == STASH_V1 && own_valid) st_global_row<D>(q0stash + (po * D + li) * D, *reinterpret_cast<float(*)[D]>(aug));
    wave_sync();  // all rows read before the pivot-row buffer (aliasing them) is written
    float piv;
    int pos;
    gauss_jordan<D, D + 4>(aug, li, qb, piv, pos);
    const float u0 = -aug[D] / piv;
    if (own_valid) {
      if (WRITE_U) u_out[po * D + pos] = u0;
      if (status != nullptr && !isfinite(u0)) atomicOr(status, TTC_LQR_STATUS_NONFINITE);
    }
  };

  int t = T - 1;
  bool failed = false;
  while (!failed && t >= 1) {
    failed = step(t);
    --t;
  }
  if (!failed) {
    step0();
    return;
  }
  // breakdown: mark the wave's problems for lqr_rescue_kernel
  if (lane < PPW && pbase + lane < P) {
    const float nan = __builtin_nanf("");
    if (WRITE_U) u_out[(pbase + lane) * D] = nan;
    else q0stash[(pbase + lane) * D * D] = nan;
  }
}

}  // namespace ttc
