#pragma once
// ttc_lqr_hamw.hpp -- certified Hamiltonian backward for d = du = 32 / 64 on the matrix cores.
//
// The head-group rollout of lqr_ham16_mfma_kernel (the reference's forward Hamiltonian
// differentiation, ttc/solvers/symplectic_iter.py:764-885, rolled from lambda_1 = V_1 h_1;
// same recursion, certificate and outputs as lqr_ham_bwd_kernel) widened to D = 16 NW.
// A workgroup of NW waves rolls one head group: 8 consecutive heads of one token (H % 8 == 0),
// primal and adjoint, i.e. 16 trajectories.  Wave I owns state rows 16I..16I+15 of all 16
// trajectories in the MFMA C layout (lane (g, c) holds rows 16I+4g..16I+4g+3 of trajectory
// c; trajectory c is problem c & 7, adjoint when c >= 8).
//
// Each per-step product -- Q (q o S), B' Lambda, B (beta o U) -- is for wave I the row block
// I of a D x D times D x 16 product: NW k-blocks of 4 v_mfma_f32_16x16x4f32 with the matrix
// block [I][J] held in registers (A operand, loaded once) and trajectory block J read from
// LDS, where its owner stored it lane-major (one 16-byte read per lane).  The head-summed
// gradients grad_B += Lambda Pi (beta o U)', grad_Q += (q o S) Pi (q o S)' (Pi swaps primal
// and adjoint) are the NW output tiles of row block I, their operands read back from a
// row-major copy of the same tiles.  Three workgroup barriers per step order the exchanges:
// each region is written once per step and read only between the two barriers that follow
// its write, so single buffers suffice.  The per-problem pieces -- w_0 = -Quu_0^{-1} d_u,
// lambda_1 = V_1 h_1, the terminal certificate lambda_T = Q_f h_T and grad Q_f -- run in the
// row layout (D lanes per problem, two passes of 64 / D problems per wave).
//
// A group whose problems all pass the certificate writes its per-problem gradients and the
// group sums of grad_B / grad_Q (the token's sums when H == 8); otherwise it writes nothing
// and appends its index to fail_list, and the caller recomputes the group on the stable path.
#include "ttc_lqr_ham16.hpp"

namespace ttc {

template <int D>
struct HamW {
  static_assert(D == 32 || D == 64, "wide Hamiltonian backward: d = 32 or 64");
  static constexpr int NW = D / 16;                 // waves = row blocks
  static constexpr int THREADS = 64 * NW;
  static constexpr int MINW = D == 32 ? 3 : 2;     // waves per SIMD the registers must allow
  static constexpr int LD = Ham16::LD;              // row-major tile [state row][trajectory]
  static constexpr int RM = 16 * LD;
  static constexpr int LM = 256;                    // lane-major tile: 64 lanes x 4 rows
  static constexpr int LDT = D + 4;                 // trajectory-major rows [trajectory][state]
  static constexpr int PPP = 64 / D;                // row-layout problems per wave and pass
  static constexpr int PROW = D + 8;                // pivot row + skew
  // tile kinds: Z = q o S, X = Lambda, Y = beta o U
  static constexpr int OFF_RM = 0;                  // [3][NW] row-major tiles
  static constexpr int OFF_LM = 3 * NW * RM;        // [3][NW] lane-major tiles
  static constexpr int OFF_TS = OFF_LM + 3 * NW * LM;
  static constexpr int OFF_TL = OFF_TS + 16 * LDT;
  static constexpr int OFF_PV = OFF_TL + 16 * LDT;  // [NW][PPP] pivot rows
  static constexpr int OFF_RED = OFF_PV + NW * PPP * PROW;
  static constexpr int FLOATS = OFF_RED + NW * 8;
  static constexpr size_t LDS_BYTES = sizeof(float) * FLOATS;
  // after the rollout the NW x NW grad_Q tiles are exchanged through the tile regions
  static_assert(NW * NW * RM <= OFF_TS, "grad_Q exchange fits the rollout tiles");
};

// acc += sum_J M[I][J] X_J: row block I of a D x D by D x 16 product, X_J lane-major in LDS.
template <int NW>
__device__ __forceinline__ v4f block_product(const float (&M)[NW][4], const float* lm, int lane, v4f acc) {
#pragma unroll
  for (int J = 0; J < NW; ++J) {
    const v4f x = ld4(lm + J * 256 + 4 * lane);
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = mfma16x16x4(M[J][s], x[s], acc);
  }
  return acc;
}

// acc[J] += X_I Pi Y_J' over the trajectory index (tiles row-major in LDS, blocks RM apart):
// acc[J][i][j] += sum_k X_I[i][k] Y_J[j][k ^ 8].
template <int NW, int RM>
__device__ __forceinline__ void cross_blocks(const float* Xi, const float* Y0, int g, int c, v4f (&acc)[NW]) {
  const v4f a = ld4(Xi + c * Ham16::LD + 4 * g);
#pragma unroll
  for (int J = 0; J < NW; ++J) {
    const v4f b = ld4(Y0 + J * RM + c * Ham16::LD + 4 * (g ^ 2));
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[J] = mfma16x16x4(a[s], b[s], acc[J]);
  }
}

// acc[J] += X_I,p X_J,a' (primal trajectories of block I against the adjoints of block J),
// tiles stored by st_tile_interleaved: acc[J][i][j] += sum_{k < 8} X_I[i][k] X_J[j][k + 8].
// The full X_I Pi X_J' is acc[I][J] + acc[J][I]', formed once after the rollout.
template <int NW, int RM>
__device__ __forceinline__ void half_cross_blocks(const float* Xi, const float* X0, int g, int c, v4f (&acc)[NW]) {
  const v4f a = ld4(Xi + c * Ham16::LD + 4 * g);
#pragma unroll
  for (int J = 0; J < NW; ++J) {
    const v4f b = ld4(X0 + J * RM + c * Ham16::LD + 4 * g);
    acc[J] = mfma16x16x4(a[0], b[2], acc[J]);
    acc[J] = mfma16x16x4(a[1], b[3], acc[J]);
  }
}

template <int D, bool DIRECT>
__global__ __launch_bounds__(HamW<D>::THREADS) __attribute__((amdgpu_waves_per_eu(HamW<D>::MINW))) void lqr_hamw_mfma_kernel(
    const float* __restrict__ A_diag, const float* __restrict__ Bg, const float* __restrict__ Qg,
    const float* __restrict__ Rinv, const float* __restrict__ Qf, const float* __restrict__ lgA,
    const float* __restrict__ lgB, const float* __restrict__ lgQ, const float* __restrict__ h0,
    const float* __restrict__ u0g, const float* __restrict__ dU, const float* __restrict__ v1s,
    const float* __restrict__ q0s, int64_t P, int H, int T, float tau, float* __restrict__ gA,
    float* __restrict__ gRinv, float* __restrict__ gQf, float* __restrict__ glgA, float* __restrict__ glgB,
    float* __restrict__ glgQ, float* __restrict__ gh0, float* __restrict__ gBg, float* __restrict__ gQg,
    float grad_limit, int* __restrict__ fail_list, int* __restrict__ fail_count, int* __restrict__ status) {
  using W = HamW<D>;
  constexpr int NW = W::NW;
  constexpr int LDT = W::LDT;
  extern __shared__ __align__(16) float sm[];
  constexpr float kLog2e = 1.4426950408889634f;
  const int lane = threadIdx.x & 63;
  const int I = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // my row block
  const int g = lane >> 4;
  const int c = lane & 15;        // trajectory
  const int j = c & 7;            // its problem within the group
  const bool adj = c >= 8;
  const int r0 = 16 * I + 4 * g;  // first of my four state rows
  const int64_t G = blockIdx.x;
  if (G * 8 >= P) return;         // whole workgroups only: no barrier follows
  const int64_t p0 = G * 8;
  const int64_t n = p0 / H;       // the group's token
  const int64_t p = p0 + j;
  // row layout: D lanes per problem, PPP problems per wave and pass, two passes
  const int li = lane % D;
  const int slot = lane / D;
  float* TS = sm + W::OFF_TS;     // [trajectory][state] exchange
  float* TL = sm + W::OFF_TL;
  float* prow = sm + W::OFF_PV + (I * W::PPP + slot) * W::PROW;
  float* ZR = sm + W::OFF_RM;
  float* XR = ZR + NW * W::RM;
  float* YR = XR + NW * W::RM;
  float* ZL = sm + W::OFF_LM;
  float* XL = ZL + NW * W::LM;
  float* YL = XL + NW * W::LM;

  // ---- t = 0: adjoint feed-forward w_0 = -Quu_0^{-1} d_u (row layout) --------------
#pragma unroll 1
  for (int pa = 0; pa < 2; ++pa) {
    const int jj = (pa * NW + I) * W::PPP + slot;
    const int64_t pp = p0 + jj;
    float aug[D + 4];
    ld_global_row<D>(q0s + (pp * D + li) * D, *reinterpret_cast<float(*)[D]>(aug));
    aug[D] = dU[pp * D + li];
    aug[D + 1] = aug[D + 2] = aug[D + 3] = 0.f;
    float piv;
    int pos;
    gauss_jordan<D, D + 4, 0, D + 1>(aug, li, prow, piv, pos);
    TS[(8 + jj) * LDT + pos] = -aug[D] / piv;  // adjoint column of problem jj
  }
  __syncthreads();

  // ---- per-lane constants: rows r0..r0+3 of problem j --------------------------------
  const v4f a4 = ld4(A_diag + p * D + r0);
  v4f lb2, lq2, rinv, nrr2;  // nrr2 = -1 / (2 R_inv^2): half of d(1/R_inv)/dR_inv per lane
  {
    const v4f b = ld4(lgB + p * D + r0), q = ld4(lgQ + p * D + r0), r = ld4(Rinv + p * D + r0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      lb2[k] = b[k] * kLog2e;
      lq2[k] = q[k] * kLog2e;
      rinv[k] = r[k];
      const float rr = 1.0f / r[k];
      nrr2[k] = -0.5f * rr * rr;
    }
  }
  const float la2 = lgA[p] * kLog2e;
  v4f U = adj ? ld4(TS + c * LDT + r0) : ld4(u0g + p * D + r0);  // u_0 | w_0
  v4f S = adj ? v4f{0.f, 0.f, 0.f, 0.f} : ld4(h0 + p * D + r0);   // h_0 | h~_0 = 0
  // matrix blocks [I][J] of the token as A operands: B, B', sym(Q)
  float Bm[NW][4], Bt[NW][4], Qa[NW][4];
  {
    const float* bq = Bg + n * D * D;
    const float* qq = Qg + n * D * D;
#pragma unroll
    for (int J = 0; J < NW; ++J) {
      const v4f brow = ld4(bq + (16 * I + c) * D + 16 * J + 4 * g);
      const v4f qrow = ld4(qq + (16 * I + c) * D + 16 * J + 4 * g);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        Bm[J][s] = brow[s];
        Bt[J][s] = bq[(16 * J + 4 * g + s) * D + 16 * I + c];
        Qa[J][s] = 0.5f * (qrow[s] + qq[(16 * J + 4 * g + s) * D + 16 * I + c]);
      }
    }
  }

  const float eA0 = __builtin_amdgcn_exp2f(la2);
  v4f al0, be0, BU;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    al0[k] = fmaf(a4[k], eA0, 1.0f);
    be0[k] = __builtin_amdgcn_exp2f(lb2[k]);
    BU[k] = be0[k] * U[k];
  }
  // h_1 = alpha_0 h_0 + B (beta_0 u_0)
  st_tile_rowmajor(YR + I * W::RM, g, c, BU);
  st4(YL + I * W::LM + 4 * lane, BU);
  __syncthreads();
  const v4f S1 = block_product<NW>(Bm, YL, lane, al0 * S);
  st4(TS + c * LDT + r0, S1);  // every wave has read its w_0 column (barrier above)
  __syncthreads();
  // lambda_1 = V_1 h_1 (row layout)
#pragma unroll 1
  for (int pa = 0; pa < 2; ++pa) {
    const int jj = (pa * NW + I) * W::PPP + slot;
    const int64_t pp = p0 + jj;
    float lam = 0.f, lamb = 0.f;
#pragma unroll
    for (int k0 = 0; k0 < D; k0 += 16) {
      float vrow[16], hv[16], hbv[16];
      ld_global_row<16>(v1s + (pp * D + li) * D + k0, vrow);
      ld_row<16>(TS + jj * LDT + k0, hv);
      ld_row<16>(TS + (8 + jj) * LDT + k0, hbv);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        lam = fmaf(vrow[k], hv[k], lam);
        lamb = fmaf(vrow[k], hbv[k], lamb);
      }
    }
    TL[jj * LDT + li] = lam;
    TL[(8 + jj) * LDT + li] = lamb;
  }
  __syncthreads();
  v4f L = ld4(TL + c * LDT + r0);
  st_tile_rowmajor(XR + I * W::RM, g, c, L);
  st4(XL + I * W::LM + 4 * lane, L);
  __syncthreads();
  // B' lambda_1
  v4f BtL = block_product<NW>(Bt, XL, lane, v4f{0.f, 0.f, 0.f, 0.f});

  // per-lane partial accumulators (primal and adjoint lanes are summed at the end)
  // (grad lgB / grad R_inv: sP, sPt sum the terms of steps t >= 1 below; they start from the
  // step-0 terms, primal + adjoint lanes, in the same scaling)
  v4f accA, accLA, accLQ, accH0, sP, sPt;
  {
    const v4f Lx = swap8(L), BtLx = swap8(BtL), Ux = swap8(U);
    v4f cLB, cR;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float gAt = S[k] * Lx[k];                  // h_0 lambda~_1 (h~_0 = 0)
      accA[k] = gAt * eA0;
      accLA[k] = gAt * eA0;                            // times a at the end
      cLB[k] = be0[k] * U[k] * BtLx[k];                // beta_0 (u_0 B'lambda~_1 | w_0 B'lambda_1)
      cR[k] = U[k] * Ux[k] * nrr2[k];                  // -u_0 w_0 / R_inv^2, half per lane
      accLQ[k] = 0.f;
      accH0[k] = adj ? al0[k] * L[k] : 0.f;            // alpha_0 lambda~_1
    }
    cLB += swap8(cLB);
    cR += swap8(cR);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sP[k] = rinv[k] * cR[k];
      sPt[k] = 0.5f * cLB[k];
    }
  }
  v4f gB[NW], gQ[NW];
#pragma unroll
  for (int J = 0; J < NW; ++J) {
    gB[J] = v4f{0.f, 0.f, 0.f, 0.f};
    gQ[J] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  // grad_B += Lambda Pi (beta o U)'
  cross_blocks<NW, W::RM>(XR + I * W::RM, YR, g, c, gB);
  S = S1;

  // Steps t >= 1 need no u_t of their own: with u_t = -R^{-1} beta_t B' lambda_{t+1},
  // beta o U = -R_inv beta^2 B'Lambda, and W_t = (beta o U) o (B' Lambda~) = -R_inv beta^2 P_t,
  // P_t = (B' lambda_{t+1}) o (B' lambda~_{t+1}) (the same on primal and adjoint lanes up to
  // rounding),
  //   grad lgB:   (t+1) beta (u B'lambda~ + w B'lambda) = 2 (t+1) W,
  //   grad R_inv: -u w / R_inv^2                          = W / R_inv,
  // so the loop sums W and (t+1) W (sP, sPt; one lane of each pair suffices).
  // Discounts by recurrence: q_t = exp(lgQ t), e^{lgA (t+1)} and -R_inv beta_t^2 are multiplied
  // by their one-step factors each step and recomputed from the exponential every kRefresh
  // steps, so the rounding of the products spans at most kRefresh - 1 multiplications
  // (< 1e-6 relative).
  constexpr int kRefresh = 8;
  v4f lb4, eq, eb, q, nb2;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    lb4[k] = 2.0f * lb2[k];
    eq[k] = __builtin_amdgcn_exp2f(lq2[k]);
    eb[k] = __builtin_amdgcn_exp2f(lb4[k]);
    // held in registers: otherwise the allocator recomputes the exponentials in the loop
    asm volatile("" : "+v"(eq[k]), "+v"(eb[k]));
  }
  float ea = __builtin_amdgcn_exp2f(la2);
  asm volatile("" : "+v"(ea));
  float eA = 0.f;
  // Primal / adjoint cross terms take the partner column c ^ 8 of X1, Lambda and beta o U
  // from this wave's own row-major tiles (LDS reads instead of cross-lane moves; each term is
  // summed over the two lanes of a problem at the end, so either factor may come from the
  // partner).  Z = q o S is stored with interleaved trajectory columns (st_tile_interleaved):
  // its partner column is at (4 (c & 3) + (c >> 2)) ^ 2.
  const int cx = c ^ 8;
  const int ix = (4 * (c & 3) + (c >> 2)) ^ 2;
  float tf = 0.0f;
  for (int t = 1; t < T; ++t) {
    tf += 1.0f;
    const float tp1 = tf + 1.0f;
    if ((t - 1) % kRefresh == 0) {  // uniform branch
      eA = __builtin_amdgcn_exp2f(la2 * tp1);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        q[k] = __builtin_amdgcn_exp2f(lq2[k] * tf);
        nb2[k] = -rinv[k] * __builtin_amdgcn_exp2f(lb4[k] * tp1);
      }
    } else {
      eA *= ea;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        q[k] *= eq[k];
        nb2[k] *= eb[k];
      }
    }
    // state cost on h_t: Qc_t = D_t Q D_t, D_t = diag(exp(lgQ t))
    v4f X1;
#pragma unroll
    for (int k = 0; k < 4; ++k) X1[k] = q[k] * S[k];
    st_tile_interleaved(ZR + I * W::RM, g, c, X1);
    st4(ZL + I * W::LM + 4 * lane, X1);
    __syncthreads();  // Z written
    const v4f QX = block_product<NW>(Qa, ZL, lane, v4f{0.f, 0.f, 0.f, 0.f});
    v4f al;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // t (h Qc h~ | h~ Qc h): Qc h = q o QX, q the same on primal and adjoint lanes
      accLQ[k] = fmaf(tf * QX[k], ZR[I * W::RM + (4 * g + k) * Ham16::LD + ix], accLQ[k]);
      al[k] = fmaf(a4[k], eA, 1.0f);
      L[k] = fmaf(-q[k], QX[k], L[k]) * __builtin_amdgcn_rcpf(al[k]);
    }
    st_tile_rowmajor(XR + I * W::RM, g, c, L);
    st4(XL + I * W::LM + 4 * lane, L);
    half_cross_blocks<NW, W::RM>(ZR + I * W::RM, ZR, g, c, gQ);
    __syncthreads();  // X written, Z read
    BtL = block_product<NW>(Bt, XL, lane, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int k = 0; k < 4; ++k) BU[k] = nb2[k] * BtL[k];
    st_tile_rowmajor(YR + I * W::RM, g, c, BU);
    st4(YL + I * W::LM + 4 * lane, BU);
    const float tea = tp1 * eA;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // h_t lambda~_{t+1} | h~_t lambda_{t+1}
      const float gAt = S[k] * XR[I * W::RM + (4 * g + k) * Ham16::LD + cx];
      accA[k] = fmaf(gAt, eA, accA[k]);
      accLA[k] = fmaf(gAt, tea, accLA[k]);
    }
    __syncthreads();  // Y written, X read
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float w = BtL[k] * YR[I * W::RM + (4 * g + k) * Ham16::LD + cx];  // W_t
      sP[k] += w;
      sPt[k] = fmaf(tp1, w, sPt[k]);
    }
    // h_{t+1} = alpha_t h_t + B (beta o U);  grad_B += Lambda Pi (beta o U)'
    S = block_product<NW>(Bm, YL, lane, al * S);
    cross_blocks<NW, W::RM>(XR + I * W::RM, YR, g, c, gB);
  }
  // grad_Q tiles: gQ[I][J] + gQ[J][I]' through LDS (the rollout tiles are free now)
  __syncthreads();
#pragma unroll
  for (int J = 0; J < NW; ++J) st_tile_rowmajor(sm + (I * NW + J) * W::RM, g, c, gQ[J]);
  __syncthreads();
#pragma unroll
  for (int J = 0; J < NW; ++J) gQ[J] += ld4(sm + (J * NW + I) * W::RM + c * Ham16::LD + 4 * g);

  // ---- terminal: grad Q_f = sym(h_T h~_T'), certificate lambda_T = Q_f h_T (row layout) ----
  __syncthreads();  // T == 1: the row-layout reads of TS / TL above are done
  st4(TS + c * LDT + r0, S);
  st4(TL + c * LDT + r0, L);
  __syncthreads();
  unsigned bad = 0u;
  float fin = 0.f;
  float gmax = 0.f;  // largest guarded gradient magnitude of the lane
#pragma unroll 1
  for (int pa = 0; pa < 2; ++pa) {
    const int jj = (pa * NW + I) * W::PPP + slot;
    const int64_t pp = p0 + jj;
    const float* hs = TS + jj * LDT;
    const float* hbs = TS + (8 + jj) * LDT;
    const float lam = TL[jj * LDT + li], lamb = TL[(8 + jj) * LDT + li];
    const float hc = hs[li], hbc = hbs[li];
    const float* qfp = Qf + pp * D * D;
    float fh = 0.f, fhb = 0.f;
#pragma unroll
    for (int k0 = 0; k0 < D; k0 += 16) {
      float hv[16], hbv[16], qr[16], gq[16];
      ld_row<16>(hs + k0, hv);
      ld_row<16>(hbs + k0, hbv);
      ld_global_row<16>(qfp + li * D + k0, qr);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float qf2 = qr[k] + qfp[(k0 + k) * D + li];  // 2 sym(Q_f)
        fh = fmaf(qf2, hv[k], fh);
        fhb = fmaf(qf2, hbv[k], fhb);
        gq[k] = 0.5f * fmaf(hc, hbv[k], hbc * hv[k]);      // grad Q_f row li
        fin += fabsf(gq[k]);
        gmax = fmaxf(gmax, fabsf(gq[k]));
      }
      // stored now; a group that fails the certificate is rewritten by the stable path
      st_global_row<16>(gQf + (pp * D + li) * D + k0, gq);
    }
    fh *= 0.5f;
    fhb *= 0.5f;
    const float E1 = __uint_as_float(group_max_u32<D>(__float_as_uint(fabsf(lam - fh))));
    const float E2 = __uint_as_float(group_max_u32<D>(__float_as_uint(fabsf(lamb - fhb))));
    const float M1 = __uint_as_float(group_max_u32<D>(__float_as_uint(fabsf(fh) + fabsf(lam))));
    const float M2 = __uint_as_float(group_max_u32<D>(__float_as_uint(fabsf(fhb) + fabsf(lamb))));
    // an infinite magnitude (a trajectory beyond the fp32 range) fails: inf <= tau * inf would pass
    if (!(E1 <= tau * M1 && E2 <= tau * M2 && isfinite(M1) && isfinite(M2))) bad = 1u;
  }

  // finish the per-problem sums: primal + adjoint lanes; glgA over the D rows (all waves)
#pragma unroll
  for (int J = 0; J < NW; ++J) gQ[J] *= 0.5f;
  const v4f fA = accA + swap8(accA);
  v4f fLB, fR;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    fLB[k] = 2.0f * sPt[k];
    fR[k] = sP[k] / rinv[k];
  }
  const v4f fLQ = accLQ + swap8(accLQ), fH0 = accH0 + swap8(accH0);
  float la_part = accLA[0] * a4[0] + accLA[1] * a4[1] + accLA[2] * a4[2] + accLA[3] * a4[3];
  la_part += swap8(la_part);
  la_part += __shfl_xor(la_part, 16, 64);
  la_part += __shfl_xor(la_part, 32, 64);  // rows 16I..16I+15 of problem j
  fin += fabsf(la_part);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    fin += fabsf(fA[k]) + fabsf(fLB[k]) + fabsf(fR[k]) + fabsf(fLQ[k]) + fabsf(fH0[k]);
#pragma unroll
  for (int J = 0; J < NW; ++J)
#pragma unroll
    for (int k = 0; k < 4; ++k) fin += fabsf(gB[J][k]) + fabsf(gQ[J][k]);
  // every accumulator finite <=> the sum is (a sum of finite values overflows only near 1e38)
  if (!isfinite(fin)) bad = 1u;
  float* red = sm + W::OFF_RED;
  if (lane < 8) red[I * 8 + lane] = la_part;  // lane j = trajectory j: problem j's partial
  if (__syncthreads_or((int)bad)) {
    if (threadIdx.x == 0) fail_list[atomicAdd(fail_count, 1)] = (int)G;
    return;
  }
  float la_sum = 0.f;
#pragma unroll
  for (int J = 0; J < NW; ++J) la_sum += red[J * 8 + j];

  // Past the certificate every output of the group is finite (their magnitudes sum to the
  // finite `fin`), so the guard reduces to the largest magnitude against the limit.  The
  // reference's guard covers A_diag, B, Q, R_inv, Q_f and h0, not the log-discounts.
  if (!adj) {
#pragma unroll
    for (int k = 0; k < 4; ++k) gmax = fmaxf(gmax, fmaxf(fabsf(fA[k]), fmaxf(fabsf(fR[k]), fabsf(fH0[k]))));
    st4(gA + p * D + r0, fA);
    st4(glgB + p * D + r0, fLB);
    st4(gRinv + p * D + r0, fR);
    st4(glgQ + p * D + r0, fLQ);
    st4(gh0 + p * D + r0, fH0);
    if (I == 0 && g == 0) glgA[p] = la_sum;
  }
  // group sums of grad_B / grad_Q: rows r0 + r, columns 16J + c
  float* ob = gBg + (DIRECT ? n : G) * D * D;
  float* oq = gQg + (DIRECT ? n : G) * D * D;
#pragma unroll
  for (int J = 0; J < NW; ++J)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (DIRECT)  // the token's head sums; otherwise headsum_kernel checks the completed sums
        gmax = fmaxf(gmax, fmaxf(fabsf(gB[J][r]), fabsf(gQ[J][r])));
      ob[(r0 + r) * D + 16 * J + c] = gB[J][r];
      oq[(r0 + r) * D + 16 * J + c] = gQ[J][r];
    }
  if (gmax >= grad_limit && status != nullptr) atomicOr(status, TTC_LQR_STATUS_LARGE);
}

}  // namespace ttc

namespace ttc {

template <int D>
int launch_hamw_mfma_t(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                       const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                       float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                       float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                       int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  if (H % 8 != 0 || P % 8 != 0) return TTC_LQR_EINVAL;
  const dim3 grid((unsigned)(P / 8)), block(HamW<D>::THREADS);
  if (H == 8)
    hipLaunchKernelGGL((lqr_hamw_mfma_kernel<D, true>), grid, block, HamW<D>::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB,
                       lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh0, gBg, gQg, limit,
                       fail_list, fail_count, status);
  else
    hipLaunchKernelGGL((lqr_hamw_mfma_kernel<D, false>), grid, block, HamW<D>::LDS_BYTES, s, A, B, Q, R, Qf, lA,
                       lB, lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh0, gBg, gQg, limit,
                       fail_list, fail_count, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
