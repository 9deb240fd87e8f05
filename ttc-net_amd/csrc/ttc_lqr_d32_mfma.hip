// ttc_lqr_d32_mfma.hip -- launcher of the d = du = 32 matrix-core forward kernels (the
// certified symplectic sweep, or blocked-Cholesky Riccati steps) and their rescue pass
// (row-layout recompute of the problems the certificate rejects or whose Cholesky broke down).
#include "ttc_lqr_mfma_blk.hpp"

namespace ttc {

template <int SM, bool WU, int PPW, int WPB, bool SYM, bool RESC = false>
static void launch_b32_w(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                         const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                         float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s) {
  using G = MB<32, PPW, WPB, SYM>;
  constexpr int PPB = PPW * WPB;
  const dim3 grid((unsigned)((P + PPB - 1) / PPB)), block(G::THREADS);
  hipLaunchKernelGGL((lqr_fwd_blk_kernel<32, PPW, WPB, SM, WU, SYM, RESC>), grid, block, G::LDS_BYTES, s, A, B, Q, R,
                     Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status);
}

// The symplectic sweep runs one-wave workgroups of 2 problems that share B and Q in LDS (an
// even head count keeps each pair in one token; at two waves per SIMD, four problems per wave
// would spill).  Riccati steps: with a head count that is a multiple of 16, 4-wave workgroups
// of 4 problems per wave share one token's B and Q in LDS (every aligned group of 16 problems
// is one token); otherwise one-wave workgroups of 2 problems keep B and Q in registers.
template <int SM, bool WU>
static void launch_b32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s, bool sym,
                       bool fp64_rescue, int32_t* rescue_ws) {
  if (fp64_rescue) {
    // long horizons (even head counts): the symplectic sweep, its rejected problems recomputed
    // by the pivoted row-layout sweep in fp64
    if (H % 8 == 0)
      launch_b32_w<SM, WU, 2, 4, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    else
      launch_b32_w<SM, WU, 2, 1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    launch_rescue_k<32, SM, WU, double>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s,
                                        rescue_ws);
    return;
  }
  if (sym && H % 2 == 0) {
    // H % 8 == 0: 4-wave workgroups of one token share its B, B' and Q in LDS
    if (H % 8 == 0)
      launch_b32_w<SM, WU, 2, 4, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    else
      launch_b32_w<SM, WU, 2, 1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    // problems the certificate rejected: Riccati steps on the matrix cores first (only the
    // workgroups that hold one run), the row layout for what still breaks down
    if (H % 16 == 0)
      launch_b32_w<SM, WU, 4, 4, false, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    else
      launch_b32_w<SM, WU, 2, 1, false, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  } else if (H % 16 == 0)
    launch_b32_w<SM, WU, 4, 4, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  else
    launch_b32_w<SM, WU, 2, 1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  launch_rescue_k<32, SM, WU>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
}

// Stash modes STASH_NONE and STASH_V1; the per-step gains (STASH_GAINS) come from the
// row-layout kernel.
int launch_fwd_d32_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        bool sym, bool fp64_rescue, int32_t* rescue_ws) {
  if (P <= 0) return TTC_LQR_OK;
  if (fp64_rescue && H % 2 != 0) return TTC_LQR_EINVAL;  // the symplectic sweep pairs heads of one token
  switch (sm) {
    case STASH_NONE:
      launch_b32<STASH_NONE, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym, fp64_rescue,
                                   rescue_ws);
      break;
    case STASH_V1:
      if (u != nullptr)
        launch_b32<STASH_V1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym,
                                   fp64_rescue, rescue_ws);
      else
        launch_b32<STASH_V1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym,
                                    fp64_rescue, rescue_ws);
      break;
    default:
      return TTC_LQR_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
