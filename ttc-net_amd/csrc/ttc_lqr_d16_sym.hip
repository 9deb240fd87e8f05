// ttc_lqr_d16_sym.hip -- launcher of the d = du = 16 symplectic matrix-core forward kernel
// and its rescue pass (the per-step Riccati kernel on the problems the certificate rejects, or
// the fp64 row-layout sweep under TTC_LQR_FLAG_FP64_RESCUE).
#include "ttc_lqr_mfma_blk.hpp"

namespace ttc {

template <int SM, bool WU>
static void launch_s16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s, bool fp64_rescue,
                       int32_t* rescue_ws, RescueSlots rs) {
  using G = MB<16, 4, 1, true>;
  using GT = MB<16, 4, 1, true, true>;
  const dim3 grid((unsigned)((P + G::PPW - 1) / G::PPW)), block(G::THREADS);
  // H % 4 == 0: the four problems of a wave are heads of one token and share its B and Q
  if (H % 4 == 0)
    hipLaunchKernelGGL((lqr_fwd_blk_kernel<16, 4, 1, SM, WU, true, false, true>), grid, block, GT::LDS_BYTES, s, A, B,
                       Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status);
  else
    hipLaunchKernelGGL((lqr_fwd_blk_kernel<16, 4, 1, SM, WU, true>), grid, block, G::LDS_BYTES, s, A, B, Q, R, Qf,
                       lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status);
  if (fp64_rescue) {
    // long horizons: the rejected problems are the ill-conditioned ones, recomputed in fp64 --
    // listed, on the matrix cores (the LU row-layout sweep finishing any whose Cholesky breaks
    // down); without a list workspace by the row-layout sweep alone
    if (rescue_ws != nullptr && launch_rescue64_d16(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, SM,
                                                    status, s, rescue_ws, rs) != TTC_LQR_EUNSUPPORTED)
      return;
    launch_rescue_k<16, SM, WU, double>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s,
                                        rescue_ws);
    return;
  }
  // rescue: the per-step Riccati kernel on the marked problems (its own breakdown guard
  // finishes on the pivoted row-layout sweep)
  const int64_t groups = (P + 3) / 4;
  hipLaunchKernelGGL((lqr_rescue16_mfma_kernel<SM, WU>), dim3((unsigned)(groups < 2048 ? groups : 2048)),
                     dim3(M16::THREADS), M16::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b,
                     status);
}

// Stash modes STASH_NONE and STASH_V1; the per-step gains (STASH_GAINS) come from the
// Riccati kernels.
int launch_fwd_d16_sym(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                       int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                       bool fp64_rescue, int32_t* rescue_ws, RescueSlots rs) {
  if (P <= 0) return TTC_LQR_OK;
  switch (sm) {
    case STASH_NONE:
      launch_s16<STASH_NONE, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, fp64_rescue,
                                   rescue_ws, rs);
      break;
    case STASH_V1:
      if (u != nullptr)
        launch_s16<STASH_V1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, fp64_rescue,
                                   rescue_ws, rs);
      else
        launch_s16<STASH_V1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, fp64_rescue,
                                    rescue_ws, rs);
      break;
    default:
      return TTC_LQR_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
