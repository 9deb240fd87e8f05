// ttc_lqr_d16_mfma.hip -- launcher of the d = du = 16 matrix-core forward kernel.
#include "ttc_lqr_mfma16.hpp"

namespace ttc {

template <int SM, bool WU>
static void launch_m16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s) {
  const dim3 grid((unsigned)((P + 3) / 4)), block(M16::THREADS);
  hipLaunchKernelGGL((lqr_fwd16_mfma_kernel<SM, WU>), grid, block, M16::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB, lQ, h0,
                     P, H, T, u, st_a, st_b, status);
}

int launch_fwd_d16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  switch (sm) {
    case STASH_NONE:
      launch_m16<STASH_NONE, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
      break;
    case STASH_GAINS:
      launch_m16<STASH_GAINS, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
      break;
    case STASH_V1:
      if (u != nullptr)
        launch_m16<STASH_V1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
      else
        launch_m16<STASH_V1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
      break;
    default:
      return TTC_LQR_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
