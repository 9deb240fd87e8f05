// ttc_lqr_d16_mfma.hip -- launcher of the d = du = 16 matrix-core forward kernel.
#include "ttc_lqr_mfma16.cuh"

namespace ttc {

int launch_fwd_d16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* kst, float* q0s, int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  const dim3 grid((unsigned)((P + 3) / 4)), block(M16::THREADS);
  const size_t sh = M16::LDS_BYTES;
  if (kst != nullptr) {
    if (u != nullptr)
      hipLaunchKernelGGL((lqr_fwd16_mfma_kernel<true, true>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P,
                         H, T, u, kst, q0s, status);
    else
      hipLaunchKernelGGL((lqr_fwd16_mfma_kernel<true, false>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0,
                         P, H, T, u, kst, q0s, status);
  } else {
    hipLaunchKernelGGL((lqr_fwd16_mfma_kernel<false, true>), grid, block, sh, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P,
                       H, T, u, kst, q0s, status);
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
