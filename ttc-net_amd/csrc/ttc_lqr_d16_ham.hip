// ttc_lqr_d16_ham.hip -- launcher of the d = du = 16 matrix-core Hamiltonian backward
// (head groups of 8; see ttc_lqr_ham16.hpp).
#include "ttc_lqr_ham16.hpp"

namespace ttc {

int launch_ham16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                      const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                      float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                      float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                      int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  if (H % 8 != 0) return TTC_LQR_EINVAL;
  const int64_t groups = P / 8;
  const dim3 grid((unsigned)((groups + Ham16::WPB - 1) / Ham16::WPB)), block(Ham16::THREADS);
  if (H == 8)
    hipLaunchKernelGGL((lqr_ham16_mfma_kernel<true>), grid, block, Ham16::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB, lQ,
                       h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh0, gBg, gQg, limit,
                       fail_list, fail_count, status);
  else
    hipLaunchKernelGGL((lqr_ham16_mfma_kernel<false>), grid, block, Ham16::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB,
                       lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh0, gBg, gQg, limit,
                       fail_list, fail_count, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
