// ttc_lqr_d64_ham.hip -- launcher of the d = du = 64 matrix-core Hamiltonian backward
// (head groups of 8, 64/16 waves per group; see ttc_lqr_hamw.hpp).
#include "ttc_lqr_hamw.hpp"

namespace ttc {

int launch_ham64_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                      const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                      float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                      float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                      int32_t* status, hipStream_t s) {
  return launch_hamw_mfma_t<64>(A, B, Q, R, Qf, lA, lB, lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA,
                                 glB, glQ, gh0, gBg, gQg, limit, fail_list, fail_count, status, s);
}

}  // namespace ttc
