// ttc_lqr_d64_mfma.hip -- launcher of the d = du = 64 matrix-core forward kernels (the
// certified symplectic sweep, or blocked-Cholesky Riccati steps) and their rescue pass
// (row-layout recompute of the problems the certificate rejects or whose Cholesky broke down).
#include "ttc_lqr_mfma_blk.hpp"

namespace ttc {

template <int SM, bool WU, int WPB, bool SYM, bool RESC = false>
static void launch_b64_w(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                         const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                         float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s) {
  using G = MB<64, 1, WPB, SYM>;
  const dim3 grid((unsigned)((P + WPB - 1) / WPB)), block(G::THREADS);
  hipLaunchKernelGGL((lqr_fwd_blk_kernel<64, 1, WPB, SM, WU, SYM, RESC>), grid, block, G::LDS_BYTES, s, A, B, Q, R,
                     Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status);
}

// Four-wave workgroups share one token's B and Q in LDS: every aligned group of four
// problems belongs to one token when the head count is a multiple of 4 (the symplectic
// sweep needs it; the Riccati steps fall back to one-wave workgroups otherwise).
template <int SM, bool WU>
static void launch_b64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s, bool sym) {
  if (sym && H % 4 == 0) {
    launch_b64_w<SM, WU, 4, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
    // problems the certificate rejected: Riccati steps on the matrix cores first (only the
    // workgroups that hold one run), the row layout for what still breaks down
    launch_b64_w<SM, WU, 4, false, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  } else if (H % 4 == 0)
    launch_b64_w<SM, WU, 4, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  else
    launch_b64_w<SM, WU, 1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
  launch_rescue_k<64, SM, WU>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s);
}

// Stash modes STASH_NONE and STASH_V1; the per-step gains (STASH_GAINS) come from the
// row-layout kernel.
int launch_fwd_d64_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        bool sym) {
  if (P <= 0) return TTC_LQR_OK;
  switch (sm) {
    case STASH_NONE:
      launch_b64<STASH_NONE, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym);
      break;
    case STASH_V1:
      if (u != nullptr)
        launch_b64<STASH_V1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym);
      else
        launch_b64<STASH_V1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, sym);
      break;
    default:
      return TTC_LQR_EINVAL;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
