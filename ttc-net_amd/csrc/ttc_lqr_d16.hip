// ttc_lqr_d16.hip -- kernels instantiated for d = du = 16.
#include "ttc_lqr_kernels.hpp"

namespace ttc {

int launch_fwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s, int flags,
                  int32_t* rescue_ws, RescueSlots rs) {
  // the stable backward's gains at long horizons: fp64 on the matrix cores
  if (sm == STASH_GAINS && (flags & TTC_LQR_FLAG_FP64_RESCUE) &&
      !(flags & (TTC_LQR_FLAG_ROW_KERNEL | TTC_LQR_FLAG_RICCATI_STEPS | TTC_LQR_FLAG_FP64_RICCATI)))
    return launch_gains64_d16(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, st_a, st_b, status, s);
  // fp64 rescue of a symplectic sweep: without a symplectic sweep to certify (the stable
  // backward's gains, row-layout or Riccati-step kernels asked for) the sweep is fp64 throughout
  if ((flags & TTC_LQR_FLAG_FP64_RESCUE) &&
      (sm == STASH_GAINS || (flags & (TTC_LQR_FLAG_ROW_KERNEL | TTC_LQR_FLAG_RICCATI_STEPS))))
    flags |= TTC_LQR_FLAG_FP64_RICCATI;
  // fp32 sweeps run on the matrix cores unless the row-layout kernel is asked for: the
  // symplectic sweep by default, per-step Riccati when asked for or when every gain is
  // stored (the stable backward)
  if (!(flags & (TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_ROW_KERNEL))) {
    if (sm != STASH_GAINS && !(flags & TTC_LQR_FLAG_RICCATI_STEPS))
      return launch_fwd_d16_sym(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, sm, status, s,
                                (flags & TTC_LQR_FLAG_FP64_RESCUE) != 0, rescue_ws, rs);
    return launch_fwd_d16_mfma(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, sm, status, s);
  }
  return launch_fwd<16, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, sm, status, s, flags);
}

int launch_bwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, void* traj, bool fp64, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s, const int32_t* gidx,
                  const double* gsl, const double* q0sl) {
  if (fp64)
    return launch_bwd<16, double>(A, B, Q, R, Qf, lA, lB, lQ, h0, dU, kst, q0s, P, H, T, static_cast<double4*>(traj),
                                 gA, gR, gQf, glA, glB, glQ, gh0, gBp, gQp, limit, status, s, gidx, gsl, q0sl);
  if (gidx != nullptr) return TTC_LQR_EINVAL;  // kept gains are fp64
  return launch_bwd<16>(A, B, Q, R, Qf, lA, lB, lQ, h0, dU, kst, q0s, P, H, T, static_cast<float4*>(traj), gA, gR,
                       gQf, glA, glB, glQ, gh0, gBp, gQp, limit, status, s);
}

int launch_ham_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                  const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                  float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* fail_list, int32_t* fail_count, int32_t* status,
                  hipStream_t s, bool fp64, const int32_t* plist,
                  const int32_t* slot_of, const double* slots, int64_t nslot) {
  if (fp64)
    return launch_ham<16, double>(A, B, Q, R, Qf, lA, lB, lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB,
                       glQ, gh0, gBp, gQp, limit, fail_list, fail_count, status, s, plist, slot_of, slots, nslot);
  return launch_ham<16>(A, B, Q, R, Qf, lA, lB, lQ, h0, u0, dU, v1s, q0s, P, H, T, tau, gA, gR, gQf, glA, glB,
                       glQ, gh0, gBp, gQp, limit, fail_list, fail_count, status, s, plist);
}

}  // namespace ttc
