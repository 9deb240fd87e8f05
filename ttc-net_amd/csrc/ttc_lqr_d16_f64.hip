// ttc_lqr_d16_f64.hip -- launchers of the d = du = 16 fp64 matrix-core Riccati sweep
// (lqr_fwd64_mfma_kernel): the long-horizon rescue of a symplectic sweep's rejected problems and
// the stable backward's fp64 gains.
#include "ttc_lqr_mfma64.hpp"

namespace ttc {

namespace {

// Waves of the fp64 matrix-core kernel resident on the device (one per block).
template <int SM, bool WU, bool LISTED, bool SYMP = false>
int64_t resident_waves64() {
  const int cus = device_cus();
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, lqr_fwd64_mfma_kernel<SM, WU, LISTED, SYMP>, 64,
                                                   M64::LDS_BYTES) != hipSuccess ||
      per_cu <= 0)
    per_cu = 4;
  return (int64_t)(cus > 0 ? cus : 256) * per_cu;
}

}  // namespace

// The problems a symplectic sweep marked (u[p][0], or Quu_0[p][0][0] without u, is NaN), listed,
// in fp64 on the matrix cores.  TTC_LQR_EUNSUPPORTED (nothing launched) when the device's CU
// count is unknown or P too large for the list.
template <int SM, bool WU>
static int rescue64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                    const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                    float* u, float* st_a, float* st_b, int32_t* status, hipStream_t s, int32_t* rescue_ws,
                    const RescueSlots& rs) {
  if (device_cus() <= 0 || P >= ((int64_t)1 << 31)) return TTC_LQR_EUNSUPPORTED;
  const float* mark = WU ? u : st_b;
  const int64_t mstride = WU ? 16 : 256;
  hipLaunchKernelGGL(rescue_list_reset_kernel, dim3(1), dim3(1), 0, s, rescue_ws);
  hipLaunchKernelGGL(rescue_list_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, P, mark, mstride,
                     rescue_ws, status);
  const int64_t waves = resident_waves64<SM, WU, true>();
  hipLaunchKernelGGL((lqr_fwd64_mfma_kernel<SM, WU, true>), dim3((unsigned)waves), dim3(64), M64::LDS_BYTES, s, A,
                     B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, rescue_ws, rs.slot_of, rs.slots,
                     rs.nslot, rs.gains, rs.ngslot);
  return TTC_LQR_OK;  // launch errors are the caller's to collect (hipGetLastError)
}

int launch_rescue64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        int32_t* rescue_ws, RescueSlots rs) {
  if (P <= 0) return TTC_LQR_OK;
  if (rescue_ws == nullptr) return TTC_LQR_EINVAL;
  switch (sm) {
    case STASH_NONE:
      return rescue64<STASH_NONE, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s, rescue_ws,
                                        RescueSlots{});
    case STASH_V1:
      if (u != nullptr)
        return rescue64<STASH_V1, true>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s,
                                        rescue_ws, rs);
      return rescue64<STASH_V1, false>(A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, u, st_a, st_b, status, s,
                                       rescue_ws, rs);
  }
  return TTC_LQR_EINVAL;
}

// fp64 V_1 and Quu_0 of listed problems by the fp64 symplectic sweep on the matrix cores: list[0]
// (on the device) is their count, at most max_list, and list[64 + k] problem k; the values of a
// problem that passes the sweep's certificate go to slots[k] (2 x 256 doubles) and k to
// slot_of[problem] (the others keep slot_of -1).  Nothing else is written.  The backward's third
// rollout tier.
int launch_v1slots64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                         const float* lA, const float* lB, const float* lQ, const float* h0, int H, int T,
                         const int32_t* list, int64_t max_list, int32_t* slot_of, double* slots, int64_t nslot,
                         hipStream_t s) {
  if (max_list <= 0) return TTC_LQR_OK;
  if (device_cus() <= 0) return TTC_LQR_EUNSUPPORTED;
  // the kernel takes ceil(count / waves) problems per wave (at most four)
  const int64_t res = resident_waves64<STASH_V1, false, true, true>();
  const int64_t waves = max_list < res ? max_list : res;
  hipLaunchKernelGGL((lqr_fwd64_mfma_kernel<STASH_V1, false, true, true>), dim3((unsigned)waves), dim3(64),
                     M64::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB, lQ, h0, max_list, H, T, nullptr, nullptr, nullptr,
                     nullptr, list, slot_of, slots, nslot);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

// Every gain K_t [P,T,16,16] and Quu_0 [P,16,16] in fp64 (the stable backward), on the matrix
// cores.
int launch_gains64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* kst, float* q0s, int32_t* status, hipStream_t s) {
  if (P <= 0) return TTC_LQR_OK;
  // as many waves as fit at once, up to one per problem: the kernel then takes ceil(P / waves)
  // problems per wave (at most four), so a pass shorter than four per wave runs fewer per wave
  const int64_t res = resident_waves64<STASH_GAINS, false, false>();
  const int64_t waves = P < res ? P : res;
  hipLaunchKernelGGL((lqr_fwd64_mfma_kernel<STASH_GAINS, false, false>), dim3((unsigned)waves), dim3(64),
                     M64::LDS_BYTES, s, A, B, Q, R, Qf, lA, lB, lQ, h0, P, H, T, nullptr, kst, q0s, status, nullptr);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
