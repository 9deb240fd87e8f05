// ttc_lqr_internal.h -- per-D kernel launchers shared by the translation units of libttc_lqr.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ttc {
int launch_fwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* kst, float* q0s, int32_t* status, hipStream_t s, int flags);
int launch_fwd_d16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* kst, float* q0s, int32_t* status, hipStream_t s);
int launch_bwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, float4* traj, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s);
int launch_fwd_d32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* kst, float* q0s, int32_t* status, hipStream_t s, int flags);
int launch_bwd_d32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, float4* traj, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s);
int launch_fwd_d64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* kst, float* q0s, int32_t* status, hipStream_t s, int flags);
int launch_bwd_d64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, float4* traj, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s);
}  // namespace ttc
