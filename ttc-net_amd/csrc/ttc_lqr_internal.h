// ttc_lqr_internal.h -- per-D kernel launchers shared by the translation units of libttc_lqr.so.
//
// Forward launchers take a stash mode `sm` (STASH_NONE / STASH_GAINS / STASH_V1, see
// ttc_lqr_kernels.hpp) and its two buffers st_a (gains or V_1) and st_b (Quu_0); rescue_ws
// (optional, rescue_ws_bytes(P)) lets the fp64 rescue of a symplectic sweep pack its problems.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ttc {
// Bytes of the fp64 rescue's problem list for P problems: a 64-word header (the count in
// word 0), then one index per problem.
inline size_t rescue_ws_bytes(int64_t P) { return (size_t)(64 + (P > 0 ? P : 0)) * sizeof(int32_t); }

// TTC_LQR_FLAG_RESCUE_V1: where the d = 16 fp64 rescue keeps the fp64 V_1 and Quu_0 of list positions
// below nslot (slots[k]: 256 doubles of V_1, then 256 of Quu_0; slot_of[problem] = k).
// TTC_LQR_FLAG_RESCUE_GAINS adds every gain K_t of list positions below ngslot (<= nslot) in
// gains[k] ([T][16][16] doubles).
struct RescueSlots {
  int32_t* slot_of = nullptr;
  double* slots = nullptr;
  int64_t nslot = 0;
  double* gains = nullptr;
  int64_t ngslot = 0;
};

int launch_fwd_d16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s);
// fp64_rescue: the problems the symplectic sweep's certificate rejects are recomputed by the
// fp64 row-layout sweep (TTC_LQR_FLAG_FP64_RESCUE) instead of the fp32 rescue tiers.
int launch_fwd_d16_sym(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                       int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                       bool fp64_rescue, int32_t* rescue_ws = nullptr, RescueSlots rs = RescueSlots{});
// d = 16, fp64 on the matrix cores (ttc_lqr_d16_f64.hip): the rescue of the problems a symplectic
// sweep marked (sm = STASH_NONE / STASH_V1; rescue_ws of rescue_ws_bytes(P)), and every gain
// K_t plus Quu_0 of P problems in fp64 (the stable backward).
int launch_rescue64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        int32_t* rescue_ws, RescueSlots rs = RescueSlots{});
int launch_gains64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                       const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                       float* kst, float* q0s, int32_t* status, hipStream_t s);
// the fp64 V_1 / Quu_0 of listed problems into slots (list[0] their count, list[64 + k] the
// problems; the backward's third rollout tier)
int launch_v1slots64_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                         const float* lA, const float* lB, const float* lQ, const float* h0, int H, int T,
                         const int32_t* list, int64_t max_list, int32_t* slot_of, double* slots, int64_t nslot,
                         hipStream_t s);
int launch_fwd_d32_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        bool sym, bool fp64_rescue, int32_t* rescue_ws = nullptr);
int launch_fwd_d64_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                        const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H,
                        int T, float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s,
                        bool sym);
int launch_fwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s, int flags,
                  int32_t* rescue_ws = nullptr, RescueSlots rs = RescueSlots{});
int launch_bwd_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, void* traj, bool fp64, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s,
                   const int32_t* gidx = nullptr, const double* gsl = nullptr, const double* q0sl = nullptr);
// fp64: the row-layout Hamiltonian rollout in fp64 (long horizons, TTC_LQR_FLAG_FP64_*)
int launch_ham_d16(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                  const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                  float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* fail_list, int32_t* fail_count, int32_t* status,
                  hipStream_t s, bool fp64, const int32_t* plist = nullptr, const int32_t* slot_of = nullptr,
                  const double* slots = nullptr, int64_t nslot = 0);
int launch_fwd_d32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s, int flags,
                  int32_t* rescue_ws = nullptr);
int launch_bwd_d32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, void* traj, bool fp64, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s);
int launch_ham_d32(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                  const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                  float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* fail_list, int32_t* fail_count, int32_t* status,
                  hipStream_t s, bool fp64, const int32_t* plist = nullptr);
int launch_fwd_d64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, int64_t P, int H, int T,
                  float* u, float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s, int flags,
                  int32_t* rescue_ws = nullptr);
int launch_bwd_d64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                  const float* kst, const float* q0s, int64_t P, int H, int T, void* traj, bool fp64, float* gA,
                  float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* status, hipStream_t s);
int launch_ham_d64(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                  const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                  const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                  float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, float* gBp,
                  float* gQp, float limit, int32_t* fail_list, int32_t* fail_count, int32_t* status,
                  hipStream_t s, bool fp64, const int32_t* plist = nullptr);
// d = 16 Hamiltonian backward on the matrix cores over head groups of 8 (H % 8 == 0):
// writes the group sums of grad_B / grad_Q to gBg / gQg ([P/8, 16, 16]; when H == 8 a group
// is a token and gBg / gQg may be the final outputs) and lists rejected groups.
int launch_ham16_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                      const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                      float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                      float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                      int32_t* status, hipStream_t s);
// the same for d = 32 / 64 (d / 16 waves per head group; ttc_lqr_hamw.hpp)
int launch_ham32_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                      const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                      float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                      float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                      int32_t* status, hipStream_t s);
int launch_ham64_mfma(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                      const float* lA, const float* lB, const float* lQ, const float* h0, const float* u0,
                      const float* dU, const float* v1s, const float* q0s, int64_t P, int H, int T, float tau,
                      float* gA, float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0,
                      float* gBg, float* gQg, float limit, int32_t* fail_list, int32_t* fail_count,
                      int32_t* status, hipStream_t s);
// Low-rank front-end (ttc_lqr_factored.hip): expansion of coefficient x basis sums and
// their chain rule.  Rows of E = d * du floats; ranks R <= 64; E in {256, 1024, 4096}.
int launch_expand(const float* coeff, int64_t M, int R, const float* basis, int E, float* out, hipStream_t s);
// the same with bf16 coefficients (bit patterns), widened in registers
int launch_expand(const uint16_t* coeff, int64_t M, int R, const float* basis, int E, float* out, hipStream_t s);
int launch_project(const float* X, int64_t M, int E, const float* basis, int R, float* out, hipStream_t s);
int launch_reduce(const float* coeff, int64_t M, int R, const float* X, int E, float* partial, float* out,
                  int accumulate, hipStream_t s);
// launch_project(X, M, E, basis, R, proj) and launch_reduce(coeff, M, R, X, E, partial, out,
// accumulate) with the same results, in one pass over X when E == 256 and R <= 16.
int launch_project_reduce(const float* coeff, int64_t M, int R, const float* X, int E, const float* basis,
                          float* proj, float* partial, float* out, int accumulate, hipStream_t s);
int64_t factor_slabs(int64_t M, int R, int E);
int launch_pack_upper(const float* in, int64_t P, int D, float* out, hipStream_t s);
int launch_unpack_quu0(const float* packed, const float* B, const float* lgB, const float* Rinv, int64_t P, int H,
                       int D, float* v1, float* q0, hipStream_t s);
int launch_bf16_to_f32(const uint16_t* in, int64_t n, float* out, hipStream_t s);
int launch_f32_to_bf16(const float* in, int64_t n, uint16_t* out, hipStream_t s);
size_t factor_partial_floats(int64_t M, int R, int E);
// The body of ttc_lqr_backward (argument checks, then the backward over the given workspace);
// ttc_lqr_backward_noalloc calls it with its fixed device scratch.
int backward_entry(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                   const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                   const float* u, const float* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                   int32_t T, int32_t flags, const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                   float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A, float* grad_log_gamma_B,
                   float* grad_log_gamma_Q, float* grad_h0, void* workspace, size_t workspace_bytes,
                   float grad_limit, int32_t* status, int64_t* n_fallback, void* stream);
}  // namespace ttc
