// ttc_lqr_capi.hip -- C ABI of libttc_lqr.so (see include/ttc_lqr.h): argument
// validation, backward chunking and workspace layout, dispatch to the per-D kernels.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

#define TTC_LQR_VERSION_STRING "ttc-lqr-gfx950 0.2.0"

namespace ttc {

// grad_B / grad_Q: sum the per-problem partials over the H heads of each token.
__global__ void headsum_kernel(const float* __restrict__ part, int64_t N, int H, int DD,
                               float* __restrict__ out, float grad_limit, int* __restrict__ status) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * DD) return;
  const int64_t n = e / DD;
  const int r = (int)(e % DD);
  float s = 0.f;
  for (int h = 0; h < H; ++h) s += part[(n * H + h) * DD + r];
  out[e] = s;
  if (status != nullptr) {
    if (!isfinite(s)) atomicOr(status, TTC_LQR_STATUS_NONFINITE);
    else if (fabsf(s) >= grad_limit) atomicOr(status, TTC_LQR_STATUS_LARGE);
  }
}

static int launch_headsum(const float* part, int64_t N, int H, int DD, float* out, float limit, int32_t* status,
                          hipStream_t s) {
  const int64_t total = N * DD;
  if (total <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(headsum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, N, H, DD, out,
                     limit, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

struct BwdLayout {
  size_t kst, q0s, traj, gBp, gQp, total;
};

static BwdLayout bwd_layout(int64_t chunk_tokens, int H, int d, int T, bool with_stash) {
  const size_t Pc = (size_t)chunk_tokens * (size_t)H;
  BwdLayout L{};
  size_t off = 0;
  L.kst = off;
  off += with_stash ? 0 : align256(Pc * (size_t)T * d * d * sizeof(float));
  L.q0s = off;
  off += with_stash ? 0 : align256(Pc * (size_t)d * d * sizeof(float));
  L.traj = off;
  off += align256(Pc * (size_t)T * d * 4 * sizeof(float));
  L.gBp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.gQp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.total = off;
  return L;
}

}  // namespace ttc

using namespace ttc;

extern "C" {

const char* ttc_lqr_version(void) { return TTC_LQR_VERSION_STRING; }

const char* ttc_lqr_strerror(int code) {
  switch (code) {
    case TTC_LQR_OK: return "ok";
    case TTC_LQR_EINVAL: return "invalid argument (sizes, null pointer or workspace too small)";
    case TTC_LQR_EUNSUPPORTED: return "unsupported (d, du): kernels exist for d == du in {16, 32, 64}";
    case TTC_LQR_ELAUNCH: return "HIP kernel launch failed";
    default: return "unknown error";
  }
}

int ttc_lqr_supported(int32_t d, int32_t du) { return (d == du && (d == 16 || d == 32 || d == 64)) ? 1 : 0; }

int ttc_lqr_supported_flags(int32_t d, int32_t du, int32_t flags) {
  if (!ttc_lqr_supported(d, du)) return 0;
  if ((flags & TTC_LQR_FLAG_FP64_RICCATI) && d > 32) return 0;
  return (flags & ~(TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_ROW_KERNEL)) ? 0 : 1;
}

size_t ttc_lqr_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0 || T <= 0) return 0;
  const size_t P = (size_t)n_tokens * (size_t)heads;
  return sizeof(float) * P * ((size_t)T * du * d + (size_t)du * du);
}

size_t ttc_lqr_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                               int32_t with_stash) {
  if (chunk_tokens <= 0 || heads <= 0 || d <= 0 || du != d || T <= 0) return 0;
  return bwd_layout(chunk_tokens, heads, d, T, with_stash != 0).total;
}

int ttc_lqr_forward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                    const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                    int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags, float* u,
                    float* gain_stash, float* quu0_stash, int32_t* status, void* stream) {
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !u)
    return TTC_LQR_EINVAL;
  if ((gain_stash == nullptr) != (quu0_stash == nullptr)) return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (d) {
    case 16: return launch_fwd_d16(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s, flags);
    case 32: return launch_fwd_d32(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s, flags);
    case 64: return launch_fwd_d64(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, gain_stash, quu0_stash, status, s, flags);
  }
  return TTC_LQR_EUNSUPPORTED;
}

int ttc_lqr_backward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                     const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                     const float* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                     int32_t flags, const float* gain_stash, const float* quu0_stash, float* grad_A_diag, float* grad_B,
                     float* grad_Q, float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                     float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, void* workspace,
                     size_t workspace_bytes, float grad_limit, int32_t* status, void* stream) {
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !d_u ||
      !grad_A_diag || !grad_B || !grad_Q || !grad_R_inv || !grad_Q_f || !grad_log_gamma_A || !grad_log_gamma_B ||
      !grad_log_gamma_Q || !grad_h0 || !workspace)
    return TTC_LQR_EINVAL;
  if ((gain_stash == nullptr) != (quu0_stash == nullptr)) return TTC_LQR_EINVAL;
  const bool with_stash = gain_stash != nullptr;
  const size_t per_token = bwd_layout(1, heads, d, T, with_stash).total;
  if (workspace_bytes < per_token) return TTC_LQR_EINVAL;
  // largest chunk whose layout fits (layout is monotone in the chunk size)
  int64_t chunk = (int64_t)(workspace_bytes / per_token);
  if (chunk > n_tokens) chunk = n_tokens;
  while (chunk > 1 && bwd_layout(chunk, heads, d, T, with_stash).total > workspace_bytes) --chunk;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t dd = (int64_t)d * d;
  for (int64_t n0 = 0; n0 < n_tokens; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * heads, Pc = nc * heads;
    const BwdLayout L = bwd_layout(nc, heads, d, T, with_stash);
    const float* a = A_diag + p0 * d;
    const float* b = B + n0 * dd;
    const float* q = Q + n0 * dd;
    const float* r = R_inv + p0 * du;
    const float* qf = Q_f + p0 * dd;
    const float* la = log_gamma_A + p0;
    const float* lb = log_gamma_B + p0 * du;
    const float* lq = log_gamma_Q + p0 * d;
    const float* hz = h0 + p0 * d;
    const float* dz = d_u + p0 * du;
    float* kst;
    float* q0s;
    int rc = TTC_LQR_OK;
    if (with_stash) {
      kst = const_cast<float*>(gain_stash) + p0 * (int64_t)T * dd;
      q0s = const_cast<float*>(quu0_stash) + p0 * dd;
    } else {
      kst = reinterpret_cast<float*>(ws + L.kst);
      q0s = reinterpret_cast<float*>(ws + L.q0s);
      switch (d) {
        case 16: rc = launch_fwd_d16(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s, flags); break;
        case 32: rc = launch_fwd_d32(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s, flags); break;
        case 64: rc = launch_fwd_d64(a, b, q, r, qf, la, lb, lq, hz, Pc, heads, T, nullptr, kst, q0s, nullptr, s, flags); break;
      }
      if (rc != TTC_LQR_OK) return rc;
    }
    float4* traj = reinterpret_cast<float4*>(ws + L.traj);
    float* gBp = reinterpret_cast<float*>(ws + L.gBp);
    float* gQp = reinterpret_cast<float*>(ws + L.gQp);
    float* gA = grad_A_diag + p0 * d;
    float* gR = grad_R_inv + p0 * du;
    float* gQf = grad_Q_f + p0 * dd;
    float* glA = grad_log_gamma_A + p0;
    float* glB = grad_log_gamma_B + p0 * du;
    float* glQ = grad_log_gamma_Q + p0 * d;
    float* gh = grad_h0 + p0 * d;
    switch (d) {
      case 16: rc = launch_bwd_d16(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
      case 32: rc = launch_bwd_d32(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
      case 64: rc = launch_bwd_d64(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, heads, T, traj, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, status, s); break;
    }
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gBp, nc, heads, (int)dd, grad_B + n0 * dd, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gQp, nc, heads, (int)dd, grad_Q + n0 * dd, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
  }
  return TTC_LQR_OK;
}

}  // extern "C"
