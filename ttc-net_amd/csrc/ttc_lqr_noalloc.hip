// ttc_lqr_noalloc.hip -- ttc_lqr_backward_noalloc: ttc_lqr_backward over a fixed device scratch,
// for callers that cannot allocate (tight serving loops, harnesses that forbid hipMalloc).  Like
// ttc_lqr_backward it synchronises the stream once to five times per token chunk (it reads the counts of
// problems the certificates rejected), so it cannot be recorded by HIP graph capture.
//
// The scratch is a file-scope device array of TTC_LQR_NOALLOC_SCRATCH_BYTES; every GPU the library
// runs this entry point on holds its own copy until the process ends.  Its device address is taken
// once per device with hipGetSymbolAddress (with that device current) and cached; host code never
// passes the array's name itself to a kernel or a copy (on the host that name is a stand-in, not a
// device address).  Nothing here calls hipMalloc / hipFree.  The backward keeps nothing in the
// scratch between calls that it reads before writing (its fallback counter is cleared by a kernel
// each pass), but calls that overlap on one device share the array and race: order them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

namespace {

static __device__ __align__(256) unsigned char scratch[TTC_LQR_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};
std::mutex g_mu;

// Device address of `scratch` on the current device (null if it cannot be had).
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

size_t ttc_lqr_noalloc_scratch_bytes(void) { return (size_t)TTC_LQR_NOALLOC_SCRATCH_BYTES; }

int ttc_lqr_backward_noalloc(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                             const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                             const float* log_gamma_Q, const float* h0, const float* u, const float* d_u,
                             int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags,
                             const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                             float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A, float* grad_log_gamma_B,
                             float* grad_log_gamma_Q, float* grad_h0, float grad_limit, int32_t* status,
                             int64_t* n_fallback, void* stream) {
  if (n_fallback) *n_fallback = 0;
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if (n_tokens == 0) return TTC_LQR_OK;
  // the backward walks the tokens in chunks that fit the scratch: one token's layout must fit
  if (ttc_lqr_workspace_bytes(1, heads, d, du, T, stash != nullptr ? 1 : 0, flags) > ttc_lqr_noalloc_scratch_bytes())
    return TTC_LQR_ESCRATCH;
  void* ws = scratch_ptr();
  if (ws == nullptr) return TTC_LQR_ELAUNCH;
  return ttc::backward_entry(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, u, d_u, n_tokens,
                             heads, d, du, T, flags, stash, grad_A_diag, grad_B, grad_Q, grad_R_inv, grad_Q_f,
                             grad_log_gamma_A, grad_log_gamma_B, grad_log_gamma_Q, grad_h0, ws,
                             ttc_lqr_noalloc_scratch_bytes(), grad_limit, status, n_fallback, stream);
}

}  // extern "C"
