// ttc_lqr_capi.hip -- C ABI of libttc_lqr.so (see include/ttc_lqr.h): argument
// validation, workspace layouts, the backward's fast path and its per-problem
// fallback, dispatch to the per-D kernels.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

#define TTC_LQR_VERSION_STRING "ttc-lqr-gfx950 0.3.0"

namespace ttc {

constexpr int kStashV1 = 2;     // STASH_V1 of ttc_lqr_kernels.hpp
constexpr int kStashGains = 1;  // STASH_GAINS

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

__global__ void set_i32_kernel(int* p, int v) { *p = v; }

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Third rollout tier: of the n problems the fp64 tier rejected (list), those without an fp64 V_1
// of the forward's (slot_of null, or slot_of[p] < 0) go to list3[64 + k] for k < n3 (count in
// c3, may exceed n3), the rest to the stable path's list (count in cs).
__global__ void tier3_split_kernel(const int* __restrict__ list, int64_t n, const int32_t* __restrict__ slot_of,
                                   int32_t* __restrict__ list3, int64_t n3, int32_t* c3, int32_t* __restrict__ stable,
                                   int32_t* cs) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int32_t p = list[e];
  if (slot_of == nullptr || slot_of[p] < 0) {
    const int32_t k = atomicAdd(c3, 1);
    if (k < n3) {
      list3[64 + k] = p;
      return;
    }
  }
  stable[atomicAdd(cs, 1)] = p;
}

// list3[0] = the third tier's problem count, min(c3, n3)
__global__ void tier3_close_kernel(const int32_t* c3, int64_t n3, int32_t* list3) {
  const int32_t c = *c3;
  list3[0] = c < n3 ? c : (int32_t)n3;
}

// The stable path's n problems (list) reordered into out[0 .. n): first those whose gains the
// forward did not keep (count in cr), then those it kept, with a slot below ngslot (count in ck).
__global__ void kept_split_kernel(const int* __restrict__ list, int64_t n, const int32_t* __restrict__ slot_of,
                                  int64_t ngslot, int32_t* __restrict__ out, int32_t* ck, int32_t* cr) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int32_t p = list[e];
  const int32_t k = slot_of[p];
  if (k >= 0 && k < ngslot) out[n - 1 - atomicAdd(ck, 1)] = p;
  else out[atomicAdd(cr, 1)] = p;
}

// Slots of the listed problems list[base + i], i < n, whose gains are kept: -1 for the first
// nrest of the list (swept), slot_of[problem] for the others.
__global__ void gather_slot_kernel(const int* __restrict__ list, int64_t base, int64_t n, int64_t nrest,
                                   const int32_t* __restrict__ slot_of, int32_t* __restrict__ gi) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) gi[i] = (base + i < nrest) ? -1 : slot_of[list[base + i]];
}

// The nine inputs and d_u of the listed problems (chunk-local indices), gathered into
// contiguous arrays of `cnt` one-head problems (the head-shared B and Q are copied per
// problem), so the stable path can recompute them as cnt tokens with H = 1.
struct Compact {
  float *A, *B, *Q, *R, *Qf, *lA, *lB, *lQ, *h0, *dU;               // inputs
  float *gA, *gB, *gQ, *gR, *gQf, *glA, *glB, *glQ, *gh0;            // gradients
  int32_t* gi;  // TTC_LQR_FLAG_RESCUE_GAINS: each problem's slot of kept gains
};

__device__ __forceinline__ void copy_span(float* __restrict__ dst, const float* __restrict__ src, int n) {
  for (int e = threadIdx.x; e < n; e += blockDim.x) dst[e] = src[e];
}

__global__ void gather_kernel(const int* __restrict__ list, int64_t base, int H, int d, int du,
                              const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ Q,
                              const float* __restrict__ R, const float* __restrict__ Qf, const float* __restrict__ lA,
                              const float* __restrict__ lB, const float* __restrict__ lQ,
                              const float* __restrict__ h0, const float* __restrict__ dU, Compact c) {
  const int64_t i = blockIdx.x;
  const int64_t p = list[base + i];
  const int64_t n = p / H;
  copy_span(c.A + i * d, A + p * d, d);
  copy_span(c.B + i * d * du, B + n * d * du, d * du);
  copy_span(c.Q + i * d * d, Q + n * d * d, d * d);
  copy_span(c.R + i * du, R + p * du, du);
  copy_span(c.Qf + i * d * d, Qf + p * d * d, d * d);
  copy_span(c.lA + i, lA + p, 1);
  copy_span(c.lB + i * du, lB + p * du, du);
  copy_span(c.lQ + i * d, lQ + p * d, d);
  copy_span(c.h0 + i * d, h0 + p * d, d);
  copy_span(c.dU + i * du, dU + p * du, du);
}

__global__ void scatter_kernel(const int* __restrict__ list, int64_t base, int d, int du, Compact c,
                               float* __restrict__ gA, float* __restrict__ gR, float* __restrict__ gQf,
                               float* __restrict__ glA, float* __restrict__ glB, float* __restrict__ glQ,
                               float* __restrict__ gh0, float* __restrict__ gBp, float* __restrict__ gQp) {
  const int64_t i = blockIdx.x;
  const int64_t p = list[base + i];
  copy_span(gA + p * d, c.gA + i * d, d);
  copy_span(gR + p * du, c.gR + i * du, du);
  copy_span(gQf + p * d * d, c.gQf + i * d * d, d * d);
  copy_span(glA + p, c.glA + i, 1);
  copy_span(glB + p * du, c.glB + i * du, du);
  copy_span(glQ + p * d, c.glQ + i * d, d);
  copy_span(gh0 + p * d, c.gh0 + i * d, d);
  copy_span(gBp + p * d * du, c.gB + i * d * du, d * du);  // one-head problems: grad_B is the partial
  copy_span(gQp + p * d * d, c.gQ + i * d * d, d * d);
}

// Head groups (8 consecutive heads of one token, chunk-local index list[base + i]) gathered
// as compact 8-head tokens for the stable path, and their gradients scattered back: per
// problem, and the group's sums of grad_B / grad_Q (to the token's outputs when H == 8).
__global__ void gather_group_kernel(const int* __restrict__ list, int64_t base, int H, int d, int du,
                                    const float* __restrict__ A, const float* __restrict__ B,
                                    const float* __restrict__ Q, const float* __restrict__ R,
                                    const float* __restrict__ Qf, const float* __restrict__ lA,
                                    const float* __restrict__ lB, const float* __restrict__ lQ,
                                    const float* __restrict__ h0, const float* __restrict__ dU, Compact c) {
  const int64_t i = blockIdx.x;
  const int64_t p0 = (int64_t)list[base + i] * 8;
  const int64_t n = p0 / H;
  const int64_t q0 = i * 8;  // compact problems of this group
  copy_span(c.B + i * d * du, B + n * d * du, d * du);
  copy_span(c.Q + i * d * d, Q + n * d * d, d * d);
  copy_span(c.A + q0 * d, A + p0 * d, 8 * d);
  copy_span(c.R + q0 * du, R + p0 * du, 8 * du);
  copy_span(c.Qf + q0 * d * d, Qf + p0 * d * d, 8 * d * d);
  copy_span(c.lA + q0, lA + p0, 8);
  copy_span(c.lB + q0 * du, lB + p0 * du, 8 * du);
  copy_span(c.lQ + q0 * d, lQ + p0 * d, 8 * d);
  copy_span(c.h0 + q0 * d, h0 + p0 * d, 8 * d);
  copy_span(c.dU + q0 * du, dU + p0 * du, 8 * du);
}

__global__ void scatter_group_kernel(const int* __restrict__ list, int64_t base, int H, int d, int du, Compact c,
                                     float* __restrict__ gA, float* __restrict__ gR, float* __restrict__ gQf,
                                     float* __restrict__ glA, float* __restrict__ glB, float* __restrict__ glQ,
                                     float* __restrict__ gh0, float* __restrict__ gBg, float* __restrict__ gQg) {
  const int64_t i = blockIdx.x;
  const int64_t G = list[base + i];
  const int64_t p0 = G * 8;
  const int64_t q0 = i * 8;
  const int64_t o = (H == 8) ? p0 / H : G;
  copy_span(gA + p0 * d, c.gA + q0 * d, 8 * d);
  copy_span(gR + p0 * du, c.gR + q0 * du, 8 * du);
  copy_span(gQf + p0 * d * d, c.gQf + q0 * d * d, 8 * d * d);
  copy_span(glA + p0, c.glA + q0, 8);
  copy_span(glB + p0 * du, c.glB + q0 * du, 8 * du);
  copy_span(glQ + p0 * d, c.glQ + q0 * d, 8 * d);
  copy_span(gh0 + p0 * d, c.gh0 + q0 * d, 8 * d);
  copy_span(gBg + o * d * du, c.gB + i * d * du, d * du);
  copy_span(gQg + o * d * d, c.gQ + i * d * d, d * d);
}

// Problems of the listed head groups (8 per group, chunk-local indices) for the second tier.
__global__ void expand_groups_kernel(const int* __restrict__ glist, int64_t ngroups, int* __restrict__ plist) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < ngroups * 8) plist[e] = glist[e / 8] * 8 + (int)(e % 8);
}

// grad_B / grad_Q of the listed head groups as the sums of their eight problems' partials
// (part, at the problems' own indices) into the group's slot of out -- the token's output when
// H == 8, checked against the guard there (status non-null).
__global__ void groupsum_kernel(const int* __restrict__ glist, int64_t ngroups, const float* __restrict__ part,
                                int DD, float* __restrict__ out, float grad_limit, int* __restrict__ status) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= ngroups * DD) return;
  const int64_t G = glist[e / DD];
  const int r = (int)(e % DD);
  float s = 0.f;
  for (int k = 0; k < 8; ++k) s += part[(G * 8 + k) * DD + r];
  out[G * DD + r] = s;
  if (status != nullptr) {
    if (!isfinite(s)) atomicOr(status, TTC_LQR_STATUS_NONFINITE);
    else if (fabsf(s) >= grad_limit) atomicOr(status, TTC_LQR_STATUS_LARGE);
  }
}

static int launch_groupsum(const int32_t* glist, int64_t ngroups, const float* part, int DD, float* out,
                           float limit, int32_t* status, hipStream_t s) {
  const int64_t total = ngroups * DD;
  if (total <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(groupsum_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, glist, ngroups, part,
                     DD, out, limit, status);
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
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

// ---- stable path: gains recomputed (or stashed), closed-loop costates ----------------
// The stable path runs in fp64 under any fp64 flag (kernels for d <= 32).
static bool fp64_stable(int flags, int d) {
  return (flags & (TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_FP64_RESCUE | TTC_LQR_FLAG_FP64_FALLBACK)) != 0 &&
         d <= 32;
}

// The fast path's Hamiltonian rollout runs in fp64 (row layout) under the long-horizon flags;
// under TTC_LQR_FLAG_FP64_FALLBACK it stays the fp32 rollout.
static bool fp64_rollout(int flags, int d) {
  return (flags & (TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_FP64_RESCUE)) != 0 && d <= 32;
}

// Flags of a forward sweep (stash mode sm): TTC_LQR_FLAG_FP64_FALLBACK's forward is
// TTC_LQR_FLAG_FP64_RESCUE's -- the fp32 symplectic sweep with its rejected problems recomputed in
// fp64, and the stable path's gains in fp64 -- except at d = 32 with an odd head count, which has
// no symplectic sweep to certify and keeps the fp32 Riccati-step tiers for u and the stash.
static int forward_flags(int flags, int d, int H, int sm) {
  if (!(flags & TTC_LQR_FLAG_FP64_FALLBACK)) return flags;
  flags &= ~TTC_LQR_FLAG_FP64_FALLBACK;
  if (sm != kStashGains && d == 32 && H % 2 != 0) return flags;
  return flags | TTC_LQR_FLAG_FP64_RESCUE;
}

struct StableLayout {
  size_t kst, q0s, traj, gBp, gQp, total;
};

static StableLayout stable_layout(int64_t chunk_tokens, int H, int d, int T, bool fp64) {
  const size_t Pc = (size_t)chunk_tokens * (size_t)H;
  const size_t e = fp64 ? sizeof(double) : sizeof(float);  // the sweep's arithmetic
  StableLayout L{};
  size_t off = 0;
  L.kst = off;  // gains K_t
  off += align256(Pc * (size_t)T * d * d * e);
  L.q0s = off;  // Quu_0
  off += align256(Pc * (size_t)d * d * e);
  L.traj = off;  // (h, h~, u, w) per step
  off += align256(Pc * (size_t)T * d * 4 * e);
  L.gBp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.gQp = off;
  off += align256(Pc * (size_t)d * d * sizeof(float));
  L.total = off;
  return L;
}

static int fwd_d(int d, const float* a, const float* b, const float* q, const float* r, const float* qf,
                 const float* la, const float* lb, const float* lq, const float* hz, int64_t P, int H, int T, float* u,
                 float* st_a, float* st_b, int sm, int32_t* status, hipStream_t s, int flags,
                 int32_t* rescue_ws = nullptr, RescueSlots rs = RescueSlots{}) {
  flags = forward_flags(flags, d, H, sm);
  switch (d) {
    case 16:
      return launch_fwd_d16(a, b, q, r, qf, la, lb, lq, hz, P, H, T, u, st_a, st_b, sm, status, s, flags, rescue_ws,
                            rs);
    case 32:
      return launch_fwd_d32(a, b, q, r, qf, la, lb, lq, hz, P, H, T, u, st_a, st_b, sm, status, s, flags, rescue_ws);
    case 64:
      return launch_fwd_d64(a, b, q, r, qf, la, lb, lq, hz, P, H, T, u, st_a, st_b, sm, status, s, flags, rescue_ws);
  }
  return TTC_LQR_EUNSUPPORTED;
}

// Gradients of every problem by the stable path, token chunk by token chunk inside ws.
// limit: the magnitude guard of the per-problem gradients; sum_limit: that of the head sums
// of grad_B / grad_Q (INFINITY where they are partial sums that a later head sum completes).
static int stable_backward(const float* A, const float* B, const float* Q, const float* R, const float* Qf,
                           const float* lA, const float* lB, const float* lQ, const float* h0, const float* dU,
                           int64_t n_tokens, int H, int d, int T, int flags, float* gA, float* gB, float* gQ,
                           float* gR, float* gQf, float* glA, float* glB, float* glQ, float* gh0, char* ws,
                           size_t ws_bytes, float limit, float sum_limit, int32_t* status, hipStream_t s,
                           const int32_t* gidx = nullptr, const double* gsl = nullptr,
                           const double* q0sl = nullptr, int64_t nsweep = -1) {
  // gidx (d = 16, fp64): a problem p with gidx[p] >= 0 has the gains and Quu_0 the forward
  // rescue kept in slot gidx[p] (gsl, q0sl); the sweep then runs over the first nsweep problems
  // only (the others must all have one)
  const bool fp64 = fp64_stable(flags, d);
  if (gidx != nullptr && (d != 16 || !fp64)) return TTC_LQR_EINVAL;
  if (ws_bytes < stable_layout(1, H, d, T, fp64).total) return TTC_LQR_EINVAL;
  int64_t chunk = 1, hi = n_tokens;  // largest token chunk whose layout fits
  while (chunk < hi) {
    const int64_t mid = chunk + (hi - chunk + 1) / 2;
    if (stable_layout(mid, H, d, T, fp64).total <= ws_bytes) chunk = mid;
    else hi = mid - 1;
  }
  const int64_t dd = (int64_t)d * d;
  for (int64_t n0 = 0; n0 < n_tokens; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * H, Pc = nc * H;
    const StableLayout L = stable_layout(nc, H, d, T, fp64);
    const float *a = A + p0 * d, *b = B + n0 * dd, *q = Q + n0 * dd, *r = R + p0 * d, *qf = Qf + p0 * dd;
    const float *la = lA + p0, *lb = lB + p0 * d, *lq = lQ + p0 * d, *hz = h0 + p0 * d, *dz = dU + p0 * d;
    float* kst = reinterpret_cast<float*>(ws + L.kst);
    float* q0s = reinterpret_cast<float*>(ws + L.q0s);
    int rc = TTC_LQR_OK;
    int64_t sw = Pc;  // problems of this chunk that the sweep takes (the leading ones)
    if (gidx != nullptr && nsweep >= 0) sw = nsweep <= p0 ? 0 : (nsweep - p0 < Pc ? nsweep - p0 : Pc);
    if (sw > 0) {
      rc = fwd_d(d, a, b, q, r, qf, la, lb, lq, hz, sw, H, T, nullptr, kst, q0s, kStashGains, nullptr, s, flags);
      if (rc != TTC_LQR_OK) return rc;
    }
    void* traj = ws + L.traj;
    float* gBp = reinterpret_cast<float*>(ws + L.gBp);
    float* gQp = reinterpret_cast<float*>(ws + L.gQp);
    switch (d) {
      case 16: rc = launch_bwd_d16(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, H, T, traj, fp64, gA + p0 * d, gR + p0 * d, gQf + p0 * dd, glA + p0, glB + p0 * d, glQ + p0 * d, gh0 + p0 * d, gBp, gQp, limit, status, s, gidx ? gidx + p0 : nullptr, gsl, q0sl); break;
      case 32: rc = launch_bwd_d32(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, H, T, traj, fp64, gA + p0 * d, gR + p0 * d, gQf + p0 * dd, glA + p0, glB + p0 * d, glQ + p0 * d, gh0 + p0 * d, gBp, gQp, limit, status, s); break;
      case 64: rc = launch_bwd_d64(a, b, q, r, qf, la, lb, lq, hz, dz, kst, q0s, Pc, H, T, traj, fp64, gA + p0 * d, gR + p0 * d, gQf + p0 * dd, glA + p0, glB + p0 * d, glQ + p0 * d, gh0 + p0 * d, gBp, gQp, limit, status, s); break;
      default: return TTC_LQR_EUNSUPPORTED;
    }
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gBp, nc, H, (int)dd, gB + n0 * dd, sum_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gQp, nc, H, (int)dd, gQ + n0 * dd, sum_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
  }
  return TTC_LQR_OK;
}

// ---- fast path: Hamiltonian rollout, fallback region for the problems it rejects ----
static size_t compact_floats(int d, int du) {  // inputs + gradients of one problem
  const size_t in = (size_t)d + d * du + d * d + du + d * d + 1 + du + d + d + du;
  const size_t out = (size_t)d + d * du + d * d + du + d * d + 1 + du + d + d;
  return in + out;
}

// The 19 compact arrays (inputs and gradients) of F gathered problems, then a slot index each.
static size_t compact_sizes(int64_t F64, int d, int du, size_t (&sizes)[19]) {
  const size_t F = (size_t)F64;
  const size_t v[19] = {F * d, F * d * du, F * d * d, F * du, F * d * d, F, F * du, F * d, F * d, F * du,
                        F * d, F * d * du, F * d * d, F * du, F * d * d, F, F * du, F * d, F * d};
  size_t total = 0;
  for (int k = 0; k < 19; ++k) {
    sizes[k] = v[k];
    total += align256(v[k] * sizeof(float));
  }
  return total + align256(F * sizeof(int32_t));
}

// Bytes of the fallback region for F rejected problems: their compact inputs and gradients,
// then the stable path's layout for all of them in one pass.
static size_t fallback_bytes(int64_t F, int d, int du, int T, bool fp64) {
  size_t sizes[19];
  return compact_sizes(F, d, du, sizes) + stable_layout(F, 1, d, T, fp64).total;
}

// Rejected problems one fallback pass can take within `bytes`: a multiple of 8 (the head
// group of the matrix-core backward), at least 8.
static int64_t fallback_capacity(size_t bytes, int d, int du, int T, bool fp64) {
  if (bytes > ((size_t)1 << 50)) bytes = (size_t)1 << 50;  // keeps the products below in range
  if (fallback_bytes(8, d, du, T, fp64) > bytes) return 8;
  int64_t fit = 1;  // in units of 8 problems: 8 * fit fits, 16 * fit does not
  while (fallback_bytes(16 * fit, d, du, T, fp64) <= bytes) fit *= 2;
  int64_t lo = fit, hi = 2 * fit - 1;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (fallback_bytes(8 * mid, d, du, T, fp64) <= bytes) lo = mid;
    else hi = mid - 1;
  }
  return 8 * lo;
}

// Problems one round of the fp64 row-layout sweep holds on the current device: 64 / d problems
// per wave, one wave per SIMD (their registers allow no more), four SIMDs per CU.  A fallback
// pass of a multiple of this many problems fills every round it starts; each round is a serial
// T-step sweep, so a pass that ends with a part-filled round wastes most of one.
static int64_t fp64_round_problems(int d) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 0;
  return (int64_t)(64 / d) * 4 * cus;
}

// Fallback region reserved by the workspace size queries; a larger workspace gives the
// fallback larger passes (backward_core uses whatever the main chunk leaves).
constexpr size_t kFallbackReserve = (size_t)256 << 20;

struct FastLayout {
  size_t v1, q0, gBp, gQp, gBg, gQg, list, glist, plist, cnt, l3, so3, sl3, fb, total;
  int64_t F;   // fallback capacity within the reserve
  int64_t n3;  // problems the third rollout tier can take (0: no third tier)
};

// The fast path rolls head groups of 8 on the matrix cores in fp32 (H % 8 == 0), else one
// problem per row-layout rollout (fp32, or fp64 under the long-horizon flags).
static bool head_group_path(int H, int flags, int d) {
  (void)d;
  return H % 8 == 0 && !(flags & TTC_LQR_FLAG_ROW_KERNEL);
}

// Under the long-horizon flags the head-group rollout is the first of two tiers: the problems
// of the groups it rejects are rolled again one by one in fp64 on the row layout, and only
// those that rollout rejects take the stable path.
static bool two_tier_path(int H, int flags, int d) { return head_group_path(H, flags, d) && fp64_rollout(flags, d); }

// At d = du = 16 a third tier follows: the problems the fp64 rollout rejects that started from
// the fp32 stash's V_1 get an fp64 V_1 / Quu_0 from an fp64 sweep on the matrix cores and are
// rolled once more from it, up to one problem in eight of the chunk (the rest of them, and
// whatever that rollout rejects, take the stable path).
static int64_t tier3_problems(int64_t Pc, int H, int flags, int d, int du) {
  if (!two_tier_path(H, flags, d) || d != 16 || du != 16) return 0;
  const int64_t s = Pc / 8 > 64 ? Pc / 8 : 64;
  return s < Pc ? s : Pc;
}

static FastLayout fast_layout(int64_t chunk_tokens, int H, int d, int du, int T, bool with_stash, int flags) {
  const bool fp64 = fp64_stable(flags, d);
  const bool groups = head_group_path(H, flags, d);
  const bool tiers = two_tier_path(H, flags, d);
  const size_t Pc = (size_t)chunk_tokens * (size_t)H;
  // partial grad_B / grad_Q sums, added up per token by the head sum: one per problem of the
  // row-layout rollouts (per problem index; under two tiers for the second tier's problems),
  // one per head group (none when a group is the whole token: it writes the outputs)
  const size_t gparts = groups ? (size_t)chunk_tokens * (size_t)(H == 8 ? 0 : H / 8) : 0;
  const size_t parts = (!groups || tiers) ? Pc : 0;
  FastLayout L{};
  size_t off = 0;
  L.v1 = off;
  off += with_stash ? 0 : align256(Pc * (size_t)d * d * sizeof(float));
  L.q0 = off;
  off += with_stash ? 0 : align256(Pc * (size_t)du * du * sizeof(float));
  L.gBp = off;
  off += align256(parts * (size_t)d * du * sizeof(float));
  L.gQp = off;
  off += align256(parts * (size_t)d * d * sizeof(float));
  L.gBg = off;
  off += align256(gparts * (size_t)d * du * sizeof(float));
  L.gQg = off;
  off += align256(gparts * (size_t)d * d * sizeof(float));
  L.list = off;
  off += align256(Pc * sizeof(int32_t));
  L.glist = off;
  off += tiers ? align256(Pc / 8 * sizeof(int32_t)) : 0;
  L.plist = off;
  off += tiers ? align256(Pc * sizeof(int32_t)) : 0;
  L.cnt = off;  // [0]: rejected problems (or groups), [1] / [2]: the second / third tier's,
  off += 256;   // [3]: the stable path's problems after the third tier
  L.n3 = tier3_problems((int64_t)Pc, H, flags, d, du);
  L.l3 = off;   // the third tier's list: count, then its problems from index 64
  off += L.n3 > 0 ? align256((size_t)(64 + L.n3) * sizeof(int32_t)) : 0;
  L.so3 = off;  // slot per chunk problem (-1: none)
  off += L.n3 > 0 ? align256(Pc * sizeof(int32_t)) : 0;
  L.sl3 = off;  // fp64 V_1 / Quu_0 per slot
  off += align256((size_t)L.n3 * ((size_t)d * d + (size_t)du * du) * sizeof(double));
  L.fb = off;
  const int64_t cap = fallback_capacity(kFallbackReserve, d, du, T, fp64);
  L.F = (int64_t)Pc < cap ? (int64_t)Pc : cap;
  L.total = off + fallback_bytes(L.F, d, du, T, fp64);
  return L;
}

static Compact compact_at(char* base, int64_t F64, int d, int du) {
  size_t sizes[19];
  compact_sizes(F64, d, du, sizes);
  float* ptr[19];
  size_t off = 0;
  for (int k = 0; k < 19; ++k) {
    ptr[k] = reinterpret_cast<float*>(base + off);
    off += align256(sizes[k] * sizeof(float));
  }
  Compact c;
  c.A = ptr[0]; c.B = ptr[1]; c.Q = ptr[2]; c.R = ptr[3]; c.Qf = ptr[4]; c.lA = ptr[5]; c.lB = ptr[6];
  c.lQ = ptr[7]; c.h0 = ptr[8]; c.dU = ptr[9];
  c.gA = ptr[10]; c.gB = ptr[11]; c.gQ = ptr[12]; c.gR = ptr[13]; c.gQf = ptr[14]; c.glA = ptr[15];
  c.glB = ptr[16]; c.glQ = ptr[17]; c.gh0 = ptr[18];
  c.gi = reinterpret_cast<int32_t*>(base + off);
  return c;
}

// Gradients of n_tokens tokens (inputs already validated), token chunk by token chunk
// inside ws: the certified Hamiltonian rollout with its per-problem fallback, or the
// stable path for every problem under TTC_LQR_FLAG_STABLE_BWD.  v1s / q0s: the forward's
// stash halves (V_1 [P,d,d], Quu_0 [P,du,du]) or null to recompute them per chunk.
static int backward_core(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                         const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q,
                         const float* h0, const float* u, const float* d_u, int64_t n_tokens, int H, int d, int du,
                         int T, int flags, const float* v1s, const float* q0s, float* grad_A_diag, float* grad_B,
                         float* grad_Q, float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                         float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, char* ws,
                         size_t workspace_bytes, float grad_limit, int32_t* status, int64_t* n_fallback,
                         hipStream_t s, RescueSlots rs = RescueSlots{}) {
  const bool fp64 = fp64_stable(flags, d);
  if (flags & TTC_LQR_FLAG_STABLE_BWD) {
    if (n_fallback) *n_fallback = n_tokens * H;
    return stable_backward(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, d_u, n_tokens, H, d,
                           T, flags, grad_A_diag, grad_B, grad_Q, grad_R_inv, grad_Q_f, grad_log_gamma_A,
                           grad_log_gamma_B, grad_log_gamma_Q, grad_h0, ws, workspace_bytes, grad_limit, grad_limit,
                           status, s);
  }
  const bool with_stash = v1s != nullptr;
  // largest token chunk whose layout fits the workspace (the layout grows with the chunk)
  if (workspace_bytes < fast_layout(1, H, d, du, T, with_stash, flags).total) return TTC_LQR_EINVAL;
  int64_t chunk = 1, hi = n_tokens;
  while (chunk < hi) {
    const int64_t mid = chunk + (hi - chunk + 1) / 2;
    if (fast_layout(mid, H, d, du, T, with_stash, flags).total <= workspace_bytes) chunk = mid;
    else hi = mid - 1;
  }
  const int64_t dd = (int64_t)d * d;
  const float tau = TTC_LQR_CERT_TOL;
  int64_t total_fb = 0;
  for (int64_t n0 = 0; n0 < n_tokens; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * H, Pc = nc * H;
    const FastLayout L = fast_layout(nc, H, d, du, T, with_stash, flags);
    // rejected problems per fallback pass: whatever the workspace holds beyond the main layout
    int64_t Frun = fallback_capacity(workspace_bytes - L.fb, d, du, T, fp64);
    if (Frun < L.F) Frun = L.F;
    if (Frun > Pc) Frun = Pc;
    if (fp64) {  // whole rounds of the fp64 sweep per pass (a multiple of 8 problems)
      const int64_t rnd = fp64_round_problems(d);
      if (rnd > 0 && rnd % 8 == 0 && Frun > rnd) Frun -= Frun % rnd;
    }
    size_t csz[19];
    const size_t fb_stable = L.fb + compact_sizes(Frun, d, du, csz);
    const float *a = A_diag + p0 * d, *b = B + n0 * dd, *q = Q + n0 * dd, *r = R_inv + p0 * du;
    const float *qf = Q_f + p0 * dd, *la = log_gamma_A + p0, *lb = log_gamma_B + p0 * du;
    const float *lq = log_gamma_Q + p0 * d, *hz = h0 + p0 * d, *dz = d_u + p0 * du, *uz = u + p0 * du;
    float *gA = grad_A_diag + p0 * d, *gR = grad_R_inv + p0 * du, *gQf = grad_Q_f + p0 * dd;
    float *glA = grad_log_gamma_A + p0, *glB = grad_log_gamma_B + p0 * du, *glQ = grad_log_gamma_Q + p0 * d;
    float* gh = grad_h0 + p0 * d;
    const float *v1, *q0;
    int rc = TTC_LQR_OK;
    if (with_stash) {
      v1 = v1s + p0 * dd;
      q0 = q0s + p0 * (int64_t)du * du;
    } else {
      float* v1w = reinterpret_cast<float*>(ws + L.v1);
      float* q0w = reinterpret_cast<float*>(ws + L.q0);
      rc = fwd_d(d, a, b, q, r, qf, la, lb, lq, hz, Pc, H, T, nullptr, v1w, q0w, kStashV1, nullptr, s, flags);
      if (rc != TTC_LQR_OK) return rc;
      v1 = v1w;
      q0 = q0w;
    }
    float* gBp = reinterpret_cast<float*>(ws + L.gBp);
    float* gQp = reinterpret_cast<float*>(ws + L.gQp);
    int32_t* list = reinterpret_cast<int32_t*>(ws + L.list);
    int32_t* cnt = reinterpret_cast<int32_t*>(ws + L.cnt);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, s, cnt, (int64_t)6, 0);
    // a device count the host needs: one stream synchronisation
    auto read_count = [&](const int32_t* c, int64_t cap, int32_t& v) -> int {
      v = 0;
      if (hipMemcpyAsync(&v, c, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess) return TTC_LQR_ELAUNCH;
      if (hipStreamSynchronize(s) != hipSuccess) return TTC_LQR_ELAUNCH;
      return (v < 0 || v > cap) ? TTC_LQR_ELAUNCH : TTC_LQR_OK;
    };
    // the listed problems (nfail) recomputed by the stable path in passes of Frun, their
    // outputs and grad_B / grad_Q partials scattered to their own problem indices; kept: each
    // has gains the forward's fp64 rescue kept (TTC_LQR_FLAG_RESCUE_GAINS), read instead of swept
    auto stable_problems = [&](const int32_t* list, int32_t nfail, int32_t nrest) -> int {
      // nrest >= 0: only the first nrest listed problems are swept; the others have gains the
      // forward's fp64 rescue kept (TTC_LQR_FLAG_RESCUE_GAINS), read by the same gradient pass
      const bool kept = nrest >= 0;
      const Compact c = compact_at(ws + L.fb, Frun, d, du);
      for (int64_t f0 = 0; f0 < nfail; f0 += Frun) {
        const int64_t fc = (f0 + Frun <= nfail) ? Frun : (nfail - f0);
        hipLaunchKernelGGL(gather_kernel, dim3((unsigned)fc), dim3(256), 0, s, list, f0, H, d, du, a, b, q, r, qf, la,
                           lb, lq, hz, dz, c);
        if (kept)
          hipLaunchKernelGGL(gather_slot_kernel, dim3((unsigned)((fc + 255) / 256)), dim3(256), 0, s, list, f0, fc,
                             (int64_t)nrest, rs.slot_of + p0, c.gi);
        if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
        const int64_t sweep = !kept ? -1 : (nrest <= f0 ? 0 : (nrest - f0 < fc ? nrest - f0 : fc));
        const int rcs = stable_backward(c.A, c.B, c.Q, c.R, c.Qf, c.lA, c.lB, c.lQ, c.h0, c.dU, fc, 1, d, T, flags,
                                        c.gA, c.gB, c.gQ, c.gR, c.gQf, c.glA, c.glB, c.glQ, c.gh0, ws + fb_stable,
                                        workspace_bytes - fb_stable, grad_limit, INFINITY, status,
                                        s,  // per-problem partials
                                        kept ? c.gi : nullptr, kept ? rs.gains : nullptr, kept ? rs.slots : nullptr,
                                        sweep);
        if (rcs != TTC_LQR_OK) return rcs;
        hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)fc), dim3(256), 0, s, list, f0, d, du, c, gA, gR, gQf, glA,
                           glB, glQ, gh, gBp, gQp);
        if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
      }
      return TTC_LQR_OK;
    };
    if (head_group_path(H, flags, d)) {
      // head groups of 8 on the matrix cores in fp32: grad_B / grad_Q summed inside the kernel
      // (straight into the outputs when a group is a token, H == 8)
      const bool direct = H == 8;
      const bool tiers = two_tier_path(H, flags, d);
      float* gBg = direct ? grad_B + n0 * dd : reinterpret_cast<float*>(ws + L.gBg);
      float* gQg = direct ? grad_Q + n0 * dd : reinterpret_cast<float*>(ws + L.gQg);
      int32_t* glist = tiers ? reinterpret_cast<int32_t*>(ws + L.glist) : list;
      auto* launch = d == 16 ? launch_ham16_mfma : (d == 32 ? launch_ham32_mfma : launch_ham64_mfma);
      rc = launch(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, Pc, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBg,
                  gQg, grad_limit, glist, cnt, status, s);
      if (rc != TTC_LQR_OK) return rc;
      int32_t nfail = 0;
      rc = read_count(cnt, Pc / 8, nfail);
      if (rc != TTC_LQR_OK) return rc;
      if (tiers) {
        // long horizons: the problems of the rejected groups rolled again one by one in fp64 on
        // the row layout (which accepts most of them), the rest by the stable path, and the
        // groups' grad_B / grad_Q summed from the per-problem partials of the two
        if (nfail > 0) {
          int32_t* plist = reinterpret_cast<int32_t*>(ws + L.plist);
          const int64_t np = 8 * (int64_t)nfail;
          hipLaunchKernelGGL(expand_groups_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, s, glist,
                             (int64_t)nfail, plist);
          if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
          switch (d) {
            case 16: rc = launch_ham_d16(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, np, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, list, cnt + 1, status, s, true, plist, rs.slot_of ? rs.slot_of + p0 : nullptr, rs.slots, rs.nslot); break;
            case 32: rc = launch_ham_d32(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, np, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, list, cnt + 1, status, s, true, plist); break;
            default: return TTC_LQR_EUNSUPPORTED;
          }
          if (rc != TTC_LQR_OK) return rc;
          int32_t nfail2 = 0;
          rc = read_count(cnt + 1, np, nfail2);
          if (rc != TTC_LQR_OK) return rc;
          const int32_t* slist = list;  // the stable path's problems
          int32_t nstable = nfail2;
          if (L.n3 > 0 && nfail2 > 0) {
            // third tier: those that started from the fp32 V_1 get an fp64 one and roll again;
            // the stable path's list goes to plist (free once the second tier has run)
            int32_t* list3 = reinterpret_cast<int32_t*>(ws + L.l3);
            int32_t* so3 = reinterpret_cast<int32_t*>(ws + L.so3);
            double* sl3 = reinterpret_cast<double*>(ws + L.sl3);
            hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((Pc + 255) / 256)), dim3(256), 0, s, so3, Pc, -1);
            hipLaunchKernelGGL(tier3_split_kernel, dim3((unsigned)((nfail2 + 255) / 256)), dim3(256), 0, s, list,
                               (int64_t)nfail2, rs.slot_of ? rs.slot_of + p0 : nullptr, list3, L.n3, cnt + 2, plist,
                               cnt + 3);
            hipLaunchKernelGGL(tier3_close_kernel, dim3(1), dim3(1), 0, s, cnt + 2, L.n3, list3);
            if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
            rc = launch_v1slots64_d16(a, b, q, r, qf, la, lb, lq, hz, H, T, list3,
                                      nfail2 < L.n3 ? (int64_t)nfail2 : L.n3, so3, sl3, L.n3, s);
            if (rc != TTC_LQR_OK) return rc;
            int32_t n3 = 0;
            rc = read_count(list3, L.n3, n3);
            if (rc != TTC_LQR_OK) return rc;
            if (n3 > 0) {
              rc = launch_ham_d16(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, n3, H, T, tau, gA, gR, gQf, glA,
                                  glB, glQ, gh, gBp, gQp, grad_limit, plist, cnt + 3, status, s, true, list3 + 64, so3,
                                  sl3, L.n3);
              if (rc != TTC_LQR_OK) return rc;
            }
            rc = read_count(cnt + 3, nfail2, nstable);
            if (rc != TTC_LQR_OK) return rc;
            slist = plist;
          }
          total_fb += nstable;
          if (rs.gains != nullptr && slist == plist && nstable > 0) {
            // the problems whose gains the forward kept skip the sweep: the list reordered into
            // list (free once the third tier has split it), those without first
            hipLaunchKernelGGL(kept_split_kernel, dim3((unsigned)((nstable + 255) / 256)), dim3(256), 0, s, plist,
                               (int64_t)nstable, rs.slot_of + p0, rs.ngslot, list, cnt + 4, cnt + 5);
            if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
            int32_t nrest = 0;
            rc = read_count(cnt + 5, nstable, nrest);
            if (rc != TTC_LQR_OK) return rc;
            rc = stable_problems(list, nstable, nrest);
          } else {
            rc = stable_problems(slist, nstable, -1);
          }
          if (rc != TTC_LQR_OK) return rc;
          rc = launch_groupsum(glist, nfail, gBp, (int)(d * du), gBg, grad_limit, direct ? status : nullptr, s);
          if (rc != TTC_LQR_OK) return rc;
          rc = launch_groupsum(glist, nfail, gQp, (int)dd, gQg, grad_limit, direct ? status : nullptr, s);
          if (rc != TTC_LQR_OK) return rc;
        }
      } else {
        // a rejected group is recomputed whole by the stable path, gathered as a compact 8-head token
        total_fb += 8 * (int64_t)nfail;
        const Compact c = compact_at(ws + L.fb, Frun, d, du);
        const int64_t Fg = Frun / 8;  // groups per fallback batch
        for (int64_t f0 = 0; f0 < nfail; f0 += Fg) {
          const int64_t fc = (f0 + Fg <= nfail) ? Fg : (nfail - f0);
          hipLaunchKernelGGL(gather_group_kernel, dim3((unsigned)fc), dim3(256), 0, s, list, f0, H, d, du, a, b, q,
                             r, qf, la, lb, lq, hz, dz, c);
          if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
          // a group's sums are the token's head sums only when H == 8
          rc = stable_backward(c.A, c.B, c.Q, c.R, c.Qf, c.lA, c.lB, c.lQ, c.h0, c.dU, fc, 8, d, T, flags, c.gA, c.gB,
                               c.gQ, c.gR, c.gQf, c.glA, c.glB, c.glQ, c.gh0, ws + fb_stable,
                               workspace_bytes - fb_stable, grad_limit, direct ? grad_limit : INFINITY, status, s);
          if (rc != TTC_LQR_OK) return rc;
          hipLaunchKernelGGL(scatter_group_kernel, dim3((unsigned)fc), dim3(256), 0, s, list, f0, H, d, du, c, gA,
                             gR, gQf, glA, glB, glQ, gh, gBg, gQg);
          if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
        }
      }
      if (!direct) {
        rc = launch_headsum(gBg, nc, H / 8, (int)(d * du), grad_B + n0 * d * du, grad_limit, status, s);
        if (rc != TTC_LQR_OK) return rc;
        rc = launch_headsum(gQg, nc, H / 8, (int)dd, grad_Q + n0 * dd, grad_limit, status, s);
        if (rc != TTC_LQR_OK) return rc;
      }
      continue;
    }
    switch (d) {
      case 16: rc = launch_ham_d16(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, Pc, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, list, cnt, status, s, fp64_rollout(flags, d)); break;
      case 32: rc = launch_ham_d32(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, Pc, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, list, cnt, status, s, fp64_rollout(flags, d)); break;
      case 64: rc = launch_ham_d64(a, b, q, r, qf, la, lb, lq, hz, uz, dz, v1, q0, Pc, H, T, tau, gA, gR, gQf, glA, glB, glQ, gh, gBp, gQp, grad_limit, list, cnt, status, s, fp64_rollout(flags, d)); break;
      default: return TTC_LQR_EUNSUPPORTED;
    }
    if (rc != TTC_LQR_OK) return rc;
    // how many problems the certificate rejected (one stream synchronisation per chunk)
    int32_t nfail = 0;
    rc = read_count(cnt, Pc, nfail);
    if (rc != TTC_LQR_OK) return rc;
    total_fb += nfail;
    rc = stable_problems(list, nfail, -1);
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gBp, nc, H, (int)(d * du), grad_B + n0 * d * du, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
    rc = launch_headsum(gQp, nc, H, (int)dd, grad_Q + n0 * dd, grad_limit, status, s);
    if (rc != TTC_LQR_OK) return rc;
  }
  if (n_fallback) *n_fallback = total_fb;
  return TTC_LQR_OK;
}



// ---- factored inputs: expanded B / Q / Q_f per token chunk ---------------------------
// Workspace of the factored entry points, for token chunks of nc tokens.  Chunk-independent
// regions first: the bases and the basis gradients in fp32 (bf16 storage only).  Then the
// chunk's expanded B, Q, Q_f; for the backward their gradients, the reduction partials;
// for bf16 storage the chunk's inputs (and d_u) and per-problem gradients in fp32; last,
// ttc_lqr_backward's own workspace for the chunk.
struct FactLayout {
  size_t bas, gbas, Bx, Qx, Qfx, gB, gQ, gQf, part, cin[10], cg[9], v1t, q0t, rlist, inner, total;
};

// TTC_LQR_FLAG_KEEP_EXPANDED: byte offsets of the expanded B [N,d,du], Q [N,d,d], Q_f [N,H,d,d]
// after the V_1 stash (which is align256 of the full or compact stash bytes).
struct KeptLayout {
  size_t B, Q, Qf, total;
};

static KeptLayout kept_layout(int64_t N, int H, int d, int du) {
  KeptLayout K{};
  size_t off = 0;
  K.B = off;
  off += align256((size_t)N * d * du * sizeof(float));
  K.Q = off;
  off += align256((size_t)N * d * d * sizeof(float));
  K.Qf = off;
  off += align256((size_t)N * H * d * d * sizeof(float));
  K.total = off;
  return K;
}

// TTC_LQR_FLAG_RESCUE_V1: after the stash (align256 of its bytes), a slot index per problem
// (int32, -1 = none) and min(P, max(64, P / 8)) slots of the fp64 V_1 and Quu_0 (d = du = 16).
static int64_t rescue_nslot(int64_t P) {
  const int64_t s = P / 8 > 64 ? P / 8 : 64;
  return s < P ? s : P;
}

static size_t rescue_record_bytes(int64_t P, int d, int du) {
  return align256((size_t)P * sizeof(int32_t)) +
         align256((size_t)rescue_nslot(P) * ((size_t)d * d + (size_t)du * du) * sizeof(double));
}

// TTC_LQR_FLAG_RESCUE_GAINS: after that record, every gain K_t [T][du][d] (fp64) of the first
// min(S, max(64, P / 16)) slots.
static int64_t rescue_gains_nslot(int64_t P) {
  const int64_t g = P / 16 > 64 ? P / 16 : 64;
  const int64_t s = rescue_nslot(P);
  return g < s ? g : s;
}

static size_t rescue_gains_bytes(int64_t P, int d, int du, int T) {
  return align256((size_t)rescue_gains_nslot(P) * (size_t)T * (size_t)d * du * sizeof(double));
}

static RescueSlots rescue_slots(const float* stash, int64_t P, int d, int du, int T, bool gains) {
  char* base = reinterpret_cast<char*>(const_cast<float*>(stash)) +
               align256((size_t)P * ((size_t)d * d + (size_t)du * du) * sizeof(float));
  RescueSlots rs;
  rs.slot_of = reinterpret_cast<int32_t*>(base);
  rs.slots = reinterpret_cast<double*>(base + align256((size_t)P * sizeof(int32_t)));
  rs.nslot = rescue_nslot(P);
  if (gains) {
    rs.gains = reinterpret_cast<double*>(base + rescue_record_bytes(P, d, du));
    rs.ngslot = rescue_gains_nslot(P);
  }
  return rs;
}

// The expanded arrays of a KEEP_EXPANDED stash buffer.
struct Kept {
  float *B, *Q, *Qf;
};

static Kept kept_arrays(const float* stash, int64_t N, int H, int d, int du, bool compact) {
  const size_t v1 = compact ? (size_t)N * H * ((size_t)d * (d + 1) / 2) * sizeof(float)
                            : (size_t)N * H * ((size_t)d * d + (size_t)du * du) * sizeof(float);
  char* base = reinterpret_cast<char*>(const_cast<float*>(stash)) + align256(v1);
  const KeptLayout K = kept_layout(N, H, d, du);
  return Kept{reinterpret_cast<float*>(base + K.B), reinterpret_cast<float*>(base + K.Q),
              reinterpret_cast<float*>(base + K.Qf)};
}

// Elements of the per-problem / per-token arrays of a chunk, in argument order:
// A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, lgA, lgB, lgQ, h0 (and d_u).
static void io_counts(int64_t nc, int H, int d, int du, int rb, int rq, size_t (&n)[10]) {
  const size_t N = (size_t)nc, P = (size_t)nc * (size_t)H;
  const size_t v[10] = {P * d, N * rb, N * rq, P * du, P * rq, P, P * du, P * d, P * d, P * du};
  for (int k = 0; k < 10; ++k) n[k] = v[k];
}

// with_stash: the forward's stash is passed (compact: as the upper triangles of V_1, whose
// full V_1 and Quu_0 the chunk then holds in v1t / q0t, in the forward before packing and in
// the backward after unpacking).
static FactLayout fact_layout(int64_t nc, int H, int d, int du, int rb, int rq, int T, bool with_stash,
                              bool backward, bool bf16, bool compact, int flags) {
  const bool fp64 = fp64_stable(flags, d);
  const bool kept = (flags & TTC_LQR_FLAG_KEEP_EXPANDED) != 0;  // B, Q, Q_f live in the stash buffer
  const size_t N = (size_t)nc, P = (size_t)nc * (size_t)H, Eb = (size_t)d * du, Eq = (size_t)d * d;
  const size_t nbas = (size_t)rb * Eb + (size_t)rq * Eq;
  FactLayout L{};
  size_t off = 0;
  L.bas = off;
  off += bf16 ? align256(nbas * sizeof(float)) : 0;
  L.gbas = off;
  off += (bf16 && backward) ? align256(nbas * sizeof(float)) : 0;
  L.Bx = off;
  off += kept ? 0 : align256(N * Eb * sizeof(float));
  L.Qx = off;
  off += kept ? 0 : align256(N * Eq * sizeof(float));
  L.Qfx = off;
  off += kept ? 0 : align256(P * Eq * sizeof(float));
  if (backward) {
    L.gB = off;
    off += align256(N * Eb * sizeof(float));
    L.gQ = off;
    off += align256(N * Eq * sizeof(float));
    L.gQf = off;
    off += align256(P * Eq * sizeof(float));
    size_t part = factor_partial_floats(nc, rb, (int)Eb);
    const size_t pq = factor_partial_floats(nc, rq, (int)Eq), pf = factor_partial_floats((int64_t)P, rq, (int)Eq);
    part = part > pq ? part : pq;
    part = part > pf ? part : pf;
    L.part = off;
    off += align256(part * sizeof(float));
  }
  if (bf16) {
    size_t n[10];
    io_counts(nc, H, d, du, rb, rq, n);
    for (int k = 0; k < (backward ? 10 : 9); ++k) {
      L.cin[k] = off;
      // the forward's expansion reads the bf16 coefficients directly (the backward's basis
      // reductions read fp32 copies)
      if (!backward && (k == 1 || k == 2 || k == 4)) continue;
      off += align256(n[k] * sizeof(float));
    }
    if (backward) {
      for (int k = 0; k < 9; ++k) {
        L.cg[k] = off;
        off += align256(n[k] * sizeof(float));
      }
    }
  }
  if (compact && with_stash) {
    L.v1t = off;
    off += align256(P * Eq * sizeof(float));
    L.q0t = off;
    off += align256(P * (size_t)du * du * sizeof(float));
  }
  if (!backward && fp64) {  // the fp64 rescue's problem list of the chunk
    L.rlist = off;
    off += align256(rescue_ws_bytes((int64_t)P));
  }
  if (backward) {
    L.inner = off;
    // ttc_lqr_backward's workspace for this chunk in one pass; the stable path (flag
    // TTC_LQR_FLAG_STABLE_BWD) splits the chunk further inside it (one token at least)
    const size_t fast = fast_layout(nc, H, d, du, T, with_stash, flags).total;
    const size_t stab = stable_layout(1, H, d, T, fp64).total;
    off += fast > stab ? fast : stab;
  }
  L.total = off;
  return L;
}

static bool fact_args_ok(int64_t n_tokens, int H, int d, int du, int rb, int rq, int T) {
  return n_tokens >= 0 && H > 0 && d > 0 && du > 0 && T > 0 && rb >= 1 && rb <= 64 && rq >= 1 && rq <= 64;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest token chunk whose factored layout fits ws_bytes (0 when not even one token fits).
static int64_t fact_chunk(int64_t n_tokens, int H, int d, int du, int rb, int rq, int T, bool with_stash,
                          bool backward, bool bf16, bool compact, int flags, size_t ws_bytes) {
  if (fact_layout(1, H, d, du, rb, rq, T, with_stash, backward, bf16, compact, flags).total > ws_bytes) return 0;
  int64_t chunk = 1, hi = n_tokens;
  while (chunk < hi) {
    const int64_t mid = chunk + (hi - chunk + 1) / 2;
    if (fact_layout(mid, H, d, du, rb, rq, T, with_stash, backward, bf16, compact, flags).total <= ws_bytes)
      chunk = mid;
    else hi = mid - 1;
  }
  return chunk;
}

template <typename TC>
static int expand_chunk(const TC* cB, const TC* cQ, const TC* cQf, const float* Bs, const float* Gs,
                        int64_t nc, int H, int d, int du, int rb, int rq, float* Bx, float* Qx, float* Qfx,
                        hipStream_t s) {
  int rc = launch_expand(cB, nc, rb, Bs, d * du, Bx, s);
  if (rc == TTC_LQR_OK) rc = launch_expand(cQ, nc, rq, Gs, d * d, Qx, s);
  if (rc == TTC_LQR_OK) rc = launch_expand(cQf, nc * H, rq, Gs, d * d, Qfx, s);
  return rc;
}

// Storage of the factored inputs and gradients: fp32 as is, bf16 (bit patterns) converted
// to / from fp32 arrays in the workspace.
template <typename TS>
struct Store {
  static constexpr bool BF16 = std::is_same<TS, uint16_t>::value;
  // fp32 view of in[off .. off + n): the array itself, or its conversion into dst
  static const float* in(const TS* a, int64_t off, size_t n, float* dst, hipStream_t s, int& rc) {
    if constexpr (BF16) {
      if (rc == TTC_LQR_OK) rc = launch_bf16_to_f32(a + off, (int64_t)n, dst, s);
      return dst;
    } else {
      (void)n; (void)dst; (void)s;
      return a + off;
    }
  }
  // where the kernels write out[off ..): the array itself, or a workspace array converted afterwards
  static float* out(TS* a, int64_t off, float* tmp) {
    if constexpr (BF16) {
      (void)a; (void)off;
      return tmp;
    } else {
      (void)tmp;
      return a + off;
    }
  }
  static void flush(TS* a, int64_t off, size_t n, const float* tmp, hipStream_t s, int& rc) {
    if constexpr (BF16) {
      if (rc == TTC_LQR_OK) rc = launch_f32_to_bf16(tmp, (int64_t)n, a + off, s);
    } else {
      (void)a; (void)off; (void)n; (void)tmp; (void)s;
    }
  }
};

template <typename TS>
static int forward_factored(const TS* A_diag, const TS* coeff_B, const TS* coeff_Q, const TS* R_inv,
                            const TS* coeff_Qf, const TS* log_gamma_A, const TS* log_gamma_B, const TS* log_gamma_Q,
                            const TS* h0, const TS* B_basis, const TS* Q_basis, int64_t n_tokens, int H, int d,
                            int du, int rb, int rq, int T, int flags, float* u, float* stash, char* ws,
                            size_t ws_bytes, int32_t* status, hipStream_t s) {
  using St = Store<TS>;
  const bool compact = stash != nullptr && (flags & TTC_LQR_FLAG_COMPACT_STASH);
  const bool fp64 = fp64_stable(flags, d);
  const bool kept = stash != nullptr && (flags & TTC_LQR_FLAG_KEEP_EXPANDED);
  const Kept K = kept ? kept_arrays(stash, n_tokens, H, d, du, compact) : Kept{};
  const int64_t chunk = fact_chunk(n_tokens, H, d, du, rb, rq, T, stash != nullptr, false, St::BF16, compact, flags,
                                   ws_bytes);
  if (chunk == 0) return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * H, dd = (int64_t)d * d;
  const size_t nb = (size_t)rb * d * du, nq = (size_t)rq * d * d;
  const FactLayout L0 = fact_layout(chunk, H, d, du, rb, rq, T, stash != nullptr, false, St::BF16, compact, flags);
  int rc = TTC_LQR_OK;
  float* bas = reinterpret_cast<float*>(ws + L0.bas);
  const float* Bs = St::in(B_basis, 0, nb, bas, s, rc);
  const float* Gs = St::in(Q_basis, 0, nq, bas + nb, s, rc);
  for (int64_t n0 = 0; n0 < n_tokens && rc == TTC_LQR_OK; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * H;
    const FactLayout L = fact_layout(nc, H, d, du, rb, rq, T, stash != nullptr, false, St::BF16, compact, flags);
    size_t n[10];
    io_counts(nc, H, d, du, rb, rq, n);
    auto cin = [&](int k) { return reinterpret_cast<float*>(ws + L.cin[k]); };
    const float* a = St::in(A_diag, p0 * d, n[0], cin(0), s, rc);
    const float* r = St::in(R_inv, p0 * du, n[3], cin(3), s, rc);
    const float* la = St::in(log_gamma_A, p0, n[5], cin(5), s, rc);
    const float* lb = St::in(log_gamma_B, p0 * du, n[6], cin(6), s, rc);
    const float* lq = St::in(log_gamma_Q, p0 * d, n[7], cin(7), s, rc);
    const float* hz = St::in(h0, p0 * d, n[8], cin(8), s, rc);
    if (rc != TTC_LQR_OK) return rc;
    float* Bx = reinterpret_cast<float*>(ws + L.Bx);
    float* Qx = reinterpret_cast<float*>(ws + L.Qx);
    float* Qfx = reinterpret_cast<float*>(ws + L.Qfx);
    if (kept) {  // into the stash buffer, where the backward reads them
      Bx = K.B + n0 * d * du;
      Qx = K.Q + n0 * dd;
      Qfx = K.Qf + p0 * dd;
    }
    // the expansion reads the coefficients as stored (bf16: widened in registers)
    rc = expand_chunk(coeff_B + n0 * rb, coeff_Q + n0 * rq, coeff_Qf + p0 * rq, Bs, Gs, nc, H, d, du, rb, rq, Bx, Qx,
                      Qfx, s);
    if (rc != TTC_LQR_OK) return rc;
    float* v1 = stash ? stash + p0 * dd : nullptr;
    float* q0 = stash ? stash + P * dd + p0 * (int64_t)du * du : nullptr;
    if (compact) {  // full V_1 / Quu_0 of the chunk in the workspace, V_1's upper triangle to the stash
      v1 = reinterpret_cast<float*>(ws + L.v1t);
      q0 = reinterpret_cast<float*>(ws + L.q0t);
    }
    int32_t* rlist = fp64 ? reinterpret_cast<int32_t*>(ws + L.rlist) : nullptr;
    rc = fwd_d(d, a, Bx, Qx, r, Qfx, la, lb, lq, hz, nc * H, H, T, u + p0 * du, v1, q0, stash ? kStashV1 : 0, status,
               s, flags & ~TTC_LQR_FLAG_COMPACT_STASH, rlist);
    if (compact && rc == TTC_LQR_OK) rc = launch_pack_upper(v1, nc * H, d, stash + p0 * (dd + d) / 2, s);
  }
  return rc;
}

template <typename TS>
static int backward_factored(const TS* A_diag, const TS* coeff_B, const TS* coeff_Q, const TS* R_inv,
                             const TS* coeff_Qf, const TS* log_gamma_A, const TS* log_gamma_B,
                             const TS* log_gamma_Q, const TS* h0, const TS* B_basis, const TS* Q_basis,
                             const float* u, const TS* d_u, int64_t n_tokens, int H, int d, int du, int rb, int rq,
                             int T, int flags, const float* stash, TS* grad_A_diag, TS* grad_coeff_B,
                             TS* grad_coeff_Q, TS* grad_R_inv, TS* grad_coeff_Qf, TS* grad_log_gamma_A,
                             TS* grad_log_gamma_B, TS* grad_log_gamma_Q, TS* grad_h0, TS* grad_B_basis,
                             TS* grad_Q_basis, char* ws, size_t ws_bytes, float grad_limit, int32_t* status,
                             int64_t* n_fallback, hipStream_t s) {
  using St = Store<TS>;
  const bool stable = (flags & TTC_LQR_FLAG_STABLE_BWD) != 0;
  const bool with_stash = stash != nullptr && !stable;
  const bool compact = with_stash && (flags & TTC_LQR_FLAG_COMPACT_STASH);
  const bool fp64 = fp64_stable(flags, d);
  const bool kept = stash != nullptr && (flags & TTC_LQR_FLAG_KEEP_EXPANDED);
  const Kept K = kept ? kept_arrays(stash, n_tokens, H, d, du, (flags & TTC_LQR_FLAG_COMPACT_STASH) != 0) : Kept{};
  flags &= ~TTC_LQR_FLAG_COMPACT_STASH;
  const int Eb = d * du, Eq = d * d;
  const size_t nb = (size_t)rb * Eb, nq = (size_t)rq * Eq;
  const int64_t chunk = fact_chunk(n_tokens > 0 ? n_tokens : 1, H, d, du, rb, rq, T, with_stash, true, St::BF16,
                                   compact, flags, ws_bytes);
  if (chunk == 0) return TTC_LQR_EINVAL;
  const FactLayout L0 = fact_layout(chunk, H, d, du, rb, rq, T, with_stash, true, St::BF16, compact, flags);
  int rc = TTC_LQR_OK;
  float* bas = reinterpret_cast<float*>(ws + L0.bas);
  float* gbas = reinterpret_cast<float*>(ws + L0.gbas);
  float* gBs = St::out(grad_B_basis, 0, gbas);
  float* gGs = St::out(grad_Q_basis, 0, gbas + nb);
  if (n_tokens == 0) {  // the basis gradients are sums over no tokens
    rc = launch_reduce(nullptr, 0, rb, nullptr, Eb, nullptr, gBs, 0, s);
    if (rc == TTC_LQR_OK) rc = launch_reduce(nullptr, 0, rq, nullptr, Eq, nullptr, gGs, 0, s);
    St::flush(grad_B_basis, 0, nb, gBs, s, rc);
    St::flush(grad_Q_basis, 0, nq, gGs, s, rc);
    return rc;
  }
  const float* Bs = St::in(B_basis, 0, nb, bas, s, rc);
  const float* Gs = St::in(Q_basis, 0, nq, bas + nb, s, rc);
  const int64_t P = n_tokens * H, dd = (int64_t)d * d;
  int64_t total_fb = 0;
  for (int64_t n0 = 0; n0 < n_tokens && rc == TTC_LQR_OK; n0 += chunk) {
    const int64_t nc = (n0 + chunk <= n_tokens) ? chunk : (n_tokens - n0);
    const int64_t p0 = n0 * H, Pc = nc * H;
    const FactLayout L = fact_layout(nc, H, d, du, rb, rq, T, with_stash, true, St::BF16, compact, flags);
    size_t n[10];
    io_counts(nc, H, d, du, rb, rq, n);
    auto cin = [&](int k) { return reinterpret_cast<float*>(ws + L.cin[k]); };
    auto cg = [&](int k) { return reinterpret_cast<float*>(ws + L.cg[k]); };
    const float* a = St::in(A_diag, p0 * d, n[0], cin(0), s, rc);
    const float* cB = St::in(coeff_B, n0 * rb, n[1], cin(1), s, rc);
    const float* cQ = St::in(coeff_Q, n0 * rq, n[2], cin(2), s, rc);
    const float* r = St::in(R_inv, p0 * du, n[3], cin(3), s, rc);
    const float* cQf = St::in(coeff_Qf, p0 * rq, n[4], cin(4), s, rc);
    const float* la = St::in(log_gamma_A, p0, n[5], cin(5), s, rc);
    const float* lb = St::in(log_gamma_B, p0 * du, n[6], cin(6), s, rc);
    const float* lq = St::in(log_gamma_Q, p0 * d, n[7], cin(7), s, rc);
    const float* hz = St::in(h0, p0 * d, n[8], cin(8), s, rc);
    const float* dz = St::in(d_u, p0 * du, n[9], cin(9), s, rc);
    float* gA = St::out(grad_A_diag, p0 * d, cg(0));
    float* gcB = St::out(grad_coeff_B, n0 * rb, cg(1));
    float* gcQ = St::out(grad_coeff_Q, n0 * rq, cg(2));
    float* gR = St::out(grad_R_inv, p0 * du, cg(3));
    float* gcQf = St::out(grad_coeff_Qf, p0 * rq, cg(4));
    float* glA = St::out(grad_log_gamma_A, p0, cg(5));
    float* glB = St::out(grad_log_gamma_B, p0 * du, cg(6));
    float* glQ = St::out(grad_log_gamma_Q, p0 * d, cg(7));
    float* gh = St::out(grad_h0, p0 * d, cg(8));
    if (rc != TTC_LQR_OK) return rc;
    float* Bx = reinterpret_cast<float*>(ws + L.Bx);
    float* Qx = reinterpret_cast<float*>(ws + L.Qx);
    float* Qfx = reinterpret_cast<float*>(ws + L.Qfx);
    float* gB = reinterpret_cast<float*>(ws + L.gB);
    float* gQ = reinterpret_cast<float*>(ws + L.gQ);
    float* gQf = reinterpret_cast<float*>(ws + L.gQf);
    float* part = reinterpret_cast<float*>(ws + L.part);
    if (kept) {  // expanded by the forward
      Bx = K.B + n0 * d * du;
      Qx = K.Q + n0 * dd;
      Qfx = K.Qf + p0 * dd;
    } else {
      rc = expand_chunk(cB, cQ, cQf, Bs, Gs, nc, H, d, du, rb, rq, Bx, Qx, Qfx, s);
      if (rc != TTC_LQR_OK) return rc;
    }
    const float* v1 = with_stash ? stash + p0 * dd : nullptr;
    const float* q0 = with_stash ? stash + P * dd + p0 * (int64_t)du * du : nullptr;
    if (compact) {  // V_1 from its upper triangle, Quu_0 = R + B_0' V_1 B_0 recomputed
      float* v1w = reinterpret_cast<float*>(ws + L.v1t);
      float* q0w = reinterpret_cast<float*>(ws + L.q0t);
      rc = launch_unpack_quu0(stash + p0 * (dd + d) / 2, Bx, lb, r, Pc, H, d, v1w, q0w, s);
      if (rc != TTC_LQR_OK) return rc;
      v1 = v1w;
      q0 = q0w;
    }
    int64_t nfb = 0;
    rc = backward_core(a, Bx, Qx, r, Qfx, la, lb, lq, hz, u ? u + p0 * du : nullptr, dz, nc, H, d, du, T, flags, v1,
                       q0, gA, gB, gQ, gR, gQf, glA, glB, glQ, gh, ws + L.inner, ws_bytes - L.inner, grad_limit, status,
                       &nfb, s);  // the workspace beyond the chunk's layout widens the fallback passes
    if (rc != TTC_LQR_OK) return rc;
    total_fb += nfb;
    // chain rule of the expansion: coefficient gradients, then the basis sums
    // (each gradient read once where launch_project_reduce fuses the two)
    const int first = n0 == 0 ? 0 : 1;
    rc = launch_project_reduce(cB, nc, rb, gB, Eb, Bs, gcB, part, gBs, first, s);
    if (rc == TTC_LQR_OK) rc = launch_project_reduce(cQ, nc, rq, gQ, Eq, Gs, gcQ, part, gGs, first, s);
    if (rc == TTC_LQR_OK) rc = launch_project_reduce(cQf, Pc, rq, gQf, Eq, Gs, gcQf, part, gGs, 1, s);
    St::flush(grad_A_diag, p0 * d, n[0], gA, s, rc);
    St::flush(grad_coeff_B, n0 * rb, n[1], gcB, s, rc);
    St::flush(grad_coeff_Q, n0 * rq, n[2], gcQ, s, rc);
    St::flush(grad_R_inv, p0 * du, n[3], gR, s, rc);
    St::flush(grad_coeff_Qf, p0 * rq, n[4], gcQf, s, rc);
    St::flush(grad_log_gamma_A, p0, n[5], glA, s, rc);
    St::flush(grad_log_gamma_B, p0 * du, n[6], glB, s, rc);
    St::flush(grad_log_gamma_Q, p0 * d, n[7], glQ, s, rc);
    St::flush(grad_h0, p0 * d, n[8], gh, s, rc);
  }
  St::flush(grad_B_basis, 0, nb, gBs, s, rc);
  St::flush(grad_Q_basis, 0, nq, gGs, s, rc);
  if (n_fallback && rc == TTC_LQR_OK) *n_fallback = total_fb;
  return rc;
}

template <typename TS>
static int forward_factored_entry(const TS* A_diag, const TS* coeff_B, const TS* coeff_Q, const TS* R_inv,
                                  const TS* coeff_Qf, const TS* lgA, const TS* lgB, const TS* lgQ, const TS* h0,
                                  const TS* B_basis, const TS* Q_basis, int64_t n_tokens, int32_t heads, int32_t d,
                                  int32_t du, int32_t rb, int32_t rq, int32_t T, int32_t flags, float* u,
                                  float* stash, void* workspace, size_t workspace_bytes, int32_t* status,
                                  void* stream) {
  if (!fact_args_ok(n_tokens, heads, d, du, rb, rq, T)) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if ((flags & TTC_LQR_FLAG_KEEP_EXPANDED) && !stash) return TTC_LQR_EINVAL;
  if (flags & TTC_LQR_FLAG_RESCUE_V1) return TTC_LQR_EUNSUPPORTED;  // materialised entry points only
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !coeff_B || !coeff_Q || !R_inv || !coeff_Qf || !lgA || !lgB || !lgQ || !h0 || !B_basis ||
      !Q_basis || !u || !workspace)
    return TTC_LQR_EINVAL;
  if (!Store<TS>::BF16 && (!aligned16(B_basis) || !aligned16(Q_basis))) return TTC_LQR_EINVAL;
  return forward_factored<TS>(A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, lgA, lgB, lgQ, h0, B_basis, Q_basis,
                              n_tokens, heads, d, du, rb, rq, T, flags, u, stash, static_cast<char*>(workspace),
                              workspace_bytes, status, reinterpret_cast<hipStream_t>(stream));
}

template <typename TS>
static int backward_factored_entry(const TS* A_diag, const TS* coeff_B, const TS* coeff_Q, const TS* R_inv,
                                   const TS* coeff_Qf, const TS* lgA, const TS* lgB, const TS* lgQ, const TS* h0,
                                   const TS* B_basis, const TS* Q_basis, const float* u, const TS* d_u,
                                   int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t rb, int32_t rq,
                                   int32_t T, int32_t flags, const float* stash, TS* gA, TS* gcB, TS* gcQ, TS* gR,
                                   TS* gcQf, TS* glA, TS* glB, TS* glQ, TS* gh0, TS* gBs, TS* gQs, void* workspace,
                                   size_t workspace_bytes, float grad_limit, int32_t* status, int64_t* n_fallback,
                                   void* stream) {
  if (n_fallback) *n_fallback = 0;
  if (!fact_args_ok(n_tokens, heads, d, du, rb, rq, T)) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if ((flags & TTC_LQR_FLAG_KEEP_EXPANDED) && !stash) return TTC_LQR_EINVAL;
  if (flags & TTC_LQR_FLAG_RESCUE_V1) return TTC_LQR_EUNSUPPORTED;  // materialised entry points only
  const bool stable = (flags & TTC_LQR_FLAG_STABLE_BWD) != 0;
  if (!gBs || !gQs || !workspace) return TTC_LQR_EINVAL;
  if (n_tokens > 0 &&
      (!A_diag || !coeff_B || !coeff_Q || !R_inv || !coeff_Qf || !lgA || !lgB || !lgQ || !h0 || !B_basis ||
       !Q_basis || !d_u || !gA || !gcB || !gcQ || !gR || !gcQf || !glA || !glB || !glQ || !gh0 || (!stable && !u)))
    return TTC_LQR_EINVAL;
  if (n_tokens > 0 && !Store<TS>::BF16 && (!aligned16(B_basis) || !aligned16(Q_basis))) return TTC_LQR_EINVAL;
  return backward_factored<TS>(A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, lgA, lgB, lgQ, h0, B_basis, Q_basis, u, d_u,
                               n_tokens, heads, d, du, rb, rq, T, flags, stash, gA, gcB, gcQ, gR, gcQf, glA, glB, glQ,
                               gh0, gBs, gQs, static_cast<char*>(workspace), workspace_bytes, grad_limit, status,
                               n_fallback, reinterpret_cast<hipStream_t>(stream));
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
    case TTC_LQR_ESCRATCH:
      return "problem too large for the fixed scratch of ttc_lqr_backward_noalloc (one token's backward layout "
             "exceeds ttc_lqr_noalloc_scratch_bytes()); use ttc_lqr_backward with a workspace";
    default: return "unknown error";
  }
}

int ttc_lqr_supported(int32_t d, int32_t du) { return (d == du && (d == 16 || d == 32 || d == 64)) ? 1 : 0; }

int ttc_lqr_supported_flags(int32_t d, int32_t du, int32_t flags) {
  if (!ttc_lqr_supported(d, du)) return 0;
  if ((flags & (TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_FP64_RESCUE | TTC_LQR_FLAG_FP64_FALLBACK)) && d > 32)
    return 0;
  if ((flags & TTC_LQR_FLAG_RESCUE_V1) && (d != 16 || du != 16)) return 0;  // the d = 16 fp64 rescue keeps them
  if ((flags & TTC_LQR_FLAG_RESCUE_GAINS) && !(flags & TTC_LQR_FLAG_RESCUE_V1)) return 0;  // in its slots
  const int32_t known = TTC_LQR_FLAG_FP64_RICCATI | TTC_LQR_FLAG_ROW_KERNEL | TTC_LQR_FLAG_STABLE_BWD |
                        TTC_LQR_FLAG_RICCATI_STEPS | TTC_LQR_FLAG_COMPACT_STASH | TTC_LQR_FLAG_FP64_RESCUE |
                        TTC_LQR_FLAG_FP64_FALLBACK | TTC_LQR_FLAG_KEEP_EXPANDED | TTC_LQR_FLAG_RESCUE_V1 |
                        TTC_LQR_FLAG_RESCUE_GAINS;
  return (flags & ~known) ? 0 : 1;
}

size_t ttc_lqr_compact_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0) return 0;
  return sizeof(float) * (size_t)n_tokens * (size_t)heads * ((size_t)d * (d + 1) / 2);
}

size_t ttc_lqr_expanded_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0) return 0;
  return kept_layout(n_tokens, heads, d, du).total;
}

size_t ttc_lqr_rescue_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0) return 0;
  return rescue_record_bytes(n_tokens * heads, d, du);
}

size_t ttc_lqr_rescue_gains_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0 || T <= 0) return 0;
  return rescue_gains_bytes(n_tokens * heads, d, du, T);
}

size_t ttc_lqr_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T) {
  if (n_tokens < 0 || heads <= 0 || d <= 0 || du <= 0 || T <= 0) return 0;
  const size_t P = (size_t)n_tokens * (size_t)heads;
  return sizeof(float) * P * ((size_t)d * d + (size_t)du * du);
}

size_t ttc_lqr_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                               int32_t with_stash, int32_t flags) {
  if (chunk_tokens <= 0 || heads <= 0 || d <= 0 || du != d || T <= 0) return 0;
  if (flags & TTC_LQR_FLAG_STABLE_BWD)
    return stable_layout(chunk_tokens, heads, d, T, fp64_stable(flags, d)).total;
  return fast_layout(chunk_tokens, heads, d, du, T, with_stash != 0, flags).total;
}

size_t ttc_lqr_fallback_bytes(int64_t problems, int32_t d, int32_t du, int32_t T, int32_t flags) {
  if (problems <= 0 || d <= 0 || du != d || T <= 0) return 0;
  return fallback_bytes(problems, d, du, T, fp64_stable(flags, d));
}

size_t ttc_lqr_forward_workspace_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                                       int32_t flags) {
  if (n_tokens <= 0 || heads <= 0 || d <= 0 || du != d || T <= 0) return 0;
  // only the fp64 rescue uses one
  if (!(flags & (TTC_LQR_FLAG_FP64_RESCUE | TTC_LQR_FLAG_FP64_FALLBACK)) || d > 32) return 0;
  return ttc::rescue_ws_bytes(n_tokens * heads);
}

int ttc_lqr_forward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                    const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                    int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags, float* u,
                    float* stash, int32_t* status, void* stream) {
  return ttc_lqr_forward_ws(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, n_tokens, heads, d,
                            du, T, flags, u, stash, nullptr, 0, status, stream);
}

int ttc_lqr_forward_ws(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                       const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                       int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags, float* u,
                       float* stash, void* workspace, size_t workspace_bytes, int32_t* status, void* stream) {
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if (flags & TTC_LQR_FLAG_COMPACT_STASH) return TTC_LQR_EUNSUPPORTED;  // factored entry points only
  if ((flags & TTC_LQR_FLAG_RESCUE_V1) && !stash) return TTC_LQR_EINVAL;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !u)
    return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float* v1 = stash;
  float* q0 = stash ? stash + P * (int64_t)d * d : nullptr;
  // a workspace too small for the rescue list is not used (the rescue then runs unpacked)
  const size_t need = ttc_lqr_forward_workspace_bytes(n_tokens, heads, d, du, T, flags);
  int32_t* rws = (workspace != nullptr && need > 0 && workspace_bytes >= need) ? static_cast<int32_t*>(workspace)
                                                                                : nullptr;
  // the list's count starts at 0 whichever rescue route runs (the unlisted ones never write it)
  if (rws != nullptr) {
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, s, rws, 0);
    if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
  }
  // TTC_LQR_FLAG_RESCUE_V1: no problem has a slot until the listed fp64 rescue gives it one
  RescueSlots rs{};
  if (flags & TTC_LQR_FLAG_RESCUE_V1) {
    rs = rescue_slots(stash, P, d, du, T, (flags & TTC_LQR_FLAG_RESCUE_GAINS) != 0);
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((P + 255) / 256)), dim3(256), 0, s, rs.slot_of, P, -1);
    if (hipGetLastError() != hipSuccess) return TTC_LQR_ELAUNCH;
    if (rws == nullptr) rs = RescueSlots{};
  }
  return fwd_d(d, A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, P, heads, T, u, v1, q0,
               stash ? kStashV1 : 0, status, s, flags, rws, rs);
}

int ttc_lqr_backward(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                     const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                     const float* u, const float* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                     int32_t T, int32_t flags, const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                     float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A, float* grad_log_gamma_B,
                     float* grad_log_gamma_Q, float* grad_h0, void* workspace, size_t workspace_bytes,
                     float grad_limit, int32_t* status, int64_t* n_fallback, void* stream) {
  return ttc::backward_entry(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, u, d_u, n_tokens,
                             heads, d, du, T, flags, stash, grad_A_diag, grad_B, grad_Q, grad_R_inv, grad_Q_f,
                             grad_log_gamma_A, grad_log_gamma_B, grad_log_gamma_Q, grad_h0, workspace,
                             workspace_bytes, grad_limit, status, n_fallback, stream);
}

}  // extern "C"

namespace ttc {

int backward_entry(const float* A_diag, const float* B, const float* Q, const float* R_inv, const float* Q_f,
                   const float* log_gamma_A, const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                   const float* u, const float* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                   int32_t T, int32_t flags, const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                   float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A, float* grad_log_gamma_B,
                   float* grad_log_gamma_Q, float* grad_h0, void* workspace, size_t workspace_bytes,
                   float grad_limit, int32_t* status, int64_t* n_fallback, void* stream) {
  if (n_fallback) *n_fallback = 0;
  if (n_tokens < 0 || heads <= 0 || T <= 0 || d <= 0 || du <= 0) return TTC_LQR_EINVAL;
  if (!ttc_lqr_supported_flags(d, du, flags)) return TTC_LQR_EUNSUPPORTED;
  if (flags & TTC_LQR_FLAG_COMPACT_STASH) return TTC_LQR_EUNSUPPORTED;  // factored entry points only
  if ((flags & TTC_LQR_FLAG_RESCUE_V1) && !stash) return TTC_LQR_EINVAL;
  if (n_tokens == 0) return TTC_LQR_OK;
  const bool stable = (flags & TTC_LQR_FLAG_STABLE_BWD) != 0;
  if (!A_diag || !B || !Q || !R_inv || !Q_f || !log_gamma_A || !log_gamma_B || !log_gamma_Q || !h0 || !d_u ||
      !grad_A_diag || !grad_B || !grad_Q || !grad_R_inv || !grad_Q_f || !grad_log_gamma_A || !grad_log_gamma_B ||
      !grad_log_gamma_Q || !grad_h0 || !workspace || (!stable && !u))
    return TTC_LQR_EINVAL;
  const float* v1s = stash;
  const float* q0s = stash ? stash + n_tokens * heads * (int64_t)d * d : nullptr;
  const RescueSlots rs = (flags & TTC_LQR_FLAG_RESCUE_V1)
                             ? rescue_slots(stash, n_tokens * heads, d, du, T, (flags & TTC_LQR_FLAG_RESCUE_GAINS) != 0)
                             : RescueSlots{};
  return backward_core(A_diag, B, Q, R_inv, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, u, d_u, n_tokens, heads,
                       d, du, T, flags, v1s, q0s, grad_A_diag, grad_B, grad_Q, grad_R_inv, grad_Q_f,
                       grad_log_gamma_A, grad_log_gamma_B, grad_log_gamma_Q, grad_h0,
                       static_cast<char*>(workspace), workspace_bytes, grad_limit, status, n_fallback,
                       reinterpret_cast<hipStream_t>(stream), rs);
}

}  // namespace ttc

extern "C" {


size_t ttc_lqr_factored_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du, int32_t b_rank,
                                        int32_t q_rank, int32_t T, int32_t with_stash, int32_t backward,
                                        int32_t bf16, int32_t flags) {
  if (chunk_tokens <= 0 || !fact_args_ok(chunk_tokens, heads, d, du, b_rank, q_rank, T) || du != d) return 0;
  return fact_layout(chunk_tokens, heads, d, du, b_rank, q_rank, T, with_stash != 0, backward != 0, bf16 != 0,
                     with_stash == 2, flags)
      .total;
}

int ttc_lqr_forward_factored(const float* A_diag, const float* coeff_B, const float* coeff_Q, const float* R_inv,
                             const float* coeff_Qf, const float* log_gamma_A, const float* log_gamma_B,
                             const float* log_gamma_Q, const float* h0, const float* B_basis, const float* Q_basis,
                             int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t b_rank, int32_t q_rank,
                             int32_t T, int32_t flags, float* u, float* stash, void* workspace,
                             size_t workspace_bytes, int32_t* status, void* stream) {
  return forward_factored_entry<float>(A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, log_gamma_A, log_gamma_B,
                                       log_gamma_Q, h0, B_basis, Q_basis, n_tokens, heads, d, du, b_rank, q_rank, T,
                                       flags, u, stash, workspace, workspace_bytes, status, stream);
}

int ttc_lqr_forward_factored_bf16(const uint16_t* A_diag, const uint16_t* coeff_B, const uint16_t* coeff_Q,
                                  const uint16_t* R_inv, const uint16_t* coeff_Qf, const uint16_t* log_gamma_A,
                                  const uint16_t* log_gamma_B, const uint16_t* log_gamma_Q, const uint16_t* h0,
                                  const uint16_t* B_basis, const uint16_t* Q_basis, int64_t n_tokens, int32_t heads,
                                  int32_t d, int32_t du, int32_t b_rank, int32_t q_rank, int32_t T, int32_t flags,
                                  float* u, float* stash, void* workspace, size_t workspace_bytes, int32_t* status,
                                  void* stream) {
  return forward_factored_entry<uint16_t>(A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, log_gamma_A, log_gamma_B,
                                          log_gamma_Q, h0, B_basis, Q_basis, n_tokens, heads, d, du, b_rank, q_rank,
                                          T, flags, u, stash, workspace, workspace_bytes, status, stream);
}

int ttc_lqr_backward_factored(const float* A_diag, const float* coeff_B, const float* coeff_Q, const float* R_inv,
                              const float* coeff_Qf, const float* log_gamma_A, const float* log_gamma_B,
                              const float* log_gamma_Q, const float* h0, const float* B_basis, const float* Q_basis,
                              const float* u, const float* d_u, int64_t n_tokens, int32_t heads, int32_t d,
                              int32_t du, int32_t b_rank, int32_t q_rank, int32_t T, int32_t flags,
                              const float* stash, float* grad_A_diag, float* grad_coeff_B, float* grad_coeff_Q,
                              float* grad_R_inv, float* grad_coeff_Qf, float* grad_log_gamma_A,
                              float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0,
                              float* grad_B_basis, float* grad_Q_basis, void* workspace, size_t workspace_bytes,
                              float grad_limit, int32_t* status, int64_t* n_fallback, void* stream) {
  return backward_factored_entry<float>(
      A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, log_gamma_A, log_gamma_B, log_gamma_Q, h0, B_basis, Q_basis, u, d_u,
      n_tokens, heads, d, du, b_rank, q_rank, T, flags, stash, grad_A_diag, grad_coeff_B, grad_coeff_Q, grad_R_inv,
      grad_coeff_Qf, grad_log_gamma_A, grad_log_gamma_B, grad_log_gamma_Q, grad_h0, grad_B_basis, grad_Q_basis,
      workspace, workspace_bytes, grad_limit, status, n_fallback, stream);
}

int ttc_lqr_backward_factored_bf16(const uint16_t* A_diag, const uint16_t* coeff_B, const uint16_t* coeff_Q,
                                   const uint16_t* R_inv, const uint16_t* coeff_Qf, const uint16_t* log_gamma_A,
                                   const uint16_t* log_gamma_B, const uint16_t* log_gamma_Q, const uint16_t* h0,
                                   const uint16_t* B_basis, const uint16_t* Q_basis, const float* u,
                                   const uint16_t* d_u, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                                   int32_t b_rank, int32_t q_rank, int32_t T, int32_t flags, const float* stash,
                                   uint16_t* grad_A_diag, uint16_t* grad_coeff_B, uint16_t* grad_coeff_Q,
                                   uint16_t* grad_R_inv, uint16_t* grad_coeff_Qf, uint16_t* grad_log_gamma_A,
                                   uint16_t* grad_log_gamma_B, uint16_t* grad_log_gamma_Q, uint16_t* grad_h0,
                                   uint16_t* grad_B_basis, uint16_t* grad_Q_basis, void* workspace,
                                   size_t workspace_bytes, float grad_limit, int32_t* status, int64_t* n_fallback,
                                   void* stream) {
  return backward_factored_entry<uint16_t>(
      A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf, log_gamma_A, log_gamma_B, log_gamma_Q, h0, B_basis, Q_basis, u, d_u,
      n_tokens, heads, d, du, b_rank, q_rank, T, flags, stash, grad_A_diag, grad_coeff_B, grad_coeff_Q, grad_R_inv,
      grad_coeff_Qf, grad_log_gamma_A, grad_log_gamma_B, grad_log_gamma_Q, grad_h0, grad_B_basis, grad_Q_basis,
      workspace, workspace_bytes, grad_limit, status, n_fallback, stream);
}

}  // extern "C"
