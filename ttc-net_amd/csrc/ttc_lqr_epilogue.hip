// ttc_lqr_epilogue.hip -- the layer's rescale of the solver output (ttc/layers/ttc_layer.py:142-147)
// on the device, forward and backward:
//   l2_norm:  y = u / sqrt(sum(u^2) + 1e-6)          (fla's l2norm over the control dim)
//   h0_norm:  y = u / ||u|| * ||h0||                 (both norms detached, as the reference)
// 16 lanes per problem, D / 16 consecutive elements per lane (coalesced), sums over the
// problem's 16 lanes by DPP row rotations.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

namespace ttc {

static __device__ __forceinline__ float rowsum16(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xF, 0xF, false));  // row_ror:2
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xF, 0xF, false));  // row_ror:1
  return v;
}

template <int R>  // elements per lane; D = 16 R
__global__ __launch_bounds__(256) void rescale_kernel(const float* __restrict__ u, const float* __restrict__ h0,
                                                      int64_t P, int mode, float* __restrict__ y) {
  constexpr int D = 16 * R;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t p = t >> 4;  // whole 16-lane rows are in or out together
  if (p >= P) return;
  const int li = (int)(t & 15);
  float v[R];
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] = u[p * D + li * R + k];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < R; ++k) ss = fmaf(v[k], v[k], ss);
  ss = rowsum16(ss);
  if (mode == TTC_LQR_RESCALE_L2NORM) {
    const float s = rsqrtf(ss + 1e-6f);
#pragma unroll
    for (int k = 0; k < R; ++k) y[p * D + li * R + k] = v[k] * s;
  } else {
    float hh = 0.f;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const float h = h0[p * D + li * R + k];
      hh = fmaf(h, h, hh);
    }
    const float hn = sqrtf(rowsum16(hh)), un = sqrtf(ss);
#pragma unroll
    for (int k = 0; k < R; ++k) y[p * D + li * R + k] = v[k] / un * hn;
  }
}

template <int R>
__global__ __launch_bounds__(256) void rescale_backward_kernel(const float* __restrict__ u,
                                                               const float* __restrict__ h0,
                                                               const float* __restrict__ dy, int64_t P, int mode,
                                                               float* __restrict__ du) {
  constexpr int D = 16 * R;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t p = t >> 4;
  if (p >= P) return;
  const int li = (int)(t & 15);
  float v[R], g[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    v[k] = u[p * D + li * R + k];
    g[k] = dy[p * D + li * R + k];
  }
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    ss = fmaf(v[k], v[k], ss);
    dot = fmaf(v[k], g[k], dot);
  }
  ss = rowsum16(ss);
  if (mode == TTC_LQR_RESCALE_L2NORM) {
    // d/du_j [u_j s] with s = (|u|^2 + eps)^(-1/2):  s dy_j - u_j s^3 (u . dy)
    dot = rowsum16(dot);
    const float s = rsqrtf(ss + 1e-6f);
    const float c = s * s * s * dot;
#pragma unroll
    for (int k = 0; k < R; ++k) du[p * D + li * R + k] = fmaf(-v[k], c, s * g[k]);
  } else {
    float hh = 0.f;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const float h = h0[p * D + li * R + k];
      hh = fmaf(h, h, hh);
    }
    const float hn = sqrtf(rowsum16(hh)), un = sqrtf(ss);
#pragma unroll
    for (int k = 0; k < R; ++k) du[p * D + li * R + k] = g[k] / un * hn;  // the norms are constants
  }
}

}  // namespace ttc

using namespace ttc;

extern "C" {

int ttc_lqr_rescale(const float* u, const float* h0, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                    int32_t mode, float* y, void* stream) {
  if (n_tokens < 0 || heads <= 0 || !ttc_lqr_supported(d, du)) return n_tokens < 0 || heads <= 0 ? TTC_LQR_EINVAL
                                                                                                 : TTC_LQR_EUNSUPPORTED;
  if (mode != TTC_LQR_RESCALE_L2NORM && mode != TTC_LQR_RESCALE_H0NORM) return TTC_LQR_EINVAL;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!u || !y || (mode == TTC_LQR_RESCALE_H0NORM && !h0)) return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((P * 16 + 255) / 256)), block(256);
  switch (du) {
    case 16: hipLaunchKernelGGL(rescale_kernel<1>, grid, block, 0, s, u, h0, P, mode, y); break;
    case 32: hipLaunchKernelGGL(rescale_kernel<2>, grid, block, 0, s, u, h0, P, mode, y); break;
    default: hipLaunchKernelGGL(rescale_kernel<4>, grid, block, 0, s, u, h0, P, mode, y); break;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

int ttc_lqr_rescale_backward(const float* u, const float* h0, const float* d_y, int64_t n_tokens, int32_t heads,
                             int32_t d, int32_t du, int32_t mode, float* d_u, void* stream) {
  if (n_tokens < 0 || heads <= 0 || !ttc_lqr_supported(d, du)) return n_tokens < 0 || heads <= 0 ? TTC_LQR_EINVAL
                                                                                                 : TTC_LQR_EUNSUPPORTED;
  if (mode != TTC_LQR_RESCALE_L2NORM && mode != TTC_LQR_RESCALE_H0NORM) return TTC_LQR_EINVAL;
  if (n_tokens == 0) return TTC_LQR_OK;
  if (!u || !d_y || !d_u || (mode == TTC_LQR_RESCALE_H0NORM && !h0)) return TTC_LQR_EINVAL;
  const int64_t P = n_tokens * heads;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((P * 16 + 255) / 256)), block(256);
  switch (du) {
    case 16: hipLaunchKernelGGL(rescale_backward_kernel<1>, grid, block, 0, s, u, h0, d_y, P, mode, d_u); break;
    case 32: hipLaunchKernelGGL(rescale_backward_kernel<2>, grid, block, 0, s, u, h0, d_y, P, mode, d_u); break;
    default: hipLaunchKernelGGL(rescale_backward_kernel<4>, grid, block, 0, s, u, h0, d_y, P, mode, d_u); break;
  }
  return hipGetLastError() == hipSuccess ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // extern "C"
