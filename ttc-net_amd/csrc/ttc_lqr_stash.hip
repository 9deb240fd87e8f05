// ttc_lqr_stash.hip -- the compact stash of the factored entry points: only the upper
// triangle of each problem's V_1 (d(d+1)/2 floats, rows i <= j packed row by row) is kept
// between forward and backward; the backward unpacks it per token chunk and recomputes
//   Quu_0 = R + B_0' V_1 B_0,   B_0 = B diag(exp(lgB)),  R = diag(1 / R_inv)
// (the step-0 control Hessian the forward formed, lin_solver_lqr.py:113-212) on the
// matrix cores: two D x D x D products per problem, one wave per problem.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

namespace ttc {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int64_t packed_index(int D, int i, int j) {  // i <= j
  return (int64_t)i * D - (int64_t)i * (i - 1) / 2 + (j - i);
}

// in [P, D, D] row-major -> out [P, D(D+1)/2]: one thread per (p, i, j), j >= i stores.
__global__ __launch_bounds__(256) void pack_upper_kernel(const float* __restrict__ in, int64_t P, int D,
                                                         float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t DD = (int64_t)D * D;
  if (t >= P * DD) return;
  const int64_t p = t / DD;
  const int e = (int)(t - p * DD), i = e / D, j = e % D;
  if (j >= i) out[p * (DD + D) / 2 + packed_index(D, i, j)] = in[t];
}

// out[p][i][j] = packed (min(i, j), max(i, j)): the symmetric matrix of the upper triangle.
__global__ __launch_bounds__(256) void unpack_upper_kernel(const float* __restrict__ in, int64_t P, int D,
                                                           float* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t DD = (int64_t)D * D;
  if (t >= P * DD) return;
  const int64_t p = t / DD;
  const int e = (int)(t - p * DD), i = e / D, j = e % D;
  out[t] = in[p * (DD + D) / 2 + (i <= j ? packed_index(D, i, j) : packed_index(D, j, i))];
}

// Quu_0 of every problem from V_1 [P, D, D], the token's B [N, D, D], lgB and R_inv [P, D].
// MFMA operands (lane (g, c), instruction s): W = V_1 B_0 takes V_1[16I + c][16K + 4g + s] and
// B_0[16K + 4g + s][16J + c]; Quu = R + B_0' W takes B_0[16K + 4g + s][16I + c] and the C-layout
// W[16K + 4g + s][16J + c] that the lane already holds.
template <int NB>
__global__ __launch_bounds__(256) void quu0_kernel(const float* __restrict__ v1, const float* __restrict__ Bg,
                                                   const float* __restrict__ lgB, const float* __restrict__ Rinv,
                                                   int64_t P, int H, float* __restrict__ q0) {
  constexpr int D = 16 * NB;
  constexpr float kLog2e = 1.4426950408889634f;
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (p >= P) return;  // whole waves: no barrier follows
  const int64_t n = p / H;
  const float* V = v1 + p * D * D;
  const float* B = Bg + n * D * D;
  float beta[NB];  // beta_0 of control column 16J + c (the forward's exp2 of the base-2 exponent)
#pragma unroll
  for (int J = 0; J < NB; ++J) beta[J] = __builtin_amdgcn_exp2f(lgB[p * D + 16 * J + c] * kLog2e);
  v4f W[NB][NB];
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int J = 0; J < NB; ++J) W[I][J] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int K = 0; K < NB; ++K) {
      const float4 a = *reinterpret_cast<const float4*>(V + (16 * I + c) * D + 16 * K + 4 * g);
#pragma unroll
      for (int J = 0; J < NB; ++J) {
        const float* bk = B + (16 * K + 4 * g) * D + 16 * J + c;
        W[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, bk[0] * beta[J], W[I][J], 0, 0, 0);
        W[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, bk[D] * beta[J], W[I][J], 0, 0, 0);
        W[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, bk[2 * D] * beta[J], W[I][J], 0, 0, 0);
        W[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, bk[3 * D] * beta[J], W[I][J], 0, 0, 0);
      }
    }
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    float at[NB][4];  // B_0[16K + 4g + s][16I + c]
#pragma unroll
    for (int K = 0; K < NB; ++K)
#pragma unroll
      for (int s = 0; s < 4; ++s) at[K][s] = B[(16 * K + 4 * g + s) * D + 16 * I + c] * beta[I];
#pragma unroll
    for (int J = 0; J < NB; ++J) {
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
      if (I == J) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * g + r == c) acc[r] = 1.0f / Rinv[p * D + 16 * I + c];
      }
#pragma unroll
      for (int K = 0; K < NB; ++K)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(at[K][s], W[K][J][s], acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) q0[p * D * D + (16 * I + 4 * g + r) * D + 16 * J + c] = acc[r];
    }
  }
}

static bool launched() { return hipGetLastError() == hipSuccess; }

int launch_pack_upper(const float* in, int64_t P, int D, float* out, hipStream_t s) {
  const int64_t n = P * D * D;
  if (n <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(pack_upper_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, P, D, out);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

int launch_unpack_quu0(const float* packed, const float* B, const float* lgB, const float* Rinv, int64_t P, int H,
                       int D, float* v1, float* q0, hipStream_t s) {
  const int64_t n = P * D * D;
  if (n <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(unpack_upper_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, packed, P, D, v1);
  if (!launched()) return TTC_LQR_ELAUNCH;
  const dim3 grid((unsigned)((P + 3) / 4)), block(256);
  switch (D) {
    case 16: hipLaunchKernelGGL(quu0_kernel<1>, grid, block, 0, s, v1, B, lgB, Rinv, P, H, q0); break;
    case 32: hipLaunchKernelGGL(quu0_kernel<2>, grid, block, 0, s, v1, B, lgB, Rinv, P, H, q0); break;
    case 64: hipLaunchKernelGGL(quu0_kernel<4>, grid, block, 0, s, v1, B, lgB, Rinv, P, H, q0); break;
    default: return TTC_LQR_EUNSUPPORTED;
  }
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

}  // namespace ttc
