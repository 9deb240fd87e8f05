// ttc_lqr_factored.hip -- the low-rank front-end of TTCLayer on the device
// (ttc/layers/ttc_layer.py:117-123):
//   B_n      = sum_r coeff_B[n,r]    Bs[r]      (token-shared, d x du)
//   Q_n      = sum_r coeff_Q[n,r]    G[r]       (token-shared, d x d)
//   Q_f[n,h] = sum_r coeff_Qf[n,h,r] G[r]       (per problem,  d x d)
// expanded token chunk by token chunk into the caller's workspace right before the
// solver kernels read them, and the chain rule of those sums for the backward:
//   d coeff[m,r] = <dX_m, basis_r>                 (project_kernel, one matrix product)
//   d basis[r]  += sum_m coeff[m,r] dX_m           (reduce_kernel: per-slab partials on the
//                                                   matrix cores, then sum_slabs_kernel in a
//                                                   fixed order: deterministic)
// All three are HBM-bound streams over the d x d matrices; the products run on
// v_mfma_f32_16x16x4f32 so the vector ALU never limits them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ttc_lqr.h"
#include "ttc_lqr_internal.h"

namespace ttc {

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kExpandRows = 8;  // rows of one expand thread: each basis load feeds 8 rows
constexpr int kExpandChunk = 16;  // ranks whose loads are issued together

// out[m][e] = sum_r coeff[m][r] basis[r][e]; E % 256 == 0.  One thread per 4 consecutive e of
// kExpandRows consecutive rows, so the basis (re-read from L1/L2 by every thread) costs one
// 16-byte load per 32 FMAs.  With E % 256 == 0 the 64 lanes of a wave share their row block:
// its index goes through readfirstlane, so the coefficient loads are scalar loads and every
// vector memory instruction left is a basis load or a 1 KB row store.  The ranks go in chunks
// of kExpandChunk whose basis and coefficient loads are all issued before their FMAs (one
// memory latency per chunk instead of one per rank), and the rows leave with nontemporal
// stores (written once, read by the next kernel from HBM): 2.1 -> 6.5 TB/s of stores.
// Coefficients as stored: fp32, or bf16 bit patterns (widened exactly in registers, so bf16
// storage needs no fp32 copy of them).
__device__ __forceinline__ float coeff_value(const float* p) { return *p; }
__device__ __forceinline__ float coeff_value(const uint16_t* p) { return __uint_as_float((uint32_t)*p << 16); }

template <typename TC>
__global__ __launch_bounds__(256) void expand_kernel(const TC* __restrict__ coeff, int64_t M, int R,
                                                     const float* __restrict__ basis, int E,
                                                     float* __restrict__ out) {
  const int E4 = E >> 2;
  const int64_t nblk = (M + kExpandRows - 1) / kExpandRows;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= nblk * E4) return;  // wave-uniform: nblk * E4 is a multiple of 64
  const int64_t t0 = t - (threadIdx.x & 63);  // the wave's first thread
  const int64_t mb_l = t0 / E4;
  const int64_t mb = ((int64_t)__builtin_amdgcn_readfirstlane((int)(mb_l >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(mb_l & 0xffffffff));
  const int e = (int)(t - mb * E4) * 4;
  const int64_t m0 = mb * kExpandRows;
  const TC* crow[kExpandRows];
#pragma unroll
  for (int i = 0; i < kExpandRows; ++i) crow[i] = coeff + (m0 + i < M ? m0 + i : M - 1) * R;  // tail: clamped, not stored
  float acc[kExpandRows][4];
#pragma unroll
  for (int i = 0; i < kExpandRows; ++i) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0.f;
  int r0 = 0;
  for (; r0 + kExpandChunk <= R; r0 += kExpandChunk) {
    float4 b[kExpandChunk];
    float cr[kExpandRows][kExpandChunk];
#pragma unroll
    for (int k = 0; k < kExpandChunk; ++k) b[k] = *reinterpret_cast<const float4*>(basis + (int64_t)(r0 + k) * E + e);
#pragma unroll
    for (int i = 0; i < kExpandRows; ++i)
#pragma unroll
      for (int k = 0; k < kExpandChunk; ++k) cr[i][k] = coeff_value(crow[i] + r0 + k);
#pragma unroll
    for (int k = 0; k < kExpandChunk; ++k)
#pragma unroll
      for (int i = 0; i < kExpandRows; ++i) {
        acc[i][0] = fmaf(cr[i][k], b[k].x, acc[i][0]);
        acc[i][1] = fmaf(cr[i][k], b[k].y, acc[i][1]);
        acc[i][2] = fmaf(cr[i][k], b[k].z, acc[i][2]);
        acc[i][3] = fmaf(cr[i][k], b[k].w, acc[i][3]);
      }
  }
  for (; r0 < R; ++r0) {  // ranks past the last full chunk
    const float4 b = *reinterpret_cast<const float4*>(basis + (int64_t)r0 * E + e);
#pragma unroll
    for (int i = 0; i < kExpandRows; ++i) {
      const float cr = coeff_value(crow[i] + r0);
      acc[i][0] = fmaf(cr, b.x, acc[i][0]);
      acc[i][1] = fmaf(cr, b.y, acc[i][1]);
      acc[i][2] = fmaf(cr, b.z, acc[i][2]);
      acc[i][3] = fmaf(cr, b.w, acc[i][3]);
    }
  }
#pragma unroll
  for (int i = 0; i < kExpandRows; ++i)
    if (m0 + i < M) {
      float* o = out + (m0 + i) * E + e;
#pragma unroll
      for (int k = 0; k < 4; ++k) __builtin_nontemporal_store(acc[i][k], o + k);
    }
}

// out[m][r] = sum_e X[m][e] basis[r][e]   (M x E times E x R; E % 16 == 0, R <= 16 RT).
// One wave per 16-row tile (grid-stride).  MFMA operands: lane (g, c) supplies
// X[16 tile + c][k0 + 4g + s] and basis[16 rt + c][k0 + 4g + s] to instruction s, and
// ends up holding out[16 tile + 4g + i][16 rt + c], i = 0..3.
template <int RT>
__global__ __launch_bounds__(256) void project_kernel(const float* __restrict__ X, int64_t M, int E,
                                                      const float* __restrict__ basis, int R,
                                                      float* __restrict__ out) {
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int64_t ntiles = (M + 15) / 16;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const float* br[RT];
  bool bv[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = 16 * rt + c;
    bv[rt] = r < R;
    br[rt] = basis + (int64_t)(bv[rt] ? r : 0) * E + 4 * g;
  }
  for (int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); tile < ntiles; tile += nwaves) {
    const int64_t row = tile * 16 + c;
    const bool rv = row < M;
    const float* xr = X + (rv ? row : 0) * E + 4 * g;
    v4f acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < E; k0 += 64) {  // E % 64 == 0; a chunk's loads go out before its MFMAs
      float4 a[4], b[RT][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (rv) a[u] = *reinterpret_cast<const float4*>(xr + k0 + 16 * u);
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          b[rt][u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (bv[rt]) b[rt][u] = *reinterpret_cast<const float4*>(br[rt] + k0 + 16 * u);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          acc[rt] = mfma4(a[u].x, b[rt][u].x, acc[rt]);
          acc[rt] = mfma4(a[u].y, b[rt][u].y, acc[rt]);
          acc[rt] = mfma4(a[u].z, b[rt][u].z, acc[rt]);
          acc[rt] = mfma4(a[u].w, b[rt][u].w, acc[rt]);
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int r = 16 * rt + c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = tile * 16 + 4 * g + i;
        if (m < M && r < R) out[m * R + r] = acc[rt][i];
      }
    }
  }
}

// partial[s][r][e] = sum_{m in slab s} coeff[m][r] X[m][e]  (R x M times M x E, split over
// slabs of rows_per rows, rows_per % 16 == 0).  One wave per (slab, group of ET 16-column
// tiles); E % (16 ET) == 0, R <= 16 RT.  Instruction s of a 16-row step: lane (g, c)
// supplies coeff[m][16 rt + c] and X[m][e0 + 16 et + c] with m = m0 + 4g + s, and holds
// partial[16 rt + 4g + i][e0 + 16 et + c].
template <int RT, int ET>
__global__ __launch_bounds__(64) void reduce_kernel(const float* __restrict__ coeff, int64_t M, int R,
                                                    const float* __restrict__ X, int E, int64_t rows_per,
                                                    float* __restrict__ partial) {
  const int lane = threadIdx.x, g = lane >> 4, c = lane & 15;
  const int n_eg = E / (16 * ET);
  const int eg = (int)(blockIdx.x % n_eg);
  const int64_t s = blockIdx.x / n_eg;
  const int64_t m_begin = s * rows_per;
  const int64_t m_end = (m_begin + rows_per < M) ? (m_begin + rows_per) : M;
  const int e0 = eg * 16 * ET;
  v4f acc[RT][ET];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int et = 0; et < ET; ++et) acc[rt][et] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t m0 = m_begin; m0 < m_end; m0 += 16) {
#pragma unroll
    for (int si = 0; si < 4; ++si) {
      const int64_t m = m0 + 4 * g + si;
      const bool mv = m < m_end;
      float a[RT], b[ET];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r = 16 * rt + c;
        a[rt] = (mv && r < R) ? coeff[m * R + r] : 0.f;
      }
#pragma unroll
      for (int et = 0; et < ET; ++et) b[et] = mv ? X[m * E + e0 + 16 * et + c] : 0.f;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int et = 0; et < ET; ++et) acc[rt][et] = mfma4(a[rt], b[et], acc[rt][et]);
    }
  }
  float* ps = partial + s * (int64_t)R * E;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * rt + 4 * g + i;
      if (r < R) {
#pragma unroll
        for (int et = 0; et < ET; ++et) ps[(int64_t)r * E + e0 + 16 * et + c] = acc[rt][et][i];
      }
    }
}

// project_kernel<1> and reduce_kernel<1, 16> of one X in a single pass over it, for E == 256 and
// R <= 16: one wave per slab of rows_per rows (the slabs of reduce_kernel), every row read from
// HBM once.  Each 16-row block is loaded in reduce_kernel's operand layout (lane (g, c): X[m0 + 4g +
// si][16 et + c]) and feeds its MFMAs from registers; the block also goes to an LDS tile (rows
// padded to kPRLd floats: 16-byte aligned, lanes of a store on distinct banks) and comes back in
// project_kernel's layout (lane (g, c): X[m0 + c][16 j + 4g .. + 3]) for the projection against
// basis row c, held in registers for the whole slab.  Same products in the same order as the two
// kernels, so the same results.
constexpr int kPRLd = 260;
__global__ __launch_bounds__(64) void project_reduce_kernel(const float* __restrict__ coeff, int64_t M, int R,
                                                            const float* __restrict__ X, int64_t rows_per,
                                                            const float* __restrict__ basis,
                                                            float* __restrict__ proj,
                                                            float* __restrict__ partial) {
  constexpr int E = 256;
  __shared__ __align__(16) float tile[16 * kPRLd];
  const int lane = threadIdx.x, g = lane >> 4, c = lane & 15;
  const int64_t s = blockIdx.x;
  const int64_t m_begin = s * rows_per;
  const int64_t m_end = (m_begin + rows_per < M) ? (m_begin + rows_per) : M;
  const bool cv = c < R;
  float4 bas[16];  // basis[c][16 j + 4g .. + 3]
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    bas[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (cv) bas[j] = *reinterpret_cast<const float4*>(basis + (int64_t)c * E + 16 * j + 4 * g);
  }
  v4f acc[16];
#pragma unroll
  for (int et = 0; et < 16; ++et) acc[et] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t m0 = m_begin; m0 < m_end; m0 += 16) {
    float a[4], b[4][16];
#pragma unroll
    for (int si = 0; si < 4; ++si) {
      const int64_t m = m0 + 4 * g + si;
      const bool mv = m < m_end;
      a[si] = (mv && cv) ? coeff[m * R + c] : 0.f;
#pragma unroll
      for (int et = 0; et < 16; ++et) b[si][et] = mv ? X[m * E + 16 * et + c] : 0.f;
    }
#pragma unroll
    for (int si = 0; si < 4; ++si) {
#pragma unroll
      for (int et = 0; et < 16; ++et) tile[(4 * g + si) * kPRLd + 16 * et + c] = b[si][et];
#pragma unroll
      for (int et = 0; et < 16; ++et) acc[et] = mfma4(a[si], b[si][et], acc[et]);
    }
    __syncthreads();  // the block's tile is written (one wave: orders its LDS accesses)
    v4f p = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(tile + c * kPRLd + 16 * j + 4 * g);
      p = mfma4(x.x, bas[j].x, p);
      p = mfma4(x.y, bas[j].y, p);
      p = mfma4(x.z, bas[j].z, p);
      p = mfma4(x.w, bas[j].w, p);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + 4 * g + i;
      if (m < m_end && cv) proj[m * R + c] = p[i];
    }
    __syncthreads();  // the tile is read before the next block overwrites it
  }
  float* ps = partial + s * (int64_t)R * E;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * g + i;
    if (r < R) {
#pragma unroll
      for (int et = 0; et < 16; ++et) ps[(int64_t)r * E + 16 * et + c] = acc[et][i];
    }
  }
}

// out[j][i] = (accumulate ? out[j][i] : 0) + sum_{k in [j G, min(S, (j+1) G))} in[k][i], in the
// order of k.  Grid: (ceil(n / 256), ceil(S / G)).
__global__ __launch_bounds__(256) void sum_slabs_kernel(const float* __restrict__ in, int64_t S, int64_t n,
                                                        int64_t G, float* __restrict__ out, int accumulate) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t j = blockIdx.y;
  const int64_t k0 = j * G;
  const int64_t k1 = (k0 + G < S) ? (k0 + G) : S;
  float acc = accumulate ? out[j * n + i] : 0.f;
  for (int64_t k = k0; k < k1; ++k) acc += in[k * n + i];
  out[j * n + i] = acc;
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

constexpr int kSlabGroup = 64;  // first-level group of sum_slabs_kernel

// bf16 storage (bit patterns) <-> fp32: widening is exact; narrowing rounds to nearest even
// (NaN stays NaN), as torch's .to(torch.bfloat16).
__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ in, int64_t n,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = __uint_as_float((uint32_t)in[i] << 16);
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ in, int64_t n,
                                                          uint16_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t u = __float_as_uint(in[i]);
  uint16_t r;
  if ((u & 0x7fffffffu) > 0x7f800000u) r = (uint16_t)((u >> 16) | 0x40u);  // NaN: quiet, keep the sign
  else r = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  out[i] = r;
}

static bool launched() { return hipGetLastError() == hipSuccess; }

int launch_bf16_to_f32(const uint16_t* in, int64_t n, float* out, hipStream_t s) {
  if (n <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, n, out);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

int launch_f32_to_bf16(const float* in, int64_t n, uint16_t* out, hipStream_t s) {
  if (n <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, n, out);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

// Tile shape of reduce_kernel for rank R: (RT, ET) = (1, 16), (2, 16) or (4, 8).
static void reduce_shape(int R, int& RT, int& ET) {
  RT = (R + 15) / 16;
  if (RT == 3) RT = 4;
  ET = RT <= 2 ? 16 : 8;
}

// Number of row slabs of a reduction of M rows over E columns: about 2048 waves.
int64_t factor_slabs(int64_t M, int R, int E) {
  int RT, ET;
  reduce_shape(R, RT, ET);
  const int64_t n_eg = E / (16 * ET);
  int64_t S = 2048 / n_eg;
  if (S < 1) S = 1;
  const int64_t tiles = (M + 15) / 16;
  if (S > tiles) S = tiles;
  return S < 1 ? 1 : S;
}

size_t factor_partial_floats(int64_t M, int R, int E) {
  const int64_t S = factor_slabs(M, R, E);
  const int64_t S2 = (S + kSlabGroup - 1) / kSlabGroup;
  return (size_t)(S + S2) * (size_t)R * (size_t)E;
}

template <typename TC>
static int launch_expand_t(const TC* coeff, int64_t M, int R, const float* basis, int E, float* out, hipStream_t s) {
  if (E % 256 != 0) return TTC_LQR_EINVAL;
  const int64_t threads = (M + kExpandRows - 1) / kExpandRows * (E / 4);
  if (threads <= 0) return TTC_LQR_OK;
  hipLaunchKernelGGL(expand_kernel<TC>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, coeff, M, R, basis,
                     E, out);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

int launch_expand(const float* coeff, int64_t M, int R, const float* basis, int E, float* out, hipStream_t s) {
  return launch_expand_t(coeff, M, R, basis, E, out, s);
}

int launch_expand(const uint16_t* coeff, int64_t M, int R, const float* basis, int E, float* out, hipStream_t s) {
  return launch_expand_t(coeff, M, R, basis, E, out, s);
}

int launch_project(const float* X, int64_t M, int E, const float* basis, int R, float* out, hipStream_t s) {
  if (E % 64 != 0) return TTC_LQR_EINVAL;
  if (M <= 0) return TTC_LQR_OK;
  const int64_t tiles = (M + 15) / 16;
  const int64_t blocks = (tiles + 3) / 4 < 4096 ? (tiles + 3) / 4 : 4096;
  const dim3 grid((unsigned)blocks), block(256);
  if (R <= 16) hipLaunchKernelGGL(project_kernel<1>, grid, block, 0, s, X, M, E, basis, R, out);
  else if (R <= 32) hipLaunchKernelGGL(project_kernel<2>, grid, block, 0, s, X, M, E, basis, R, out);
  else hipLaunchKernelGGL(project_kernel<4>, grid, block, 0, s, X, M, E, basis, R, out);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

// out = (accumulate ? out : 0) + the sum of the S slab partials of R x E values (sum_slabs_kernel
// twice: groups of kSlabGroup slabs, then the groups).
static int launch_sum_slabs(float* partial, int64_t S, int64_t n, float* out, int accumulate, hipStream_t s) {
  const int64_t S2 = (S + kSlabGroup - 1) / kSlabGroup;
  float* level2 = partial + S * n;
  const unsigned bx = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(sum_slabs_kernel, dim3(bx, (unsigned)S2), dim3(256), 0, s, partial, S, n, (int64_t)kSlabGroup,
                     level2, 0);
  if (!launched()) return TTC_LQR_ELAUNCH;
  hipLaunchKernelGGL(sum_slabs_kernel, dim3(bx, 1u), dim3(256), 0, s, level2, S2, n, S2, out, accumulate);
  return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
}

int launch_reduce(const float* coeff, int64_t M, int R, const float* X, int E, float* partial, float* out,
                  int accumulate, hipStream_t s) {
  const int64_t n = (int64_t)R * E;
  if (M <= 0) {
    if (accumulate) return TTC_LQR_OK;
    hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, n);
    return launched() ? TTC_LQR_OK : TTC_LQR_ELAUNCH;
  }
  int RT, ET;
  reduce_shape(R, RT, ET);
  const int64_t S = factor_slabs(M, R, E);
  const int64_t tiles = (M + 15) / 16;
  const int64_t rows_per = 16 * ((tiles + S - 1) / S);
  const int n_eg = E / (16 * ET);
  const dim3 grid((unsigned)(S * n_eg)), block(64);
  if (RT == 1) hipLaunchKernelGGL((reduce_kernel<1, 16>), grid, block, 0, s, coeff, M, R, X, E, rows_per, partial);
  else if (RT == 2) hipLaunchKernelGGL((reduce_kernel<2, 16>), grid, block, 0, s, coeff, M, R, X, E, rows_per, partial);
  else hipLaunchKernelGGL((reduce_kernel<4, 8>), grid, block, 0, s, coeff, M, R, X, E, rows_per, partial);
  if (!launched()) return TTC_LQR_ELAUNCH;
  // slabs whose row range is empty (rows_per * S > rows) hold zeros: reduce_kernel wrote them
  return launch_sum_slabs(partial, S, n, out, accumulate, s);
}

int launch_project_reduce(const float* coeff, int64_t M, int R, const float* X, int E, const float* basis,
                          float* proj, float* partial, float* out, int accumulate, hipStream_t s) {
  if (E != 256 || R > 16 || M <= 0) {
    int rc = launch_project(X, M, E, basis, R, proj, s);
    if (rc == TTC_LQR_OK) rc = launch_reduce(coeff, M, R, X, E, partial, out, accumulate, s);
    return rc;
  }
  const int64_t S = factor_slabs(M, R, E);  // reduce_kernel<1, 16>'s slabs: one group of columns
  const int64_t tiles = (M + 15) / 16;
  const int64_t rows_per = 16 * ((tiles + S - 1) / S);
  hipLaunchKernelGGL(project_reduce_kernel, dim3((unsigned)S), dim3(64), 0, s, coeff, M, R, X, rows_per, basis, proj,
                     partial);
  if (!launched()) return TTC_LQR_ELAUNCH;
  return launch_sum_slabs(partial, S, (int64_t)R * E, out, accumulate, s);
}

}  // namespace ttc
