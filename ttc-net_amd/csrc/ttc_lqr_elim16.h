// ttc_lqr_elim16.h -- one pivot step of the d = 16 row-layout LDL' elimination as
// fused DPP multiply-adds.
//
// Row layout: lane (g, c) of a wave holds row c of problem g's stacked matrix
// [Quu; W; I] in registers q[16], w[16], i[16].  Pivot k subtracts a multiple of the
// pivot row (row k of the trailing Quu, held by lane k of the same 16-lane row) from
// every row:  x[m] += bcast_k(q[m]) * nx  for m > k,  nx = -x[k] / pivot.
// `v_fmac_f32_dpp dst, src0, src1 row_newbcast:k` computes dst += src0[lane k] * src1,
// so each update is one instruction with the broadcast folded in.  The pivot row is
// read before it is updated (the w and i updates come before the q update of the
// same column), which keeps lane k's own row intact until its last use.
//
// One asm statement per pivot keeps the order of its updates fixed.  Hazard: a DPP
// source must not be written by a VALU instruction in the two preceding wait states.
// Every q[m] read here was written by the previous pivot's statement, and between the
// two statements sit at least the pivot broadcast, the reciprocal and the multiplier
// products that this statement consumes (three VALU instructions).
#pragma once
#include <hip/hip_runtime.h>

#define TTC_E2(K, M)                                                                  \
  "v_fmac_f32_dpp %[w" #M "], %[q" #M "], %[nw] row_newbcast:" #K                   \
  " row_mask:0xf bank_mask:0xf\n\t"                                                   \
  "v_fmac_f32_dpp %[q" #M "], %[q" #M "], %[nq] row_newbcast:" #K                   \
  " row_mask:0xf bank_mask:0xf\n\t"
#define TTC_E3(K, M)                                                                  \
  "v_fmac_f32_dpp %[w" #M "], %[q" #M "], %[nw] row_newbcast:" #K                   \
  " row_mask:0xf bank_mask:0xf\n\t"                                                   \
  "v_fmac_f32_dpp %[i" #M "], %[q" #M "], %[ni] row_newbcast:" #K                   \
  " row_mask:0xf bank_mask:0xf\n\t"                                                   \
  "v_fmac_f32_dpp %[q" #M "], %[q" #M "], %[nq] row_newbcast:" #K                   \
  " row_mask:0xf bank_mask:0xf\n\t"

// E(K, M) for M = first..15
#define TTC_R15(E, K) E(K, 15)
#define TTC_R14(E, K) E(K, 14) TTC_R15(E, K)
#define TTC_R13(E, K) E(K, 13) TTC_R14(E, K)
#define TTC_R12(E, K) E(K, 12) TTC_R13(E, K)
#define TTC_R11(E, K) E(K, 11) TTC_R12(E, K)
#define TTC_R10(E, K) E(K, 10) TTC_R11(E, K)
#define TTC_R9(E, K) E(K, 9) TTC_R10(E, K)
#define TTC_R8(E, K) E(K, 8) TTC_R9(E, K)
#define TTC_R7(E, K) E(K, 7) TTC_R8(E, K)
#define TTC_R6(E, K) E(K, 6) TTC_R7(E, K)
#define TTC_R5(E, K) E(K, 5) TTC_R6(E, K)
#define TTC_R4(E, K) E(K, 4) TTC_R5(E, K)
#define TTC_R3(E, K) E(K, 3) TTC_R4(E, K)
#define TTC_R2(E, K) E(K, 2) TTC_R3(E, K)
#define TTC_R1(E, K) E(K, 1) TTC_R2(E, K)

#define TTC_OPS16(X, a)                                                                              \
  [X##0] "+v"(a[0]), [X##1] "+v"(a[1]), [X##2] "+v"(a[2]), [X##3] "+v"(a[3]), [X##4] "+v"(a[4]),   \
  [X##5] "+v"(a[5]), [X##6] "+v"(a[6]), [X##7] "+v"(a[7]), [X##8] "+v"(a[8]), [X##9] "+v"(a[9]),   \
  [X##10] "+v"(a[10]), [X##11] "+v"(a[11]), [X##12] "+v"(a[12]), [X##13] "+v"(a[13]),              \
  [X##14] "+v"(a[14]), [X##15] "+v"(a[15])

namespace ttc {

template <int K>
struct Elim16;

#define TTC_ELIM16(K, FIRST)                                                                              \
  template <>                                                                                             \
  struct Elim16<K> {                                                                                      \
    static __device__ __forceinline__ void qw(float (&q)[16], float (&w)[16], float nq, float nw) {       \
      asm volatile(TTC_R##FIRST(TTC_E2, K) : TTC_OPS16(q, q), TTC_OPS16(w, w) : [nq] "v"(nq), [nw] "v"(nw)); \
    }                                                                                                     \
    static __device__ __forceinline__ void qwi(float (&q)[16], float (&w)[16], float (&i)[16], float nq,   \
                                               float nw, float ni) {                                      \
      asm volatile(TTC_R##FIRST(TTC_E3, K)                                                                \
                   : TTC_OPS16(q, q), TTC_OPS16(w, w), TTC_OPS16(i, i)                                    \
                   : [nq] "v"(nq), [nw] "v"(nw), [ni] "v"(ni));                                           \
    }                                                                                                     \
  };

TTC_ELIM16(0, 1)
TTC_ELIM16(1, 2)
TTC_ELIM16(2, 3)
TTC_ELIM16(3, 4)
TTC_ELIM16(4, 5)
TTC_ELIM16(5, 6)
TTC_ELIM16(6, 7)
TTC_ELIM16(7, 8)
TTC_ELIM16(8, 9)
TTC_ELIM16(9, 10)
TTC_ELIM16(10, 11)
TTC_ELIM16(11, 12)
TTC_ELIM16(12, 13)
TTC_ELIM16(13, 14)
TTC_ELIM16(14, 15)

#undef TTC_ELIM16

// Gauss-Jordan elimination without row exchanges in the row layout, one or two systems
// [M | b] per lane (lane li of a problem's 16 lanes owns row li: x[0..15] = row li of M,
// x[16] = b[li]; likewise y).  The updates of pivot k are one asm statement (the compiler
// does not fold a row_newbcast move into v_fmac_f32):  x[m] += bcast_k(x[m]) * nx for
// m > k, where nx = 0 on lane k keeps the pivot row itself.  Hazard: a DPP source must not
// be written by a VALU instruction in the two preceding wait states, so each statement
// starts and ends with s_nop 1.
#define TTC_GJ_ONE(K, M)                                                                    \
  "v_fmac_f32_dpp %[x" #M "], %[x" #M "], %[nx] row_newbcast:" #K                          \
  " row_mask:0xf bank_mask:0xf\n\t"
#define TTC_GJ_PAIR(K, M)                                                                   \
  TTC_GJ_ONE(K, M)                                                                          \
  "v_fmac_f32_dpp %[y" #M "], %[y" #M "], %[ny] row_newbcast:" #K                          \
  " row_mask:0xf bank_mask:0xf\n\t"
#define TTC_R16(E, K)

template <int K>
struct GjSpd;

#define TTC_GJSPD(K, FIRST)                                                                                 \
  template <>                                                                                               \
  struct GjSpd<K> {                                                                                         \
    static __device__ __forceinline__ void upd(float (&x)[17], float nx) {                                  \
      asm volatile("s_nop 1\n\t" TTC_R##FIRST(TTC_GJ_ONE, K) TTC_GJ_ONE(K, 16) "s_nop 1"                    \
                   : TTC_OPS16(x, x), [x16] "+v"(x[16])                                                     \
                   : [nx] "v"(nx));                                                                         \
    }                                                                                                       \
    static __device__ __forceinline__ void upd(float (&x)[17], float (&y)[17], float nx, float ny) {        \
      asm volatile("s_nop 1\n\t" TTC_R##FIRST(TTC_GJ_PAIR, K) TTC_GJ_PAIR(K, 16) "s_nop 1"                  \
                   : TTC_OPS16(x, x), [x16] "+v"(x[16]), TTC_OPS16(y, y), [y16] "+v"(y[16])                  \
                   : [nx] "v"(nx), [ny] "v"(ny));                                                           \
    }                                                                                                       \
  };

TTC_GJSPD(0, 1)
TTC_GJSPD(1, 2)
TTC_GJSPD(2, 3)
TTC_GJSPD(3, 4)
TTC_GJSPD(4, 5)
TTC_GJSPD(5, 6)
TTC_GJSPD(6, 7)
TTC_GJSPD(7, 8)
TTC_GJSPD(8, 9)
TTC_GJSPD(9, 10)
TTC_GJSPD(10, 11)
TTC_GJSPD(11, 12)
TTC_GJSPD(12, 13)
TTC_GJSPD(13, 14)
TTC_GJSPD(14, 15)
TTC_GJSPD(15, 16)

#undef TTC_GJSPD
#undef TTC_R16
#undef TTC_GJ_PAIR
#undef TTC_GJ_ONE

}  // namespace ttc
