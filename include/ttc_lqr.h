/*
 * ttc_lqr.h -- C ABI of the MI355X (gfx950) batched receding-horizon LQR solver
 * behind TTC-Net's TTCLayer (solver_impl="hip").
 *
 * The reference has no native boundary: its hot path is the Python/Triton pair
 *   fused_lqr_layer_fwd   (ttc/solvers/fused_lqr.py:18-146)
 *   fused_lqr_layer_bwd   (ttc/solvers/fused_lqr.py:148-253)
 * called from FusedLQRSolveFunc (fused_lqr.py:255-291).  The entry points below
 * replace exactly those two functions; the Python autograd Function in
 * ttc-net_amd/ttc/solvers/hip_lqr.py binds them with ctypes.
 *
 * Conventions
 *   - All tensors are fp32, contiguous, row-major, device pointers.  Shapes use
 *     N tokens, H heads, state dim d, control dim du, horizon T, P = N*H:
 *       A_diag [N,H,d]  B [N,d,du]  Q [N,d,d]  R_inv [N,H,du]  Q_f [N,H,d,d]
 *       log_gamma_A [N,H]  log_gamma_B [N,H,du]  log_gamma_Q [N,H,d]  h0 [N,H,d]
 *     (the reference's shapes, fused_lqr.py:37-45).
 *   - The kernels implement d == du in {16, 32, 64}; other sizes are padded by
 *     the caller (zero state rows / unit-cost dummy controls leave the solution
 *     unchanged).  Anything else returns TTC_LQR_EUNSUPPORTED.
 *   - Nothing here allocates device memory or throws.  All work is enqueued on
 *     `stream` (a hipStream_t, NULL = default stream); only ttc_lqr_backward
 *     synchronises it (one to five times per token chunk, to size its fallback).
 *   - `status` (device int32, caller-zeroed, may be NULL) receives bit flags:
 *     TTC_LQR_STATUS_NONFINITE if any output is NaN/Inf, TTC_LQR_STATUS_LARGE if
 *     a gradient has |g| >= grad_limit.  The caller reads it after the stream
 *     completes and raises on those two bits (the reference raises RuntimeError,
 *     fused_lqr.py:101,246); TTC_LQR_STATUS_RESCUED is informational.
 *   - Q and Q_f enter through their symmetric parts; the Q / Q_f gradients are
 *     the symmetric gradients (as the reference's fused/kkt solvers return).
 *   - Thread-safe and re-entrant; calls that share a workspace or stash must be
 *     ordered by the caller.
 */
#ifndef TTC_LQR_H
#define TTC_LQR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTC_LQR_OK 0
#define TTC_LQR_EINVAL 1        /* bad sizes / null pointer / workspace too small */
#define TTC_LQR_EUNSUPPORTED 2  /* d, du combination not compiled */
#define TTC_LQR_ELAUNCH 3       /* HIP launch error */
#define TTC_LQR_ESCRATCH 4      /* ttc_lqr_backward_noalloc: one token's layout exceeds its fixed scratch */

#define TTC_LQR_STATUS_NONFINITE 1
#define TTC_LQR_STATUS_LARGE 2
/* Informational, not an error: the forward's matrix-core kernel handed some problems to
 * its rescue pass (pivoted row-layout recompute).  The rescue pass skips its scan when
 * `status` is given and this bit is clear. */
#define TTC_LQR_STATUS_RESCUED 4

/* `flags` bits.  TTC_LQR_FLAG_FP64_RICCATI runs the backward-in-time Riccati sweep
 * (the gains) in fp64 arithmetic; inputs, outputs and the stash stay fp32.  Needed
 * for long, barely-discounted horizons (e.g. T = 1024 with log-normal inputs),
 * where fp32 rounding of V ~ 1e17 corrupts the gains.  The backward's stable path
 * (problems the certificate rejects, or TTC_LQR_FLAG_STABLE_BWD) then also runs in
 * fp64: gains |K| up to ~1e19 stored in fp64 in the workspace, rollouts and costates in
 * fp64, gradients written as fp32. */
#define TTC_LQR_FLAG_FP64_RICCATI 1
/* TTC_LQR_FLAG_ROW_KERNEL selects the row-layout (vector-ALU only) fp32 kernels -- the
 * forward sweep and the backward's Hamiltonian rollout, one problem per d lanes -- instead
 * of the matrix-core kernels (which roll the backward over head groups of 8 when H % 8 == 0).
 * Results agree to fp32 rounding; it serves as an independent cross-check and as a fallback. */
#define TTC_LQR_FLAG_ROW_KERNEL 2
/* TTC_LQR_FLAG_STABLE_BWD makes ttc_lqr_backward take the stable path for every problem
 * (feedback gains recomputed and stored per step, closed-loop costates) instead of the
 * certified Hamiltonian rollout.  Same results to fp32 rounding; slower. */
#define TTC_LQR_FLAG_STABLE_BWD 4
/* TTC_LQR_FLAG_RICCATI_STEPS makes the fp32 forward take a Riccati step (with its Cholesky
 * factorisation) at every horizon step on the matrix cores, instead of the default
 * symplectic sweep (three matrix products per step, one pivoted solve at the end, a
 * conditioning certificate per problem and a row-layout recompute of the problems that
 * miss it; at d = 32 for even head counts, at d = 64 for head counts that are multiples of
 * 4, otherwise Riccati steps anyway).  Same results to fp32 rounding. */
#define TTC_LQR_FLAG_RICCATI_STEPS 8
/* TTC_LQR_FLAG_COMPACT_STASH (factored entry points only): the stash holds only the upper
 * triangle of each problem's V_1 (ttc_lqr_compact_stash_bytes: d(d+1)/2 floats per problem,
 * rows i <= j packed row by row, problem-major) and the backward recomputes Quu_0 =
 * R + B_0' V_1 B_0 from it on the matrix cores -- 4x smaller at d = 64, so the stash of an
 * 8.4 M-problem d = 64 batch fits beside its inputs (70 GB instead of 275 GB) and the
 * backward needs no forward sweep.  Pass the same flag to both calls.  Same results to
 * fp32 rounding. */
#define TTC_LQR_FLAG_COMPACT_STASH 16
/* TTC_LQR_FLAG_FP64_RESCUE (d <= 32): fp64 where long horizons need it, fp32 matrix cores
 * elsewhere.  The forward runs the fp32 symplectic sweep and recomputes the problems its
 * certificate rejects -- the ill-conditioned ones, whose value matrices grow to ~1e17 -- with
 * a Riccati sweep in fp64 (instead of the fp32 rescue tiers: at d = 16 on the matrix cores,
 * given the forward workspace, else on the row layout); the backward's stable path runs in
 * fp64 (at d = 16 its gains on the matrix cores).  Combined with
 * TTC_LQR_FLAG_ROW_KERNEL or TTC_LQR_FLAG_RICCATI_STEPS (no symplectic sweep to certify), or at
 * d = 32 with an odd head count, it acts as TTC_LQR_FLAG_FP64_RICCATI. */
#define TTC_LQR_FLAG_FP64_RESCUE 32
/* TTC_LQR_FLAG_FP64_FALLBACK (d <= 32): fp64 only for the problems a certificate rejects, at
 * any horizon.  The forward is TTC_LQR_FLAG_FP64_RESCUE's (the fp32 symplectic sweep; the
 * problems its certificate rejects recomputed by an fp64 Riccati sweep, and TTC_LQR_STATUS_RESCUED
 * set when there were any).  The backward keeps the fp32 Hamiltonian rollout (head groups on the
 * matrix cores) and runs its stable path -- the problems the rollout's certificate rejects -- in
 * fp64.  A caller whose forward did not report TTC_LQR_STATUS_RESCUED may drop the flag for the
 * backward: the rejected problems of a batch whose sweep certified every problem are accurate on
 * the fp32 stable path, which is cheaper. */
#define TTC_LQR_FLAG_FP64_FALLBACK 64
/* TTC_LQR_FLAG_KEEP_EXPANDED (factored entry points only, with a stash): the forward expands
 * B, Q and Q_f into the stash buffer instead of its workspace, and the backward reads them from
 * there instead of expanding them again -- what the reference's layer does by keeping its
 * einsums' outputs for autograd.  The stash buffer is then align256(ttc_lqr_stash_bytes, or
 * ttc_lqr_compact_stash_bytes with TTC_LQR_FLAG_COMPACT_STASH) + ttc_lqr_expanded_bytes bytes:
 * after the V_1 stash, at 256-byte boundaries, B [N,d,du], Q [N,d,d] and Q_f [N,H,d,d] in fp32.
 * Pass the same flag and buffer to both calls; NULL stash with this flag: TTC_LQR_EINVAL.  The
 * other entry points ignore it.  Same results. */
#define TTC_LQR_FLAG_KEEP_EXPANDED 128
/* TTC_LQR_FLAG_RESCUE_V1 (d = du = 16, with TTC_LQR_FLAG_FP64_RESCUE, ttc_lqr_forward_ws /
 * ttc_lqr_backward / ttc_lqr_backward_noalloc, with a stash): the forward's fp64 rescue also keeps
 * the fp64 V_1 and Quu_0 of up to max(64, P/8) of the problems it recomputes (P = N * H), after
 * the stash, and the backward's fp64 second rollout tier starts those problems from them instead
 * of the stash's fp32 roundings, so more of them pass its certificate and fewer take the stable
 * path.  The stash buffer is then align256(ttc_lqr_stash_bytes) + ttc_lqr_rescue_stash_bytes
 * bytes: a slot index per problem (int32, -1 = none), then the slots (fp64 V_1 then Quu_0).
 * Pass the same flag and buffer to both calls; NULL stash with this flag: TTC_LQR_EINVAL.  Same
 * results to the certificate's tolerance. */
#define TTC_LQR_FLAG_RESCUE_V1 256
/* TTC_LQR_FLAG_RESCUE_GAINS (with TTC_LQR_FLAG_RESCUE_V1): the forward's fp64 rescue also keeps
 * every gain K_t (fp64) of the problems in its first G = min(S, max(64, P / 16)) slots (S as
 * below), after the TTC_LQR_FLAG_RESCUE_V1 record, and the backward's stable path reads them
 * instead of sweeping those problems again.  The stash buffer is then
 * align256(ttc_lqr_stash_bytes) + ttc_lqr_rescue_stash_bytes + ttc_lqr_rescue_gains_bytes bytes
 * (2 MB per kept problem at d = 16, T = 1024).  Pass the same flag and buffer to both calls.
 * Same results to the rounding of the fp64 sweep (the same kernel). */
#define TTC_LQR_FLAG_RESCUE_GAINS 512

/* Relative tolerance of the backward's certificate: a problem's Hamiltonian rollout is
 * accepted when |lambda_T - Q_f h_T| <= TOL * (|Q_f h_T| + |lambda_T|) (max norms) holds
 * for the primal and the adjoint trajectory and every gradient is finite. */
#define TTC_LQR_CERT_TOL 1e-5f

/* Library version string. */
const char* ttc_lqr_version(void);

/* Human-readable text for a TTC_LQR_* return code. */
const char* ttc_lqr_strerror(int code);

/* 1 if the kernels were compiled for this (d, du), else 0. */
int ttc_lqr_supported(int32_t d, int32_t du);

/* 1 if (d, du) is supported with these `flags` (fp64 Riccati: d <= 32), else 0.
 * TTC_LQR_FLAG_ROW_KERNEL and TTC_LQR_FLAG_STABLE_BWD are accepted for every supported (d, du). */
int ttc_lqr_supported_flags(int32_t d, int32_t du, int32_t flags);

/* Bytes of the stash ttc_lqr_forward can leave for ttc_lqr_backward: per problem the
 * value matrix V_1 (d*d floats, the cost-to-go Hessian at step 1) and the step-0 control
 * Hessian Quu_0 (du*du floats).  `T` is accepted for signature stability (unused). */
size_t ttc_lqr_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T);

/* Bytes of the compact stash (TTC_LQR_FLAG_COMPACT_STASH): 4 * N * H * d(d+1)/2. */
size_t ttc_lqr_compact_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du);

/* Bytes of the expanded B, Q and Q_f that TTC_LQR_FLAG_KEEP_EXPANDED keeps after the stash:
 * align256(4 N d du) + align256(4 N d d) + align256(4 N H d d). */
size_t ttc_lqr_expanded_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du);

/* Bytes that TTC_LQR_FLAG_RESCUE_V1 keeps after the stash: align256(4 P) + align256(8 S (d d +
 * du du)) for P = N * H problems and S = min(P, max(64, P / 8)) slots. */
size_t ttc_lqr_rescue_stash_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du);

/* Bytes that TTC_LQR_FLAG_RESCUE_GAINS keeps after that record: align256(8 G T du d) with
 * G = min(S, max(64, P / 16)). */
size_t ttc_lqr_rescue_gains_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T);

/* Workspace bytes ttc_lqr_backward needs to process `chunk_tokens` tokens per pass
 * (it loops over the tokens in chunks of that size) with these `flags` (the stable path's
 * arithmetic, fp32 or fp64, sets its size).  `with_stash` != 0 when the forward's stash is
 * passed to the backward (then V_1 / Quu_0 are not recomputed).  Includes a region of up to
 * 256 MiB for problems the certificate rejects; any workspace beyond the size returned here
 * widens that region, so the rejected problems are recomputed in fewer, larger passes. */
size_t ttc_lqr_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du, int32_t T,
                               int32_t with_stash, int32_t flags);

/* Bytes of the fallback region that recomputes `problems` rejected problems in one pass
 * (their gathered inputs and gradients and the stable path's per-step gains and
 * trajectories; about 2.6 MB per problem at d = 16, T = 1024 in fp64).  A caller that
 * expects many rejections (long, barely discounted horizons) adds this to the workspace. */
size_t ttc_lqr_fallback_bytes(int64_t problems, int32_t d, int32_t du, int32_t T, int32_t flags);

/* Forward: u = first optimal action [N,H,du] of every problem.
 * Replaces fused_lqr_layer_fwd (ttc/solvers/fused_lqr.py:18-146).
 * stash: NULL, or ttc_lqr_stash_bytes() of device memory, laid out as
 *   V_1 [P,d,d] (row-major) followed by Quu_0 [P,du,du];
 * pass it to ttc_lqr_backward to skip their recomputation (the reference keeps
 * lam0 / LU / Y3 for the same purpose, fused_lqr.py:272). */
int ttc_lqr_forward(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                    const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                    const float* log_gamma_Q, const float* h0, int64_t n_tokens, int32_t heads,
                    int32_t d, int32_t du, int32_t T, int32_t flags, float* u, float* stash,
                    int32_t* status, void* stream);

/* Bytes of the forward's optional workspace: 4 * (P + 64) with TTC_LQR_FLAG_FP64_RESCUE or
 * TTC_LQR_FLAG_FP64_FALLBACK (d <= 32), where it holds the list of problems the fp64 rescue
 * recomputes (word 0: their count; from word 64: their indices); 0 otherwise.
 * Same forward as fused_lqr_layer_fwd (ttc/solvers/fused_lqr.py:18-146); the reference's
 * solver keeps no such list (its fp32 sweep solves every problem the same way). */
size_t ttc_lqr_forward_workspace_bytes(int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                                       int32_t T, int32_t flags);

/* ttc_lqr_forward with a workspace of ttc_lqr_forward_workspace_bytes(): the fp64 rescue of
 * a symplectic sweep then lists its problems and runs full sweeps of 64 / d problems per wave
 * (without it, or with a smaller one, each wave sweeps whichever of 64 / d consecutive problems
 * are marked).  Results are identical either way.  The list is complete when the call's stream
 * has finished (a count of 0 when the certificate accepted every problem). */
int ttc_lqr_forward_ws(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                       const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                       const float* log_gamma_Q, const float* h0, int64_t n_tokens, int32_t heads,
                       int32_t d, int32_t du, int32_t T, int32_t flags, float* u, float* stash,
                       void* workspace, size_t workspace_bytes, int32_t* status, void* stream);

/* Backward: gradients of sum(d_u * u) w.r.t. the nine inputs.
 * Replaces fused_lqr_layer_bwd (ttc/solvers/fused_lqr.py:148-253).
 * u: the forward's output (needed by the fast path; may be NULL with
 * TTC_LQR_FLAG_STABLE_BWD).  stash: from ttc_lqr_forward, or NULL (V_1 and Quu_0 are
 * then recomputed by one forward sweep inside `workspace`).
 * Fast path: a Hamiltonian rollout per problem (the reference's fused backward,
 * symplectic_iter.py:542-885) with a terminal certificate (TTC_LQR_CERT_TOL); problems
 * that fail it are recomputed by the stable path (gains stored per step in the
 * workspace, closed-loop costates).  With heads % 8 == 0 the rollout runs over head
 * groups of 8 in fp32; under TTC_LQR_FLAG_FP64_RICCATI / _FP64_RESCUE the problems of
 * the groups it rejects are rolled again one by one in fp64 before any reaches the
 * stable path, and at d = 16 those that still fail after starting from the stash's fp32
 * V_1 once more from an fp64 V_1 of a certified fp64 symplectic sweep.  *n_fallback (host,
 * may be NULL) receives the number of problems that took the stable path.  Reading the
 * rejected counts synchronises `stream` once per token chunk (twice with the fp64 second
 * rollout, four times with the third, five with TTC_LQR_FLAG_RESCUE_GAINS).
 * grad_B / grad_Q are summed over heads (B and Q are head-shared).
 * workspace_bytes must be at least ttc_lqr_workspace_bytes(1, ...); larger workspaces
 * give fewer, larger passes.  grad_limit: |g| >= grad_limit sets TTC_LQR_STATUS_LARGE
 * (the reference uses 1e6, fused_lqr.py:245); pass INFINITY to disable. */
int ttc_lqr_backward(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                     const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                     const float* log_gamma_Q, const float* h0, const float* u, const float* d_u,
                     int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags,
                     const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                     float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                     float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, void* workspace,
                     size_t workspace_bytes, float grad_limit, int32_t* status, int64_t* n_fallback,
                     void* stream);

/* ---- Factored inputs: the low-rank front-end of TTCLayer (ttc/layers/ttc_layer.py:117-123) ----
 * Instead of B, Q, Q_f the solver takes the layer's mixture coefficients and bases:
 *   coeff_B [N,rb]  coeff_Q [N,rq]  coeff_Qf [N,H,rq]  B_basis [rb,d,du]  Q_basis [rq,d,d]
 *   B_n = sum_r coeff_B[n,r] B_basis[r],  Q_n = sum_r coeff_Q[n,r] Q_basis[r],
 *   Q_f[n,h] = sum_r coeff_Qf[n,h,r] Q_basis[r]
 * (the reference's einsums "...r,rmn->...mn"; for q_reparam="cholesky" the caller passes
 * Q_basis[r] = Qs[r] Qs[r]' / sqrt(h_dim)).  The library expands them token chunk by
 * token chunk inside `workspace` just before the solver kernels read them, so the
 * [N,H,d,d] Q_f (137 GB at d = 64, 8.4 M problems) and its gradient never exist in full.
 * Ranks 1..64; basis pointers 16-byte aligned.  Results equal ttc_lqr_forward /
 * ttc_lqr_backward on the expanded tensors (same kernels), up to the fp32 rounding of
 * the expansion.  No counterpart in the reference (whose layer materialises B, Q, Q_f),
 * proposed as its next component; the entry points keep the conventions above. */

/* Workspace bytes of the factored entry points for `chunk_tokens` tokens per pass:
 * with_stash = 0 (no stash), 1 (stash), 2 (compact stash: plus the chunk's full V_1 and Quu_0);
 * backward = 0 for ttc_lqr_forward_factored (the expanded B, Q, Q_f of a chunk),
 * backward != 0 for ttc_lqr_backward_factored (plus the chunk's B / Q / Q_f gradients,
 * the reduction partials and ttc_lqr_backward's own workspace); bf16 != 0 for the _bf16
 * entry points (plus fp32 copies of the chunk's inputs, gradients and the bases); flags as for
 * ttc_lqr_workspace_bytes (the backward's beyond-layout workspace widens its fallback passes). */
size_t ttc_lqr_factored_workspace_bytes(int64_t chunk_tokens, int32_t heads, int32_t d, int32_t du,
                                        int32_t b_rank, int32_t q_rank, int32_t T, int32_t with_stash,
                                        int32_t backward, int32_t bf16, int32_t flags);

/* Forward on factored inputs; u, stash, status and flags as ttc_lqr_forward.
 * workspace_bytes >= ttc_lqr_factored_workspace_bytes(1, ..., backward = 0). */
int ttc_lqr_forward_factored(const float* A_diag, const float* coeff_B, const float* coeff_Q,
                             const float* R_inv, const float* coeff_Qf, const float* log_gamma_A,
                             const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                             const float* B_basis, const float* Q_basis, int64_t n_tokens, int32_t heads,
                             int32_t d, int32_t du, int32_t b_rank, int32_t q_rank, int32_t T,
                             int32_t flags, float* u, float* stash, void* workspace, size_t workspace_bytes,
                             int32_t* status, void* stream);

/* Backward on factored inputs: the gradients of sum(d_u * u) w.r.t. the eleven inputs.
 * grad_coeff_B [N,rb] = <grad_B_n, B_basis[r]>, grad_coeff_Q [N,rq], grad_coeff_Qf [N,H,rq]
 * likewise with Q_basis, grad_B_basis [rb,d,du] = sum_n coeff_B[n,r] grad_B_n and
 * grad_Q_basis [rq,d,d] = sum_n coeff_Q[n,r] grad_Q_n + sum_(n,h) coeff_Qf[n,h,r] grad_Q_f[n,h],
 * where grad_B / grad_Q / grad_Q_f are ttc_lqr_backward's (head-summed, symmetric).  The
 * basis gradients are summed in a fixed order (deterministic).  grad_limit and the status
 * bits apply to grad_B / grad_Q / grad_Q_f as in ttc_lqr_backward.
 * workspace_bytes >= ttc_lqr_factored_workspace_bytes(1, ..., backward = 1). */
int ttc_lqr_backward_factored(const float* A_diag, const float* coeff_B, const float* coeff_Q,
                              const float* R_inv, const float* coeff_Qf, const float* log_gamma_A,
                              const float* log_gamma_B, const float* log_gamma_Q, const float* h0,
                              const float* B_basis, const float* Q_basis, const float* u, const float* d_u,
                              int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t b_rank,
                              int32_t q_rank, int32_t T, int32_t flags, const float* stash,
                              float* grad_A_diag, float* grad_coeff_B, float* grad_coeff_Q,
                              float* grad_R_inv, float* grad_coeff_Qf, float* grad_log_gamma_A,
                              float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0,
                              float* grad_B_basis, float* grad_Q_basis, void* workspace,
                              size_t workspace_bytes, float grad_limit, int32_t* status,
                              int64_t* n_fallback, void* stream);

/* ---- Layer epilogue: the rescale of the solver output (ttc/layers/ttc_layer.py:142-147) ----
 * y = rescale(u) per problem over the control dim, on `stream`; d == du in {16, 32, 64}
 * (padded dims: padded controls are 0, padded states of h0 are 0, so norms are unchanged).
 *   TTC_LQR_RESCALE_L2NORM:  y = u / sqrt(sum(u^2) + 1e-6)   (fla's l2norm; h0 unused)
 *   TTC_LQR_RESCALE_H0NORM:  y = u / ||u|| * ||h0||           (norms treated as constants
 *                            in the backward, as the reference detaches them)
 * ttc_lqr_rescale_backward maps d_y to d_u (the gradient into ttc_lqr_backward*); no
 * gradient flows to h0.  Replaces the torch ops of the layer's back-end; with them the
 * layer needs no NaN check of its own (ttc_layer.py:139): non-finite u already sets
 * TTC_LQR_STATUS_NONFINITE in the forward's status word. */
#define TTC_LQR_RESCALE_L2NORM 1
#define TTC_LQR_RESCALE_H0NORM 2
int ttc_lqr_rescale(const float* u, const float* h0, int64_t n_tokens, int32_t heads, int32_t d, int32_t du,
                    int32_t mode, float* y, void* stream);
int ttc_lqr_rescale_backward(const float* u, const float* h0, const float* d_y, int64_t n_tokens,
                             int32_t heads, int32_t d, int32_t du, int32_t mode, float* d_u, void* stream);

/* bf16 storage (config 4 stores its activations in bf16): the same two entry points with
 * every input, d_u and every gradient stored as bf16 (raw bit patterns, uint16_t); u and
 * the stash stay fp32 (the backward's rollout starts from u).  Each token chunk is widened
 * to fp32 inside `workspace` (exact), the kernels keep their fp32 state and arithmetic, and
 * the gradients are rounded to bf16 (nearest even) when stored: the results are the fp32
 * entry points' on the widened inputs, rounded.  No 16-byte alignment is required. */
int ttc_lqr_forward_factored_bf16(const uint16_t* A_diag, const uint16_t* coeff_B, const uint16_t* coeff_Q,
                                  const uint16_t* R_inv, const uint16_t* coeff_Qf, const uint16_t* log_gamma_A,
                                  const uint16_t* log_gamma_B, const uint16_t* log_gamma_Q, const uint16_t* h0,
                                  const uint16_t* B_basis, const uint16_t* Q_basis, int64_t n_tokens,
                                  int32_t heads, int32_t d, int32_t du, int32_t b_rank, int32_t q_rank, int32_t T,
                                  int32_t flags, float* u, float* stash, void* workspace, size_t workspace_bytes,
                                  int32_t* status, void* stream);

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
                                   void* stream);

/* ---- Allocation-free backward ----
 * No counterpart in the reference.  For callers that cannot allocate device memory -- tight
 * serving loops, harnesses that forbid hipMalloc: ttc_lqr_backward with the workspace replaced by
 * a fixed device scratch of TTC_LQR_NOALLOC_SCRATCH_BYTES (256 MiB), a file-scope array of the
 * library that each GPU it runs on holds until the process ends.  Same arguments, results and
 * status bits as ttc_lqr_backward; the tokens are processed in chunks that fit the scratch, and
 * each chunk reads its rejected-problem count back to the host and synchronises the stream, so
 * the call cannot be recorded by HIP graph capture.  Returns TTC_LQR_ESCRATCH when even one
 * token's layout does not fit (e.g. d = 64 with T = 1024).  Calls no hipMalloc / hipFree.  Calls
 * that overlap on one GPU share its scratch and race: the caller orders them. */
#define TTC_LQR_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)

/* Size of the fixed scratch of ttc_lqr_backward_noalloc. */
size_t ttc_lqr_noalloc_scratch_bytes(void);

int ttc_lqr_backward_noalloc(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                             const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                             const float* log_gamma_Q, const float* h0, const float* u, const float* d_u,
                             int64_t n_tokens, int32_t heads, int32_t d, int32_t du, int32_t T, int32_t flags,
                             const float* stash, float* grad_A_diag, float* grad_B, float* grad_Q,
                             float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A, float* grad_log_gamma_B,
                             float* grad_log_gamma_Q, float* grad_h0, float grad_limit, int32_t* status,
                             int64_t* n_fallback, void* stream);

/* ---- Host (CPU) solver: the same problems on CPU tensors ----
 * Replace the reference's device-agnostic pure-PyTorch solvers for CPU tensors:
 *   ttc_lqr_forward_host   <- direct_lqr_solve / kkt_lqr_solve forward (ttc/solvers/torch_lqr.py:93-140,
 *                             the Riccati sweep of lin_solver_lqr.py:113-212)
 *   ttc_lqr_backward_host  <- KKTLQRSolveFunc.backward (torch_lqr.py:34-63) chained through the
 *                             discount expansion (torch_lqr.py:65-91)
 * so that TTCLayer(..., solver_impl="riccati" | "kkt") runs without a GPU.  Host pointers
 * (fp32, contiguous, the shapes above), any d, du >= 1; arithmetic in fp64; no GPU call.
 * `status` (host, may be NULL) receives the status bits as above (the backward's magnitude
 * guard covers the gradients of A_diag, B, Q, R_inv, Q_f and h0, as fused_lqr.py:243-246).
 * n_threads: worker threads (<= 0: all hardware threads); tokens are split over them, and
 * the head sums of grad_B / grad_Q are formed in head order (deterministic). */
int ttc_lqr_forward_host(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                         const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                         const float* log_gamma_Q, const float* h0, int64_t n_tokens, int32_t heads, int32_t d,
                         int32_t du, int32_t T, float* u, int32_t* status, int32_t n_threads);

int ttc_lqr_backward_host(const float* A_diag, const float* B, const float* Q, const float* R_inv,
                          const float* Q_f, const float* log_gamma_A, const float* log_gamma_B,
                          const float* log_gamma_Q, const float* h0, const float* d_u, int64_t n_tokens,
                          int32_t heads, int32_t d, int32_t du, int32_t T, float* grad_A_diag, float* grad_B,
                          float* grad_Q, float* grad_R_inv, float* grad_Q_f, float* grad_log_gamma_A,
                          float* grad_log_gamma_B, float* grad_log_gamma_Q, float* grad_h0, float grad_limit,
                          int32_t* status, int32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif /* TTC_LQR_H */
