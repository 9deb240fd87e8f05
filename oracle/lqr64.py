"""fp64 numpy oracle: discounted receding-horizon LQR, forward ``u0`` and all nine
input gradients.  TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Problem (one per token ``n`` and head ``h``), restating the reference:

* discount expansion, ``ttc/solvers/torch_lqr.py:65-91``::

      A_k  = diag(1 + a * exp(lgA*(k+1)))           k = 0..T-1
      B_k  = B @ diag(exp(lgB*(k+1)))
      Qc_k = diag(exp(lgQ*k)) Q diag(exp(lgQ*k))     cost on h_k, k = 1..T-1
      Q_f                                           cost on h_T
      R    = diag(1 / R_inv)

* Riccati sweep and first action, ``ttc/solvers/lin_solver_lqr.py:113-212``
  (``solve_traj_actions``), done here entirely in fp64 (the reference casts the
  gain solve to fp32 at :175-177; ``ref_torch`` keeps that cast, this oracle
  does not -- it is the exact-arithmetic stand-in).
* backward: the implicit-differentiation formulas of ``KKTLQRSolveFunc``
  (``ttc/solvers/torch_lqr.py:34-63``): an adjoint LQR with linear control cost
  ``d_u`` on ``u_0`` and ``h_0 = 0``, closed-loop rollouts of both problems,
  reverse costate sweeps (``lin_solver_lqr.py:13-110``), outer-product
  gradients, then the chain rule through the discount expansion (which the
  reference leaves to torch autograd through ``_generate_parameters``).

Symmetry convention: the QP optimum depends on ``Q`` and ``Q_f`` only through
their symmetric parts, so this oracle symmetrises both on entry and returns the
symmetric gradient for them (identical to the reference for symmetric inputs,
which is what ``TTCLayer`` produces and what ``bench_lqr_solvers.py:125,127``
feeds).

Pinning (tests/test_oracle.py):
* ``expand_step``: closed forms checked element-wise against an independent
  vectorised expansion written from the formulas above, plus an off-by-one
  mutation that must fail.
* ``solve_u0``: fp64 dense QP brute force (``dense_qp``), the T=1 closed form,
  scipy ``solve_discrete_are`` in the undiscounted long-horizon limit,
  linearity in ``h0`` and symmetric-part invariance.
* ``solve_grads``: fp64 autograd of the dense QP on all nine inputs, finite
  differences, and ``torch.autograd.gradcheck`` of the dense QP itself.
"""
from __future__ import annotations

import numpy as np

__all__ = ["LQRProblem", "solve_u0", "solve_grads", "expand_step"]


def _f64(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def _mv(M, v):
    return (M @ v[:, :, None])[:, :, 0]


def _sym(m):
    return 0.5 * (m + np.swapaxes(m, -1, -2))


class LQRProblem:
    """The nine solver inputs, flattened to ``P = N*H`` independent problems.

    Input shapes follow the reference boundary (``fused_lqr.py:37-45``):
    ``A_diag [N,H,d]``, ``B [N,d,du]``, ``Q [N,d,d]``, ``R_inv [N,H,du]``,
    ``Q_f [N,H,d,d]``, ``lgA [N,H]``, ``lgB [N,H,du]``, ``lgQ [N,H,d]``,
    ``h0 [N,H,d]``.
    """

    def __init__(self, A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0, T: int):
        A_diag, B, Q, R_inv, Q_f = map(_f64, (A_diag, B, Q, R_inv, Q_f))
        lgA, lgB, lgQ, h0 = map(_f64, (lgA, lgB, lgQ, h0))
        N, H, d = A_diag.shape
        du = B.shape[-1]
        assert B.shape == (N, d, du) and Q.shape == (N, d, d)
        assert R_inv.shape == (N, H, du) and Q_f.shape == (N, H, d, d)
        assert lgA.shape == (N, H) and lgB.shape == (N, H, du)
        assert lgQ.shape == (N, H, d) and h0.shape == (N, H, d)
        assert T >= 1
        self.N, self.H, self.d, self.du, self.T = N, H, d, du, int(T)
        P = N * H
        self.P = P
        self.a = A_diag.reshape(P, d)
        self.Bm = np.repeat(B, H, axis=0)                    # [P,d,du], head-shared
        self.Qm = np.repeat(_sym(Q), H, axis=0)              # [P,d,d], head-shared
        self.r = R_inv.reshape(P, du)
        self.Qf = _sym(Q_f).reshape(P, d, d)
        self.lgA = lgA.reshape(P)
        self.lgB = lgB.reshape(P, du)
        self.lgQ = lgQ.reshape(P, d)
        self.h0 = h0.reshape(P, d)


def expand_step(pb: LQRProblem, k: int):
    """System at step ``k`` (0-based): ``(alpha_k [P,d], B_k [P,d,du], Qc_k [P,d,d] or
    None for k == 0)``; restates ``torch_lqr.py:76-89`` one step at a time."""
    alpha = 1.0 + pb.a * np.exp(pb.lgA * (k + 1))[:, None]
    beta = np.exp(pb.lgB * (k + 1))
    Bk = pb.Bm * beta[:, None, :]
    if k == 0:
        Qc = None
    else:
        q = np.exp(pb.lgQ * k)
        Qc = q[:, :, None] * pb.Qm * q[:, None, :]
    return alpha, Bk, Qc


def _riccati(pb: LQRProblem, keep_gains: bool):
    """Backward Riccati sweep (``lin_solver_lqr.py:155-185``) in fp64.

    Returns ``K [T,P,du,d]`` (or only ``K_0``) and ``Quu_0 [P,du,du]``.
    """
    T = pb.T
    V = pb.Qf.copy()
    Ks = [None] * T if keep_gains else None
    K0 = Quu0 = None
    Rdiag = 1.0 / pb.r
    for k in range(T - 1, -1, -1):
        alpha, Bk, Qc = expand_step(pb, k)
        # Qt_aug = Q_cost + F^T V F with F = [A | B]  (:164)
        VA = V * alpha[:, None, :]                                  # V @ A
        Qxx = alpha[:, :, None] * VA                                # A V A
        if Qc is not None:
            Qxx = Qxx + Qc
        BkT = np.swapaxes(Bk, -1, -2)
        Qux = BkT @ VA                                              # B^T V A
        Quu = BkT @ (V @ Bk)                                        # B^T V B
        Quu[:, np.arange(pb.du), np.arange(pb.du)] += Rdiag
        Quu = _sym(Quu)
        K = -np.linalg.solve(Quu, Qux)                              # (:176)
        # (:184) writes V = Qxx + Qxu K + K'Qux + K'Quu K.  Since K'Quu K = -K'Qux
        # this equals Qxx + Qxu K in exact arithmetic; the 4-term form cancels
        # catastrophically once V reaches ~1e17 (config 5, T=1024), so the
        # oracle uses the 2-term form and keeps V exactly symmetric.
        V = _sym(Qxx + np.swapaxes(Qux, -1, -2) @ K)
        if keep_gains:
            Ks[k] = K
        if k == 0:
            K0, Quu0 = K, Quu
    return (np.stack(Ks) if keep_gains else K0), Quu0


def solve_u0(pb: LQRProblem) -> np.ndarray:
    """First optimal action ``u0 [N,H,du]`` (``lin_solver_lqr.py:204-210``)."""
    K0, _ = _riccati(pb, keep_gains=False)
    u0 = (K0 @ pb.h0[:, :, None])[:, :, 0]
    return u0.reshape(pb.N, pb.H, pb.du)


def solve_grads(pb: LQRProblem, dU) -> dict:
    """``u0`` and the gradients of ``sum(dU * u0)`` w.r.t. the nine inputs.

    Restates ``KKTLQRSolveFunc.backward`` (``torch_lqr.py:34-63``) plus the
    chain rule through ``_generate_parameters`` (``torch_lqr.py:76-89``).
    Memory is ``O(T*P*du*d)``: meant for test-sized problems.
    """
    dU = _f64(dU).reshape(pb.P, pb.du)
    P, d, du, T = pb.P, pb.d, pb.du, pb.T
    K, Quu0 = _riccati(pb, keep_gains=True)
    steps = [expand_step(pb, k) for k in range(T)]

    # closed-loop rollouts (lin_solver_lqr.py:195-210): primal from h0, adjoint
    # from 0 with feed-forward k_0 = -Quu_0^{-1} d_u at t = 0 only (torch_lqr.py:41-45)
    h = np.zeros((T + 1, P, d)); hb = np.zeros((T + 1, P, d))
    u = np.zeros((T, P, du)); w = np.zeros((T, P, du))
    h[0] = pb.h0
    k0 = -np.linalg.solve(Quu0, dU[:, :, None])[:, :, 0]
    for k in range(T):
        alpha, Bk, _ = steps[k]
        u[k] = _mv(K[k], h[k])
        w[k] = _mv(K[k], hb[k]) + (k0 if k == 0 else 0.0)
        h[k + 1] = alpha * h[k] + _mv(Bk, u[k])
        hb[k + 1] = alpha * hb[k] + _mv(Bk, w[k])

    # reverse costate sweeps (lin_solver_lqr.py:82-98): lam[k] = lambda_k, k = 1..T.
    # The reference recursion is lambda_k = Qc_k h_k + A_k lambda_{k+1}.  Adding
    # K_k' (R u_k + B_k' lambda_{k+1}) -- zero in exact arithmetic by stationarity
    # of u_k -- turns it into the closed-loop recursion
    #   lambda_k = Qc_k h_k + (A_k + B_k K_k)' lambda_{k+1} + K_k' R u_k,
    # which propagates rounding errors with the (contracting) closed-loop matrix
    # instead of A_k.  Same value; the open-loop form loses every digit, even in
    # fp64, on long-horizon config-5 problems where A_k ~ 1.8 for 1000 steps.
    lam = np.zeros((T + 1, P, d)); lamb = np.zeros((T + 1, P, d))
    lam[T] = _mv(pb.Qf, h[T])
    lamb[T] = _mv(pb.Qf, hb[T])
    Rdiag = 1.0 / pb.r
    for k in range(T - 1, 0, -1):
        alpha, Bk, Qc = steps[k]
        cu = Rdiag * u[k] + _mv(np.swapaxes(Bk, -1, -2), lam[k + 1])
        cw = Rdiag * w[k] + _mv(np.swapaxes(Bk, -1, -2), lamb[k + 1])
        lam[k] = _mv(Qc, h[k]) + alpha * lam[k + 1] + _mv(np.swapaxes(K[k], -1, -2), cu)
        lamb[k] = _mv(Qc, hb[k]) + alpha * lamb[k + 1] + _mv(np.swapaxes(K[k], -1, -2), cw)

    g = {k_: None for k_ in ("A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0")}
    gA = np.zeros((P, d)); glgA = np.zeros(P)
    gBp = np.zeros((P, d, du)); glgB = np.zeros((P, du))
    gQp = np.zeros((P, d, d)); glgQ = np.zeros((P, d))
    gr = np.zeros((P, du))
    for k in range(T):
        alpha, Bk, _ = steps[k]
        eA = np.exp(pb.lgA * (k + 1))
        # torch_lqr.py:51  A_grad = h_{k} * lam_bwd_{k+1} + hb_{k} * lam_fwd_{k+1}
        gAk = h[k] * lamb[k + 1] + hb[k] * lam[k + 1]
        gA += gAk * eA[:, None]
        glgA += (gAk * pb.a).sum(-1) * (k + 1) * eA
        # torch_lqr.py:53  B_grad = lam_bwd u_fwd^T + lam_fwd u_bwd^T
        gBk = lamb[k + 1][:, :, None] * u[k][:, None, :] + lam[k + 1][:, :, None] * w[k][:, None, :]
        eB = np.exp(pb.lgB * (k + 1))
        gBp += gBk * eB[:, None, :]
        glgB += (gBk * pb.Bm).sum(1) * (k + 1) * eB
        # torch_lqr.py:59  R_grad = u_fwd * u_bwd ;  R = 1/R_inv
        gr += u[k] * w[k] * (-1.0 / pb.r ** 2)
        # torch_lqr.py:55  Q_grad (symmetric) on the state h_{k+1}
        gQk = 0.5 * (hb[k + 1][:, :, None] * h[k + 1][:, None, :] + h[k + 1][:, :, None] * hb[k + 1][:, None, :])
        if k == T - 1:
            g["Q_f"] = gQk.reshape(pb.N, pb.H, d, d)
        else:
            q = np.exp(pb.lgQ * (k + 1))
            Qc = q[:, :, None] * pb.Qm * q[:, None, :]
            gQp += q[:, :, None] * gQk * q[:, None, :]
            glgQ += ((gQk * Qc).sum(2) + (gQk * Qc).sum(1)) * (k + 1)
    alpha0 = steps[0][0]
    N, H = pb.N, pb.H
    g["A_diag"] = gA.reshape(N, H, d)
    g["lgA"] = glgA.reshape(N, H)
    g["B"] = gBp.reshape(N, H, d, du).sum(1)
    g["lgB"] = glgB.reshape(N, H, du)
    g["Q"] = gQp.reshape(N, H, d, d).sum(1)
    g["lgQ"] = glgQ.reshape(N, H, d)
    g["R_inv"] = gr.reshape(N, H, du)
    g["h0"] = (alpha0 * lamb[1]).reshape(N, H, d)            # torch_lqr.py:61, lin_solver_lqr.py:100-106
    g["u"] = u[0].reshape(N, H, du)
    return g
