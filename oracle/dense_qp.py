"""fp64 brute-force dense QP for the discounted LQR (TEST INFRASTRUCTURE ONLY).

Independent of any Riccati recursion: all controls ``z = (u_0..u_{T-1})`` are
stacked, the states are written as ``h_k = S_k z + f_k`` by direct forward
substitution of the dynamics, the quadratic ``0.5 z'Hz + c'z`` is assembled and
solved with one dense Cholesky solve.  Every operation is a torch op, so
autograd gives all nine input gradients.  The discount expansion is written
here in vectorised form from the closed forms of ``torch_lqr.py:76-89`` (it is
not shared with ``lqr64.expand_step``, so the two pin each other).

Sizes: ``T*du`` up to a few hundred, a handful of problems.

Pinning: checked by ``torch.autograd.gradcheck`` on tiny sizes and against the
T=1 closed form ``u0 = -(R + B0'Qf B0)^{-1} B0'Qf A0 h0`` (tests/test_oracle.py).
"""
from __future__ import annotations

import torch

__all__ = ["dense_qp_u0"]


def dense_qp_u0(A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0, T: int):
    """First optimal action ``u0 [N,H,du]`` of the discounted LQR, fp64, differentiable.

    Q and Q_f enter only through the quadratic forms of the objective.
    """
    N, H, d = A_diag.shape
    du = B.shape[-1]
    dt = torch.float64
    P = N * H
    a = A_diag.reshape(P, d).to(dt)
    Bm = B.to(dt).repeat_interleave(H, dim=0)                      # [P,d,du]
    # Q, Q_f enter only through the quadratic forms h'Qh (no explicit symmetrisation):
    # S'CS is symmetrised once below, which is exactly the symmetric part's contribution.
    Qm = Q.to(dt).repeat_interleave(H, dim=0)
    Qf = Q_f.to(dt).reshape(P, d, d)
    r = R_inv.to(dt).reshape(P, du)
    la = lgA.to(dt).reshape(P)
    lb = lgB.to(dt).reshape(P, du)
    lq = lgQ.to(dt).reshape(P, d)
    x0 = h0.to(dt).reshape(P, d)

    t = torch.arange(1, T + 1, dtype=dt)
    alphas = 1.0 + a[:, None, :] * torch.exp(la[:, None, None] * t[None, :, None])  # [P,T,d]
    betas = torch.exp(lb[:, None, :] * t[None, :, None])                           # [P,T,du]
    nz = T * du
    S = torch.zeros(P, d, nz, dtype=dt)
    f = x0
    Hm = torch.diag_embed((1.0 / r).repeat(1, T))                                  # R blocks
    c = torch.zeros(P, nz, dtype=dt)
    for k in range(T):
        # h_{k+1} = A_k h_k + B_k u_k
        Bk = Bm * betas[:, k, None, :]
        S = alphas[:, k, :, None] * S
        S = torch.cat([S[:, :, : k * du], S[:, :, k * du:(k + 1) * du] + Bk, S[:, :, (k + 1) * du:]], dim=2)
        f = alphas[:, k, :] * f
        if k + 1 < T:
            q = torch.exp(lq * (k + 1))                                             # cost on h_{k+1}
            C = q[:, :, None] * Qm * q[:, None, :]
        else:
            C = Qf
        Cs = 0.5 * (C + C.transpose(1, 2))     # gradient of the quadratic form h'Ch/2
        CS = Cs @ S
        Hm = Hm + S.transpose(1, 2) @ CS
        c = c + (CS.transpose(1, 2) @ f[:, :, None])[:, :, 0]
    Hm = 0.5 * (Hm + Hm.transpose(1, 2))
    L = torch.linalg.cholesky(Hm)
    z = -torch.cholesky_solve(c[:, :, None], L)[:, :, 0]
    return z[:, :du].reshape(N, H, du)
