"""Op-for-op torch restatement of the reference's pure-PyTorch LQR solvers
(TEST INFRASTRUCTURE ONLY; the CPU baseline of ``bench.py``).

* ``riccati_solve`` restates ``direct_lqr_solve`` (``ttc/solvers/torch_lqr.py:93-118``):
  ``_generate_parameters`` (:65-91) then ``solve_traj_actions`` (``lin_solver_lqr.py:113-212``),
  including the fp32 cast of the gain solve (:175-177), the 4-term value update
  (:184) and no symmetrisation; backward is torch autograd through the sweep.
* ``kkt_solve`` restates ``kkt_lqr_solve`` (``torch_lqr.py:120-140``) with the
  ``KKTLQRSolveFunc`` implicit-differentiation backward (:12-63) and
  ``solve_traj_states`` (``lin_solver_lqr.py:13-110``), including its
  default-dtype scratch allocations.

Deliberately faithful, so both inherit the reference's limits: ``u`` is reshaped
with ``d`` (``torch_lqr.py:118,140``) so ``du == d`` is required, and ``Q``/``Q_f``
are used as given (callers symmetrise, as ``bench_lqr_solvers.py:125,127`` does).

Pinning: against the fp64 oracle (``lqr64``) within fp32 tolerance on nominal
inputs (tests/test_oracle.py); the reference itself is never imported.
"""
from __future__ import annotations

import torch

__all__ = ["generate_parameters", "traj_actions", "traj_states", "riccati_solve", "kkt_solve"]


def _mv(mat, vec):
    return (mat @ vec.unsqueeze(-1)).squeeze(-1)


def _vmv(vec, mat):
    return (vec.unsqueeze(-2) @ mat @ vec.unsqueeze(-1)).squeeze(-1).squeeze(-1)


def generate_parameters(A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, T: int):
    """torch_lqr.py:65-91: per-step discounted system, materialised over T."""
    bs, h, d = A_diag.shape
    du = B.shape[-1]
    steps = (torch.arange(T, device=A_diag.device, dtype=A_diag.dtype) + 1.0)[None, None, :]
    A = A_diag[..., None, :] * torch.exp(lgA[..., None, None] * steps[..., None]) + 1.0
    Bt = B[..., None, None, :, :] * torch.exp(lgB[..., None, None, :] * steps[..., None, None])
    dq = torch.exp(lgQ[..., None, :] * steps[..., :-1, None])
    Qt = dq[..., None, :] * Q[..., None, None, :, :] * dq[..., :, None]
    Qt = torch.cat([Qt, Q_f[..., None, :, :]], dim=-3)
    R = 1.0 / R_inv_diag[..., None, :].expand(*R_inv_diag.shape[:-1], T, du)
    return A, Bt, Qt, R


def traj_actions(A_diag, B, Q, R_diag, h, r_traj=None, return_traj=False):
    """lin_solver_lqr.py:113-212 (Riccati sweep with affine term, optional rollout)."""
    bs, T, ns, nc = B.shape
    dtype = Q.dtype
    A = torch.diag_embed(A_diag)
    R = torch.diag_embed(R_diag)
    F = torch.cat([A, B], dim=-1)
    C = torch.zeros(bs, T, ns + nc, ns + nc, device=h.device, dtype=dtype)
    C[:, 1:, :ns, :ns] = Q[:, :-1]
    C[:, :, ns:, ns:] = R
    c = torch.zeros(bs, T, ns + nc, device=h.device, dtype=dtype)
    if r_traj is not None:
        c[:, :, ns:] = r_traj
    V = Q[:, -1]
    v = torch.zeros(bs, ns, device=h.device, dtype=dtype)
    Ks = torch.zeros(bs, T, nc, ns, device=h.device, dtype=dtype)
    ks = torch.zeros(bs, T, nc, device=h.device, dtype=dtype)
    for t in range(T - 1, -1, -1):
        Ft = F[:, t]
        FtT = Ft.transpose(-1, -2)
        Qa = C[:, t] + FtT @ V @ Ft
        qa = c[:, t] + _mv(FtT, v)
        Qxx, Qxu = Qa[:, :ns, :ns], Qa[:, :ns, ns:]
        Qux, Quu = Qa[:, ns:, :ns], Qa[:, ns:, ns:]
        qx, qu = qa[:, :ns], qa[:, ns:]
        Quu32 = Quu.to(torch.float32)
        Kt = -torch.linalg.solve(Quu32, Qux.to(torch.float32)).to(dtype)
        kt = -torch.linalg.solve(Quu32, qu.unsqueeze(-1).to(torch.float32)).squeeze(-1).to(dtype)
        Ks[:, t] = Kt
        ks[:, t] = kt
        KtT = Kt.transpose(-1, -2)
        V = Qxx + Qxu @ Kt + KtT @ Qux + KtT @ Quu @ Kt
        v = qx + _mv(Qxu, kt) + _mv(KtT, qu) + _mv(KtT @ Quu, kt)
    if return_traj:
        u = torch.zeros(bs, T, nc, device=h.device, dtype=dtype)
        x = h
        for t in range(T):
            ut = _mv(Ks[:, t], x) + ks[:, t]
            u[:, t] = ut
            if t < T - 1:
                x = _mv(A[:, t], x) + _mv(B[:, t], ut)
        return u
    return _mv(Ks[:, 0], h) + ks[:, 0]


def traj_states(u_traj, A_diag, B, Q, R_diag, h, r_traj=None):
    """lin_solver_lqr.py:13-110 with return_states/costates/lambda0."""
    bs, T, d = A_diag.shape
    du = B.shape[-1]
    dev = A_diag.device
    if r_traj is None:
        r_traj = torch.zeros(bs, T, du, device=dev)
    if h is None:
        h = torch.zeros(bs, d, device=dev)
    A = torch.diag_embed(A_diag)
    R = torch.diag_embed(R_diag)
    states = torch.zeros(bs, T, d, device=dev)
    cost = torch.zeros(bs, device=dev)
    x = h
    for t in range(T):
        ut = u_traj[:, t, :]
        x = _mv(A[:, t], x) + _mv(B[:, t], ut)
        cost = cost + 0.5 * _vmv(x, Q[:, t]) + 0.5 * _vmv(ut, R[:, t]) + torch.sum(ut * r_traj[:, t], dim=-1)
        states[:, t, :] = x
    lam = torch.zeros(bs, T, d, device=dev)
    lam[:, T - 1, :] = _mv(Q[:, T - 1], states[:, T - 1])
    for t in range(T - 2, -1, -1):
        lam[:, t, :] = _mv(Q[:, t], states[:, t]) + _mv(A[:, t + 1].transpose(-1, -2), lam[:, t + 1])
    lam0 = _mv(A[:, 0].transpose(-1, -2), lam[:, 0, :])
    return cost, states, lam, lam0


def riccati_solve(A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, h0, T: int):
    """``direct_lqr_solve`` (torch_lqr.py:93-118)."""
    bs, h, d = A_diag.shape
    du = B.shape[-1]
    A, Bt, Qt, R = generate_parameters(A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, T)
    u = traj_actions(A.reshape(-1, T, d), Bt.reshape(-1, T, d, du), Qt.reshape(-1, T, d, d),
                     R.reshape(-1, T, du), h0.reshape(-1, d))
    return u.reshape(bs, h, d)


class _KKTFunc(torch.autograd.Function):
    """KKTLQRSolveFunc (torch_lqr.py:12-63)."""

    @staticmethod
    def forward(ctx, A_diag, B, Q, R_diag, h0):
        bs, T, d = A_diag.shape
        u = traj_actions(A_diag, B, Q, R_diag, h0)
        ctx.save_for_backward(h0, A_diag, B, Q, R_diag)
        ctx.T = T
        return u

    @staticmethod
    def backward(ctx, d_u):
        h0, A_diag, B, Q, R_diag = ctx.saved_tensors
        T = ctx.T
        bs, _, d = A_diag.shape
        du = B.shape[-1]
        r_g = torch.zeros(bs, T, du, device=d_u.device)
        r_g[:, 0, :] = d_u
        u_f = traj_actions(A_diag, B, Q, R_diag, h0, return_traj=True)
        u_b = traj_actions(A_diag, B, Q, R_diag, torch.zeros_like(h0), r_traj=r_g, return_traj=True)
        _, hs_f, lam_f, _ = traj_states(u_f, A_diag, B, Q, R_diag, h0)
        _, hs_b, lam_b, lam0_b = traj_states(u_b, A_diag, B, Q, R_diag, None, r_traj=r_g)
        hs_f_sh = torch.cat((h0[:, None, :], hs_f[:, :-1, :]), dim=1)
        hs_b_sh = torch.cat((torch.zeros_like(h0[:, None, :]), hs_b[:, :-1, :]), dim=1)
        gA = hs_f_sh * lam_b + hs_b_sh * lam_f
        gB = lam_b[..., None] * u_f[..., None, :] + lam_f[..., None] * u_b[..., None, :]
        gQ = (hs_b[..., :, None] * hs_f[..., None, :] + hs_f[..., :, None] * hs_b[..., None, :]) / 2.0
        gR = u_f * u_b
        return gA, gB, gQ, gR, lam0_b


def kkt_solve(A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, h0, T: int):
    """``kkt_lqr_solve`` (torch_lqr.py:120-140)."""
    bs, h, d = A_diag.shape
    du = B.shape[-1]
    A, Bt, Qt, R = generate_parameters(A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, T)
    u = _KKTFunc.apply(A.reshape(-1, T, d), Bt.reshape(-1, T, d, du), Qt.reshape(-1, T, d, d),
                       R.reshape(-1, T, du), h0.reshape(-1, d))
    return u.reshape(bs, h, d)
