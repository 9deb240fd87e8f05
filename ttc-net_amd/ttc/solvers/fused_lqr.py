"""``fused_lqr_solve``: the reference's fused-solver entry point (``ttc/solvers/fused_lqr.py:294-304``),
same name, module path and signature, backed by the gfx950 HIP solver of ``libttc_lqr.so``.

``fused_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T, inv_guard=False)``
returns ``u [N,H,du]``; ``FusedLQRSolveFunc`` is the autograd Function behind it
(:class:`~ttc.solvers.hip_lqr.HipLQRSolveFunc`).  ``inv_guard`` is accepted and has no effect:
in the reference it selects a ridge on the symplectic basis ``Y1`` (``symplectic_iter.py:303-305``)
but ``fused_lqr_solve`` passes it into ``FusedLQRSolveFunc``'s ``cache_level`` slot
(``fused_lqr.py:268,304``), so it never reaches the kernel there either; this solver's final
solves are pivoted and certified instead.  CUDA tensors only (the reference's fused solver is
GPU-only too).
"""
from __future__ import annotations

from .hip_lqr import HipLQRSolveFunc, hip_lqr_solve

__all__ = ["fused_lqr_solve", "FusedLQRSolveFunc"]

FusedLQRSolveFunc = HipLQRSolveFunc


def fused_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T: int, inv_guard: bool = False):
    """First optimal action ``u [N,H,du]`` of every (token, head) problem (reference
    ``fused_lqr_solve``, ``fused_lqr.py:294-304``); ``gamma_*`` are the log-discounts."""
    return hip_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T, inv_guard)
