"""``fused_lqr_solve`` / ``FusedLQRSolveFunc``: the reference's fused-solver entry points
(``ttc/solvers/fused_lqr.py:255-304``), same names, module path and signatures, backed by the
gfx950 HIP solver of ``libttc_lqr.so``.

``fused_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T, inv_guard=False)``
returns ``u [N,H,du]``.  ``FusedLQRSolveFunc.apply(..., h0, T, cache_level="LU", inv_guard=False)``
is the autograd Function behind it, with the reference's positional slots: its backward returns
the nine input gradients and ``None`` for ``T``, ``cache_level`` and ``inv_guard``.  Both run
:class:`~ttc.solvers.hip_lqr.HipLQRSolveFunc`'s forward and backward with its defaults
(``precision="auto"``, the reference's 1e6 gradient guard).  ``cache_level`` and ``inv_guard``
are accepted and have no effect: in the reference ``cache_level`` picks what the forward keeps
for the backward (this solver keeps its own stash) and ``inv_guard`` selects a ridge on the
symplectic basis ``Y1`` (``symplectic_iter.py:303-305``), but ``fused_lqr_solve`` passes
``inv_guard`` into the ``cache_level`` slot (``fused_lqr.py:268,304``), so it never reaches the
kernel there either; this solver's final solves are pivoted and certified instead.  CUDA tensors
only (the reference's fused solver is GPU-only too).
"""
from __future__ import annotations

import torch

from .hip_lqr import HipLQRSolveFunc

__all__ = ["fused_lqr_solve", "FusedLQRSolveFunc"]


class FusedLQRSolveFunc(torch.autograd.Function):
    """Reference signature (``fused_lqr.py:255-291``) over the HIP solver's autograd Function."""

    @staticmethod
    def forward(ctx, A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T: int, cache_level="LU",
                inv_guard: bool = False):
        return HipLQRSolveFunc.forward(ctx, A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T)

    @staticmethod
    def backward(ctx, d_u):
        grads = HipLQRSolveFunc.backward(ctx, d_u)
        return tuple(grads[:9]) + (None, None, None)


def fused_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T: int, inv_guard: bool = False):
    """First optimal action ``u [N,H,du]`` of every (token, head) problem (reference
    ``fused_lqr_solve``, ``fused_lqr.py:294-304``); ``gamma_*`` are the log-discounts.  As in the
    reference, ``inv_guard`` lands in ``FusedLQRSolveFunc``'s ``cache_level`` slot."""
    return FusedLQRSolveFunc.apply(A_diag, B, Q, R_inv_diag, Q_f, gamma_A, gamma_B, gamma_Q, h0, T, inv_guard)
