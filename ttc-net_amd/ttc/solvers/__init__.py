"""LQR solvers.  ``hip_lqr_solve`` is the gfx950 HIP solver (``solver_impl="hip"``);
``fused_lqr_solve`` is kept as an alias so code written against the reference's
default ``solver_impl="fused"`` (``ttc/solvers/fused_lqr.py:294``) runs unchanged.
``hip_lqr_solve_factored`` takes the layer's low-rank factors instead of ``B``, ``Q``, ``Q_f``."""
from .hip_lqr import hip_lqr_solve, HipLQRSolveFunc, hip_lqr_solve_factored, HipLQRFactoredFunc

fused_lqr_solve = hip_lqr_solve

__all__ = ["hip_lqr_solve", "fused_lqr_solve", "HipLQRSolveFunc", "hip_lqr_solve_factored", "HipLQRFactoredFunc"]
