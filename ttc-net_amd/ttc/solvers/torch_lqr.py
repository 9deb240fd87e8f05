"""``direct_lqr_solve`` (``riccati``) and ``kkt_lqr_solve`` (``kkt``): the reference's
device-agnostic solvers (``ttc/solvers/torch_lqr.py:93-140``), same names, signatures and
module path, so ``from ttc.solvers.torch_lqr import direct_lqr_solve, kkt_lqr_solve`` and
``TTCLayer(..., solver_impl="riccati" | "kkt")`` work unchanged.

Both take the nine solver inputs and ``T`` and return ``u [N,H,du]`` in the input dtype,
differentiable in all nine inputs.  They dispatch on the device of the inputs:

* CUDA tensors run the gfx950 kernels of ``libttc_lqr.so`` (:func:`~ttc.solvers.hip_lqr.hip_lqr_solve`):
  ``direct_lqr_solve`` with a Riccati step at every horizon step on the matrix cores (fp64
  sweep for ``T >= 512``), as the reference's ``riccati`` sweeps Riccati steps; ``kkt_lqr_solve``
  likewise, with the backward taken by the implicit-differentiation path for every problem
  (per-step gains, closed-loop rollouts and costates), the structure of the reference's
  ``KKTLQRSolveFunc`` (``torch_lqr.py:12-63``);
* CPU tensors run the native host solver of the same library
  (:class:`~ttc.solvers.host_lqr.HostLQRSolveFunc`: fp64 Riccati sweep, KKT backward).

Differences from the reference, by design: ``u`` has ``du`` entries (the reference reshapes
it with ``d``, ``torch_lqr.py:118,140``, so it requires ``du == d``); ``Q`` / ``Q_f`` enter
through their symmetric parts and their gradients are the symmetric gradients (the
reference's ``riccati`` autograd returns a non-symmetric one for the same QP); the backward
raises ``RuntimeError`` on non-finite gradients, or gradients at or above ``1e6``, of
``A_diag``, ``B``, ``Q``, ``R_inv``, ``Q_f``, ``h0`` (the guard of ``fused_lqr.py:243-246``).
"""
from __future__ import annotations

import torch

from .host_lqr import host_lqr_solve

__all__ = ["direct_lqr_solve", "kkt_lqr_solve"]


def _solve(ins, T, stable_backward):
    if all(t.is_cuda for t in ins):
        from .hip_lqr import hip_lqr_solve
        return hip_lqr_solve(*ins, T, precision="riccati", stable_backward=stable_backward)
    assert all(t.device.type == "cpu" for t in ins), "LQR solver inputs must all be on the CPU or all on a GPU"
    return host_lqr_solve(*ins, T)


def direct_lqr_solve(A_diag: torch.Tensor, B: torch.Tensor, Q: torch.Tensor, R_inv_diag: torch.Tensor,
                     Q_f: torch.Tensor, log_gamma_A: torch.Tensor, log_gamma_B: torch.Tensor,
                     log_gamma_Q: torch.Tensor, h0: torch.Tensor, T: int) -> torch.Tensor:
    """The ``riccati`` solver (reference ``direct_lqr_solve``, ``torch_lqr.py:93-118``)."""
    return _solve([A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0], T, False)


def kkt_lqr_solve(A_diag: torch.Tensor, B: torch.Tensor, Q: torch.Tensor, R_inv_diag: torch.Tensor,
                  Q_f: torch.Tensor, log_gamma_A: torch.Tensor, log_gamma_B: torch.Tensor,
                  log_gamma_Q: torch.Tensor, h0: torch.Tensor, T: int) -> torch.Tensor:
    """The ``kkt`` solver (reference ``kkt_lqr_solve``, ``torch_lqr.py:120-140``)."""
    return _solve([A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0], T, True)
