"""Host (CPU) LQR solver: the autograd Function behind ``direct_lqr_solve`` / ``kkt_lqr_solve``
for CPU tensors.

The reference's ``riccati`` and ``kkt`` solvers (``ttc/solvers/torch_lqr.py:93-140``) are plain
PyTorch and run on any device; ``TTCLayer(..., solver_impl="riccati")`` on the CPU is the
reference's config-1 use.  Here the CPU case runs in the native host code of ``libttc_lqr.so``
(``ttc_lqr_forward_host`` / ``ttc_lqr_backward_host``, ``include/ttc_lqr.h``): the Riccati sweep
with pivoted gain solves and the KKT implicit-differentiation backward, in fp64 arithmetic.
This module only validates, allocates and checks the status word; it never sees CUDA tensors.

Same inputs, shapes, outputs and errors as :func:`ttc.solvers.hip_lqr.hip_lqr_solve`:
``u [N,H,du]`` in the input dtype, gradients for all nine tensors (``grad_B`` / ``grad_Q``
summed over heads, the symmetric gradient for ``Q`` / ``Q_f``), ``RuntimeError`` with the
reference's messages on non-finite results or gradients at or above ``grad_limit``.
"""
from __future__ import annotations

import math

import torch

from ._lib import lib, check

__all__ = ["HostLQRSolveFunc", "host_lqr_solve"]

_FWD_MSG = "Numerical instability detected during fused LQR forward recurrence."
_BWD_MSG = "Numerical instability detected during fused LQR backward pass."


def _check_shapes(A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T):
    bs, nh, d = A_diag.shape
    du = B.shape[-1]
    assert int(T) > 0
    assert B.shape == (bs, d, du) and Q.shape == (bs, d, d)
    assert R_inv_diag.shape == (bs, nh, du) and Q_f.shape == (bs, nh, d, d)
    assert log_gamma_A.shape == (bs, nh) and log_gamma_B.shape == (bs, nh, du)
    assert log_gamma_Q.shape == (bs, nh, d) and h0.shape == (bs, nh, d)
    return bs, nh, d, du


class HostLQRSolveFunc(torch.autograd.Function):

    @staticmethod
    def forward(ctx, A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T: int,
                grad_limit: float = 1e6):
        ins = [A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0]
        assert all(x.device.type == "cpu" for x in ins), "the host LQR solver takes CPU tensors"
        bs, nh, d, du = _check_shapes(*ins, T)
        T = int(T)
        f32 = [x.detach().to(torch.float32).contiguous() for x in ins]
        u = torch.empty(bs, nh, du, dtype=torch.float32)
        status = torch.zeros(1, dtype=torch.int32)
        rc = lib.ttc_lqr_forward_host(*[t.data_ptr() for t in f32], bs, nh, d, du, T, u.data_ptr(),
                                      status.data_ptr(), torch.get_num_threads())
        check(rc, "ttc_lqr_forward_host")
        if int(status.item()) & 3:
            raise RuntimeError(_FWD_MSG)
        if any(ctx.needs_input_grad[:9]):
            ctx.save_for_backward(*f32)
        ctx.meta = (bs, nh, d, du, T, float(grad_limit), [x.dtype for x in ins])
        return u.to(Q.dtype)

    @staticmethod
    def backward(ctx, d_u):
        bs, nh, d, du, T, grad_limit, dtypes = ctx.meta
        f32 = list(ctx.saved_tensors)
        dU = d_u.detach().to(torch.float32).contiguous()
        shapes = [(bs, nh, d), (bs, d, du), (bs, d, d), (bs, nh, du), (bs, nh, d, d), (bs, nh), (bs, nh, du),
                  (bs, nh, d), (bs, nh, d)]
        g = [torch.empty(s, dtype=torch.float32) for s in shapes]
        status = torch.zeros(1, dtype=torch.int32)
        limit = grad_limit if math.isfinite(grad_limit) else float("inf")
        rc = lib.ttc_lqr_backward_host(*[t.data_ptr() for t in f32], dU.data_ptr(), bs, nh, d, du, T,
                                       *[t.data_ptr() for t in g], limit, status.data_ptr(), torch.get_num_threads())
        check(rc, "ttc_lqr_backward_host")
        if int(status.item()) & 3:
            raise RuntimeError(_BWD_MSG)
        out = tuple(o.to(dt) if need else None for o, dt, need in zip(g, dtypes, ctx.needs_input_grad[:9]))
        return out + (None, None)


def host_lqr_solve(A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T: int,
                   grad_limit: float = 1e6) -> torch.Tensor:
    """First optimal action ``u [N,H,du]`` of every problem, computed on the host CPU."""
    return HostLQRSolveFunc.apply(A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T,
                                  grad_limit)
