"""Test helper: parameter gradients of a ``TTCLayer`` by fp64 autograd of the oracle layer
restatement (``oracle/layer_ref.py``) around the fp64 oracle solve (``oracle/lqr64.py``), whose
nine solver-input gradients enter through a custom autograd Function.  Test infrastructure only."""
from __future__ import annotations

import torch

from oracle.layer_ref import LayerParams, back_end, front_end
from oracle.lqr64 import LQRProblem, solve_grads, solve_u0

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]


class _OracleSolve(torch.autograd.Function):

    @staticmethod
    def forward(ctx, A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0, T):
        ins = [A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0]
        ctx.save_for_backward(*ins)
        ctx.T = T
        return torch.from_numpy(solve_u0(LQRProblem(*[t.detach() for t in ins], T)))

    @staticmethod
    def backward(ctx, d_u):
        g = solve_grads(LQRProblem(*ctx.saved_tensors, ctx.T), d_u.detach().numpy())
        return tuple(torch.from_numpy(g[n]) for n in NAMES) + (None,)


def oracle_layer_grads(layer, x: torch.Tensor, dy: torch.Tensor, T: int) -> dict:
    """Gradients of sum(dy * layer(x, T)) w.r.t. in_proj / out_proj weights, Bs and Qs, in fp64
    (bias-free layer with q_reparam="plain", rescale="l2_norm", no gamma bias)."""
    p = LayerParams(layer.in_dim, layer.out_dim, layer.h_dim, layer.num_heads, layer.b_rank, layer.q_rank,
                    u_dim=layer.u_dim, q_reparam=layer.q_reparam, rescale=layer.rescale)
    leaves = {
        "in_proj": layer.in_proj.weight.detach().cpu().double().requires_grad_(True),
        "out_proj": layer.out_proj.weight.detach().cpu().double().requires_grad_(True),
        "Bs": layer.Bs.detach().cpu().double().requires_grad_(True),
        "Qs": layer.Qs.detach().cpu().double().requires_grad_(True),
    }
    p.W_in, p.W_out, p.Bs, p.Qs = leaves["in_proj"], leaves["out_proj"], leaves["Bs"], leaves["Qs"]
    ins, lead = front_end(p, x.detach().cpu().double())
    u = _OracleSolve.apply(*ins, T)
    y = back_end(p, u, ins[8], lead)
    (y * dy.detach().cpu().double()).sum().backward()
    return {k: v.grad.numpy() for k, v in leaves.items()}
