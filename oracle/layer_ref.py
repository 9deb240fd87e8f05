"""Torch restatement of the ``TTCLayer`` around the solver call (TEST INFRASTRUCTURE ONLY).

Follows ``ttc/layers/ttc_layer.py``:
* parameters and init: ``:56-70`` and ``_init_module`` ``:72-96``;
* front-end producing the nine solver inputs: ``:104-135``;
* back-end: NaN check ``:139-140``, rescale ``:142-147``, ``out_proj`` ``:149-150``.

Deliberate generalisation (documented, not a reference behaviour): ``x`` may
have any number of leading dimensions; they are flattened to tokens, which is
what ``ttc_layer.py:105`` does once the 3-D unpack at ``:104`` is relaxed (the
README's 4-D example input fails in the reference).  ``coeff_Qf`` is sized
``q_rank`` per head (the reference sizes it ``h_dim`` at ``:109`` but contracts it
against ``q_rank`` bases at ``:120``; identical whenever ``q_rank == h_dim``).

``l2norm`` restates fla 0.3.x ``l2norm`` as ``x / sqrt(sum(x^2) + 1e-6)`` over
the last dimension.  fla is not installed here, so this is *parity unpinned*
(it sits outside the solver hot path).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["l2norm", "LayerParams", "make_layer_params", "front_end", "back_end"]


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt((x.float() * x.float()).sum(-1, keepdim=True) + eps).to(x.dtype)


class LayerParams:
    def __init__(self, in_dim, out_dim, h_dim, num_heads, b_rank, q_rank, u_dim=None,
                 q_reparam="plain", rescale="l2_norm", gamma_bias=False):
        self.in_dim, self.out_dim, self.h_dim = in_dim, out_dim, h_dim
        self.num_heads, self.b_rank, self.q_rank = num_heads, b_rank, q_rank
        self.u_dim = h_dim if u_dim is None else u_dim
        self.q_reparam, self.rescale = q_reparam, rescale
        self.gamma_bias = gamma_bias
        self.W_in = self.W_out = self.Bs = self.Qs = self.bias_gamma = None

    @property
    def head_width(self):
        # [h0 | A_diag | R_inv | coeff_Qf | log_gammas(1 + u + h)]
        return self.h_dim + self.h_dim + self.u_dim + self.q_rank + (1 + self.u_dim + self.h_dim)


def make_layer_params(in_dim, out_dim, h_dim, num_heads, b_rank, q_rank, seed=0,
                      u_dim=None, q_reparam="plain", rescale="l2_norm", gamma_bias=False,
                      std=0.02) -> LayerParams:
    """Random-init weights drawn as the reference does (``nn.Linear`` default
    kaiming-uniform for the projections, ``_init_module`` for ``Bs``/``Qs``)."""
    p = LayerParams(in_dim, out_dim, h_dim, num_heads, b_rank, q_rank, u_dim, q_reparam, rescale, gamma_bias)
    g = torch.Generator().manual_seed(seed)
    n_in = p.head_width * num_heads + b_rank + q_rank
    bound_in = 1.0 / math.sqrt(in_dim)
    p.W_in = (torch.rand(n_in, in_dim, generator=g) * 2 - 1) * bound_in
    bound_out = 1.0 / math.sqrt(p.u_dim * num_heads)
    p.W_out = (torch.rand(out_dim, p.u_dim * num_heads, generator=g) * 2 - 1) * bound_out
    p.Bs = torch.randn(b_rank, h_dim, p.u_dim, generator=g) * std
    Qs = torch.randn(q_rank, h_dim, h_dim, generator=g) * std
    if q_reparam == "plain":
        Qs = Qs @ Qs.transpose(1, 2) / math.sqrt(h_dim)
    p.Qs = Qs
    if gamma_bias:
        p.bias_gamma = torch.full((1 + p.u_dim + h_dim,), math.log(1 / math.sqrt(h_dim)))
    return p


def front_end(p: LayerParams, x: torch.Tensor):
    """``x [..., in_dim]`` -> the nine solver inputs (``ttc_layer.py:104-135``) and ``lead`` shape."""
    lead = x.shape[:-1]
    xt = x.reshape(-1, p.in_dim)
    dt = x.dtype
    proj = xt @ p.W_in.to(dt).t()
    H, hd, ud, qr = p.num_heads, p.h_dim, p.u_dim, p.q_rank
    heads, cB, cQ = torch.split(proj, [p.head_width * H, p.b_rank, p.q_rank], dim=-1)
    h0, A_diag, R_inv, cQf, lg = torch.split(heads.reshape(-1, H, p.head_width),
                                             [hd, hd, ud, qr, 1 + ud + hd], dim=-1)
    A_diag = l2norm(A_diag)
    cB, cQ, cQf = l2norm(cB), l2norm(F.softplus(cQ)), l2norm(F.softplus(cQf))
    Bs, Qs = p.Bs.to(dt), p.Qs.to(dt)
    B = torch.einsum("nr,rmk->nmk", cB, Bs)
    if p.q_reparam == "plain":
        Q = torch.einsum("nr,rmk->nmk", cQ, Qs)
        Q_f = torch.einsum("nhr,rmk->nhmk", cQf, Qs)
    else:
        Q = torch.einsum("nr,rmk,rlk->nml", cQ, Qs, Qs) / math.sqrt(hd)
        Q_f = torch.einsum("nhr,rmk,rlk->nhml", cQf, Qs, Qs) / math.sqrt(hd)
    R_inv = torch.clamp(l2norm(F.softplus(R_inv)), min=1e-6)
    if p.bias_gamma is not None:
        lg = -F.softplus(lg) - F.relu(-p.bias_gamma.to(dt)[None, None, :])
    else:
        lg = -F.softplus(lg)
    lgA, lgB, lgQ = torch.split(lg, [1, ud, hd], dim=-1)
    lgA = lgA.squeeze(-1)
    ins = [A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0]
    return [t.contiguous() for t in ins], lead


def back_end(p: LayerParams, u: torch.Tensor, h0: torch.Tensor, lead):
    """``ttc_layer.py:139-150`` (NaN check, rescale, out_proj)."""
    if torch.isnan(u).any():
        raise RuntimeError("NaN detected in TTC layer solver output.")
    if p.rescale == "l2_norm":
        u = l2norm(u)
    elif p.rescale == "h0_norm":
        h0n = torch.linalg.norm(h0, dim=-1).detach()
        un = torch.linalg.norm(u, dim=-1).detach()
        u = u / un[..., None] * h0n[..., None]
    out = u.reshape(*lead, p.u_dim * p.num_heads)
    return out @ p.W_out.to(out.dtype).t()
