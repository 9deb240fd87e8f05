"""``TTCLayer``: the Test-Time Control layer, mirroring ``ttc/layers/ttc_layer.py``.

Same constructor arguments and semantics as the reference
(``ttc_layer.py:25-70``, init ``:72-96``, forward ``:98-153``); the solver call
at ``:137`` dispatches through ``LQR_SOLVER_IMPL_MAP`` (``:18-22``), which here
holds the gfx950 HIP solver under ``"hip"`` and the reference's keys ``"fused"`` (the same
HIP solver), ``"riccati"`` and ``"kkt"`` (HIP kernels on CUDA tensors, the library's native
host solver on CPU tensors, so the layer runs without a GPU).  The front-end (projections, ``l2norm``, softplus and
the low-rank ``B``/``Q``/``Q_f`` mixtures) and the back-end (rescale, ``out_proj``)
are ordinary torch ops around that call.

With ``factored=True`` (the default wherever the solver has a factored form,
``LQR_FACTORED_IMPL_MAP``) the layer hands the solver the mixture coefficients and
bases instead of ``B``, ``Q`` and ``Q_f``: the library expands them per token chunk on
the device, so the ``[N, H, h, h]`` ``Q_f`` (and its gradient) is never formed in full
-- 137 GB at h_dim = 64 with 8.4 M problems.  On that path the rescale of ``u``
(``ttc_layer.py:142-147``) runs fused into the solver call (fp32), and the NaN check of
``:139`` is the solver's device status word instead of a separate reduction and host
sync.  Same values and gradients up to fp32 rounding; ``factored=False`` runs the
reference's materialised formulation and back-end.

Generalisations over the reference (each keeps the reference result whenever
the reference runs at all):
* ``x`` may have any number of leading dims (flattened to tokens); the README's
  ``[batch, seq, heads, in_dim]`` example fails the reference's 3-D unpack.
* ``coeff_Qf`` has ``q_rank`` entries per head (the reference sizes it ``h_dim``
  but contracts it with ``q_rank`` bases, so it only works when they agree).

``l2norm`` is ``x / sqrt(sum(x^2) + 1e-6)`` over the last dim, restating
fla 0.3.x's ``l2norm`` (fla itself is not a dependency).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..solvers.fused_lqr import fused_lqr_solve
from ..solvers.hip_lqr import hip_lqr_solve, hip_lqr_solve_factored
from ..solvers.torch_lqr import direct_lqr_solve, kkt_lqr_solve

__all__ = ["TTCLayer", "LQR_SOLVER_IMPL_MAP", "LQR_FACTORED_IMPL_MAP", "l2norm"]

# the reference's keys (ttc_layer.py:18-22) plus "hip"; "riccati" / "kkt" run on CPU tensors too
LQR_SOLVER_IMPL_MAP = {
    "riccati": direct_lqr_solve,
    "kkt": kkt_lqr_solve,
    "fused": fused_lqr_solve,
    "hip": hip_lqr_solve,
}

# solvers that can take (coeff_B, coeff_Q, coeff_Qf, B_basis, Q_basis) in place of B, Q, Q_f
LQR_FACTORED_IMPL_MAP = {
    "hip": hip_lqr_solve_factored,
    "fused": hip_lqr_solve_factored,
}


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)).to(x.dtype)


class TTCLayer(nn.Module):
    def __init__(self, in_dim: int, out_dim: int, h_dim: int, num_heads: int,
                 b_rank: int, q_rank: int, u_dim: int = None,
                 bias: bool = False, gamma_bias: bool = False, gamma_bias_init: str = "sqrt_dim",
                 rescale: str = "l2_norm", q_reparam: str = "plain", solver_impl: str = "hip",
                 factored: bool | None = None):
        super().__init__()
        if u_dim is None:
            u_dim = h_dim
        assert solver_impl in LQR_SOLVER_IMPL_MAP, f"Unknown LQR solver {solver_impl}"
        self.solver = LQR_SOLVER_IMPL_MAP[solver_impl]
        if factored is None:
            factored = solver_impl in LQR_FACTORED_IMPL_MAP
        assert not factored or solver_impl in LQR_FACTORED_IMPL_MAP, f"{solver_impl} has no factored form"
        self.factored = bool(factored)
        self.solver_factored = LQR_FACTORED_IMPL_MAP.get(solver_impl)
        assert rescale in ["none", "l2_norm", "h0_norm"], f"Unknown rescale method {rescale}"
        self.rescale = rescale
        assert q_reparam in ["plain", "cholesky"], f"Unknown Q reparameterization {q_reparam}"
        self.q_reparam = q_reparam
        self.in_dim, self.out_dim = in_dim, out_dim
        self.num_heads, self.h_dim, self.u_dim = num_heads, h_dim, u_dim
        self.q_rank, self.b_rank = q_rank, b_rank

        # per head: h0 | A_diag | R_inv | coeff_Qf | log_gammas (1 + u + h); shared: coeff_B | coeff_Q
        self._head_split = [h_dim, h_dim, u_dim, q_rank, 1 + u_dim + h_dim]
        self.in_proj = nn.Linear(in_dim, sum(self._head_split) * num_heads + b_rank + q_rank, bias=bias)
        self.out_proj = nn.Linear(u_dim * num_heads, out_dim, bias=bias)
        self.Bs = nn.Parameter(torch.empty(b_rank, h_dim, u_dim))
        self.Qs = nn.Parameter(torch.empty(q_rank, h_dim, h_dim))
        assert gamma_bias_init in ["sqrt_dim", "zero"], f"Unknown gamma bias initialization {gamma_bias_init}"
        self.ttc_gamma_bias_init = gamma_bias_init
        self.bias_gamma = None
        if gamma_bias:
            self.bias_gamma = nn.Parameter(torch.empty(1 + u_dim + h_dim, dtype=torch.float32))
        TTCLayer._init_module(self)

    @staticmethod
    def _init_module(module, std=0.02):
        with torch.no_grad():
            module.Bs.data.normal_(mean=0.0, std=std)
            if module.q_reparam == "plain":
                # start PSD: Qs Qs^T / sqrt(h_dim)  (ttc_layer.py:79-83)
                Qs = torch.empty_like(module.Qs).normal_(mean=0.0, std=std)
                module.Qs.data.copy_(Qs @ Qs.transpose(1, 2) / math.sqrt(module.h_dim))
            else:
                module.Qs.data.normal_(mean=0.0, std=std)
            if module.bias_gamma is not None:
                fill = math.log(1 / math.sqrt(module.h_dim)) if module.ttc_gamma_bias_init == "sqrt_dim" else 0.0
                module.bias_gamma.data.fill_(fill)

    def _front_end(self, x: torch.Tensor):
        """Projections, normalisations and discounts (``ttc_layer.py:104-135``) up to the
        low-rank mixtures: per-token coefficients, the bases they mix, the per-head inputs."""
        H, hd, ud, qr = self.num_heads, self.h_dim, self.u_dim, self.q_rank
        xt = x.reshape(-1, self.in_dim)
        heads, coeff_B, coeff_Q = torch.split(self.in_proj(xt), [sum(self._head_split) * H, self.b_rank, qr], dim=-1)
        h0, A_diag, R_inv_diag, coeff_Qf, log_gammas = torch.split(
            heads.reshape(-1, H, sum(self._head_split)), self._head_split, dim=-1)
        A_diag = l2norm(A_diag)
        coeff_B, coeff_Q, coeff_Qf = l2norm(coeff_B), l2norm(F.softplus(coeff_Q)), l2norm(F.softplus(coeff_Qf))
        if self.q_reparam == "plain":
            Q_basis = self.Qs
        else:  # "...r,rmn,rkn->...mk" / sqrt(h_dim) = sum_r coeff_r (Qs_r Qs_r') / sqrt(h_dim)
            Q_basis = torch.matmul(self.Qs, self.Qs.transpose(1, 2)) / math.sqrt(hd)
        R_inv_diag = torch.clamp(l2norm(F.softplus(R_inv_diag)), min=1e-6)
        if self.bias_gamma is not None:
            log_gammas = -F.softplus(log_gammas) - F.relu(-self.bias_gamma[None, None, :])
        else:
            log_gammas = -F.softplus(log_gammas)
        lgA, lgB, lgQ = torch.split(log_gammas, [1, ud, hd], dim=-1)
        return A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, lgA.squeeze(-1), lgB, lgQ, h0, Q_basis

    def solver_inputs(self, x: torch.Tensor):
        """Front-end (``ttc_layer.py:104-135``): ``x [..., in_dim]`` -> the nine solver inputs."""
        A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, lgA, lgB, lgQ, h0, _ = self._front_end(x)
        B = torch.einsum("...r,rmn->...mn", coeff_B, self.Bs)
        if self.q_reparam == "plain":
            Q = torch.einsum("...r,rmn->...mn", coeff_Q, self.Qs)
            Q_f = torch.einsum("...r,rmn->...mn", coeff_Qf, self.Qs)
        else:
            Q = torch.einsum("...r,rmn,rkn->...mk", coeff_Q, self.Qs, self.Qs) / math.sqrt(self.h_dim)
            Q_f = torch.einsum("...r,rmn,rkn->...mk", coeff_Qf, self.Qs, self.Qs) / math.sqrt(self.h_dim)
        return A_diag, B, Q, R_inv_diag, Q_f, lgA, lgB, lgQ, h0

    def factored_inputs(self, x: torch.Tensor):
        """The eleven inputs of the factored solver: ``(A_diag, coeff_B, coeff_Q, R_inv, coeff_Qf,
        lgA, lgB, lgQ, h0, B_basis, Q_basis)``."""
        A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, lgA, lgB, lgQ, h0, Q_basis = self._front_end(x)
        return A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, lgA, lgB, lgQ, h0, self.Bs, Q_basis

    def forward(self, h0: torch.Tensor, T: int):
        lead = h0.shape[:-1]
        if T == 0:
            # horizon zero disables the layer (ttc_layer.py:101-102)
            return torch.zeros(*lead, self.out_dim, device=h0.device, dtype=h0.dtype)
        rescaled = False
        if self.factored:
            ins = self.factored_inputs(h0)
            x0 = ins[8]
            # fp32: the rescale runs fused into the solver call; the solver's device status word
            # already raises on a non-finite u, so no separate NaN reduction / host sync
            rescaled = self.rescale != "none" and all(t.dtype == torch.float32 for t in ins)
            u = self.solver_factored(*ins, T, rescale=self.rescale if rescaled else "none")
        else:
            A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, x0 = self.solver_inputs(h0)
            u = self.solver(A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, x0, T)
            if torch.isnan(u).any():
                raise RuntimeError("NaN detected in TTC layer solver output.")
        if not rescaled and self.rescale == "l2_norm":
            u = l2norm(u)
        elif not rescaled and self.rescale == "h0_norm":
            h0_norm = torch.linalg.norm(x0, dim=-1, ord=2).detach()
            u_norm = torch.linalg.norm(u, dim=-1, ord=2).detach()
            u = u / u_norm[..., None] * h0_norm[..., None]
        out = u.reshape(*lead, self.u_dim * self.num_heads)
        return self.out_proj(out)
