"""Seeded synthetic inputs (TEST INFRASTRUCTURE ONLY).

* ``CONFIGS``: the five BASELINE configurations (layer shape, ``x`` shape,
  storage dtype, input scaling).
* ``make_x``: seeded ``x`` for a config, optionally only ``n_tokens`` tokens
  (a parity slice draws its own tokens from the same distribution; it is not
  a literal prefix of the full tensor).
* ``layer_solver_inputs``: random-init layer weights (``layer_ref``) applied
  to ``x`` -> the nine solver inputs.
* ``bench_solver_inputs``: the reference's solver-level distribution,
  restating ``ttc/solvers/bench_lqr_solvers.py:71-101`` (seed 0) and the
  ``Q``/``Q_f`` symmetrisation done by ``run_solver_with_backward`` (:125,127).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .layer_ref import make_layer_params, front_end

__all__ = ["CONFIGS", "make_x", "layer_solver_inputs", "bench_solver_inputs", "layer_for"]

CONFIGS = {
    1: dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=64,
            x_shape=(2, 128, 8, 32), dtype=torch.float32, scale=1.0, lognormal=None),
    2: dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=64,
            x_shape=(16, 2048, 8, 32), dtype=torch.float32, scale=1.0, lognormal=None),
    3: dict(in_dim=64, out_dim=64, h_dim=64, num_heads=16, b_rank=32, q_rank=32, T=128,
            x_shape=(8, 4096, 16, 64), dtype=torch.float32, scale=1.0, lognormal=None),
    4: dict(in_dim=64, out_dim=64, h_dim=32, num_heads=32, b_rank=32, q_rank=32, T=256,
            x_shape=(4, 8192, 32, 64), dtype=torch.bfloat16, scale=0.02, lognormal=None),
    5: dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=1024,
            x_shape=(256, 1, 8, 32), dtype=torch.float32, scale=1.0, lognormal=1.5),
    "5b": dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=1024,
               x_shape=(4, 1024, 8, 32), dtype=torch.float32, scale=1.0, lognormal=1.5),
}


def make_x(cfg, n_tokens=None, seed=0, device="cpu"):
    c = CONFIGS[cfg] if not isinstance(cfg, dict) else cfg
    shape = c["x_shape"] if n_tokens is None else (n_tokens, c["in_dim"])
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * c["scale"]
    if c["lognormal"] is not None:
        tok = x.shape[:-1]
        s = torch.exp(c["lognormal"] * torch.randn(tok, generator=g, device=device))
        x = x * s[..., None]
    return x.to(c["dtype"])


def layer_for(cfg, seed=0):
    c = CONFIGS[cfg] if not isinstance(cfg, dict) else cfg
    return make_layer_params(c["in_dim"], c["out_dim"], c["h_dim"], c["num_heads"], c["b_rank"],
                             c["q_rank"], seed=seed)


def layer_solver_inputs(cfg, x, seed=0):
    """Nine solver inputs (fp32) for ``x`` through a seeded random-init layer front-end."""
    p = layer_for(cfg, seed)
    ins, lead = front_end(p, x.float())
    return ins


def bench_solver_inputs(batch_size, num_heads, dim, seed=0, dtype=torch.float32):
    """``bench_lqr_solvers.generate_inputs`` (:71-101) on a CPU generator, with Q, Q_f
    symmetrised as ``run_solver_with_backward`` does (:125,127)."""
    g = torch.Generator().manual_seed(seed)

    def normalize(x):
        if x.ndim == 3:
            return x / torch.linalg.norm(x, dim=-1, ord=2, keepdim=True)
        return x / torch.linalg.norm(x, dim=(-2, -1), ord="fro", keepdim=True)

    A = normalize(torch.rand(batch_size, num_heads, dim, generator=g))
    B = torch.randn(batch_size, dim, dim, generator=g)
    Q = normalize(torch.randn(batch_size, dim, dim, generator=g))
    Q = Q @ Q.transpose(-1, -2) / math.sqrt(dim)
    Q_f = normalize(torch.randn(batch_size, num_heads, dim, dim, generator=g))
    Q_f = Q_f @ Q_f.transpose(-1, -2) / math.sqrt(dim)
    R_inv = F.softplus(torch.rand(batch_size, num_heads, dim, generator=g))
    h0 = torch.randn(batch_size, num_heads, dim, generator=g)
    lgA = -F.softplus(torch.randn(batch_size, num_heads, generator=g)) - 1.328
    lgB = -F.softplus(torch.randn(batch_size, num_heads, dim, generator=g)) - 1.328
    lgQ = -F.softplus(torch.randn(batch_size, num_heads, dim, generator=g)) - 1.328
    Q = (Q + Q.transpose(-1, -2)) / 2
    Q_f = (Q_f + Q_f.transpose(-1, -2)) / 2
    return [t.to(dtype) for t in (A, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0)]
