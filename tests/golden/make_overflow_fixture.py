"""Generate tests/golden/oracle_cfg5b_undiscounted.npz (run from the repo root).

Four tokens (32 problems, d = 16, T = 1024) of bench config 5b -- the BASELINE
numerical-stress case, log-normal token scales -- whose open-loop states grow almost
undiscounted (log_gamma_A ~ -3e-5, 1 + A_diag up to 1.73) while control is expensive
(R_inv down to 1e-6).  Their closed-loop rollouts leave the fp32 range before the
horizon ends, yet every gradient is small (fp64 oracle: |grad| <= 152), so a solver
that rolls them out in fp32 returns inf / NaN where the answer is finite.

Inputs come from ``bench.layer_workload("5b", seed=0)`` on the GPU (the workload is
drawn on the device; tokens 1151, 3182, 5268, 8689 are the first four whose
gradients were non-finite before the stable backward ran in fp64), or from a file of
captured inputs (``--inputs``: a torch file with ``ins`` = the nine solver inputs of
those tokens and ``du``).  Expected outputs: the fp64 oracle (oracle/lqr64.py).

The gains of these problems reach |K| ~ 4e19, and the gradients of A_diag and B (and,
less so, of log_gamma_A / log_gamma_B) are ill-conditioned: perturbing the inputs by
a relative 1e-12 moves the oracle's own A_diag gradient by 6e-3 and its B gradient by
9e-2 (relative to their maxima), lgA / lgB by 1.5e-6 / 1.2e-5.  fp32 inputs cannot
pin those to 1e-4, so the fixture carries per-output tolerances (``tol_<name>``; inf =
finite only): 1e-4 for u, Q, R_inv, Q_f, lgQ, h0; 1e-2 for lgA / lgB; finiteness for
A_diag and B.

Usage: python tests/golden/make_overflow_fixture.py [--inputs captured.pt]
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
TOKENS = [1151, 3182, 5268, 8689]
T = 1024


def capture():
    import torch
    import bench
    ins, d_u, _ = bench.layer_workload("5b", 0, torch.device("cuda:0"))
    idx = torch.tensor(TOKENS, device=d_u.device)
    return [t[idx].cpu() for t in ins], d_u[idx].cpu()


def main():
    import torch
    from oracle.lqr64 import LQRProblem, solve_grads
    ap = argparse.ArgumentParser()
    ap.add_argument("--inputs", default=None)
    a = ap.parse_args()
    if a.inputs:
        z = torch.load(a.inputs, weights_only=True)
        ins, du = z["ins"], z["du"]
    else:
        ins, du = capture()
    ins = [t.float() for t in ins]
    dU = du.double().numpy()
    ref = solve_grads(LQRProblem(*[t.double() for t in ins], T), dU)
    out = {f"out_{k}": np.asarray(ref[k], dtype=np.float64) for k in ["u"] + NAMES}
    path = os.path.join(HERE, "oracle_cfg5b_undiscounted.npz")
    np.savez_compressed(path, T=T, dU=dU,
                        meta=f"config 5b tokens {TOKENS}: near-undiscounted unstable modes, expensive control",
                        **{f"in_{k}": t.numpy() for k, t in zip(NAMES, ins)}, **out,
                        tol_A_diag=np.inf, tol_B=np.inf, tol_lgA=1e-2, tol_lgB=1e-2)
    print("wrote", path, {k: float(np.abs(v).max()) for k, v in out.items()})


if __name__ == "__main__":
    main()
