"""Generate tests/golden/oracle_cfg5b_undiscounted.npz (run from the repo root).

Four tokens (32 problems, d = 16, T = 1024) of bench config 5b -- the BASELINE
numerical-stress case, log-normal token scales -- whose open-loop states grow almost
undiscounted (log_gamma_A ~ -3e-5, 1 + A_diag up to 1.73) while control is expensive
(R_inv down to 1e-6).  Their closed-loop rollouts leave the fp32 range before the
horizon ends, yet every gradient is small (|grad| <= 152), so a solver that rolls them
out in fp32 returns inf / NaN where the answer is finite.

Inputs: ``bench.layer_workload("5b", seed=0)`` on the GPU (the workload is drawn on the
device; tokens 1151, 3182, 5268, 8689 are the first four whose gradients were
non-finite when the stable backward ran in fp32), a file of captured inputs
(``--inputs``: a torch file with ``ins`` = the nine solver inputs and ``du``), or the
inputs of the existing fixture (``--from-fixture``).

Expected outputs (``out_*``): u and the nine gradients solved in 40-digit arithmetic
(``make_golden.mp_solve_grads``: Riccati sweep, closed-loop rollouts, lambda_t = V_t h_t,
the reference's KKT gradient formulas, torch_lqr.py:34-63), one process per problem.

On these problems the Riccati value matrices reach ~1e17 with a huge eigenvalue spread,
and fp64 cannot represent their small eigen-directions, on which the gains depend: any
fp64 solve loses digits of the A_diag and B gradients.  The fixture therefore also stores
the fp64 oracle's outputs (``fp64_*``), and per-output tolerances ``tol_<name>`` =
max(1e-4, 4 x the fp64 oracle's own error against the 40-digit answer) -- finite, derived
from that measurement, and re-measured by tests/test_oracle.py.

Usage: python tests/golden/make_overflow_fixture.py [--inputs captured.pt | --from-fixture] [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
TOKENS = [1151, 3182, 5268, 8689]
T = 1024
PATH = os.path.join(HERE, "oracle_cfg5b_undiscounted.npz")
DPS = 40


def capture():
    import torch
    import bench
    ins, d_u, _ = bench.layer_workload("5b", 0, torch.device("cuda:0"))
    idx = torch.tensor(TOKENS, device=d_u.device)
    return [t[idx].cpu() for t in ins], d_u[idx].cpu()


def _mp_one(args):
    from make_golden import mp_solve_grads
    sp, dU = args
    return mp_solve_grads(sp, T, dU, dps=DPS)


def mp_outputs(ins, dU, jobs):
    """40-digit u and gradients of every problem; B / Q summed over heads."""
    from multiprocessing import Pool
    N, H = ins[0].shape[:2]
    work = []
    for n in range(N):
        for h in range(H):
            sp = [ins[0][n:n + 1, h:h + 1], ins[1][n:n + 1], ins[2][n:n + 1], ins[3][n:n + 1, h:h + 1],
                  ins[4][n:n + 1, h:h + 1], ins[5][n:n + 1, h:h + 1], ins[6][n:n + 1, h:h + 1],
                  ins[7][n:n + 1, h:h + 1], ins[8][n:n + 1, h:h + 1]]
            work.append((sp, dU[n, h]))
    with Pool(jobs) as pool:
        res = pool.map(_mp_one, work)
    out = {}
    for k in ["u"] + NAMES:
        parts = [r[k] for r in res]
        if k in ("B", "Q"):  # head-shared inputs: per-problem gradients summed over heads
            out[k] = np.stack([sum(parts[n * H + h] for h in range(H))[0] for n in range(N)])
        else:
            out[k] = np.concatenate(parts, 0).reshape((N, H) + parts[0].shape[2:])
    return out


def main():
    import torch
    from oracle.lqr64 import LQRProblem, solve_grads
    ap = argparse.ArgumentParser()
    ap.add_argument("--inputs", default=None)
    ap.add_argument("--from-fixture", action="store_true")
    ap.add_argument("--jobs", type=int, default=os.cpu_count() or 1)
    a = ap.parse_args()
    if a.from_fixture:
        z = np.load(PATH)
        ins = [torch.from_numpy(z[f"in_{k}"]) for k in NAMES]
        du = torch.from_numpy(z["dU"])
    elif a.inputs:
        z = torch.load(a.inputs, weights_only=True)
        ins, du = z["ins"], z["du"]
    else:
        ins, du = capture()
    ins = [t.float().numpy().astype(np.float64) for t in ins]
    dU = du.double().numpy()
    mp = mp_outputs(ins, dU, a.jobs)
    f64 = solve_grads(LQRProblem(*ins, T), dU)
    tol = {}
    for k in ["u"] + NAMES:
        err = float(np.abs(f64[k] - mp[k]).max() / np.abs(mp[k]).max())
        tol[k] = max(1e-4, 4.0 * err)
        print(f"{k}: fp64 oracle vs {DPS}-digit: {err:.2e} -> tolerance {tol[k]:.2e}")
    np.savez_compressed(PATH, T=T, dU=dU,
                        meta=f"config 5b tokens {TOKENS}: near-undiscounted unstable modes, expensive control; "
                             f"outputs in {DPS}-digit arithmetic",
                        **{f"in_{k}": t.astype(np.float32) for k, t in zip(NAMES, ins)},
                        **{f"out_{k}": np.asarray(mp[k], dtype=np.float64) for k in ["u"] + NAMES},
                        **{f"fp64_{k}": np.asarray(f64[k], dtype=np.float64) for k in ["u"] + NAMES},
                        **{f"tol_{k}": tol[k] for k in ["u"] + NAMES})
    print("wrote", PATH)


if __name__ == "__main__":
    main()
