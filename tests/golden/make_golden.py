"""Generate the committed golden fixtures under tests/golden/ (run from the repo root).

``mp_stress_*.npz``: single LQR problems (N=1, H=1) cut from the config-5 stress
distribution (log-normal token scale, the worst problem of a seeded slice), solved
in 50-digit arithmetic with mpmath -- a Riccati sweep, closed-loop rollouts and the
costates taken directly as lambda_t = V_t h_t (no recursion), then the gradient
formulas of the reference ``KKTLQRSolveFunc`` (ttc/solvers/torch_lqr.py:34-63)
chained through the discount expansion (torch_lqr.py:65-91).  Independent of the
fp64 oracle's code path; pins it where the dense QP is too ill-conditioned to.

``oracle_cfg*.npz``: small seeded slices of each BASELINE config with fp64 oracle
outputs (u and the nine gradients), consumed by the GPU parity tests so a run on
the GPU box checks against committed numbers.

Usage: python tests/golden/make_golden.py [--skip-mp]
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


def mp_solve_grads(ins, T, dU, dps=50):
    """ins: nine float64 arrays for N=1, H=1; returns dict of u and the nine gradients."""
    import mpmath as mp
    mp.mp.dps = dps
    A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0 = [np.asarray(x, dtype=np.float64) for x in ins]
    d, du = B.shape[-2], B.shape[-1]
    f = lambda x: mp.mpf(float(x))
    M = lambda A: mp.matrix([[f(v) for v in row] for row in A])
    a = [f(v) for v in A_diag.reshape(d)]
    Bm = M(B.reshape(d, du))
    Qm = M(0.5 * (Q.reshape(d, d) + Q.reshape(d, d).T))
    r = [f(v) for v in R_inv.reshape(du)]
    Qf = M(0.5 * (Q_f.reshape(d, d) + Q_f.reshape(d, d).T))
    la, lb, lq = f(lgA.reshape(())), [f(v) for v in lgB.reshape(du)], [f(v) for v in lgQ.reshape(d)]
    x0 = mp.matrix([f(v) for v in h0.reshape(d)])
    g = mp.matrix([f(v) for v in np.asarray(dU).reshape(du)])

    def step(k):
        al = [1 + a[i] * mp.exp(la * (k + 1)) for i in range(d)]
        be = [mp.exp(lb[j] * (k + 1)) for j in range(du)]
        Bk = mp.matrix(d, du)
        for i in range(d):
            for j in range(du):
                Bk[i, j] = Bm[i, j] * be[j]
        return al, be, Bk

    def qscale(k):
        return [mp.exp(lq[i] * k) for i in range(d)]

    Vs = [None] * (T + 1)
    Ks = [None] * T
    V = Qf
    Vs[T] = V
    Qi0 = None
    for k in range(T - 1, -1, -1):
        al, be, Bk = step(k)
        VA = mp.matrix(d, d)
        for i in range(d):
            for j in range(d):
                VA[i, j] = V[i, j] * al[j]
        Qux = Bk.T * VA
        Quu = Bk.T * V * Bk
        for j in range(du):
            Quu[j, j] += 1 / r[j]
        Qi = mp.inverse(Quu)
        K = -(Qi * Qux)
        Ks[k] = K
        X = Qux.T * K
        q = qscale(k) if k > 0 else None
        Vn = mp.matrix(d, d)
        for i in range(d):
            for j in range(d):
                Vn[i, j] = al[i] * VA[i, j] + X[i, j] + (q[i] * Qm[i, j] * q[j] if q else 0)
        V = (Vn + Vn.T) / 2
        Vs[k] = V
        if k == 0:
            Qi0 = Qi
    h = [x0]
    hb = [mp.matrix(d, 1)]
    u, w = [], []
    w0 = -(Qi0 * g)
    for k in range(T):
        al, be, Bk = step(k)
        uk = Ks[k] * h[k]
        wk = Ks[k] * hb[k] + (w0 if k == 0 else mp.matrix(du, 1))
        u.append(uk)
        w.append(wk)
        Bu, Bw = Bk * uk, Bk * wk
        hn, hbn = mp.matrix(d, 1), mp.matrix(d, 1)
        for i in range(d):
            hn[i] = al[i] * h[k][i] + Bu[i]
            hbn[i] = al[i] * hb[k][i] + Bw[i]
        h.append(hn)
        hb.append(hbn)
    lam = [None] + [Vs[k] * h[k] for k in range(1, T + 1)]
    lamb = [None] + [Vs[k] * hb[k] for k in range(1, T + 1)]
    z = lambda: mp.mpf(0)
    gA = [z() for _ in range(d)]
    glgA = z()
    gB = mp.matrix(d, du)
    glgB = [z() for _ in range(du)]
    gQ = mp.matrix(d, d)
    glgQ = [z() for _ in range(d)]
    gr = [z() for _ in range(du)]
    for k in range(T):
        al, be, Bk = step(k)
        eA = mp.exp(la * (k + 1))
        for i in range(d):
            gAk = h[k][i] * lamb[k + 1][i] + hb[k][i] * lam[k + 1][i]
            gA[i] += gAk * eA
            glgA += gAk * a[i] * (k + 1) * eA
        for i in range(d):
            for j in range(du):
                gBk = lamb[k + 1][i] * u[k][j] + lam[k + 1][i] * w[k][j]
                gB[i, j] += gBk * be[j]
                glgB[j] += gBk * Bm[i, j] * (k + 1) * be[j]
        for j in range(du):
            gr[j] += -u[k][j] * w[k][j] / r[j] ** 2
        if k < T - 1:
            q = qscale(k + 1)
            for i in range(d):
                for j in range(d):
                    gq = (hb[k + 1][i] * h[k + 1][j] + h[k + 1][i] * hb[k + 1][j]) / 2
                    gQ[i, j] += q[i] * gq * q[j]
                    glgQ[i] += 2 * gq * q[i] * Qm[i, j] * q[j] * (k + 1)
    al0 = step(0)[0]
    F = lambda x: float(x)
    out = {
        "u": np.array([F(x) for x in u[0]]).reshape(1, 1, du),
        "A_diag": np.array([F(x) for x in gA]).reshape(1, 1, d),
        "B": np.array([[F(gB[i, j]) for j in range(du)] for i in range(d)]).reshape(1, d, du),
        "Q": np.array([[F(gQ[i, j]) for j in range(d)] for i in range(d)]).reshape(1, d, d),
        "R_inv": np.array([F(x) for x in gr]).reshape(1, 1, du),
        "Q_f": np.array([[F((hb[T][i] * h[T][j] + h[T][i] * hb[T][j]) / 2) for j in range(d)]
                         for i in range(d)]).reshape(1, 1, d, d),
        "lgA": np.array(F(glgA)).reshape(1, 1),
        "lgB": np.array([F(x) for x in glgB]).reshape(1, 1, du),
        "lgQ": np.array([F(x) for x in glgQ]).reshape(1, 1, d),
        "h0": np.array([F(al0[i] * lamb[1][i]) for i in range(d)]).reshape(1, 1, d),
    }
    return out


def single_problem(ins, p, H):
    n, hh = divmod(p, H)
    A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0 = [t.detach().double().numpy() for t in ins]
    return [A_diag[n:n + 1, hh:hh + 1], B[n:n + 1], Q[n:n + 1], R_inv[n:n + 1, hh:hh + 1],
            Q_f[n:n + 1, hh:hh + 1], lgA[n:n + 1, hh:hh + 1], lgB[n:n + 1, hh:hh + 1],
            lgQ[n:n + 1, hh:hh + 1], h0[n:n + 1, hh:hh + 1]]


def worst_problem(ins, T, seed):
    """Index of the problem whose |A_diag grad| relative error of an fp32 forward
    Riccati + open-loop costates would be largest -- i.e. the most ill-conditioned
    costate sweep, picked with the fp64 oracle alone (largest lambda growth)."""
    import torch
    from oracle.lqr64 import LQRProblem, solve_grads
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed + 7)).double().numpy()
    ref = solve_grads(pb, dU)
    mags = np.abs(ref["h0"]).reshape(pb.P, -1).max(-1)
    return int(np.argmax(mags)), dU.reshape(pb.P, -1)


def make_mp(name, cfg, n_tokens, seed, T):
    import torch
    from oracle.inputs import layer_solver_inputs, make_x
    x = make_x(cfg, n_tokens=n_tokens, seed=seed)
    ins = layer_solver_inputs(cfg, x)
    p, dU = worst_problem(ins, T, seed)
    sp = single_problem(ins, p, ins[0].shape[1])
    out = mp_solve_grads(sp, T, dU[p])
    path = os.path.join(HERE, name)
    np.savez_compressed(path, T=T, dU=dU[p].reshape(1, 1, -1), **{f"in_{k}": v for k, v in zip(NAMES, sp)},
                        **{f"out_{k}": v for k, v in out.items()},
                        meta=np.array(f"cfg{cfg} seed{seed} n_tokens{n_tokens} problem{p} T{T} mpmath dps=50"))
    print("wrote", path)


def make_oracle_fixtures():
    import torch
    from oracle.inputs import CONFIGS, layer_solver_inputs, make_x, bench_solver_inputs
    from oracle.lqr64 import LQRProblem, solve_grads
    cases = [("oracle_bench.npz", None, 4, 0, 64), ("oracle_cfg1.npz", 1, 8, 0, 64), ("oracle_cfg2.npz", 2, 16, 1, 64),
             ("oracle_cfg3.npz", 3, 1, 2, 128), ("oracle_cfg4.npz", 4, 1, 3, 256),
             ("oracle_cfg5.npz", 5, 2, 5, 1024), ("oracle_cfg5b.npz", "5b", 2, 6, 1024)]
    for name, cfg, nt, seed, T in cases:
        if cfg is None:
            ins = bench_solver_inputs(nt, 4, 16, seed=seed)
        else:
            ins = layer_solver_inputs(cfg, make_x(cfg, n_tokens=nt, seed=seed))
        pb = LQRProblem(*ins, T)
        dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed + 7)).double().numpy()
        ref = solve_grads(pb, dU)
        np.savez_compressed(os.path.join(HERE, name), T=T, dU=dU,
                            **{f"in_{k}": t.numpy() for k, t in zip(NAMES, ins)},
                            **{f"out_{k}": ref[k] for k in ["u"] + NAMES},
                            meta=np.array(f"cfg{cfg} seed{seed} n_tokens{nt} T{T} fp64 oracle"))
        print("wrote", name)


def make_beyond_fp64(name="mp_cfg5b_beyond_fp64.npz", n_tokens=12288, seed=21, p=5086, T=1024):
    """u of one config-5b problem that fp64 does not resolve (problem 5086 of a 12,288-token
    sample: the fp64 oracle and both fp64 rescue routes of the solver miss it by 10-33 %), in
    40-digit arithmetic, with the problem's inputs."""
    from oracle.inputs import layer_solver_inputs, make_x
    ins = layer_solver_inputs("5b", make_x("5b", n_tokens=n_tokens, seed=seed))
    sp = single_problem(ins, p, ins[0].shape[1])
    out = mp_solve_grads(sp, T, np.zeros((1, 1, sp[1].shape[-1])), dps=40)
    path = os.path.join(HERE, name)
    np.savez_compressed(path, T=T, p=p, n_tokens=n_tokens, seed=seed, out_u=out["u"],
                        **{f"in_{k}": v for k, v in zip(NAMES, sp)},
                        meta=np.array(f"cfg5b seed{seed} n_tokens{n_tokens} problem{p} T{T} mpmath dps=40 (u only)"))
    print("wrote", path)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-mp", action="store_true")
    ap.add_argument("--beyond-fp64", action="store_true", help="write only mp_cfg5b_beyond_fp64.npz")
    a = ap.parse_args()
    if a.beyond_fp64:
        make_beyond_fp64()
        raise SystemExit(0)
    make_oracle_fixtures()
    if not a.skip_mp:
        make_mp("mp_stress_cfg5_T64.npz", 5, 64, 5, 64)
        make_mp("mp_stress_cfg5_T1024.npz", 5, 16, 0, 1024)
        make_beyond_fp64()
