"""CPU tests of the reference API surface and the library's native host solver (no GPU).

* ``TTCLayer(..., solver_impl="riccati")`` runs BASELINE config 1 on the CPU (the reference's
  CPU-runnable case) and matches the oracle layer with the fp64 solve;
* ``direct_lqr_solve`` / ``kkt_lqr_solve`` on CPU tensors (``ttc_lqr_forward_host`` /
  ``ttc_lqr_backward_host``) against the fp64 oracle: ``u`` and all nine gradients, on the
  reference bench distribution, rectangular B (d != du), stress inputs, ``A_0 = 0`` and T = 1;
* the reference's export surface and signatures (``ttc.solvers``, ``ttc.solvers.torch_lqr``,
  ``ttc.solvers.fused_lqr``, ``LQR_SOLVER_IMPL_MAP``, ``fused_lqr_solve(..., T, inv_guard)``);
* the backward's guard (``fused_lqr.py:243-246``): RuntimeError when a gradient of A_diag, B,
  Q, R_inv, Q_f or h0 reaches the limit, none when only a log-discount gradient does.
Tolerance: per tensor max|x - x64| / max|x64| <= 1e-4 (north_star); the host solver computes
in fp64, so it sits at fp32 output rounding (~1e-7).
"""
import inspect
import math

import numpy as np
import pytest
import torch

from oracle.inputs import CONFIGS, bench_solver_inputs, layer_solver_inputs, make_x
from oracle.lqr64 import LQRProblem, solve_grads, solve_u0

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
TOL = 1e-4


def _relerr(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(x - ref).max() / max(np.abs(ref).max(), 1e-30))


def _run(fn, ins, T, dU, **kw):
    xs = [t.detach().clone().float().requires_grad_(True) for t in ins]
    u = fn(*xs, T, **kw)
    (u * torch.as_tensor(dU, dtype=u.dtype)).sum().backward()
    out = {"u": u.detach().double().numpy()}
    out.update({n: t.grad.double().numpy() for n, t in zip(NAMES, xs)})
    return out


def _check(label, ins, T, fn=None, seed=0, **kw):
    from ttc.solvers import direct_lqr_solve
    fn = fn or direct_lqr_solve
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed + 3)).double().numpy()
    ref = solve_grads(pb, dU)
    out = _run(fn, ins, T, dU, **kw)
    errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES}
    print(f"[{label}] " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()))
    bad = {k: v for k, v in errs.items() if not v <= TOL}
    assert not bad, f"{label}: {bad}"
    return out, ref


def test_config1_layer_on_cpu_matches_oracle():
    """BASELINE config 1 as the reference runs it: TTCLayer(32, 32, 16, 8, 16, 16,
    solver_impl="riccati") forward on the CPU, x [2, 128, 8, 32] ~ N(0, 1), T = 64 (16,384
    problems), against the oracle layer restatement with the fp64 solve: the solver output
    and the layer output within 1e-4."""
    from ttc import TTCLayer
    from oracle.layer_ref import LayerParams, back_end, front_end
    c = CONFIGS[1]
    torch.manual_seed(0)
    layer = TTCLayer(c["in_dim"], c["out_dim"], c["h_dim"], c["num_heads"], c["b_rank"], c["q_rank"],
                     solver_impl="riccati")
    assert not layer.factored
    x = make_x(1)
    assert tuple(x.shape) == c["x_shape"]
    with torch.no_grad():
        ins_layer = layer.solver_inputs(x)
        u = layer.solver(*ins_layer, c["T"])
        y = layer(x, T=c["T"])
    p = LayerParams(c["in_dim"], c["out_dim"], c["h_dim"], c["num_heads"], c["b_rank"], c["q_rank"])
    p.W_in, p.W_out = layer.in_proj.weight.detach(), layer.out_proj.weight.detach()
    p.Bs, p.Qs = layer.Bs.detach(), layer.Qs.detach()
    ins, lead = front_end(p, x)
    u64 = solve_u0(LQRProblem(*ins, c["T"]))
    y_ref = back_end(p, torch.from_numpy(u64).float(), ins[8], lead)
    eu, ey = _relerr(u.numpy(), u64), _relerr(y.numpy(), y_ref.numpy())
    print(f"config 1 on CPU: u rel err {eu:.1e}, y rel err {ey:.1e}")
    assert y.shape == (2, 128, 8, 32)
    assert eu <= TOL and ey <= TOL


def test_bench_distribution_riccati_and_kkt():
    from ttc.solvers import direct_lqr_solve, kkt_lqr_solve
    ins = bench_solver_inputs(4, 4, 16, seed=0)  # bench_lqr_solvers.py:173-207 shape
    a, _ = _check("riccati", ins, 64, direct_lqr_solve)
    b, _ = _check("kkt", ins, 64, kkt_lqr_solve)
    for k in a:  # same native solver on the CPU
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("d,du,H,T", [(12, 8, 3, 9), (7, 13, 2, 5), (16, 16, 8, 1), (33, 20, 1, 17)])
def test_rectangular_and_short_horizons(d, du, H, T):
    g = torch.Generator().manual_seed(d * 100 + du)
    ins = bench_solver_inputs(3, H, max(d, du), seed=d + du)
    A, _, Q, _, Qf, lgA, _, lgQ, h0 = ins
    B = torch.randn(3, d, du, generator=g) / math.sqrt(max(d, du))
    R_inv = torch.nn.functional.softplus(torch.rand(3, H, du, generator=g))
    lgB = -torch.nn.functional.softplus(torch.randn(3, H, du, generator=g)) - 1.0
    ins = [A[..., :d], B, Q[:, :d, :d], R_inv, Qf[:, :, :d, :d], lgA, lgB, lgQ[..., :d], h0[..., :d]]
    _check(f"d{d} du{du} H{H} T{T}", [t.contiguous() for t in ins], T)


@pytest.mark.parametrize("T", [64, 256])
def test_stress_inputs(T):
    """Config-5 inputs (log-normal token scales): gradients beyond the reference's 1e6 guard
    occur, so the guard is lifted."""
    from ttc.solvers.host_lqr import host_lqr_solve
    x = make_x(5, n_tokens=4, seed=17)
    _check(f"cfg5 T{T}", layer_solver_inputs(5, x), T, host_lqr_solve, grad_limit=math.inf)


def _A0_zero_inputs(seed=3):
    """a_i = -exp(-lgA) for every state of problem 0, so A_0 = diag(1 + a exp(lgA)) = 0: the
    state is reset at the first step and only B_0 u_0 drives h_1 (a case the host can set; the
    reference's fused solver divides by A_k there)."""
    ins = [t.clone() for t in bench_solver_inputs(2, 2, 16, seed=seed)]
    A, lgA = ins[0], ins[5]
    A[0, 0] = -torch.exp(-lgA[0, 0])
    return ins


def test_A0_zero():
    out, _ = _check("A0=0", _A0_zero_inputs(), 24)
    alpha0 = 1.0 + _A0_zero_inputs()[0][0, 0].double() * torch.exp(_A0_zero_inputs()[5][0, 0].double())
    assert float(alpha0.abs().max()) < 1e-6
    # with A_0 = 0, u_0 cannot depend on h_0: d u_0 / d h_0 = 0 for that problem
    assert np.abs(out["h0"][0, 0]).max() <= 1e-6 * max(np.abs(out["h0"]).max(), 1.0)


def test_reference_export_surface():
    import ttc
    import ttc.solvers as S
    from ttc.layers.ttc_layer import LQR_SOLVER_IMPL_MAP
    from ttc.solvers.fused_lqr import fused_lqr_solve, FusedLQRSolveFunc
    from ttc.solvers.torch_lqr import direct_lqr_solve, kkt_lqr_solve
    assert hasattr(ttc, "TTCLayer")
    for name in ("direct_lqr_solve", "kkt_lqr_solve", "fused_lqr_solve"):
        assert name in S.__all__ and callable(getattr(S, name))
    assert S.direct_lqr_solve is direct_lqr_solve and S.kkt_lqr_solve is kkt_lqr_solve
    for key in ("riccati", "kkt", "fused"):
        assert key in LQR_SOLVER_IMPL_MAP
    ref_params = ["A_diag", "B", "Q", "R_inv_diag", "Q_f", "gamma_A", "gamma_B", "gamma_Q", "h0", "T", "inv_guard"]
    assert list(inspect.signature(fused_lqr_solve).parameters) == ref_params
    # the autograd Function keeps the reference's positional slots (fused_lqr.py:255-269):
    # apply(..., h0, T, cache_level="LU", inv_guard=False)
    fsig = inspect.signature(FusedLQRSolveFunc.forward)
    assert list(fsig.parameters) == ["ctx"] + ref_params[:10] + ["cache_level", "inv_guard"]
    assert fsig.parameters["cache_level"].default == "LU" and fsig.parameters["inv_guard"].default is False
    assert FusedLQRSolveFunc is not S.HipLQRSolveFunc
    sig = inspect.signature(S.hip_lqr_solve)
    assert list(sig.parameters)[10] == "inv_guard"
    for k in ("grad_limit", "stash", "precision", "stable_backward"):
        assert sig.parameters[k].kind is inspect.Parameter.KEYWORD_ONLY
    names = list(inspect.signature(direct_lqr_solve).parameters)
    assert names == ["A_diag", "B", "Q", "R_inv_diag", "Q_f", "log_gamma_A", "log_gamma_B", "log_gamma_Q", "h0", "T"]


def test_hip_key_rejects_cpu_tensors():
    """The HIP solver never falls back to the host: CPU tensors raise."""
    from ttc.solvers import hip_lqr_solve
    ins = bench_solver_inputs(1, 1, 16, seed=0)
    with pytest.raises(AssertionError, match="GPU"):
        hip_lqr_solve(*ins, 4)


def test_nan_input_raises_on_cpu():
    from ttc.solvers import direct_lqr_solve
    ins = bench_solver_inputs(2, 2, 16, seed=1)
    ins[8] = ins[8].clone()
    ins[8][0, 0, 0] = float("nan")
    with pytest.raises(RuntimeError, match="Numerical instability"):
        direct_lqr_solve(*ins, 8)


def guard_inputs(H=2, seed=5):
    """Long, barely discounted horizons with a small A_diag: the (t+1) factor of the
    log-discount gradients makes them larger than every gradient the guard covers."""
    ins = bench_solver_inputs(2, H, 16, seed=seed)
    ins[0] = ins[0] * 0.1
    ins[5], ins[6], ins[7] = ins[5] * 0.005, ins[6] * 0.005, ins[7] * 0.005
    return ins


GUARD_T = 256
GUARDED = ("A_diag", "B", "Q", "R_inv", "Q_f", "h0")


def test_grad_guard_covers_the_reference_six():
    """The magnitude guard raises when a gradient of A_diag, B, Q, R_inv, Q_f or h0 reaches the
    limit, and not when only a log-discount gradient does (fused_lqr.py:243-246 checks those six)."""
    from ttc.solvers.host_lqr import host_lqr_solve
    ins = guard_inputs()
    dU = np.zeros((2, 2, 16))
    dU[:, 0] = 1.0  # head 0 only: head 1's adjoint, hence its gradient contribution, is zero
    g = _run(host_lqr_solve, ins, GUARD_T, dU, grad_limit=math.inf)
    guarded = max(np.abs(g[k]).max() for k in GUARDED)
    lg = max(np.abs(g[k]).max() for k in ("lgA", "lgB", "lgQ"))
    assert lg > 1.2 * guarded, (lg, guarded)
    _run(host_lqr_solve, ins, GUARD_T, dU, grad_limit=math.sqrt(lg * guarded))  # no error
    with pytest.raises(RuntimeError, match="backward"):
        _run(host_lqr_solve, ins, GUARD_T, dU, grad_limit=0.5 * guarded)


def test_layer_parameter_gradients_on_cpu_match_oracle():
    """TTCLayer(solver_impl="riccati") on the CPU: gradients of in_proj, out_proj, Bs and Qs
    against fp64 autograd of the oracle layer around the fp64 oracle solve (chained with the
    oracle's nine solver gradients), T = 16."""
    from ttc import TTCLayer
    from _layer_oracle import oracle_layer_grads
    torch.manual_seed(1)
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="riccati")
    x = torch.randn(3, 5, 32, generator=torch.Generator().manual_seed(2))
    dy = torch.randn(3, 5, 32, generator=torch.Generator().manual_seed(3))
    y = layer(x, T=16)
    (y * dy).sum().backward()
    ref = oracle_layer_grads(layer, x, dy, 16)
    for name, p in (("in_proj", layer.in_proj.weight), ("out_proj", layer.out_proj.weight), ("Bs", layer.Bs),
                    ("Qs", layer.Qs)):
        e = _relerr(p.grad.numpy(), ref[name])
        print(f"layer grad {name}: {e:.1e}")
        assert e <= TOL, name
