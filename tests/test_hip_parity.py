"""GPU parity: the HIP solver (through the C ABI, via the autograd Function) against
the fp64 oracle, on seeded inputs from every BASELINE configuration.

Tolerance (north_star): per tensor, max|x - x64| / max|x64| <= 1e-4 for ``u`` and
all nine gradients.  ``Q`` / ``Q_f`` gradients are the symmetric gradients on
both sides.  Gradients of the stress configuration can exceed the reference's
1e6 guard, so those cases pass ``grad_limit=inf``.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle.inputs import CONFIGS, bench_solver_inputs, layer_solver_inputs, make_x
from oracle.lqr64 import LQRProblem, solve_grads, solve_u0

pytestmark = pytest.mark.gpu

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
TOL = 1e-4


def _solver():
    from ttc.solvers.hip_lqr import hip_lqr_solve
    return hip_lqr_solve


def _relerr(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(x - ref).max() / max(np.abs(ref).max(), 1e-30))


def run_hip(ins, T, dU, grad_limit=1e6, stash=None, precision="auto", stable=False):
    solve = _solver()
    from ttc.solvers.hip_lqr import last_backward_stats
    dev = torch.device("cuda:0")
    xs = [t.detach().to(dev).float().requires_grad_(True) for t in ins]
    u = solve(*xs, T, grad_limit=grad_limit, stash=stash, precision=precision, stable_backward=stable)
    (u * torch.as_tensor(dU, device=dev, dtype=u.dtype)).sum().backward()
    out = {"u": u.detach().cpu().double().numpy()}
    for n, t in zip(NAMES, xs):
        out[n] = t.grad.detach().cpu().double().numpy()
    out["_fallback"] = last_backward_stats["fallback"]
    return out


def check_case(label, ins, T, seed=0, grad_limit=1e6, stash=None, tol=TOL, precision="auto", stable=False):
    pb = LQRProblem(*ins, T)
    g = torch.Generator().manual_seed(seed + 7)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=g).double().numpy()
    ref = solve_grads(pb, dU)
    print(f"[{label}] N={pb.N} H={pb.H} d={pb.d} du={pb.du} T={T} stash={stash} precision={precision} "
          f"stable={stable}", flush=True)
    out = run_hip(ins, T, dU, grad_limit=grad_limit, stash=stash, precision=precision, stable=stable)
    errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES}
    print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()) + f"  fallback={out['_fallback']}/{pb.P}",
          flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"{label}: rel err above {tol}: {bad}"
    return out


def test_reference_correctness_shape():
    """bench_lqr_solvers.py:173-207 shape: batch 4, heads 4, d 16, T 64."""
    check_case("bench-check", bench_solver_inputs(4, 4, 16, seed=0), 64)


@pytest.mark.parametrize("stash", ["always", "never"])
def test_config1_layer_slice(stash):
    c = CONFIGS[1]
    x = make_x(1, n_tokens=24, seed=0)
    check_case("cfg1", layer_solver_inputs(1, x), c["T"], stash=stash)


@pytest.mark.parametrize("precision", ["fp32", "fp32-riccati", "fp32-row", "fp64"])
def test_config2_layer_slice(precision):
    c = CONFIGS[2]
    x = make_x(2, n_tokens=64, seed=1)
    out = check_case("cfg2", layer_solver_inputs(2, x), c["T"], precision=precision)
    assert out["_fallback"] == 0  # nominal inputs: every problem passes the certificate


@pytest.mark.parametrize("cfg,n_tok", [(2, 32), (3, 2), (4, 1)])
def test_stable_backward_path(cfg, n_tok):
    """The stable path alone (per-step gains + closed-loop costates) on nominal configs."""
    x = make_x(cfg, n_tokens=n_tok, seed=6)
    out = check_case(f"cfg{cfg}-stable", layer_solver_inputs(cfg, x), CONFIGS[cfg]["T"], stable=True)
    assert out["_fallback"] == out["u"].shape[0] * out["u"].shape[1]


def test_certificate_rejects_stress_problems_and_fallback():
    """Config-5 inputs at T=64: some problems fail the certificate and take the stable
    path; the mixed result agrees with the all-stable run and the fp64 oracle."""
    x = make_x(5, n_tokens=16, seed=5)
    ins = layer_solver_inputs(5, x)
    pb = LQRProblem(*ins, 64)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(3)).double().numpy()
    fast = run_hip(ins, 64, dU, grad_limit=math.inf)
    slow = run_hip(ins, 64, dU, grad_limit=math.inf, stable=True)
    print(f"fallback {fast['_fallback']}/{pb.P}", flush=True)
    assert 0 < fast["_fallback"] < pb.P
    ref = solve_grads(pb, dU)
    for k in ["u"] + NAMES:
        assert _relerr(fast[k], ref[k]) <= TOL, k
        assert _relerr(fast[k], slow[k]) <= TOL, k


def _regroup_heads(ins, H_new):
    """Problems of consecutive tokens regrouped into tokens of H_new heads (the token-shared
    B and Q of each new token are those of its first old token)."""
    A, B, Q, R, Qf, lA, lB, lQ, h0 = ins
    N, H = A.shape[:2]
    k = H_new // H
    N2 = N // k
    per = lambda t: t[:N2 * k].reshape(N2, H_new, *t.shape[2:])  # noqa: E731
    return [per(A), B[:N2 * k:k], Q[:N2 * k:k], per(R), per(Qf), per(lA), per(lB), per(lQ), per(h0)]


@pytest.mark.parametrize("N,H,T", [(3, 8, 64), (2, 16, 40), (2, 24, 17), (4, 8, 1), (3, 16, 2)])
def test_d16_head_groups_matrix_core_backward(N, H, T):
    """The d = 16 backward over head groups of 8 on the matrix cores: one group per token
    (H = 8, head sums written directly) and several (H = 16, 24: group sums, then head
    sums), T = 1 and 2 included."""
    ins = bench_solver_inputs(N, H, 16, seed=N + H + T)
    out = check_case(f"groups N={N} H={H}", ins, T)
    assert out["_fallback"] % 8 == 0


def test_d16_head_groups_with_rejected_groups():
    """Config-5 stress problems regrouped to 16 heads per token: groups that fail the
    certificate go through the stable path as whole groups, and the head sums of grad_B /
    grad_Q combine matrix-core groups and stable-path groups of the same token."""
    x = make_x(5, n_tokens=24, seed=11)
    ins = _regroup_heads(layer_solver_inputs(5, x), 16)
    pb = LQRProblem(*ins, 64)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(4)).double().numpy()
    fast = run_hip(ins, 64, dU, grad_limit=math.inf)
    print(f"fallback {fast['_fallback']}/{pb.P}", flush=True)
    assert 0 < fast["_fallback"] < pb.P and fast["_fallback"] % 8 == 0
    ref = solve_grads(pb, dU)
    for k in ["u"] + NAMES:
        assert _relerr(fast[k], ref[k]) <= TOL, k


@pytest.mark.parametrize("d", [32, 64])
@pytest.mark.parametrize("N,H,T", [(3, 8, 40), (2, 16, 33), (1, 24, 2), (2, 8, 1)])
def test_wide_head_groups_matrix_core_backward(d, N, H, T):
    """The d = 32 / 64 backward over head groups of 8 on the matrix cores (d / 16 waves per
    group): one group per token (H = 8, head sums written directly), several (H = 16, 24),
    T = 1 and 2 included."""
    ins = bench_solver_inputs(N, H, d, seed=d + N + H + T)
    out = check_case(f"groups{d} N={N} H={H}", ins, T)
    assert out["_fallback"] % 8 == 0


@pytest.mark.parametrize("d,H,T", [(32, 16, 128), (64, 8, 96)])
def test_wide_head_groups_on_stress_inputs(d, H, T):
    """Head groups on the stress inputs of the symplectic tests (log-normal scalings of Q,
    Q_f and R_inv, barely discounted): whatever groups the certificate rejects take the
    stable path as whole groups, and every tensor stays within the bound."""
    ins = bench_solver_inputs(4, H, d, seed=T + d + 1)
    g = torch.Generator().manual_seed(T + 2)
    s = torch.exp(1.5 * torch.randn(4, generator=g))
    A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0 = ins
    Q = Q * s[:, None, None]
    Qf = Qf * s[:, None, None, None].flip(0)
    R_inv = R_inv * torch.exp(torch.randn(4, H, 1, generator=g))
    lgA, lgB, lgQ = lgA * 0.05, lgB * 0.05, lgQ * 0.05
    out = check_case(f"groups{d}-stress-T{T}", [A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0], T,
                     grad_limit=math.inf)
    assert out["_fallback"] % 8 == 0


@pytest.mark.parametrize("d,T", [(32, 128), (64, 96)])
def test_wide_head_groups_with_rejected_groups(d, T):
    """Stress inputs on the second head group of every token only (heads 8..15: barely
    discounted, log-normal scalings of Q_f and R_inv): its groups fail the certificate and
    take the stable path as whole groups while the first groups stay on the matrix cores,
    and the head sums of grad_B / grad_Q combine both kinds of group of the same token."""
    H = 16
    ins = bench_solver_inputs(3, H, d, seed=T + d + 3)
    A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0 = [t.clone() for t in ins]
    g = torch.Generator().manual_seed(T + 5)
    hi = slice(8, 16)
    Qf[:, hi] *= torch.exp(1.5 * torch.randn(3, 1, 1, 1, generator=g))
    R_inv[:, hi] *= torch.exp(torch.randn(3, 8, 1, generator=g))
    lgA[:, hi] *= 0.05
    lgB[:, hi] *= 0.05
    lgQ[:, hi] *= 0.05
    out = check_case(f"groups{d}-mixed-T{T}", [A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0], T,
                     grad_limit=math.inf)
    P = 3 * H
    assert 0 < out["_fallback"] < P and out["_fallback"] % 8 == 0


def test_config3_layer_slice():
    c = CONFIGS[3]
    x = make_x(3, n_tokens=2, seed=2)
    check_case("cfg3", layer_solver_inputs(3, x), c["T"])


@pytest.mark.parametrize("precision", ["fp32", "fp64"])
def test_config4_layer_slice(precision):
    c = CONFIGS[4]
    x = make_x(4, n_tokens=1, seed=3)
    check_case("cfg4", layer_solver_inputs(4, x), c["T"], precision=precision)


@pytest.mark.parametrize("cfg,n_tok,precision", [(3, 3, "fp32-row"), (4, 2, "fp32-row"), (3, 2, "fp32-riccati"),
                                              (4, 1, "fp32-riccati")])
def test_wide_configs_row_kernel(cfg, n_tok, precision):
    """d = 64 / 32 through the row-layout kernel: an independent cross-check of the
    matrix-core kernel that the default precision selects."""
    x = make_x(cfg, n_tokens=n_tok, seed=8)
    check_case(f"cfg{cfg}-row", layer_solver_inputs(cfg, x), CONFIGS[cfg]["T"], precision=precision)


@pytest.mark.parametrize("d,N,H,T", [(32, 3, 3, 40), (64, 2, 3, 33), (32, 1, 1, 1), (64, 1, 2, 2),
                                     (32, 2, 16, 24), (64, 2, 4, 24), (32, 1, 16, 1), (64, 1, 4, 1)])
@pytest.mark.parametrize("stash", ["always", "never"])
@pytest.mark.parametrize("precision", ["fp32", "fp32-riccati"])
def test_wide_matrix_core_ragged(d, N, H, T, stash, precision):
    """d = 32 / 64 matrix-core kernels on the reference's bench distribution: odd problem
    counts (an idle problem slot in the last d = 32 wave), head counts that select the
    one-wave (H = 1, 2, 3) or the 4-wave shared-B/Q workgroups (H = 16 at d = 32, H = 4 at
    d = 64), and short horizons (T = 1: step 0 only).  d = 32 with an even head count runs
    the symplectic sweep under "fp32" and blocked-Cholesky Riccati steps under "fp32-riccati"."""
    check_case(f"mc{d}", bench_solver_inputs(N, H, d, seed=d + T), T, stash=stash, precision=precision)


def _indefinite_wide_inputs(d, mode, H=2, seed=2):
    """d = 32 / 64 inputs whose Cholesky pivot breaks down while the problem stays well
    conditioned (B orthogonal, so B'B = I and Quu = R + beta^2 V in the step where it
    happens).  mode "terminal": problem 1 has Q_f = -3 I, so Quu is negative definite
    from the first step (t = T-1) on.  mode "mid": token 0 has Q = -10 I (barely
    discounted) and Q_f = 0.1 I, so Quu is positive definite at t = T-1 and negative
    definite from t = T-2 on.  The matrix-core kernel marks the affected waves and the
    rescue pass recomputes those problems with the pivoted row-layout sweep.  (Condition
    numbers of Quu stay below 3; the reference's own fp32 solvers are within 2e-5.)"""
    ins = bench_solver_inputs(2, H, d, seed=seed)
    g = torch.Generator().manual_seed(seed)
    B, _ = torch.linalg.qr(torch.randn(2, d, d, generator=g))
    lgB = torch.full((2, H, d), -0.01)
    A_diag, _, Q, R_inv, Qf, lgA, _, lgQ, h0 = [t.clone() for t in ins]
    if mode == "terminal":
        Qf[0, 1] = -3.0 * torch.eye(d)
    else:
        Q[0] = -10.0 * torch.eye(d)
        lgQ[0] = -0.01
        Qf[0] = 0.1 * torch.eye(d)
    return [A_diag, B.contiguous(), Q, R_inv, Qf, lgA, lgB, lgQ, h0]


@pytest.mark.parametrize("d,H", [(32, 2), (64, 2), (32, 16), (64, 4)])
@pytest.mark.parametrize("mode", ["terminal", "mid"])
@pytest.mark.parametrize("stash", ["always", "never"])
@pytest.mark.parametrize("precision", ["fp32", "fp32-riccati"])
def test_wide_indefinite_Quu_rescued(d, H, mode, stash, precision):
    """H = 2: one-wave workgroups; H = 16 (d = 32) / 4 (d = 64): workgroups of 4 waves that
    share the token's B and Q in LDS.  ("fp32" at d = 32 runs the symplectic sweep, which
    has no Cholesky to break down: these inputs then check it on indefinite Q and Q_f.)"""
    check_case(f"indef{d}-H{H}-{mode}", _indefinite_wide_inputs(d, mode, H), 6, stash=stash, precision=precision)


@pytest.mark.parametrize("d,H,T", [(32, 2, 64), (32, 2, 256), (64, 4, 64), (64, 4, 128)])
def test_wide_symplectic_stress(d, H, T):
    """The d = 32 / 64 symplectic sweeps on inputs with a wide conditioning spread (per-token
    log-normal scalings of Q, Q_f and R_inv, barely discounted): u and all gradients within
    the bound, whatever their certificate accepts or hands to the rescue pass."""
    ins = bench_solver_inputs(6, H, d, seed=T + d)
    g = torch.Generator().manual_seed(T + 1)
    s = torch.exp(1.5 * torch.randn(6, generator=g))
    A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0 = ins
    Q = Q * s[:, None, None]
    Qf = Qf * s[:, None, None, None].flip(0)
    R_inv = R_inv * torch.exp(torch.randn(6, H, 1, generator=g))
    lgA, lgB, lgQ = lgA * 0.05, lgB * 0.05, lgQ * 0.05
    check_case(f"sym{d}-T{T}", [A_diag, B, Q, R_inv, Qf, lgA, lgB, lgQ, h0], T, grad_limit=math.inf,
               precision="fp32")


@pytest.mark.parametrize("cfg,T,seed", [(5, 64, 5), (5, 1024, 5), ("5b", 1024, 55), (5, 2048, 7), ("5b", 2048, 57)])
def test_config5_stress(cfg, T, seed):
    """Config 5 / 5b share the layer and the log-normal token scales; 5b draws its own tokens
    (another seed), so the two cases cover different problems.  T = 2048 is the longest horizon
    of the reference bench's sweep (bench_lqr_solvers.py:30-37)."""
    x = make_x(cfg, n_tokens=4, seed=seed)
    check_case(f"cfg{cfg}", layer_solver_inputs(cfg, x), T, grad_limit=math.inf)


@pytest.mark.parametrize("d,H", [(16, 8), (16, 16), (32, 8)])
def test_long_horizon_two_tier_rollout(d, H, monkeypatch):
    """T = 1024, heads % 8 == 0 (TTC_LQR_FLAG_FP64_RESCUE): the backward rolls head groups of 8
    in fp32 on the matrix cores, rolls the problems of the groups that rejects again one by one
    in fp64 on the row layout, and sends only what that rejects to the stable path.  The same
    forward under TTC_LQR_FLAG_FP64_FALLBACK sends every rejected group whole to the stable path
    (its count is 8 x the rejected groups), so the two-tier count lies strictly between 0 and it
    when all three tiers run.  Both agree with the fp64 oracle: one group per token (H = 8, head
    sums written directly) and two (H = 16: group sums from the per-problem partials of the second
    tier and the stable path, then head sums).  d = 32: the config-5 problems zero-padded to
    d = 24 (an equivalent problem; the solver pads it to its d = 32 kernels)."""
    import ttc.solvers.hip_lqr as hl
    from ttc.solvers._lib import FLAG_FP64_FALLBACK
    ins = layer_solver_inputs(5, make_x(5, n_tokens=16 * H // 8, seed=31))
    if H != 8:
        ins = _regroup_heads(ins, H)
    if d != 16:
        ins = [t.float() for t in hl._pad_inputs([t.double() for t in ins], 16, 16, 24)]
    T = 1024
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(9)).double().numpy()
    ref = solve_grads(pb, dU)
    print(f"[two-tier d={d} H={H}] N={pb.N} T={T}", flush=True)
    tiers = run_hip(ins, T, dU, grad_limit=math.inf)
    monkeypatch.setattr(hl, "riccati_flags", lambda precision, T_, Dp: FLAG_FP64_FALLBACK)
    groups = run_hip(ins, T, dU, grad_limit=math.inf)
    print(f"   stable path: two tiers {tiers['_fallback']}, whole groups {groups['_fallback']} of {pb.P}",
          flush=True)
    assert groups["_fallback"] % 8 == 0
    assert 0 < tiers["_fallback"] < groups["_fallback"]
    for label, out in (("two tiers", tiers), ("whole groups", groups)):
        errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES}
        print(f"   {label}: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
        assert all(v <= TOL for v in errs.values()), (label, errs)


def test_rescue_v1_slots_cut_the_stable_path(monkeypatch):
    """TTC_LQR_FLAG_RESCUE_V1 at T = 1024 on config-5b token scales: the forward's fp64 rescue keeps
    the fp64 V_1 / Quu_0 of the problems it recomputes, and the backward's fp64 second rollout tier
    starts those problems from them instead of their fp32 roundings.  Some then pass its
    certificate and skip the stable path: fewer problems take it than without the slots, and both
    runs agree with the fp64 oracle."""
    import ttc.solvers.hip_lqr as hl
    ins = layer_solver_inputs("5b", make_x("5b", n_tokens=64, seed=3))
    T = 1024
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(8)).double().numpy()
    ref = solve_grads(pb, dU)
    orig = hl._rescue_v1
    outs = {}
    for on in (False, True):
        monkeypatch.setattr(hl, "_rescue_v1", lambda flags, Dp, on=on: on and orig(flags, Dp))
        print(f"[rescue-v1 cfg5b T={T} slots={on}]", flush=True)
        outs[on] = run_hip(ins, T, dU, grad_limit=math.inf)
        errs = {k: _relerr(outs[on][k], ref[k]) for k in ["u"] + NAMES}
        print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()) + f"  fallback={outs[on]['_fallback']}",
              flush=True)
        assert all(v <= TOL for v in errs.values()), errs
    assert outs[True]["_fallback"] < outs[False]["_fallback"]


def test_rescue_gains_are_the_oracle_gains():
    """TTC_LQR_FLAG_RESCUE_GAINS (with _RESCUE_V1, _FP64_RESCUE) at T = 1024 on config-5b token
    scales, through the C ABI: the forward's fp64 rescue keeps every gain K_t of the problems in
    its first slots, after the fp64 V_1 / Quu_0 record.  Each kept problem's gains are the fp64
    oracle's (the Riccati sweep, lin_solver_lqr.py:155-185) to 1e-6 of its largest gain, at every
    step; problems without a slot are the ones the symplectic sweep accepted."""
    from ttc.solvers._lib import FLAG_FP64_RESCUE, FLAG_RESCUE_GAINS, FLAG_RESCUE_V1, lib
    from oracle.lqr64 import _riccati
    ins = [t.float().contiguous() for t in layer_solver_inputs("5b", make_x("5b", n_tokens=32, seed=3))]
    N, H, d = ins[0].shape
    T, P = 1024, N * H
    flags = FLAG_FP64_RESCUE | FLAG_RESCUE_V1 | FLAG_RESCUE_GAINS
    a256 = lambda n: (n + 255) // 256 * 256  # noqa: E731
    sb = lib.ttc_lqr_stash_bytes(N, H, d, d, T)
    rec = lib.ttc_lqr_rescue_stash_bytes(N, H, d, d)
    gb = lib.ttc_lqr_rescue_gains_bytes(N, H, d, d, T)
    nslot = min(P, max(64, P // 8))
    ngslot = min(nslot, max(64, P // 16))
    assert gb == a256(8 * ngslot * T * 256)
    dev = torch.device("cuda:0")
    xs = [t.to(dev) for t in ins]
    u = torch.empty(N, H, d, device=dev)
    st = torch.zeros((a256(sb) + rec + gb) // 4, device=dev)
    nws = lib.ttc_lqr_forward_workspace_bytes(N, H, d, d, T, flags)
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"[rescue-gains cfg5b] N={N} H={H} T={T} slots={nslot} gain slots={ngslot}", flush=True)
    rc = lib.ttc_lqr_forward_ws(*[t.data_ptr() for t in xs], N, H, d, d, T, flags, u.data_ptr(), st.data_ptr(),
                                ws.data_ptr(), nws, status.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0 and int(status.item()) & 4, (rc, int(status.item()))
    raw = st.view(torch.uint8)
    slot_of = raw[a256(sb):a256(sb) + 4 * P].view(torch.int32).cpu().numpy()
    gains = raw[a256(sb) + rec:a256(sb) + rec + 8 * ngslot * T * 256].view(torch.float64)
    kept = [(p, int(k)) for p, k in enumerate(slot_of) if 0 <= k < ngslot]
    assert kept and all(k < nslot for _, k in kept) and len({k for _, k in kept}) == len(kept)
    assert np.all((slot_of == -1) | ((slot_of >= 0) & (slot_of < nslot)))
    K, _ = _riccati(LQRProblem(*ins, T), keep_gains=True)  # [T, P, du, d]
    worst = 0.0
    for p, k in kept:
        g = gains[k * T * 256:(k + 1) * T * 256].view(T, 16, 16).cpu().numpy()
        ref = K[:, p]
        worst = max(worst, float(np.abs(g - ref).max() / np.abs(ref).max()))
    print(f"   kept {len(kept)} problems: worst gain error {worst:.1e}", flush=True)
    assert worst <= 1e-6


def test_rescue_gains_read_by_the_stable_path(monkeypatch):
    """Config-5b token scales, T = 1024, 64 tokens: with and without the forward's kept fp64 gains
    (TTC_LQR_FLAG_RESCUE_GAINS), u and all nine gradients agree with the fp64 oracle, and the same
    number of problems takes the stable path (the gains change how it gets them, not who needs
    them; the rescue list's atomic order may move one or two)."""
    import ttc.solvers.hip_lqr as hl
    ins = layer_solver_inputs("5b", make_x("5b", n_tokens=64, seed=3))
    T = 1024
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(8)).double().numpy()
    ref = solve_grads(pb, dU)
    fb = {}
    for on in (False, True):
        monkeypatch.setattr(hl, "_keep_rescue_gains", lambda dev, policy, nbytes, on=on: on)
        print(f"[rescue-gains cfg5b T={T} kept={on}]", flush=True)
        out = run_hip(ins, T, dU, grad_limit=math.inf)
        errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES}
        print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()) + f"  fallback={out['_fallback']}",
              flush=True)
        assert all(v <= TOL for v in errs.values()), errs
        fb[on] = out["_fallback"]
    assert fb[True] > 0 and abs(fb[True] - fb[False]) <= 2, fb


@pytest.mark.parametrize("slots", [False, True])
def test_certificate_rejects_trajectories_beyond_fp32(slots, monkeypatch):
    """Config-5b token 29207 (of the 32,768-token sample, seed 3), T = 1024: started from the
    forward's fp64 V_1, head 3's fp64 Hamiltonian rollout grows to |lambda| ~ 1e52 -- finite in fp64,
    beyond the fp32 range -- while its gradient sums stay below 1e34.  The certificate compares
    residual and magnitude as fp32 values, where both are +inf; it must reject such a problem
    (inf <= tau * inf holds) and leave it to the stable path.  Every output within 1e-4 of the fp64
    oracle, with and without the rescue's fp64 slots."""
    import ttc.solvers.hip_lqr as hl
    full = layer_solver_inputs("5b", make_x("5b", n_tokens=32768, seed=3))
    ins = [t[29207:29208].clone() for t in full]
    del full
    orig = hl._rescue_v1
    monkeypatch.setattr(hl, "_rescue_v1", lambda flags, Dp: slots and orig(flags, Dp))
    check_case(f"cfg5b token 29207 slots={slots}", ins, 1024, seed=4, grad_limit=math.inf)


@pytest.mark.parametrize("cfg,n_tok", [(5, 64), ("5b", 64)])
def test_forward_workspace_packs_the_fp64_rescue(cfg, n_tok):
    """Long horizons (T = 1024, FP64_RESCUE): ttc_lqr_forward_ws lists the problems the
    symplectic sweep rejects and sweeps them in fp64 on the matrix cores (Cholesky steps, the
    LU row-layout sweep finishing any whose Cholesky breaks down); ttc_lqr_forward (no
    workspace) sweeps each marked problem with the LU row-layout sweep.  Both rescue some
    problems (status bit TTC_LQR_STATUS_RESCUED), and u and the V_1 / Quu_0 stash agree to
    within 1e-5 of their largest magnitude (two fp64 factorisations, rounded to fp32)."""
    from ttc.solvers._lib import FLAG_FP64_RESCUE, lib
    x = make_x(cfg, n_tokens=n_tok, seed=17)
    ins = [t.float().contiguous().cuda() for t in layer_solver_inputs(cfg, x)]
    N, H, d = ins[0].shape
    T = 1024
    P = N * H
    ptrs = [t.data_ptr() for t in ins]
    stream = torch.cuda.current_stream().cuda_stream
    nws = lib.ttc_lqr_forward_workspace_bytes(N, H, d, d, T, FLAG_FP64_RESCUE)
    assert nws == 4 * (P + 64)
    print(f"[fwd-ws cfg{cfg}] N={N} H={H} T={T}", flush=True)
    outs = []
    for with_ws in (False, True):
        u = torch.full((N, H, d), 7.0, device="cuda")
        st = torch.zeros(lib.ttc_lqr_stash_bytes(N, H, d, d, T) // 4, device="cuda")
        status = torch.zeros(1, device="cuda", dtype=torch.int32)
        ws = torch.full((nws,), 0xAB, device="cuda", dtype=torch.uint8)
        rc = lib.ttc_lqr_forward_ws(*ptrs, N, H, d, d, T, FLAG_FP64_RESCUE, u.data_ptr(), st.data_ptr(),
                                    ws.data_ptr() if with_ws else None, nws if with_ws else 0, status.data_ptr(),
                                    stream)
        assert rc == 0
        torch.cuda.synchronize()
        outs.append((u.cpu(), st.cpu(), int(status.item())))
    (u0, s0, f0), (u1, s1, f1) = outs
    assert torch.isfinite(u0).all() and torch.isfinite(u1).all()
    assert f0 == f1 == 4, (f0, f1)  # TTC_LQR_STATUS_RESCUED only
    du = ((u1 - u0).abs().max() / u0.abs().max()).item()
    ds = ((s1 - s0).abs().max() / s0.abs().max()).item()
    changed = int((u1 != u0).any(-1).sum())
    print(f"   u rel diff {du:.2e}, stash rel diff {ds:.2e}, {changed} of {P} problems not bitwise equal",
          flush=True)
    assert du <= 1e-5 and ds <= 1e-5


def test_rescue_routes_at_scale_and_a_problem_beyond_fp64():
    """Config-5b scales at 12,288 tokens (98,304 problems, T = 1024, ~5.8 k rescued).  The listed
    fp64 rescue on the matrix cores (the default, with the forward's workspace) and the unlisted
    one (no workspace: the LU row-layout sweep) agree on u and the fp32 V_1 / Quu_0 stash to 1e-5
    of their largest magnitude.  The exceptions are problems where they disagree by more than 1e-4
    of the problem's own |u|: at most 3, and here only problem 5086.  That problem is beyond
    fp64: against its 40-digit u (tests/golden/mp_cfg5b_beyond_fp64.npz), the listed route misses
    by 0.23 of its |u| max, the row-layout route by 0.095 and the fp64 oracle by 0.33.  The
    bounds below pin those figures, the limit the accuracy notes record."""
    from ttc.solvers._lib import FLAG_FP64_RESCUE, lib
    fx = np.load(os.path.join(GOLDEN, "mp_cfg5b_beyond_fp64.npz"))
    x = make_x("5b", n_tokens=int(fx["n_tokens"]), seed=int(fx["seed"]))
    cpu = layer_solver_inputs("5b", x)
    p = int(fx["p"])
    n, h = divmod(p, 8)
    assert np.array_equal(cpu[0][n, h].numpy(), fx["in_A_diag"].reshape(-1))  # the same problem
    ins = [t.float().contiguous().cuda() for t in cpu]
    N, H, d = ins[0].shape
    T, P = int(fx["T"]), N * H
    nws = lib.ttc_lqr_forward_workspace_bytes(N, H, d, d, T, FLAG_FP64_RESCUE)
    stream = torch.cuda.current_stream().cuda_stream
    print(f"[rescue routes cfg5b] N={N} H={H} T={T}", flush=True)
    outs = []
    for wsb in (0, nws):
        u = torch.full((N, H, d), 7.0, device="cuda")
        st = torch.zeros(lib.ttc_lqr_stash_bytes(N, H, d, d, T) // 4, device="cuda")
        status = torch.zeros(1, device="cuda", dtype=torch.int32)
        ws = torch.zeros(nws, device="cuda", dtype=torch.uint8)
        rc = lib.ttc_lqr_forward_ws(*[t.data_ptr() for t in ins], N, H, d, d, T, FLAG_FP64_RESCUE, u.data_ptr(),
                                    st.data_ptr(), ws.data_ptr() if wsb else None, wsb, status.data_ptr(), stream)
        assert rc == 0
        torch.cuda.synchronize()
        outs.append((u.cpu().double().reshape(P, d), st.cpu(), int(status.item())))
    (u0, s0, f0), (u1, s1, f1) = outs
    assert f0 == f1 == 4 and torch.isfinite(u0).all() and torch.isfinite(u1).all()
    own = (u1 - u0).abs().amax(1) / u0.abs().amax(1).clamp_min(1e-30)
    apart = torch.nonzero(own > 1e-4).flatten().tolist()
    keep = torch.ones(P, dtype=torch.bool)
    keep[apart] = False
    du = float((u1 - u0)[keep].abs().max() / u0.abs().max())
    per = lambda st: torch.cat([st[:P * d * d].reshape(P, -1), st[P * d * d:].reshape(P, -1)], 1)  # noqa: E731
    ds = float((per(s1) - per(s0))[keep].abs().max() / s0.abs().max())
    true = torch.from_numpy(fx["out_u"].reshape(-1))
    err = {k: float((v[p] - true).abs().max() / true.abs().max()) for k, v in (("listed", u1), ("row", u0))}
    print(f"   routes apart on {apart}; elsewhere u {du:.1e} stash {ds:.1e}; problem {p} against 40 digits: "
          f"listed {err['listed']:.3f}, row-layout {err['row']:.3f}", flush=True)
    assert len(apart) <= 3 and du <= 1e-5 and ds <= 1e-5
    assert err["listed"] <= 0.25 and err["row"] <= 0.1


@pytest.mark.parametrize("cfg,n_tok,d_pad", [(4, 1, None), (4, 1, 24)])
def test_fp64_stable_backward_d32(cfg, n_tok, d_pad):
    """The fp64 stable path at d = 32 (lqr_bwd_kernel<32, double>): a config-4 slice, and the
    same problems cut to d = du = 24 (padded to 32 inside), both against the fp64 oracle."""
    x = make_x(cfg, n_tokens=n_tok, seed=9)
    ins = layer_solver_inputs(cfg, x)
    if d_pad is not None:
        k = d_pad
        A, B, Q, R, Qf, lA, lB, lQ, h0 = ins
        ins = [t.contiguous() for t in (A[..., :k], B[:, :k, :k], Q[:, :k, :k], R[..., :k], Qf[:, :, :k, :k], lA,
                                        lB[..., :k], lQ[..., :k], h0[..., :k])]
    out = check_case(f"cfg{cfg}-fp64-stable-d{d_pad or 32}", ins, CONFIGS[cfg]["T"], precision="fp64", stable=True)
    assert out["_fallback"] == out["u"].shape[0] * out["u"].shape[1]


def _guard_inputs(H):
    """Two tokens; head 0 of each is a long, barely discounted problem with a small A_diag (the
    (t+1) factor makes its log-discount gradients exceed every gradient the reference's guard
    covers), the other heads copy head 1.  d_u is nonzero on head 0 only, so every other head's
    adjoint, hence its gradient contribution, is zero: the head sums of grad_B / grad_Q are
    head 0's, and the magnitudes are the same for every head count."""
    ins = bench_solver_inputs(2, 2, 16, seed=5)
    ins[0] = ins[0] * 0.1
    ins[5], ins[6], ins[7] = ins[5] * 0.005, ins[6] * 0.005, ins[7] * 0.005
    idx = torch.tensor([0] + [1] * (H - 1))
    ins = [t if k in (1, 2) else t[:, idx].contiguous() for k, t in enumerate(ins)]
    dU = np.zeros((2, H, 16))
    dU[:, 0] = 1.0
    return ins, dU


@pytest.mark.parametrize("H,precision,stable", [(8, "fp32", False), (16, "fp32", False), (2, "fp32", False),
                                                (8, "fp32", True), (8, "fp32-row", False)])
def test_grad_guard_covers_the_reference_six(H, precision, stable):
    """The backward's magnitude guard (fused_lqr.py:243-246) covers the gradients of A_diag, B,
    Q, R_inv, Q_f and h0: with a limit between their largest entry and the largest log-discount
    gradient nothing is raised; at half their largest entry the RuntimeError is.  H = 8: head
    group = token (sums stored directly); H = 16: group sums then head sums; H = 2: row-layout
    rollout; stable path; row-layout kernels."""
    T = 256
    ins, dU = _guard_inputs(H)
    g = run_hip(ins, T, dU, grad_limit=math.inf, precision=precision, stable=stable)
    guarded = max(np.abs(g[k]).max() for k in ("A_diag", "B", "Q", "R_inv", "Q_f", "h0"))
    lg = max(np.abs(g[k]).max() for k in ("lgA", "lgB", "lgQ"))
    print(f"H={H} {precision} stable={stable}: guarded max {guarded:.3e}, log-discount max {lg:.3e}", flush=True)
    assert lg > 1.2 * guarded
    run_hip(ins, T, dU, grad_limit=math.sqrt(lg * guarded), precision=precision, stable=stable)
    with pytest.raises(RuntimeError, match="backward"):
        run_hip(ins, T, dU, grad_limit=0.5 * guarded, precision=precision, stable=stable)


def _A0_zero_inputs(H, d=16, seed=3):
    """a_i = -exp(-lgA) for every state of the first problem: A_0 = diag(1 + a exp(lgA)) = 0."""
    ins = [t.clone() for t in bench_solver_inputs(2, H, d, seed=seed)]
    ins[0][0, 0] = -torch.exp(-ins[5][0, 0])
    return ins


@pytest.mark.parametrize("d,H,precision,stable", [(16, 8, "fp32", False), (16, 8, "fp32-riccati", False),
                                                  (16, 8, "fp32-row", False), (16, 8, "fp64", False),
                                                  (16, 8, "fp32", True), (16, 2, "fp32", False),
                                                  (32, 8, "fp32", False), (64, 8, "fp32", False)])
def test_A0_zero(d, H, precision, stable):
    """A_0 = 0 (a_i = -exp(-lgA), which the host can set; the reference's fused kernels divide by A_k):
    symplectic, per-step Riccati, row-layout and fp64 forwards, the head-group backward (whose
    Hamiltonian rollout divides by A_t from t = 1 on, so A_0 = 0 is reachable) and the stable
    path, against the fp64 oracle."""
    check_case(f"A0=0 d{d} H{H}", _A0_zero_inputs(H, d), 24, precision=precision, stable=stable)


def test_fused_lqr_solve_reference_signature():
    """fused_lqr_solve(..., h0, T, inv_guard) as the reference calls it (fused_lqr.py:294-304):
    inv_guard=True is accepted and changes nothing (the reference routes it into an unused slot)."""
    from ttc.solvers import fused_lqr_solve
    ins = [t.cuda() for t in bench_solver_inputs(2, 8, 16, seed=2)]
    a = fused_lqr_solve(*ins, 16, True)
    b = fused_lqr_solve(*ins, 16)
    assert torch.equal(a, b)


@pytest.mark.parametrize("extra", [(), (False,), ("LU",), ("LU", False), ("LU", True)])
def test_fused_lqr_solve_func_reference_slots(extra):
    """FusedLQRSolveFunc.apply with the reference's positional slots (fused_lqr.py:255-291):
    (..., h0, T[, cache_level[, inv_guard]]), including the reference's own fused_lqr_solve call
    that puts inv_guard in the cache_level slot; forward and the nine gradients of the backward
    are bitwise those of hip_lqr_solve, and within 1e-4 of the fp64 oracle."""
    from ttc.solvers import FusedLQRSolveFunc
    ins = bench_solver_inputs(2, 8, 16, seed=2)
    T = 24
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(3))
    ref = run_hip(ins, T, dU.double().numpy())
    xs = [t.cuda().requires_grad_(True) for t in ins]
    u = FusedLQRSolveFunc.apply(*xs, T, *extra)
    (u * dU.cuda()).sum().backward()
    assert torch.equal(u.detach().cpu().double(), torch.from_numpy(ref["u"]))
    for n, t in zip(NAMES, xs):
        assert torch.equal(t.grad.cpu().double(), torch.from_numpy(ref[n])), n
    ref64 = solve_grads(pb, dU.double().numpy())
    for k in ["u"] + NAMES:
        assert _relerr(ref[k], ref64[k]) <= TOL, k


def test_layer_parameter_gradients_match_oracle():
    """TTCLayer(solver_impl="hip") (factored solve, fused rescale) on the GPU: gradients of
    in_proj, out_proj, Bs and Qs against fp64 autograd of the oracle layer around the fp64
    oracle solve, T = 16."""
    from ttc import TTCLayer
    from _layer_oracle import oracle_layer_grads
    torch.manual_seed(1)
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="hip").cuda()
    x = torch.randn(3, 5, 32, generator=torch.Generator().manual_seed(2))
    dy = torch.randn(3, 5, 32, generator=torch.Generator().manual_seed(3))
    y = layer(x.cuda(), T=16)
    (y * dy.cuda()).sum().backward()
    ref = oracle_layer_grads(layer, x, dy, 16)
    for name, p in (("in_proj", layer.in_proj.weight), ("out_proj", layer.out_proj.weight), ("Bs", layer.Bs),
                    ("Qs", layer.Qs)):
        e = _relerr(p.grad.cpu().numpy(), ref[name])
        print(f"layer grad {name}: {e:.1e}", flush=True)
        assert e <= TOL, name


@pytest.mark.parametrize("T", [64, 256])
def test_layer_default_path_on_config5_scales(T):
    """TTCLayer(solver_impl="hip") with its defaults (factored solve, fused l2_norm rescale,
    precision "auto") on 512 config-5 tokens (per-token log-normal scales, 4,096 problems):
    the output and the gradients of in_proj, out_proj, Bs and Qs against fp64 autograd of the
    oracle layer around the fp64 oracle solve."""
    from ttc import TTCLayer
    from _layer_oracle import oracle_layer_grads
    torch.manual_seed(5)
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="hip").cuda()
    x = make_x(5, n_tokens=512, seed=31 + T)
    dy = torch.randn(512, 32, generator=torch.Generator().manual_seed(T))
    print(f"[layer cfg5-scales T={T}] x {tuple(x.shape)}", flush=True)
    y = layer(x.cuda(), T=T)
    (y * dy.cuda()).sum().backward()
    ref = oracle_layer_grads(layer, x, dy, T)
    for name, p in (("in_proj", layer.in_proj.weight), ("out_proj", layer.out_proj.weight), ("Bs", layer.Bs),
                    ("Qs", layer.Qs)):
        e = _relerr(p.grad.cpu().numpy(), ref[name])
        print(f"   layer grad {name}: {e:.1e}", flush=True)
        assert e <= TOL, name


@pytest.mark.parametrize("T", [64, 1024])
@pytest.mark.parametrize("key,factored", [("riccati", None), ("kkt", None), ("fused", None), ("fused", False)])
def test_layer_reference_keys_on_gpu(key, factored, T):
    """TTCLayer(solver_impl=key).cuda() for the reference's registry keys (ttc_layer.py:18-22):
    "riccati" / "kkt" (HIP kernels with Riccati steps; kkt with the stable backward for every
    problem; fp64 sweeps at T = 1024), "fused" on its default factored path and on the
    reference's materialised one (fused_lqr_solve / FusedLQRSolveFunc): the gradients of
    in_proj, out_proj, Bs and Qs against fp64 autograd of the oracle layer, T = 64 and 1024."""
    from ttc import TTCLayer
    from _layer_oracle import oracle_layer_grads
    torch.manual_seed(7)
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl=key, factored=factored).cuda()
    x = torch.randn(3, 4, 32, generator=torch.Generator().manual_seed(T + 1))
    dy = torch.randn(3, 4, 32, generator=torch.Generator().manual_seed(T + 2))
    print(f"[layer key={key} factored={layer.factored} T={T}]", flush=True)
    y = layer(x.cuda(), T=T)
    (y * dy.cuda()).sum().backward()
    ref = oracle_layer_grads(layer, x, dy, T)
    for name, p in (("in_proj", layer.in_proj.weight), ("out_proj", layer.out_proj.weight), ("Bs", layer.Bs),
                    ("Qs", layer.Qs)):
        e = _relerr(p.grad.cpu().numpy(), ref[name])
        print(f"   layer grad {name}: {e:.1e}", flush=True)
        assert e <= TOL, name


@pytest.mark.parametrize("T,cfg,n_tok,seed", [(64, 5, 16, 5), (1024, 5, 8, 5), (64, 2, 8, 1)])
@pytest.mark.parametrize("name", ["direct_lqr_solve", "kkt_lqr_solve"])
def test_reference_solvers_on_cuda_tensors(name, T, cfg, n_tok, seed):
    """direct_lqr_solve / kkt_lqr_solve (ttc.solvers.torch_lqr, the reference's module path and
    signature, torch_lqr.py:93-140) on CUDA tensors: u and the nine gradients against the fp64
    oracle on config-5 token scales (T = 64 and 1024) and a config-2 slice.  They keep the
    reference's 1e6 guard, so d_u is scaled (gradients are linear in it) to put the largest
    guarded gradient at 1e3."""
    import ttc.solvers.torch_lqr as TL
    fn = getattr(TL, name)
    ins = layer_solver_inputs(cfg, make_x(cfg, n_tokens=n_tok, seed=seed))
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed + 3)).double().numpy()
    ref = solve_grads(pb, dU)
    s = min(1.0, 1e3 / max(np.abs(ref[k]).max() for k in ("A_diag", "B", "Q", "R_inv", "Q_f", "h0")))
    xs = [t.cuda().requires_grad_(True) for t in ins]
    u = fn(*xs, T)
    (u * torch.from_numpy(dU * s).float().cuda()).sum().backward()
    errs = {"u": _relerr(u.detach().cpu().numpy(), ref["u"])}
    for n, t in zip(NAMES, xs):
        errs[n] = _relerr(t.grad.cpu().numpy(), ref[n] * s)
    print(f"[{name} cfg{cfg} T={T}] d_u scale {s:.1e} " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()),
          flush=True)
    assert max(errs.values()) <= TOL, errs


def test_padding_odd_dims_and_ragged_problem_count():
    """d=12, du=8 (padded to 16 inside), N*H = 21 problems (not a multiple of the block)."""
    g = torch.Generator().manual_seed(11)
    N, H, d, du, T = 7, 3, 12, 8, 9
    ins = bench_solver_inputs(N, H, d, seed=4)
    B = torch.randn(N, d, du, generator=g) * 0.5
    R_inv = torch.nn.functional.softplus(torch.rand(N, H, du, generator=g))
    lgB = -torch.nn.functional.softplus(torch.randn(N, H, du, generator=g)) - 0.3
    ins = [ins[0], B, ins[2], R_inv, ins[4], ins[5], lgB, ins[7], ins[8]]
    check_case("pad", ins, T)


def _random_case(seed):
    """A seeded draw of (N, H, d, du, T, precision) and inputs of the bench distribution
    with a rectangular B: every padded width (16 / 32 / 64), head counts that do and do not
    form head groups of 8, T from 1 up, and each fp32 kernel family."""
    rng = np.random.default_rng(seed)
    d = int(rng.integers(3, 65))
    du = int(rng.integers(2, 65))
    H = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 24]))
    N = int(rng.integers(1, 4))
    T = int(rng.integers(3, 65)) if rng.random() < 0.75 else int(rng.choice([1, 2]))
    precision = str(rng.choice(["fp32", "fp32-riccati", "fp32-row"]))
    g = torch.Generator().manual_seed(seed)
    ins = bench_solver_inputs(N, H, max(d, du), seed=seed)
    A, _, Q, _, Qf, lgA, _, lgQ, h0 = ins
    B = torch.randn(N, d, du, generator=g) / math.sqrt(max(d, du))
    R_inv = torch.nn.functional.softplus(torch.rand(N, H, du, generator=g))
    lgB = -torch.nn.functional.softplus(torch.randn(N, H, du, generator=g)) - 1.328
    ins = [A[..., :d], B, Q[:, :d, :d], R_inv, Qf[:, :, :d, :d], lgA, lgB, lgQ[..., :d], h0[..., :d]]
    return [t.contiguous() for t in ins], T, precision


@pytest.mark.parametrize("seed", range(20))
def test_random_shapes(seed):
    """Seeded random shapes and kernels against the fp64 oracle (u and all nine gradients)."""
    ins, T, precision = _random_case(1000 + seed)
    out = check_case(f"rand{seed}", ins, T, precision=precision, grad_limit=math.inf)
    assert np.isfinite(out["u"]).all()


def _indefinite_terminal_inputs(s, seed=2, H=4):
    """Problem 1 of 8 gets Q_f = -s I with a strong, barely discounted B: Quu turns
    indefinite (nonsingular), so the matrix-core kernel's Cholesky guard fires for the
    wave holding problems 0-3 and that wave finishes on the pivoted row-layout sweep,
    while problems 4-7 stay on the matrix cores.  s = 2: indefinite from the last step
    (t = T-1) on; s = 0.2: positive definite until t = 0 (a mid-horizon switch)."""
    ins = bench_solver_inputs(2, H, 16, seed=seed)
    g = torch.Generator().manual_seed(seed)
    B = torch.randn(2, 16, 16, generator=g) * 0.25
    lgB = torch.full((2, H, 16), -0.01)
    Qf = ins[4].clone()
    Qf[0, 1] = -s * torch.eye(16)
    return [ins[0], B, ins[2], ins[3], Qf, ins[5], lgB, ins[7], ins[8]]


@pytest.mark.parametrize("s", [2.0, 0.2])
@pytest.mark.parametrize("stash", ["always", "never"])
@pytest.mark.parametrize("precision", ["fp32", "fp32-riccati"])
def test_indefinite_Quu_switches_to_pivoted_sweep(s, stash, precision):
    check_case(f"indef{s}", _indefinite_terminal_inputs(s), 6, stash=stash, precision=precision)


@pytest.mark.parametrize("s", [2.0, 0.2])
@pytest.mark.parametrize("stash", ["always", "never"])
def test_head_group_backward_with_indefinite_Quu0(s, stash):
    """H = 8: the d = 16 head-group Hamiltonian backward on a group whose problem 1 has
    Q_f = -s I, so that its Quu_0 is indefinite; s = 2 sends the group to the stable path,
    s = 0.2 stays on the head-group kernel, whose solve of Quu_0 w_0 = -d_u (elimination
    without row exchanges, valid for positive definite Quu_0) then meets a negative pivot
    and is redone with partial pivoting."""
    check_case(f"indef-h8-{s}", _indefinite_terminal_inputs(s, H=8), 6, stash=stash)


@pytest.mark.parametrize("s", [2.0, 0.2])
@pytest.mark.parametrize("stable", [True, False])
def test_long_horizon_indefinite_Quu_finishes_on_lu(s, stable):
    """T = 512 (FP64_RESCUE): problem 1 has Q_f = -s I, so its Quu turns indefinite.  Through
    the stable path for every problem, the fp64 matrix-core gain sweep's Cholesky guard fires
    for it and the LU row-layout sweep finishes it (the other problems keep their Cholesky
    gains); on the default path the same holds for the forward's fp64 rescue when the
    symplectic certificate rejects it.  u and every gradient against the fp64 oracle."""
    check_case(f"indef-T512-{s}", _indefinite_terminal_inputs(s, H=4), 512, grad_limit=math.inf, stable=stable)


@pytest.mark.parametrize("T", [64, 256])
def test_symplectic_certificate_on_stress_inputs(T):
    """Config-5 inputs: the d = 16 symplectic sweep's certificate (conditioning of Y1,
    symmetry of V_1) rejects the ill-conditioned problems (about 8 % of them), which the
    rescue pass recomputes with the pivoted row-layout sweep; u and every gradient match
    the fp64 oracle and the per-step Riccati kernel."""
    x = make_x(5, n_tokens=16, seed=13)
    ins = layer_solver_inputs(5, x)
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(4)).double().numpy()
    sym = run_hip(ins, T, dU, grad_limit=math.inf, precision="fp32")
    ric = run_hip(ins, T, dU, grad_limit=math.inf, precision="fp32-riccati")
    ref = solve_grads(pb, dU)
    for k in ["u"] + NAMES:
        assert _relerr(sym[k], ref[k]) <= TOL, k
        assert _relerr(sym[k], ric[k]) <= TOL, k


@pytest.mark.parametrize("T,seed", [(64, 21), (256, 23)])
def test_default_precision_on_config5_scales_below_fp64_horizon(T, seed):
    """The default precision on config-5 token scales at horizons below 512, on samples large
    enough (512 tokens, 4,096 problems) to hold the ill-conditioned problems that fp32 Riccati
    values cannot resolve: the symplectic certificate rejects them, the forward recomputes them
    in fp64 (TTC_LQR_FLAG_FP64_FALLBACK), and the problems the backward's certificate rejects
    take the fp64 stable path.  u and all nine gradients within 1e-4 of the fp64 oracle (the
    fp32-only tiers missed it on these samples by up to 8e-3 at T = 64 and 0.2 at T = 256)."""
    x = make_x(5, n_tokens=512, seed=seed)
    out = check_case(f"cfg5-scales T={T}", layer_solver_inputs(5, x), T, seed=seed, grad_limit=math.inf)
    assert out["_fallback"] > 0  # the sample exercises the backward's fallback


@pytest.mark.parametrize("cfg,n_tok,T,seed", [(2, 16, 64, 1), (5, 16, 64, 5), (5, 4, 1024, 5)])
def test_deferred_status_equals_sync(cfg, n_tok, T, seed):
    """status_check="deferred": the forward returns without reading its status word, the backward
    reads it (and picks the backward's arithmetic from it, as the synchronous forward does);
    u and the nine gradients bit for bit those of the default mode, on nominal inputs and on
    config-5 scales whose forward rescues problems in fp64."""
    from ttc.solvers.hip_lqr import _deferred, check_deferred_status
    check_deferred_status()
    ins = layer_solver_inputs(cfg, make_x(cfg, n_tokens=n_tok, seed=seed))
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed)).double().numpy()
    a = run_hip(ins, T, dU, grad_limit=math.inf)
    solve = _solver()
    xs = [t.cuda().float().requires_grad_(True) for t in ins]
    u = solve(*xs, T, grad_limit=math.inf, status_check="deferred")
    assert len(_deferred) == 1
    (u * torch.as_tensor(dU, device="cuda", dtype=u.dtype)).sum().backward()
    assert len(_deferred) == 0  # the backward read it
    assert torch.equal(u.detach().cpu().double(), torch.from_numpy(a["u"]))
    for n, t in zip(NAMES, xs):
        assert torch.equal(t.grad.cpu().double(), torch.from_numpy(a[n])), n


def test_deferred_status_raises_later():
    """A NaN input under status_check="deferred": the forward returns; check_deferred_status()
    raises the reference's forward RuntimeError, and so does the backward of such a forward."""
    from ttc.solvers.hip_lqr import check_deferred_status
    ins = bench_solver_inputs(2, 8, 16, seed=1)
    ins[8] = ins[8].clone()
    ins[8][0, 0, 0] = float("nan")
    solve = _solver()
    check_deferred_status()
    with torch.no_grad():
        solve(*[t.cuda() for t in ins], 8, status_check="deferred")
    with pytest.raises(RuntimeError, match="forward recurrence"):
        check_deferred_status()
    check_deferred_status()  # forgotten once read
    xs = [t.cuda().requires_grad_(True) for t in ins]
    u = solve(*xs, 8, status_check="deferred")
    with pytest.raises(RuntimeError, match="forward recurrence"):
        u.sum().backward()


@pytest.mark.parametrize("cfg,T", [(2, 64), (5, 64)])
def test_deferred_forward_in_a_hip_graph(cfg, T):
    """With status_check="deferred" the forward makes no host synchronisation, so it can be
    recorded by HIP graph capture (torch.cuda.graph): replayed on three inputs copied into the
    captured input tensors, with eager work and synchronisations between the replays, each
    replay's u equals the eager forward on the same inputs bit for bit, and its status word
    (kept, re-read after each replay) reports the same rescue as the eager forward (config-5
    scales: problems recomputed in fp64 inside the graph)."""
    from ttc.solvers.hip_lqr import _deferred, check_deferred_status
    solve = _solver()
    draws = [layer_solver_inputs(cfg, make_x(cfg, n_tokens=16, seed=40 + k)) for k in range(4)]
    static = [t.cuda().float().contiguous() for t in draws[0]]
    check_deferred_status()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.no_grad():  # warm-up outside the capture
        solve(*static, T, status_check="deferred")
    torch.cuda.current_stream().wait_stream(side)
    check_deferred_status()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        u_graph = solve(*static, T, status_check="deferred")
    assert len(_deferred) == 1
    status_word = _deferred[0]
    rescued = 0
    for k in (1, 2, 3):
        for dst, src in zip(static, draws[k]):
            dst.copy_(src)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got, got_status = u_graph.clone(), int(status_word.item())
        check_deferred_status(keep=True)
        with torch.no_grad():
            ref = solve(*[t.cuda().float() for t in draws[k]], T)  # eager, synchronous status
        torch.cuda.synchronize()
        print(f"[graph cfg{cfg} replay {k}] status {got_status}", flush=True)
        assert torch.equal(got, ref), k
        assert got_status & 3 == 0
        rescued += got_status & 4
    assert (rescued > 0) == (cfg == 5)
    _deferred.clear()


@pytest.mark.parametrize("factored", [False, True])
def test_profiler_ranges_name_the_reference_stages(factored):
    """A torch.profiler trace of a forward + backward attributes the solver's time to ranges named
    after the reference's stages (fused_lqr.py:58,186,200): fwd:lqr_symplectic_rev_iter,
    bwd:lqr_symplectic_fwd_iter_diff, plus the host's status waits (and, through TTCLayer's factored
    path, the fused rescale's two ranges)."""
    from ttc import TTCLayer
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="hip", factored=factored).cuda()
    x = torch.randn(2, 3, 32, device="cuda")
    layer(x, T=8).sum().backward()  # warm-up outside the trace
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        layer(x, T=8).sum().backward()
    names = {e.name for e in prof.events()}
    want = {"fwd:lqr_symplectic_rev_iter", "bwd:lqr_symplectic_fwd_iter_diff", "fwd:ttc_lqr_status",
            "bwd:ttc_lqr_status"}
    if factored:
        want |= {"fwd:ttc_lqr_rescale", "bwd:ttc_lqr_rescale_backward"}
    print(sorted(n for n in names if ":" in n and ("fwd" in n or "bwd" in n)), flush=True)
    assert want <= names, want - names


def test_T1_closed_form():
    ins = bench_solver_inputs(3, 2, 16, seed=9)
    check_case("T1", ins, 1)


def test_stash_modes_bitwise_equal():
    x = make_x(2, n_tokens=8, seed=4)
    ins = layer_solver_inputs(2, x)
    dU = np.ones((8, 8, 16))
    a = run_hip(ins, 64, dU, stash="always")
    b = run_hip(ins, 64, dU, stash="never")
    for k in a:
        assert np.array_equal(a[k], b[k]), k


def test_nonsymmetric_Q_uses_symmetric_part():
    ins = bench_solver_inputs(2, 2, 16, seed=3)
    g = torch.Generator().manual_seed(5)
    skew = torch.randn(2, 16, 16, generator=g) * 0.01
    skew = skew - skew.transpose(-1, -2)
    Qns = ins[2] + skew
    solve = _solver()
    dev = torch.device("cuda:0")
    u_sym = solve(*[t.to(dev) for t in ins], 16)
    ins2 = list(ins)
    ins2[2] = Qns
    u_ns = solve(*[t.to(dev) for t in ins2], 16)
    torch.testing.assert_close(u_ns, u_sym, rtol=1e-5, atol=1e-6)


def test_nan_input_raises():
    ins = bench_solver_inputs(2, 2, 16, seed=1)
    ins[8] = ins[8].clone()
    ins[8][0, 0, 0] = float("nan")
    solve = _solver()
    with pytest.raises(RuntimeError, match="Numerical instability"):
        solve(*[t.cuda() for t in ins], 8)


def test_empty_batch():
    ins = [t[:0] for t in bench_solver_inputs(2, 2, 16, seed=1)]
    solve = _solver()
    u = solve(*[t.cuda() for t in ins], 8)
    assert u.shape == (0, 2, 16)


def test_layer_end_to_end_matches_oracle_layer():
    """TTCLayer(solver_impl='hip') == the oracle layer restatement with the fp64 solver."""
    from ttc import TTCLayer
    from oracle.layer_ref import front_end, back_end, LayerParams
    torch.manual_seed(0)
    layer = TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="hip").cuda()
    x = torch.randn(2, 5, 8, 32, device="cuda")
    y = layer(x, T=16)
    assert y.shape == (2, 5, 8, 32)
    # oracle: same weights, fp64 solve on CPU
    p = LayerParams(32, 32, 16, 8, 16, 16)
    p.W_in = layer.in_proj.weight.detach().cpu()
    p.W_out = layer.out_proj.weight.detach().cpu()
    p.Bs, p.Qs = layer.Bs.detach().cpu(), layer.Qs.detach().cpu()
    ins, lead = front_end(p, x.cpu())
    u64 = solve_u0(LQRProblem(*ins, 16))
    y_ref = back_end(p, torch.from_numpy(u64).float(), ins[8], lead)
    torch.testing.assert_close(y.cpu(), y_ref, rtol=1e-4, atol=1e-5)


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Outputs on which a fixture's recorded tolerance (4 x the fp64 oracle's own error against the
# higher-precision solve) lies far above what this solver achieves: bounds at about 2.5-3x the
# achieved error, so that a regression of the solver fails even where the fixture allows more.
# oracle_cfg5b_undiscounted: achieved 3.6e-4 (A_diag) and 2.1e-2 (B) with the fp64 Riccati
# sweep on the matrix cores, against recorded tolerances of 3.5e-2 and 0.13.
ACHIEVED_BOUNDS = {"oracle_cfg5b_undiscounted.npz": {"A_diag": 1e-3, "B": 5e-2}}


# mp_cfg5b_beyond_fp64.npz holds one problem's u only (its own test above)
@pytest.mark.parametrize("name", sorted(f for f in os.listdir(GOLDEN)
                                        if f.endswith(".npz") and f != "mp_cfg5b_beyond_fp64.npz"))
def test_against_committed_golden(name):
    """HIP solver vs the committed fixtures: fp64 oracle slices of every config and
    the two 50-digit mpmath stress problems (tests/golden/make_golden.py)."""
    z = np.load(os.path.join(GOLDEN, name))
    ins = [torch.from_numpy(z[f"in_{k}"]).float() for k in NAMES]
    T = int(z["T"])
    print(f"[golden {name}] {z['meta']}", flush=True)
    out = run_hip(ins, T, z["dU"], grad_limit=math.inf)
    errs = {k: _relerr(out[k], z[f"out_{k}"]) for k in ["u"] + NAMES}
    # 1e-4 (north_star) unless the fixture records a finite per-output tolerance derived from
    # the fp64 oracle's own measured error against a higher-precision solve of its problems
    # (tests/test_oracle.py re-measures it); never a lifted (infinite) one
    tol = {k: float(z[f"tol_{k}"]) if f"tol_{k}" in z.files else TOL for k in errs}
    assert all(np.isfinite(t) and t >= TOL for t in tol.values()), tol
    for k, b in ACHIEVED_BOUNDS.get(name, {}).items():
        tol[k] = min(tol[k], b)
    print("   achieved rel err " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    print("   tolerance        " + " ".join(f"{k}:{tol[k]:.1e}" for k in errs), flush=True)
    assert all(np.isfinite(out[k]).all() for k in errs), f"{name}: non-finite output"
    bad = {k: (v, tol[k]) for k, v in errs.items() if not (v <= tol[k])}
    assert not bad, f"{name}: rel err above tolerance: {bad}"


@pytest.mark.parametrize("cfg,n_tok", [(1, 8), (2, 8), (4, 1)])
def test_against_reference_riccati_and_kkt_restatements(cfg, n_tok):
    """The HIP solver against the reference's own pure-PyTorch solvers, restated op for op
    in fp32 (oracle/ref_torch.py: `riccati` = direct_lqr_solve with autograd,
    `kkt` = kkt_lqr_solve with its implicit-differentiation backward), on identical
    seeded inputs: u and all nine gradients within 1e-4 of both, and all three within
    1e-4 of the fp64 oracle.  (Q / Q_f gradients compared as symmetric gradients:
    riccati's autograd returns a non-symmetric one.)"""
    from oracle.ref_torch import riccati_solve, kkt_solve
    x = make_x(cfg, n_tokens=n_tok, seed=21)
    ins = layer_solver_inputs(cfg, x)
    T = CONFIGS[cfg]["T"]
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(2)).double().numpy()
    ref64 = solve_grads(pb, dU)
    hip = run_hip(ins, T, dU)

    def torch_ref(fn):
        xs = [t.detach().float().clone().requires_grad_(True) for t in ins]
        u = fn(*xs, T)
        (u * torch.from_numpy(dU).float()).sum().backward()
        out = {"u": u.detach().double().numpy()}
        for n, t in zip(NAMES, xs):
            g = t.grad.double().numpy()
            out[n] = 0.5 * (g + np.swapaxes(g, -1, -2)) if n in ("Q", "Q_f") else g
        return out

    for name, fn in (("riccati", riccati_solve), ("kkt", kkt_solve)):
        r = torch_ref(fn)
        errs = {k: _relerr(hip[k], r[k]) for k in ["u"] + NAMES}
        ref_errs = {k: _relerr(r[k], ref64[k]) for k in ["u"] + NAMES}
        print(f"[cfg{cfg} vs {name}] " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
        print(f"   {name} vs fp64: " + " ".join(f"{k}:{v:.1e}" for k, v in ref_errs.items()), flush=True)
        assert max(errs.values()) <= TOL, (name, errs)
        assert max(ref_errs.values()) <= TOL, (name, ref_errs)
