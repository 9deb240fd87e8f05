"""GPU parity of the factored solver (``hip_lqr_solve_factored`` -> ``ttc_lqr_forward_factored`` /
``ttc_lqr_backward_factored``): the layer's low-rank mixtures (``ttc/layers/ttc_layer.py:117-123``)
are expanded on the device per token chunk instead of materialising B, Q, Q_f.

Oracle: the factors are expanded in fp64 on the host, the fp64 oracle solves the LQR problems
and returns the gradients of B, Q, Q_f (``oracle/lqr64.solve_grads``), and the chain rule of
the (linear) expansion gives the coefficient and basis gradients exactly:
    d coeff_B[n,r] = <dB_n, Bs_r>,   d Bs_r = sum_n coeff_B[n,r] dB_n   (Q, Q_f likewise).
Tolerance: per tensor max|x - x64| / max|x64| <= 1e-4 (the north_star bound).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.inputs import CONFIGS, layer_solver_inputs, make_x
from oracle.lqr64 import LQRProblem, solve_grads

pytestmark = pytest.mark.gpu

TOL = 1e-4
NAMES11 = ["A_diag", "coeff_B", "coeff_Q", "R_inv", "coeff_Qf", "lgA", "lgB", "lgQ", "h0", "B_basis", "Q_basis"]


def _relerr(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.abs(x - ref).max() / max(np.abs(ref).max(), 1e-30))


def factored_inputs(cfg, n_tok, rb=None, rq=None, d=None, scale=0.3, seed=0):
    """Per-head inputs of a config's seeded layer slice, plus seeded low-rank factors with
    the layer's normalisations (l2norm coefficients, softplus for the Q mixtures, PSD Q bases)."""
    c = CONFIGS[cfg]
    x = make_x(cfg, n_tokens=n_tok, seed=seed)
    A, _B, _Q, R, _Qf, lA, lB, lQ, h0 = layer_solver_inputs(cfg, x)
    N, H, d0 = A.shape
    rb = rb or c["b_rank"]
    rq = rq or c["q_rank"]
    if d is not None and d != d0:  # other state sizes: fresh per-head inputs of that size
        g = torch.Generator().manual_seed(seed + 11)
        A = F.normalize(torch.rand(N, H, d, generator=g), dim=-1)
        R = torch.clamp(F.normalize(F.softplus(torch.randn(N, H, d, generator=g)), dim=-1), min=1e-6)
        lB = -F.softplus(torch.randn(N, H, d, generator=g))
        lQ = -F.softplus(torch.randn(N, H, d, generator=g))
        h0 = torch.randn(N, H, d, generator=g)
        d0 = d
    g = torch.Generator().manual_seed(seed + 5)
    l2 = lambda t: t / torch.sqrt((t * t).sum(-1, keepdim=True) + 1e-6)  # noqa: E731
    cB = l2(torch.randn(N, rb, generator=g))
    cQ = l2(F.softplus(torch.randn(N, rq, generator=g)))
    cQf = l2(F.softplus(torch.randn(N, H, rq, generator=g)))
    Bs = scale * torch.randn(rb, d0, d0, generator=g)
    Ms = scale * torch.randn(rq, d0, d0, generator=g)
    Gs = Ms @ Ms.transpose(1, 2) / math.sqrt(d0)
    return [A, cB, cQ, R, cQf, lA, lB, lQ, h0, Bs, Gs]


def oracle_factored(ins, T, dU):
    """fp64: expand, solve, chain the gradients through the expansion."""
    A, cB, cQ, R, cQf, lA, lB, lQ, h0, Bs, Gs = [t.double().numpy() for t in ins]
    B = np.einsum("nr,rij->nij", cB, Bs)
    Q = np.einsum("nr,rij->nij", cQ, Gs)
    Qf = np.einsum("nhr,rij->nhij", cQf, Gs)
    ref = solve_grads(LQRProblem(A, B, Q, R, Qf, lA, lB, lQ, h0, T), dU)
    gB, gQ, gQf = ref["B"], ref["Q"], ref["Q_f"]
    return {
        "u": ref["u"], "A_diag": ref["A_diag"], "R_inv": ref["R_inv"], "lgA": ref["lgA"], "lgB": ref["lgB"],
        "lgQ": ref["lgQ"], "h0": ref["h0"],
        "coeff_B": np.einsum("nij,rij->nr", gB, Bs),
        "coeff_Q": np.einsum("nij,rij->nr", gQ, Gs),
        "coeff_Qf": np.einsum("nhij,rij->nhr", gQf, Gs),
        "B_basis": np.einsum("nr,nij->rij", cB, gB),
        "Q_basis": np.einsum("nr,nij->rij", cQ, gQ) + np.einsum("nhr,nhij->rij", cQf, gQf),
    }


def run_factored(ins, T, dU, **kw):
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored, last_backward_stats
    dev = torch.device("cuda:0")
    xs = [t.detach().to(dev).float().requires_grad_(True) for t in ins]
    u = hip_lqr_solve_factored(*xs, T, **kw)
    (u * torch.as_tensor(dU, device=dev, dtype=u.dtype)).sum().backward()
    out = {"u": u.detach().cpu().double().numpy(), "_fallback": last_backward_stats["fallback"]}
    for n, t in zip(NAMES11, xs):
        out[n] = t.grad.detach().cpu().double().numpy()
    return out


def check_factored(label, ins, T, seed=0, tol=TOL, **kw):
    N, H, d = ins[0].shape
    du = ins[3].shape[-1]
    dU = torch.randn(N, H, du, generator=torch.Generator().manual_seed(seed + 7)).double().numpy()
    print(f"[{label}] N={N} H={H} d={d} rb={ins[1].shape[1]} rq={ins[2].shape[1]} T={T} {kw}", flush=True)
    ref = oracle_factored(ins, T, dU)
    out = run_factored(ins, T, dU, **kw)
    errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES11}
    print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()) + f"  fallback={out['_fallback']}",
          flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"{label}: rel err above {tol}: {bad}"
    return out


@pytest.mark.parametrize("cfg,n_tok", [(2, 24), (3, 2), (4, 1)])
@pytest.mark.parametrize("stash", ["always", "compact", "never"])
def test_factored_config_slices(cfg, n_tok, stash):
    check_factored(f"cfg{cfg}", factored_inputs(cfg, n_tok), CONFIGS[cfg]["T"], stash=stash)


@pytest.mark.parametrize("stash", ["always", "compact"])
def test_factored_long_horizon_fp64_rescue(stash):
    """Config 5 at T = 1024 on the factored entry points: the symplectic sweep's rejected
    problems recomputed in fp64 from the rescue list in the factored workspace; stress
    gradients exceed the reference's 1e6 guard, so no limit."""
    check_factored("cfg5-factored", factored_inputs(5, 4, seed=6), 1024, stash=stash, grad_limit=math.inf)


@pytest.mark.parametrize("rb,rq", [(8, 40), (1, 64), (17, 3)])
def test_factored_ranks(rb, rq):
    """Ranks below, between and at the 16-wide tiles of the projection / reduction kernels."""
    check_factored(f"ranks {rb},{rq}", factored_inputs(2, 40, rb=rb, rq=rq), 24)


@pytest.mark.parametrize("d", [24, 64])
def test_factored_padded_and_wide_dims(d):
    """d = 24 runs padded to 32 (bases zero-padded on the host); d = 64 at 16 heads."""
    check_factored(f"d={d}", factored_inputs(3, 3, d=d, rb=12, rq=20), 20)


def test_factored_stable_backward():
    check_factored("stable", factored_inputs(2, 20), 32, stable_backward=True)


def test_factored_token_chunks_match_single_pass(monkeypatch):
    """A workspace of a few tokens forces many token chunks (expansion per chunk, basis
    gradients accumulated over chunks): u bitwise equal to one pass, gradients within fp32
    summation-order rounding, and both within the oracle bound."""
    from ttc.solvers._lib import lib
    ins = factored_inputs(2, 37, seed=3)
    T = 16
    dU = torch.randn(37, 8, 16, generator=torch.Generator().manual_seed(9)).double().numpy()
    one = run_factored(ins, T, dU, stash="never")
    ws = lib.ttc_lqr_factored_workspace_bytes(5, 8, 16, 16, 16, 16, T, 0, 1, 0, 0)
    monkeypatch.setenv("TTC_LQR_WORKSPACE_BYTES", str(ws))
    many = run_factored(ins, T, dU, stash="never")
    assert np.array_equal(one["u"], many["u"])
    for k in NAMES11:
        assert _relerr(many[k], one[k]) <= 1e-5, k
    ref = oracle_factored(ins, T, dU)
    for k in ["u"] + NAMES11:
        assert _relerr(many[k], ref[k]) <= TOL, k


@pytest.mark.parametrize("cfg,n_tok,T,stash", [(2, 24, 64, "always"), (5, 8, 1024, "always"),
                                              (4, 2, 256, "always"), (2, 24, 64, "compact")])
def test_kept_expansion_equals_reexpansion(cfg, n_tok, T, stash, monkeypatch):
    """TTC_LQR_FLAG_KEEP_EXPANDED: the forward expands B, Q, Q_f into the stash buffer and the
    backward reads them there instead of expanding again.  The same values reach the same kernels,
    so u and all eleven gradients are bitwise those of the run that expands twice -- with the full
    and the compact stash, and at T = 1024 (fp64 rescue, two rollout tiers, stable path); the
    keep decision is forced both ways and recorded, so both branches run."""
    import ttc.solvers.hip_lqr as hl
    ins = factored_inputs(cfg, n_tok, seed=2)
    N, H, d = ins[0].shape
    dU = torch.randn(N, H, ins[3].shape[-1], generator=torch.Generator().manual_seed(5)).double().numpy()
    decided, outs = [], []
    for keep in (False, True):
        monkeypatch.setattr(hl, "_keep_expanded", lambda *a, keep=keep: decided.append(keep) or keep)
        print(f"[keep-expanded cfg{cfg} T={T} stash={stash} keep={keep}]", flush=True)
        outs.append(run_factored(ins, T, dU, stash=stash, grad_limit=math.inf))
    assert decided == [False, True]
    for k in ["u"] + NAMES11:
        assert np.array_equal(outs[0][k], outs[1][k]), k
    assert outs[0]["_fallback"] == outs[1]["_fallback"]


def test_factored_equals_materialised_hip_solver():
    """Same HIP kernels on both sides: the factored entry points against hip_lqr_solve on
    torch-expanded B, Q, Q_f with torch's chain rule of the einsums."""
    from ttc.solvers.hip_lqr import hip_lqr_solve
    ins = factored_inputs(2, 16, seed=4)
    T = 64
    dev = torch.device("cuda:0")
    dU = torch.randn(16, 8, 16, generator=torch.Generator().manual_seed(1)).to(dev)
    out_f = run_factored(ins, T, dU.cpu().double().numpy())
    xs = [t.to(dev).float().requires_grad_(True) for t in ins]
    A, cB, cQ, R, cQf, lA, lB, lQ, h0, Bs, Gs = xs
    B = torch.einsum("nr,rij->nij", cB, Bs)
    Q = torch.einsum("nr,rij->nij", cQ, Gs)
    Qf = torch.einsum("nhr,rij->nhij", cQf, Gs)
    u = hip_lqr_solve(A, B, Q, R, Qf, lA, lB, lQ, h0, T)
    (u * dU).sum().backward()
    assert _relerr(out_f["u"], u.detach().cpu()) <= 1e-5
    for n, t in zip(NAMES11, xs):
        assert _relerr(out_f[n], t.grad.cpu()) <= 1e-4, n


def test_factored_empty_batch_zero_basis_grads():
    ins = [t.cuda().float().requires_grad_(True) for t in factored_inputs(2, 2)]
    sl = [t[:0] if i < 9 else t for i, t in enumerate(ins)]
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored
    u = hip_lqr_solve_factored(*sl, 8)
    assert u.shape == (0, 8, 16)
    u.sum().backward()
    assert float(ins[9].grad.abs().max()) == 0.0 and float(ins[10].grad.abs().max()) == 0.0


@pytest.mark.parametrize("q_reparam", ["plain", "cholesky"])
def test_layer_factored_equals_materialised(q_reparam):
    """TTCLayer(factored=True) against TTCLayer(factored=False) with the same weights: outputs
    and every parameter gradient (in_proj, out_proj, Bs, Qs)."""
    from ttc import TTCLayer
    torch.manual_seed(0)
    a = TTCLayer(32, 32, 16, 8, 16, 16, q_reparam=q_reparam, solver_impl="hip", factored=True).cuda()
    b = TTCLayer(32, 32, 16, 8, 16, 16, q_reparam=q_reparam, solver_impl="hip", factored=False).cuda()
    b.load_state_dict(a.state_dict())
    with torch.no_grad():  # larger bases than the 0.02 init, so every gradient is well above rounding
        for m in (a, b):
            m.Bs.mul_(10.0)
            m.Qs.mul_(10.0 if q_reparam == "plain" else 3.0)
    x = torch.randn(3, 7, 8, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3))
    dy = torch.randn(3, 7, 8, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(4))
    ya, yb = a(x, T=32), b(x, T=32)
    (ya * dy).sum().backward()
    (yb * dy).sum().backward()
    assert _relerr(ya.detach().cpu(), yb.detach().cpu()) <= 1e-5
    for (n, pa), (_, pb) in zip(a.named_parameters(), b.named_parameters()):
        assert _relerr(pa.grad.cpu(), pb.grad.cpu()) <= 1e-4, n


def _run_grads(ins, T, dU, dtype, **kw):
    """u and the eleven gradients of sum(dU * u), inputs of `dtype` (outputs as returned)."""
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored
    dev = torch.device("cuda:0")
    xs = [t.detach().to(dev).to(dtype).requires_grad_(True) for t in ins]
    u = hip_lqr_solve_factored(*xs, T, **kw)
    torch.autograd.backward(u, torch.as_tensor(dU, device=dev).to(u.dtype))
    return [u.detach()] + [t.grad.detach() for t in xs]


@pytest.mark.parametrize("cfg,n_tok,d", [(2, 24, None), (4, 2, None), (2, 9, 24)])
def test_factored_bf16_storage_is_rounded_fp32(cfg, n_tok, d):
    """bf16 storage (ttc_lqr_*_factored_bf16): inputs widened per chunk, fp32 arithmetic,
    gradients rounded on store -- so every output equals the fp32 entry points' output on the
    widened inputs, rounded to bf16, bit for bit (d = 24 also checks bf16 padding)."""
    ins = [t.to(torch.bfloat16) for t in factored_inputs(cfg, n_tok, d=d)]
    N, H, dd = ins[0].shape
    T = CONFIGS[cfg]["T"]
    dU = torch.randn(N, H, ins[3].shape[-1], generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    got = _run_grads(ins, T, dU, torch.bfloat16)
    ref = _run_grads([t.float() for t in ins], T, dU.float(), torch.float32)
    for k, (a, b) in enumerate(zip(got, ref)):
        assert a.dtype == torch.bfloat16
        assert torch.equal(a, b.to(torch.bfloat16)), (["u"] + NAMES11)[k]


def test_factored_bf16_token_chunks(monkeypatch):
    """bf16 storage over many token chunks: u bitwise equal to one pass; gradients equal up
    to the fp32 summation order of the basis sums (one bf16 ulp)."""
    from ttc.solvers._lib import lib
    ins = [t.to(torch.bfloat16) for t in factored_inputs(2, 30, seed=6)]
    T = 16
    dU = torch.randn(30, 8, 16, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    one = _run_grads(ins, T, dU, torch.bfloat16, stash="never")
    monkeypatch.setenv("TTC_LQR_WORKSPACE_BYTES", str(lib.ttc_lqr_factored_workspace_bytes(4, 8, 16, 16, 16, 16,
                                                                                        T, 0, 1, 1, 0)))
    many = _run_grads(ins, T, dU, torch.bfloat16, stash="never")
    assert torch.equal(one[0], many[0])
    for k in range(1, 12):
        a, b = one[k].float(), many[k].float()
        assert float((a - b).abs().max()) <= 2 ** -7 * float(b.abs().max()), NAMES11[k - 1]


def test_layer_bf16_runs_on_bf16_storage():
    """A bf16 TTCLayer (config 4's storage) passes bf16 tensors to the solver; output and
    parameter gradients track the fp32 layer to bf16 accuracy."""
    from ttc import TTCLayer
    torch.manual_seed(1)
    a = TTCLayer(64, 64, 32, 4, 32, 32, solver_impl="hip").cuda()
    b = TTCLayer(64, 64, 32, 4, 32, 32, solver_impl="hip").cuda()
    b.load_state_dict(a.state_dict())
    b = b.to(torch.bfloat16)
    with torch.no_grad():
        for m in (a, b):
            m.Bs.mul_(10.0)
            m.Qs.mul_(10.0)
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = (0.02 * torch.randn(2, 16, 4, 64, device="cuda", generator=gen)).to(torch.bfloat16)
    ya, yb = a(x.float(), T=32), b(x, T=32)
    assert yb.dtype == torch.bfloat16
    dy = torch.randn(ya.shape, device="cuda", generator=gen)
    (ya * dy).sum().backward()
    (yb.float() * dy).sum().backward()
    assert _relerr(yb.detach().float().cpu(), ya.detach().cpu()) <= 3e-2
    for (n, pa), (_, pb) in zip(a.named_parameters(), b.named_parameters()):
        assert pb.grad.dtype == torch.bfloat16
        assert _relerr(pb.grad.float().cpu(), pa.grad.cpu()) <= 5e-2, n


@pytest.mark.parametrize("mode", ["l2_norm", "h0_norm"])
@pytest.mark.parametrize("d", [16, 24, 64])
def test_fused_rescale_matches_torch_backend(mode, d):
    """ttc_lqr_rescale / _backward (the layer's back-end, ttc_layer.py:142-147) fused into the
    factored call: values and the gradients of all eleven inputs equal the unfused call
    followed by the torch rescale (detached norms for h0_norm), to fp32 rounding."""
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored
    from ttc.layers.ttc_layer import l2norm
    ins = factored_inputs(3 if d != 16 else 2, 4, d=None if d == 16 else d, rb=12, rq=20)
    dev = torch.device("cuda:0")
    N, H, dd = ins[0].shape
    dY = torch.randn(N, H, ins[3].shape[-1], device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    xa = [t.to(dev).float().requires_grad_(True) for t in ins]
    ya = hip_lqr_solve_factored(*xa, 24, rescale=mode)
    (ya * dY).sum().backward()
    xb = [t.to(dev).float().requires_grad_(True) for t in ins]
    u = hip_lqr_solve_factored(*xb, 24)
    if mode == "l2_norm":
        yb = l2norm(u)
    else:
        yb = u / torch.linalg.norm(u, dim=-1).detach()[..., None] * torch.linalg.norm(xb[8], dim=-1).detach()[..., None]
    (yb * dY).sum().backward()
    assert _relerr(ya.detach().cpu(), yb.detach().cpu()) <= 1e-6
    for n, a, b in zip(NAMES11, xa, xb):
        assert _relerr(a.grad.cpu(), b.grad.cpu()) <= 1e-5, n


def test_layer_h0_norm_factored_equals_materialised():
    from ttc import TTCLayer
    torch.manual_seed(2)
    a = TTCLayer(32, 32, 16, 8, 16, 16, rescale="h0_norm", solver_impl="hip", factored=True).cuda()
    b = TTCLayer(32, 32, 16, 8, 16, 16, rescale="h0_norm", solver_impl="hip", factored=False).cuda()
    b.load_state_dict(a.state_dict())
    x = torch.randn(2, 9, 8, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(5))
    ya, yb = a(x, T=16), b(x, T=16)
    ya.square().sum().backward()
    yb.square().sum().backward()
    assert _relerr(ya.detach().cpu(), yb.detach().cpu()) <= 1e-5
    for (n, pa), (_, pb) in zip(a.named_parameters(), b.named_parameters()):
        assert _relerr(pa.grad.cpu(), pb.grad.cpu()) <= 1e-4, n


@pytest.mark.parametrize("cfg,n_tok", [(2, 40), (3, 3), (4, 2)])
def test_compact_stash_matches_full_stash(cfg, n_tok, monkeypatch):
    """The compact stash (V_1's upper triangles; Quu_0 recomputed on the matrix cores in the
    backward) against the full stash: u bitwise (same forward), gradients to fp32 rounding;
    also over several token chunks."""
    from ttc.solvers._lib import lib
    ins = factored_inputs(cfg, n_tok, seed=8)
    N, H, d = ins[0].shape
    T = CONFIGS[cfg]["T"]
    dU = torch.randn(N, H, d, generator=torch.Generator().manual_seed(6)).double().numpy()
    full = run_factored(ins, T, dU, stash="always")
    comp = run_factored(ins, T, dU, stash="compact")
    assert np.array_equal(full["u"], comp["u"])
    for k in NAMES11:
        assert _relerr(comp[k], full[k]) <= 2e-5, k
    ws = lib.ttc_lqr_factored_workspace_bytes(1, H, d, d, ins[1].shape[1], ins[2].shape[1], T, 2, 1, 0, 0)
    monkeypatch.setenv("TTC_LQR_WORKSPACE_BYTES", str(ws))
    chunked = run_factored(ins, T, dU, stash="compact")
    assert np.array_equal(full["u"], chunked["u"])
    for k in NAMES11:
        assert _relerr(chunked[k], full[k]) <= 2e-5, k


BF16_TOL = 2.0 ** -8  # results are fp32 computations rounded to bf16 (half an ulp: 2^-9 of each value)


@pytest.mark.parametrize("cfg,n_tok", [(4, 2), (2, 16)])
def test_bf16_storage_against_oracle(cfg, n_tok):
    """bf16 storage (config 4 stores its activations in bf16): the eleven factored inputs and
    d_u handed over as bf16 (``ttc_lqr_*_factored_bf16``), u and all eleven gradients returned
    as bf16, against the fp64 oracle evaluated on the same bf16 values (widened exactly).
    Tolerance: per tensor max|x - x64| / max|x64| <= 2^-8 -- the fp32 solve (~1e-6) plus the
    rounding of each output to bf16 (at most half an ulp, 2^-9 relative)."""
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored
    ins = [t.to(torch.bfloat16) for t in factored_inputs(cfg, n_tok, seed=17)]
    T = CONFIGS[cfg]["T"]
    N, H, d = ins[0].shape
    dU = torch.randn(N, H, d, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    ref = oracle_factored([t.float() for t in ins], T, dU.double().numpy())
    dev = torch.device("cuda:0")
    xs = [t.to(dev).requires_grad_(True) for t in ins]
    u = hip_lqr_solve_factored(*xs, T)
    assert u.dtype == torch.bfloat16
    (u * dU.to(dev)).sum().backward()
    out = {"u": u.detach().float().cpu().double().numpy()}
    for n, t in zip(NAMES11, xs):
        assert t.grad.dtype == torch.bfloat16
        out[n] = t.grad.float().cpu().double().numpy()
    errs = {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES11}
    print(f"[bf16 cfg{cfg}] N={N} H={H} d={d} T={T}: " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()),
          flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= BF16_TOL)}
    assert not bad, f"bf16 cfg{cfg}: rel err above {BF16_TOL}: {bad}"
