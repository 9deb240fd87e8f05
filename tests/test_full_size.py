"""Configs 2, 5 and 5b at their full size on the GPU, forward and backward through the autograd
Function: config 2, x [16, 2048, 8, 32] -> 262,144 tokens x 8 heads = 2,097,152 problems at
T = 64; configs 5 and 5b, x [256, 1, 8, 32] and [4, 1024, 8, 32] -> 2,048 and 32,768 tokens x 8
heads = 16,384 and 262,144 problems at T = 1024 (the fp32 sweep, its fp64 rescue, the three
rollout tiers and the fp64 stable path; config 5's short lists run one problem per wave, config
5b's four).  Configs 3 and 4 follow below on the factored entry points.

At these sizes the fp64 oracle runs only on a sample, so the whole-size run is checked by
* parity on a seeded sample of tokens against the fp64 oracle, at the 1e-4 bar of the other
  parity tests;
* a token permutation: a problem's arithmetic depends at most on the other heads of its token
  (they share B and Q and one head group), never on the wave, list position or chunk it lands
  in, so permuting the tokens permutes u and all nine gradients bit for bit -- an indexing slip,
  a race or a read of another token's data breaks it;
* the scaling h0 -> 2 h0: u is linear in h0 and every gradient but grad_h0 is a product of one
  primal factor (scaled by 2) and one adjoint factor (independent of h0), while grad_h0 =
  A_0 lambda~_1 is purely adjoint.  Scaling by a power of two is exact in floating point except
  where a value or an intermediate product falls below the smallest normal number, so u and
  those eight gradients double and grad_h0 stays: bit for bit at config 2, and to 1e-6 of each
  tensor's largest entry at configs 5 and 5b, whose tiniest entries (|x| < 1e-32) are subnormal in
  fp32 or come from products that are.
"""
import numpy as np
import pytest
import torch

from oracle.inputs import CONFIGS, layer_solver_inputs, make_x
from oracle.lqr64 import LQRProblem, solve_grads

pytestmark = pytest.mark.gpu

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
TOL = 1e-4
# config: (x seed, problems, sampled tokens)
CASES = {2: (3, 2_097_152, 64), 5: (6, 16_384, 8), "5b": (4, 262_144, 8)}


def _run(ins, dU, T):
    """u and the nine gradients of sum(dU * u), on cuda:0, as fp32 host arrays."""
    from ttc.solvers.hip_lqr import hip_lqr_solve, last_backward_stats
    dev = torch.device("cuda:0")
    xs = [t.to(dev).requires_grad_(True) for t in ins]
    u = hip_lqr_solve(*xs, T, grad_limit=float("inf"))
    (u * dU.to(dev)).sum().backward()
    out = {"u": u.detach().cpu().numpy()}
    for n, t in zip(NAMES, xs):
        out[n] = t.grad.detach().cpu().numpy()
    out["_fallback"] = last_backward_stats["fallback"]
    del xs, u
    torch.cuda.empty_cache()
    return out


@pytest.fixture(scope="module", params=list(CASES), ids=lambda c: f"cfg{c}")
def full(request):
    cfg = request.param
    seed, problems, _ = CASES[cfg]
    T = CONFIGS[cfg]["T"]
    x = make_x(cfg, seed=seed)  # the config's full x
    ins = [t.detach().float().contiguous() for t in layer_solver_inputs(cfg, x)]
    N, H = ins[0].shape[:2]
    du = ins[1].shape[-1]
    assert N * H == problems
    dU = torch.randn(N, H, du, generator=torch.Generator().manual_seed(11))
    print(f"[cfg{cfg} full] N={N} H={H} T={T}", flush=True)
    out = _run(ins, dU, T)
    print(f"   fallback {out['_fallback']}/{N * H}", flush=True)
    return cfg, T, ins, dU, out


def test_full_size_sample_against_oracle(full):
    cfg, T, ins, dU, out = full
    N = ins[0].shape[0]
    idx = np.sort(np.random.default_rng(5).choice(N, size=CASES[cfg][2], replace=False))
    sel = torch.as_tensor(idx)
    pb = LQRProblem(*[t[sel].double() for t in ins], T)
    ref = solve_grads(pb, dU[sel].double().numpy())
    errs = {}
    for k in ["u"] + NAMES:
        x = out[k][idx].astype(np.float64)
        r = np.asarray(ref[k], dtype=np.float64)
        errs[k] = float(np.abs(x - r).max() / max(np.abs(r).max(), 1e-30))
    print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    bad = {k: v for k, v in errs.items() if not (v <= TOL)}
    assert not bad, f"rel err above {TOL}: {bad}"


def test_full_size_token_permutation(full):
    cfg, T, ins, dU, out = full
    N = ins[0].shape[0]
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(17))
    res = _run([t[perm] for t in ins], dU[perm], T)
    assert res["_fallback"] == out["_fallback"]
    p = perm.numpy()
    for k in ["u"] + NAMES:
        assert np.array_equal(res[k], out[k][p]), k


def test_full_size_h0_scaling(full):
    cfg, T, ins, dU, out = full
    res = _run(ins[:8] + [2.0 * ins[8]], dU, T)
    assert res["_fallback"] == out["_fallback"]
    for k in ["u"] + NAMES:
        ref = out[k] if k == "h0" else 2.0 * out[k]
        if cfg == 2:
            assert np.array_equal(res[k], ref), k
        else:
            d = np.abs(res[k].astype(np.float64) - ref).max()
            assert d <= 1e-6 * np.abs(ref).max(), (k, d)


# ---- configs 3 and 4 at full size through the factored entry points ---------------------------
# Materialised, Q_f alone would be 137 GB at either config, so these run on the layer's low-rank
# factors (hip_lqr_solve_factored), formed on the device by a seeded random-init TTCLayer's
# front-end from the config's full x, as bench.py's full-size entries do.  The basis gradients
# are sums over every token, so the sample checks the per-token outputs; the permutation and
# scaling checks cover all eleven gradients.
NAMES11 = ["A_diag", "coeff_B", "coeff_Q", "R_inv", "coeff_Qf", "lgA", "lgB", "lgQ", "h0", "B_basis", "Q_basis"]
PER_TOKEN = NAMES11[:9]


def _factored_full(cfg, seed):
    from ttc import TTCLayer
    c = CONFIGS[cfg]
    dev = torch.device("cuda:0")
    torch.manual_seed(seed)
    layer = TTCLayer(c["in_dim"], c["out_dim"], c["h_dim"], c["num_heads"], c["b_rank"], c["q_rank"],
                     solver_impl="hip").to(dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    x = (torch.randn(c["x_shape"], generator=g, device=dev) * c["scale"]).to(c["dtype"]).float()
    with torch.no_grad():
        ins = [t.detach().float().contiguous() for t in layer.factored_inputs(x)]
    del layer, x
    return ins


def _run_factored(ins, dU, T):
    """u and the eleven gradients, left on the device."""
    from ttc.solvers.hip_lqr import hip_lqr_solve_factored, last_backward_stats
    xs = [t.detach().requires_grad_(True) for t in ins]  # no copies: the inputs are tens of GB
    u = hip_lqr_solve_factored(*xs, T, grad_limit=float("inf"))
    (u * dU).sum().backward()
    out = {"u": u.detach()}
    for n, t in zip(NAMES11, xs):
        out[n] = t.grad.detach()
    out["_fallback"] = last_backward_stats["fallback"]
    del xs, u
    torch.cuda.empty_cache()
    return out


# "4-bf16": config 4 with the eleven inputs and d_u stored as bf16 (its activations' storage),
# through the _bf16 entry points; u and the gradients come back as bf16
@pytest.fixture(scope="module", params=[3, 4, "4-bf16"], ids=lambda c: f"cfg{c}")
def full_factored(request):
    cfg = request.param
    base = 4 if cfg == "4-bf16" else cfg
    T = CONFIGS[base]["T"]
    ins = _factored_full(base, seed=20 + base)
    N, H, d = ins[0].shape
    dU = torch.randn(N, H, d, generator=torch.Generator(device=ins[0].device).manual_seed(13), device=ins[0].device)
    if cfg == "4-bf16":
        ins = [t.to(torch.bfloat16) for t in ins]
        dU = dU.to(torch.bfloat16)
    print(f"[cfg{cfg} full, factored] N={N} H={H} d={d} T={T}: solving", flush=True)
    out = _run_factored(ins, dU, T)
    print(f"   fallback {out['_fallback']}/{N * H}", flush=True)
    yield cfg, T, ins, dU, out
    del ins, dU, out
    torch.cuda.empty_cache()


def test_full_size_factored_sample_against_oracle(full_factored):
    from test_factored import oracle_factored
    cfg, T, ins, dU, out = full_factored
    N = ins[0].shape[0]
    idx = np.sort(np.random.default_rng(7).choice(N, size=2, replace=False))
    sel = torch.as_tensor(idx, device=ins[0].device)
    per_tok = [ins[k][sel].float().cpu() for k in range(9)] + [ins[9].float().cpu(), ins[10].float().cpu()]
    ref = oracle_factored(per_tok, T, dU[sel].double().cpu().numpy())
    errs = {}
    for k in ["u"] + PER_TOKEN:
        x = out[k][sel].double().cpu().numpy()
        r = np.asarray(ref[k], dtype=np.float64)
        errs[k] = float(np.abs(x - r).max() / max(np.abs(r).max(), 1e-30))
    print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    # bf16 outputs: the fp32 solve plus half a bf16 ulp (2^-9 relative) of rounding
    tol = 2.0 ** -8 if cfg == "4-bf16" else TOL
    bad = {k: v for k, v in errs.items() if not (v <= tol)}
    assert not bad, f"rel err above {tol}: {bad}"


def test_full_size_factored_token_permutation(full_factored):
    cfg, T, ins, dU, out = full_factored
    N = ins[0].shape[0]
    perm = torch.randperm(N, generator=torch.Generator(device=ins[0].device).manual_seed(19), device=ins[0].device)
    res = _run_factored([t[perm] for t in ins[:9]] + ins[9:], dU[perm], T)
    assert res["_fallback"] == out["_fallback"]
    for k in ["u"] + PER_TOKEN:
        assert torch.equal(res[k], out[k][perm]), k
    for k in NAMES11[9:]:  # sums over the tokens: the order of the terms changed
        d = (res[k].float() - out[k].float()).abs().max().item()
        tol = 2.0 ** -7 if cfg == "4-bf16" else 1e-5  # bf16: one ulp of the rounded sum
        assert d <= tol * out[k].float().abs().max().item(), (k, d)
    del res
    torch.cuda.empty_cache()


def test_full_size_factored_h0_scaling(full_factored):
    cfg, T, ins, dU, out = full_factored
    res = _run_factored(ins[:8] + [2.0 * ins[8]] + ins[9:], dU, T)
    assert res["_fallback"] == out["_fallback"]
    for k in ["u"] + NAMES11:
        ref = out[k] if k == "h0" else 2.0 * out[k]
        assert torch.equal(res[k], ref), k
