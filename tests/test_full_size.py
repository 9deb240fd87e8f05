"""Configs 2 and 5b at their full size on the GPU, forward and backward through the autograd
Function: config 2, x [16, 2048, 8, 32] -> 262,144 tokens x 8 heads = 2,097,152 problems at
T = 64; config 5b, x [4, 1024, 8, 32] -> 32,768 tokens x 8 heads = 262,144 problems at T = 1024
(the fp32 sweep, its fp64 rescue, the three rollout tiers and the fp64 stable path).

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
  tensor's largest entry at config 5b, whose tiniest entries (|x| < 1e-32) are subnormal in
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
CASES = {2: (3, 2_097_152, 64), "5b": (4, 262_144, 8)}


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
