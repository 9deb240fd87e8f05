"""The reference-side ctypes binding that the repository's integration guide gives a maintainer
(``ttc/solvers/hip_lqr_binding.py`` plus its ``LQR_SOLVER_IMPL_MAP["hip"]`` entry), executed
from the guide's own code block, so that the documented binding is the tested one.

CPU: the block binds every symbol it names and picks the flags of the precision policy.
GPU: the registered solver against the fp64 oracle (u and all nine gradients within 1e-4) on a
config-2 slice and on config-5 token scales at T = 64 and T = 1024, whose forward rescues some
problems (status bit 4, which the binding must not treat as an error).  The binding keeps the
reference's 1e6 gradient guard, so d_u is scaled (gradients are linear in it) to keep the
largest guarded gradient at 1e3.
"""
import os
import re

import numpy as np
import pytest
import torch

from oracle.inputs import layer_solver_inputs, make_x
from oracle.lqr64 import LQRProblem, solve_grads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")
NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]
GUARDED = ["A_diag", "B", "Q", "R_inv", "Q_f", "h0"]


def _stub_source():
    with open(GUIDE) as f:
        text = f.read()
    m = re.search(r"```python\n(# ttc/solvers/hip_lqr_binding\.py\n.*?)```", text, re.S)
    assert m, f"{GUIDE} has no ttc/solvers/hip_lqr_binding.py block"
    return m.group(1)


def _load_stub(monkeypatch):
    from ttc.solvers._lib import lib_path
    monkeypatch.setenv("TTC_LQR_LIB", lib_path())
    ns = {"LQR_SOLVER_IMPL_MAP": {}}
    exec(compile(_stub_source(), "hip_lqr_binding.py", "exec"), ns)
    return ns


def test_stub_binds_the_library(monkeypatch):
    ns = _load_stub(monkeypatch)
    assert callable(ns["LQR_SOLVER_IMPL_MAP"]["hip"])
    lib = ns["_lib"]
    for sym in re.findall(r"_lib\.(ttc_lqr_\w+)", _stub_source()):
        assert getattr(lib, sym) is not None, sym
    f = ns["_flags"]
    assert (f(16, 64), f(32, 511), f(16, 512), f(32, 1024), f(64, 64), f(64, 1024)) == (64, 64, 32, 32, 0, 0)
    assert ns["_ERRORS"] == 3 and ns["_RESCUED"] == 4


@pytest.mark.gpu
@pytest.mark.parametrize("cfg,n_tok,T,seed,rescued", [(2, 16, 64, 1, False), (5, 64, 64, 21, True),
                                                      (5, 16, 1024, 5, True)])
def test_stub_against_oracle(monkeypatch, cfg, n_tok, T, seed, rescued):
    ns = _load_stub(monkeypatch)
    lib = ns["_lib"]
    solve = ns["LQR_SOLVER_IMPL_MAP"]["hip"]
    ins = layer_solver_inputs(cfg, make_x(cfg, n_tokens=n_tok, seed=seed))
    pb = LQRProblem(*ins, T)
    dU = torch.randn(pb.N, pb.H, pb.du, generator=torch.Generator().manual_seed(seed + 7)).double().numpy()
    ref = solve_grads(pb, dU)
    s = min(1.0, 1e3 / max(np.abs(ref[k]).max() for k in GUARDED))
    print(f"[stub cfg{cfg} T={T}] N={pb.N} H={pb.H} d_u scale {s:.1e}", flush=True)
    # whether the forward's certificate rejects problems of this sample (the rescue the binding runs)
    f32 = [t.float().contiguous().cuda() for t in ins]
    flags = ns["_flags"](pb.d, T)
    u0 = torch.empty(pb.N, pb.H, pb.du, device="cuda")
    st = torch.zeros(1, dtype=torch.int32, device="cuda")
    nws = max(lib.ttc_lqr_forward_workspace_bytes(pb.N, pb.H, pb.d, pb.du, T, flags), 1)
    fws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    rc = lib.ttc_lqr_forward_ws(*[t.data_ptr() for t in f32], pb.N, pb.H, pb.d, pb.du, T, flags, u0.data_ptr(), None,
                                fws.data_ptr(), nws, st.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert bool(int(st.item()) & 4) == rescued
    xs = [t.cuda().requires_grad_(True) for t in f32]
    u = solve(*xs, T)
    (u * torch.from_numpy(dU * s).float().cuda()).sum().backward()
    errs = {"u": np.abs(u.detach().cpu().double().numpy() - ref["u"]).max() / np.abs(ref["u"]).max()}
    for n, t in zip(NAMES, xs):
        r = ref[n] * s
        errs[n] = float(np.abs(t.grad.cpu().double().numpy() - r).max() / max(np.abs(r).max(), 1e-30))
    print("   " + " ".join(f"{k}:{v:.1e}" for k, v in errs.items()), flush=True)
    assert max(errs.values()) <= 1e-4, errs
