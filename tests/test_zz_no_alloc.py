"""GPU test of ttc_lqr_backward_noalloc (the allocation-free backward over the library's fixed
device scratch) through the C ABI: on two calls in a row, the second with a smaller input, its
nine gradients, status word and fallback count equal those of ttc_lqr_backward on the same inputs
with a caller-allocated workspace, bit for bit (the same kernels on independent problems; the
token chunks and fallback passes the scratch imposes do not change any problem's arithmetic or
the order of a token's head sums).  Cases: a config-2 slice (one chunk), a batch that the
256 MiB scratch splits into several token chunks, and config-5 stress inputs whose rejected
problems take the stable path inside the scratch (asserted: the fallback count is positive), at
T = 64 and at T = 1024 under TTC_LQR_FLAG_FP64_RESCUE (the fp32 head-group rollout, the fp64
second and third rollout tiers and the fp64 stable path, all inside the scratch), and config-5b
inputs at T = 1024 whose forward kept the rescue's fp64 V_1 and gains (flags 256 and 512: the
stable path reads the kept gains inside the scratch).  Each case runs its forward once and both
backwards from that stash."""
import ctypes
import math

import numpy as np
import pytest
import torch

from oracle.inputs import layer_solver_inputs, make_x

pytestmark = pytest.mark.gpu

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]


def _inputs(cfg, n_tok, seed):
    ins = layer_solver_inputs(cfg, make_x(cfg, n_tokens=n_tok, seed=seed))
    return [t.contiguous().cuda() for t in ins]


def _grads_like(ins):
    A, B, Q, R, Qf, lA, lB, lQ, h0 = ins
    return [torch.empty_like(t) for t in (A, B, Q, R, Qf, lA, lB, lQ, h0)]


def _forward(ins, T, stash, flags):
    """u and the stash; under TTC_LQR_FLAG_RESCUE_V1 (256) through ttc_lqr_forward_ws, with the
    rescue's records after the stash (and its gains under 512)."""
    from ttc.solvers._lib import lib
    N, H, d = ins[0].shape
    dev = ins[0].device
    u = torch.empty(N, H, d, device=dev)
    a256 = lambda n: (n + 255) // 256 * 256  # noqa: E731
    nst = lib.ttc_lqr_stash_bytes(N, H, d, d, T)
    if flags & 256:
        nst = a256(nst) + lib.ttc_lqr_rescue_stash_bytes(N, H, d, d)
        if flags & 512:
            nst += lib.ttc_lqr_rescue_gains_bytes(N, H, d, d, T)
    st = torch.empty(nst // 4, device=dev) if stash else None
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    if flags & 256:
        nws = lib.ttc_lqr_forward_workspace_bytes(N, H, d, d, T, flags)
        ws = torch.empty(nws, dtype=torch.uint8, device=dev)
        rc = lib.ttc_lqr_forward_ws(*[t.data_ptr() for t in ins], N, H, d, d, T, flags, u.data_ptr(), st.data_ptr(),
                                    ws.data_ptr(), nws, status.data_ptr(), s)
    else:
        rc = lib.ttc_lqr_forward(*[t.data_ptr() for t in ins], N, H, d, d, T, flags, u.data_ptr(),
                                 None if st is None else st.data_ptr(), status.data_ptr(), s)
    assert rc == 0
    torch.cuda.synchronize()
    return u, st


def _backward(ins, T, noalloc, stash, flags=0, fwd=None):
    from ttc.solvers._lib import lib
    N, H, d = ins[0].shape
    dev = ins[0].device
    u, st = fwd if fwd is not None else _forward(ins, T, stash, flags)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    dU = torch.randn(N, H, d, generator=torch.Generator(device=dev).manual_seed(N + T), device=dev)
    g = _grads_like(ins)
    n_fb = ctypes.c_int64(-1)
    common = [*[t.data_ptr() for t in ins], u.data_ptr(), dU.data_ptr(), N, H, d, d, T, flags,
              None if st is None else st.data_ptr(), *[t.data_ptr() for t in g]]
    if noalloc:
        rc = lib.ttc_lqr_backward_noalloc(*common, math.inf, status.data_ptr(), ctypes.byref(n_fb), s)
    else:
        ws_bytes = lib.ttc_lqr_workspace_bytes(N, H, d, d, T, int(stash), flags)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        rc = lib.ttc_lqr_backward(*common, ws.data_ptr(), ws.numel(), math.inf, status.data_ptr(),
                                  ctypes.byref(n_fb), s)
    assert rc == 0, lib.ttc_lqr_strerror(rc)
    torch.cuda.synchronize()
    return [t.cpu() for t in g], int(status.item()), int(n_fb.value)


@pytest.mark.parametrize("cfg,n1,n2,T,stash,flags", [(2, 256, 40, 64, True, 0), (2, 1200, 300, 64, False, 0),
                                                     (5, 64, 16, 64, True, 0), (5, 32, 8, 1024, True, 32),
                                                     ("5b", 64, 24, 1024, True, 32 | 256 | 512)])
def test_noalloc_backward_equals_workspace_backward(cfg, n1, n2, T, stash, flags):
    for n_tok in (n1, n2):  # two calls in a row, the second smaller
        ins = _inputs(cfg, n_tok, seed=n_tok + (cfg if isinstance(cfg, int) else 50))
        print(f"[noalloc cfg{cfg} tokens={n_tok} T={T} stash={stash} flags={flags}]", flush=True)
        fwd = _forward(ins, T, stash, flags)  # one forward for both: the rescue's slot order is not fixed
        ref, st_ref, fb_ref = _backward(ins, T, noalloc=False, stash=stash, flags=flags, fwd=fwd)
        out, st_out, fb_out = _backward(ins, T, noalloc=True, stash=stash, flags=flags, fwd=fwd)
        errs = {n: float((a.double() - b.double()).abs().max() / max(b.double().abs().max(), 1e-30))
                for n, a, b in zip(NAMES, out, ref)}
        same = all(torch.equal(a, b) for a, b in zip(out, ref))
        print(f"cfg{cfg} tokens={n_tok} T={T} stash={stash}: fallback {fb_out} (workspace path {fb_ref}), "
              f"bitwise equal {same}, max rel diff {max(errs.values()):.1e}", flush=True)
        assert st_out == st_ref
        assert fb_out == fb_ref
        if cfg in (5, "5b"):
            assert fb_ref > 0  # the stable path ran inside the scratch
        assert max(errs.values()) <= 1e-4, errs
        assert same
