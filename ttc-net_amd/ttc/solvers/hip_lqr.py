"""HIP (gfx950) LQR solver: the autograd Function behind ``solver_impl="hip"``.

Mirrors the reference ``FusedLQRSolveFunc`` / ``fused_lqr_solve``
(``ttc/solvers/fused_lqr.py:255-304``): same positional inputs
``(A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T)``,
same shape assertions (``fused_lqr.py:37-45``), ``u`` returned in the input dtype,
gradients for all nine tensors (``grad_B`` / ``grad_Q`` summed over heads, the
symmetric gradient for ``Q`` / ``Q_f``), ``RuntimeError`` on numerical trouble
(``fused_lqr.py:101,246``).  The arithmetic runs in the C ABI of
``libttc_lqr.so`` (``include/ttc_lqr.h``); this module only validates, pads,
allocates with torch's caching allocator and checks the device status word.

Differences from the reference, by design:
* ``d`` / ``du`` of any size up to 64: the kernels handle ``d == du`` in
  {16, 32, 64}; other sizes are zero-padded here (padded states start at 0 and
  are neither driven nor costed; padded controls act on nothing and cost
  ``u^2/2``), which leaves the solution unchanged.
* backward: the forward keeps a small stash per problem (``V_1``, the step-1 value
  matrix, and ``Quu_0``; d^2 + du^2 floats) and the backward rolls the optimal
  primal and adjoint trajectories forward with the Hamiltonian recursion, as the
  reference's fused backward does (``symplectic_iter.py:542-885``), but every
  problem is certified (the terminal condition ``lambda_T = Q_f h_T`` must hold to
  ``TTC_LQR_CERT_TOL``) and problems that fail are recomputed by the stable path
  (per-step gains, closed-loop costates).  ``stable_backward=True`` uses the stable
  path for every problem.
* ``precision``: the Riccati sweep (the feedback gains) runs in fp32 or fp64.
  The fp32 sweep runs on the matrix cores (MFMA) as the symplectic sweep (three
  matrix products per step, one certified solve at the end; the problems the
  certificate rejects are recomputed with Riccati steps, then by the row-layout
  kernel).  ``"auto"`` (default): for horizons ``T >= FP64_HORIZON`` (512) the
  problems the symplectic certificate rejects are recomputed in fp64 instead, and the
  backward's stable path runs in fp64 -- on long, barely discounted horizons the value
  matrix reaches ~1e17 and fp32 rounding corrupts the gains of those problems (the
  reference's own fp32 solvers lose the gradients entirely there).  ``"fp64"``: every
  sweep in fp64 (row layout).  ``"fp32-riccati"`` selects per-step Riccati on the matrix
  cores, ``"fp32-row"`` the vector-ALU row-layout kernels (forward sweep and backward
  rollout), ``"riccati"`` per-step Riccati in fp32 or, at long horizons, in fp64.

Environment knobs:
``TTC_LQR_STASH`` = ``auto`` (default: keep the stash from the forward when it fits
in half of the device memory available at forward time (free on the device plus
held unallocated by torch's caching allocator), capped by
``TTC_LQR_STASH_MAX_BYTES`` if set) | ``always`` | ``never`` (the backward then
recomputes it with one forward sweep).
``TTC_LQR_STATUS_CHECK`` = ``sync`` (default) | ``deferred``: the default of ``status_check``
(see :func:`hip_lqr_solve`).
``TTC_LQR_WORKSPACE_BYTES``: backward workspace per call (default: 16 GiB or half of the
memory available at backward time, whichever is smaller; the library splits the tokens
into passes that fit, and one pass is fastest).
"""
from __future__ import annotations

import contextlib
import ctypes
import math
import os

import torch

from ._lib import lib, check, FLAG_FP64_RICCATI, FLAG_ROW_KERNEL, FLAG_STABLE_BWD, FLAG_RICCATI_STEPS, \
    FLAG_COMPACT_STASH, FLAG_FP64_RESCUE, FLAG_FP64_FALLBACK, FLAG_KEEP_EXPANDED, FLAG_RESCUE_V1, FLAG_RESCUE_GAINS

__all__ = ["hip_lqr_solve", "HipLQRSolveFunc", "hip_lqr_solve_factored", "HipLQRFactoredFunc", "padded_dim",
           "check_deferred_status",
           "SUPPORTED_DIMS", "last_backward_stats"]

SUPPORTED_DIMS = (16, 32, 64)
FP64_HORIZON = 512
_FWD_MSG = "Numerical instability detected during fused LQR forward recurrence."
_BWD_MSG = "Numerical instability detected during fused LQR backward pass."
_ERROR_BITS = 1 | 2  # TTC_LQR_STATUS_NONFINITE | TTC_LQR_STATUS_LARGE (4 = RESCUED is informational)
_RESCUED = 4  # TTC_LQR_STATUS_RESCUED
_RESCALE_MODES = {"none": 0, "l2_norm": 1, "h0_norm": 2}  # TTC_LQR_RESCALE_*

# problems / fallback problems of the most recent backward call (observability)
last_backward_stats = {"problems": 0, "fallback": 0}


def padded_dim(d: int, du: int) -> int:
    m = max(d, du)
    for s in SUPPORTED_DIMS:
        if m <= s:
            return s
    raise AssertionError(f"state/control dims up to {SUPPORTED_DIMS[-1]} are supported, got d={d}, du={du}")


def _env_bytes(name: str, default: int) -> int:
    v = os.environ.get(name)
    return int(float(v)) if v else default


def _pad_inputs(ins, d, du, Dp):
    """Zero-pad the nine solver inputs from (d, du) to (Dp, Dp)."""
    A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0 = ins
    if d == Dp and du == Dp:
        return ins
    pd, pu = Dp - d, Dp - du
    F = torch.nn.functional
    A_diag = F.pad(A_diag, (0, pd))
    B = F.pad(B, (0, pu, 0, pd))
    Q = F.pad(Q, (0, pd, 0, pd))
    R_inv = F.pad(R_inv, (0, pu), value=1.0)
    Q_f = F.pad(Q_f, (0, pd, 0, pd))
    lgB = F.pad(lgB, (0, pu))
    lgQ = F.pad(lgQ, (0, pd))
    h0 = F.pad(h0, (0, pd))
    return [t.contiguous() for t in (A_diag, B, Q, R_inv, Q_f, lgA, lgB, lgQ, h0)]


def riccati_flags(precision: str, T: int, Dp: int) -> int:
    """Kernel flags for the requested Riccati arithmetic (fp64 kernels exist for d <= 32).

    ``"fp32"``: the fastest fp32 kernels (matrix cores; symplectic sweep); ``"riccati"``:
    as ``"auto"``, with a Riccati step at every horizon step where the sweep runs in fp32;
    ``"fp32-riccati"``: per-step Riccati on the matrix cores; ``"fp32-row"``: the
    row-layout fp32 kernels (vector ALU only, forward and the backward's rollout) -- an
    independent cross-check of the matrix-core kernels; ``"fp64"``:
    fp64 sweep; ``"auto"`` (state dims up to 32): for T >= FP64_HORIZON the fp64 rescue of the
    sweep's rejected problems and the fp64 backward (``TTC_LQR_FLAG_FP64_RESCUE``); below it the
    fp64 rescue with the fp32 matrix-core backward, whose rejected problems take the fp64
    stable path (``TTC_LQR_FLAG_FP64_FALLBACK``); d = 64 stays fp32.
    """
    assert precision in ("fp32", "fp32-riccati", "fp32-row", "fp64", "auto", "riccati"), \
        f"unknown precision {precision}"
    long_fp64 = T >= FP64_HORIZON and lib.ttc_lqr_supported_flags(Dp, Dp, FLAG_FP64_RICCATI)
    if precision == "riccati":
        return FLAG_FP64_RICCATI if long_fp64 else FLAG_RICCATI_STEPS
    if precision == "fp32-row":
        return FLAG_ROW_KERNEL
    if precision == "fp32-riccati":
        return FLAG_RICCATI_STEPS
    if precision == "fp64":
        assert lib.ttc_lqr_supported_flags(Dp, Dp, FLAG_FP64_RICCATI), \
            f"fp64 Riccati kernels exist for state dims up to 32, got {Dp}"
        return FLAG_FP64_RICCATI
    if precision == "auto" and long_fp64:
        return FLAG_FP64_RESCUE
    if precision == "auto" and lib.ttc_lqr_supported_flags(Dp, Dp, FLAG_FP64_FALLBACK):
        return FLAG_FP64_FALLBACK
    return 0


def backward_flags(flags: int, forward_status: int) -> int:
    """Flags of the backward after a forward that reported ``forward_status``: under
    ``TTC_LQR_FLAG_FP64_FALLBACK`` the stable path runs in fp64 only when the forward's certificate
    rejected some problem of the batch (``TTC_LQR_STATUS_RESCUED``); a batch it certified whole
    has no problem that needs fp64, and the fp32 stable path is cheaper."""
    if flags & FLAG_FP64_FALLBACK and not forward_status & _RESCUED:
        return flags & ~FLAG_FP64_FALLBACK
    return flags


def _fallback_slack(P: int, Dp: int, T: int, flags: int) -> int:
    """Extra backward workspace for the problems the certificate rejects: long horizons reject
    many (config 5: about a fifth), and each fallback pass is a serial T-step sweep, so give
    room for a quarter of the problems in one pass (capped by the workspace budget)."""
    if T < FP64_HORIZON or P <= 0:
        return 0
    return lib.ttc_lqr_fallback_bytes(max(P // 4, 8), Dp, Dp, T, flags)


def _stash_budget(device) -> int:
    """Half of the memory available to new tensors: free on the device plus what torch's
    caching allocator holds unallocated (e.g. the previous step's freed stash)."""
    free, _total = torch.cuda.mem_get_info(device)
    cached = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    budget = (free + max(cached, 0)) // 2
    cap = os.environ.get("TTC_LQR_STASH_MAX_BYTES")
    return min(budget, int(float(cap))) if cap else budget


def _stash_fits(device, nbytes: int) -> bool:
    """``nbytes <= _stash_budget(device)``, deciding from the device's free memory alone when
    half of it suffices (one driver query, a few microseconds): torch's allocator counters,
    which the full budget reads, cost hundreds of microseconds per call."""
    cap = os.environ.get("TTC_LQR_STASH_MAX_BYTES")
    if cap and nbytes > int(float(cap)):
        return False
    free, _total = torch.cuda.mem_get_info(device)
    return nbytes <= free // 2 or nbytes <= _stash_budget(device)


def _stream_handle(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


@contextlib.contextmanager
def _stage(dev, name: str):
    """The device of a library call, inside a profiler range named after the reference's stage it
    covers (``torch.profiler.record_function``, as the reference names its stages,
    ``fused_lqr.py:58,103,112,186,200``): ``fwd:lqr_symplectic_rev_iter`` is the forward call
    (the sweep, the final solve -- the reference's ``fwd:torch.linalg.lu_solve`` -- and step 0 --
    its ``fwd:lqr_symplectic_dec_first_step`` -- run in one launch sequence here),
    ``bwd:lqr_symplectic_fwd_iter_diff`` the backward call (its ``Quu_0`` solve is the
    reference's ``bwd:torch.linalg.lu_solve``); ``*:ttc_lqr_status`` is the host's wait for the
    status word."""
    if dev is None:
        with torch.profiler.record_function(name):
            yield
        return
    with torch.cuda.device(dev), torch.profiler.record_function(name):
        yield


def _read_status(status, name: str) -> int:
    with _stage(None, name):
        return int(status.item())


# Status words of forwards run with status_check="deferred" that nothing has read yet.
_deferred: list = []
_DEFERRED_MAX = 1024  # pending words that trigger a check of all of them


def _deferred_mode(status_check: str | None) -> bool:
    mode = status_check or os.environ.get("TTC_LQR_STATUS_CHECK", "sync")
    assert mode in ("sync", "deferred"), f"unknown status_check {mode}"
    return mode == "deferred"


def _defer(status):
    """Keep a forward's device status word for a later check (no host synchronisation now)."""
    if len(_deferred) >= _DEFERRED_MAX:
        check_deferred_status()
    _deferred.append(status)


def _take_deferred(status) -> int:
    """Read one deferred status word (the backward's own forward), raising the forward's error."""
    for i, t in enumerate(_deferred):
        if t is status:
            del _deferred[i]
            break
    fst = _read_status(status, "bwd:ttc_lqr_forward_status")
    if fst & _ERROR_BITS:
        raise RuntimeError(_FWD_MSG)
    return fst


def check_deferred_status(keep: bool = False) -> None:
    """Read the status words of the forwards run with ``status_check="deferred"`` that no backward
    has read yet (one synchronisation), forget them (unless ``keep``), and raise the reference's
    forward ``RuntimeError`` (``fused_lqr.py:101``) if any of those forwards met a non-finite value.
    A forward in deferred mode enqueues its kernels and returns without waiting for them, so it can
    be recorded by HIP graph capture; its error surfaces here, or in its backward.  A forward
    captured in a graph registers its status word once, when it is captured, and every replay
    rewrites that word: ``keep=True`` checks it after each replay without dropping it."""
    pending = list(_deferred)
    if not keep:
        _deferred.clear()
    bad = False
    for t in pending:
        bad |= bool(_read_status(t, "fwd:ttc_lqr_status") & _ERROR_BITS)
    if bad:
        raise RuntimeError(_FWD_MSG)


class HipLQRSolveFunc(torch.autograd.Function):

    @staticmethod
    def forward(ctx, A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T: int,
                grad_limit: float = 1e6, stash: str | None = None, precision: str = "auto",
                stable_backward: bool = False, status_check: str | None = None):
        ins = [A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0]
        assert all(x.is_cuda for x in ins), "hip LQR solver inputs must be on a GPU"
        bs, nh, d = A_diag.shape
        du = B.shape[-1]
        T = int(T)
        assert T > 0
        assert A_diag.shape == (bs, nh, d)
        assert Q.shape == (bs, d, d)
        assert B.shape == (bs, d, du)
        assert R_inv_diag.shape == (bs, nh, du)
        assert Q_f.shape == (bs, nh, d, d)
        assert log_gamma_A.shape == (bs, nh)
        assert log_gamma_B.shape == (bs, nh, du)
        assert log_gamma_Q.shape == (bs, nh, d)
        assert h0.shape == (bs, nh, d)
        dev = A_diag.device
        out_dtype = Q.dtype
        Dp = padded_dim(d, du)
        flags = riccati_flags(precision, T, Dp)
        f32 = [x.detach().to(torch.float32).contiguous() for x in ins]
        f32 = _pad_inputs(f32, d, du, Dp)
        u = torch.empty(bs, nh, Dp, device=dev, dtype=torch.float32)
        status = torch.zeros(1, device=dev, dtype=torch.int32)

        policy = stash or os.environ.get("TTC_LQR_STASH", "auto")
        assert policy in ("auto", "always", "never"), f"unknown stash policy {policy}"
        need_grad = any(ctx.needs_input_grad[:9])
        stash_bytes = lib.ttc_lqr_stash_bytes(bs, nh, Dp, Dp, T)
        keep = (need_grad and bs > 0 and not stable_backward
                and (policy == "always" or (policy == "auto" and _stash_fits(dev, stash_bytes))))
        st_bytes = stash_bytes
        if keep and _rescue_v1(flags, Dp):  # the rescue's fp64 V_1 / Quu_0 after the stash
            flags |= FLAG_RESCUE_V1
            st_bytes = _align256(stash_bytes) + lib.ttc_lqr_rescue_stash_bytes(bs, nh, Dp, Dp)
            # and its fp64 gains, when they fit the stash budget too
            with_gains = st_bytes + lib.ttc_lqr_rescue_gains_bytes(bs, nh, Dp, Dp, T)
            if _keep_rescue_gains(dev, policy, with_gains):
                flags |= FLAG_RESCUE_GAINS
                st_bytes = with_gains
        st = torch.empty(st_bytes // 4, device=dev, dtype=torch.float32) if keep else None
        # the fp64 rescue's problem list (4 bytes a problem; long horizons only)
        fws_bytes = lib.ttc_lqr_forward_workspace_bytes(bs, nh, Dp, Dp, T, flags)
        fws = torch.empty(fws_bytes, device=dev, dtype=torch.uint8) if fws_bytes > 0 else None
        with _stage(dev, "fwd:lqr_symplectic_rev_iter"):
            rc = lib.ttc_lqr_forward_ws(*[t.data_ptr() for t in f32], bs, nh, Dp, Dp, T, flags, u.data_ptr(),
                                        None if st is None else st.data_ptr(),
                                        None if fws is None else fws.data_ptr(), fws_bytes, status.data_ptr(),
                                        _stream_handle(dev))
        check(rc, "ttc_lqr_forward_ws")
        ctx.fwd_status = None
        if _deferred_mode(status_check):  # read by the backward or check_deferred_status()
            _defer(status)
            ctx.fwd_status = status
        else:
            fst = _read_status(status, "fwd:ttc_lqr_status")
            if fst & _ERROR_BITS:
                raise RuntimeError(_FWD_MSG)
            flags = backward_flags(flags, fst)
        if need_grad:
            ctx.save_for_backward(*f32, u, *([st] if st is not None else []))
        ctx.meta = (bs, nh, d, du, Dp, T, float(grad_limit), st is not None, [x.dtype for x in ins],
                    flags | (FLAG_STABLE_BWD if stable_backward else 0))
        return u[..., :du].to(out_dtype)

    @staticmethod
    def backward(ctx, d_u):
        bs, nh, d, du, Dp, T, grad_limit, has_stash, dtypes, flags = ctx.meta
        if ctx.fwd_status is not None:  # deferred: the forward's status word, read now
            flags = backward_flags(flags, _take_deferred(ctx.fwd_status))
        saved = ctx.saved_tensors
        f32 = list(saved[:9])
        u = saved[9]
        st = saved[10] if has_stash else None
        dev = f32[0].device
        if du == Dp:
            dU = d_u.to(torch.float32).contiguous()
        else:
            dU = torch.zeros(bs, nh, Dp, device=dev, dtype=torch.float32)
            dU[..., :du] = d_u.to(torch.float32)
        g = {
            "A": torch.empty(bs, nh, Dp, device=dev), "B": torch.empty(bs, Dp, Dp, device=dev),
            "Q": torch.empty(bs, Dp, Dp, device=dev), "R": torch.empty(bs, nh, Dp, device=dev),
            "Qf": torch.empty(bs, nh, Dp, Dp, device=dev), "lA": torch.empty(bs, nh, device=dev),
            "lB": torch.empty(bs, nh, Dp, device=dev), "lQ": torch.empty(bs, nh, Dp, device=dev),
            "h0": torch.empty(bs, nh, Dp, device=dev),
        }
        status = torch.zeros(1, device=dev, dtype=torch.int32)
        with_st = 1 if st is not None else 0
        # one pass over all tokens when it fits the budget; the library picks the largest
        # token chunk that fits whatever it is given (at least one token's worth)
        full = lib.ttc_lqr_workspace_bytes(bs, nh, Dp, Dp, T, with_st, flags) + _fallback_slack(bs * nh, Dp, T, flags)
        ws = torch.empty(_workspace_bytes(full, lib.ttc_lqr_workspace_bytes(1, nh, Dp, Dp, T, with_st, flags), dev),
                         device=dev, dtype=torch.uint8)
        limit = grad_limit if math.isfinite(grad_limit) else float("inf")
        n_fb = ctypes.c_int64(0)
        with _stage(dev, "bwd:lqr_symplectic_fwd_iter_diff"):
            rc = lib.ttc_lqr_backward(
                *[t.data_ptr() for t in f32], u.data_ptr(), dU.data_ptr(), bs, nh, Dp, Dp, T, flags,
                None if st is None else st.data_ptr(),
                g["A"].data_ptr(), g["B"].data_ptr(), g["Q"].data_ptr(), g["R"].data_ptr(), g["Qf"].data_ptr(),
                g["lA"].data_ptr(), g["lB"].data_ptr(), g["lQ"].data_ptr(), g["h0"].data_ptr(),
                ws.data_ptr(), ws.numel(), limit, status.data_ptr(), ctypes.byref(n_fb), _stream_handle(dev))
        check(rc, "ttc_lqr_backward")
        last_backward_stats.update(problems=bs * nh, fallback=int(n_fb.value))
        if _read_status(status, "bwd:ttc_lqr_status") & _ERROR_BITS:
            raise RuntimeError(_BWD_MSG)
        out = (g["A"][..., :d], g["B"][:, :d, :du], g["Q"][:, :d, :d], g["R"][..., :du], g["Qf"][:, :, :d, :d],
               g["lA"], g["lB"][..., :du], g["lQ"][..., :d], g["h0"][..., :d])
        out = tuple(o.to(dt) if need else None for o, dt, need in zip(out, dtypes, ctx.needs_input_grad[:9]))
        return out + (None, None, None, None, None, None)


def hip_lqr_solve(A_diag: torch.Tensor, B: torch.Tensor, Q: torch.Tensor, R_inv_diag: torch.Tensor,
                  Q_f: torch.Tensor, log_gamma_A: torch.Tensor, log_gamma_B: torch.Tensor,
                  log_gamma_Q: torch.Tensor, h0: torch.Tensor, T: int, inv_guard: bool = False, *,
                  grad_limit: float = 1e6, stash: str | None = None, precision: str = "auto",
                  stable_backward: bool = False, status_check: str | None = None) -> torch.Tensor:
    """First optimal action ``u [N,H,du]`` of every (token, head) LQR problem.

    Drop-in for the reference ``fused_lqr_solve`` (``fused_lqr.py:294-304``): the same ten
    positional inputs and ``inv_guard`` in the eleventh slot.  ``inv_guard`` has no effect
    (as in the reference, whose ``fused_lqr_solve`` passes it into the ``cache_level`` slot of
    ``FusedLQRSolveFunc``, ``fused_lqr.py:268,304``); the keyword-only knobs below have no
    reference counterpart.
    ``grad_limit``: the backward raises when a gradient of ``A_diag``, ``B``, ``Q``, ``R_inv``,
    ``Q_f`` or ``h0`` reaches it (the reference's 1e6 guard, ``fused_lqr.py:243-246``, which
    does not cover the log-discount gradients); ``math.inf`` disables the magnitude check.
    ``stash``: ``"auto" | "always" | "never"`` overrides ``TTC_LQR_STASH``.
    ``precision``: ``"auto" | "riccati" | "fp32" | "fp32-riccati" | "fp32-row" | "fp64"``
    arithmetic (and, for ``"riccati"`` / ``"fp32-riccati"`` / ``"fp32-row"``, kernel) of the
    sweep; see ``riccati_flags``.
    ``stable_backward``: skip the certified Hamiltonian rollout and compute every
    problem's gradients with the stable path.
    ``status_check``: ``"sync"`` (default; ``TTC_LQR_STATUS_CHECK`` overrides it) reads the device
    status word after the forward's kernels and raises at once, as the reference does
    (``fused_lqr.py:99-110``); ``"deferred"`` returns without waiting for the kernels (no host
    synchronisation in the forward, so it can be recorded by HIP graph capture) and raises the same
    ``RuntimeError`` from the backward or from :func:`check_deferred_status`.
    """
    return HipLQRSolveFunc.apply(A_diag, B, Q, R_inv_diag, Q_f, log_gamma_A, log_gamma_B, log_gamma_Q, h0, T,
                                 grad_limit, stash, precision, stable_backward, status_check)


def _workspace_budget(dev) -> int:
    return _env_bytes("TTC_LQR_WORKSPACE_BYTES", min(16 << 30, max(1 << 30, _stash_budget(dev))))


def _align256(n: int) -> int:
    return (n + 255) // 256 * 256


def _rescue_v1(flags: int, Dp: int) -> bool:
    """Whether a forward with a stash keeps the fp64 V_1 / Quu_0 of the problems its fp64 rescue
    recomputes (``TTC_LQR_FLAG_RESCUE_V1``, d = 16, under ``TTC_LQR_FLAG_FP64_RESCUE``): the
    backward's fp64 second rollout tier then starts them from those instead of their fp32
    roundings, and more of them pass its certificate (each that does skips a stable-path sweep).
    When the stash budget also holds their fp64 gains (``TTC_LQR_FLAG_RESCUE_GAINS``, 2 MB a kept
    problem at T = 1024), the forward keeps those too and the backward's stable path reads them
    instead of sweeping those problems again."""
    return bool(flags & FLAG_FP64_RESCUE) and Dp == 16


def _keep_rescue_gains(dev, policy: str, nbytes: int) -> bool:
    """Whether a forward that keeps the rescue's fp64 V_1 also keeps its fp64 gains
    (``TTC_LQR_FLAG_RESCUE_GAINS``): when the stash with them (``nbytes``) fits the stash budget,
    or the stash policy is "always"."""
    return policy == "always" or _stash_fits(dev, nbytes)


def _keep_expanded(dev, kind: str, stash_bytes: int, expanded_bytes: int) -> bool:
    """Whether the factored forward keeps its expansion of B, Q and Q_f for the backward
    (``TTC_LQR_FLAG_KEEP_EXPANDED``: the backward then does not expand them again): with the full
    stash, when the stash and the expansion fit the stash budget together; never beside a compact
    stash, which is chosen when memory is short."""
    return kind == "full" and _stash_fits(dev, _align256(stash_bytes) + expanded_bytes)


def _workspace_bytes(full: int, floor: int, dev) -> int:
    """Bytes of a call's workspace: ``full`` (one pass) when the budget allows, else the budget,
    at least ``floor`` (one token's worth).  The default budget is never below 1 GiB, so a
    smaller ``full`` skips the device memory query; up to 16 GiB and half the device's free
    memory (one driver query) ``full`` is within the budget too, which then need not read
    torch's allocator counters (hundreds of microseconds per call)."""
    if not os.environ.get("TTC_LQR_WORKSPACE_BYTES"):
        if full <= 1 << 30:
            return max(full, floor, 256)
        if full <= 16 << 30 and full <= torch.cuda.mem_get_info(dev)[0] // 2:
            return max(full, floor, 256)
    return max(min(full, _workspace_budget(dev)), floor, 256)


class HipLQRFactoredFunc(torch.autograd.Function):
    """The solve on the layer's low-rank factors (``ttc_layer.py:117-123``): ``B``, ``Q`` and
    ``Q_f`` are expanded by the library per token chunk (in full only in the stash, see below).

    Inputs: ``A_diag [N,H,d]``, ``coeff_B [N,rb]``, ``coeff_Q [N,rq]``, ``R_inv [N,H,du]``,
    ``coeff_Qf [N,H,rq]``, ``log_gamma_A [N,H]``, ``log_gamma_B [N,H,du]``,
    ``log_gamma_Q [N,H,d]``, ``h0 [N,H,d]``, ``B_basis [rb,d,du]``, ``Q_basis [rq,d,d]``, ``T``;
    ``B = einsum("nr,rij->nij", coeff_B, B_basis)``, ``Q`` likewise, ``Q_f[n,h] =
    einsum("r,rij->ij", coeff_Qf[n,h], Q_basis)``.  Same ``u``, arithmetic, certificate,
    stash and error behaviour as :class:`HipLQRSolveFunc` on the expanded tensors.
    When all eleven tensors are bf16 they are handed to the library as bf16 (the ``_bf16``
    entry points widen each token chunk to fp32 in the workspace, and store the gradients as
    bf16); ``u`` is computed and kept in fp32 and returned as bf16.  Any other dtype mix is
    computed from fp32 copies.
    Stash: as :class:`HipLQRSolveFunc`; when the full stash does not fit the budget (``"auto"``)
    or ``stash="compact"``, only the upper triangles of ``V_1`` are kept
    (``TTC_LQR_FLAG_COMPACT_STASH``: 4x smaller at d = 64) and the backward recomputes
    ``Quu_0`` from them instead of re-running the forward sweep.  With the full stash, when the
    budget also holds the forward's expansion of ``B``, ``Q`` and ``Q_f`` (2.7 GB at config 2),
    the stash keeps it and the backward reads it instead of expanding again
    (``TTC_LQR_FLAG_KEEP_EXPANDED``; what the reference's layer keeps for autograd).
    ``rescale`` (``"none" | "l2_norm" | "h0_norm"``, fp32 storage): the layer's rescale of
    ``u`` (``ttc_layer.py:142-147``) fused into the call -- the result is the rescaled output
    and the backward takes its gradient (``ttc_lqr_rescale`` / ``ttc_lqr_rescale_backward``).
    """

    @staticmethod
    def forward(ctx, A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, log_gamma_A, log_gamma_B, log_gamma_Q, h0,
                B_basis, Q_basis, T: int, grad_limit: float = 1e6, stash: str | None = None,
                precision: str = "auto", stable_backward: bool = False, rescale: str = "none",
                status_check: str | None = None):
        ins = [A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, log_gamma_A, log_gamma_B, log_gamma_Q, h0,
               B_basis, Q_basis]
        assert rescale in _RESCALE_MODES, f"Unknown rescale method {rescale}"
        assert all(x.is_cuda for x in ins), "hip LQR solver inputs must be on a GPU"
        bs, nh, d = A_diag.shape
        rb, _, du = B_basis.shape
        rq = Q_basis.shape[0]
        T = int(T)
        assert T > 0
        assert coeff_B.shape == (bs, rb) and coeff_Q.shape == (bs, rq) and coeff_Qf.shape == (bs, nh, rq)
        assert B_basis.shape == (rb, d, du) and Q_basis.shape == (rq, d, d)
        assert R_inv_diag.shape == (bs, nh, du) and log_gamma_A.shape == (bs, nh)
        assert log_gamma_B.shape == (bs, nh, du) and log_gamma_Q.shape == (bs, nh, d) and h0.shape == (bs, nh, d)
        assert 1 <= rb <= 64 and 1 <= rq <= 64, f"ranks 1..64 are supported, got b_rank={rb}, q_rank={rq}"
        dev = A_diag.device
        out_dtype = A_diag.dtype
        bf16 = all(x.dtype == torch.bfloat16 for x in ins)
        store = torch.bfloat16 if bf16 else torch.float32
        mode = _RESCALE_MODES[rescale]
        assert not (mode and bf16), "the fused rescale runs on fp32 storage; rescale bf16 outputs outside"
        Dp = padded_dim(d, du)
        flags = riccati_flags(precision, T, Dp)
        F = torch.nn.functional
        xs = [x.detach().to(store).contiguous() for x in ins]
        pd, pu = Dp - d, Dp - du
        if pd or pu:  # zero-padded states / unit-cost dummy controls, as HipLQRSolveFunc
            xs[0] = F.pad(xs[0], (0, pd))
            xs[3] = F.pad(xs[3], (0, pu), value=1.0)
            xs[6] = F.pad(xs[6], (0, pu))
            xs[7] = F.pad(xs[7], (0, pd))
            xs[8] = F.pad(xs[8], (0, pd))
            xs[9] = F.pad(xs[9], (0, pu, 0, pd))
            xs[10] = F.pad(xs[10], (0, pd, 0, pd))
            xs = [t.contiguous() for t in xs]
        u = torch.empty(bs, nh, Dp, device=dev, dtype=torch.float32)
        status = torch.zeros(1, device=dev, dtype=torch.int32)
        policy = stash or os.environ.get("TTC_LQR_STASH", "auto")
        assert policy in ("auto", "always", "compact", "never"), f"unknown stash policy {policy}"
        need_grad = any(ctx.needs_input_grad[:11])
        stash_bytes = lib.ttc_lqr_stash_bytes(bs, nh, Dp, Dp, T)
        compact_bytes = lib.ttc_lqr_compact_stash_bytes(bs, nh, Dp, Dp)
        kind = None  # full / compact stash, or none (the backward re-runs the forward sweep)
        if need_grad and bs > 0 and not stable_backward and policy != "never":
            if policy == "always" or (policy == "auto" and _stash_fits(dev, stash_bytes)):
                kind = "full"
            elif policy == "compact" or _stash_fits(dev, compact_bytes):
                kind = "compact"
        if kind == "compact":
            flags |= FLAG_COMPACT_STASH
        st_bytes = stash_bytes if kind == "full" else compact_bytes
        if kind is not None and _keep_expanded(dev, kind, st_bytes, lib.ttc_lqr_expanded_bytes(bs, nh, Dp, Dp)):
            flags |= FLAG_KEEP_EXPANDED
            st_bytes = _align256(st_bytes) + lib.ttc_lqr_expanded_bytes(bs, nh, Dp, Dp)
        st = None if kind is None else torch.empty(st_bytes // 4, device=dev, dtype=torch.float32)
        ws_stash = {None: 0, "full": 1, "compact": 2}[kind]
        full = lib.ttc_lqr_factored_workspace_bytes(max(bs, 1), nh, Dp, Dp, rb, rq, T, ws_stash, 0, int(bf16), flags)
        one = lib.ttc_lqr_factored_workspace_bytes(1, nh, Dp, Dp, rb, rq, T, ws_stash, 0, int(bf16), flags)
        ws = torch.empty(_workspace_bytes(full, one, dev), device=dev, dtype=torch.uint8)
        fwd = lib.ttc_lqr_forward_factored_bf16 if bf16 else lib.ttc_lqr_forward_factored
        with _stage(dev, "fwd:lqr_symplectic_rev_iter"):
            rc = fwd(*[t.data_ptr() for t in xs], bs, nh, Dp, Dp, rb, rq, T, flags, u.data_ptr(),
                     None if st is None else st.data_ptr(), ws.data_ptr(), ws.numel(), status.data_ptr(),
                     _stream_handle(dev))
        check(rc, "ttc_lqr_forward_factored" + ("_bf16" if bf16 else ""))
        del ws
        y = u
        if mode:
            y = torch.empty_like(u)
            with _stage(dev, "fwd:ttc_lqr_rescale"):
                rc = lib.ttc_lqr_rescale(u.data_ptr(), xs[8].data_ptr(), bs, nh, Dp, Dp, mode, y.data_ptr(),
                                         _stream_handle(dev))
            check(rc, "ttc_lqr_rescale")
        ctx.fwd_status = None
        if _deferred_mode(status_check):  # read by the backward or check_deferred_status()
            _defer(status)
            ctx.fwd_status = status
        else:
            fst = _read_status(status, "fwd:ttc_lqr_status")
            if fst & _ERROR_BITS:
                raise RuntimeError(_FWD_MSG)
            flags = backward_flags(flags, fst)
        if need_grad:
            ctx.save_for_backward(*xs, u, *([st] if st is not None else []))
        ctx.meta = (bs, nh, d, du, Dp, rb, rq, T, float(grad_limit), st is not None, [x.dtype for x in ins],
                    flags | (FLAG_STABLE_BWD if stable_backward else 0), bf16, mode)
        return y[..., :du].to(out_dtype)

    @staticmethod
    def backward(ctx, d_u):
        bs, nh, d, du, Dp, rb, rq, T, grad_limit, has_stash, dtypes, flags, bf16, mode = ctx.meta
        if ctx.fwd_status is not None:  # deferred: the forward's status word, read now
            flags = backward_flags(flags, _take_deferred(ctx.fwd_status))
        saved = ctx.saved_tensors
        xs = list(saved[:11])
        u = saved[11]
        st = saved[12] if has_stash else None
        dev = xs[0].device
        store = torch.bfloat16 if bf16 else torch.float32
        if du == Dp:
            dU = d_u.to(store).contiguous()
        else:
            dU = torch.zeros(bs, nh, Dp, device=dev, dtype=store)
            dU[..., :du] = d_u.to(store)
        if mode:  # d_y -> d_u through the fused rescale
            dY, dU = dU, torch.empty_like(dU)
            with _stage(dev, "bwd:ttc_lqr_rescale_backward"):
                rc = lib.ttc_lqr_rescale_backward(u.data_ptr(), xs[8].data_ptr(), dY.data_ptr(), bs, nh, Dp, Dp, mode,
                                                  dU.data_ptr(), _stream_handle(dev))
            check(rc, "ttc_lqr_rescale_backward")
        E = lambda *shape: torch.empty(*shape, device=dev, dtype=store)  # noqa: E731
        g = [E(bs, nh, Dp), E(bs, rb), E(bs, rq), E(bs, nh, Dp), E(bs, nh, rq), E(bs, nh), E(bs, nh, Dp),
             E(bs, nh, Dp), E(bs, nh, Dp), E(rb, Dp, Dp), E(rq, Dp, Dp)]
        status = torch.zeros(1, device=dev, dtype=torch.int32)
        with_st = 0 if st is None else (2 if flags & FLAG_COMPACT_STASH else 1)
        full = (lib.ttc_lqr_factored_workspace_bytes(max(bs, 1), nh, Dp, Dp, rb, rq, T, with_st, 1, int(bf16), flags)
                + _fallback_slack(bs * nh, Dp, T, flags))
        one = lib.ttc_lqr_factored_workspace_bytes(1, nh, Dp, Dp, rb, rq, T, with_st, 1, int(bf16), flags)
        ws = torch.empty(_workspace_bytes(full, one, dev), device=dev, dtype=torch.uint8)
        limit = grad_limit if math.isfinite(grad_limit) else float("inf")
        n_fb = ctypes.c_int64(0)
        bwd = lib.ttc_lqr_backward_factored_bf16 if bf16 else lib.ttc_lqr_backward_factored
        with _stage(dev, "bwd:lqr_symplectic_fwd_iter_diff"):
            rc = bwd(*[t.data_ptr() for t in xs], u.data_ptr(), dU.data_ptr(), bs, nh, Dp, Dp, rb, rq, T, flags,
                     None if st is None else st.data_ptr(), *[t.data_ptr() for t in g], ws.data_ptr(), ws.numel(),
                     limit, status.data_ptr(), ctypes.byref(n_fb), _stream_handle(dev))
        check(rc, "ttc_lqr_backward_factored" + ("_bf16" if bf16 else ""))
        last_backward_stats.update(problems=bs * nh, fallback=int(n_fb.value))
        if _read_status(status, "bwd:ttc_lqr_status") & _ERROR_BITS:
            raise RuntimeError(_BWD_MSG)
        out = (g[0][..., :d], g[1], g[2], g[3][..., :du], g[4], g[5], g[6][..., :du], g[7][..., :d],
               g[8][..., :d], g[9][:, :d, :du], g[10][:, :d, :d])
        out = tuple(o.to(dt) if need else None for o, dt, need in zip(out, dtypes, ctx.needs_input_grad[:11]))
        return out + (None, None, None, None, None, None, None)


def hip_lqr_solve_factored(A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, log_gamma_A, log_gamma_B, log_gamma_Q,
                           h0, B_basis, Q_basis, T: int, grad_limit: float = 1e6, stash: str | None = None,
                           precision: str = "auto", stable_backward: bool = False,
                           rescale: str = "none", status_check: str | None = None) -> torch.Tensor:
    """``hip_lqr_solve`` on the layer's low-rank factors (see :class:`HipLQRFactoredFunc`):
    equal to ``hip_lqr_solve(A_diag, einsum(coeff_B, B_basis), einsum(coeff_Q, Q_basis), R_inv,
    einsum(coeff_Qf, Q_basis), ...)`` with gradients for the coefficients and both bases."""
    return HipLQRFactoredFunc.apply(A_diag, coeff_B, coeff_Q, R_inv_diag, coeff_Qf, log_gamma_A, log_gamma_B,
                                    log_gamma_Q, h0, B_basis, Q_basis, T, grad_limit, stash, precision,
                                    stable_backward, rescale, status_check)
