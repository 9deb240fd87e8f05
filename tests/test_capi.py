"""CPU tests of the C ABI boundary (no GPU work is launched).

* libttc_lqr.so loads and exports every function declared in include/ttc_lqr.h;
* size helpers follow the documented formulas;
* argument validation returns the documented codes before touching a device.
"""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ttc_lqr.h")
FLAG_ROW_KERNEL = 2  # TTC_LQR_FLAG_ROW_KERNEL


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ttc_lqr_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from ttc.solvers._lib import lib
    return lib


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted([
        "ttc_lqr_backward", "ttc_lqr_forward", "ttc_lqr_stash_bytes", "ttc_lqr_strerror",
        "ttc_lqr_supported", "ttc_lqr_supported_flags", "ttc_lqr_version", "ttc_lqr_workspace_bytes",
        "ttc_lqr_compact_stash_bytes", "ttc_lqr_expanded_bytes", "ttc_lqr_rescue_stash_bytes",
        "ttc_lqr_rescue_gains_bytes",
        "ttc_lqr_factored_workspace_bytes", "ttc_lqr_forward_factored", "ttc_lqr_backward_factored",
        "ttc_lqr_forward_factored_bf16", "ttc_lqr_backward_factored_bf16", "ttc_lqr_rescale",
        "ttc_lqr_rescale_backward", "ttc_lqr_forward_host", "ttc_lqr_backward_host", "ttc_lqr_fallback_bytes",
        "ttc_lqr_backward_noalloc", "ttc_lqr_noalloc_scratch_bytes", "ttc_lqr_forward_workspace_bytes",
        "ttc_lqr_forward_ws"])


def test_library_exports_every_declared_symbol(L):
    from ttc.solvers._lib import lib_path
    raw = ctypes.CDLL(lib_path())
    for name in declared_functions():
        assert hasattr(raw, name), f"{name} not exported by {lib_path()}"


def test_version_and_strerror(L):
    assert L.ttc_lqr_version().decode().startswith("ttc-lqr-gfx950")
    for code in range(5):
        assert L.ttc_lqr_strerror(code)
    assert L.ttc_lqr_strerror(99) == b"unknown error"


def test_supported_dims(L):
    for d in (16, 32, 64):
        assert L.ttc_lqr_supported(d, d) == 1
    for d, du in [(16, 32), (8, 8), (24, 24), (128, 128), (0, 0)]:
        assert L.ttc_lqr_supported(d, du) == 0


def test_supported_flags(L):
    assert L.ttc_lqr_supported_flags(16, 16, 1) == 1 and L.ttc_lqr_supported_flags(32, 32, 1) == 1
    assert L.ttc_lqr_supported_flags(64, 64, 1) == 0 and L.ttc_lqr_supported_flags(64, 64, 0) == 1
    assert L.ttc_lqr_supported_flags(16, 16, 4) == 1 and L.ttc_lqr_supported_flags(64, 64, 4 | 2) == 1
    assert L.ttc_lqr_supported_flags(16, 16, 8) == 1 and L.ttc_lqr_supported_flags(32, 32, 8 | 4) == 1
    assert L.ttc_lqr_supported_flags(64, 64, 16) == 1 and L.ttc_lqr_supported_flags(16, 16, 1024) == 0
    assert L.ttc_lqr_supported_flags(64, 64, 128 | 16) == 1  # TTC_LQR_FLAG_KEEP_EXPANDED, any d
    # TTC_LQR_FLAG_FP64_FALLBACK (64) needs the fp64 kernels: d <= 32
    assert L.ttc_lqr_supported_flags(16, 16, 64) == 1 and L.ttc_lqr_supported_flags(32, 32, 64) == 1
    assert L.ttc_lqr_supported_flags(64, 64, 64) == 0
    # it lists the fp64 rescue's problems in the forward workspace, as TTC_LQR_FLAG_FP64_RESCUE does
    assert L.ttc_lqr_forward_workspace_bytes(3, 8, 16, 16, 64, 64) == 4 * (3 * 8 + 64)
    assert L.ttc_lqr_forward_workspace_bytes(3, 8, 16, 16, 64, 0) == 0
    assert _fwd(L, flags=16) == 2          # the compact stash needs the factored entry points
    assert _fwd(L, d=64, du=64, flags=1) == 2


def test_stash_bytes_formula(L):
    # per problem: V_1 (d x d) + Quu_0 (du x du), fp32 -- independent of T
    N, H, d, T = 262144, 8, 16, 64
    assert L.ttc_lqr_stash_bytes(N, H, d, d, T) == 4 * N * H * (d * d + d * d)
    assert L.ttc_lqr_stash_bytes(N, H, d, d, 1024) == L.ttc_lqr_stash_bytes(N, H, d, d, T)
    assert L.ttc_lqr_stash_bytes(-1, H, d, d, T) == 0


def test_workspace_bytes_monotone_and_stash_smaller(L):
    a = L.ttc_lqr_workspace_bytes(1, 8, 16, 16, 64, 0, 0)
    b = L.ttc_lqr_workspace_bytes(100000, 8, 16, 16, 64, 0, 0)
    s = L.ttc_lqr_workspace_bytes(100000, 8, 16, 16, 64, 1, 0)
    assert 0 < a < b and 0 < s < b
    P = 800000
    # without the stash: V_1 and Quu_0 of every problem
    assert b - s >= 4 * P * (2 * 256)
    # the fallback region is capped (256 MiB + alignment), so large chunks grow linearly.  Per
    # problem: the fallback-list entry, and the grad_B / grad_Q partials of the head sums --
    # none when a head group of 8 is the token (H = 8, it writes the outputs) ...
    c = L.ttc_lqr_workspace_bytes(200000, 8, 16, 16, 64, 1, 0)
    assert abs((c - s) - 4 * P * 1) < 4096
    # ... one per head group of 8 (H = 16: two per token) ...
    s16 = L.ttc_lqr_workspace_bytes(50000, 16, 16, 16, 64, 1, 0)
    c16 = L.ttc_lqr_workspace_bytes(100000, 16, 16, 16, 64, 1, 0)
    assert abs((c16 - s16) - 4 * P * (1 + 2 * 256 / 8)) < 4096
    # ... one per problem on the row-layout rollout
    sr = L.ttc_lqr_workspace_bytes(100000, 8, 16, 16, 64, 1, FLAG_ROW_KERNEL)
    cr = L.ttc_lqr_workspace_bytes(200000, 8, 16, 16, 64, 1, FLAG_ROW_KERNEL)
    assert abs((cr - sr) - 4 * P * (1 + 2 * 256)) < 4096
    assert L.ttc_lqr_workspace_bytes(0, 8, 16, 16, 64, 0, 0) == 0


def _fwd(L, n=1, h=1, d=16, du=16, T=1, null_inputs=False, flags=0):
    p = None if null_inputs else ctypes.c_void_p(16)   # never dereferenced: validation fails first
    return L.ttc_lqr_forward(*([p] * 9), n, h, d, du, T, flags, p, None, None, None)


def test_forward_argument_validation(L):
    from ttc.solvers._lib import lib  # noqa: F401
    assert _fwd(L, n=-1) == 1                 # TTC_LQR_EINVAL
    assert _fwd(L, T=0) == 1
    assert _fwd(L, d=24, du=24) == 2          # TTC_LQR_EUNSUPPORTED
    assert _fwd(L, d=16, du=32) == 2
    assert _fwd(L, n=0) == 0                  # empty batch: nothing to do
    assert _fwd(L, null_inputs=True) == 1


def test_forward_workspace_bytes(L):
    """The forward's optional workspace holds the fp64 rescue's problem list: 4 bytes a
    problem plus a 256-byte header, only under TTC_LQR_FLAG_FP64_RESCUE at d <= 32."""
    from ttc.solvers._lib import FLAG_FP64_RESCUE
    assert L.ttc_lqr_forward_workspace_bytes(1000, 8, 16, 16, 1024, FLAG_FP64_RESCUE) == 4 * (8000 + 64)
    assert L.ttc_lqr_forward_workspace_bytes(1000, 8, 32, 32, 1024, FLAG_FP64_RESCUE) == 4 * (8000 + 64)
    assert L.ttc_lqr_forward_workspace_bytes(1000, 8, 64, 64, 1024, FLAG_FP64_RESCUE) == 0
    assert L.ttc_lqr_forward_workspace_bytes(1000, 8, 16, 16, 64, 0) == 0
    assert L.ttc_lqr_forward_workspace_bytes(0, 8, 16, 16, 1024, FLAG_FP64_RESCUE) == 0
    # validation of the workspace entry matches ttc_lqr_forward's
    p = ctypes.c_void_p(16)
    assert L.ttc_lqr_forward_ws(*([p] * 9), -1, 1, 16, 16, 1, 0, p, None, None, 0, None, None) == 1
    assert L.ttc_lqr_forward_ws(*([p] * 9), 1, 1, 24, 24, 1, 0, p, None, None, 0, None, None) == 2
    assert L.ttc_lqr_forward_ws(*([p] * 9), 0, 1, 16, 16, 1, 0, p, None, None, 0, None, None) == 0


def test_backward_argument_validation(L):
    p = ctypes.c_void_p(16)
    head = [p] * 11                      # nine inputs, u, d_u
    tail = [float("inf"), None, None, None]   # grad_limit, status, n_fallback, stream
    args = head + [1, 1, 16, 16, 4, 0, None] + [p] * 9
    assert L.ttc_lqr_backward(*args, p, 0, *tail) == 1            # workspace too small
    bad = head + [1, 1, 20, 20, 4, 0, None] + [p] * 9
    assert L.ttc_lqr_backward(*bad, p, 1 << 30, *tail) == 2       # unsupported dims
    no_u = [p] * 9 + [None, p] + [1, 1, 16, 16, 4, 0, None] + [p] * 9
    assert L.ttc_lqr_backward(*no_u, p, 1 << 30, *tail) == 1      # fast path needs u
    n_fb = ctypes.c_int64(-7)
    empty = head + [0, 1, 16, 16, 4, 0, None] + [p] * 9
    assert L.ttc_lqr_backward(*empty, p, 0, float("inf"), None, ctypes.byref(n_fb), None) == 0
    assert n_fb.value == 0


def test_factored_workspace_bytes(L):
    # forward: the expanded B, Q (per token) and Q_f (per problem) of one chunk
    N, H, d, T = 1000, 8, 16, 64
    f = L.ttc_lqr_factored_workspace_bytes(N, H, d, d, 16, 16, T, 0, 0, 0, 0)
    assert 4 * N * (2 * d * d + H * d * d) <= f < 4 * N * (2 * d * d + H * d * d) + 1024
    # backward: also the chunk's gradients of B, Q, Q_f and ttc_lqr_backward's own workspace
    b = L.ttc_lqr_factored_workspace_bytes(N, H, d, d, 16, 16, T, 1, 1, 0, 0)
    assert b >= 2 * f + L.ttc_lqr_workspace_bytes(N, H, d, d, T, 1, 0)
    assert L.ttc_lqr_factored_workspace_bytes(2 * N, H, d, d, 16, 16, T, 1, 1, 0, 0) > b
    # bf16 storage: plus fp32 copies of the chunk's inputs (and d_u, gradients) and of the bases
    per_in = 3 * d + 2 * d + 1 + 16              # A, R, lgB, lgQ, h0, lgA, coeff_Qf per problem
    fb = L.ttc_lqr_factored_workspace_bytes(N, H, d, d, 16, 16, T, 0, 0, 1, 0)
    # the forward's expansion reads bf16 coefficients directly: no fp32 copy of coeff_B / Q / Q_f
    assert 4 * (N * H * (per_in - 16) + 2 * 16 * d * d) <= fb - f < 4 * (N * H * per_in + 2 * 16 * d * d)
    bb = L.ttc_lqr_factored_workspace_bytes(N, H, d, d, 16, 16, T, 1, 1, 1, 0)
    assert bb - b >= 4 * (N * H * (2 * per_in + d) + 4 * 16 * d * d)
    for bad in [(N, H, d, d, 0, 16), (N, H, d, d, 16, 65), (0, H, d, d, 16, 16), (N, H, 16, 32, 16, 16)]:
        assert L.ttc_lqr_factored_workspace_bytes(*bad, T, 0, 0, 0, 0) == 0


def test_factored_argument_validation(L):
    p = ctypes.c_void_p(16)
    odd = ctypes.c_void_p(20)   # not 16-byte aligned
    ws = 1 << 30

    def fwd(n=1, rb=16, rq=16, basis=p, work=ws, d=16):
        return L.ttc_lqr_forward_factored(*([p] * 9), basis, basis, n, 1, d, d, rb, rq, 4, 0, p, None, p, work,
                                          None, None)
    assert fwd(rb=0) == 1 and fwd(rq=65) == 1 and fwd(n=-1) == 1
    assert fwd(d=24) == 2
    assert fwd(basis=odd) == 1
    assert fwd(work=16) == 1                  # workspace below one token's expansion
    assert fwd(n=0) == 0

    def bwd(rb=16, basis=p, work=ws):
        n_fb = ctypes.c_int64(-3)
        rc = L.ttc_lqr_backward_factored(*([p] * 9), basis, basis, p, p, 1, 1, 16, 16, rb, 16, 4, 0, None,
                                         *([p] * 11), p, work, float("inf"), None, ctypes.byref(n_fb), None)
        return rc, n_fb.value
    assert bwd(rb=70) == (1, 0)
    assert bwd(basis=odd) == (1, 0)
    assert bwd(work=64) == (1, 0)


def test_keep_expanded_sizing_and_validation(L):
    """TTC_LQR_FLAG_KEEP_EXPANDED (128): the expanded B, Q, Q_f after the stash take
    align256 of each array; the factored workspaces then hold no expansion of their own; and
    the flag without a stash is rejected before any device work."""
    a = lambda n: (n + 255) // 256 * 256  # noqa: E731
    assert L.ttc_lqr_expanded_bytes(10, 8, 16, 16) == a(4 * 10 * 256) + a(4 * 10 * 256) + a(4 * 80 * 256)
    assert L.ttc_lqr_expanded_bytes(3, 2, 32, 32) == a(4 * 3 * 1024) * 2 + a(4 * 6 * 1024)
    for backward in (0, 1):
        plain = L.ttc_lqr_factored_workspace_bytes(100, 8, 16, 16, 16, 16, 64, 1, backward, 0, 0)
        kept = L.ttc_lqr_factored_workspace_bytes(100, 8, 16, 16, 16, 16, 64, 1, backward, 0, 128)
        assert plain - kept == a(4 * 100 * 256) * 2 + a(4 * 800 * 256)
    p = ctypes.c_void_p(16)
    assert L.ttc_lqr_forward_factored(*([p] * 11), 1, 1, 16, 16, 16, 16, 4, 128, p, None, p, 1 << 30,
                                      None, None) == 1
    n_fb = ctypes.c_int64(-3)
    assert L.ttc_lqr_backward_factored(*([p] * 11), p, p, 1, 1, 16, 16, 16, 16, 4, 128, None, *([p] * 11), p,
                                       1 << 30, float("inf"), None, ctypes.byref(n_fb), None) == 1


def test_rescue_v1_sizing_and_validation(L):
    """TTC_LQR_FLAG_RESCUE_V1 (256): d = du = 16 only; after the stash a slot index per problem and
    min(P, max(64, P / 8)) slots of 2 x 256 doubles, each region 256-byte aligned; the flag without
    a stash is rejected, and the factored entry points do not take it."""
    a = lambda n: (n + 255) // 256 * 256  # noqa: E731
    assert L.ttc_lqr_supported_flags(16, 16, 256 | 32) == 1
    assert L.ttc_lqr_supported_flags(32, 32, 256 | 32) == 0 and L.ttc_lqr_supported_flags(64, 64, 256) == 0
    for n, h in ((1000, 8), (3, 2), (20, 8)):
        P = n * h
        slots = min(P, max(64, P // 8))
        assert L.ttc_lqr_rescue_stash_bytes(n, h, 16, 16) == a(4 * P) + a(8 * slots * 512)
    p = ctypes.c_void_p(16)
    assert _fwd(L, flags=256 | 32) == 1                      # no stash
    n_fb = ctypes.c_int64(-3)
    assert L.ttc_lqr_backward(*([p] * 11), 1, 1, 16, 16, 4, 256 | 32, None, *([p] * 9), p, 1 << 30,
                              float("inf"), None, ctypes.byref(n_fb), None) == 1
    assert L.ttc_lqr_forward_factored(*([p] * 11), 1, 1, 16, 16, 16, 16, 4, 256 | 32, p, p, p, 1 << 30,
                                      None, None) == 2


def test_rescue_gains_sizing_and_validation(L):
    """TTC_LQR_FLAG_RESCUE_GAINS (512): only with TTC_LQR_FLAG_RESCUE_V1 (so d = du = 16); after
    that record every gain K_t of G = min(S, max(64, P / 16)) slots in fp64, T x du x d each,
    256-byte aligned; the factored entry points do not take it."""
    a = lambda n: (n + 255) // 256 * 256  # noqa: E731
    assert L.ttc_lqr_supported_flags(16, 16, 512 | 256 | 32) == 1
    assert L.ttc_lqr_supported_flags(16, 16, 512 | 32) == 0          # without the slots
    assert L.ttc_lqr_supported_flags(32, 32, 512 | 256 | 32) == 0
    for n, h, T in ((1000, 8, 1024), (3, 2, 5), (20, 8, 64), (32768, 8, 1024)):
        P = n * h
        S = min(P, max(64, P // 8))
        G = min(S, max(64, P // 16))
        assert L.ttc_lqr_rescue_gains_bytes(n, h, 16, 16, T) == a(8 * G * T * 256)
    # config 5b: 16,384 kept problems of 2 MB each
    assert L.ttc_lqr_rescue_gains_bytes(32768, 8, 16, 16, 1024) == 16384 * 1024 * 256 * 8
    assert L.ttc_lqr_rescue_gains_bytes(-1, 8, 16, 16, 4) == 0 and L.ttc_lqr_rescue_gains_bytes(1, 8, 16, 16, 0) == 0
    p = ctypes.c_void_p(16)
    assert _fwd(L, flags=512 | 32) == 2                       # unsupported without 256
    assert _fwd(L, flags=512 | 256 | 32) == 1                 # no stash
    assert L.ttc_lqr_forward_factored(*([p] * 11), 1, 1, 16, 16, 16, 16, 4, 512 | 256 | 32, p, p, p, 1 << 30,
                                      None, None) == 2


def test_rescale_argument_validation(L):
    p = ctypes.c_void_p(16)
    assert L.ttc_lqr_rescale(p, p, 1, 1, 16, 16, 3, p, None) == 1          # unknown mode
    assert L.ttc_lqr_rescale(p, None, 1, 1, 16, 16, 2, p, None) == 1       # h0_norm needs h0
    assert L.ttc_lqr_rescale(p, p, 1, 1, 24, 24, 1, p, None) == 2          # unpadded dims
    assert L.ttc_lqr_rescale(p, p, 0, 1, 16, 16, 1, p, None) == 0          # nothing to do
    assert L.ttc_lqr_rescale_backward(p, p, None, 1, 1, 16, 16, 1, p, None) == 1


def test_compact_stash_bytes(L):
    assert L.ttc_lqr_compact_stash_bytes(1000, 16, 64, 64) == 4 * 16000 * 2080
    assert 4 * L.ttc_lqr_compact_stash_bytes(10, 8, 64, 64) < L.ttc_lqr_stash_bytes(10, 8, 64, 64, 1) * 1.02
    # the compact layout holds the chunk's full V_1 and Quu_0 besides
    a = L.ttc_lqr_factored_workspace_bytes(100, 8, 16, 16, 16, 16, 64, 1, 1, 0, 0)
    b = L.ttc_lqr_factored_workspace_bytes(100, 8, 16, 16, 16, 16, 64, 2, 1, 0, 0)
    assert b - a >= 4 * 800 * 2 * 256


def test_fallback_and_precision_sizing(L):
    """The stable path's region is sized by its arithmetic: fp64 (either fp64 flag, d <= 32)
    stores gains, Quu_0 and trajectories in doubles; fp32 runs need half of that."""
    FP64, RESCUE, STABLE = 1, 32, 4
    d, T = 16, 1024
    f32 = L.ttc_lqr_fallback_bytes(100, d, d, T, 0)
    f64 = L.ttc_lqr_fallback_bytes(100, d, d, T, FP64)
    assert f64 == L.ttc_lqr_fallback_bytes(100, d, d, T, RESCUE)
    # per problem and step: gains d*d, trajectory 4*d (fp64 doubles them)
    assert 8 * 100 * T * (d * d + 4 * d) <= f64 < 8 * 100 * T * (d * d + 4 * d) + 100 * 20000
    assert f32 < 0.6 * f64
    assert L.ttc_lqr_fallback_bytes(200, d, d, T, FP64) > f64 > 0
    assert L.ttc_lqr_fallback_bytes(0, d, d, T, FP64) == 0
    # d = 64 has no fp64 kernels: the flags do not change its size
    assert L.ttc_lqr_fallback_bytes(10, 64, 64, 128, FP64) == L.ttc_lqr_fallback_bytes(10, 64, 64, 128, 0)
    # the backward's workspace: the main layout (with the stash: two d x d partials and a list
    # entry per problem) plus a fallback reserve of at most 256 MiB, fp32 or fp64
    P = 8000
    # (under RESCUE at d = 16 with head groups of 8, also the third rollout tier: a list, a slot
    # index per problem and the fp64 V_1 / Quu_0 of up to one problem in eight)
    for flags in (0, RESCUE):
        w = L.ttc_lqr_workspace_bytes(1000, 8, d, d, 64, 1, flags)
        main = 4 * P * (2 * d * d + 1)
        if flags == RESCUE:
            main += 4 * P + 8 * (P // 8) * 2 * d * d
        assert main <= w <= main + (256 << 20) + (1 << 16)
    # the third tier needs d = du = 16 and head groups of 8
    t3 = 4 * P + 8 * (P // 8) * 2 * d * d
    assert (L.ttc_lqr_workspace_bytes(1000, 8, d, d, 64, 1, RESCUE) - L.ttc_lqr_workspace_bytes(1000, 8, d, d, 64, 1, 0)
            >= t3)
    assert (L.ttc_lqr_workspace_bytes(1000, 4, d, d, 64, 1, RESCUE) - L.ttc_lqr_workspace_bytes(1000, 4, d, d, 64, 1, 0)
            < t3 // 2)
    # stable-path-only workspace: the stable layout for the chunk
    ws = L.ttc_lqr_workspace_bytes(10, 8, d, d, 64, 0, STABLE | FP64)
    assert ws >= 8 * 80 * 64 * (d * d + 4 * d)
    assert L.ttc_lqr_supported_flags(16, 16, RESCUE) == 1 and L.ttc_lqr_supported_flags(64, 64, RESCUE) == 0


def test_noalloc_argument_validation(L):
    """ttc_lqr_backward_noalloc rejects what its fixed scratch cannot hold before touching a device."""
    assert L.ttc_lqr_noalloc_scratch_bytes() == 256 << 20
    p = ctypes.c_void_p(16)
    n_fb = ctypes.c_int64(-1)
    args = lambda n, d, T, flags: ([p] * 11 + [n, 16, d, d, T, flags, None] + [p] * 9  # noqa: E731
                                   + [float("inf"), None, ctypes.byref(n_fb), None])
    assert L.ttc_lqr_backward_noalloc(*args(0, 16, 64, 0)) == 0 and n_fb.value == 0   # empty batch
    assert L.ttc_lqr_backward_noalloc(*args(1, 24, 64, 0)) == 2                       # unsupported dims
    assert L.ttc_lqr_backward_noalloc(*args(-1, 16, 64, 0)) == 1                      # bad sizes
    # d = 64, T = 4096, 16 heads: one token's fallback layout alone exceeds 256 MiB
    assert L.ttc_lqr_workspace_bytes(1, 16, 64, 64, 4096, 0, 0) > 256 << 20
    assert L.ttc_lqr_backward_noalloc(*args(1, 64, 4096, 0)) == 4                     # TTC_LQR_ESCRATCH
    assert b"scratch" in L.ttc_lqr_strerror(4)
