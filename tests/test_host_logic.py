"""CPU tests of the host-side logic around the kernels (no GPU).

* zero-padding to the compiled sizes leaves the LQR solution and gradients
  unchanged (checked with the fp64 oracle on the padded vs unpadded problem);
* the TTCLayer mirror: constructor validation, solver registry, parameter
  shapes and init, front-end shapes for 3-D and 4-D inputs, T == 0.
"""
import numpy as np
import pytest
import torch

from oracle.inputs import bench_solver_inputs
from oracle.lqr64 import LQRProblem, solve_grads

NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]


def test_padded_dim():
    from ttc.solvers.hip_lqr import padded_dim
    assert padded_dim(16, 16) == 16
    assert padded_dim(12, 8) == 16
    assert padded_dim(17, 3) == 32
    assert padded_dim(33, 64) == 64
    with pytest.raises(AssertionError):
        padded_dim(65, 16)


def test_precision_flags():
    """"auto": fp64 for the certificate's rejected problems at every horizon where the fp64
    kernels exist (d <= 32) -- the long-horizon flag from T = 512 on, the fallback flag below --
    and fp32 at d = 64; the fallback flag reaches the backward only after a forward that
    rescued some problem (TTC_LQR_STATUS_RESCUED = 4)."""
    from ttc.solvers.hip_lqr import backward_flags, riccati_flags
    from ttc.solvers._lib import FLAG_FP64_FALLBACK, FLAG_FP64_RESCUE, FLAG_FP64_RICCATI, FLAG_RICCATI_STEPS
    assert riccati_flags("auto", 64, 16) == FLAG_FP64_FALLBACK
    assert riccati_flags("auto", 511, 32) == FLAG_FP64_FALLBACK
    assert riccati_flags("auto", 512, 16) == FLAG_FP64_RESCUE
    assert riccati_flags("auto", 64, 64) == 0 and riccati_flags("auto", 1024, 64) == 0
    assert riccati_flags("fp32", 64, 16) == 0 and riccati_flags("fp32", 1024, 16) == 0
    assert riccati_flags("riccati", 64, 16) == FLAG_RICCATI_STEPS
    assert riccati_flags("riccati", 1024, 16) == FLAG_FP64_RICCATI
    assert backward_flags(FLAG_FP64_FALLBACK, 0) == 0
    assert backward_flags(FLAG_FP64_FALLBACK, 4) == FLAG_FP64_FALLBACK
    assert backward_flags(FLAG_FP64_FALLBACK | 4, 1) == 4  # stable-backward bit kept
    assert backward_flags(FLAG_FP64_RESCUE, 0) == FLAG_FP64_RESCUE


@pytest.mark.parametrize("d,du", [(12, 8), (5, 9), (16, 10)])
def test_padding_preserves_solution_and_gradients(d, du):
    from ttc.solvers.hip_lqr import _pad_inputs, padded_dim
    g = torch.Generator().manual_seed(d * 31 + du)
    N, H, T = 3, 2, 7
    base = bench_solver_inputs(N, H, d, seed=d + du)
    B = torch.randn(N, d, du, generator=g) * 0.5
    R_inv = torch.nn.functional.softplus(torch.rand(N, H, du, generator=g))
    lgB = -torch.nn.functional.softplus(torch.randn(N, H, du, generator=g)) - 0.5
    ins = [base[0], B, base[2], R_inv, base[4], base[5], lgB, base[7], base[8]]
    Dp = padded_dim(d, du)
    pins = _pad_inputs([t.double() for t in ins], d, du, Dp)
    dU = np.random.RandomState(0).randn(N, H, du)
    dUp = np.zeros((N, H, Dp))
    dUp[..., :du] = dU
    ref = solve_grads(LQRProblem(*ins, T), dU)
    pad = solve_grads(LQRProblem(*pins, T), dUp)
    sl = {"u": (..., slice(0, du)), "A_diag": (..., slice(0, d)), "B": (slice(None), slice(0, d), slice(0, du)),
          "Q": (slice(None), slice(0, d), slice(0, d)), "R_inv": (..., slice(0, du)),
          "Q_f": (slice(None), slice(None), slice(0, d), slice(0, d)), "lgA": (...,),
          "lgB": (..., slice(0, du)), "lgQ": (..., slice(0, d)), "h0": (..., slice(0, d))}
    for k in ["u"] + NAMES:
        np.testing.assert_allclose(pad[k][sl[k]], ref[k], rtol=1e-10, atol=1e-12, err_msg=k)
    # padded controls are exactly zero
    assert np.abs(pad["u"][..., du:]).max() == 0.0


def test_layer_registry_and_validation():
    from ttc import TTCLayer
    from ttc.layers.ttc_layer import LQR_SOLVER_IMPL_MAP
    assert "hip" in LQR_SOLVER_IMPL_MAP and "fused" in LQR_SOLVER_IMPL_MAP
    with pytest.raises(AssertionError):
        TTCLayer(32, 32, 16, 8, 16, 16, solver_impl="nope")
    with pytest.raises(AssertionError):
        TTCLayer(32, 32, 16, 8, 16, 16, rescale="bad")
    with pytest.raises(AssertionError):
        TTCLayer(32, 32, 16, 8, 16, 16, q_reparam="bad")


def test_layer_parameters_and_init():
    from ttc import TTCLayer
    torch.manual_seed(0)
    m = TTCLayer(32, 24, 16, 8, 12, 10, gamma_bias=True)
    head = 16 + 16 + 16 + 10 + (1 + 16 + 16)
    assert m.in_proj.weight.shape == (head * 8 + 12 + 10, 32)
    assert m.out_proj.weight.shape == (24, 16 * 8)
    assert m.Bs.shape == (12, 16, 16) and m.Qs.shape == (10, 16, 16)
    # plain reparam starts PSD and symmetric (ttc_layer.py:79-83)
    Qs = m.Qs.detach()
    torch.testing.assert_close(Qs, Qs.transpose(1, 2))
    assert torch.linalg.eigvalsh(Qs.double()).min() > -1e-10
    torch.testing.assert_close(m.bias_gamma.detach(), torch.full((33,), float(np.log(1 / 4.0))))


def test_layer_front_end_shapes_3d_and_4d():
    from ttc import TTCLayer
    m = TTCLayer(32, 32, 16, 8, 16, 16)
    for shape in [(2, 5, 32), (2, 3, 8, 32)]:
        x = torch.randn(shape)
        ins = m.solver_inputs(x)
        N = int(np.prod(shape[:-1]))
        exp = [(N, 8, 16), (N, 16, 16), (N, 16, 16), (N, 8, 16), (N, 8, 16, 16), (N, 8), (N, 8, 16), (N, 8, 16),
               (N, 8, 16)]
        assert [tuple(t.shape) for t in ins] == exp
        R = ins[3]
        assert (R >= 1e-6).all() and (R <= 1 + 1e-6).all()
        assert (ins[5] < 0).all() and (ins[6] < 0).all() and (ins[7] < 0).all()


def test_layer_T0_returns_zeros():
    from ttc import TTCLayer
    m = TTCLayer(32, 20, 16, 8, 16, 16)
    y = m(torch.randn(2, 3, 32), T=0)
    assert y.shape == (2, 3, 20) and not y.any()


def test_bench_traffic_records_and_single_gpu_contract():
    """bench.py's roofline.traffic comes from the committed rocprofv3 summaries: each forward
    record parses and lies between the algorithmic bytes of its sample and twice them; and a
    multi-GPU request exits with status 2 and a message instead of a figure."""
    import json
    import subprocess
    import sys
    import bench
    algorithmic = {"lqr_fwd_cfg2": 1668 * 2_097_152}  # bytes per problem x problems of the workload
    for tag, alg in algorithmic.items():
        t = bench.traffic_from_profiles(tag)
        assert t is not None, tag
        assert alg <= t <= 2 * alg, (tag, t, alg)
    assert bench.traffic_from_profiles("no_such_kernel") is None
    res = subprocess.run([sys.executable, bench.__file__, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in json.loads(res.stdout.strip().splitlines()[-1])["error"]


def test_bench_cpu_leg_child(tmp_path):
    """bench.py's CPU-baseline leg as the benchmark runs it: a child process that never touches the
    GPU (no HIP library is loaded in it) times the reference restatement on a CPU sample, measures
    the reference's fp32 solvers against the fp64 oracle, writes the sample and the oracle outputs
    for the GPU process, prints one JSON line and exits 0."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = tmp_path / "leg.npz"
    code = ("import runpy, sys; sys.argv = ['bench.py', '--cpu-leg', %r, '--config', '2', '--cpu-sample-tokens', "
            "'2', '--horizon', '6']; runpy.run_path(%r, run_name='__main__'); "
            "assert not [m for m in sys.modules if m == 'ttc' or m.startswith('ttc.')], 'HIP library loaded'"
            % (str(out), os.path.join(root, "bench.py")))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, cwd=root)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads([line for line in r.stdout.splitlines() if line.startswith("{")][-1])
    assert res["kind"] == "port" and res["value"] > 0 and res["fwd_value"] > 0
    assert res["accuracy"]["reference_riccati_fp32"]["max"] < 1e-4
    z = np.load(out)
    assert int(z["T"]) == 6 and z["in_A_diag"].shape == (2, 8, 16) and z["ref_u"].shape == (2, 8, 16)
