#!/usr/bin/env python
"""Benchmark of the TTC-Net LQR solver hot path on one MI355X.

Workload: TTCLayer(in=32, out=32, h=16, heads=8, b_rank=16,
q_rank=16), T=64, x [16, 2048, 8, 32] ~ N(0,1) (seeded, synthetic), random-init
weights (seed 0).  The layer front-end turns x into the nine solver inputs
(N = 262144 tokens, P = N*8 = 2097152 LQR problems), which stay resident in HBM.
A timed *step* is one solver forward + backward over all P problems with the
upstream gradient d_u that dy ~ N(0,1) induces through the layer back-end.

Prints one JSON line: value = forward+backward LQR solves/s; the forward-only
rate, tokens/s, the fp32 roofline of the forward kernel (algorithmic flops per
problem F_fwd = T(4 d^2 du + 2 d^3), timed with HIP events on the launch stream)
and a CPU baseline (an op-for-op restatement of the reference `riccati` solver,
fwd and autograd fwd+bwd, on a bounded token sample, all host cores, with the reference's
fp32 solvers' and this solver's errors against the fp64 oracle on that sample) ride along,
as do configs 3 and 4 on 8,192-token samples (`extra_configs`, config 4 also with bf16
storage) and configs 3 and 4 at full size, one step each (`full_size`).
`--sweep horizon|batch` runs the reference bench's sweeps instead (one line per point).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ttc-net_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "LQR solves/sec fwd & fwd+bwd (h=16,T=64) + % HBM/MFMA roofline, 1×MI355X"


def metric_for(d, T):
    """BASELINE.json's metric for the headline config (h=16, T=64); the same measure of other
    configurations names their own h and T."""
    return METRIC.replace("(h=16,T=64)", f"(h={d},T={T})")


PEAK_FP32_MFMA = 157.3e12   # MI355X dense fp32 matrix peak (published)
PEAK_FP64 = 78.6e12         # MI355X fp64 peak (published; vector and matrix)
PEAK_HBM = 8.0e12

CONFIGS = {
    "2": dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=64, x_shape=(16, 2048, 8, 32)),
    "3": dict(in_dim=64, out_dim=64, h_dim=64, num_heads=16, b_rank=32, q_rank=32, T=128, x_shape=(8, 4096, 16, 64)),
    # x stored bf16, N(0,1) * 0.02 (post-norm activations); the solver computes in fp32
    "4": dict(in_dim=64, out_dim=64, h_dim=32, num_heads=32, b_rank=32, q_rank=32, T=256, x_shape=(4, 8192, 32, 64),
              x_scale=0.02, x_bf16=True),
    # numerical stress, long horizon: every token scaled by exp(N(0, 1.5)); decode-like x and a
    # 4 x 1024 batch
    # (its gradients legitimately exceed the reference's 1e6 guard: no limit)
    "5": dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=1024, x_shape=(256, 1, 8, 32),
              x_lognormal=1.5, grad_limit=float("inf")),
    "5b": dict(in_dim=32, out_dim=32, h_dim=16, num_heads=8, b_rank=16, q_rank=16, T=1024,
               x_shape=(4, 1024, 8, 32), x_lognormal=1.5, grad_limit=float("inf")),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="2", choices=list(CONFIGS))
    ap.add_argument("--tokens", type=int, default=0, help="override token count (0 = the config's full x)")
    ap.add_argument("--stash", default=None, choices=["auto", "always", "never"])
    ap.add_argument("--cpu-sample-tokens", type=int, default=0,
                    help="tokens of the CPU baseline sample (0: 64 below T = 512, 1 from there; the reference "
                         "restatement's autograd through 1,024 steps takes seconds per token)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-leg", default=None, metavar="NPZ", help=argparse.SUPPRESS)
    ap.add_argument("--precision", default="auto",
                    choices=["auto", "riccati", "fp32", "fp32-riccati", "fp32-row", "fp64"],
                    help="the solver's precision / kernel choice (hip_lqr_solve's `precision`): 'riccati' times what "
                         "TTCLayer(solver_impl='riccati') runs on CUDA tensors, with --stable-backward what 'kkt' runs")
    ap.add_argument("--stable-backward", action="store_true",
                    help="the stable backward for every problem (the 'kkt' key's backward)")
    ap.add_argument("--status-check", default="sync", choices=["sync", "deferred"],
                    help="hip_lqr_solve's status_check: 'deferred' takes the host synchronisation out of the "
                         "forward (its status word is read by the backward)")
    ap.add_argument("--fwd-only", action="store_true",
                    help="profiling aid: time only the forward solve (the JSON value is then fwd solves/s)")
    ap.add_argument("--extra-configs", default="3,4,5,5b",
                    help="comma list of further configs measured after the main one (forward and fwd+bwd, "
                         "reported under 'extra_configs'): 3 and 4 on a token sample, 5 and 5b at full size; "
                         "'' for none")
    ap.add_argument("--extra-tokens", type=int, default=8192, help="token sample of the extra configs")
    ap.add_argument("--no-factored-extra", action="store_true",
                    help="skip the factored-input measurement of the main config (profiling aid)")
    ap.add_argument("--no-full-size", action="store_true",
                    help="skip the full-size configs 3 and 4 (one step each, ~1 minute) of the default line")
    ap.add_argument("--factored", action="store_true",
                    help="measure the solver on the layer's low-rank factors (coeff_B, coeff_Q, coeff_Qf + bases, "
                         "expanded per token chunk on the device) instead of materialised B, Q, Q_f: the only "
                         "form in which configs 3 and 4 fit one GPU at full size")
    ap.add_argument("--sweep", default=None, choices=["horizon", "batch"],
                    help="the reference bench's sweeps (bench_lqr_solvers.py:259-425) on its solver-level "
                         "distribution (batch 1024, 1 head, d 64, T 64): one JSON line per point with fwd+bwd "
                         "time, solves/s, FLOP/s and peak memory; skips the main measurement")
    ap.add_argument("--sweep-dim", type=int, default=64)
    ap.add_argument("--horizon", type=int, default=0,
                    help="profiling aid: override the config's horizon T (0 = the config's own); kernel time "
                         "against T separates the per-step cost from the per-problem work outside the sweep")
    ap.add_argument("--progress", action="store_true", help="print a line to stderr after every solver call")
    ap.add_argument("--copy-calibration", type=float, default=0.0, metavar="GIB",
                    help="profiling aid: run one plain device copy of this many GiB and exit "
                         "(scales rocprofv3 FETCH_SIZE/WRITE_SIZE to bytes)")
    return ap.parse_args()


def traffic_from_profiles(kernel_tag: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE),
    as recorded in profiles/<kernel_tag>_pmc.md ("traffic_bytes_per_launch: N")."""
    path = os.path.join(ROOT, "profiles", f"{kernel_tag}_pmc.md")
    try:
        with open(path) as f:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read())
        return float(m.group(1)) if m else None
    except OSError:
        return None


def _relerr(x, ref):
    import numpy as np
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    e = float(np.abs(x - ref).max() / max(float(np.abs(ref).max()), 1e-30)) if ref.size else 0.0
    return e if math.isfinite(e) else None  # None: non-finite (NaN / inf) output


NAMES = ["A_diag", "B", "Q", "R_inv", "Q_f", "lgA", "lgB", "lgQ", "h0"]


def _cpu_model() -> str:
    """The host CPU's model name (the `lscpu` "Model name" line), from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _oracle_cfg(cfg: str):
    return int(cfg) if cfg.isdigit() else cfg


def _sample_tokens(args, T: int) -> int:
    return args.cpu_sample_tokens if args.cpu_sample_tokens > 0 else (64 if T < 512 else 1)


def _per_output_errors(out, ref):
    return {k: _relerr(out[k], ref[k]) for k in ["u"] + NAMES}


def _max_or_none(per):
    vals = [v for k, v in per.items() if k != "error"]
    return None if (not vals or any(v is None for v in vals)) else max(vals)


def cpu_leg(args):
    """`--cpu-leg NPZ`: the CPU half of the baseline, in a process of its own that bench.py starts
    before it touches the GPU; this process never does (no HIP library, no torch.cuda).

    On a seeded sample of the configuration's workload (oracle/inputs.py: the layer front-end on
    synthetic x, the same distribution as the GPU run): times the op-for-op restatement of the
    reference `riccati` solver (oracle/ref_torch.py; forward, and forward + autograd backward) on
    all host cores, and measures the reference's fp32 `riccati` and `kkt` solvers against the fp64
    oracle (oracle/lqr64.py) on the same sample and upstream gradient.  Writes the sample, the
    gradient and the oracle's outputs to NPZ (the benchmark process measures the HIP solver on
    them) and prints one JSON line."""
    import numpy as np
    import torch
    from oracle.inputs import layer_solver_inputs, make_x
    from oracle.lqr64 import LQRProblem, solve_grads
    from oracle.ref_torch import kkt_solve, riccati_solve
    c = CONFIGS[args.config]
    T = args.horizon if args.horizon > 0 else c["T"]
    n = _sample_tokens(args, T)
    ocfg = _oracle_cfg(args.config)
    ins = layer_solver_inputs(ocfg, make_x(ocfg, n_tokens=n, seed=0))
    H = ins[0].shape[1]
    P = n * H
    d_u = torch.randn(n, H, ins[1].shape[-1], generator=torch.Generator().manual_seed(1))
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)

    def fwd():
        with torch.no_grad():
            riccati_solve(*ins, T)

    def fwdbwd():
        xs = [t.clone().requires_grad_(True) for t in ins]
        u = riccati_solve(*xs, T)
        torch.autograd.grad(u, xs, torch.ones_like(u))

    reps_fb = 5 if T < 512 else 3
    rate = {}
    for name, fn, reps in (("fwd", fwd, 5), ("fwd_bwd", fwdbwd, reps_fb)):
        fn()
        _note(f"cpu baseline {name}: warm-up done")
        ts = []
        for i in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
            _note(f"cpu baseline {name}: rep {i + 1}/{reps} {ts[-1]:.1f} s")
        rate[name] = P / statistics.median(ts)
    ref = solve_grads(LQRProblem(*ins, T), d_u.double().numpy())
    _note("cpu baseline: fp64 oracle done")
    acc = {}
    for name, fn in (("reference_riccati_fp32", riccati_solve), ("reference_kkt_fp32", kkt_solve)):
        try:
            xs = [t.detach().clone().requires_grad_(True) for t in ins]
            with np.errstate(all="ignore"):
                u = fn(*xs, T)
                gs = torch.autograd.grad(u, xs, d_u, allow_unused=True)
                out = {"u": u.detach().double().numpy()}
                for k, g in zip(NAMES, gs):
                    g = g.detach().double().numpy()
                    out[k] = 0.5 * (g + np.swapaxes(g, -1, -2)) if k in ("Q", "Q_f") else g
            per = _per_output_errors(out, ref)
        except RuntimeError as e:  # e.g. a singular solve in fp32
            per = {"error": str(e)}
        acc[name] = {"max": _max_or_none(per), "per_output": per}
        _note(f"cpu baseline: {name} accuracy done")
    np.savez(args.cpu_leg, T=T, dU=d_u.numpy(), **{f"in_{k}": t.numpy() for k, t in zip(NAMES, ins)},
             **{f"ref_{k}": ref[k] for k in ["u"] + NAMES})
    print(json.dumps({
        "value": rate["fwd_bwd"], "unit": "solves/s", "cores": torch.get_num_threads(), "kind": "port",
        "fwd_value": rate["fwd"],
        "sample": f"{n} tokens x {H} heads = {P} problems of the same workload (oracle/inputs.py, seed 0), T={T}; "
                  f"oracle/ref_torch.riccati_solve (reference direct_lqr_solve restated), fwd median of 5, "
                  f"fwd+bwd (autograd) median of {reps_fb}, each after 1 warm-up, torch threads="
                  f"{torch.get_num_threads()}, os.cpu_count()={cores}, cpu: {_cpu_model()}; run in a process of "
                  f"its own that never touches the GPU, before the GPU measurement",
        "accuracy": acc}), flush=True)


def run_cpu_leg(args):
    """Run `cpu_leg` in a child process (before this process initialises the GPU) and wait for it:
    returns (its JSON result or None, the NPZ path, its exit status)."""
    import subprocess
    import tempfile
    fd, path = tempfile.mkstemp(prefix="ttc_cpu_leg_", suffix=".npz")
    os.close(fd)
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-leg", path, "--config", args.config,
           "--cpu-sample-tokens", str(args.cpu_sample_tokens), "--horizon", str(args.horizon)]
    if PROGRESS:
        cmd.append("--progress")
    _note(f"cpu baseline: child process {' '.join(cmd[1:])}")
    try:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900)
        rc, text = r.returncode, r.stdout
    except subprocess.TimeoutExpired as e:
        rc, text = "timeout", e.stdout or ""
        text = text.decode() if isinstance(text, bytes) else text
    lines = [line for line in text.splitlines() if line.startswith("{")]
    res = json.loads(lines[-1]) if lines else None
    return res, path, rc


def hip_accuracy(path, grad_limit, solver_kw):
    """This solver on the CPU leg's sample (NPZ) against the fp64 oracle outputs saved with it."""
    import numpy as np
    import torch
    from ttc.solvers.hip_lqr import hip_lqr_solve
    z = np.load(path)
    T = int(z["T"])
    xs = [torch.from_numpy(z[f"in_{k}"]).cuda().float().requires_grad_(True) for k in NAMES]
    try:
        u = hip_lqr_solve(*xs, T, grad_limit=grad_limit, **solver_kw)
        gs = torch.autograd.grad(u, xs, torch.from_numpy(z["dU"]).cuda().to(u.dtype))
        out = {"u": u.detach().cpu().double().numpy()}
        out.update({k: g.detach().cpu().double().numpy() for k, g in zip(NAMES, gs)})
        per = _per_output_errors(out, {k: z[f"ref_{k}"] for k in ["u"] + NAMES})
    except RuntimeError as e:  # a guard of the solver
        per = {"error": str(e)}
    return {"max": _max_or_none(per), "per_output": per}


def _solver_for(ins):
    from ttc.solvers.hip_lqr import hip_lqr_solve, hip_lqr_solve_factored
    return hip_lqr_solve_factored if len(ins) == 11 else hip_lqr_solve


def layer_workload(cfg, tokens, dev, factored=False, normal_du=False):
    """Solver inputs of a config (seeded layer front-end on synthetic x: the nine materialised
    inputs, or with `factored` the eleven low-rank ones) and the d_u that dy ~ N(0,1) induces
    through the layer back-end (l2norm rescale + out_proj); with `normal_du`, d_u ~ N(0,1)
    directly (no extra solver forward: the full-size entries)."""
    import torch
    from ttc import TTCLayer
    from ttc.layers.ttc_layer import l2norm
    c = CONFIGS[cfg]
    torch.manual_seed(0)
    layer = TTCLayer(c["in_dim"], c["out_dim"], c["h_dim"], c["num_heads"], c["b_rank"], c["q_rank"],
                     solver_impl="hip").to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    xshape = c["x_shape"] if tokens == 0 else (tokens, c["in_dim"])
    x = torch.randn(xshape, generator=g, device=dev) * c.get("x_scale", 1.0)
    if c.get("x_lognormal"):
        x = x * torch.exp(c["x_lognormal"] * torch.randn(xshape[:-1], generator=g, device=dev))[..., None]
    if c.get("x_bf16"):
        x = x.to(torch.bfloat16).float()
    T = c["T"]
    with torch.no_grad():
        front = layer.factored_inputs(x) if factored else layer.solver_inputs(x)
        ins = [t.detach().float().contiguous() for t in front]
        del front
        if normal_du:
            d_u = torch.randn(ins[0].shape[0], c["num_heads"], c["h_dim"], generator=g, device=dev)
            _note(f"workload cfg{cfg}: {ins[0].shape[0]} tokens, factored={factored}, d_u ~ N(0,1)")
            return ins, d_u, list(xshape)
        u0 = _solver_for(ins)(*ins, T)
    _note(f"workload cfg{cfg}: {ins[0].shape[0]} tokens, factored={factored}")
    u_req = u0.clone().requires_grad_(True)
    y = layer.out_proj(l2norm(u_req).reshape(*x.shape[:-1], -1))
    dy = torch.randn(y.shape, generator=g, device=dev)
    (d_u,) = torch.autograd.grad(y, u_req, dy)
    return ins, d_u.contiguous(), list(xshape)


PROGRESS = False


def _note(msg):
    if PROGRESS:
        print(f"[bench] {msg}", file=sys.stderr, flush=True)


def einsum_step_ms(ins_f, d_u, T, steps, warmup, grad_limit=1e6):
    """fwd+bwd wall time of the layer's other route from the same eleven factored inputs: B, Q and
    Q_f materialised by torch einsums (as the reference layer does, `ttc_layer.py:117-123`) and
    solved on them, gradients through the einsums by autograd."""
    import torch
    from ttc.solvers.hip_lqr import hip_lqr_solve
    xs = [t.clone().requires_grad_(True) for t in ins_f]

    def step():
        A, cB, cQ, R, cQf, lA, lB, lQ, h0, Bb, Qb = xs
        B = torch.einsum("nr,rij->nij", cB, Bb)
        Q = torch.einsum("nr,rij->nij", cQ, Qb)
        Qf = torch.einsum("nhr,rij->nhij", cQf, Qb)
        u = hip_lqr_solve(A, B, Q, R, Qf, lA, lB, lQ, h0, T, grad_limit=grad_limit)
        return torch.autograd.grad(u, xs, d_u)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def time_solver(ins, d_u, T, steps, warmup, stash=None, fwd_only=False, grad_limit=1e6, solver_kw=None):
    """Forward: mean per-call GPU time from HIP events on the launch stream.  fwd+bwd: wall
    time of `steps` steps between two device synchronisations, and the peak device memory the
    steps allocate beyond what is allocated before them (the reference bench's measure,
    `bench_lqr_solvers.py:48-68`: max_memory_allocated - memory_allocated around fwd+bwd)."""
    import torch
    solve = _solver_for(ins)
    kw = dict(solver_kw or {})
    hip_lqr_solve = (lambda *a, **k: solve(*a, **kw, **k)) if kw else solve
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        with torch.no_grad():
            hip_lqr_solve(*ins, T)
        _note(f"warm-up forward {i + 1}/{warmup}")
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        with torch.no_grad():
            hip_lqr_solve(*ins, T)
        e1.record(stream)
        _note("timed forward")
    torch.cuda.synchronize()
    res = {"fwd_wall_ms": (time.perf_counter() - t0) / steps * 1e3,
           "fwd_ms": statistics.mean(e0.elapsed_time(e1) for e0, e1 in evs)}
    if fwd_only:
        return res
    xs = [t.clone().requires_grad_(True) for t in ins]

    def step():
        u = hip_lqr_solve(*xs, T, stash=stash, grad_limit=grad_limit)
        return torch.autograd.grad(u, xs, d_u)

    for i in range(warmup):
        step()
        _note(f"warm-up fwd+bwd {i + 1}/{warmup}")
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
        _note(f"timed fwd+bwd {i + 1}/{steps}")
    torch.cuda.synchronize()
    res["step_ms"] = (time.perf_counter() - t0) / steps * 1e3
    res["peak_mem_bytes"] = max(0, torch.cuda.max_memory_allocated() - base)
    from ttc.solvers.hip_lqr import check_deferred_status
    check_deferred_status()  # forwards timed with a deferred status check (outside the timed regions)
    from ttc.solvers.hip_lqr import last_backward_stats
    res["bwd_fallback_problems"] = last_backward_stats["fallback"]
    return res


def flops_fwd(d, T):
    return T * (4 * d * d * d + 2 * d ** 3)


def flops_bwd(d, T):
    return T * (7 * d * d + 11 * d * d)


def sweep(args):
    """Horizon / batch sweeps of the reference bench (bench_lqr_solvers.py:259-425): its
    solver-level distribution, fwd+bwd median of 5, peak memory above the inputs.  The
    reference labels 4 * batch * d^3 * T / t as "GB/s"; it is reported here as
    `ref_metric` next to solves/s and the algorithmic FLOP/s."""
    import torch
    from oracle.inputs import bench_solver_inputs
    from ttc.solvers.hip_lqr import check_deferred_status, hip_lqr_solve
    dev = torch.device("cuda:0")
    d = args.sweep_dim
    points = [(2 ** i, 1024) for i in range(4, 12)] if args.sweep == "horizon" else [(64, 2 ** i) for i in range(4, 14)]
    for T, batch in points:
        ins = [t.to(dev) for t in bench_solver_inputs(batch, 1, d, seed=0)]
        xs = [t.clone().requires_grad_(True) for t in ins]
        gr = torch.randn(batch, 1, d, device=dev, generator=torch.Generator(device=dev).manual_seed(1))

        def step():
            u = hip_lqr_solve(*xs, T, status_check=args.status_check)
            return torch.autograd.grad(u, xs, gr)

        def fwd():
            with torch.no_grad():
                hip_lqr_solve(*ins, T, status_check=args.status_check)

        step()
        fwd()
        torch.cuda.synchronize()
        tf = []
        for _ in range(5):  # one forward, waited for: its latency
            t0 = time.perf_counter()
            fwd()
            torch.cuda.synchronize()
            tf.append(time.perf_counter() - t0)
        t0 = time.perf_counter()
        for _ in range(5):  # five forwards back to back: with a deferred status they queue up
            fwd()
        torch.cuda.synchronize()
        tf_pipe = (time.perf_counter() - t0) / 5
        ts, peaks = [], []
        for _ in range(5):
            torch.cuda.reset_peak_memory_stats()
            before = torch.cuda.memory_allocated()
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
            peaks.append(torch.cuda.max_memory_allocated() - before)
        t = statistics.median(ts)
        check_deferred_status()  # the deferred forwards' status words (outside the timed regions)
        print(json.dumps({"sweep": args.sweep, "T": T, "batch": batch, "heads": 1, "d": d,
                          "status_check": args.status_check, "fwd_ms": statistics.median(tf) * 1e3,
                          "fwd_back_to_back_ms": tf_pipe * 1e3,
                          "fwd_bwd_ms": t * 1e3, "solves_per_s": batch / t,
                          "tflops": batch * (flops_fwd(d, T) + flops_bwd(d, T)) / t / 1e12,
                          "ref_metric": 4 * batch * d ** 3 * T * 1e-9 / t,
                          "peak_mem_gb": statistics.median(peaks) / 1e9}), flush=True)


def main():
    global PROGRESS
    args = parse()
    PROGRESS = args.progress
    if args.cpu_leg:
        cpu_leg(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the LQR problems shard over tokens with no "
                                   "exchange (each rank would run these kernels on its N/G tokens), so a "
                                   "multi-GPU figure is not produced here",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    # the CPU baseline first, in a child process that never touches the GPU, started before this
    # process initialises it (and finished before the GPU is timed, so the two do not share the host)
    leg = None
    if not (args.no_cpu_baseline or args.copy_calibration > 0 or args.sweep or args.fwd_only):
        leg = run_cpu_leg(args)
    import torch
    if args.copy_calibration > 0:
        n = int(args.copy_calibration * (1 << 30)) // 4
        a = torch.ones(n, device="cuda:0")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 4 * n}))
        return
    if args.sweep:
        sweep(args)
        return
    if args.horizon > 0:
        CONFIGS[args.config] = dict(CONFIGS[args.config], T=args.horizon)

    c = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    T, H, d = c["T"], c["num_heads"], c["h_dim"]
    ins, d_u, xshape = layer_workload(args.config, args.tokens, dev, factored=args.factored)
    N = ins[0].shape[0]
    P = N * H
    solver_kw = {}
    if args.precision != "auto":
        solver_kw["precision"] = args.precision
    if args.stable_backward:
        solver_kw["stable_backward"] = True
    if args.status_check != "sync":
        solver_kw["status_check"] = args.status_check
    r = time_solver(ins, d_u, T, args.steps, args.warmup, stash=args.stash, fwd_only=args.fwd_only,
                    grad_limit=c.get("grad_limit", 1e6), solver_kw=solver_kw)
    fwd_gpu_ms = r["fwd_ms"]
    if args.fwd_only:
        print(json.dumps({"mode": "fwd-only", "fwd_ms": fwd_gpu_ms, "fwd_solves_per_s": P / (fwd_gpu_ms * 1e-3),
                          "problems": P}), flush=True)
        return
    step_s = r["step_ms"] * 1e-3

    F_fwd = flops_fwd(d, T)
    achieved = F_fwd * P / (fwd_gpu_ms * 1e-3)
    fwd_bytes = 4 * (3 * d + 2 * d + d * d + 1 + d) + 4 * (d * d + d * d) / H
    traffic = traffic_from_profiles(f"lqr_fwd_cfg{args.config}")
    kern = f"lqr_fwd_blk_kernel<{d}>" + (" (symplectic sweep)" if d in (16, 32, 64) else "")
    # precision="auto" at T >= 512 (d <= 32): the same fp32 matrix-core sweep, the problems its
    # certificate rejects (a few per cent) recomputed in fp64 (d = 16 on the matrix cores, d = 32
    # by the row-layout sweep); priced against the fp32 matrix peak as a whole
    long_h = T >= 512 and d <= 32
    if long_h:
        kern += (" + fp64 matrix-core rescue of the rejected problems (lqr_fwd64_mfma_kernel)" if d == 16 else
                 " + fp64 row-layout rescue of the rejected problems (lqr_rescue_listed_kernel<double>)")
    out = {
        "metric": metric_for(d, T),
        "value": P / step_s,
        "unit": "solves/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+f64" if long_h else "f32",
        "data": "synthetic (seeded N(0,1) x, random-init layer weights)",
        "config": {"workload": f"cfg{args.config}: TTCLayer(in={c['in_dim']},out={c['out_dim']},h={d},heads={H},"
                               f"b_rank={c['b_rank']},q_rank={c['q_rank']}) T={T}, x{xshape} -> "
                               f"{N} tokens, {P} LQR problems, solver fwd+bwd"
                               + (" on the layer's low-rank factors (B, Q, Q_f expanded on the device)"
                                  if args.factored else ""),
                   "tokens": N, "heads": H, "d": d, "du": d, "T": T, "problems": P},
        "fwd_solves_per_s": P / (fwd_gpu_ms * 1e-3),
        "fwd_ms": fwd_gpu_ms,
        "fwd_wall_ms": r["fwd_wall_ms"],
        "bwd_fallback_problems": r["bwd_fallback_problems"],
        "peak_mem_bytes_fwd_bwd": r["peak_mem_bytes"],
        "solver": {"precision": args.precision, "stable_backward": args.stable_backward,
                   "status_check": args.status_check},
        "tokens_per_s_fwd_bwd": N / step_s,
        "tokens_per_s_fwd": N / (fwd_gpu_ms * 1e-3),
        "fwd_bwd_tflops": (F_fwd + flops_bwd(d, T)) * P / step_s / 1e12,
        "roofline": {"bound": "mfma+fp64" if long_h else "mfma", "achieved": achieved / 1e12,
                     "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_MFMA,
                     "traffic": traffic, "kernel": kern, "flops_per_problem": F_fwd,
                     "algorithmic_bytes_per_problem": fwd_bytes},
    }
    if long_h:
        out["roofline"]["peak_note"] = ("fp32 matrix peak of the symplectic sweep; the rescue's fp64 sweeps run on "
                                        + ("the matrix cores" if d == 16 else "the vector ALU")
                                        + " (78.6 TFLOP/s fp64)")
        out["roofline"]["frac_of_fp64_peak"] = achieved / PEAK_FP64
    extras = []
    for cfg in [x.strip() for x in args.extra_configs.split(",") if x.strip()]:
        if cfg == args.config:
            continue
        # configs 5 / 5b (decode-size and 4 x 1024 batches) at their full BASELINE size
        extras.append(extra_entry(cfg, 0 if cfg in ("5", "5b") else args.extra_tokens, dev))
    if args.config == "2" and "4" in args.extra_configs:
        # config 4 as stored (bf16): the factored bf16 entry points on the same token sample
        extras.append(extra_entry("4", args.extra_tokens, dev, bf16=True))
    out["extra_configs"] = extras
    if not args.factored and not args.no_factored_extra:
        # the layer's default path: the same solve on the low-rank factors, B / Q / Q_f expanded per
        # token chunk on the device (no [N,H,d,d] Q_f in HBM)
        ins_f, du_f, _ = layer_workload(args.config, args.tokens, dev, factored=True)
        rf = time_solver(ins_f, du_f, T, 3, 1, stash=args.stash, grad_limit=c.get("grad_limit", 1e6))
        out["factored"] = {"fwd_ms": rf["fwd_ms"], "fwd_bwd_ms": rf["step_ms"],
                           "fwd_bwd_solves_per_s": P / (rf["step_ms"] * 1e-3),
                           "peak_mem_bytes_fwd_bwd": rf["peak_mem_bytes"],
                           "input_bytes_per_problem": 4 * (5 * d + 1 + (c["b_rank"] + c["q_rank"]) / H + c["q_rank"]),
                           # the same step with B / Q / Q_f materialised by torch einsums instead
                           "torch_einsum_materialised_fwd_bwd_ms": einsum_step_ms(
                               ins_f, du_f, T, 3, 1, grad_limit=c.get("grad_limit", 1e6))}
        del ins_f, du_f
        torch.cuda.empty_cache()
    if args.config == "2" and not args.no_full_size:
        # BASELINE configs 3 and 4 at full size under this run's clock: one forward and one
        # forward+backward step each, on the factored inputs (the materialised Q_f alone would be
        # 137 GB); d_u ~ N(0,1)
        out["full_size"] = [full_size_entry(cfg, dev) for cfg in ("3", "4")]
    out["cpu_baseline"] = None
    if leg is not None:
        res, path, rc = leg
        if res is not None:
            acc = res.pop("accuracy")
            acc["hip"] = hip_accuracy(path, c.get("grad_limit", 1e6), solver_kw)
            res["ref_rel_err"] = acc["reference_riccati_fp32"]["max"]
            res["ref_kkt_rel_err"] = acc["reference_kkt_fp32"]["max"]
            res["hip_rel_err"] = acc["hip"]["max"]
            res["accuracy"] = {"vs": "fp64 oracle (oracle/lqr64.py) on the CPU sample, same upstream gradient "
                                     "(N(0,1)); per tensor max|x-x64|/max|x64| over u and the nine gradients "
                                     "(None: non-finite output)", **acc}
        out["cpu_baseline"] = res
        if rc != 0:
            out["cpu_baseline_exit_status"] = rc
        try:
            os.unlink(path)
        except OSError:
            pass
    print(json.dumps(out), flush=True)


def extra_entry(cfg, tokens, dev, bf16=False):
    """A further configuration on a token sample: forward (HIP events) and fwd+bwd, roofline
    fraction of the forward, measured HBM traffic where profiled.  bf16: the factored inputs
    stored as bf16 (config 4's storage), through the _bf16 entry points."""
    import torch
    ce = CONFIGS[cfg]
    Te, He, de = ce["T"], ce["num_heads"], ce["h_dim"]
    ins_e, du_e, xs_e = layer_workload(cfg, tokens, dev, factored=bf16)
    if bf16:
        ins_e = [t.to(torch.bfloat16) for t in ins_e]
        du_e = du_e.to(torch.bfloat16)
    Pe = ins_e[0].shape[0] * He
    re_ = time_solver(ins_e, du_e, Te, 3, 1, grad_limit=ce.get("grad_limit", 1e6))
    ach = flops_fwd(de, Te) * Pe / (re_["fwd_ms"] * 1e-3)
    ach_fb = (flops_fwd(de, Te) + flops_bwd(de, Te)) * Pe / (re_["step_ms"] * 1e-3)
    e = {"config": f"cfg{cfg}" + ("-bf16" if bf16 else ""), "x": xs_e, "d": de, "T": Te, "heads": He,
         "problems": Pe, "storage": "bf16 (factored inputs, d_u and gradients)" if bf16 else "fp32",
         "fwd_ms": re_["fwd_ms"], "fwd_solves_per_s": Pe / (re_["fwd_ms"] * 1e-3),
         "fwd_bwd_ms": re_["step_ms"], "fwd_bwd_solves_per_s": Pe / (re_["step_ms"] * 1e-3),
         "tokens_per_s_fwd_bwd": ins_e[0].shape[0] / (re_["step_ms"] * 1e-3),
         "bwd_fallback_problems": re_["bwd_fallback_problems"],
         "peak_mem_bytes_fwd_bwd": re_["peak_mem_bytes"],
         "roofline_frac": ach / PEAK_FP32_MFMA, "achieved_tflops": ach / 1e12,
         "fwd_bwd_tflops": ach_fb / 1e12, "fwd_bwd_frac": ach_fb / PEAK_FP32_MFMA,
         "traffic": None if bf16 else traffic_from_profiles(f"lqr_fwd_cfg{cfg}")}
    if Te >= 512 and de <= 32:
        # precision "auto": the fp32 symplectic sweep, its rejected problems and the backward in fp64
        e["dtype"] = "f32+f64"
        e["roofline_frac_of_fp64_peak"] = ach / PEAK_FP64
        e["fwd_bwd_frac_of_fp64_peak"] = ach_fb / PEAK_FP64
    del ins_e, du_e
    torch.cuda.empty_cache()
    return e


def full_size_entry(cfg, dev):
    """One config at its full BASELINE size on the factored inputs: one timed forward (HIP events)
    and one timed forward+backward step, no warm-up."""
    import torch
    ce = CONFIGS[cfg]
    Te, He, de = ce["T"], ce["num_heads"], ce["h_dim"]
    t0 = time.perf_counter()
    ins_f, du_f, xs = layer_workload(cfg, 0, dev, factored=True, normal_du=True)
    Pe = ins_f[0].shape[0] * He
    re_ = time_solver(ins_f, du_f, Te, 1, 0, grad_limit=ce.get("grad_limit", 1e6))
    ach = flops_fwd(de, Te) * Pe / (re_["fwd_ms"] * 1e-3)
    e = {"config": f"cfg{cfg}", "x": xs, "d": de, "T": Te, "heads": He, "problems": Pe,
         "workload": "full BASELINE x through the factored solver (B, Q, Q_f expanded per token chunk on the "
                     "device), d_u ~ N(0,1), one forward and one fwd+bwd step, no warm-up",
         "fwd_ms": re_["fwd_ms"], "fwd_solves_per_s": Pe / (re_["fwd_ms"] * 1e-3),
         "fwd_bwd_ms": re_["step_ms"], "fwd_bwd_solves_per_s": Pe / (re_["step_ms"] * 1e-3),
         "tokens_per_s_fwd_bwd": ins_f[0].shape[0] / (re_["step_ms"] * 1e-3),
         "bwd_fallback_problems": re_["bwd_fallback_problems"],
         "peak_mem_bytes_fwd_bwd": re_["peak_mem_bytes"],
         "roofline_frac": ach / PEAK_FP32_MFMA, "achieved_tflops": ach / 1e12,
         "wall_s": None}
    del ins_f, du_f
    torch.cuda.empty_cache()
    e["wall_s"] = time.perf_counter() - t0
    return e


if __name__ == "__main__":
    main()
