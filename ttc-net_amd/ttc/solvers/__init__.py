"""LQR solvers, with the reference's export surface (``ttc/solvers/__init__.py:1-4``):

* ``fused_lqr_solve`` (``ttc.solvers.fused_lqr``): the gfx950 HIP solver behind the reference's
  fused entry point (``fused_lqr.py:294``); ``hip_lqr_solve`` is the same solver with this
  build's keyword-only knobs, ``hip_lqr_solve_factored`` takes the layer's low-rank factors;
* ``direct_lqr_solve`` (``riccati``) and ``kkt_lqr_solve`` (``kkt``) (``ttc.solvers.torch_lqr``):
  HIP kernels for CUDA tensors, the library's native host solver for CPU tensors.
"""
from .fused_lqr import fused_lqr_solve, FusedLQRSolveFunc
from .torch_lqr import direct_lqr_solve, kkt_lqr_solve
from .hip_lqr import hip_lqr_solve, HipLQRSolveFunc, hip_lqr_solve_factored, HipLQRFactoredFunc
from .host_lqr import host_lqr_solve, HostLQRSolveFunc

__all__ = ["direct_lqr_solve", "kkt_lqr_solve", "fused_lqr_solve", "FusedLQRSolveFunc", "hip_lqr_solve",
           "HipLQRSolveFunc", "hip_lqr_solve_factored", "HipLQRFactoredFunc", "host_lqr_solve", "HostLQRSolveFunc"]
