"""Build ``libttc_lqr.so`` for gfx950 in-tree (``ttc-net_amd/lib/``).

Usage: ``python ttc-net_amd/csrc/build.py [--jobs N]``.  Called by
``__graft_entry__.build()``.  Always recompiles.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.normpath(os.path.join(HERE, "..", ".."))
OUT_DIR = os.path.normpath(os.path.join(HERE, "..", "lib"))
SOURCES = ["ttc_lqr_capi.hip", "ttc_lqr_d16.hip", "ttc_lqr_d16_mfma.hip", "ttc_lqr_d32.hip", "ttc_lqr_d64.hip",
           "ttc_lqr_d32_mfma.hip", "ttc_lqr_d64_mfma.hip", "ttc_lqr_d16_sym.hip",
           "ttc_lqr_factored.hip", "ttc_lqr_d16_ham.hip", "ttc_lqr_d32_ham.hip", "ttc_lqr_d64_ham.hip",
           "ttc_lqr_epilogue.hip", "ttc_lqr_stash.hip", "ttc_lqr_noalloc.hip", "ttc_lqr_d16_f64.hip"]
HOST_SOURCES = ["ttc_lqr_host.cpp"]  # CPU code (no GPU kernels): compiled by the host compiler
ARCH = os.environ.get("TTC_LQR_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (some of their forms have given wrong results
# on the GPUs this builds for; the compiler emits them from ordinary float code otherwise)
CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-I", os.path.join(ROOT, "include")]
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", os.path.join(ROOT, "include")]
# Per translation unit: the fp64 matrix-core sweeps keep their MFMA accumulators in VGPRs instead
# of routing every product through an AGPR tile and back (at one wave per SIMD their registers are
# full; the symplectic step's loop falls from 489 to 321 instructions, with no accumulator moves).
EXTRA_FLAGS = {"ttc_lqr_d16_f64.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if errs.strip() and verbose:
        print(errs, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Compile each translation unit in parallel, then link the shared library."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OUT_DIR, exist_ok=True)
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    out = os.path.join(OUT_DIR, "libttc_lqr.so")
    tmp = out + ".tmp"
    objs = [os.path.join(obj_dir, os.path.splitext(s)[0] + ".o") for s in SOURCES + HOST_SOURCES]
    cxx = os.environ.get("CXX", "g++")
    cmds = [[hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(s, []), "-c", os.path.join(HERE, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    cmds += [[cxx, *CXX_FLAGS, "-c", os.path.join(HERE, s), "-o", o]
             for s, o in zip(HOST_SOURCES, objs[len(SOURCES):])]
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", *objs, "-lpthread", "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    argparse.ArgumentParser(description=__doc__).parse_args()
    print(build())
