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
SOURCES = ["ttc_lqr.hip"]
ARCH = os.environ.get("TTC_LQR_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (see DESIGN notes on this pool)
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", os.path.join(ROOT, "include")]


def build(verbose: bool = True) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    out = os.path.join(OUT_DIR, "libttc_lqr.so")
    tmp = out + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-shared", *[os.path.join(HERE, s) for s in SOURCES], "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if errs.strip() and verbose:
        print(errs, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    argparse.ArgumentParser(description=__doc__).parse_args()
    print(build())
