"""TTC-Net's Test-Time Control layer on AMD MI355X (gfx950).

``from ttc import TTCLayer`` as with the reference package (``ttc/__init__.py``);
the LQR solve inside runs in hand-written HIP kernels (``libttc_lqr.so``).
"""
from .layers.ttc_layer import TTCLayer

__all__ = ["TTCLayer"]
