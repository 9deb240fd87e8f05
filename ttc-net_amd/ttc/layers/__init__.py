from .ttc_layer import TTCLayer, LQR_SOLVER_IMPL_MAP

__all__ = ["TTCLayer", "LQR_SOLVER_IMPL_MAP"]
