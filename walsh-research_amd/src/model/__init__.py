"""Walsh ternary structured-linear hot path on MI355X (HIP kernels behind a C ABI).

Same public surface as the reference package ``src.model``
(src/model/__init__.py:1-2).
"""
from .chassis import KVCache, Walsh, WalshConfig
from .mhc import SinkhornKnopp, mHCResidualStream, mHCWalsh

__all__ = ["Walsh", "WalshConfig", "KVCache", "mHCWalsh", "mHCResidualStream", "SinkhornKnopp"]
