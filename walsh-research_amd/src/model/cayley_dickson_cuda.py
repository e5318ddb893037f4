"""Import path of the reference's octonion module
(src/model/cayley_dickson_cuda.py); the layers live in .octonion and run on
the HIP kernels."""
from .constants import SIGN_TABLE, WEIGHT_IDX  # noqa: F401
from .octonion import (OctonionFusedLinear, OctonionHeadMixerFused, OctonionPackedLinear,  # noqa: F401
                       cayley_dickson_fused, optimize_for_inference, pack_ternary_weights,
                       unpack_ternary_weights)
