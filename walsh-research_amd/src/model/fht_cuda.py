"""Import path of the reference's Hadamard module (src/model/fht_cuda.py);
the layers live in .hadamard and run on the HIP kernels."""
from .hadamard import (ALGEBRA_DIM, FHTFunction, HadamardHeadMixer, HadamardHeadMixerFused,  # noqa: F401
                       HadamardLinear, HadamardPackedLinear, HadamardTernaryLinear, HadamardTernaryLinearTuple, fht,
                       fht_butterfly, fht_reference, hadamard_matrix, optimize_for_inference, pack_ternary_weights,
                       unpack_ternary_weights)
