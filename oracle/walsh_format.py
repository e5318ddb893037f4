"""Oracle: the .walsh v4 bitmask + sign storage of ternary tensors.

Test infrastructure only (see ``oracle/__init__.py``).

Encoder ``compress.py:36-93`` (quantize_to_bitmask_ternary: bitmask of the
non-zeros, LSB-first within each byte, padded to whole bytes; signs of the
non-zeros in order, 1 = +1, LSB-first) and decoder
``generate_compressed.py:70-105`` (unpack_bitmask_ternary, positions past
``num_nonzero`` stay 0), restated with numpy on given codes.
"""
import numpy as np


def encode_codes(codes):
    """Ternary codes (any shape) -> (bitmask bytes, sign bytes, num_nonzero)."""
    c = np.asarray(codes).reshape(-1).astype(np.int8)
    nz = c != 0
    bitmask = np.packbits(nz, bitorder='little')
    signs = np.packbits(c[nz] == 1, bitorder='little')
    return bitmask.astype(np.uint8), signs.astype(np.uint8), int(nz.sum())


def decode_codes(bitmask, sign_bits, shape, num_nonzero) -> np.ndarray:
    """Inverse of encode_codes -> int8 codes of ``shape``."""
    total = int(np.prod(shape))
    bits = np.unpackbits(np.asarray(bitmask, np.uint8), bitorder='little')[:total]
    pos = np.flatnonzero(bits)[:num_nonzero]
    sgn = np.unpackbits(np.asarray(sign_bits, np.uint8), bitorder='little')[:len(pos)]
    out = np.zeros(total, np.int8)
    out[pos[:len(sgn)]] = np.where(sgn == 1, 1, -1)
    return out.reshape(shape)
