"""Oracle: absmean ternary quantisation and the 2-bit packed format.

Test infrastructure only (see ``oracle/__init__.py``).
"""
import numpy as np
import torch

EPS_GAMMA = 1e-8


def absmean_gamma(w) -> np.float32:
    """gamma = mean(|W|) + 1e-8 over the whole tensor, float32.

    Follows ``src/model/physics.py:24`` (and the identical MoE variant at
    ``src/model/moe.py:279``).  The reference computes this with torch on
    the device holding the weight; on the CPU path that is torch-CPU's
    float32 ``abs().mean()``, so the oracle uses exactly that expression to
    be bit-identical with the reference's CPU arithmetic.
    """
    t = torch.as_tensor(np.ascontiguousarray(w, dtype=np.float32))
    g = t.abs().mean() + EPS_GAMMA
    return np.float32(g.item())


def absmean_gamma_exact(w) -> float:
    """Float64 mean(|W|) + 1e-8: the value ``absmean_gamma`` approximates."""
    return float(np.abs(np.asarray(w, dtype=np.float64)).mean() + EPS_GAMMA)


def exact_abs_sum(w):
    """sum(|W|) of float32 values as an exact rational (numerator, denominator).

    Every float32 is m * 2^(s - 149) with an integer m < 2^24 and
    0 <= s < 255, so the sum is an integer over 2^149: the mantissas are
    summed per exponent (float64 sums of at most 2^29 integers below 2^24
    are exact) and combined as Python integers."""
    a = np.abs(np.ascontiguousarray(w, dtype=np.float32)).ravel()
    bits = a.view(np.uint32).astype(np.int64)
    exp = (bits >> 23) & 0xFF
    man = bits & 0x7FFFFF
    man = np.where(exp > 0, man | 0x800000, man)
    shift = np.where(exp > 0, exp - 1, 0)
    assert a.size < (1 << 29) and not np.any(exp == 0xFF), "finite inputs below 2^29 elements"
    per = np.bincount(shift, weights=man.astype(np.float64), minlength=1)
    total = 0
    for s, v in enumerate(per):
        if v:
            total += int(v) << s
    return total, 1 << 149


def round_to_f32(num: int, den: int) -> np.float32:
    """num/den rounded to the nearest float32, ties to even (exact rational
    comparison of the candidates around the double quotient)."""
    from fractions import Fraction
    q = Fraction(num, den)
    f = np.float32(num / den)            # Python int division is correctly rounded to double
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = None
    for c in cands:
        d = abs(Fraction(float(c)) - q)
        if best is None or d < best[0] or (d == best[0] and int(np.float32(c).view(np.uint32)) % 2 == 0):
            best = (d, c)
    return np.float32(best[1])


def absmean_gamma_rounded(w) -> np.float32:
    """gamma = mean(|W|) + 1e-8 (``physics.py:24``, ``moe.py:279``) with the
    mean rounded correctly: the exact mean of the float32 weights rounded to
    the nearest float32, then the float32 addition of 1e-8 (torch casts the
    Python scalar to the tensor's float32 first).

    This is the value a float32 reduction approximates; torch-CPU's own
    ``abs().mean()`` lands within an ulp of it, and which ulp depends on
    the reduction order and on the number of threads torch uses."""
    num, den = exact_abs_sum(w)
    n = int(np.asarray(w).size)
    mean = round_to_f32(num, den * n)
    return np.float32(mean + np.float32(EPS_GAMMA))


def ternary_codes(w, gamma) -> np.ndarray:
    """codes = clamp(round_half_even(W / gamma), -1, 1) as int8.

    Follows ``src/model/physics.py:27-29``: float32 division, torch.round
    (round half to even), clamp to [-1, 1].
    """
    w32 = np.asarray(w, dtype=np.float32)
    q = np.rint(w32 / np.float32(gamma))          # IEEE f32 divide, ties-to-even
    return np.clip(q, -1, 1).astype(np.int8)


def ste_value(w, codes) -> np.ndarray:
    """The float value ``quantize_ternary`` returns in the forward pass.

    ``src/model/physics.py:50-51``: c = clamp(W, -1.5, 1.5); value =
    c + (q - c) evaluated in float32.  (It equals q exactly; the oracle tests
    check that by brute force.)
    """
    w32 = np.asarray(w, dtype=np.float32)
    c = np.clip(w32, np.float32(-1.5), np.float32(1.5))
    q = codes.astype(np.float32)
    return (c + (q - c)).astype(np.float32)


def moe_quantized(w):
    """MoE variant: returns (codes, gamma, code * gamma in float32).

    ``src/model/moe.py:276-288``: same codes as ``ternary_codes`` but the
    forward value is scaled back by gamma and there is no latent clamp.
    """
    g = absmean_gamma(w)
    c = ternary_codes(w, g)
    return c, g, (c.astype(np.float32) * g).astype(np.float32)


def tie_margin(w, gamma) -> float:
    """Smallest distance of |W/gamma| to a rounding boundary (0.5 or 1.5).

    A GPU-side gamma that differs from the oracle's by d (relative) can only
    flip codes whose margin is below about d * 1.5; tests report this.
    """
    r = np.abs(np.asarray(w, dtype=np.float64) / float(gamma))
    return float(np.min(np.minimum(np.abs(r - 0.5), np.abs(r - 1.5))))


def pack_codes(codes) -> np.ndarray:
    """2-bit pack along the last axis: byte = v0<<6 | v1<<4 | v2<<2 | v3.

    Encoding v = code + 1 (-1 -> 0b00, 0 -> 0b01, +1 -> 0b10), following
    ``src/model/fht_cuda.py:65-93`` (duplicated at
    ``src/model/cayley_dickson_cuda.py:134-161``).  The reference asserts
    K % 4 == 0 (``fht_cuda.py:78``); for other K this build pads K up to a
    multiple of 4 with code 0 (v = 0b01), which is what ``pad=True`` does.
    """
    c = np.asarray(codes, dtype=np.int8)
    K = c.shape[-1]
    if K % 4:
        pad = (-K) % 4
        c = np.concatenate([c, np.zeros(c.shape[:-1] + (pad,), np.int8)], axis=-1)
    v = (c.astype(np.int16) + 1).astype(np.uint8)
    v = v.reshape(c.shape[:-1] + (c.shape[-1] // 4, 4))
    return ((v[..., 0] << 6) | (v[..., 1] << 4) | (v[..., 2] << 2) | v[..., 3]).astype(np.uint8)


def unpack_codes(packed, K) -> np.ndarray:
    """Inverse of ``pack_codes`` (``src/model/fht_cuda.py:96-117``)."""
    p = np.asarray(packed, dtype=np.uint8)
    parts = [((p >> s) & 3).astype(np.int8) - 1 for s in (6, 4, 2, 0)]
    out = np.stack(parts, axis=-1).reshape(p.shape[:-1] + (p.shape[-1] * 4,))
    return out[..., :K].copy()
