"""Pins for oracle.ternary (absmean quantiser and 2-bit packing)."""
import numpy as np

from oracle import ternary


def test_rounding_closed_forms():
    # gamma = 1 exactly, so W/gamma = W; half-to-even at the 0.5 boundary,
    # clamp at +-1.5 (rounds to +-2 first).
    w = np.array([0.5, -0.5, 1.5, -1.5, 2.5, 0.49999997, 0.50000006, 0.0, -0.0, 1.0, -1.0, 7.0],
                 dtype=np.float32)
    got = ternary.ternary_codes(w, np.float32(1.0))
    assert got.tolist() == [0, 0, 1, -1, 1, 0, 1, 0, 0, 1, -1, 1]


def test_codes_match_float64_away_from_ties():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(100_000) * 0.02).astype(np.float32)
    g = ternary.absmean_gamma(w)
    c = ternary.ternary_codes(w, g)
    r = w.astype(np.float64) / float(g)
    ref = np.clip(np.round(r), -1, 1)          # float64 rounding, no ties in practice
    safe = np.minimum(np.abs(np.abs(r) - 0.5), np.abs(np.abs(r) - 1.5)) > 1e-6
    assert np.array_equal(c[safe], ref[safe].astype(np.int8))
    # about a third of each value for N(0, s) weights (absmean threshold 0.5*gamma)
    frac = np.bincount(c + 1, minlength=3) / c.size
    assert np.all(np.abs(frac - np.array([0.345, 0.31, 0.345])) < 0.03), frac


def test_gamma_matches_exact_mean():
    rng = np.random.default_rng(1)
    for n in (1, 7, 4096, 262_144):
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        g = ternary.absmean_gamma(w)
        exact = ternary.absmean_gamma_exact(w)
        assert abs(float(g) - exact) <= 4 * np.spacing(np.float32(exact)), (n, g, exact)


def test_rounded_gamma_closed_forms():
    """Correct rounding of the mean, ties to even: mean(1, 1 + 2^-23) =
    1 + 2^-24 lies halfway between 1 and 1 + 2^-23 and rounds to 1;
    mean(1, 1 + 3*2^-23) = 1 + 3*2^-24 rounds up to 1 + 2^-22 (even);
    equal values give themselves; subnormals are summed exactly."""
    one = np.float32(1.0)
    u = np.float32(2.0 ** -23)
    m = lambda a: ternary.round_to_f32(*_mean_rational(a))  # noqa: E731
    assert m(np.array([one, one + u], np.float32)) == one
    assert m(np.array([one, one + 3 * u], np.float32)) == np.float32(1 + 2.0 ** -22)
    assert m(np.full(1000, np.float32(0.0123), np.float32)) == np.float32(0.0123)
    tiny = np.float32(2.0 ** -149)
    assert m(np.array([tiny, tiny, tiny, -tiny], np.float32)) == tiny
    g = ternary.absmean_gamma_rounded(np.array([one, -one - u], np.float32))
    assert g == np.float32(one + np.float32(1e-8))


def _mean_rational(a):
    num, den = ternary.exact_abs_sum(a)
    return num, den * a.size


def test_rounded_gamma_brute_force_and_torch():
    """The exact integer sum equals a Fraction sum of the same floats; the
    rounded mean is the float32 nearest to the exact mean; torch-CPU's
    float32 abs().mean() (the reference's CPU expression) is within one ulp
    of it at every thread count, and which ulp it lands on varies."""
    from fractions import Fraction
    import torch
    rng = np.random.default_rng(11)
    for n in (3, 100, 5000):
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        num, den = ternary.exact_abs_sum(w)
        assert Fraction(num, den) == sum(Fraction(float(abs(v))) for v in w)
        q = Fraction(num, den * n)
        r = ternary.round_to_f32(num, den * n)
        for c in (np.nextafter(r, np.float32(-1)), np.nextafter(r, np.float32(1))):
            assert abs(Fraction(float(r)) - q) <= abs(Fraction(float(c)) - q)
    threads = torch.get_num_threads()
    try:
        for seed in range(4):
            w = (np.random.default_rng(seed).standard_normal((128, 128, 32)) * 0.02).astype(np.float32)
            g = ternary.absmean_gamma_rounded(w)
            for nt in (1, 2, 4, 8):
                torch.set_num_threads(nt)
                gt = ternary.absmean_gamma(w)
                assert abs(int(gt.view(np.int32)) - int(g.view(np.int32))) <= 1, (seed, nt, gt, g)
    finally:
        torch.set_num_threads(threads)


def test_gamma_zero_tensor():
    w = np.zeros(64, np.float32)
    g = ternary.absmean_gamma(w)
    assert g == np.float32(1e-8)
    assert np.all(ternary.ternary_codes(w, g) == 0)


def test_ste_value_equals_code_exactly():
    # quantize_ternary returns clamp(w) + (q - clamp(w)); brute force over
    # many magnitudes shows it is exactly q in float32.
    rng = np.random.default_rng(2)
    for scale in (1e-4, 0.02, 0.5, 1.0, 3.0):
        w = (rng.standard_normal(50_000) * scale).astype(np.float32)
        g = ternary.absmean_gamma(w)
        c = ternary.ternary_codes(w, g)
        v = ternary.ste_value(w, c)
        assert np.array_equal(v, c.astype(np.float32))


def test_moe_quantized_scales_by_gamma():
    rng = np.random.default_rng(3)
    w = rng.uniform(-1, 1, size=(4, 16, 8)).astype(np.float32)
    c, g, v = ternary.moe_quantized(w)
    assert abs(float(g) - 0.5) < 0.02                     # mean |U(-1,1)| = 1/2
    assert np.array_equal(v, c.astype(np.float32) * g)
    assert set(np.unique(v).tolist()) <= {-float(g), 0.0, float(g)}


def test_pack_bit_layout():
    codes = np.array([[-1, 0, 1, 0, 1, 1, -1, -1]], np.int8)
    p = ternary.pack_codes(codes)
    # v = code+1: [0,1,2,1] -> 0<<6|1<<4|2<<2|1 = 25 ; [2,2,0,0] -> 160
    assert p.tolist() == [[25, 160]]


def test_pack_roundtrip_and_padding():
    rng = np.random.default_rng(4)
    for K in (4, 16, 43, 128, 342):
        c = rng.integers(-1, 2, size=(3, 5, K)).astype(np.int8)
        p = ternary.pack_codes(c)
        assert p.shape == (3, 5, (K + 3) // 4)
        assert np.array_equal(ternary.unpack_codes(p, K), c)
        if K % 4:
            # padding uses code 0 (v = 0b01) in the unused low slots
            pad = (-K) % 4
            last = p[..., -1]
            assert np.all((last & ((1 << (2 * pad)) - 1)) == int('01' * pad, 2))
