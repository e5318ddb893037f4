"""Pins for oracle.hadamard: Sylvester H, FHT, HadamardLinear forward."""
import math

import numpy as np
import scipy.linalg

from oracle import hadamard, ternary


def test_sylvester_matches_scipy():
    for n in (1, 2, 4, 8, 16, 32, 64):
        assert np.array_equal(hadamard.sylvester(n, normalize=False), scipy.linalg.hadamard(n))


def test_sylvester_symmetric_orthonormal():
    H = hadamard.sylvester(32)
    assert np.array_equal(H, H.T)
    assert np.allclose(H @ H, np.eye(32), atol=1e-14)


def test_fht_unit_vectors():
    e0 = np.zeros(32)
    e0[0] = 1
    assert np.allclose(hadamard.fht(e0), np.full(32, 1 / math.sqrt(32)))
    ones = np.ones(32)
    ref = np.zeros(32)
    ref[0] = math.sqrt(32)
    assert np.allclose(hadamard.fht(ones), ref)


def test_rust_kat_self_inverse():
    # inference/src/hadamard.rs:232-247: x[i] = i, fht_32 twice returns x
    # within 1e-5 (float32 arithmetic).
    x = np.arange(32, dtype=np.float32)
    y = hadamard.fht(hadamard.fht(x))
    assert y.dtype == np.float32
    assert np.max(np.abs(y - x)) < 1e-5


def test_rust_kat_norm_preserving():
    # inference/src/hadamard.rs:249-265: x[i] = (i+1)/32, ||fht_32(x)|| = ||x||
    # within 1e-5.
    x = (np.arange(32, dtype=np.float32) + 1) / 32
    assert abs(np.linalg.norm(hadamard.fht(x)) - np.linalg.norm(x)) < 1e-5


def test_fht_equals_matrix_product():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 32))
    assert np.allclose(hadamard.fht(x), x @ hadamard.sylvester(32), atol=1e-12)


def _layer(in_o, out_o, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-1, 2, size=(32, out_o, in_o)).astype(np.int8)
    alpha = rng.uniform(0.5, 1.5, size=(32, in_o))
    beta = rng.uniform(0.1, 0.4, size=(32, out_o))
    return codes, alpha, beta


def test_layer_matches_dense_matrix():
    for in_o, out_o in ((1, 1), (16, 16), (16, 43), (43, 16), (3, 5)):
        codes, alpha, beta = _layer(in_o, out_o, in_o * 100 + out_o)
        x = np.random.default_rng(1).standard_normal((7, 32 * in_o))
        A = hadamard.dense_matrix(codes, alpha, beta)
        assert np.allclose(hadamard.hadamard_linear_f64(x, codes, alpha, beta), x @ A.T, atol=1e-10)


def test_layer_scalar_closed_form():
    # in_o = out_o = 1: the layer is y = beta * H diag(w) H (alpha*x); with
    # all codes +1 it is the identity up to beta*alpha.
    codes = np.ones((32, 1, 1), np.int8)
    x = np.random.default_rng(2).standard_normal((3, 32))
    y = hadamard.hadamard_linear_f64(x, codes, np.full((32, 1), 2.0), np.full((32, 1), 0.5))
    assert np.allclose(y, x)


def test_torch32_path_close_to_float64():
    codes, alpha, beta = _layer(16, 16, 3)
    x = np.random.default_rng(4).standard_normal((64, 512)).astype(np.float32)
    y32 = hadamard.hadamard_linear_torch32(x, codes, alpha, beta).numpy()
    y64 = hadamard.hadamard_linear_f64(x, codes, alpha, beta)
    assert np.linalg.norm(y32 - y64) / np.linalg.norm(y64) < 1e-6


def test_init_weight_quantises_to_thirds():
    import torch
    g = torch.Generator().manual_seed(0)
    w = hadamard.init_weight(16, 16, g).numpy()
    norms = np.linalg.norm(w.reshape(32, -1), axis=1)
    assert np.allclose(norms, 0.02 * 16, rtol=1e-5)
    c = ternary.ternary_codes(w, ternary.absmean_gamma(w))
    frac = np.bincount(c.reshape(-1) + 1, minlength=3) / c.size
    assert np.all(np.abs(frac - np.array([0.345, 0.31, 0.345])) < 0.04)


def test_head_mixer_identity_weights():
    # W[h] = I: H H = I (normalised Sylvester), so the mixer is beta * x
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 32, 5, 8))
    beta = rng.uniform(0.1, 0.9, size=8)
    W = np.broadcast_to(np.eye(8), (32, 8, 8))
    assert np.allclose(hadamard.head_mixer_f64(x, W, beta), x * beta, atol=1e-12)


def test_head_mixer_equals_hadamard_linear_on_rows():
    # with ternary W the mixer is a Hadamard linear on the token rows
    # [32 heads x D]: codes[g, o, i] = W[g, i, o], alpha = 1, beta per column
    rng = np.random.default_rng(8)
    B, T, D = 2, 3, 12
    x = rng.standard_normal((B, 32, T, D))
    W = rng.integers(-1, 2, size=(32, D, D)).astype(np.float64)
    beta = rng.uniform(0.1, 0.9, size=D)
    y = hadamard.head_mixer_f64(x, W, beta)
    rows = x.transpose(0, 2, 1, 3).reshape(B * T, 32 * D)
    ref = hadamard.hadamard_linear_f64(rows, W.transpose(0, 2, 1).astype(np.int8), np.ones((32, D)),
                                       np.broadcast_to(beta, (32, D)))
    assert np.allclose(y.transpose(0, 2, 1, 3).reshape(B * T, 32 * D), ref, atol=1e-10)


def _freqs(T, D, theta=10000.0):
    import torch
    f = 1.0 / (theta ** (torch.arange(0, D, 2)[: D // 2].float() / D))
    ang = torch.outer(torch.arange(T).float(), f)
    return torch.polar(torch.ones_like(ang), ang)


def test_rope_matches_complex_multiply():
    # the real-arithmetic rotation equals torch's complex product
    import torch
    rng = np.random.default_rng(9)
    B, T, H, D = 2, 6, 3, 8
    y = rng.standard_normal((B, T, H * D)).astype(np.float32)
    fc = _freqs(T, D)
    yc = torch.view_as_complex(torch.from_numpy(y).reshape(B, T, H, D // 2, 2))
    ref = torch.view_as_real(yc * fc[:T].unsqueeze(0).unsqueeze(2)).reshape(B, T, H * D).numpy()
    assert np.allclose(hadamard.rope_f64(y, fc.numpy(), D), ref, atol=1e-6)


def test_rope_position_zero_identity_and_norm():
    rng = np.random.default_rng(10)
    y = rng.standard_normal((1, 5, 16))
    fc = _freqs(5, 8).numpy()
    r = hadamard.rope_f64(y, fc, 8)
    assert np.allclose(r[:, 0], y[:, 0])
    pn = lambda v: np.hypot(v.reshape(1, 5, 8, 2)[..., 0], v.reshape(1, 5, 8, 2)[..., 1])
    assert np.allclose(pn(r), pn(y))


# ---------------------------------------------------------------- backward

def _torch_layer_f64(x, latent, alpha, beta):
    """fht_cuda.py:489-519 with physics.quantize_ternary (physics.py:43-50),
    written with torch float64 ops so that autograd derives the gradients."""
    import torch
    M = x.shape[0]
    G, out_o, in_o = latent.shape
    gamma = latent.abs().mean() + 1e-8
    wq = torch.clamp(torch.round(latent / gamma), -1, 1)
    wc = latent.clamp(-1.5, 1.5)
    w = wc + (wq - wc).detach()
    H = torch.tensor(hadamard.sylvester(G), dtype=torch.float64)
    xs = x.view(M, G, in_o) * alpha
    xm = (xs.transpose(-2, -1) @ H).transpose(-2, -1)
    yp = torch.einsum('mgi,goi->mgo', xm, w)
    ym = (yp.transpose(-2, -1) @ H).transpose(-2, -1)
    return (ym * beta).reshape(M, G * out_o), wq


def _bwd_case(M, in_o, out_o, seed, big=0.0):
    import torch
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(M, 32 * in_o, generator=gen, dtype=torch.float64)
    latent = hadamard.init_weight(out_o, in_o, gen).double()
    if big:
        # push some latent weights past the STE clamp at +-1.5
        sel = torch.rand(latent.shape, generator=gen) < 0.2
        latent = torch.where(sel, latent.sign() * (1.5 + big * torch.rand(latent.shape, generator=gen,
                                                                               dtype=torch.float64)), latent)
    alpha = 1 + 0.5 * torch.randn(32, in_o, generator=gen, dtype=torch.float64)
    beta = 0.3 * torch.randn(32, out_o, generator=gen, dtype=torch.float64)
    gy = torch.randn(M, 32 * out_o, generator=gen, dtype=torch.float64)
    return x, latent, alpha, beta, gy


def test_bwd_oracle_matches_torch_autograd():
    for (M, in_o, out_o, seed, big) in ((7, 3, 5, 0, 0.0), (20, 4, 4, 1, 2.0), (5, 16, 8, 2, 0.5)):
        x, latent, alpha, beta, gy = _bwd_case(M, in_o, out_o, seed, big)
        xr, lr, ar, br = (t.clone().requires_grad_(True) for t in (x, latent, alpha, beta))
        y, wq = _torch_layer_f64(xr, lr, ar, br)
        y.backward(gy)
        codes = wq.detach().numpy().astype(np.int8)
        if big:
            assert (np.abs(latent.numpy()) > 1.5).any()
        dx, da, db, dw = hadamard.hadamard_linear_bwd_f64(x.numpy(), codes, alpha.numpy(), beta.numpy(), gy.numpy(),
                                                         latent=latent.numpy())
        for got, ref in ((dx, xr.grad), (da, ar.grad), (db, br.grad), (dw, lr.grad)):
            ref = ref.numpy()
            assert got.shape == ref.shape
            assert np.max(np.abs(got - ref)) <= 1e-12 * max(1.0, np.max(np.abs(ref)))


def test_bwd_dx_is_transpose_of_dense_matrix():
    # dx = gy A with A the layer's dense matrix (Kronecker construction)
    rng = np.random.default_rng(3)
    in_o, out_o, M = 3, 2, 6
    codes = rng.integers(-1, 2, size=(32, out_o, in_o)).astype(np.int8)
    alpha = rng.normal(size=(32, in_o))
    beta = rng.normal(size=(32, out_o))
    x = rng.normal(size=(M, 32 * in_o))
    gy = rng.normal(size=(M, 32 * out_o))
    A = hadamard.dense_matrix(codes, alpha, beta)
    dx, _, _, _ = hadamard.hadamard_linear_bwd_f64(x, codes, alpha, beta, gy)
    assert np.allclose(dx, gy @ A, rtol=1e-12, atol=1e-12)


def test_bwd_finite_differences():
    # central differences of the float64 forward in alpha, beta and the
    # (continuous) per-group matrices
    rng = np.random.default_rng(4)
    in_o, out_o, M = 2, 3, 4
    W = rng.normal(size=(32, out_o, in_o))
    alpha = rng.normal(size=(32, in_o))
    beta = rng.normal(size=(32, out_o))
    x = rng.normal(size=(M, 32 * in_o))
    gy = rng.normal(size=(M, 32 * out_o))
    _, da, db, dw = hadamard.hadamard_linear_bwd_f64(x, W, alpha, beta, gy)

    def loss(W_, a_, b_):
        return float(np.sum(hadamard.hadamard_linear_f64(x, W_, a_, b_) * gy))

    h = 1e-6
    for (idx, ref) in (((5, 1), da), ((31, 0), da)):
        e = np.zeros_like(alpha)
        e[idx] = h
        fd = (loss(W, alpha + e, beta) - loss(W, alpha - e, beta)) / (2 * h)
        assert abs(fd - ref[idx]) <= 1e-6 * max(1.0, abs(fd))
    for idx in ((0, 0), (17, 2)):
        e = np.zeros_like(beta)
        e[idx] = h
        fd = (loss(W, alpha, beta + e) - loss(W, alpha, beta - e)) / (2 * h)
        assert abs(fd - db[idx]) <= 1e-6 * max(1.0, abs(fd))
    for idx in ((0, 0, 0), (9, 2, 1), (31, 1, 0)):
        e = np.zeros_like(W)
        e[idx] = h
        fd = (loss(W + e, alpha, beta) - loss(W - e, alpha, beta)) / (2 * h)
        assert abs(fd - dw[idx]) <= 1e-6 * max(1.0, abs(fd))
