"""Pins for oracle.octonion: tables re-derived from Cayley-Dickson doubling."""
import numpy as np

from oracle import octonion


def _qmul(a, b):
    a0, a1, a2, a3 = a
    b0, b1, b2, b3 = b
    return np.array([a0 * b0 - a1 * b1 - a2 * b2 - a3 * b3,
                     a0 * b1 + a1 * b0 + a2 * b3 - a3 * b2,
                     a0 * b2 - a1 * b3 + a2 * b0 + a3 * b1,
                     a0 * b3 + a1 * b2 - a2 * b1 + a3 * b0])


def _qconj(a):
    return np.array([a[0], -a[1], -a[2], -a[3]])


def _omul(x, w):
    """Octonion product by Cayley-Dickson doubling of the quaternions:
    (a, b)(c, d) = (ac - d*b, da + bc*), with x = (a, b), w = (c, d)."""
    a, b, c, d = x[:4], x[4:], w[:4], w[4:]
    return np.concatenate([_qmul(a, c) - _qmul(_qconj(d), b),
                           _qmul(d, a) + _qmul(b, _qconj(c))])


def test_quaternion_sanity():
    i, j, k = np.eye(4)[1], np.eye(4)[2], np.eye(4)[3]
    assert np.array_equal(_qmul(i, j), k) and np.array_equal(_qmul(j, i), -k)
    assert np.array_equal(_qmul(i, i), -np.eye(4)[0])


def test_tables_are_the_cayley_dickson_product():
    E = np.eye(8)
    for j in range(8):
        for k in range(8):
            p = _omul(E[j], E[k])
            m = int(np.flatnonzero(p)[0])
            assert np.count_nonzero(p) == 1
            # x = e_j, w = e_k contributes only to y_m with W index k
            assert m == (j ^ k) and octonion.WEIGHT_IDX[m, j] == k
            assert p[m] == octonion.SIGN_TABLE[m, j]


def test_layer_with_unit_blocks_is_the_octonion_product():
    rng = np.random.default_rng(0)
    for _ in range(20):
        x = rng.standard_normal(8)
        w = rng.standard_normal(8)
        y = octonion.octonion_linear_f64(x.reshape(8, 1, 1), w.reshape(8, 1, 1), np.ones(1))
        assert np.allclose(y.reshape(8), _omul(x, w), atol=1e-12)


def test_octonion_norm_multiplicative():
    # |x w| = |x| |w| holds for octonions; a wrong sign breaks it.
    rng = np.random.default_rng(1)
    x, w = rng.standard_normal(8), rng.standard_normal(8)
    y = octonion.octonion_linear_f64(x.reshape(8, 1, 1), w.reshape(8, 1, 1), np.ones(1)).reshape(8)
    assert np.isclose(np.linalg.norm(y), np.linalg.norm(x) * np.linalg.norm(w))


def test_layer_matches_dense_matrix():
    rng = np.random.default_rng(2)
    in_o, out_o, M = 5, 3, 6
    codes = rng.integers(-1, 2, size=(8, out_o, in_o)).astype(np.int8)
    beta = rng.uniform(0.1, 1, size=out_o)
    x = rng.standard_normal((8, M, in_o))
    y = octonion.octonion_linear_f64(x, codes, beta)                 # [8, M, out_o]
    A = octonion.dense_matrix(codes, beta)
    xf = x.transpose(1, 0, 2).reshape(M, 8 * in_o)
    yf = (xf @ A.T).reshape(M, 8, out_o).transpose(1, 0, 2)
    assert np.allclose(y, yf, atol=1e-12)


def test_bf16_round():
    v = np.array([1.0, 1.00390625, 1.001953125, 1.0058594, -3.14159, 0.0], np.float32)
    r = octonion.bf16_round(v)
    assert r[0] == 1.0
    assert r[1] == 1.0                        # 1+2^-8 is a tie -> even (1.0)
    assert r[2] == 1.0                        # below the tie
    assert r[3] == np.float32(1.0078125)      # above the tie
    assert abs(r[4] - (-3.140625)) < 1e-7
    assert r[5] == 0.0


def test_bf16_round_matches_torch():
    import torch
    v = np.random.default_rng(7).standard_normal(1000).astype(np.float32)
    t = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(octonion.bf16_round(v), t)


def test_bwd_oracle_matches_torch_autograd():
    """The gradient oracle against torch float64 autograd of the table-driven
    forward with physics.quantize_ternary's STE (physics.py:43-50)."""
    import torch
    gen = torch.Generator().manual_seed(7)
    M, in_o, out_o = 9, 5, 3
    x = torch.randn(8, M, in_o, generator=gen, dtype=torch.float64, requires_grad=True)
    latent = (torch.rand(8, out_o, in_o, generator=gen, dtype=torch.float64) * 4 - 2).requires_grad_(True)
    beta = torch.randn(out_o, generator=gen, dtype=torch.float64, requires_grad=True)
    gy = torch.randn(8, M, out_o, generator=gen, dtype=torch.float64)
    gamma = latent.abs().mean() + 1e-8
    wq = torch.clamp(torch.round(latent / gamma), -1, 1)
    wc = latent.clamp(-1.5, 1.5)
    w = wc + (wq - wc).detach()
    ys = []
    for i in range(8):
        yi = 0
        for j in range(8):
            yi = yi + int(octonion.SIGN_TABLE[i, j]) * (x[j] @ w[int(octonion.WEIGHT_IDX[i, j])].T)
        ys.append(yi * beta)
    (torch.stack(ys) * gy).sum().backward()
    assert (latent.abs() > 1.5).any()
    dx, dW, db = octonion.octonion_linear_bwd_f64(x.detach().numpy(), wq.detach().numpy(), beta.detach().numpy(),
                                                  gy.numpy(), latent=latent.detach().numpy())
    for got, ref in ((dx, x.grad), (dW, latent.grad), (db, beta.grad)):
        assert np.allclose(got, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_bwd_dx_is_transpose_of_dense_matrix():
    rng = np.random.default_rng(8)
    M, in_o, out_o = 4, 3, 2
    codes = rng.integers(-1, 2, size=(8, out_o, in_o)).astype(np.int8)
    beta = rng.normal(size=out_o)
    x = rng.normal(size=(8, M, in_o))
    gy = rng.normal(size=(8, M, out_o))
    A = octonion.dense_matrix(codes, beta)
    dx, _, _ = octonion.octonion_linear_bwd_f64(x, codes, beta, gy)
    g_rows = np.concatenate(list(gy), axis=1)           # [M, 8*out_o], part-major
    dx_rows = np.concatenate(list(dx), axis=1)
    assert np.allclose(dx_rows, g_rows @ A, rtol=1e-12, atol=1e-12)
